"""GPU tests of the fused LayerNorm (ngt_layernorm_fwd/bwd) and FusedLayerNorm,
the encoder's nn.LayerNorm under bf16 autocast, against float64 LayerNorm of
the same inputs (fp32 math: 1e-5; bf16 outputs: their own rounding)."""
import pytest
import torch
import torch.nn as nn
import torch.nn.functional as F

from neutrongt_amd.layernorm import FusedLayerNorm, _LayerNormFn
from tests._util import relerr

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)


@pytest.mark.parametrize("n,c,in_dt,out_bf16", [
    (32768, 768, torch.bfloat16, True), (32768, 768, torch.float32, False),
    (1000, 128, torch.float32, False), (777, 64, torch.bfloat16, False),
    (5, 2048, torch.float32, True), (3, 4, torch.float32, False), (64, 1000, torch.bfloat16, True)])
def test_layernorm_matches_fp64(n, c, in_dt, out_bf16):
    _say(f"case layernorm n={n} c={c} {in_dt} out_bf16={out_bf16}")
    g = torch.Generator(device="cuda").manual_seed(n + c)
    x = (torch.randn(n, c, device="cuda", generator=g) * 3 + 1).to(in_dt)
    w = torch.randn(c, device="cuda", generator=g)
    b = torch.randn(c, device="cuda", generator=g)
    gy = torch.randn(n, c, device="cuda", generator=g)
    xr = x.detach().requires_grad_(True)
    wr = w.clone().requires_grad_(True)
    br = b.clone().requires_grad_(True)
    y = _LayerNormFn.apply(xr, wr, br, 1e-5, out_bf16)
    assert y.dtype == (torch.bfloat16 if out_bf16 else torch.float32)
    y.backward(gy.to(y.dtype))
    x64 = x.double().requires_grad_(True)
    w64 = w.double().requires_grad_(True)
    b64 = b.double().requires_grad_(True)
    y64 = F.layer_norm(x64, (c,), w64, b64, 1e-5)
    y64.backward(gy.to(y.dtype).double())
    tol_y = 5e-3 if out_bf16 else 1e-5
    assert relerr(y, y64) < tol_y
    # dx is written in the input's dtype
    assert xr.grad.dtype == in_dt
    assert relerr(xr.grad, x64.grad) < (5e-3 if in_dt == torch.bfloat16 else 1e-5)
    assert relerr(wr.grad, w64.grad) < 1e-5
    assert relerr(br.grad, b64.grad) < 1e-5
    # fixed summation order: a second backward gives the same parameter grads
    wr2 = w.clone().requires_grad_(True)
    br2 = b.clone().requires_grad_(True)
    _LayerNormFn.apply(x, wr2, br2, 1e-5, out_bf16).backward(gy.to(y.dtype))
    assert torch.equal(wr2.grad, wr.grad) and torch.equal(br2.grad, br.grad)


def test_fused_layernorm_module_under_autocast():
    """Same parameters as nn.LayerNorm; under bf16 autocast the fp32-output
    variant matches autocast's own LayerNorm, the bf16 variant its rounding."""
    _say("case FusedLayerNorm module")
    torch.manual_seed(0)
    ref = nn.LayerNorm(96).cuda()
    nn.init.normal_(ref.weight)
    nn.init.normal_(ref.bias)
    for out_bf16 in (False, True):
        mod = FusedLayerNorm(96, out_bf16=out_bf16).cuda()
        mod.load_state_dict(ref.state_dict())
        x = torch.randn(2, 300, 96, device="cuda").to(torch.bfloat16).requires_grad_(True)
        x2 = x.detach().clone().requires_grad_(True)
        gy = torch.randn(2, 300, 96, device="cuda")
        with torch.autocast("cuda", dtype=torch.bfloat16):
            y = mod(x)
            y_ref = ref(x2)
        assert y_ref.dtype == torch.float32
        assert y.dtype == (torch.bfloat16 if out_bf16 else torch.float32)
        assert relerr(y.float(), y_ref) < (5e-3 if out_bf16 else 1e-5)
        y.backward(gy.to(y.dtype))
        y_ref.backward(gy)
        assert x.grad.dtype == torch.bfloat16
        assert relerr(x.grad.float(), x2.grad.float()) < 1e-2
        assert relerr(mod.weight.grad, ref.weight.grad) < (5e-3 if out_bf16 else 1e-5)
        ref.weight.grad = ref.bias.grad = None
    # outside autocast: nn.LayerNorm itself
    assert torch.equal(mod(x.detach().float()), ref(x.detach().float()))


@pytest.mark.parametrize("n,c,dt,p", [(32768, 768, torch.bfloat16, 0.3), (1000, 128, torch.float32, 0.5),
                                      (513, 64, torch.bfloat16, 0.0), (7, 2048, torch.float32, 0.1)])
def test_add_dropout_layernorm_matches_fp64(n, c, dt, p):
    """s = x + dropout(y), out = LN(s) in one pass, against the same formula
    in float64 with the oracle's mask; dx = dS + LN backward, dy = dx * mask."""
    from neutrongt_amd.layernorm import _AddLayerNormFn
    from oracle import attention as OA
    _say(f"case add+dropout+LN n={n} c={c} {dt} p={p}")
    g = torch.Generator(device="cuda").manual_seed(n + c)
    x = torch.randn(n, c, device="cuda", generator=g).to(dt)
    y = torch.randn(n, c, device="cuda", generator=g).to(dt)
    w = torch.randn(c, device="cuda", generator=g)
    b = torch.randn(c, device="cuda", generator=g)
    g_s = torch.randn(n, c, device="cuda", generator=g).to(dt)
    g_o = torch.randn(n, c, device="cuda", generator=g).to(dt)
    seed = 1234 + n
    xr, yr = x.clone().requires_grad_(True), y.clone().requires_grad_(True)
    wr, br = w.clone().requires_grad_(True), b.clone().requires_grad_(True)
    s, out = _AddLayerNormFn.apply(xr, yr, wr, br, 1e-5, p, seed, dt == torch.bfloat16)
    (s.float() * g_s.float()).sum().add_((out.float() * g_o.float()).sum()).backward()
    mult = torch.from_numpy(OA.dropout_multiplier(seed, 1, n, c, p)[0]).cuda().double()
    s_ref = (x.double() + y.double() * mult).to(dt)  # the stored sum is in the input dtype
    if p == 0.0:
        assert torch.equal(s, s_ref)
    assert relerr(s, s_ref) < (5e-3 if dt == torch.bfloat16 else 1e-6)
    s64 = s.detach().double().requires_grad_(True)
    w64, b64 = w.double().requires_grad_(True), b.double().requires_grad_(True)
    o64 = F.layer_norm(s64, (c,), w64, b64, 1e-5)
    (o64 * g_o.double()).sum().backward()
    assert relerr(out, o64) < (5e-3 if dt == torch.bfloat16 else 1e-5)
    dx64 = s64.grad + g_s.double()
    tol = 5e-3 if dt == torch.bfloat16 else 1e-5
    assert relerr(xr.grad, dx64) < tol
    assert relerr(yr.grad, dx64 * mult) < tol
    assert relerr(wr.grad, w64.grad) < 1e-5 and relerr(br.grad, b64.grad) < 1e-5
    if p > 0:
        kept = (mult > 0).float().mean().item()
        assert abs(kept - (1 - p)) < 0.02

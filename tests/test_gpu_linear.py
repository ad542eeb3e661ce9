"""GPU tests of WgradLinear (the encoder's nn.Linear with a split-K weight
gradient and the HIP bias gradient ngt_colsum_bf16).

The reference computes these gradients with autograd (fp32 in the reference,
bf16 GEMMs under autocast here); the check is against float64 products of
the same bf16 inputs, where fp32 accumulation is within 1e-5."""
import pytest
import torch
import torch.nn as nn

from neutrongt_amd.linear import WgradLinear, chunk_sum, colsum_bf16, weight_grad
from tests._util import relerr

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)


@pytest.mark.parametrize("K,n_out,n_in", [(32768, 768, 768), (1000, 64, 128), (37, 24, 40),
                                          (5000, 1536, 768), (300, 136, 8), (1, 8, 8),
                                          (70001, 128, 256), (32768, 47, 768), (32768, 768, 100),
                                          (513, 9, 13), (300, 1, 8)])
def test_weight_and_bias_grad_match_fp64(K, n_out, n_in):
    _say(f"case wgrad K={K} n_out={n_out} n_in={n_in}")
    g = torch.Generator(device="cuda").manual_seed(K + n_out)
    x = torch.randn(K, n_in, device="cuda", generator=g).to(torch.bfloat16)
    dy = torch.randn(K, n_out, device="cuda", generator=g).to(torch.bfloat16)
    dw = weight_grad(x, dy)
    db = colsum_bf16(dy)
    assert dw.dtype == db.dtype == torch.float32
    assert relerr(dw, dy.double().T @ x.double()) < 1e-5
    assert relerr(db, dy.double().sum(0)) < 1e-5
    assert torch.equal(colsum_bf16(dy), db)  # fixed summation order


def test_colsum_edge_cases():
    _say("case colsum edges")
    empty = torch.empty(0, 16, device="cuda", dtype=torch.bfloat16)
    assert colsum_bf16(empty).abs().sum().item() == 0
    base = torch.randn(513, 40, device="cuda").to(torch.bfloat16)
    view = base[1:]  # rows start 80 bytes in: not 16-byte aligned -> 2-byte loads
    assert relerr(colsum_bf16(view), view.double().sum(0)) < 1e-5
    # the two load widths add each column's rows in the same order: same bits
    assert torch.equal(colsum_bf16(view), colsum_bf16(view.clone()))
    for n in (1, 7, 47, 100, 263):
        dy = torch.randn(1000, n, device="cuda").to(torch.bfloat16)
        assert relerr(colsum_bf16(dy), dy.double().sum(0)) < 1e-5, n


@pytest.mark.parametrize("chunks,n", [(1, 12), (3, 10), (4, 589824), (5, 7), (16, 589824),
                                      (17, 1001), (8, 2304 * 768)])
def test_chunk_sum_adds_the_chunks_in_order(chunks, n):
    """ngt_chunk_sum_f32 equals a sequential fp32 sum over the chunks, chunk 0
    first, bit for bit, with 16-byte and with scalar loads."""
    _say(f"case chunk_sum chunks={chunks} n={n}")
    g = torch.Generator(device="cuda").manual_seed(chunks * 7 + n)
    parts = torch.randn(chunks, n, device="cuda", generator=g) * torch.logspace(
        -3, 3, chunks, device="cuda")[:, None]
    want = parts[0].clone()
    for c in range(1, chunks):
        want = want + parts[c]  # one fp32 rounding per chunk, in order
    got = chunk_sum(parts)
    assert torch.equal(got, want)
    buf = torch.empty(chunks * n + 1, device="cuda")
    odd = buf[1:].view(chunks, n)  # 4 bytes in: scalar loads
    odd.copy_(parts)
    assert torch.equal(chunk_sum(odd), want)


@pytest.mark.parametrize("n_in,n_out", [(100, 768), (768, 47)])
def test_wgrad_linear_any_width(n_in, n_out):
    """The node encoder (100 -> 768) and a 47-class readout take the split-K
    dW and the HIP db too: dW/db as float64 products, forward as nn.Linear."""
    _say(f"case WgradLinear width {n_in} -> {n_out}")
    torch.manual_seed(2)
    ref = nn.Linear(n_in, n_out).cuda()
    mod = WgradLinear(n_in, n_out).cuda()
    mod.load_state_dict(ref.state_dict())
    x = torch.randn(32768, n_in, device="cuda")
    gy = torch.randn(32768, n_out, device="cuda")
    with torch.autocast("cuda", dtype=torch.bfloat16):
        y = mod(x)
        y_ref = ref(x)
    assert torch.equal(y, y_ref)
    y.backward(gy)
    x16 = x.to(torch.bfloat16).double()
    g16 = gy.to(torch.bfloat16).double()
    assert mod.weight.grad.dtype == torch.float32
    assert relerr(mod.weight.grad, g16.T @ x16) < 1e-5
    assert relerr(mod.bias.grad, g16.sum(0)) < 1e-5


def test_wgrad_linear_module_under_autocast():
    """Same forward as nn.Linear under bf16 autocast; dX as autocast's
    backward; dW/db as float64 products of the saved bf16 activations."""
    _say("case WgradLinear module")
    torch.manual_seed(0)
    ref = nn.Linear(96, 40).cuda()
    mod = WgradLinear(96, 40).cuda()
    mod.load_state_dict(ref.state_dict())
    x = torch.randn(3, 500, 96, device="cuda", requires_grad=True)
    x2 = x.detach().clone().requires_grad_(True)
    gy = torch.randn(3, 500, 40, device="cuda")
    with torch.autocast("cuda", dtype=torch.bfloat16):
        y = mod(x)
        y_ref = ref(x2)
    assert y.dtype == y_ref.dtype == torch.bfloat16
    assert torch.equal(y, y_ref)
    y.backward(gy)
    y_ref.backward(gy)
    assert x.grad.dtype == torch.float32
    assert relerr(x.grad, x2.grad) < 1e-2  # both bf16 GEMMs of the same operands
    x16 = x.detach().to(torch.bfloat16).reshape(-1, 96).double()
    g16 = gy.to(torch.bfloat16).reshape(-1, 40).double()
    assert relerr(mod.weight.grad, g16.T @ x16) < 1e-5
    assert relerr(mod.bias.grad, g16.sum(0)) < 1e-5
    assert relerr(mod.weight.grad, ref.weight.grad) < 1e-2  # autocast rounds dW to bf16
    # outside autocast it is nn.Linear
    y32 = mod(x.detach())
    assert y32.dtype == torch.float32


@pytest.mark.parametrize("use", ["qkv", "qv", "k"])
def test_projection_group_matches_separate_layers(use):
    """project(x, q, k, v): forward bit-equal to the separate layers; dX (summed
    inside the GEMMs) as close to the float64 sum of the bf16 products as
    autograd's sum of the separate layers' bf16 dX; dW/db as float64.  Outputs
    left out of the loss get no weight gradient."""
    from neutrongt_amd.linear import project
    _say(f"case projection group use={use}")
    torch.manual_seed(1)
    n_in, n_out = 128, 96
    refs = [nn.Linear(n_in, n_out).cuda() for _ in range(3)]
    mods = [WgradLinear(n_in, n_out).cuda() for _ in range(3)]
    for m, r in zip(mods, refs):
        m.load_state_dict(r.state_dict())
    x = torch.randn(2, 3000, n_in, device="cuda", requires_grad=True)
    x2 = x.detach().clone().requires_grad_(True)
    gys = [torch.randn(2, 3000, n_out, device="cuda") for _ in range(3)]
    with torch.autocast("cuda", dtype=torch.bfloat16):
        ys = project(x, *mods)
        ys_ref = [r(x2) for r in refs]
    for y, yr in zip(ys, ys_ref):
        assert y.dtype == torch.bfloat16 and torch.equal(y, yr)
    picked = [i for i, c in enumerate("qkv") if c in use]
    sum(((ys[i].float() * gys[i]).sum() for i in picked)).backward()
    sum(((ys_ref[i].float() * gys[i]).sum() for i in picked)).backward()
    x16 = x.detach().to(torch.bfloat16).reshape(-1, n_in).double()
    exact = sum(gys[i].to(torch.bfloat16).reshape(-1, n_out).double()
                @ mods[i].weight.detach().to(torch.bfloat16).double() for i in picked)
    err = relerr(x.grad.reshape(-1, n_in), exact)
    err_ref = relerr(x2.grad.reshape(-1, n_in), exact)
    assert err < 8e-3 and err <= 1.5 * err_ref + 1e-4, (err, err_ref)
    for i in range(3):
        if i not in picked:
            assert mods[i].weight.grad is None and mods[i].bias.grad is None
            continue
        g16 = gys[i].to(torch.bfloat16).reshape(-1, n_out).double()
        assert relerr(mods[i].weight.grad, g16.T @ x16) < 1e-5
        assert relerr(mods[i].bias.grad, g16.sum(0)) < 1e-5


def test_projection_group_without_input_grad():
    from neutrongt_amd.linear import project
    _say("case projection group, input without grad")
    mods = [WgradLinear(64, 64).cuda() for _ in range(3)]
    x = torch.randn(700, 64, device="cuda")
    with torch.autocast("cuda", dtype=torch.bfloat16):
        ys = project(x, *mods)
    sum(y.float().sum() for y in ys).backward()
    x16 = x.to(torch.bfloat16).double()
    for m in mods:
        assert relerr(m.weight.grad, torch.ones(700, 64, dtype=torch.float64, device="cuda").T @ x16) < 1e-5


@pytest.mark.parametrize("bias", [True, False])
def test_projection_group_with_interleaved_gradients(bias):
    """Output gradients that are column blocks of one [M, 3 n] matrix (the
    sparse core's interleaved dQ/dK/dV) take the stacked path: dX one GEMM
    against the stacked weights, dW one split-K GEMM, db one column sum --
    dW/db as float64 products, dX as close to the float64 sum as the
    separate path, and both paths' dW/db within fp32 accumulation."""
    from neutrongt_amd.linear import _joint_rows, project
    _say(f"case projection group, interleaved gradients bias={bias}")
    torch.manual_seed(3)
    n_in, n_out, m = 128, 96, 6000
    mods = [WgradLinear(n_in, n_out, bias=bias).cuda() for _ in range(3)]
    x = torch.randn(1, m, n_in, device="cuda", requires_grad=True)
    buf = torch.randn(m, 3, n_out, device="cuda").to(torch.bfloat16)
    gys = [buf[:, i].view(1, m, n_out) for i in range(3)]
    assert _joint_rows(gys, n_out) is not None
    assert _joint_rows([g.clone() for g in gys], n_out) is None  # separate buffers
    with torch.autocast("cuda", dtype=torch.bfloat16):
        ys = project(x, *mods)
    torch.autograd.backward(ys, gys)
    x16 = x.detach().to(torch.bfloat16).reshape(-1, n_in).double()
    g64 = [buf[:, i].double() for i in range(3)]
    exact = sum(g @ mod.weight.detach().to(torch.bfloat16).double() for g, mod in zip(g64, mods))
    assert relerr(x.grad.reshape(-1, n_in), exact) < 8e-3
    for g, mod in zip(g64, mods):
        assert mod.weight.grad.shape == (n_out, n_in) and mod.weight.grad.is_contiguous()
        assert relerr(mod.weight.grad, g.T @ x16) < 1e-5
        if bias:
            assert relerr(mod.bias.grad, g.sum(0)) < 1e-5
        else:
            assert mod.bias is None

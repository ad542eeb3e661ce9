"""GPU tests of WgradLinear (the encoder's nn.Linear with a split-K weight
gradient and the HIP bias gradient ngt_colsum_bf16).

The reference computes these gradients with autograd (fp32 in the reference,
bf16 GEMMs under autocast here); the check is against float64 products of
the same bf16 inputs, where fp32 accumulation is within 1e-5."""
import pytest
import torch
import torch.nn as nn

from neutrongt_amd.linear import WgradLinear, colsum_bf16, weight_grad
from tests._util import relerr

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)


@pytest.mark.parametrize("K,n_out,n_in", [(32768, 768, 768), (1000, 64, 128), (37, 24, 40),
                                          (5000, 1536, 768), (300, 136, 8), (1, 8, 8),
                                          (70001, 128, 256)])
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
    view = base[1:]  # rows start 80 bytes in: not 16-byte aligned -> copied
    assert relerr(colsum_bf16(view), view.double().sum(0)) < 1e-5


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

"""GPU parity of full attention with the reference's optional terms
(attn_bias, pruning_mask, mask; graphormer_dist_node_level.py:51-58) against
the oracle, through the C ABI: output, node scores, dQ/dK/dV and the terms'
gradients, with and without dropout."""
import pytest
import torch

from neutrongt_amd import CoreAttention, dense_attention_bias
from oracle import attention as OA
from tests._util import assert_parity

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)


def _inputs(n_q, n_k, H, d, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    q, go = (torch.randn(n_q, H, d, generator=g).to(dtype) for _ in range(2))
    k, v = (torch.randn(n_k, H, d, generator=g).to(dtype) for _ in range(2))
    ab = torch.randn(1, H, n_q, n_k, generator=g)
    pm = torch.randn(1, 1, n_q, n_k, generator=g) * 0.5  # broadcast over heads
    mask = torch.rand(n_q, n_k, generator=g) < 0.2
    mask[3] = True  # one query with every key masked
    return q, k, v, go, ab, pm, mask


def _run(q, k, v, go, ab, pm, mask, p=0.0, seed=0):
    scale = q.shape[-1] ** 0.5
    qd, kd, vd = (t.cuda().unsqueeze(0).requires_grad_(True) for t in (q, k, v))
    abd = ab.cuda().requires_grad_(True) if ab is not None else None
    pmd = pm.cuda().requires_grad_(True) if pm is not None else None
    x, ns = dense_attention_bias(qd, kd, vd, scale, attn_bias=abd, pruning_mask=pmd,
                                 mask=mask.cuda() if mask is not None else None, dropout_p=p,
                                 seed=seed)
    x.backward(go.cuda())
    torch.cuda.synchronize()
    res = {"x": x.detach().cpu(), "node_scores": ns.cpu(), "dq": qd.grad[0].cpu(),
           "dk": kd.grad[0].cpu(), "dv": vd.grad[0].cpu()}
    if abd is not None:
        res["dbias"] = abd.grad.cpu()
    if pmd is not None:
        res["dpruning"] = pmd.grad.cpu()
    return res


def _check(res, q, k, v, go, ab, pm, mask, dtype, mult=None):
    kw = dict(attn_bias=ab, pruning_mask=pm, mask=mask, dropout_mult=mult)
    ref = OA.full_fwd_bwd(q.float(), k.float(), v.float(), go.float(), **kw)
    ref64 = OA.full_fwd_bwd(q.double(), k.double(), v.double(), go.double(), dtype=torch.float64,
                            **kw)
    for name in res:
        assert res[name].shape == ref[name].shape, (name, res[name].shape, ref[name].shape)
        assert_parity(res[name].float(), ref[name], ref64[name], dtype, name)


@pytest.mark.parametrize("n_q,n_k,H,d,dtype", [
    (60, 60, 2, 8, torch.float32), (45, 70, 4, 16, torch.float32),
    (64, 64, 8, 8, torch.bfloat16), (33, 50, 2, 64, torch.bfloat16)])
def test_dense_bias_pruning_mask_match_oracle(n_q, n_k, H, d, dtype):
    _say(f"case dense bias n_q={n_q} n_k={n_k} H={H} d={d} {dtype}")
    q, k, v, go, ab, pm, mask = _inputs(n_q, n_k, H, d, dtype, seed=n_q + d)
    res = _run(q, k, v, go, ab, pm, mask)
    _check(res, q, k, v, go, ab, pm, mask, dtype)


@pytest.mark.parametrize("which", ["bias", "pruning", "mask"])
def test_dense_each_term_alone(which):
    _say(f"case dense term {which}")
    q, k, v, go, ab, pm, mask = _inputs(40, 52, 2, 16, torch.float32, seed=3)
    ab = ab if which == "bias" else None
    pm = pm if which == "pruning" else None
    mask = mask if which == "mask" else None
    res = _run(q, k, v, go, ab, pm, mask)
    _check(res, q, k, v, go, ab, pm, mask, torch.float32)


def test_dense_bias_with_dropout():
    """The fused kernels' hash mask for the same seed: the oracle with that
    multiplier gives the same output and gradients."""
    _say("case dense bias dropout")
    n, H, d = 50, 2, 8
    q, k, v, go, ab, pm, mask = _inputs(n, n, H, d, torch.float32, seed=4)
    seed = 4321
    res = _run(q, k, v, go, ab, pm, mask, p=0.3, seed=seed)
    mult = OA.dropout_multiplier(seed, H, n, n, 0.3)
    _check(res, q, k, v, go, ab, pm, mask, torch.float32, mult=mult)


def test_core_attention_full_with_optional_terms():
    """CoreAttention.forward(attn_type='full', attn_bias=..., mask=...,
    pruning_mask=...) in eval mode, as the reference's struct_enc path calls it."""
    _say("case dense bias module")
    n, H, d = 48, 4, 8
    q, k, v, go, ab, pm, mask = _inputs(n, n, H, d, torch.float32, seed=5)
    m = CoreAttention(H * d, 0.5, H).cuda().eval()
    qd, kd, vd = (t.cuda().unsqueeze(0).requires_grad_(True) for t in (q, k, v))
    abd = ab.cuda().requires_grad_(True)
    x, score = m(qd, kd, vd, attn_bias=abd, attn_type="full", mask=mask.cuda(),
                 pruning_mask=pm.cuda())
    x.backward(go.reshape(1, n, H * d).cuda())
    ref = OA.full_fwd_bwd(q, k, v, go, attn_bias=ab, pruning_mask=pm, mask=mask)
    ref64 = OA.full_fwd_bwd(q.double(), k.double(), v.double(), go.double(), dtype=torch.float64,
                            attn_bias=ab, pruning_mask=pm, mask=mask)
    assert_parity(x.detach().cpu().view(n, H, d), ref["x"], ref64["x"], torch.float32, "x")
    assert_parity(score.cpu(), ref["node_scores"], ref64["node_scores"], torch.float32, "score")
    assert_parity(abd.grad.cpu(), ref["dbias"], ref64["dbias"], torch.float32, "dbias")
    assert_parity(qd.grad[0].cpu(), ref["dq"], ref64["dq"], torch.float32, "dq")


def test_dense_bias_shape_is_checked():
    q = torch.randn(1, 10, 2, 8, device="cuda")
    with pytest.raises(ValueError):
        dense_attention_bias(q, q, q, 8 ** 0.5, attn_bias=torch.zeros(1, 3, 10, 10, device="cuda"))


def test_dense_bias_under_bf16_autocast():
    """The reference's struct_enc path under torch.autocast(bfloat16), as the
    bf16 window step runs it: the Function computes in fp32 inside (autocast
    off there), so q/k/v in bf16 give the oracle's result on the same
    bf16-rounded inputs."""
    _say("case dense bias under bf16 autocast")
    n, H, d = 40, 4, 16
    q, k, v, go, ab, pm, mask = _inputs(n, n, H, d, torch.bfloat16, seed=6)
    qd, kd, vd = (t.cuda().unsqueeze(0).requires_grad_(True) for t in (q, k, v))
    abd = ab.cuda().requires_grad_(True)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        x, ns = dense_attention_bias(qd, kd, vd, d ** 0.5, attn_bias=abd, pruning_mask=pm.cuda(),
                                     mask=mask.cuda())
    assert x.dtype == torch.bfloat16 and ns.dtype == torch.float32
    x.backward(go.cuda())
    torch.cuda.synchronize()
    res = {"x": x.detach().cpu(), "node_scores": ns.cpu(), "dq": qd.grad[0].cpu(),
           "dk": kd.grad[0].cpu(), "dv": vd.grad[0].cpu(), "dbias": abd.grad.cpu()}
    assert abd.grad.dtype == torch.float32
    _check(res, q, k, v, go, ab, pm, None if mask is None else mask, torch.bfloat16)


@pytest.mark.parametrize("p", [0.0, 0.4])
def test_dense_bias_head_chunks_give_the_one_shot_bits(p):
    """The materialized path run one head at a time, two at a time and all at
    once: every output and gradient is bit-identical."""
    _say(f"case dense bias head chunks p={p}")
    n_q, n_k, H, d = 70, 90, 5, 8
    q, k, v, go, ab, pm, mask = _inputs(n_q, n_k, H, d, torch.float32, seed=7)
    runs = []
    for chunk in (H, 1, 2):
        qd, kd, vd = (t.cuda().unsqueeze(0).requires_grad_(True) for t in (q, k, v))
        abd = ab.cuda().requires_grad_(True)
        x, ns = dense_attention_bias(qd, kd, vd, d ** 0.5, attn_bias=abd, pruning_mask=pm.cuda(),
                                     mask=mask.cuda(), dropout_p=p, seed=99, head_chunk=chunk)
        x.backward(go.cuda())
        torch.cuda.synchronize()
        runs.append([x.detach().cpu(), ns.cpu(), qd.grad.cpu(), kd.grad.cpu(), vd.grad.cpu(),
                     abd.grad.cpu()])
    for other in runs[1:]:
        for a, b, name in zip(runs[0], other, ("x", "ns", "dq", "dk", "dv", "dbias")):
            assert torch.equal(a, b), f"{name} differs between head chunks"
    mult = OA.dropout_multiplier(99, H, n_q, n_k, p) if p else None
    res = dict(zip(("x", "node_scores", "dq", "dk", "dv", "dbias"),
                   [runs[0][0], runs[0][1], runs[0][2][0], runs[0][3][0], runs[0][4][0],
                    runs[0][5]]))
    _check(res, q, k, v, go, ab, pm, mask, torch.float32, mult=mult)


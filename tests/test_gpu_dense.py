"""GPU parity of the dense full-window attention (forward + backward)."""
import math
from pathlib import Path

import numpy as np
import pytest
import torch

from neutrongt_amd import CoreAttention, dense_attention
from neutrongt_amd import synthetic as S
from oracle import attention as OA
from tests._util import TOL, assert_close, assert_parity, relerr

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)


def _run(q, k, v, go):
    qd, kd, vd = (t.cuda().requires_grad_(True) for t in (q, k, v))
    x, ns = dense_attention(qd, kd, vd)
    x.backward(go.cuda())
    torch.cuda.synchronize()
    return {"x": x.detach().cpu(), "node_scores": ns.cpu(), "dq": qd.grad.cpu(),
            "dk": kd.grad.cpu(), "dv": vd.grad.cpu()}


def _qkv(n_q, n_k, H, d, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    return tuple(torch.randn(n, H, d, generator=g).to(dtype) for n in (n_q, n_k, n_k, n_q))


@pytest.mark.parametrize("n_q,n_k,H,d,dtype", [
    (70, 70, 2, 8, torch.float32), (130, 90, 3, 16, torch.float32), (64, 200, 2, 24, torch.float32),
    (50, 77, 1, 32, torch.float32), (40, 40, 2, 64, torch.float32),
    (100, 100, 8, 8, torch.bfloat16), (96, 150, 4, 16, torch.bfloat16),
    (60, 61, 2, 24, torch.bfloat16), (70, 45, 3, 32, torch.bfloat16),
    (33, 47, 2, 64, torch.bfloat16), (1, 1, 1, 8, torch.bfloat16), (130, 33, 2, 8, torch.bfloat16),
    # long key ranges: the vector-ALU forward splits the keys over blocks
    # (5, 4, 2 and 3 splits, last one ragged) and combines the splits
    (100, 3000, 2, 8, torch.float32), (37, 2100, 1, 24, torch.float32),
    (64, 1300, 3, 64, torch.float32), (50, 1800, 2, 64, torch.bfloat16)])
def test_dense_parity(n_q, n_k, H, d, dtype):
    _say(f"case dense n_q={n_q} n_k={n_k} H={H} d={d} {dtype}")
    q, k, v, go = _qkv(n_q, n_k, H, d, dtype, seed=n_q + d)
    res = _run(q, k, v, go)
    ref = OA.full_fwd_bwd(q.float(), k.float(), v.float(), go.float())
    ref64 = OA.full_fwd_bwd(q.double(), k.double(), v.double(), go.double(), dtype=torch.float64)
    for name in ("x", "node_scores", "dq", "dk", "dv"):
        assert res[name].shape == ref[name].shape
        assert_parity(res[name].float(), ref[name], ref64[name], dtype, name)


@pytest.mark.parametrize("d", [8, 16, 24, 32])
@pytest.mark.parametrize("fwd_split,dq_split,p", [(2, 3, 0.0), (3, 2, 0.5), (4, 4, 0.0)])
def test_dense_mfma_key_splits(monkeypatch, d, fwd_split, dq_split, p):
    """bf16 matrix-core kernels with the keys split over blocks (forward states
    merged by the combine, dQ partials added in split order), a ragged last
    split, with and without dropout, against the restatement."""
    _say(f"case dense mfma splits d={d} fwd={fwd_split} dq={dq_split} p={p}")
    monkeypatch.setenv("NGT_MF_FWD_SPLIT", str(fwd_split))
    monkeypatch.setenv("NGT_MF_DQ_SPLIT", str(dq_split))
    n_q, n_k, H = 200, 2100, 2
    q, k, v, go = _qkv(n_q, n_k, H, d, torch.bfloat16, seed=d + fwd_split)
    seed = 0xABCD + d
    res = _run_drop(q, k, v, go, p, seed) if p else _run(q, k, v, go)
    mult = OA.dropout_multiplier(seed, H, n_q, n_k, p) if p else None
    ref = OA.full_fwd_bwd(q.float(), k.float(), v.float(), go.float(), dropout_mult=mult)
    ref64 = OA.full_fwd_bwd(q.double(), k.double(), v.double(), go.double(), dtype=torch.float64,
                            dropout_mult=mult)
    for name in ("x", "dq", "dk", "dv") + (("node_scores",) if not p else ()):
        assert_parity(res[name].float(), ref[name], ref64[name], torch.bfloat16, f"split {name}")


@pytest.mark.parametrize("d", [8, 16, 24, 32])
@pytest.mark.parametrize("n_q,n_k,H,p", [(300, 300, 2, 0.0), (77, 1000, 3, 0.0),
                                         (200, 129, 1, 0.5), (1030, 260, 2, 0.3)])
def test_dense_single_pass_backward(monkeypatch, d, n_q, n_k, H, p):
    """The single-pass backward (NGT_DENSE_FUSED=1: dK/dV key-major with each
    tile's dS also contracted into per-block partial dQ, summed over the key
    blocks in order): ragged query stages and key blocks, with and without
    dropout, against the restatement; and bitwise reproducible."""
    _say(f"case dense single pass d={d} n_q={n_q} n_k={n_k} H={H} p={p}")
    monkeypatch.setenv("NGT_DENSE_FUSED", "1")
    q, k, v, go = _qkv(n_q, n_k, H, d, torch.bfloat16, seed=d + n_q)
    seed = 0x5EED + d
    run = (lambda: _run_drop(q, k, v, go, p, seed)) if p else (lambda: _run(q, k, v, go))
    res = run()
    mult = OA.dropout_multiplier(seed, H, n_q, n_k, p) if p else None
    ref = OA.full_fwd_bwd(q.float(), k.float(), v.float(), go.float(), dropout_mult=mult)
    ref64 = OA.full_fwd_bwd(q.double(), k.double(), v.double(), go.double(), dtype=torch.float64,
                            dropout_mult=mult)
    for name in ("x", "dq", "dk", "dv"):
        assert_parity(res[name].float(), ref[name], ref64[name], torch.bfloat16, f"fused {name}")
    again = run()
    for name in ("dq", "dk", "dv"):
        assert torch.equal(res[name], again[name]), name


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("n_q,n_k", [(0, 37), (45, 0)])
def test_dense_empty_side(n_q, n_k, dtype):
    """A window without queries or without keys: the empty softmax axis and
    P @ V give zeros (the oracle's torch ops, as the reference's): node scores
    0 over the keys and dK = dV = 0, or out = 0 and dQ = 0."""
    _say(f"case dense empty n_q={n_q} n_k={n_k} {dtype}")
    q, k, v, go = _qkv(n_q, n_k, 2, 8, dtype, seed=5)
    res = _run(q, k, v, go)
    ref = OA.full_fwd_bwd(q.float(), k.float(), v.float(), go.float())
    for name in ("x", "node_scores", "dq", "dk", "dv"):
        assert res[name].shape == ref[name].shape, name
        assert torch.equal(res[name].float(), ref[name]), name


def test_dense_golden():
    for f in sorted((Path(__file__).parent / "golden").glob("attn_dense_*.npz")):
        _say(f"case golden {f.name}")
        z = np.load(f)
        q, k, v, go = (torch.from_numpy(z[n]) for n in ("q", "k", "v", "go"))
        res = _run(q, k, v, go)
        for name in ("x", "node_scores", "dq", "dk", "dv"):
            assert_close(res[name], torch.from_numpy(z[name]), torch.float32, f"{f.name}:{name}")


def test_dense_module_drop_in():
    _say("case dense module")
    H, d, n = 2, 8, 50
    mod = CoreAttention(H * d, 0.0, H).cuda()
    q, k, v, go = _qkv(n, n, H, d, torch.float32, seed=5)
    x, score = mod(q[None].cuda(), k[None].cuda(), v[None].cuda(), None, None, "full")
    assert x.shape == (1, n, H * d)
    ref = OA.full_fwd_bwd(q, k, v, go)
    assert_close(x[0].view(n, H, d).cpu(), ref["x"], torch.float32, "x")
    assert_close(score.cpu(), ref["node_scores"], torch.float32, "score")


@pytest.mark.parametrize("fused", ["0", "1"])
def test_dense_full_size_sampled_rows_and_invariants(monkeypatch, fused):
    """16,000-node all-pairs window (H=8, d=8, bf16): sampled query rows and
    sampled key rows (dK, dV) against float64 formulas, column scores against a
    chunked CPU sum, and the size-independent identities <dQ,Q> = <dK,K>,
    sum_j dV_j = sum_i G_i; with the two-pass and the single-pass backward."""
    monkeypatch.setenv("NGT_DENSE_FUSED", fused)
    cfg = S.CONFIGS["dense_slim"]
    _say(f"case dense full-size n={cfg.n_q} fused={fused}")
    q, k, v, go = S.make_qkv(cfg, cfg.n_q)
    res = _run(q, k, v, go)
    n, H, d = cfg.n_q, cfg.n_heads, cfg.head_dim
    sc = math.sqrt(d)
    qd, kd, vd, gd = (t.double() for t in (q, k, v, go))
    rows = np.random.default_rng(1).choice(n, 48, replace=False)
    for h in range(H):
        s = (qd[rows, h] * sc) @ kd[:, h].T  # [48, n]
        p = torch.softmax(s, -1)
        x = p @ vd[:, h]
        dp = gd[rows, h] @ vd[:, h].T
        dd = (gd[rows, h] * x).sum(-1, keepdim=True)
        dq = sc * (p * (dp - dd)) @ kd[:, h]
        assert relerr(res["x"][rows, h], x) < TOL[cfg.dtype]
        assert relerr(res["dq"][rows, h], dq) < TOL[cfg.dtype]
    # dK / dV of sampled key rows (and the first and last key), elementwise:
    # a key column sums over every query, so each query row's softmax and
    # D_i = G_i . X_i are formed in float64, 2,000 rows at a time; the same
    # pass accumulates the column scores.
    keys = np.unique(np.concatenate([np.random.default_rng(2).choice(n, 48, replace=False),
                                     [0, n - 1]]))
    kt = torch.from_numpy(keys)
    ns = torch.zeros(n, dtype=torch.float64)
    dk = torch.zeros(keys.size, H, d, dtype=torch.float64)
    dv = torch.zeros(keys.size, H, d, dtype=torch.float64)
    for h in range(H):
        for c in range(0, n, 2000):
            s = (qd[c:c + 2000, h] * sc) @ kd[:, h].T  # [2000, n]
            ns += s.abs().sum(0)
            p = torch.softmax(s, -1)
            x = p @ vd[:, h]
            dd = (gd[c:c + 2000, h] * x).sum(-1, keepdim=True)
            pc = p[:, kt]
            ds = pc * (gd[c:c + 2000, h] @ vd[kt, h].T - dd)
            dk[:, h] += sc * ds.T @ qd[c:c + 2000, h]
            dv[:, h] += pc.T @ gd[c:c + 2000, h]
    ns /= H
    assert relerr(res["node_scores"], ns) < TOL[cfg.dtype]
    assert_close(res["dk"][kt].float(), dk, cfg.dtype, "dense dk keys")
    assert_close(res["dv"][kt].float(), dv, cfg.dtype, "dense dv keys")
    lhs = (res["dq"].double() * qd).sum().item()
    rhs = (res["dk"].double() * kd).sum().item()
    assert abs(lhs - rhs) / max(abs(lhs), abs(rhs)) < 10 * TOL[cfg.dtype]
    assert relerr(res["dv"].double().sum(0), gd.sum(0)) < 10 * TOL[cfg.dtype]


def _run_drop(q, k, v, go, p, seed, flash=False):
    qd, kd, vd = (t.cuda().requires_grad_(True) for t in (q, k, v))
    d = q.shape[-1]
    x, ns = dense_attention(qd, kd, vd, scale=1.0 / math.sqrt(d) if flash else None,
                            node_scores=not flash, dropout_p=p, seed=seed)
    x.backward(go.cuda())
    torch.cuda.synchronize()
    return {"x": x.detach().cpu(), "node_scores": ns.cpu(), "dq": qd.grad.cpu(),
            "dk": kd.grad.cpu(), "dv": vd.grad.cpu()}


@pytest.mark.parametrize("n_q,n_k,H,d,dtype,p", [
    (70, 71, 2, 8, torch.float32, 0.5), (64, 130, 2, 16, torch.float32, 0.3),
    (40, 40, 2, 64, torch.float32, 0.5), (100, 99, 4, 8, torch.bfloat16, 0.5),
    (96, 150, 2, 16, torch.bfloat16, 0.2), (60, 61, 2, 24, torch.bfloat16, 0.5),
    (70, 45, 3, 32, torch.bfloat16, 0.7), (33, 47, 2, 64, torch.bfloat16, 0.5),
    (50, 50, 2, 8, torch.bfloat16, 1.0), (70, 2500, 2, 16, torch.float32, 0.5)])
def test_dense_dropout_parity(n_q, n_k, H, d, dtype, p):
    """Training-mode dropout on P: the kernels' mask equals the oracle's
    (same seed), and out / dQ / dK / dV match the restatement with that mask."""
    _say(f"case dense dropout n_q={n_q} n_k={n_k} H={H} d={d} {dtype} p={p}")
    seed = 0x1234_5678_9ABC + n_q
    q, k, v, go = _qkv(n_q, n_k, H, d, dtype, seed=n_q + 3 * d)
    res = _run_drop(q, k, v, go, p, seed)
    mult = OA.dropout_multiplier(seed, H, n_q, n_k, p)
    ref = OA.full_fwd_bwd(q.float(), k.float(), v.float(), go.float(), dropout_mult=mult)
    ref64 = OA.full_fwd_bwd(q.double(), k.double(), v.double(), go.double(),
                            dtype=torch.float64, dropout_mult=mult)
    for name in ("x", "node_scores", "dq", "dk", "dv"):
        assert_parity(res[name].float(), ref[name], ref64[name], dtype, f"p={p} {name}")
    again = _run_drop(q, k, v, go, p, seed)
    for name in ("x", "dq", "dk", "dv"):
        assert torch.equal(again[name], res[name]), f"{name} not reproducible"


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_dense_dropout_mask_from_output(dtype):
    """The kept set read off the output itself: with V = identity rows
    (n_k = d) and P replaced by exact one-hot-free values, out[i, h, j] =
    P[h,i,j] * mult[h,i,j], so the zero pattern of out is the mask."""
    _say(f"case dense dropout mask {dtype}")
    H, d, n_q = 2, 16, 64
    n_k = d
    g = torch.Generator().manual_seed(11)
    q = torch.randn(n_q, H, d, generator=g).to(dtype) * 0.1
    k = torch.randn(n_k, H, d, generator=g).to(dtype) * 0.1
    v = torch.eye(d).unsqueeze(1).repeat(1, H, 1).to(dtype)  # v[j, h] = e_j
    seed = 987654321
    x, _ = dense_attention(q.cuda(), k.cuda(), v.cuda(), dropout_p=0.5, seed=seed)
    mult = OA.dropout_multiplier(seed, H, n_q, n_k, 0.5)
    kept = x.float().cpu().permute(1, 0, 2).numpy() != 0  # [H, n_q, n_k]
    assert np.array_equal(kept, mult > 0)


def test_dense_module_dropout_and_flash():
    """CoreAttention in training mode draws its seed on the device from torch's
    generator (torch.manual_seed makes it repeatable), eval mode has no
    dropout, and the flash branch (1/sqrt(d) scale, dropout always on) matches
    naive_attention."""
    _say("case dense module dropout/flash")
    H, d, n = 2, 8, 50
    mod = CoreAttention(H * d, 0.5, H).cuda()
    q, k, v, go = _qkv(n, n, H, d, torch.float32, seed=5)
    args = (q[None].cuda(), k[None].cuda(), v[None].cuda(), None, None, "full")
    mod.eval()
    x_eval, _ = mod(*args)
    ref = OA.full_fwd_bwd(q, k, v, go)
    assert_close(x_eval[0].view(n, H, d).cpu(), ref["x"], torch.float32, "eval x")
    mod.train()
    torch.manual_seed(77)
    x1, s1 = mod(*args)
    torch.manual_seed(77)
    seed = int(torch.randint(0, 2**62, (1,), dtype=torch.int64, device="cuda").item())
    torch.manual_seed(77)
    x2, _ = mod(*args)
    assert torch.equal(x1, x2)
    mult = OA.dropout_multiplier(seed, H, n, n, 0.5)
    ref = OA.full_fwd_bwd(q, k, v, go, dropout_mult=mult)
    assert_close(x1[0].view(n, H, d).cpu(), ref["x"], torch.float32, "train x")
    assert_close(s1.cpu(), ref["node_scores"], torch.float32, "train score")
    # flash branch: the reference's fp16 casts (graphormer_dist_node_level.py:111-122)
    torch.manual_seed(78)
    xf, sf = mod(q[None].cuda(), k[None].cuda(), v[None].cuda(), None, None, "flash")
    assert sf is None and xf.dtype == torch.float32 and xf.shape == (1, n, H * d)
    torch.manual_seed(78)
    seed = int(torch.randint(0, 2**62, (1,), dtype=torch.int64, device="cuda").item())
    mult = OA.dropout_multiplier(seed, H, n, n, 0.5)
    ref = OA.full_fwd_bwd(q, k, v, go, dropout_mult=mult, flash=True, flash_half=True)
    # fp16 arithmetic in the reference: every intermediate is rounded to fp16
    # (unit roundoff 2^-11 = 4.9e-4); the kernels keep them in fp32
    assert relerr(xf[0].view(n, H, d).cpu(), ref["x"]) < 2e-3
    assert torch.equal(xf, xf.half().float())  # the output is fp16-rounded


def test_flash_branch_rounds_inputs_and_gradients_to_fp16():
    """The flash branch casts q/k/v to fp16 as the reference does: inputs
    that differ below fp16's precision give the same bits, the output is
    fp16-valued, and forward and gradients stay within fp16 rounding of the
    reference's fp16 arithmetic (restated on the CPU in fp16)."""
    _say("case flash fp16")
    H, d, n_q, n_k = 2, 16, 45, 60
    q, k, v, go = _qkv(n_q, n_k, H, d, torch.float32, seed=19)
    q, k, v = (t.half().float() for t in (q, k, v))  # fp16 values
    mod = CoreAttention(H * d, 0.5, H).cuda().train()
    # (1 + 2^-14) times an fp16 value is no fp16 value but rounds back to it:
    # 2^-14 is below half of fp16's relative spacing (2^-11 at least)
    outs = []
    for bump in (0.0, 2.0 ** -14):
        qd, kd, vd = ((t * (1 + bump)).cuda()[None].requires_grad_(True) for t in (q, k, v))
        torch.manual_seed(81)
        x, _ = mod(qd, kd, vd, None, None, "flash")
        x.backward(go.reshape(1, n_q, H * d).cuda())
        torch.cuda.synchronize()
        outs.append([x.detach().cpu(), qd.grad.cpu(), kd.grad.cpu(), vd.grad.cpu()])
    for a, b in zip(*outs):
        assert torch.equal(a, b)
    x, dq, dk, dv = outs[0]
    assert torch.equal(x, x.half().float())
    for gr in (dq, dk, dv):  # the gradients pass through the fp16 cast too
        assert torch.equal(gr, gr.half().float())
    torch.manual_seed(81)
    seed = int(torch.randint(0, 2**62, (1,), dtype=torch.int64, device="cuda").item())
    mult = OA.dropout_multiplier(seed, H, n_q, n_k, 0.5)
    ref = OA.full_fwd_bwd(q, k, v, go, dropout_mult=mult, flash=True, flash_half=True)
    got = {"x": x[0].view(n_q, H, d), "dq": dq[0], "dk": dk[0], "dv": dv[0]}
    for name, t in got.items():
        e = relerr(t, ref[name])
        assert e < 2e-3, (name, e)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_dense_flash_backward(dtype):
    _say(f"case dense flash backward {dtype}")
    H, d, n_q, n_k = 2, 16, 45, 60
    q, k, v, go = _qkv(n_q, n_k, H, d, dtype, seed=9)
    seed = 555
    res = _run_drop(q, k, v, go, 0.5, seed, flash=True)
    mult = OA.dropout_multiplier(seed, H, n_q, n_k, 0.5)
    ref = OA.full_fwd_bwd(q.float(), k.float(), v.float(), go.float(), dropout_mult=mult,
                          flash=True)
    ref64 = OA.full_fwd_bwd(q.double(), k.double(), v.double(), go.double(),
                            dtype=torch.float64, dropout_mult=mult, flash=True)
    for name in ("x", "dq", "dk", "dv"):
        assert_parity(res[name].float(), ref[name], ref64[name], dtype, f"flash {name}")


def test_flash_branch_gt_twin_layout():
    """flash_layout='gt_twin' views the [b, H, N, d] result as [b, N, H*d]
    without transposing back (gt_dist_node_level_single_window.py:212-225);
    install() picks it for a module of that file."""
    _say("case flash gt twin layout")
    H, d, n = 2, 8, 40
    q, k, v, go = _qkv(n, n, H, d, torch.float32, seed=11)
    args = (q[None].cuda(), k[None].cuda(), v[None].cuda(), None, None, "flash")
    torch.manual_seed(79)
    xg, _ = CoreAttention(H * d, 0.5, H).cuda()(*args)
    torch.manual_seed(79)
    xt, _ = CoreAttention(H * d, 0.5, H, flash_layout="gt_twin").cuda()(*args)
    # the same numbers in the reference twin's memory order
    want = xg.view(1, n, H, d).transpose(1, 2).contiguous().view(1, n, H * d)
    assert torch.equal(xt, want) and not torch.equal(xt, xg)
    with pytest.raises(ValueError):
        CoreAttention(H * d, 0.5, H, flash_layout="other")

    class TwinCore(torch.nn.Module):  # shaped like the twin's CoreAttention
        def __init__(self):
            super().__init__()
            self.hidden_size_per_attention_head, self.num_heads = d, H
            self.attention_dropout_rate = 0.5

    TwinCore.__module__ = "NeutronGT.models.gt_dist_node_level_single_window"

    class Holder(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.local_attn = TwinCore()

    from neutrongt_amd import install
    h = Holder()
    assert install(h) == 1 and h.local_attn.flash_layout == "gt_twin"


def _abi_fwd_bwd(q, k, v, go, keep_f32):
    """ngt_dense_fwd / ngt_dense_bwd through the C ABI, bf16, no node scores.
    keep_f32: the forward writes an fp32 copy of the output and the backward
    takes D = G . o from it; otherwise the backward gets the bf16 output only."""
    import ctypes as C

    from neutrongt_amd import _lib
    lib = _lib.load()
    qd, kd, vd, gd = (t.cuda().contiguous() for t in (q, k, v, go))
    n_q, H, d = q.shape
    n_k = k.shape[0]
    scale = float(d) ** 0.5
    st = _lib.stream_ptr(qd.device)
    out = torch.empty_like(qd)
    out32 = torch.empty(n_q, H, d, dtype=torch.float32, device="cuda") if keep_f32 else None
    lse = torch.empty(H, n_q, dtype=torch.float32, device="cuda")
    fb, bb = C.c_size_t(), C.c_size_t()
    _lib.check(lib.ngt_dense_workspace_bytes(_lib.NGT_BF16, n_q, n_k, H, d, 0, C.byref(fb),
                                             C.byref(bb)))
    wf = torch.empty(max(fb.value, 1), dtype=torch.uint8, device="cuda")
    wb = torch.empty(max(bb.value, 1), dtype=torch.uint8, device="cuda")
    _lib.check(lib.ngt_dense_fwd(_lib.NGT_BF16, qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), n_q,
                                 n_k, H, d, scale, 0.0, 0, None, out.data_ptr(),
                                 out32.data_ptr() if keep_f32 else None, lse.data_ptr(), None,
                                 wf.data_ptr(), fb.value, st))
    gq, gk, gv = torch.empty_like(qd), torch.empty_like(kd), torch.empty_like(vd)
    _lib.check(lib.ngt_dense_bwd(_lib.NGT_BF16, qd.data_ptr(), kd.data_ptr(), vd.data_ptr(),
                                 None if keep_f32 else out.data_ptr(),
                                 out32.data_ptr() if keep_f32 else None, gd.data_ptr(),
                                 lse.data_ptr(), n_q, n_k, H, d, scale, 0.0, 0, None,
                                 gq.data_ptr(), gk.data_ptr(), gv.data_ptr(), wb.data_ptr(),
                                 bb.value, st))
    torch.cuda.synchronize()
    return {"x": out.cpu(), "dq": gq.cpu(), "dk": gk.cpu(), "dv": gv.cpu()}


@pytest.mark.parametrize("n_q,n_k,H,d", [(300, 2100, 4, 16), (130, 97, 2, 8), (64, 1500, 3, 32)])
def test_dense_bf16_backward_from_the_bf16_output(n_q, n_k, H, d):
    """The matrix-core dQ pass forms D = G . o itself: from the forward's fp32
    copy of the output when the caller kept one, else from the bf16 output
    (the C ABI allows either).  Both against the restatement; the long key
    ranges run the forward's and the dQ pass's key splits, the latter merged
    by extra blocks of the dK/dV launch."""
    _say(f"case dense bf16 D from bf16 out n_q={n_q} n_k={n_k} H={H} d={d}")
    q, k, v, go = _qkv(n_q, n_k, H, d, torch.bfloat16, seed=n_k + d)
    ref = OA.full_fwd_bwd(q.float(), k.float(), v.float(), go.float())
    ref64 = OA.full_fwd_bwd(q.double(), k.double(), v.double(), go.double(), dtype=torch.float64)
    for keep in (True, False):
        res = _abi_fwd_bwd(q, k, v, go, keep)
        for name in ("x", "dq", "dk", "dv"):
            assert_parity(res[name].float(), ref[name], ref64[name], torch.bfloat16,
                          f"{name} keep_f32={keep}")

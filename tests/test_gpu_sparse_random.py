"""A seeded sweep of random sparse windows against the oracle: sizes, head
counts (1 .. 64), head dims, dtypes, chunk and packing thresholds, hub rows on
either side, duplicate and empty rows, related keys from a second buffer, the
recomputed dQ, and the interleaved gradient hand-over -- combinations the
targeted tests cover one axis at a time.  Every case is drawn from a fixed
seed, so a failure names a reproducible window."""
import numpy as np
import pytest
import torch

from neutrongt_amd import SparseAttentionFunction, WindowAdjacency
from oracle import attention as OA
from tests._util import TOL, assert_close, assert_parity

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)


def _cases(n, seed, max_q=700, max_deg=8):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        H = int(rng.choice([1, 2, 3, 4, 5, 8, 12, 16, 32, 64]))
        d = int(rng.choice([8, 16, 24, 32, 64]))
        if H * d > 1536:  # keep the oracle quick
            d = 8 if H >= 64 else 24
        dtype = "bf16" if rng.random() < 0.5 else "f32"
        n_q = int(rng.integers(1, max_q))
        interleave = bool(rng.random() < 0.3)
        n_main = n_q if interleave else n_q + int(rng.integers(0, 400))
        n_ext = int(rng.integers(1, 300)) if rng.random() < 0.35 else 0
        chunk = int(rng.choice([7, 16, 64, 128, 256]))
        small = int(rng.integers(0, chunk))
        out.append(dict(i=f"{seed % 1000}_{i}", H=H, d=d, dtype=dtype, n_q=n_q, n_main=n_main, n_ext=n_ext,
                        E=int(rng.integers(0, max_deg * n_q + 1)), hub_q=int(rng.choice([0, 0, 300, 3000])),
                        hub_k=int(rng.choice([0, 0, 200, 2000])), chunk=chunk, small=small,
                        recompute=bool(rng.random() < 0.3), interleave=interleave,
                        seed=int(rng.integers(1 << 30))))
    return out


# small windows, many of them; then fewer, larger and denser ones
CASES = _cases(160, 20261202) + _cases(24, 77, max_q=3000, max_deg=24)


@pytest.mark.parametrize("c", CASES, ids=lambda c: f"case{c['i']}")
def test_random_window_matches_oracle(monkeypatch, c):
    _say(f"case {c}")
    monkeypatch.setenv("NGT_DQ_RECOMPUTE", "1" if c["recompute"] else "0")
    rng = np.random.default_rng(c["seed"])
    n_q, n_k = c["n_q"], c["n_main"] + c["n_ext"]
    src = [rng.integers(0, n_k, c["E"])]
    dst = [rng.integers(0, n_q, c["E"])]
    if c["hub_q"]:  # one query row with many keys (split into chunks)
        src.append(rng.integers(0, n_k, c["hub_q"]))
        dst.append(np.full(c["hub_q"], int(rng.integers(0, n_q))))
    if c["hub_k"]:  # one key row with many queries, possibly a related key
        src.append(np.full(c["hub_k"], int(rng.integers(0, n_k))))
        dst.append(rng.integers(0, n_q, c["hub_k"]))
    ei = np.stack([np.concatenate(src), np.concatenate(dst)]).astype(np.int64)
    dtype = torch.bfloat16 if c["dtype"] == "bf16" else torch.float32
    g = torch.Generator().manual_seed(c["seed"])
    H, d = c["H"], c["d"]
    q = torch.randn(n_q, H, d, generator=g).to(dtype)
    k = (1.5 * torch.randn(n_k, H, d, generator=g)).to(dtype)
    v = torch.randn(n_k, H, d, generator=g).to(dtype)
    go = torch.randn(n_q, H, d, generator=g).to(dtype)
    ref = OA.sparse_fwd_bwd(q.float(), k.float(), v.float(), torch.from_numpy(ei), go.float(), H,
                            dtype=torch.float32)
    n_main = c["n_main"]
    qd = q.cuda().requires_grad_(True)
    kd = k[:n_main].cuda().requires_grad_(True)
    vd = v[:n_main].cuda().requires_grad_(True)
    ext = (k[n_main:].cuda(), v[n_main:].cuda()) if c["n_ext"] else (None, None)
    adj = WindowAdjacency(torch.from_numpy(ei).cuda(), n_q, n_k, c["chunk"], c["small"],
                          tiled=False)
    x, ns = SparseAttentionFunction.apply(qd, kd, vd, adj, float(d) ** 0.5, -5.0, 5.0, 1e-6,
                                          ext[0], ext[1], c["interleave"])
    x.backward(go.cuda())
    torch.cuda.synchronize()
    got = {"x": x.detach().cpu(), "node_scores": ns.cpu(), "dq": qd.grad.cpu(),
           "dk": kd.grad.cpu(), "dv": vd.grad.cpu()}
    ref64 = OA.sparse_fwd_bwd(q.double(), k.double(), v.double(), torch.from_numpy(ei),
                              go.double(), H, dtype=torch.float64)
    for r in (ref, ref64):
        r["dk"], r["dv"] = r["dk"][:n_main], r["dv"][:n_main]
    for name in ("x", "node_scores"):
        assert got[name].shape == ref[name].shape, (name, got[name].shape, ref[name].shape)
        assert_close(got[name].float(), ref[name].float(), dtype, f"case{c['i']} {name}")
    # Gradient scales: |dS| <= |p| |dP - D| with p <= 1, so dQ and dK are
    # bounded by |dO| |V| |K| / sqrt(d) and |dO| |V| |Q| / sqrt(d) per edge
    # (up to the degree), dV by |dO|.  A window whose rows each have one edge
    # has dQ = dK = 0 exactly (p = 1, dP = D): there both implementations'
    # results are rounding noise, and only their absolute size is checked.
    mx = lambda t: float(t.abs().max()) if t.numel() else 0.0
    scale = {"dq": mx(go) * mx(v) * mx(k) / d ** 0.5, "dk": mx(go) * mx(v) * mx(q) / d ** 0.5,
             "dv": mx(go)}
    for name in ("dq", "dk", "dv"):
        assert got[name].shape == ref[name].shape, (name, got[name].shape, ref[name].shape)
        if mx(ref64[name]) >= 1e-3 * scale[name]:
            assert_parity(got[name].float(), ref[name].float(), ref64[name], dtype,
                          f"case{c['i']} {name}")
        else:
            worst = mx(got[name].double() - ref64[name])
            assert worst <= TOL[dtype] * scale[name], (name, worst, scale[name])

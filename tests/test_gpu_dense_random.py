"""A seeded sweep of random dense windows against the oracle (the
reference's full_attention: logits q k^T sqrt(d)): sizes from 1 to 2,500
keys, 1 to 8 heads, every head dim, fp32 (vector-ALU kernels) and bf16
(matrix-core kernels for d <= 32, vector-ALU at 64), input scales that make
the softmax peaked or flat, dropout, key splits, and the single-pass
backward.  Every case is drawn from a fixed seed."""
import math

import numpy as np
import pytest
import torch

from neutrongt_amd import dense_attention
from oracle import attention as OA
from tests._util import assert_parity

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)


def _cases(n=100, seed=4242):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        d = int(rng.choice([8, 16, 24, 32, 64]))
        dtype = "bf16" if rng.random() < 0.6 else "f32"
        n_k = int(rng.integers(1, 2500))
        fused = dtype == "bf16" and d <= 32 and n_k >= 128 and rng.random() < 0.4
        out.append(dict(i=i, H=int(rng.choice([1, 2, 3, 8])), d=d, dtype=dtype,
                        n_q=int(rng.integers(1, 400)), n_k=n_k,
                        qscale=float(rng.choice([1.0, 0.25, 0.05])),
                        p=float(rng.choice([0.0, 0.0, 0.3])),
                        fwd_split=int(rng.choice([0, 0, 2, 3])), dq_split=int(rng.choice([0, 0, 2])),
                        fused=bool(fused), seed=int(rng.integers(1 << 30))))
    return out


@pytest.mark.parametrize("c", _cases(), ids=lambda c: f"case{c['i']}")
def test_random_dense_window_matches_oracle(monkeypatch, c):
    _say(f"case {c}")
    monkeypatch.setenv("NGT_DENSE_FUSED", "1" if c["fused"] else "0")
    if c["fwd_split"]:
        monkeypatch.setenv("NGT_MF_FWD_SPLIT", str(c["fwd_split"]))
    if c["dq_split"]:
        monkeypatch.setenv("NGT_MF_DQ_SPLIT", str(c["dq_split"]))
    dtype = torch.bfloat16 if c["dtype"] == "bf16" else torch.float32
    g = torch.Generator().manual_seed(c["seed"])
    H, d, n_q, n_k, p = c["H"], c["d"], c["n_q"], c["n_k"], c["p"]
    q = (c["qscale"] * torch.randn(n_q, H, d, generator=g)).to(dtype)
    k, v = (torch.randn(n_k, H, d, generator=g).to(dtype) for _ in range(2))
    go = torch.randn(n_q, H, d, generator=g).to(dtype)
    seed = c["seed"] & 0xFFFFFF
    qd, kd, vd = (t.cuda().requires_grad_(True) for t in (q, k, v))
    x, ns = dense_attention(qd, kd, vd, dropout_p=p, seed=seed if p else None)
    x.backward(go.cuda())
    torch.cuda.synchronize()
    got = {"x": x.detach().cpu(), "node_scores": ns.cpu(), "dq": qd.grad.cpu(),
           "dk": kd.grad.cpu(), "dv": vd.grad.cpu()}
    mult = OA.dropout_multiplier(seed, H, n_q, n_k, p) if p else None
    ref = OA.full_fwd_bwd(q.float(), k.float(), v.float(), go.float(), dropout_mult=mult)
    ref64 = OA.full_fwd_bwd(q.double(), k.double(), v.double(), go.double(), dtype=torch.float64,
                            dropout_mult=mult)
    names = ("x", "dq", "dk", "dv") + (("node_scores",) if not p else ())
    for name in names:
        assert got[name].shape == ref[name].shape, (name, got[name].shape, ref[name].shape)
        assert_parity(got[name].float(), ref[name], ref64[name], dtype, f"case{c['i']} {name}")

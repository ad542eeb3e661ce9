"""GPU parity of the window preparation kernels (bit-exact integer work)."""
from pathlib import Path

import numpy as np
import pytest
import torch

from neutrongt_amd import window as W
from oracle import graph as OG

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).parent / "golden"


def _say(*a):
    print(*a, flush=True)


def _gpu_related(xadj, adjncy, ew, part, pct):
    t = lambda a, dt: torch.as_tensor(np.asarray(a), dtype=dt).cuda()
    out = W.merge_related_nodes(t(xadj, torch.int32), t(adjncy, torch.int32), t(ew, torch.int32),
                                t(part, torch.int64), pct)
    return out.cpu().numpy()


def test_related_nodes_golden():
    _say("case related golden")
    z = np.load(GOLDEN / "related_small.npz")
    for pct in (0, 25, 50, 60, 100):
        got = _gpu_related(z["xadj"], z["adjncy"], z["eweights"], z["partition"], pct)
        np.testing.assert_array_equal(got, z[f"out_{pct}"])


@pytest.mark.parametrize("n,E,n_part,seed", [(300, 3000, 50, 0), (2000, 30000, 400, 1),
                                             (50000, 400000, 3000, 2)])
def test_related_nodes_match_oracle(n, E, n_part, seed):
    _say(f"case related n={n} E={E} part={n_part}")
    rng = np.random.default_rng(seed)
    ei = rng.integers(0, n, (2, E))
    val = rng.integers(1, 5, E).astype(np.float32) / 1000  # many ties
    xadj, adjncy, ew = OG.adj_weights(ei, val)
    part = rng.permutation(int(xadj.shape[0]) - 1)[:n_part]
    for pct in (0, 8, 33, 100):
        want, _ = OG.merge_related_nodes(xadj, adjncy, ew, part, pct)
        got = _gpu_related(xadj, adjncy, ew, part, pct)
        np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("n,E,dup", [(500, 5000, 1), (60, 400, 1), (300, 20000, 8), (1, 3, 1),
                                     (2000, 30000, 40)])
def test_adj_weights_on_gpu_match_oracle(n, E, dup):
    """ngt_adj_weights bit for bit against the oracle, including keys with
    many PPR entries (dup > 1: each (u, v) pair drawn from a small pool, in
    both directions), whose fp32 sums depend on the order of the adds."""
    _say(f"case adj weights n={n} E={E} dup={dup}")
    rng = np.random.default_rng(n + E)
    if dup > 1:
        pool = rng.integers(0, n, (2, E // dup))
        pick = rng.integers(0, pool.shape[1], E)
        ei = pool[:, pick]
        flip = rng.random(E) < 0.5
        ei = np.where(flip, ei[::-1], ei)
    else:
        ei = rng.integers(0, n, (2, E))
    val = (rng.random(E).astype(np.float32) / 50).astype(np.float32)
    keys = np.minimum(ei[0], ei[1]) * n + np.maximum(ei[0], ei[1])
    if dup > 1:
        assert np.bincount(np.unique(keys, return_inverse=True)[1]).max() >= 3
    x, a, w = W.adj_weights(torch.from_numpy(ei).cuda(), torch.from_numpy(val).cuda())
    xo, ao, wo = OG.adj_weights(ei, val)
    np.testing.assert_array_equal(x.cpu().numpy(), xo)
    np.testing.assert_array_equal(a.cpu().numpy(), ao)
    np.testing.assert_array_equal(w.cpu().numpy(), wo)


def test_adj_weights_on_gpu_sum_in_entry_order():
    """A key whose three values truncate to 2 summed in entry order and to 3 in
    reverse: the GPU path adds in entry order (no atomics), both ways round."""
    _say("case adj weights order")
    a, b, c = 0.0005994238, 0.0004226872, 0.0019778889
    for ei, vals, want in (([[4, 1, 4], [1, 4, 1]], [a, b, c], 2),
                           ([[1, 4, 1], [4, 1, 4]], [c, b, a], 3)):
        x, adj, w = W.adj_weights(torch.tensor(ei).cuda(),
                                  torch.tensor(vals, dtype=torch.float32).cuda())
        assert w.tolist() == [want, want] and adj.tolist() == [4, 1]
        assert x.tolist() == [0, 0, 1, 1, 1, 2]


def test_adj_weights_rejects_negative_ids():
    _say("case adj weights bad id")
    with pytest.raises(ValueError):
        W.adj_weights(torch.tensor([[0, -1], [1, 2]]).cuda(), torch.tensor([0.1, 0.2]).cuda())


def test_window_feature_assembly_bit_exact():
    _say("case feature assembly")
    rng = np.random.default_rng(3)
    feat = torch.randn(1000, 100)
    parts = [rng.choice(1000, 200, replace=False) for _ in range(3)]
    rer, dups = W.duplicate_rerange([torch.from_numpy(p) for p in parts])
    cache_ids, idx = W.dup_cache_metadata(dups, device="cuda")
    fd = feat.cuda()
    cache = W.dup_feature_cache(fd, cache_ids)
    for r, i in zip(rer, idx):
        x = W.assemble_window_features(fd, cache, i, r)
        want = OG.assemble_window_features(feat.numpy(), cache_ids.cpu().numpy(), i.cpu().numpy(),
                                           r.cpu().numpy())
        assert torch.equal(x.cpu(), torch.from_numpy(want))
        assert torch.equal(x.cpu(), feat[r.cpu()])


def test_gather_rows_flags_bad_index():
    _say("case gather bad index")
    src = torch.arange(12, dtype=torch.float32).view(4, 3).cuda()
    out, bad = W.gather_rows(src, torch.tensor([0, 7, 3]).cuda())
    assert int(bad.item()) == 1
    assert torch.equal(out.cpu()[1], torch.zeros(3)) and torch.equal(out.cpu()[2], src.cpu()[3])

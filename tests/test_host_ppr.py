"""Host-side CSR helpers of the GPU PPR path (no GPU): the row sort the
direct step needs and the repeat count its pruning bound uses, against
brute force."""
import numpy as np
import torch

from neutrongt_amd.ppr import _sorted_rows, max_repeats


def _random_csr(rng, n, deg_max, span):
    deg = rng.integers(0, deg_max, n)
    rowptr = np.zeros(n + 1, np.int64)
    rowptr[1:] = np.cumsum(deg)
    col = rng.integers(-2, span, rowptr[-1])  # negative ids: malformed, still sortable
    return torch.from_numpy(rowptr), torch.from_numpy(col)


def test_sorted_rows_sorts_each_row_and_keeps_sorted_input():
    rng = np.random.default_rng(0)
    for _ in range(20):
        rowptr, col = _random_csr(rng, 50, 12, 30)
        got = _sorted_rows(rowptr, col).numpy()
        rp = rowptr.numpy()
        want = np.concatenate([np.sort(col.numpy()[rp[r]:rp[r + 1]]) for r in range(50)])
        np.testing.assert_array_equal(got, want)
        again = _sorted_rows(rowptr, torch.from_numpy(want))
        np.testing.assert_array_equal(again.numpy(), want)


def test_max_repeats_is_the_longest_run_within_a_row():
    rowptr = torch.tensor([0, 4, 4, 7, 9])
    col = torch.tensor([1, 1, 1, 2, 2, 3, 3, 3, 3])  # row 2 ends in 3, row 3 is [3, 3]
    assert max_repeats(rowptr, col) == 3
    assert max_repeats(torch.tensor([0, 2]), torch.tensor([4, 5])) == 1
    assert max_repeats(torch.tensor([0, 0]), torch.tensor([], dtype=torch.long)) == 1
    rng = np.random.default_rng(1)
    for _ in range(20):
        rowptr, col = _random_csr(rng, 40, 15, 6)
        col = _sorted_rows(rowptr, col)
        rp, c = rowptr.numpy(), col.numpy()
        want = max([1] + [int(np.unique(c[rp[r]:rp[r + 1]], return_counts=True)[1].max())
                          for r in range(40) if rp[r + 1] > rp[r]])
        assert max_repeats(rowptr, col) == want

"""The random row-gather probe behind the benchmark's gather ceiling: it runs
through the C ABI for the row sizes of the sparse configurations, skips
indices outside the table (its own bounds check), and leaves its sink alone."""
import ctypes as C

import pytest
import torch

from neutrongt_amd import _lib

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("row_bytes", [256, 768, 1536, 2048])
def test_probe_gathers_and_skips_out_of_range_rows(dev, row_bytes):
    print(f"probe row_bytes={row_bytes}", flush=True)
    n_rows = 1000
    table = torch.ones(n_rows * row_bytes // 4, dtype=torch.int32, device=dev)
    g = torch.Generator(device="cpu").manual_seed(row_bytes)
    idx = torch.randint(0, n_rows, (10_000,), generator=g, dtype=torch.int32)
    idx[::97] = -5  # outside the table: skipped by the kernel
    idx[1::89] = n_rows
    idx[2::83] = 1 << 30
    idx = idx.to(dev)
    sink = torch.zeros(4, dtype=torch.int32, device=dev)
    lib = _lib.load()
    st = C.c_void_p(_lib.stream_ptr(dev))
    for _ in range(2):
        _lib.check(lib.ngt_probe_gather(C.c_void_p(table.data_ptr()), n_rows, row_bytes,
                                        C.c_void_p(idx.data_ptr()), idx.numel(),
                                        C.c_void_p(sink.data_ptr()), st))
    torch.cuda.synchronize()
    # rows of equal words XOR to zero, so the sink is never written
    assert sink.cpu().tolist() == [0, 0, 0, 0]
    assert torch.equal(table, torch.ones_like(table))  # read only

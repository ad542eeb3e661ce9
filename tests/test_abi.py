"""The C-ABI library loads, exports every declared symbol and validates its
arguments -- no GPU needed (no compute call is made)."""
import ctypes as C
import re
from pathlib import Path

import pytest

from neutrongt_amd import _lib

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "ngt_attn.h"


def _declared():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(ngt_[a-z0-9_]+)\s*\(", text)))


def test_library_is_built_and_loads():
    assert _lib.LIB_PATH.exists(), "run python -m neutrongt_amd.build"
    lib = _lib.load()
    assert lib.ngt_abi_version() == _lib.ABI_VERSION


def test_every_declared_symbol_is_exported_and_bound():
    lib = _lib.load()
    names = _declared()
    assert len(names) >= 14
    for n in names:
        assert hasattr(lib, n), f"{n} declared in ngt_attn.h but not exported"
        assert n in _lib.SIGNATURES, f"{n} has no ctypes signature"


def test_struct_layout_matches_header():
    # int32 n_q, n_k; int64 n_edges; int32 chunk_q, chunk_k, small_q, small_k;
    # 14 pointers; 12 int32; 2 pointers (the row orders)
    assert C.sizeof(_lib.WindowCSR) == 8 + 8 + 16 + 14 * 8 + 12 * 4 + 2 * 8
    assert _lib.WindowCSR.rowptr.offset == 32
    assert _lib.WindowCSR.max_items_q.offset == 32 + 14 * 8
    assert _lib.WindowCSR.order_q.offset == 32 + 14 * 8 + 12 * 4


def test_csr_sizes_arithmetic():
    lib = _lib.load()
    a, b, c, d = (C.c_int32() for _ in range(4))
    assert lib.ngt_csr_sizes(1000, 100, 300, 64, 32, C.byref(a), C.byref(b), C.byref(c),
                             C.byref(d)) == 0
    assert a.value == 100 + 2 * 16 + 1 and c.value == 300 + 2 * 32 + 1
    assert b.value == 16 + 1 and d.value == 32 + 1
    assert lib.ngt_csr_sizes(-1, 1, 1, 1, 1, None, None, None, None) == 1


def test_argument_errors_are_reported_without_touching_the_gpu():
    lib = _lib.load()
    rc = lib.ngt_sparse_fwd(0, None, None, None, None, 8, 8, 1.0, -5.0, 5.0, 1e-6, None, None,
                            None, 0, None, 0, None)
    assert rc == 1
    assert b"null csr" in lib.ngt_last_error()
    s = _lib.WindowCSR()
    rc = lib.ngt_sparse_fwd(0, None, None, None, C.byref(s), 8, 12, 1.0, -5.0, 5.0, 1e-6, None,
                            None, None, 0, None, 0, None)
    assert rc == 2 and b"head_dim" in lib.ngt_last_error()
    rc = lib.ngt_dense_fwd(7, None, None, None, 1, 1, 1, 8, 1.0, 0.0, 0, None, None, None, None,
                           None, None, 0, None)
    assert rc == 1
    rc = lib.ngt_dense_fwd(0, None, None, None, 0, 0, 1, 8, 1.0, 1.5, 0, None, None, None, None,
                           None, None, 0, None)
    assert rc == 1 and b"dropout_p" in lib.ngt_last_error()
    rc = lib.ngt_dense_fwd(0, None, None, None, 0, 0, 1, 8, 1.0, float("nan"), 0, None, None, None,
                           None, None, None, 0, None)
    assert rc == 1 and b"dropout_p" in lib.ngt_last_error()
    rc = lib.ngt_dense_fwd(0, None, None, None, 65536, 131074, 1, 8, 1.0, 0.5, 0, None, None, None,
                           None, None, None, 0, None)
    assert rc == 2 and b"2^32" in lib.ngt_last_error()
    # the dense kernels need scale > 0 (the matrix-core forward scales its running maximum)
    for sc in (0.0, -2.0, float("nan")):
        rc = lib.ngt_dense_fwd(1, None, None, None, 0, 0, 1, 8, sc, 0.0, 0, None, None, None,
                               None, None, None, 0, None)
        assert rc == 1 and b"scale" in lib.ngt_last_error()
        rc = lib.ngt_dense_bwd(1, None, None, None, None, None, None, None, 0, 0, 1, 8, sc, 0.0,
                               0, None, None, None, None, None, 0, None)
        assert rc == 1 and b"scale" in lib.ngt_last_error()
    # the optional-terms softmax runs one block per (head, query) row: more
    # than 2^24 rows are refused before anything launches
    rc = lib.ngt_dense_bias_softmax_fwd(256, 0, 65537, 8, None, 1.0, None, None, 0.0, 0, None,
                                        None, None, None, None)
    assert rc == 1 and b"n_heads * n_q" in lib.ngt_last_error()
    rc = lib.ngt_dense_bias_softmax_bwd(256, 0, 65537, 8, None, None, None, 0.0, 0, None, None,
                                        None)
    assert rc == 1 and b"n_heads * n_q" in lib.ngt_last_error()
    rc = lib.ngt_dense_bias_softmax_fwd(2, -1, 4, 8, None, 1.0, None, None, 0.0, 0, None, None,
                                        None, None, None)
    assert rc == 1 and b"bad sizes" in lib.ngt_last_error()
    # the direct PPR step: K range, a total below one entry per row, and
    # counts past its int32 chunk ids are refused before anything launches
    for K, total, n_rows in ((0, 4, 4), (65, 4, 4), (5, 3, 4)):
        rc = lib.ngt_ppr_step_direct(None, None, None, 10, None, None, None, None, n_rows, K,
                                     0.85, 0.15, 1, total, None, None, None, None, None, 0, None)
        assert rc == 1 and b"ngt_ppr_step_direct" in lib.ngt_last_error()
    rc = lib.ngt_ppr_step_direct(1, 1, 1, 10, 1, 1, 1, 1, 4, 5, 0.85, 0.15, -1, 8, 1, 1, 1, 1,
                                 None, 0, None)
    assert rc == 1
    rc = lib.ngt_ppr_step_direct(1, 1, 1, 10, 1, 1, 1, 1, 4, 5, 0.85, 0.15, 1, 1 << 41, 1, 1, 1,
                                 1, None, 0, None)
    assert rc == 2 and b"too large" in lib.ngt_last_error()
    with pytest.raises(_lib.NGTError):
        _lib.check(1)


def test_strided_backward_validates_its_row_stride_without_touching_the_gpu():
    """ngt_sparse_bwd_strided: the gradients' row stride is at least H * d and
    a multiple of 16 bytes, and the gradients 16-byte aligned; anything else
    is refused before a launch."""
    lib = _lib.load()
    s = _lib.WindowCSR()  # empty window: nothing would launch anyway
    args = lambda dtype, ld, gq=None: (dtype, None, None, None, None, None, 0, None, None, None,
                                       C.byref(s), 8, 16, 4.0, -5.0, 5.0, gq, None, None, ld,
                                       None, 0, None)
    assert lib.ngt_sparse_bwd_strided(*args(1, 127)) == 1  # below H * d = 128
    assert b"row stride" in lib.ngt_last_error()
    assert lib.ngt_sparse_bwd_strided(*args(1, 132)) == 1  # 264 bytes: not a multiple of 16
    assert lib.ngt_sparse_bwd_strided(*args(0, 132)) == 0  # 528 bytes in fp32
    assert lib.ngt_sparse_bwd_strided(*args(1, 0)) == 0    # 0: contiguous rows
    assert lib.ngt_sparse_bwd_strided(*args(1, 384)) == 0  # [N, 3, H, d]
    assert lib.ngt_sparse_bwd_strided(*args(1, 384, 8)) == 1
    assert b"16-byte aligned" in lib.ngt_last_error()


def test_colsum_takes_any_width():
    """Column sums of any width (a 47-class readout's bias gradient): one fp32
    partial per 256-row chunk and column; zero columns refused."""
    lib = _lib.load()
    nb = C.c_size_t()
    for n in (1, 7, 47, 768):
        assert lib.ngt_colsum_workspace_bytes(1000, n, C.byref(nb)) == 0
        assert nb.value == 4 * n * 4  # ceil(1000 / 256) chunks
    assert lib.ngt_colsum_workspace_bytes(1000, 0, C.byref(nb)) == 1
    assert b"bad sizes" in lib.ngt_last_error()


def test_dense_workspace_query_depends_on_path_and_scores():
    """The matrix-core path (bf16, d <= 32) needs H * n_k floats of node-score
    partials and nothing without node scores; the vector-ALU path sizes its
    per-block partials only when node scores are wanted."""
    lib = _lib.load()
    fb, bb = C.c_size_t(), C.c_size_t()
    assert lib.ngt_dense_workspace_bytes(1, 300, 300, 8, 8, 1, C.byref(fb), C.byref(bb)) == 0
    a256 = lambda x: (x + 255) // 256 * 256
    assert fb.value == a256(8 * 300 * 4) and bb.value >= 300 * 8 * 4
    assert lib.ngt_dense_workspace_bytes(1, 300, 300, 8, 8, 0, C.byref(fb), C.byref(bb)) == 0
    assert fb.value == 0
    # a large window without node scores splits its keys over blocks (the split
    # states: (m, l) and unnormalised O per split, query and head); with node
    # scores their blocks share the launch and the forward takes one split
    assert lib.ngt_dense_workspace_bytes(1, 16000, 16000, 8, 8, 0, C.byref(fb), C.byref(bb)) == 0
    n_split = 2
    assert fb.value == a256(n_split * 16000 * 8 * 8) + a256(n_split * 16000 * 8 * 8 * 4)
    assert lib.ngt_dense_workspace_bytes(1, 16000, 16000, 8, 8, 1, C.byref(fb), C.byref(bb)) == 0
    assert fb.value == a256(8 * 16000 * 4)
    # the backward: D per query and head, then three key splits' partial dQ
    assert bb.value == a256(16000 * 8 * 4) + a256(3 * 16000 * 8 * 8 * 4)
    assert lib.ngt_dense_workspace_bytes(0, 500, 300, 2, 8, 1, C.byref(fb), C.byref(bb)) == 0
    with_ns = fb.value
    assert lib.ngt_dense_workspace_bytes(0, 500, 300, 2, 8, 0, C.byref(fb), C.byref(bb)) == 0
    assert with_ns >= 2 * 300 * 4 and fb.value < with_ns


def test_layernorm_rejects_misaligned_rows_without_touching_the_gpu():
    """fp32 rows move 16 bytes per lane access, bf16 rows 8: bases off that
    alignment are an argument error, before any launch."""
    lib = _lib.load()
    p16, p8 = C.c_void_p(4096), C.c_void_p(4096 + 8)
    m = C.c_void_p(8192)
    rc = lib.ngt_layernorm_fwd(0, p8, 4, 64, m, m, 1e-5, 0, p16, m, m, None)
    assert rc == 1 and b"aligned" in lib.ngt_last_error()
    rc = lib.ngt_layernorm_fwd(0, p16, 4, 64, m, m, 1e-5, 0, p8, m, m, None)
    assert rc == 1 and b"aligned" in lib.ngt_last_error()
    rc = lib.ngt_add_layernorm_fwd(0, p16, p8, 4, 64, 0.0, 0, None, m, m, 1e-5, None, 0, p16, m,
                                   m, None)
    assert rc == 1 and b"aligned" in lib.ngt_last_error()
    rc = lib.ngt_layernorm_bwd(0, p16, 0, p8, 4, 64, m, m, m, p16, None, None, m, 1 << 20, None)
    assert rc == 1 and b"aligned" in lib.ngt_last_error()


def test_noalloc_forward_rejects_windows_beyond_its_scratch_without_touching_the_gpu():
    """The allocation-free forward holds 32 MiB of static scratch: a window
    whose forward workspace is larger is refused before anything runs."""
    lib = _lib.load()
    s = _lib.WindowCSR()
    s.n_q = s.n_k = 200_000
    s.n_packed_q = s.n_packed_k = 200_000  # counters consistent with an edgeless window
    fb, bb = C.c_size_t(), C.c_size_t()
    assert lib.ngt_sparse_workspace_bytes(C.byref(s), 64, 8, C.byref(fb), C.byref(bb)) == 0
    assert fb.value > 32 << 20
    rc = lib.ngt_sparse_fwd_noalloc(1, None, None, None, C.byref(s), 64, 8, 8.0 ** 0.5, -5.0, 5.0,
                                    1e-6, None, None, None, 0, None)
    assert rc == 2 and b"static" in lib.ngt_last_error()


def test_product_never_imports_the_oracle():
    pkg = ROOT / "neutrongt_amd"
    for f in list(pkg.rglob("*.py")) + list(pkg.rglob("*.hip")):
        text = f.read_text()
        assert not re.search(r"^\s*(from|import)\s+oracle\b", text, flags=re.M), f
        assert "oracle/" not in text, f


def test_build_entry_compiles(tmp_path):
    """The build script's flags keep packed-fp32 VALU ops disabled."""
    from neutrongt_amd import build

    flags = " ".join(build.HIPCC_FLAGS)
    assert "-packed-fp32-ops" in flags and "--offload-arch=gfx950" in flags


def test_autograd_node_loads_and_matches_the_struct_without_touching_the_gpu():
    """ngt_autograd.so (the sparse attention's C++ autograd node) loads, binds
    to the library's entry points and was built against this header's
    ngt_window_csr."""
    ext = _lib.autograd_ext()
    assert ext is not None, "ngt_autograd.so is not built"
    assert ext.csr_struct_bytes() == C.sizeof(_lib.WindowCSR)
    assert callable(ext.sparse_attention)


def test_noalloc_forward_refuses_a_window_beyond_its_static_scratch():
    # A window whose forward workspace (Z and the split rows' partials) exceeds
    # the 32 MiB static array is refused before any launch or device query.
    lib = _lib.load()
    s = _lib.WindowCSR()
    s.n_q = s.n_k = 300_000
    s.n_packed_q = s.n_packed_k = 300_000  # every row packed: the counters are consistent
    H, d = 32, 24
    fb, bb = C.c_size_t(), C.c_size_t()
    assert lib.ngt_sparse_workspace_bytes(C.byref(s), H, d, C.byref(fb), C.byref(bb)) == 0
    assert fb.value > 32 << 20
    rc = lib.ngt_sparse_fwd_noalloc(1, None, None, None, C.byref(s), H, d, 4.9, -5.0, 5.0, 1e-6,
                                    None, None, None, 0, None)
    assert rc == 2
    msg = lib.ngt_last_error()
    assert b"scratch" in msg and b"ngt_sparse_fwd with a workspace" in msg
    # and the usual argument checks come first
    rc = lib.ngt_sparse_fwd_noalloc(1, None, None, None, None, H, d, 4.9, -5.0, 5.0, 1e-6, None,
                                    None, None, 0, None)
    assert rc == 1 and b"null csr" in lib.ngt_last_error()


def test_dense_bias_head_chunk_follows_the_budget():
    from neutrongt_amd import attention as A

    # 16,000 x 16,000 fp32 is 1.02 GB per matrix: 5 per head exceed 4 GiB
    assert A.dense_bias_head_chunk(8, 16000, 16000) == 1
    assert A.dense_bias_head_chunk(8, 1000, 1000) == 8
    assert A.dense_bias_head_chunk(32, 4000, 4000, budget=1 << 30) == 3
    # and the softmax launches stay within 2^24 (head, query) rows
    assert A.dense_bias_head_chunk(64, 1 << 20, 1, budget=1 << 60) == 16

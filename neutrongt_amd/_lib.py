"""ctypes binding of libngt_attn.so (declared in include/ngt_attn.h).

The library is loaded lazily on first use; a missing or stale build raises
``RuntimeError`` -- there is no CPU fallback.
"""
from __future__ import annotations

import ctypes as C
import os
import threading
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "libngt_attn.so"
ABI_VERSION = 11

NGT_F32 = 0
NGT_BF16 = 1

INFO_ITEMS_Q = 0
INFO_PARTS_Q = 1
INFO_SPLITS_Q = 2
INFO_ITEMS_K = 3
INFO_PARTS_K = 4
INFO_SPLITS_K = 5
INFO_DST_END = 6
INFO_SRC_END = 7
INFO_BAD_EDGES = 8
INFO_MAX_DEG_Q = 9
INFO_MAX_DEG_K = 10
INFO_PACKED_Q = 11
INFO_PACKED_K = 12
INFO_SMALL_Q = 13
INFO_SMALL_K = 14
SMALL_FROM_DEGREES = -1  # ngt_csr_build picks the packing threshold from the degrees
INFO_LEN = 16


class WindowCSR(C.Structure):
    """Mirror of ``ngt_window_csr``."""

    _fields_ = [
        ("n_q", C.c_int32),
        ("n_k", C.c_int32),
        ("n_edges", C.c_int64),
        ("chunk_q", C.c_int32),
        ("chunk_k", C.c_int32),
        ("small_q", C.c_int32),
        ("small_k", C.c_int32),
        ("rowptr", C.c_void_p),
        ("col", C.c_void_p),
        ("perm", C.c_void_p),
        ("t_rowptr", C.c_void_p),
        ("t_col", C.c_void_p),
        ("t_perm", C.c_void_p),
        ("q2t", C.c_void_p),
        ("items_q", C.c_void_p),
        ("splits_q", C.c_void_p),
        ("packed_q", C.c_void_p),
        ("items_k", C.c_void_p),
        ("splits_k", C.c_void_p),
        ("packed_k", C.c_void_p),
        ("info", C.c_void_p),
        ("max_items_q", C.c_int32),
        ("max_splits_q", C.c_int32),
        ("max_items_k", C.c_int32),
        ("max_splits_k", C.c_int32),
        ("n_items_q", C.c_int32),
        ("n_parts_q", C.c_int32),
        ("n_splits_q", C.c_int32),
        ("n_packed_q", C.c_int32),
        ("n_items_k", C.c_int32),
        ("n_parts_k", C.c_int32),
        ("n_splits_k", C.c_int32),
        ("n_packed_k", C.c_int32),
        ("order_q", C.c_void_p),
        ("order_k", C.c_void_p),
    ]


_i32, _i64, _f32, _vp, _sz = C.c_int32, C.c_int64, C.c_float, C.c_void_p, C.c_size_t
_u64 = C.c_uint64
_pi32 = C.POINTER(C.c_int32)
_psz = C.POINTER(C.c_size_t)
_pcsr = C.POINTER(WindowCSR)

# name -> argtypes (restype is int unless listed in _RESTYPES)
SIGNATURES = {
    "ngt_abi_version": [],
    "ngt_last_error": [],
    "ngt_csr_sizes": [_i64, _i32, _i32, _i32, _i32, _pi32, _pi32, _pi32, _pi32],
    "ngt_csr_workspace_bytes": [_i64, _i32, _i32, _psz],
    "ngt_csr_build": [_vp, _pcsr, _vp, _sz, _vp],
    "ngt_sparse_workspace_bytes": [_pcsr, _i32, _i32, _psz, _psz],
    "ngt_sparse_fwd": [_i32, _vp, _vp, _vp, _pcsr, _i32, _i32, _f32, _f32, _f32, _f32, _vp, _vp,
                       _vp, _i32, _vp, _sz, _vp],
    "ngt_sparse_fwd_noalloc": [_i32, _vp, _vp, _vp, _pcsr, _i32, _i32, _f32, _f32, _f32, _f32,
                               _vp, _vp, _vp, _i32, _vp],
    "ngt_sparse_bwd": [_i32, _vp, _vp, _vp, _vp, _vp, _vp, _pcsr, _i32, _i32, _f32, _f32, _f32,
                       _vp, _vp, _vp, _vp, _sz, _vp],
    "ngt_sparse_fwd_ext": [_i32, _vp, _vp, _vp, _vp, _vp, _i32, _pcsr, _i32, _i32, _f32, _f32,
                           _f32, _f32, _vp, _vp, _vp, _i32, _vp, _sz, _vp],
    "ngt_sparse_bwd_ext": [_i32, _vp, _vp, _vp, _vp, _vp, _i32, _vp, _vp, _vp, _pcsr, _i32, _i32,
                           _f32, _f32, _f32, _vp, _vp, _vp, _vp, _sz, _vp],
    "ngt_sparse_bwd_strided": [_i32, _vp, _vp, _vp, _vp, _vp, _i32, _vp, _vp, _vp, _pcsr, _i32,
                               _i32, _f32, _f32, _f32, _vp, _vp, _vp, _i64, _vp, _sz, _vp],
    "ngt_edge_bias_gather": [_pcsr, _i32, _vp, _i64, _i64, _i64, _vp, _vp, _vp],
    "ngt_sparse_fwd_bias": [_i32, _vp, _vp, _vp, _vp, _vp, _i32, _pcsr, _i32, _i32, _f32, _f32,
                            _f32, _f32, _vp, _vp, _vp, _vp, _i32, _vp, _sz, _vp],
    "ngt_sparse_bwd_bias": [_i32, _vp, _vp, _vp, _vp, _vp, _i32, _vp, _vp, _vp, _pcsr, _i32, _i32,
                            _f32, _f32, _f32, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _vp],
    "ngt_edge_bias_grad": [_pcsr, _i32, _vp, _vp, _i64, _i64, _i64, _vp],
    "ngt_dense_bias_softmax_fwd": [_i32, _i32, _i32, _i32, _vp, _f32, _vp, _vp, _f32, _u64, _vp,
                                   _vp, _vp, _vp, _vp],
    "ngt_dense_bias_softmax_bwd": [_i32, _i32, _i32, _i32, _vp, _vp, _vp, _f32, _u64, _vp, _vp,
                                   _vp],
    "ngt_dense_abs_head_sum": [_i32, _i32, _i32, _vp, _f32, _i32, _vp, _vp],
    "ngt_dense_abs_colsum_workspace_bytes": [_i32, _psz],
    "ngt_dense_abs_colsum": [_i32, _i32, _i32, _vp, _vp, _vp, _sz, _vp],
    "ngt_dense_workspace_bytes": [_i32, _i32, _i32, _i32, _i32, _i32, _psz, _psz],
    "ngt_dense_fwd": [_i32, _vp, _vp, _vp, _i32, _i32, _i32, _i32, _f32, _f32, _u64, _vp, _vp,
                      _vp, _vp, _vp, _vp, _sz, _vp],
    "ngt_dense_bwd": [_i32, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _i32, _i32, _i32, _f32, _f32,
                      _u64, _vp, _vp, _vp, _vp, _vp, _sz, _vp],
    "ngt_layernorm_fwd": [_i32, _vp, _i64, _i32, _vp, _vp, _f32, _i32, _vp, _vp, _vp, _vp],
    "ngt_layernorm_bwd_workspace_bytes": [_i64, _i32, _psz],
    "ngt_layernorm_bwd": [_i32, _vp, _i32, _vp, _i64, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz,
                          _vp],
    "ngt_add_layernorm_fwd": [_i32, _vp, _vp, _i64, _i32, _f32, _u64, _vp, _vp, _vp, _f32, _vp,
                              _i32, _vp, _vp, _vp, _vp],
    "ngt_add_layernorm_bwd": [_i32, _vp, _i32, _vp, _vp, _i64, _i32, _f32, _u64, _vp, _vp, _vp,
                              _vp, _vp, _vp, _vp, _vp, _vp, _sz, _vp],
    "ngt_colsum_workspace_bytes": [_i64, _i32, _psz],
    "ngt_colsum_bf16": [_vp, _i64, _i32, _vp, _vp, _sz, _vp],
    "ngt_chunk_sum_f32": [_vp, _i32, _i64, _vp, _vp],
    "ngt_related_workspace_bytes": [_i32, _i32, _psz],
    "ngt_merge_related_nodes": [_vp, _vp, _vp, _i32, _vp, _i32, _i32, _vp, _vp, _vp, _sz, _vp],
    "ngt_adj_weights_workspace_bytes": [_i64, _i64, _psz],
    "ngt_adj_weights": [_vp, _vp, _i64, _i64, _vp, _vp, _vp, _vp, _vp, _sz, _vp],
    "ngt_gather_rows": [_vp, _i64, _vp, _i64, _i64, _vp, _vp, _vp],
    "ngt_window_dup_workspace_bytes": [_i64, _psz],
    "ngt_window_dup_layout": [_vp, _i64, _vp, _i32, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _vp],
    "ngt_segment_sum_f32": [_vp, _i64, _vp, _i64, _vp, _vp, _vp],
    "ngt_ppr_count_workspace_bytes": [_i32, _vp],
    "ngt_ppr_count": [_vp, _i64, _vp, _vp, _i32, _i32, _vp, _vp, _vp, _sz, _vp],
    "ngt_ppr_step_workspace_bytes": [_i64, _i32, _vp],
    "ngt_ppr_step": [_vp, _vp, _vp, _i64, _vp, _vp, _vp, _vp, _i32, _i32, C.c_float, C.c_float,
                     _vp, _i64, _vp, _vp, _vp, _vp, _vp, _sz, _vp],
    "ngt_ppr_step_direct_workspace_bytes": [_i64, _i32, _i32, _vp],
    "ngt_ppr_step_direct": [_vp, _vp, _vp, _i64, _vp, _vp, _vp, _vp, _i32, _i32, C.c_float,
                            C.c_float, _i32, _i64, _vp, _vp, _vp, _vp, _vp, _sz, _vp],
    "ngt_subgraph_workspace_bytes": [_i64, _i64, _i32, _vp],
    "ngt_subgraph_coo": [_vp, _i64, _i64, _vp, _i32, _vp, _i64, _vp, _vp, _sz, _vp],
    "ngt_subgraph_csr": [_vp, _vp, _i64, _i64, _vp, _i32, _vp, _i64, _vp, _vp, _sz, _vp],
    "ngt_timing_enable": [_i32],
    "ngt_timing_summary": [C.c_char_p, _sz],
}
_RESTYPES = {"ngt_last_error": C.c_char_p}

_lock = threading.Lock()
_lib = None
_RAW_STREAM = getattr(torch._C, "_cuda_getCurrentRawStream", None)


class NGTError(RuntimeError):
    pass


def load(path: str | os.PathLike | None = None):
    """Returns the loaded library (loads it on first call)."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        p = Path(path or os.environ.get("NGT_LIB") or LIB_PATH)
        if not p.exists():
            raise RuntimeError(
                f"{p.name} is not built ({p}); run `python -m neutrongt_amd.build` "
                "(hipcc, gfx950). There is no CPU fallback.")
        lib = C.CDLL(str(p))
        for name, argtypes in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = argtypes
            fn.restype = _RESTYPES.get(name, C.c_int)
        ver = lib.ngt_abi_version()
        if ver != ABI_VERSION:
            raise RuntimeError(f"{p.name} ABI version {ver} != expected {ABI_VERSION}; rebuild it")
        _lib = lib
        return lib


_ext = None
EXT_PATH = Path(__file__).resolve().parent / "ngt_autograd.so"


def autograd_ext():
    """The C++ autograd node of the sparse attention (ngt_autograd.so, built
    beside the library), bound to the loaded library's entry points; None when
    it is not built -- the Python autograd.Function then drives the same
    library calls."""
    global _ext
    if _ext is not None:
        return _ext or None
    lib = load()
    with _lock:
        if _ext is None:
            if not EXT_PATH.exists():
                _ext = False
            else:
                import importlib.util

                spec = importlib.util.spec_from_file_location("ngt_autograd", EXT_PATH)
                mod = importlib.util.module_from_spec(spec)
                spec.loader.exec_module(mod)
                ext_abi = mod.abi_version() if hasattr(mod, "abi_version") else None
                if ext_abi != lib.ngt_abi_version():
                    # the entry points handed over below are cast to the
                    # prototypes the extension was compiled with
                    raise RuntimeError(f"{EXT_PATH.name} was built against ABI version {ext_abi}, "
                                       f"the library is {lib.ngt_abi_version()}; rebuild it")
                if mod.csr_struct_bytes() != C.sizeof(WindowCSR):
                    raise RuntimeError(f"{EXT_PATH.name} was built against another "
                                       "ngt_window_csr; rebuild it")
                addr = lambda fn: C.cast(fn, C.c_void_p).value
                mod.init(addr(lib.ngt_sparse_fwd_ext), addr(lib.ngt_sparse_bwd_strided),
                         addr(lib.ngt_last_error))
                _ext = mod
    return _ext or None


def stream_ptr(device) -> int:
    """hipStream_t (as an int) of torch's current stream on ``device``.

    torch.cuda.current_stream(dev).cuda_stream builds a Stream object per call
    (about 3.4 us of host time each on the benchmark host, most of a small
    window's per-layer host cost); the raw accessor returns the same pointer
    without it.  Falls back to the public API when this torch lacks it."""
    dev = device if isinstance(device, torch.device) else torch.device(device)
    idx = dev.index if dev.index is not None else torch.cuda.current_device()
    if _RAW_STREAM is not None:
        return int(_RAW_STREAM(idx))
    return torch.cuda.current_stream(dev).cuda_stream


def check(rc: int) -> None:
    """Raises NGTError with the library's message when rc != 0."""
    if rc != 0:
        msg = load().ngt_last_error()
        raise NGTError((msg or b"").decode(errors="replace") or f"ngt error {rc}")


def call(name: str, *args) -> None:
    check(getattr(load(), name)(*args))


def timing_enable(on: bool) -> None:
    check(load().ngt_timing_enable(1 if on else 0))


def timing_summary() -> dict:
    """{kernel name: (launches, total ms)} since the last summary (waits for the GPU)."""
    buf = C.create_string_buffer(1 << 16)
    check(load().ngt_timing_summary(buf, len(buf)))
    out = {}
    for line in buf.value.decode().splitlines():
        name, cnt, ms = line.split()
        out[name] = (int(cnt), float(ms))
    return out

"""ctypes binding of libmosaic_bsa.so (the C ABI declared in include/mosaic_bsa.h).

The library is loaded from this package directory.  There is no fallback: if it is missing
the first call raises ``MosaicLibraryError`` naming the build command.
"""

from __future__ import annotations

import ctypes
import os
import threading

LIB_NAME = "libmosaic_bsa.so"
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)
ABI_VERSION = 10

# mosaic_bsa_mode
MODE_FULL = 0
MODE_LOCAL_ONLY = 1
MODE_NO_COMPRESSION = 2
MODE_NO_SELECTION = 3

# mosaic_bsa_stage (mosaic_bsa_fwd_stage)
STAGE_POOL = 0
STAGE_CMP = 1
STAGE_TOPK = 2
STAGE_ATTN = 3

# mosaic_status values the Python side names
ERR_MODE = 10
ERR_SCRATCH_LIMIT = 12

# mosaic_knn_interp_fwd_ex flags
KNN_ROUND_PRODUCTS = 1
NOALLOC_SCRATCH_BYTES = 128 << 20

# mosaic_dtype
DTYPE_F32 = 0
DTYPE_BF16 = 1

EXPORTED_SYMBOLS = (
    "mosaic_bsa_workspace_size",
    "mosaic_bsa_fwd",
    "mosaic_bsa_fwd_noalloc",
    "mosaic_bsa_fwd_profiled",
    "mosaic_bsa_fwd_stage",
    "mosaic_bsa_fwd_rope",
    "mosaic_bsa_fwd_proj",
    "mosaic_knn_interp_fwd",
    "mosaic_knn_interp_fwd_ordered",
    "mosaic_knn_interp_fwd_ex",
    "mosaic_sparse_attn_bwd_workspace_size",
    "mosaic_sparse_attn_bwd",
    "mosaic_rms_norm_fwd",
    "mosaic_swiglu_fwd",
    "mosaic_resample_norm_fwd",
    "mosaic_gate_softmax_fwd",
    "mosaic_add_merge_fwd",
    "mosaic_swiglu_linear_fwd",
    "mosaic_sparse_attn_fwd",
    "mosaic_sparse_attn_fwd_workspace_size",
    "mosaic_sparse_attn_fwd_ws",
    "mosaic_block_attn_fwd",
    "mosaic_dense_attn_fwd",
    "mosaic_pool_mean_fwd",
    "mosaic_attn_topk_workspace_size",
    "mosaic_attn_topk_fwd",
    "mosaic_bsa_strerror",
    "mosaic_bsa_abi_version",
)


class MosaicLibraryError(RuntimeError):
    pass


class Bnhd(ctypes.Structure):
    _fields_ = [("ptr", ctypes.c_void_p), ("stride_b", ctypes.c_int64),
                ("stride_n", ctypes.c_int64), ("stride_h", ctypes.c_int64)]


class KnnTiles(ctypes.Structure):
    _fields_ = [("start", ctypes.c_void_p), ("src", ctypes.c_void_p), ("nsrc", ctypes.c_void_p),
                ("slot", ctypes.c_void_p), ("num_tiles", ctypes.c_int32), ("max_rows", ctypes.c_int32)]


class BsaArgs(ctypes.Structure):
    _fields_ = [
        ("batch", ctypes.c_int32), ("seq_len", ctypes.c_int32),
        ("num_q_heads", ctypes.c_int32), ("num_kv_heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32), ("block_attn_size", ctypes.c_int32),
        ("sparse_block_size", ctypes.c_int32), ("sparse_block_count", ctypes.c_int32),
        ("mode", ctypes.c_int32), ("softmax_scale", ctypes.c_float),
        ("q", Bnhd), ("k", Bnhd), ("v", Bnhd),
        ("weights", ctypes.c_void_p),
        ("w_stride_s", ctypes.c_int64), ("w_stride_b", ctypes.c_int64),
        ("w_stride_n", ctypes.c_int64), ("w_stride_h", ctypes.c_int64),
        ("out", ctypes.c_void_p),
        ("block_indices_out", ctypes.c_void_p),
        ("out_stride_b", ctypes.c_int64), ("out_stride_n", ctypes.c_int64),
    ]


class ProjArgs(ctypes.Structure):
    _fields_ = [
        ("x", ctypes.c_void_p), ("x_stride_n", ctypes.c_int64), ("x_stride_b", ctypes.c_int64),
        ("dim", ctypes.c_int32), ("weight_rows", ctypes.c_int32), ("weight", ctypes.c_void_p),
        ("rope_cos", ctypes.c_void_p), ("rope_sin", ctypes.c_void_p),
        ("q", ctypes.c_void_p), ("k", ctypes.c_void_p), ("v", ctypes.c_void_p), ("weights", ctypes.c_void_p),
    ]


_lock = threading.Lock()
_lib = None


def _declare(lib: ctypes.CDLL) -> None:
    c_int, c_i32, c_size, c_vp, c_f = ctypes.c_int, ctypes.c_int32, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_float
    P = ctypes.POINTER
    lib.mosaic_bsa_workspace_size.argtypes = [P(BsaArgs)]
    lib.mosaic_bsa_workspace_size.restype = c_size
    lib.mosaic_bsa_fwd.argtypes = [P(BsaArgs), c_vp, c_size, c_vp]
    lib.mosaic_bsa_fwd.restype = c_int
    lib.mosaic_bsa_fwd_noalloc.argtypes = [P(BsaArgs), c_vp]
    lib.mosaic_bsa_fwd_noalloc.restype = c_int
    lib.mosaic_bsa_fwd_profiled.argtypes = [P(BsaArgs), c_vp, c_size, c_vp, P(c_vp)]
    lib.mosaic_bsa_fwd_profiled.restype = c_int
    lib.mosaic_bsa_fwd_stage.argtypes = [P(BsaArgs), c_vp, c_size, c_vp, c_int]
    lib.mosaic_bsa_fwd_stage.restype = c_int
    lib.mosaic_bsa_fwd_rope.argtypes = [P(BsaArgs), c_vp, c_vp, c_vp, c_vp, c_vp, c_size, c_vp]
    lib.mosaic_bsa_fwd_rope.restype = c_int
    lib.mosaic_bsa_fwd_proj.argtypes = [P(BsaArgs), P(ProjArgs), c_vp, c_size, c_vp]
    lib.mosaic_bsa_fwd_proj.restype = c_int
    lib.mosaic_knn_interp_fwd.argtypes = [Bnhd, Bnhd, c_vp, c_vp, c_vp, c_i32, c_i32, c_i32, c_i32, c_i32, c_i32,
                                          c_f, c_vp, c_vp]
    lib.mosaic_knn_interp_fwd.restype = c_int
    lib.mosaic_knn_interp_fwd_ordered.argtypes = [Bnhd, Bnhd, c_vp, c_vp, c_vp, c_vp, c_i32, c_i32, c_i32, c_i32,
                                                  c_i32, c_i32, c_f, c_vp, c_vp]
    lib.mosaic_knn_interp_fwd_ordered.restype = c_int
    lib.mosaic_knn_interp_fwd_ex.argtypes = [Bnhd, Bnhd, c_vp, c_vp, c_vp, c_vp, P(KnnTiles), c_i32, c_i32,
                                             c_i32, c_i32, c_i32, c_i32, c_f, ctypes.c_uint32, c_vp, c_vp]
    lib.mosaic_knn_interp_fwd_ex.restype = c_int
    c_i64 = ctypes.c_int64
    lib.mosaic_rms_norm_fwd.argtypes = [c_vp, c_vp, c_i32, c_i64, c_i32, c_i64, c_i64, c_vp, c_f, c_vp, c_vp,
                                        c_i32, c_vp]
    lib.mosaic_rms_norm_fwd.restype = c_int
    lib.mosaic_swiglu_fwd.argtypes = [c_vp, c_i32, c_i64, c_i32, c_i64, c_vp, c_i32, c_vp, c_vp]
    lib.mosaic_swiglu_fwd.restype = c_int
    lib.mosaic_resample_norm_fwd.argtypes = [c_vp, c_i64, c_vp, c_vp, c_vp, c_f, c_i64, c_i32, c_i32, c_i32, c_vp, c_vp]
    lib.mosaic_resample_norm_fwd.restype = c_int
    lib.mosaic_gate_softmax_fwd.argtypes = [c_vp, c_i64, c_i64, c_i32, c_i32, c_vp, c_vp]
    lib.mosaic_gate_softmax_fwd.restype = c_int
    lib.mosaic_add_merge_fwd.argtypes = [c_vp, c_vp, c_i64, c_i32, c_i32, c_i32, c_vp, c_vp, c_vp]
    lib.mosaic_add_merge_fwd.restype = c_int
    lib.mosaic_swiglu_linear_fwd.argtypes = [c_vp, c_i64, c_i32, c_i64, c_vp, c_i32, c_vp, c_i32, c_vp, c_vp]
    lib.mosaic_swiglu_linear_fwd.restype = c_int
    lib.mosaic_sparse_attn_bwd_workspace_size.argtypes = [c_i32, c_i32, c_i32]
    lib.mosaic_sparse_attn_bwd_workspace_size.restype = c_size
    lib.mosaic_sparse_attn_bwd.argtypes = [Bnhd, Bnhd, Bnhd, c_vp, c_vp, Bnhd, c_vp, c_i32, c_i32, c_i32, c_i32,
                                           c_i32, c_i32, c_i32, c_f, c_vp, c_vp, c_vp, c_vp, c_size, c_vp]
    lib.mosaic_sparse_attn_bwd.restype = c_int
    lib.mosaic_sparse_attn_fwd.argtypes = [Bnhd, Bnhd, Bnhd, c_vp, c_i32, c_i32, c_i32, c_i32, c_i32,
                                           c_i32, c_i32, c_f, c_vp, c_vp, c_vp]
    lib.mosaic_sparse_attn_fwd.restype = c_int
    lib.mosaic_sparse_attn_fwd_workspace_size.argtypes = [c_i32, c_i32, c_i32, c_i32]
    lib.mosaic_sparse_attn_fwd_workspace_size.restype = c_size
    lib.mosaic_sparse_attn_fwd_ws.argtypes = [Bnhd, Bnhd, Bnhd, c_vp, c_i32, c_i32, c_i32, c_i32, c_i32,
                                              c_i32, c_i32, c_f, c_vp, c_vp, c_vp, c_size, c_vp]
    lib.mosaic_sparse_attn_fwd_ws.restype = c_int
    lib.mosaic_block_attn_fwd.argtypes = [Bnhd, Bnhd, Bnhd, c_i32, c_i32, c_i32, c_i32, c_i32, c_i32, c_f,
                                          c_vp, c_vp]
    lib.mosaic_block_attn_fwd.restype = c_int
    lib.mosaic_dense_attn_fwd.argtypes = [Bnhd, Bnhd, Bnhd, c_i32, c_i32, c_i32, c_i32, c_i32, c_f, c_vp, c_vp]
    lib.mosaic_dense_attn_fwd.restype = c_int
    lib.mosaic_pool_mean_fwd.argtypes = [Bnhd, c_i32, c_i32, c_i32, c_i32, c_i32, c_vp, c_vp]
    lib.mosaic_pool_mean_fwd.restype = c_int
    lib.mosaic_attn_topk_workspace_size.argtypes = [c_i32, c_i32, c_i32]
    lib.mosaic_attn_topk_workspace_size.restype = c_size
    lib.mosaic_attn_topk_fwd.argtypes = [Bnhd, Bnhd, c_i32, c_i32, c_i32, c_i32, c_i32, c_i32, c_vp, c_vp,
                                         c_size, c_vp]
    lib.mosaic_attn_topk_fwd.restype = c_int
    lib.mosaic_bsa_strerror.argtypes = [c_int]
    lib.mosaic_bsa_strerror.restype = ctypes.c_char_p
    lib.mosaic_bsa_abi_version.argtypes = []
    lib.mosaic_bsa_abi_version.restype = c_int


def lib() -> ctypes.CDLL:
    """The loaded library (loaded once per process)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise MosaicLibraryError(
                    f"{LIB_PATH} is missing: build it with `python -m mosaic_amd.build` "
                    "(hipcc, gfx950). There is no CPU fallback.")
            handle = ctypes.CDLL(LIB_PATH)
            _declare(handle)
            ver = handle.mosaic_bsa_abi_version()
            if ver != ABI_VERSION:
                raise MosaicLibraryError(f"{LIB_PATH} has ABI version {ver}, expected {ABI_VERSION}")
            _lib = handle
    return _lib


def strerror(status: int) -> str:
    return lib().mosaic_bsa_strerror(status).decode()


def check(status: int, what: str) -> None:
    if status != 0:
        raise RuntimeError(f"{what}: {strerror(status)} (mosaic status {status})")

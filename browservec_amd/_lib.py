"""ctypes binding of libbrowservec_hip.so (declared in include/browservec_hip.h).

The library is built in-tree by ``python -m browservec_amd.build``.  There is
no CPU fallback: if the shared object is missing, importing the native layer
raises, so nothing silently runs elsewhere.
"""

from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "lib", "libbrowservec_hip.so")

BV_OK = 0
BV_E_INVALID = 1
BV_E_UNSUPPORTED = 2
BV_E_DEVICE_LOST = 3
BV_E_OOM = 4
BV_E_HIP = 5
BV_E_STATE = 6

KIND_FLAT, KIND_QUANT, KIND_IVF, KIND_IVFQUANT = 0, 1, 2, 3
METRICS = {"cosine": 0, "dot": 1, "l2": 2}
SCORERS = {"asym": 0, "hamming": 1, "int8sym": 2}


class BVError(RuntimeError):
    """A failed library call; ``code`` is the BV_E_* status."""

    def __init__(self, code: int, msg: str):
        super().__init__(msg)
        self.code = code


class IndexDesc(ctypes.Structure):
    _fields_ = [
        ("size", ctypes.c_uint32),
        ("kind", ctypes.c_uint32),
        ("dim", ctypes.c_uint32),
        ("metric", ctypes.c_uint32),
        ("bits", ctypes.c_uint32),
        ("scorer", ctypes.c_uint32),
        ("seed", ctypes.c_uint32),
        ("has_seed", ctypes.c_uint32),
        ("rounds", ctypes.c_uint32),
        ("chunk_rows", ctypes.c_uint32),
        ("nlist", ctypes.c_uint32),
        ("nprobe", ctypes.c_uint32),
        ("sample_size", ctypes.c_uint32),
        ("train_size", ctypes.c_uint32),
        ("iters", ctypes.c_uint32),
        ("ivf_seed", ctypes.c_uint32),
        ("has_ivf_seed", ctypes.c_uint32),
        ("target_recall", ctypes.c_float),
        ("ivf_incremental", ctypes.c_uint32),
    ]


class IndexStats(ctypes.Structure):
    _fields_ = [
        ("rows", ctypes.c_uint64),
        ("dim", ctypes.c_uint32),
        ("padded_dim", ctypes.c_uint32),
        ("words_per_row", ctypes.c_uint32),
        ("bits", ctypes.c_uint32),
        ("chunk_count", ctypes.c_uint32),
        ("nlist", ctypes.c_uint32),
        ("nprobe", ctypes.c_uint32),
        ("tuned_recall", ctypes.c_float),
        ("last_query_ms", ctypes.c_double),
        ("last_query_gpu_ms", ctypes.c_double),
        ("build_ms", ctypes.c_double),
        ("device_bytes", ctypes.c_uint64),
        ("last_scanned_rows", ctypes.c_uint64),
        ("build_exact_rows", ctypes.c_uint64),
    ]


vp = ctypes.c_void_p
u32 = ctypes.c_uint32
u64 = ctypes.c_uint64
i32 = ctypes.c_int

# name -> argtypes (all return int status unless listed in _RESTYPE)
SIGNATURES = {
    "bv_last_error": [],
    "bv_abi_version": [],
    "bv_device_open": [ctypes.c_int, ctypes.POINTER(vp)],
    "bv_device_close": [vp],
    "bv_device_is_lost": [vp, ctypes.POINTER(ctypes.c_int)],
    "bv_debug_inject": [vp, ctypes.c_int],
    "bv_device_info": [vp, ctypes.c_char_p, u32, ctypes.POINTER(u32), ctypes.POINTER(u64)],
    "bv_index_create": [vp, ctypes.POINTER(IndexDesc), ctypes.POINTER(vp)],
    "bv_index_destroy": [vp],
    "bv_index_size": [vp, ctypes.POINTER(u64)],
    "bv_index_append": [vp, vp, u64, u64],
    "bv_index_query": [vp, vp, u32, vp, vp, vp],
    "bv_index_query_masked": [vp, vp, u32, vp, u64, vp, vp, vp],
    "bv_index_query_batch": [vp, vp, u32, u32, vp, vp, vp],
    "bv_index_set_nprobe": [vp, u32],
    "bv_index_rerank": [vp, vp, vp, u32, u32, vp, vp, vp],
    "bv_index_query_rows": [vp, vp, vp, u64, u32, vp, vp, vp],
    "bv_index_set_query_streams": [vp, u32],
    "bv_graph_create": [vp, u32, u32, u32, vp],
    "bv_graph_destroy": [vp],
    "bv_graph_append": [vp, vp, u64, u64],
    "bv_graph_upload": [vp, vp, u64],
    "bv_graph_search": [vp, vp, u32, u32, u32, u32, vp, vp, vp],
    "bv_graph_search_beams": [vp, vp, u32, vp, u32, u32, u32, vp, vp],
    "bv_index_query_rows_masked": [vp, vp, vp, u64, u32, vp, vp, vp],
    "bv_index_search": [vp, vp, u32, u32, u32, vp, vp, vp],
    "bv_index_search_device": [vp, vp, u32, u32, u32, vp, vp, vp],
    "bv_index_search_device_noalloc": [vp, vp, u32, u32, u32, vp, vp, vp],
    "bv_index_append_device": [vp, vp, u64],
    "bv_index_sync": [vp],
    "bv_index_stream": [vp, ctypes.POINTER(vp)],
    "bv_index_kernel_timing": [vp, ctypes.c_int, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(u64)],
    "bv_index_get_stats": [vp, ctypes.POINTER(IndexStats)],
    "bv_index_export_codes": [vp, u64, u64, vp, vp],
    "bv_index_export_scores": [vp, vp, vp],
    "bv_index_export_rotated_query": [vp, vp, vp],
    "bv_index_build": [vp],
    "bv_index_export_ivf": [vp, vp, vp, vp],
    "bv_index_export_probe_scores": [vp, vp, u32, vp],
    "bv_index_save_section": [vp, vp, u64, vp],
    "bv_index_load_section": [vp, vp, u64, u64, vp, u64],
}
_RESTYPE = {"bv_last_error": ctypes.c_char_p}

_lib = None


def load() -> ctypes.CDLL:
    """Load the HIP library, failing loudly when it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"{LIB_PATH} is missing: build it with `python -m browservec_amd.build` "
            "(there is no CPU fallback for the search path)"
        )
    lib = ctypes.CDLL(LIB_PATH)
    for name, args in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = _RESTYPE.get(name, ctypes.c_int)
    _lib = lib
    return lib


def check(rc: int) -> None:
    if rc != BV_OK:
        msg = load().bv_last_error().decode(errors="replace")
        raise BVError(rc, msg)

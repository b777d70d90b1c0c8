"""ctypes binding of libgpusparse.so (the gfx950 kernels) and libgs_synth.so.

Only plain pointers, sizes and a hipStream_t cross this boundary; PyTorch owns
every device buffer.  The library is loaded from this package directory, where
``gpu-sparse_amd/csrc/Makefile`` puts it.  Nothing here falls back to another
implementation: a missing library or a missing GPU raises.
"""
from __future__ import annotations

import ctypes as C
import os
import threading

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libgpusparse.so")
SYNTH_PATH = os.path.join(_HERE, "libgs_synth.so")

GS_OK, GS_EINVAL, GS_EHIP, GS_ENOSPC = 0, 1, 2, 3
GS_W_F32, GS_W_F16, GS_W_U8 = 0, 1, 2
GS_ROW_DONE, GS_ROW_DENSE = 0, 1
GS_SEARCH_PHASES = 8
NOALLOC_SCRATCH_BYTES = 256 << 20   # GS_NOALLOC_SCRATCH_BYTES
PHASE_NAMES = ("query_prep", "heavy_terms", "threshold_seed", "scoring", "candidate_select", "fp64_rescore",
               "final_sort")
ABI_VERSION = 10

WTYPE_OF_DTYPE = {torch.float32: GS_W_F32, torch.float16: GS_W_F16, torch.uint8: GS_W_U8}


class GsIndex(C.Structure):
    """Mirror of ``struct gs_index`` in include/gpusparse.h."""

    _fields_ = [
        ("doc_ids_d", C.c_void_p),
        ("weights_d", C.c_void_p),
        ("offsets_d", C.c_void_p),
        ("lengths_d", C.c_void_p),
        ("max_abs_d", C.c_void_p),
        ("dup_d", C.c_void_p),
        ("tile_bounds_d", C.c_void_p),
        ("n_slots", C.c_int64),
        ("n_docs", C.c_int64),
        ("vocab", C.c_int32),
        ("wtype", C.c_int32),
        ("tile_log2", C.c_int32),
        ("n_tiles", C.c_int32),
        ("fwd_ptr_d", C.c_void_p),
        ("fwd_terms_d", C.c_void_p),
        ("fwd_weights_d", C.c_void_p),
        ("packed_d", C.c_void_p),
        ("packed_tile_log2", C.c_int32),
        ("packed_shift", C.c_int32),
        ("heavy_d", C.c_void_p),
        ("head_d", C.c_void_p),
        ("head_rank_d", C.c_void_p),
    ]


def heavy_term_count() -> int:
    """GS_HEAVY_TERMS of the loaded library (gs_heavy_term_count): the heavy
    lists per index, and the hybrid search's matrix-product terms."""
    return int(lib().gs_heavy_term_count())


HEAD_BLOCK = 512  # GS_HEAD_BLOCK


class GsSearchOpts(C.Structure):
    """Mirror of ``struct gs_search_opts``."""

    _fields_ = [
        ("sample_tiles", C.c_int32),
        ("cand_cap", C.c_int32),
        ("unroll", C.c_int32),
        ("waves", C.c_int32),
        ("ev_score_begin", C.c_void_p),
        ("ev_score_end", C.c_void_p),
        ("tiles_per_wg", C.c_int32),
        ("ev_phases", C.POINTER(C.c_void_p)),
        ("batch_order", C.c_int32),
        ("no_hybrid", C.c_int32),
    ]


class GsSynthSpec(C.Structure):
    """Mirror of ``gs_synth_spec`` in csrc/synth.c."""

    _fields_ = [
        ("n_rows", C.c_int64),
        ("vocab", C.c_int32),
        ("wmode", C.c_int32),
        ("zipf_s", C.c_double),
        ("nnz_mean", C.c_double),
        ("nnz_sigma", C.c_double),
        ("nnz_min", C.c_int32),
        ("nnz_max", C.c_int32),
        ("w_mu", C.c_double),
        ("w_sigma", C.c_double),
        ("w_max", C.c_double),
        ("n_head_forced", C.c_int32),
        ("head_pool", C.c_int32),
        ("seed", C.c_uint64),
        ("stream", C.c_uint64),
    ]


_P = C.c_void_p
_I32, _I64, _SZ = C.c_int32, C.c_int64, C.c_size_t

# name -> (restype, argtypes); the exported C ABI of include/gpusparse.h
class GsSearchPlanInfo(C.Structure):
    """Mirror of ``struct gs_search_plan_info`` in include/gpusparse.h."""

    _fields_ = [("seed_tiles", C.c_int32), ("group_size", C.c_int32), ("unroll", C.c_int32),
                ("tiles_per_wg", C.c_int32), ("packed", C.c_int32), ("hybrid", C.c_int32),
                ("cand_cap", C.c_int32)]


SIGNATURES = {
    "gs_query_version": (C.c_int, []),
    "gs_heavy_term_count": (C.c_int, []),
    "gs_last_error": (C.c_char_p, []),
    "gs_index_count": (C.c_int, [_P, _I64, _I32, _P, _P, _P, _P, _P]),
    "gs_index_fill_workspace": (_SZ, [_I64, _I32]),
    "gs_index_fill": (C.c_int, [_P, _P, _P, _I32, _I64, _I64, _I32, _P, _P, _P, _I64, _P, _P, _P, _P,
                                _P, _SZ, _P]),
    "gs_list_max": (C.c_int, [_P, _I32, _P, _P, _I32, _P, _P, _P, _SZ, _P]),
    "gs_check_lists": (C.c_int, [_P, _P, _P, _I32, _P, _P, _P, _P]),
    "gs_chunk_bounds": (C.c_int, [_P, _P, _P, _I32, _I64, _I64, _P, _P]),
    "gs_tile_bounds": (C.c_int, [_P, _P, _P, _I32, _I64, _I32, _P, _P]),
    "gs_forward_fill_workspace": (_SZ, [_I64, _I32]),
    "gs_forward_fill": (C.c_int, [_P, _P, _I32, _P, _P, _I32, _I64, _I64, _P, _P, _P, _P, _SZ, _P]),
    "gs_pack_postings": (C.c_int, [_P, _P, _I32, _I64, _P, _P, _I32, _I64, _I32, _I32, _P, _P]),
    "gs_rows_sorted": (C.c_int, [_P, _P, _I64, _P, _P]),
    "gs_pack_shift": (C.c_int, [C.c_float, C.POINTER(C.c_int32)]),
    "gs_heavy_terms": (C.c_int, [_P, _I32, _P, _P]),
    "gs_head_fill": (C.c_int, [_P, _P, _I32, _P, _P, _I32, _P, _I32, _I64, _I64, _P, _P, _P]),
    "gs_search_workspace": (C.c_int, [C.POINTER(GsIndex), _I32, _I32, _I32, C.POINTER(GsSearchOpts),
                                      C.POINTER(_SZ)]),
    "gs_search_plan": (C.c_int, [C.POINTER(GsIndex), _I32, _I32, _I32, C.POINTER(GsSearchOpts),
                                 C.POINTER(GsSearchPlanInfo)]),
    "gs_search": (C.c_int, [C.POINTER(GsIndex), _P, _P, _I32, _I32, _I32, C.POINTER(GsSearchOpts), _P, _P,
                            _P, _P, _SZ, _P]),
    "gs_search_noalloc": (C.c_int, [C.POINTER(GsIndex), _P, _P, _I32, _I32, _I32, C.POINTER(GsSearchOpts), _P, _P,
                                    _P, _P]),
    "gs_search_counts": (C.c_int, [C.POINTER(GsIndex), _I32, _I32, _I32, C.POINTER(GsSearchOpts), _P, _SZ, _P, _P,
                                   _P]),
    "gs_search_dense_workspace": (C.c_int, [C.POINTER(GsIndex), _I32, C.POINTER(_SZ)]),
    "gs_search_dense": (C.c_int, [C.POINTER(GsIndex), _P, _P, _I32, _I32, _I32, _P, _I32, _P, _P, _P, _SZ,
                                  _P]),
    "gs_compacted_topk_workspace": (_SZ, [_I32, _I32]),
    "gs_compacted_topk": (C.c_int, [_P, _I64, _I32, _I64, _P, _I32, _I32, _P, _P, _P, _P, _SZ, _P]),
    "gs_scatter_add": (C.c_int, [C.POINTER(GsIndex), _P, _P, _P, _P, _I32, _I32, _P, _I64, _I64, _I64,
                                 _I32, _P]),
}

SYNTH_SIGNATURES = {
    "gs_synth_count": (C.c_int64, [C.POINTER(GsSynthSpec), _P, C.c_int]),
    "gs_synth_fill": (C.c_int, [C.POINTER(GsSynthSpec), _P, _P, _P, C.c_int]),
    "gs_f32_to_f16_bits": (C.c_uint16, [C.c_float]),
    "gs_f32_to_f16_array": (None, [_P, _P, _I64, C.c_int]),
}

_lock = threading.Lock()
_lib = None
_synth = None


def _bind(path, sigs):
    lib = C.CDLL(path)
    for name, (res, args) in sigs.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


def lib():
    """The loaded libgpusparse.so.  Raises if it has not been built."""
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                if not os.path.exists(LIB_PATH):
                    raise RuntimeError(
                        f"{LIB_PATH} is missing: build the HIP library first "
                        "(make -C gpu-sparse_amd/csrc, or __graft_entry__.build()).")
                L = _bind(LIB_PATH, SIGNATURES)
                v = L.gs_query_version()
                if v != ABI_VERSION:
                    raise RuntimeError(f"libgpusparse ABI version {v}, expected {ABI_VERSION}")
                _lib = L
    return _lib


def synth_lib():
    global _synth
    if _synth is None:
        with _lock:
            if _synth is None:
                if not os.path.exists(SYNTH_PATH):
                    raise RuntimeError(f"{SYNTH_PATH} is missing: run make -C gpu-sparse_amd/csrc")
                _synth = _bind(SYNTH_PATH, SYNTH_SIGNATURES)
    return _synth


def check(rc: int, what: str) -> None:
    """Maps a library status code onto the reference's exception types."""
    if rc == GS_OK:
        return
    msg = (lib().gs_last_error() or b"").decode(errors="replace")
    if rc == GS_EINVAL:
        raise ValueError(f"{what}: {msg}")
    raise RuntimeError(f"{what} failed ({rc}): {msg}")


def require_gpu(device=None) -> torch.device:
    """The device to run on; raises when no GPU is visible, as the reference
    plug-in does (lsr_benchmark_engine/gpusparse_retrieval.py:179-181)."""
    if not torch.cuda.is_available():
        raise RuntimeError("GPUSparse requires a GPU device; none was visible.")
    dev = torch.device(device if device is not None else "cuda:0")
    if dev.type != "cuda":
        raise RuntimeError(f"GPUSparse kernels run on a GPU device, not {dev}")
    if dev.index is None:
        dev = torch.device("cuda", torch.cuda.current_device())
    return dev


def stream_ptr(device: torch.device) -> int:
    """hipStream_t of the current torch stream on `device`."""
    return torch.cuda.current_stream(device).cuda_stream


def ptr(t) -> int | None:
    return None if t is None else t.data_ptr()

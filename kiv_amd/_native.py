"""ctypes binding of libkiv_hip.so (declarations in include/kiv_hip.h).

torch is imported first so that the library binds to the HIP runtime torch
already loaded (one runtime per process: torch's streams and device pointers
are then valid in the library).  A missing library is an error, never a
fallback: every caller of :func:`lib` needs the HIP kernels.
"""

from __future__ import annotations

import ctypes as C
import os
import threading
from pathlib import Path

import torch  # noqa: F401  (load torch's HIP runtime before the library)

LIB_PATH = Path(os.environ.get("KIV_LIB_PATH") or Path(__file__).resolve().parent / "_lib" / "libkiv_hip.so")

KIV_OK = 0
ERR_INVALID, ERR_HIP, ERR_OOM, ERR_UNSUPPORTED, ERR_STATE = 1, 2, 3, 4, 5
DTYPE_F32, DTYPE_F16, DTYPE_BF16 = 0, 1, 2
TIER_HOST, TIER_HBM, TIER_SPLIT = 0, 1, 2
ROUND_ACTIVATION, ROUND_FP32 = 0, 1
MASK_NONE, MASK_BOOL, MASK_F32, MASK_F16, MASK_BF16, MASK_CAUSAL = 0, 1, 2, 3, 4, 5
RETRIEVE_PRUNE = 1
STAGES = ("evict_append", "evict_finalize", "coarse_scan", "coarse_select", "fine_scan", "fine_select",
          "gather", "attend")

_I64x3 = C.c_int64 * 3
_I64x4 = C.c_int64 * 4


class StoreConfig(C.Structure):
    _fields_ = [
        ("batch", C.c_int32), ("num_q_heads", C.c_int32), ("num_kv_heads", C.c_int32),
        ("head_dim", C.c_int32), ("page_size", C.c_int32), ("dtype", C.c_int32),
        ("cold_tier", C.c_int32), ("score_rounding", C.c_int32), ("reserve_tokens", C.c_int64),
    ]


class StoreInfo(C.Structure):
    _fields_ = [
        ("cold_length", C.c_int64), ("num_pages", C.c_int64), ("partial_len", C.c_int64),
        ("k_cold_bytes", C.c_int64), ("v_cold_bytes", C.c_int64), ("summary_bytes", C.c_int64),
        ("partial_bytes", C.c_int64), ("reserved_bytes", C.c_int64), ("reserved_device_bytes", C.c_int64),
        ("reserved_host_bytes", C.c_int64), ("readahead_bytes", C.c_int64),
    ]


class RetrieveArgs(C.Structure):
    _fields_ = [
        ("q", C.c_void_p), ("q_stride", _I64x4), ("q_len", C.c_int32), ("scaling", C.c_float),
        ("top_pages", C.c_int32), ("out_width", C.c_int32), ("reuse_candidates", C.c_int32),
        ("flags", C.c_int32), ("k_out", C.c_void_p), ("v_out", C.c_void_p), ("idx_out", C.c_void_p),
        ("pages_out", C.c_void_p), ("union_count_out", C.c_void_p), ("stats_out", C.c_void_p),
        ("stats_accum", C.c_void_p), ("append_k", C.c_void_p), ("append_v", C.c_void_p),
        ("append_k_stride", _I64x3), ("append_v_stride", _I64x3), ("append_tokens", C.c_int64),
        ("hot_src_k", C.c_void_p), ("hot_src_v", C.c_void_p), ("hot_src_k_stride", _I64x3),
        ("hot_src_v_stride", _I64x3), ("hot_dst_k", C.c_void_p), ("hot_dst_v", C.c_void_p),
        ("hot_dst_k_stride", _I64x3), ("hot_dst_v_stride", _I64x3), ("hot_tokens", C.c_int64),
    ]


class AttentionArgs(C.Structure):
    _fields_ = [
        ("batch", C.c_int32), ("num_q_heads", C.c_int32), ("num_kv_heads", C.c_int32),
        ("head_dim", C.c_int32), ("q_len", C.c_int32), ("dtype", C.c_int32),
        ("q", C.c_void_p), ("q_stride", _I64x4),
        ("cold_k", C.c_void_p), ("cold_v", C.c_void_p), ("cold_len", C.c_int32), ("hot_len", C.c_int32),
        ("hot_k", C.c_void_p), ("hot_v", C.c_void_p), ("hot_k_stride", _I64x3), ("hot_v_stride", _I64x3),
        ("mask", C.c_void_p), ("mask_kind", C.c_int32), ("_pad", C.c_int32), ("mask_stride", _I64x4),
        ("scaling", C.c_float), ("_pad2", C.c_int32),
        ("out", C.c_void_p), ("workspace", C.c_void_p), ("workspace_bytes", C.c_size_t),
    ]


# Every symbol include/kiv_hip.h declares: name -> (restype, argtypes).
SIGNATURES = {
    "kiv_version": (C.c_int, []),
    "kiv_last_error": (C.c_char_p, []),
    "kiv_store_create": (C.c_int, [C.POINTER(StoreConfig), C.c_int, C.POINTER(C.c_void_p)]),
    "kiv_store_destroy": (C.c_int, [C.c_void_p]),
    "kiv_store_reset": (C.c_int, [C.c_void_p]),
    "kiv_store_info": (C.c_int, [C.c_void_p, C.POINTER(StoreInfo)]),
    "kiv_evict": (C.c_int, [C.c_void_p, C.c_void_p, _I64x3, C.c_void_p, _I64x3, C.c_int64, C.c_void_p]),
    "kiv_max_union_pages": (C.c_int, [C.c_void_p, C.c_int32, C.c_int32, C.POINTER(C.c_int64)]),
    "kiv_retrieve": (C.c_int, [C.c_void_p, C.POINTER(RetrieveArgs), C.c_void_p]),
    "kiv_fine_scan_stats": (C.c_int, [C.c_void_p, C.POINTER(C.c_int64), C.POINTER(C.c_int64)]),
    "kiv_store_read_summaries": (C.c_int, [C.c_void_p, C.c_int64, C.c_int64, C.c_void_p, C.c_void_p,
                                           C.c_void_p]),
    "kiv_store_read_tokens": (C.c_int, [C.c_void_p, C.c_int64, C.c_int64, C.c_void_p, C.c_void_p,
                                        C.c_void_p]),
    "kiv_profile_enable": (C.c_int, [C.c_void_p, C.c_int]),
    "kiv_profile_read": (C.c_int, [C.c_void_p, C.c_int64 * len(STAGES), C.c_double * len(STAGES)]),
    "kiv_probe_read_bandwidth": (C.c_int, [C.c_int32, C.c_size_t, C.c_int32, C.c_int32, C.c_int32,
                                           C.POINTER(C.c_double), C.c_void_p]),
    "kiv_attention_workspace_size": (C.c_size_t, [C.c_int32] * 7),
    "kiv_decode_attention": (C.c_int, [C.POINTER(AttentionArgs), C.c_void_p]),
    "kiv_decode_attention_noalloc": (C.c_int, [C.POINTER(AttentionArgs), C.c_void_p]),
    "kiv_retrieve_attend": (C.c_int, [C.c_void_p, C.POINTER(RetrieveArgs), C.POINTER(AttentionArgs), C.c_void_p]),
    "kiv_prefill_attention": (C.c_int, [C.POINTER(AttentionArgs), C.c_void_p]),
    "kiv_prefill_workspace_size": (C.c_size_t, [C.c_int32] * 6),
}

_lock = threading.Lock()
_lib: C.CDLL | None = None


def lib() -> C.CDLL:
    """The loaded library; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise RuntimeError(
                    f"{LIB_PATH} is missing: build the HIP library first "
                    "(python -m kiv_amd.build, or __graft_entry__.build())"
                )
            handle = C.CDLL(str(LIB_PATH))
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(handle, name)
                fn.restype = res
                fn.argtypes = args
            _lib = handle
    return _lib


class KivError(RuntimeError):
    """A failed C-ABI call; ``code`` is its KIV_ERR_* value."""

    def __init__(self, message: str, code: int) -> None:
        super().__init__(message)
        self.code = code

    @property
    def refused(self) -> bool:
        """Refused by an argument, shape or state check: the call changed nothing."""
        return self.code in (ERR_INVALID, ERR_UNSUPPORTED, ERR_STATE)


def check(rc: int, what: str) -> None:
    if rc != KIV_OK:
        msg = lib().kiv_last_error().decode(errors="replace")
        raise KivError(f"{what} failed (code {rc}): {msg}", rc)


_DTYPES = {torch.float32: DTYPE_F32, torch.float16: DTYPE_F16, torch.bfloat16: DTYPE_BF16}
_MASK_KINDS = {torch.bool: MASK_BOOL, torch.float32: MASK_F32, torch.float16: MASK_F16,
               torch.bfloat16: MASK_BF16}


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _DTYPES[dtype]
    except KeyError:
        raise TypeError(f"KIV HIP kernels support float32, float16 and bfloat16, not {dtype}") from None


def mask_kind(dtype: torch.dtype) -> int:
    try:
        return _MASK_KINDS[dtype]
    except KeyError:
        raise TypeError(f"unsupported attention mask dtype {dtype}") from None


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_ptr(device: torch.device) -> int:
    """Raw hipStream_t of torch's current stream on ``device``."""
    idx = device.index
    if idx is None:
        idx = torch.cuda.current_device()
    if _raw_stream is not None:
        return _raw_stream(idx)
    return torch.cuda.current_stream(idx).cuda_stream


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


_ARRAYS = {3: _I64x3, 4: _I64x4}
_strides_cache: dict[tuple, C.Array] = {}


def strides(t: torch.Tensor, n: int):
    """The first n strides of t (elements) as a ctypes int64 array; size-1
    dimensions get stride 0.  The arrays are shared between calls (cached
    per shape and strides): callers pass them on and never modify them."""
    key = (t.shape, t.stride(), n)
    arr = _strides_cache.get(key)
    if arr is None:
        shape, st, _ = key
        arr = _ARRAYS.get(n, C.c_int64 * n)(*[0 if shape[i] == 1 else st[i] for i in range(n)])
        if len(_strides_cache) < 4096:
            _strides_cache[key] = arr
    return arr

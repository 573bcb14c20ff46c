"""Attention over [retrieved ; hot] on the HIP kernels.

``decode_attention`` (kiv_decode_attention) replaces the wrapper's two
``torch.cat`` calls, the mask widening and the attention call
(kiv/middleware.py:330-354) for decode steps: retrieved keys are always
attended, an optional mask applies to the hot columns only.
``prefill_attention`` (kiv_prefill_attention) does the same for queries of
many positions on the matrix cores: prefill chunks (the original attention
of kiv/middleware.py:174-260) and long queries with a cold tier.
"""

from __future__ import annotations

import ctypes as C
import threading

import torch

from . import _native as nat

_ws_lock = threading.Lock()
_workspaces: dict[int, torch.Tensor] = {}
_ws_sizes: dict[tuple, int] = {}
_NO_STRIDES = nat._I64x4()


def _workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    """Split-partials scratch per device (fully rewritten by every call).

    Shared by every call on the device, so concurrent calls on different
    streams of one device must not overlap.
    """
    idx = device.index or 0
    ws = _workspaces.get(idx)
    if ws is not None and ws.numel() >= nbytes:
        return ws
    with _ws_lock:
        ws = _workspaces.get(idx)
        if ws is None or ws.numel() < nbytes:
            ws = torch.empty(max(nbytes, 1 << 20), dtype=torch.uint8, device=device)
            _workspaces[idx] = ws
        return ws


def _decode_ws_size(B: int, hq: int, hkv: int, D: int, Q: int, cold_len: int, T: int) -> int:
    key = (B, hq, hkv, D, Q, cold_len, T)
    n = _ws_sizes.get(key)
    if n is None:
        n = nat.lib().kiv_attention_workspace_size(B, hq, hkv, D, Q, cold_len, T)
        if len(_ws_sizes) < 4096:
            _ws_sizes[key] = n
    return n


def _mask_view(mask: torch.Tensor | None, hot_len: int, causal: bool = False):
    """(pointer, kind, strides b,h,q,t) of a 2-D or 4-D mask over hot columns."""
    if mask is None:
        return None, nat.MASK_CAUSAL if causal else nat.MASK_NONE, _NO_STRIDES
    if mask.shape[-1] != hot_len:
        raise ValueError(f"mask covers {mask.shape[-1]} columns, hot window has {hot_len}")
    if mask.dim() == 2:
        mask = mask[:, None, None, :]
    if mask.dim() != 4:
        raise ValueError(f"unsupported mask rank {mask.dim()}")
    return mask.data_ptr(), nat.mask_kind(mask.dtype), nat.strides(mask, 4)


def fill_args(args, query: torch.Tensor, cold_len: int, hot_k: torch.Tensor, hot_v: torch.Tensor,
              mask: torch.Tensor | None, scaling: float, causal: bool = False, workspace: bool = True):
    """Fill ``args`` (an AttentionArgs, reused by callers that attend often)
    for this query and hot window, retrieved keys still unset; returns the
    output tensor and the tensors the launch reads."""
    B, hq, Q, D = query.shape
    hkv = hot_k.shape[1]
    dt = query.dtype
    if hot_k.dtype != dt:
        hot_k, hot_v = hot_k.to(dt), hot_v.to(dt)
    if hot_k.stride(3) != 1:
        hot_k = hot_k.contiguous()
    if hot_v.stride(3) != 1:
        hot_v = hot_v.contiguous()
    q = query if query.stride(3) == 1 else query.contiguous()
    T = hot_k.shape[2]
    if workspace:
        ws = _workspace(query.device, _decode_ws_size(B, hq, hkv, D, Q, cold_len, T))
        args.workspace, args.workspace_bytes = ws.data_ptr(), ws.numel()
    else:
        args.workspace, args.workspace_bytes = None, 0
    out = torch.empty(B, Q, hq, D, dtype=dt, device=query.device)
    mptr, mkind, mstr = _mask_view(mask, T, causal)
    args.batch, args.num_q_heads, args.num_kv_heads, args.head_dim, args.q_len = B, hq, hkv, D, Q
    args.dtype = nat.dtype_code(dt)
    args.q, args.q_stride = q.data_ptr(), nat.strides(q, 4)
    args.cold_k = args.cold_v = None
    args.cold_len, args.hot_len = cold_len, T
    args.hot_k, args.hot_v = hot_k.data_ptr(), hot_v.data_ptr()
    args.hot_k_stride, args.hot_v_stride = nat.strides(hot_k, 3), nat.strides(hot_v, 3)
    args.mask, args.mask_kind, args.mask_stride = mptr, mkind, mstr
    args.scaling = scaling
    args.out = out.data_ptr()
    keep = (q, hot_k, hot_v) + ((mask,) if mask is not None else ())
    return out, keep


def _prepare(query: torch.Tensor, cold_len: int, hot_k: torch.Tensor, hot_v: torch.Tensor,
             mask: torch.Tensor | None, scaling: float, causal: bool = False, workspace: bool = True):
    """(new args without retrieved keys, output, tensors the launches read)."""
    args = nat.AttentionArgs()
    out, keep = fill_args(args, query, cold_len, hot_k, hot_v, mask, scaling, causal, workspace)
    return args, out, keep


def _set_cold(args, cold_k: torch.Tensor | None, cold_v: torch.Tensor | None, dt: torch.dtype):
    if cold_k is not None and (cold_k.dtype != dt or not cold_k.is_contiguous()):
        cold_k, cold_v = cold_k.to(dt).contiguous(), cold_v.to(dt).contiguous()
    args.cold_k, args.cold_v = nat.ptr(cold_k), nat.ptr(cold_v)
    return cold_k, cold_v


def decode_attention(query: torch.Tensor, cold_k: torch.Tensor | None, cold_v: torch.Tensor | None,
                     hot_k: torch.Tensor, hot_v: torch.Tensor, mask: torch.Tensor | None,
                     scaling: float) -> torch.Tensor:
    """softmax(q [cold; hot]^T * scaling + [0; mask]) [cold; hot] -> [B, Q, Hq, D]."""
    P = 0 if cold_k is None else cold_k.shape[2]
    args, out, _ = _prepare(query, P, hot_k, hot_v, mask, scaling)
    _set_cold(args, cold_k, cold_v, query.dtype)
    nat.check(nat.lib().kiv_decode_attention(C.byref(args), nat.stream_ptr(query.device)), "kiv_decode_attention")
    return out


def fused_supported(query: torch.Tensor, hot_k: torch.Tensor, mask: torch.Tensor | None) -> bool:
    """Shapes the merged kernel handles: one query position per step (decode),
    GQA groups of at most 64 rows, head_dim a multiple of 16 bytes."""
    if not query.is_cuda or query.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        return False
    B, hq, Q, D = query.shape
    hkv = hot_k.shape[1]
    if Q != 1 or hq % hkv:
        return False
    g = hq // hkv
    vec = 4 if query.dtype == torch.float32 else 8
    if g > 64 or g * D > 8192 or D % vec or D // vec > 64:
        return False
    if mask is not None and (mask.dim() not in (2, 4) or mask.dtype not in
                             (torch.bool, torch.float32, torch.float16, torch.bfloat16)):
        return False
    return True


def prefill_attention(query: torch.Tensor, cold_k: torch.Tensor | None, cold_v: torch.Tensor | None,
                      hot_k: torch.Tensor, hot_v: torch.Tensor, mask: torch.Tensor | None, scaling: float,
                      causal: bool = False) -> torch.Tensor:
    """softmax(q [cold; hot]^T * scaling + [0; mask]) [cold; hot] -> [B, Q, Hq, D]
    on the matrix cores.  With ``mask=None`` and ``causal`` the hot column t
    is visible to query row i iff t <= i + hot_len - Q."""
    P = 0 if cold_k is None else cold_k.shape[2]
    if mask is not None and mask.dim() == 4:
        B, hq, Q, _ = query.shape
        for n, (have, want) in enumerate(zip(mask.shape[:3], (B, hq, Q))):
            if have not in (1, want):
                raise ValueError(f"mask dim {n} is {have}, expected 1 or {want}")
    args, out, _ = _prepare(query, P, hot_k, hot_v, mask, scaling, causal=causal, workspace=False)
    B, hq, Q, D = query.shape
    need = nat.lib().kiv_prefill_workspace_size(B, hq, D, Q, P, hot_k.shape[2])
    if need:
        ws = _workspace(query.device, need)
        args.workspace, args.workspace_bytes = ws.data_ptr(), ws.numel()
    _set_cold(args, cold_k, cold_v, query.dtype)
    nat.check(nat.lib().kiv_prefill_attention(C.byref(args), nat.stream_ptr(query.device)),
              "kiv_prefill_attention")
    return out


_PREFILL_HEAD_DIMS = (32, 64, 96, 128, 192, 256)


def prefill_supported(query: torch.Tensor, hot_k: torch.Tensor, mask: torch.Tensor | None) -> bool:
    """Shapes the matrix-core attention handles: fp16/bf16, head_dim in
    32/64/96/128/192/256, a 2-D or 4-D mask of a supported dtype (or none)."""
    if not query.is_cuda or query.dtype not in (torch.float16, torch.bfloat16):
        return False
    B, hq, Q, D = query.shape
    hkv = hot_k.shape[1]
    if hq % hkv or D not in _PREFILL_HEAD_DIMS or B * hq > 65535:
        return False
    if mask is not None and (mask.dim() not in (2, 4) or mask.dtype not in
                             (torch.bool, torch.float32, torch.float16, torch.bfloat16)):
        return False
    return True

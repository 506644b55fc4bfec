"""Prefill attention over dense K/V rows: the torch-facing wrapper of
``bmx_prefill`` (include/bmx_prefill.h).

The reference's prefill (``_prefill_dense_attention``,
src/bmx/cache/chunked_attention.py:320-395) dequantizes the committed pages
to dense rows and calls torch SDPA with the model's mask.  The packed cache
keeps the dequant and attends here instead for the masks a cached prefill
carries: the causal mask of the last ``n_q`` positions (bottom-right aligned;
``n_q == n_kv`` is the ordinary causal mask) or none.  The kernel enqueues on
torch's current stream; any non-zero status raises with the library's
message (no fallback).
"""

from __future__ import annotations

import ctypes as ct

import torch

from . import _lib
from .k2b import DecodeWorkspace, _need, _stream

HEAD_DIM = 128
DTYPES = {torch.float16: 0, torch.bfloat16: 1}   # BMX_PREFILL_F16 / BF16

_WS: dict = {}


def supported(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> bool:
    """Whether bmx_prefill takes these operands: head dim 128, fp16 / bf16,
    16-byte aligned rows, K and V with the same strides, grouped heads."""
    def rows_ok(t):
        return (t.dim() == 3 and t.stride(-1) == 1 and t.stride(0) % 8 == 0 and t.stride(1) % 8 == 0
                and t.data_ptr() % 16 == 0)
    return (q.is_cuda and q.shape[-1] == HEAD_DIM and k.shape[-1] == HEAD_DIM and q.dtype in DTYPES
            and k.dtype == q.dtype and v.dtype == q.dtype and v.shape == k.shape and v.stride() == k.stride()
            and rows_ok(q) and rows_ok(k) and rows_ok(v) and k.stride(1) >= HEAD_DIM
            and q.shape[0] % k.shape[0] == 0)


def attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float, *, causal: bool,
              n_split: int = 0, out: torch.Tensor | None = None) -> torch.Tensor:
    """softmax(q k^T * scale [+ bottom-right causal mask]) v over grouped heads.

    q (h_kv * G, n_q, 128); k and v (h_kv, n_kv, 128) with the same strides;
    fp16 or bf16, rows contiguous.  Query head ``h * G + g`` reads kv head
    ``h``.  With ``causal`` query i sees keys ``j <= i + n_kv - n_q``.
    Returns (h_kv * G, n_q, 128) in q's dtype, contiguous."""
    _need(q.dim() == 3 and k.dim() == 3 and v.shape == k.shape, "q (Hq, n_q, 128), k and v (h_kv, n_kv, 128)")
    _need(q.shape[-1] == HEAD_DIM and k.shape[-1] == HEAD_DIM, "head_dim must be 128")
    _need(q.dtype in DTYPES and k.dtype == q.dtype and v.dtype == q.dtype, "q, k, v: one dtype, fp16 or bf16")
    _need(q.stride(-1) == 1 and k.stride(-1) == 1 and v.stride() == k.stride(), "rows contiguous; k, v same strides")
    _need(q.device == k.device == v.device and q.is_cuda, "operands on one HIP device")
    hq, n_q, _ = q.shape
    h_kv, n_kv, _ = k.shape
    _need(hq % h_kv == 0, "query heads must be a multiple of kv heads")
    if out is None:
        out = torch.empty(hq, n_q, HEAD_DIM, dtype=q.dtype, device=q.device)
    _need(out.shape == (hq, n_q, HEAD_DIM) and out.dtype == q.dtype and out.is_contiguous(), "out (Hq, n_q, 128)")
    a = _lib.PrefillArgs()
    a.q, a.q_stride_h, a.q_stride_t = q.data_ptr(), q.stride(0), q.stride(1)
    a.k, a.v, a.kv_stride_h, a.kv_stride_t = k.data_ptr(), v.data_ptr(), k.stride(0), k.stride(1)
    a.out = out.data_ptr()
    a.h_kv, a.n_q_groups, a.n_q, a.n_kv = h_kv, hq // h_kv, n_q, n_kv
    a.head_dim, a.dtype, a.causal, a.sm_scale = HEAD_DIM, DTYPES[q.dtype], int(bool(causal)), float(scale)
    a.n_split = int(n_split)
    L = _lib.lib()
    need = int(L.bmx_prefill_workspace_bytes(ct.byref(a)))
    if need:
        ws = _WS.setdefault(q.device, DecodeWorkspace()).get(need, q.device)
        a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel()
    _lib.check(L.bmx_prefill(ct.byref(a), _stream(q.device)), "bmx_prefill")
    return out

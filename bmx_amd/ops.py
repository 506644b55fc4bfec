"""The decode-path calls as ``torch.library`` custom operators.

``torch.ops.bmx.k2b_decode`` / ``k2b_append`` / ``rtn_decode`` / ``rtn_append``
are the same C-ABI calls as ``bmx_amd.k2b`` / ``bmx_amd.rtn`` (one ctypes call
each on the current stream), and ``torch.ops.bmx.prefill_attention`` the
prefill attention of ``bmx_amd.prefill`` (chunked_attention.py:320-395 calls
SDPA there), registered so that the dispatcher, FakeTensor
tracing, ``torch.compile`` (no graph break) and CUDA-graph capture see them as
single operators.  The reference exposes these steps as Python functions that
launch Triton kernels (cache/triton_dequant_attention.py:1232-1246 for the
fused decode, cache/packed_streaming.py:582-730 for the page commit); the
operator schema follows their arguments, with the codec constants passed by
value (inv_freq, codebook, sign words) instead of a constants object.

Only a device implementation is registered: a call on CPU tensors fails in
the dispatcher (no CPU fallback).  The fake implementations give the output's
shape and dtype without touching data.
"""

from __future__ import annotations

from typing import Optional

import torch

from . import k2b, prefill, rtn

_LIB = "bmx"


def _consts(inv_freq, rope_scaling, codebook, sign_bits) -> k2b.CodecConsts:
    return k2b.CodecConsts(tuple(float(x) for x in codebook), tuple(int(x) for x in sign_bits),
                           tuple(float(x) for x in inv_freq), float(rope_scaling))


def _tail_len(tail_len: Optional[torch.Tensor], tail_len_value: int):
    return tail_len if tail_len is not None else int(tail_len_value)


@torch.library.custom_op(f"{_LIB}::k2b_decode", mutates_args=(), device_types="cuda")
def k2b_decode(q: torch.Tensor, pages: torch.Tensor, page_table: Optional[torch.Tensor],
               packed_len: torch.Tensor, max_packed_len: int, basis16: torch.Tensor,
               inv_freq: list[float], rope_scaling: float, codebook: list[float], sign_bits: list[int],
               sm_scale: float, rank: int, k_tail: Optional[torch.Tensor] = None,
               v_tail: Optional[torch.Tensor] = None, tail_len: Optional[torch.Tensor] = None,
               tail_len_value: int = 0, tail_cap: int = 0, split_tokens: int = 0, group: int = 64,
               k_bits: int = 3) -> torch.Tensor:
    """One fused decode step over packed k2b pages plus the recent window; the
    arguments are those of ``bmx_amd.k2b.decode`` (tail_len a device int32 (B,)
    tensor, or None and the host count tail_len_value; head_dim from q)."""
    return k2b.decode(q, pages, page_table, packed_len, max_packed_len, basis16,
                      _consts(inv_freq, rope_scaling, codebook, sign_bits), sm_scale, rank=rank,
                      k_tail=k_tail, v_tail=v_tail, tail_len=_tail_len(tail_len, tail_len_value),
                      tail_cap=tail_cap, split_tokens=split_tokens, group=group, k_bits=k_bits)


@k2b_decode.register_fake
def _(q, pages, page_table, packed_len, max_packed_len, basis16, inv_freq, rope_scaling, codebook,
      sign_bits, sm_scale, rank, k_tail=None, v_tail=None, tail_len=None, tail_len_value=0, tail_cap=0,
      split_tokens=0, group=64, k_bits=3):
    torch._check(q.dim() == 4 and q.shape[-1] in k2b.HEAD_DIMS)
    return torch.empty_like(q)


@torch.library.custom_op(f"{_LIB}::k2b_append", mutates_args=("pages",), device_types="cuda")
def k2b_append(k_pre: torch.Tensor, v: torch.Tensor, basis32: torch.Tensor, basis16: torch.Tensor,
               pages: torch.Tensor, page_ids: torch.Tensor, codebook: list[float], sign_bits: list[int],
               rank: int, us_first: Optional[torch.Tensor] = None, group: int = 64, k_bits: int = 3) -> None:
    """Encode 128-token codec pages into the pool (``bmx_amd.k2b.append``);
    writes ``pages`` in place."""
    consts = k2b.CodecConsts(tuple(float(x) for x in codebook), tuple(int(x) for x in sign_bits),
                             (0.0,) * (k_pre.shape[-1] // 2))
    k2b.append(k_pre, v, basis32, basis16, pages, page_ids, consts, rank=rank, us_first=us_first, group=group,
               k_bits=k_bits)


@k2b_append.register_fake
def _(k_pre, v, basis32, basis16, pages, page_ids, codebook, sign_bits, rank, us_first=None, group=64, k_bits=3):
    return None


@torch.library.custom_op(f"{_LIB}::rtn_decode", mutates_args=(), device_types="cuda")
def rtn_decode(q: torch.Tensor, pages: torch.Tensor, page_table: torch.Tensor, packed_len: torch.Tensor,
               max_packed_len: int, sm_scale: float, k_bits: int, v_bits: int, k_group: int, v_group: int,
               k_arm: int = rtn.TOKEN, k_tail: Optional[torch.Tensor] = None,
               v_tail: Optional[torch.Tensor] = None, tail_len: Optional[torch.Tensor] = None,
               tail_len_value: int = 0, tail_cap: int = 0, split_tokens: int = 0) -> torch.Tensor:
    """One decode step over RTN pages (``bmx_amd.rtn.decode``)."""
    return rtn.decode(q, pages, page_table, packed_len, max_packed_len, sm_scale, k_bits=k_bits,
                      v_bits=v_bits, k_group=k_group, v_group=v_group, k_arm=k_arm, k_tail=k_tail,
                      v_tail=v_tail, tail_len=_tail_len(tail_len, tail_len_value), tail_cap=tail_cap,
                      split_tokens=split_tokens)


@rtn_decode.register_fake
def _(q, pages, page_table, packed_len, max_packed_len, sm_scale, k_bits, v_bits, k_group, v_group,
      k_arm=rtn.TOKEN, k_tail=None, v_tail=None, tail_len=None, tail_len_value=0, tail_cap=0, split_tokens=0):
    torch._check(q.dim() == 4 and q.shape[-1] == rtn.HEAD_DIM)
    return torch.empty_like(q)


@torch.library.custom_op(f"{_LIB}::rtn_append", mutates_args=("pages",), device_types="cuda")
def rtn_append(k: torch.Tensor, v: torch.Tensor, pages: torch.Tensor, page_ids: torch.Tensor,
               k_bits: int, v_bits: int, k_group: int, v_group: int, k_arm: int = rtn.TOKEN) -> None:
    """Quantize 128-token codec pages into the RTN pool (``bmx_amd.rtn.append``)."""
    rtn.append(k, v, pages, page_ids, k_bits=k_bits, v_bits=v_bits, k_group=k_group, v_group=v_group,
               k_arm=k_arm)


@rtn_append.register_fake
def _(k, v, pages, page_ids, k_bits, v_bits, k_group, v_group, k_arm=rtn.TOKEN):
    return None


@torch.library.custom_op(f"{_LIB}::prefill_attention", mutates_args=(), device_types="cuda")
def prefill_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, sm_scale: float, causal: bool,
                      n_split: int = 0) -> torch.Tensor:
    """Attention of (h_kv * G, n_q, 128) queries over (h_kv, n_kv, 128) K/V
    rows, grouped heads, bottom-right causal or no mask
    (``bmx_amd.prefill.attention``)."""
    return prefill.attention(q, k, v, sm_scale, causal=causal, n_split=n_split)


@prefill_attention.register_fake
def _(q, k, v, sm_scale, causal, n_split=0):
    torch._check(q.dim() == 3 and q.shape[-1] == prefill.HEAD_DIM and k.dim() == 3)
    return torch.empty(q.shape, dtype=q.dtype, device=q.device)


def consts_args(consts: k2b.CodecConsts) -> dict:
    """The constants of a CodecConsts as the operators' keyword arguments."""
    return dict(inv_freq=list(consts.inv_freq), rope_scaling=consts.rope_scaling,
                codebook=list(consts.codebook), sign_bits=list(consts.sign_bits))

"""Host wrappers of the MI355X RTN path (include/bmx_rtn.h): rtn_token keys
(post-RoPE) and values, 2..4-bit codes times a per-(token, channel group) fp16
scale, in 16-token pages of a device pool; keys may instead be rtn_channel
(k_arm=CHANNEL: a scale per (channel, group of k_group tokens)).

Mirrors the reference's fused RTN path (cache/triton_dequant_attention.py:
580-832 and 1390-1451, called from PackedStreamingLayer.attend,
cache/packed_streaming.py:904-950) with the device stacks replaced by a page
pool and a page table, as for k2b.  Every call goes to libbmx_k2b.so; there is
no CPU path.
"""

from __future__ import annotations

import ctypes as ct

import torch

from . import _lib
from .k2b import (DecodeWorkspace, _dense_out, _IO_DTYPES, _need, _ptr, _stream, _TAIL_DTYPES, _V_DTYPES,
                  set_window_rows)

HEAD_DIM = 128
PAGE_TOKENS = 16
CODEC_PAGE = 128
TOKEN, CHANNEL = 0, 1   # key arms: rtn_token, rtn_channel (BMX_RTN_TOKEN / BMX_RTN_CHANNEL)


def geom(h_kv: int, G: int = 1, *, k_bits: int, v_bits: int, k_group: int, v_group: int, k_arm: int = TOKEN):
    return _lib.RtnGeom(h_kv, G, k_bits, v_bits, k_group, v_group, k_arm)


def page_bytes(h_kv: int, *, k_bits: int = 4, v_bits: int = 4, k_group: int = 32, v_group: int = 32,
               k_arm: int = TOKEN) -> int:
    g = geom(h_kv, k_bits=k_bits, v_bits=v_bits, k_group=k_group, v_group=v_group, k_arm=k_arm)
    n = _lib.lib().bmx_rtn_page_bytes(ct.byref(g))
    if n == 0:
        raise NotImplementedError(
            f"RTN pages take 2..4-bit codes, groups of 32, 64 or 128 and 1..16 KV heads "
            f"(got h_kv {h_kv}, bits {k_bits}/{v_bits}, groups {k_group}/{v_group}, key arm {k_arm})")
    return int(n)


class PagePool:
    """Fixed-capacity device pool of RTN pages with a host free list."""

    def __init__(self, n_pages: int, h_kv: int, device, *, gen: torch.Generator | None = None, **codec):
        self.h_kv, self.codec = h_kv, codec
        self.page_bytes = page_bytes(h_kv, **codec)
        self.pages = torch.zeros(n_pages, self.page_bytes, dtype=torch.uint8, device=device)
        order = torch.randperm(n_pages, generator=gen) if gen is not None else torch.arange(n_pages)
        self.free = order.tolist()[::-1]

    def alloc(self, n: int) -> list:
        if n > len(self.free):
            raise RuntimeError(f"page pool exhausted: need {n}, have {len(self.free)}")
        return [self.free.pop() for _ in range(n)]


def append(k: torch.Tensor, v: torch.Tensor, pages: torch.Tensor, page_ids: torch.Tensor, *,
           k_bits: int, v_bits: int, k_group: int, v_group: int, k_arm: int = TOKEN) -> None:
    """Quantize n codec pages (k: (h_kv, 128n, 128) post-RoPE keys, v: same
    shape; fp16, bf16 or fp32, last dim contiguous) into the 8n pages listed in
    page_ids (int32, device)."""
    h_kv, T, d = k.shape
    _need(d == HEAD_DIM and T % CODEC_PAGE == 0, "k must be (h_kv, 128*n, 128)")
    _need(v.shape == k.shape, "v must match k")
    _need(k.dtype in _V_DTYPES and v.dtype in _V_DTYPES, "k and v must be fp16, bf16 or fp32")
    _need(k.stride(2) == 1 and v.stride(2) == 1, "k/v last dim must be contiguous")
    n = T // CODEC_PAGE
    _need(page_ids.dtype == torch.int32 and page_ids.numel() == 8 * n, "page_ids must be int32[8n]")
    pb = page_bytes(h_kv, k_bits=k_bits, v_bits=v_bits, k_group=k_group, v_group=v_group, k_arm=k_arm)
    _need(pages.dtype == torch.uint8 and pages.dim() == 2 and pages.shape[1] == pb and pages.is_contiguous(),
          "pages must be a contiguous uint8 (n_pages, page_bytes) pool")
    a = _lib.RtnAppendArgs()
    a.geom = geom(h_kv, k_bits=k_bits, v_bits=v_bits, k_group=k_group, v_group=v_group, k_arm=k_arm)
    a.n_codec_pages = n
    a.k, a.k_stride_h, a.k_stride_t, a.k_dtype = _ptr(k), k.stride(0), k.stride(1), _V_DTYPES[k.dtype]
    a.v, a.v_stride_h, a.v_stride_t, a.v_dtype = _ptr(v), v.stride(0), v.stride(1), _V_DTYPES[v.dtype]
    a.pages, a.page_ids, a.n_pool_pages = _ptr(pages), _ptr(page_ids), pages.shape[0]
    _lib.check(_lib.lib().bmx_rtn_append(ct.byref(a), _stream(pages.device)), "bmx_rtn_append")


def decode(q: torch.Tensor, pages: torch.Tensor, page_table: torch.Tensor, packed_len: torch.Tensor,
           max_packed_len: int, sm_scale: float, *, k_bits: int, v_bits: int, k_group: int, v_group: int,
           k_arm: int = TOKEN, k_tail: torch.Tensor | None = None, v_tail: torch.Tensor | None = None,
           tail_len: torch.Tensor | None = None, tail_cap: int = 0, out: torch.Tensor | None = None,
           split_tokens: int = 0, workspace: DecodeWorkspace | None = None, new_kv=None,
           _capture=None) -> torch.Tensor:
    """One decode step.  q (B, h_kv, G, 128) post-RoPE in fp32, fp16 or bf16 ->
    (B, h_kv, G, 128) in q's dtype;
    page_table (B, max_pages) int32; packed_len (B,) int32 (multiples of 128);
    k_tail/v_tail (B, h_kv, >=tail_cap, 128) fp16 or bf16 with tail_len valid rows (a
    device int32 (B,) tensor or a host int); new_kv as in k2b.set_window_rows."""
    B, h_kv, G, d = q.shape
    dev = q.device
    _need(d == HEAD_DIM and q.dtype in _IO_DTYPES and q.is_contiguous(),
          "q must be contiguous fp32, fp16 or bf16 (B, h_kv, G, 128)")
    pb = page_bytes(h_kv, k_bits=k_bits, v_bits=v_bits, k_group=k_group, v_group=v_group, k_arm=k_arm)
    _need(pages.dtype == torch.uint8 and pages.shape[1] == pb, "pages must be (n_pages, page_bytes) uint8")
    _need(page_table.dtype == torch.int32 and page_table.dim() == 2 and page_table.shape[0] == B
          and page_table.is_contiguous(), "page_table must be contiguous int32 (B, max_pages)")
    _need(packed_len.dtype == torch.int32 and packed_len.numel() == B, "packed_len must be int32[B]")
    _need(page_table.shape[1] * PAGE_TOKENS >= max_packed_len, "page_table too narrow for max_packed_len")
    if out is None:
        out = torch.empty_like(q)
    _need(out.dtype == q.dtype and out.shape == q.shape and out.is_contiguous(),
          "out must be contiguous and of q's shape and dtype")
    a = _lib.RtnDecodeArgs()
    a.geom = geom(h_kv, G, k_bits=k_bits, v_bits=v_bits, k_group=k_group, v_group=v_group, k_arm=k_arm)
    a.batch = B
    a.q, a.out = _ptr(q), _ptr(out)
    a.io_dtype = _IO_DTYPES[q.dtype]
    a.pages, a.n_pool_pages = _ptr(pages), pages.shape[0]
    a.page_table, a.max_pages = _ptr(page_table), page_table.shape[1]
    a.packed_len, a.max_packed_len = _ptr(packed_len), int(max_packed_len)
    a.sm_scale = float(sm_scale)
    if tail_cap > 0:
        _need(k_tail is not None and v_tail is not None and k_tail.shape == v_tail.shape
              and k_tail.stride() == v_tail.stride(), "k_tail/v_tail must share shape and strides")
        _need(k_tail.dtype in _TAIL_DTYPES and v_tail.dtype == k_tail.dtype and k_tail.dim() == 4
              and k_tail.shape[0] == B and k_tail.shape[1] == h_kv and k_tail.shape[2] >= tail_cap
              and k_tail.stride(3) == 1,
              "k_tail/v_tail must be fp16 or bf16 (B, h_kv, >=tail_cap, 128) with contiguous last dim")
        a.k_tail, a.v_tail = _ptr(k_tail), _ptr(v_tail)
        a.tail_dtype = _TAIL_DTYPES[k_tail.dtype]
        a.tail_stride_b, a.tail_stride_h, a.tail_stride_t = k_tail.stride(0), k_tail.stride(1), k_tail.stride(2)
    a.tail_cap = int(tail_cap)
    set_window_rows(a, B, h_kv, tail_len, tail_cap, new_kv)
    a.split_tokens = int(split_tokens)
    lib = _lib.lib()
    need = int(lib.bmx_rtn_decode_workspace_bytes(ct.byref(a)))
    ws = workspace if workspace is not None else _DEFAULT_WS.setdefault(dev, DecodeWorkspace())
    buf = ws.get(need, dev)
    a.workspace, a.workspace_bytes = buf.data_ptr(), buf.numel()
    if _capture is not None:
        _capture(a)
        return out
    _lib.check(lib.bmx_rtn_decode(ct.byref(a), _stream(dev)), "bmx_rtn_decode")
    return out


_DEFAULT_WS: dict = {}


class DecodePlan:
    """An RTN decode call with every argument bound once: ``run()`` is one C call
    (the bound tensors must stay alive and keep their storage)."""

    def __init__(self, q, pages, page_table, packed_len, max_packed_len, sm_scale, *, k_bits, v_bits,
                 k_group, v_group, k_arm=TOKEN, k_tail=None, v_tail=None, tail_len=None, tail_cap=0, out=None,
                 split_tokens=0, workspace: DecodeWorkspace | None = None):
        self.out = torch.empty_like(q) if out is None else out
        self._keep = (q, pages, page_table, packed_len, k_tail, v_tail, tail_len)
        self.ws = workspace or DecodeWorkspace()
        captured = {}
        decode(q, pages, page_table, packed_len, max_packed_len, sm_scale, k_bits=k_bits, v_bits=v_bits,
               k_group=k_group, v_group=v_group, k_arm=k_arm, k_tail=k_tail, v_tail=v_tail, tail_len=tail_len,
               tail_cap=tail_cap, out=self.out, split_tokens=split_tokens, workspace=self.ws,
               _capture=lambda a: captured.setdefault("a", a))
        self.args = captured["a"]
        self.stream = _stream(q.device)
        self._fn = _lib.lib().bmx_rtn_decode

    def run(self, *, q: torch.Tensor | None = None, tail_len: int | None = None, new_kv=None,
            out: torch.Tensor | None = None) -> torch.Tensor:
        """One call; q, tail_len, new_kv and out as in k2b.DecodePlan.run."""
        a = self.args
        if out is not None:
            _need(out.dtype == self.out.dtype and out.shape == self.out.shape and out.is_contiguous(),
                  "out must match the bound output's shape, dtype and contiguity")
        res = self.out if out is None else out
        a.out = res.data_ptr()
        if q is not None:
            _need(q.dtype == self.out.dtype, "q must keep the bound query's dtype")
            a.q = q.data_ptr()
        if tail_len is not None or new_kv is not None:
            _need(not a.tail_len, "the plan was bound with a device tail_len")
            set_window_rows(a, self.out.shape[0], self.out.shape[1],
                            a.tail_len_value if tail_len is None else tail_len, a.tail_cap, new_kv)
        rc = self._fn(ct.byref(a), self.stream)
        if rc != 0:
            _lib.check(rc, "bmx_rtn_decode")
        return res


def dequant(pages: torch.Tensor, page_ids: torch.Tensor, *, h_kv: int, k_bits: int, v_bits: int,
            k_group: int, v_group: int, k_arm: int = TOKEN, dtype: torch.dtype = torch.float32,
            out: tuple | None = None):
    """Pages (in order) -> dense (K (h_kv, 16n, 128), V (h_kv, 16n, 128)) in dtype;
    out: (K, V) views to write into, as for k2b.dequant."""
    n = page_ids.numel()
    _need(page_ids.dtype == torch.int32 and page_ids.is_contiguous(), "page_ids must be contiguous int32")
    _need(dtype in _V_DTYPES, "dtype must be fp16, bf16 or fp32")
    k_out, v_out, rows = _dense_out(out, h_kv, n * PAGE_TOKENS, dtype, pages.device)
    a = _lib.RtnDequantArgs()
    a.geom = geom(h_kv, k_bits=k_bits, v_bits=v_bits, k_group=k_group, v_group=v_group, k_arm=k_arm)
    a.pages, a.n_pool_pages = _ptr(pages), pages.shape[0]
    a.page_ids, a.n_pages = _ptr(page_ids), n
    a.k_out, a.v_out = _ptr(k_out), _ptr(v_out)
    a.out_dtype = _V_DTYPES[dtype]
    a.out_rows = rows
    _lib.check(_lib.lib().bmx_rtn_dequant(ct.byref(a), _stream(pages.device)), "bmx_rtn_dequant")
    return k_out, v_out

"""torch-facing wrappers over the k2b C-ABI (decode, append, dequant).

Tensors are HIP device tensors; the calls enqueue on torch's current stream of
the tensors' device and never allocate inside the library (workspaces come from
here).  Any non-zero status raises RuntimeError with the library's message: the
k2b decode path has no non-HIP fallback.
"""

from __future__ import annotations

import ctypes as ct
from dataclasses import dataclass

import torch

from . import _lib
from . import codecs as K

HEAD_DIM = 128
HEAD_DIMS = (32, 64, 128)   # 128: the recipe's page; 32 and 64 (and other ranks, groups, key bits): the general page
PAGE_TOKENS = 16
_V_DTYPES = {torch.float16: 0, torch.float32: 1, torch.bfloat16: 2}   # BMX_K2B_F16 / F32 / BF16
_IO_DTYPES = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}  # BMX_K2B_IO_F32 / F16 / BF16
_TAIL_DTYPES = {torch.float16: 0, torch.bfloat16: 1}                   # BMX_K2B_TAIL_F16 / BF16
GROUP = 64
CODEC_PAGE = 128


@dataclass(frozen=True)
class CodecConsts:
    """Numbers the kernels take by value: V codebook, V sign bits, RoPE."""

    codebook: tuple
    sign_bits: tuple
    inv_freq: tuple
    rope_scaling: float = 1.0

    @staticmethod
    def make(*, v_bits: int = 2, v_seed: int = 0, inv_freq=None, rope_scaling: float = 1.0,
             theta: float = 500000.0, head_dim: int = HEAD_DIM):
        if v_bits != 2:
            raise ValueError("the k2b kernels implement 2-bit V codes only")
        if head_dim not in HEAD_DIMS:
            raise ValueError(f"head_dim must be one of {HEAD_DIMS}")
        if inv_freq is None:
            inv_freq, rope_scaling = K.rope_inv_freq(head_dim=head_dim, theta=theta)
        inv = tuple(float(x) for x in torch.as_tensor(inv_freq, dtype=torch.float32).tolist())
        if len(inv) != head_dim // 2:
            raise ValueError(f"inv_freq must have {head_dim // 2} entries")
        return CodecConsts(K.gaussian_codebook(v_bits),
                           tuple(K.sign_bits(K.hadamard_signs(head_dim, v_seed))),
                           inv, float(rope_scaling))

    @property
    def head_dim(self) -> int:
        return 2 * len(self.inv_freq)

    def inv_freq64(self) -> tuple:
        """inv_freq padded to the 64 entries of the argument structs."""
        return tuple(self.inv_freq) + (0.0,) * (64 - len(self.inv_freq))


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _stream(dev: torch.device) -> ct.c_void_p:
    return ct.c_void_p(torch.cuda.current_stream(dev).cuda_stream)


def _need(cond: bool, msg: str):
    if not cond:
        raise ValueError(msg)


def set_window_rows(a, B: int, h_kv: int, tail_len, tail_cap: int, new_kv=None) -> None:
    """Fill the window-length and new-row fields of decode args a (k2b or RTN).

    tail_len: a device int32 (B,) tensor, or a host int (every sequence's window
    length, no device read), or None (0).  new_kv: (k, v) (B, h_kv, n, 128)
    post-RoPE keys and values of the window's newest n rows (rows tail_len - n
    .. tail_len - 1) in the window's dtype (a.tail_dtype), attended from there
    and copied into the window buffers by the decode call; needs a host
    tail_len."""
    if isinstance(tail_len, torch.Tensor):
        _need(tail_len.dtype == torch.int32 and tail_len.numel() == B and tail_len.is_cuda,
              "tail_len must be a device int32[B] tensor or a host int")
        a.tail_len, a.tail_len_value = tail_len.data_ptr(), 0
    else:
        T = 0 if tail_len is None else int(tail_len)
        _need(0 <= T <= tail_cap, "tail_len must be within 0..tail_cap")
        a.tail_len, a.tail_len_value = None, T
    if new_kv is None:
        a.new_k = a.new_v = None
        a.n_new = 0
        return
    k, v = new_kv
    _need(not isinstance(tail_len, torch.Tensor), "rows given apart need a host tail_len")
    wdt = torch.bfloat16 if a.tail_dtype == _TAIL_DTYPES[torch.bfloat16] else torch.float16
    _need(k.dim() == 4 and k.shape == v.shape and k.dtype == wdt and v.dtype == wdt
          and k.shape[0] == B and k.shape[1] == h_kv and k.shape[3] in HEAD_DIMS,
          f"new_kv: (B, h_kv, n, head_dim) keys and values in the window's dtype ({wdt})")
    # strides of size-1 dimensions are never used: taken as 0
    sk = tuple(0 if n == 1 else st for n, st in zip(k.shape[:3], k.stride()[:3]))
    sv = tuple(0 if n == 1 else st for n, st in zip(v.shape[:3], v.stride()[:3]))
    _need(sk == sv and k.stride(3) == 1 and v.stride(3) == 1,
          "new_kv: keys and values with the same strides, channels contiguous")
    _need(all(st % 8 == 0 for st in sk), "new_kv strides must be multiples of 8 elements")
    a.new_k, a.new_v = k.data_ptr(), v.data_ptr()
    a.new_stride_b, a.new_stride_h, a.new_stride_t = sk
    a.n_new = k.shape[2]
    _need(a.n_new <= a.tail_len_value, "new_kv holds more rows than the window")


def page_bytes(h_kv: int, rank: int, *, head_dim: int = HEAD_DIM, group: int = GROUP, k_bits: int = 3) -> int:
    return _lib.page_bytes(h_kv, rank, head_dim=head_dim, group=group, k_bits=k_bits)


def geom(h_kv: int, rank: int, n_q_groups: int = 1, *, head_dim: int = HEAD_DIM, group: int = GROUP,
         k_bits: int = 3) -> "_lib.Geom":
    return _lib.Geom(h_kv, rank, n_q_groups, head_dim, group, k_bits)


def append(k_pre: torch.Tensor, v: torch.Tensor, basis32: torch.Tensor, basis16: torch.Tensor,
           pages: torch.Tensor, page_ids: torch.Tensor, consts: CodecConsts, *, rank: int,
           us_first: torch.Tensor | None = None, group: int = GROUP, k_bits: int = 3) -> None:
    """Encode n codec pages (k_pre: (h_kv, 128n, head_dim) fp16, v: same shape in
    fp16, bf16 or fp32 -- values are encoded from their own precision; last dims
    contiguous) into the 8n physical pages listed in page_ids (int32, device).
    group / k_bits: the residual's scale group and bits (64 / 3: the recipe)."""
    h_kv, T, d = k_pre.shape
    _need(d in HEAD_DIMS and T % CODEC_PAGE == 0, "k_pre must be (h_kv, 128*n, head_dim)")
    _need(consts.head_dim == d, "consts were made for another head_dim")
    _need(v.shape == k_pre.shape, "v must match k_pre")
    _need(k_pre.dtype == torch.float16, "k_pre must be fp16")
    _need(v.dtype in _V_DTYPES, "v must be fp16, bf16 or fp32")
    _need(k_pre.stride(2) == 1 and v.stride(2) == 1, "k_pre/v last dim must be contiguous")
    n = T // CODEC_PAGE
    C = h_kv * d
    _need(basis32.shape == (C, rank) and basis32.dtype == torch.float32 and basis32.is_contiguous(),
          "basis32 must be contiguous fp32 (C, rank)")
    _need(basis16.shape == (C, rank) and basis16.dtype == torch.float16 and basis16.is_contiguous(),
          "basis16 must be contiguous fp16 (C, rank)")
    _need(page_ids.dtype == torch.int32 and page_ids.numel() == 8 * n, "page_ids must be int32[8n]")
    pb = page_bytes(h_kv, rank, head_dim=d, group=group, k_bits=k_bits)
    _need(pages.dtype == torch.uint8 and pages.dim() == 2 and pages.shape[1] == pb
          and pages.is_contiguous(), "pages must be a contiguous uint8 (n_pages, page_bytes) pool")
    if us_first is not None:
        _need(us_first.shape == (CODEC_PAGE, rank) and us_first.dtype == torch.float32
              and us_first.is_contiguous(), "us_first must be contiguous fp32 (128, rank)")
    a = _lib.AppendArgs()
    a.geom = geom(h_kv, rank, 1, head_dim=d, group=group, k_bits=k_bits)
    a.n_codec_pages = n
    a.k_pre, a.k_stride_h, a.k_stride_t = _ptr(k_pre), k_pre.stride(0), k_pre.stride(1)
    a.v, a.v_stride_h, a.v_stride_t = _ptr(v), v.stride(0), v.stride(1)
    a.basis32, a.basis16, a.us_first = _ptr(basis32), _ptr(basis16), _ptr(us_first)
    a.codebook[:] = consts.codebook
    a.v_sign_bits[:] = consts.sign_bits
    a.pages, a.page_ids, a.n_pool_pages = _ptr(pages), _ptr(page_ids), pages.shape[0]
    a.v_dtype = _V_DTYPES[v.dtype]
    _lib.check(_lib.lib().bmx_k2b_append(ct.byref(a), _stream(pages.device)), "bmx_k2b_append")


class DecodeWorkspace:
    """Grow-only device scratch for split partials (reused across calls).

    Every call writes all the partials it reads; the buffer is zero-filled when
    (re)allocated only so that its contents are defined."""

    def __init__(self):
        self.buf = None

    def get(self, nbytes: int, device) -> torch.Tensor:
        if self.buf is None or self.buf.numel() < nbytes or self.buf.device != device:
            self.buf = torch.zeros(max(nbytes, 1), dtype=torch.uint8, device=device)
        return self.buf


_DEFAULT_WS: dict = {}


def decode(q: torch.Tensor, pages: torch.Tensor, page_table: torch.Tensor | None,
           packed_len: torch.Tensor, max_packed_len: int, basis16: torch.Tensor,
           consts: CodecConsts, sm_scale: float, *, rank: int,
           k_tail: torch.Tensor | None = None, v_tail: torch.Tensor | None = None,
           tail_len: torch.Tensor | None = None, tail_cap: int = 0,
           out: torch.Tensor | None = None, split_tokens: int = 0,
           workspace: DecodeWorkspace | None = None, page_stride: int | None = None,
           new_kv=None, split_end_event: torch.cuda.Event | None = None, group: int = GROUP,
           k_bits: int = 3, _capture=None) -> torch.Tensor:
    """One decode step.  q (B, h_kv, G, head_dim) post-RoPE in fp32, fp16 or bf16
    (the model's dtype) -> (B, h_kv, G, head_dim) in q's dtype; group / k_bits
    as in append.

    page_table (B, max_pages) int32, or None for contiguous pages: logical page
    i of sequence b at pool page b * page_stride + i (page_stride defaults to
    max_packed_len / 16); packed_len (B,) int32 committed tokens (multiples of
    128, <= max_packed_len); basis16 (B, C, rank) or (C, rank) fp16;
    k_tail/v_tail (B, h_kv, >=tail_cap, 128) fp16 or bf16 post-RoPE recent window with
    tail_len valid rows (a device int32 (B,) tensor or a host int); new_kv as in
    set_window_rows."""
    B, h_kv, G, d = q.shape
    dev = q.device
    _need(d in HEAD_DIMS and q.dtype in _IO_DTYPES and q.is_contiguous(),
          "q must be contiguous fp32, fp16 or bf16 (B, h_kv, G, head_dim)")
    _need(consts.head_dim == d, "consts were made for another head_dim")
    _need(pages.dtype == torch.uint8
          and pages.shape[1] == page_bytes(h_kv, rank, head_dim=d, group=group, k_bits=k_bits),
          "pages must be (n_pages, page_bytes) uint8")
    if page_table is None:
        stride = page_stride if page_stride is not None else max(1, -(-max_packed_len // PAGE_TOKENS))
        _need(stride * PAGE_TOKENS >= max_packed_len and (B == 1 or page_stride is not None),
              "contiguous pages: page_stride * 16 must cover max_packed_len (and is required for B > 1)")
        _need(max_packed_len == 0 or (B - 1) * stride + -(-max_packed_len // PAGE_TOKENS) <= pages.shape[0],
              "contiguous pages: the pool holds fewer pages than the batch's sequences need")
    else:
        _need(page_table.dtype == torch.int32 and page_table.dim() == 2 and page_table.shape[0] == B
              and page_table.is_contiguous(), "page_table must be contiguous int32 (B, max_pages)")
        stride = page_table.shape[1]
    _need(packed_len.dtype == torch.int32 and packed_len.numel() == B, "packed_len must be int32[B]")
    C = h_kv * d
    if basis16.dim() == 2:
        _need(basis16.shape == (C, rank), "basis16 must be (C, rank)")
        bstride = 0
    else:
        _need(basis16.shape == (B, C, rank), "basis16 must be (B, C, rank)")
        bstride = basis16.stride(0)
    _need(basis16.dtype == torch.float16 and basis16.stride(-1) == 1 and basis16.stride(-2) == rank,
          "basis16 rows must be contiguous fp16")
    if out is None:
        out = torch.empty_like(q)
    _need(out.dtype == q.dtype and out.shape == q.shape and out.is_contiguous(),
          "out must be contiguous and of q's shape and dtype")
    a = _lib.DecodeArgs()
    a.geom = geom(h_kv, rank, G, head_dim=d, group=group, k_bits=k_bits)
    a.batch = B
    a.q, a.out = _ptr(q), _ptr(out)
    a.io_dtype = _IO_DTYPES[q.dtype]
    a.pages, a.page_table, a.max_pages = _ptr(pages), _ptr(page_table), stride
    a.n_pool_pages = pages.shape[0]
    _need(stride * PAGE_TOKENS >= max_packed_len, "page_table too narrow for max_packed_len")
    a.packed_len, a.max_packed_len = _ptr(packed_len), int(max_packed_len)
    a.basis, a.basis_stride = _ptr(basis16), bstride
    a.inv_freq[:] = consts.inv_freq64()
    a.rope_scaling = consts.rope_scaling
    a.sm_scale = float(sm_scale)
    a.codebook[:] = consts.codebook
    a.v_sign_bits[:] = consts.sign_bits
    if tail_cap > 0:
        _need(k_tail is not None and v_tail is not None and k_tail.shape == v_tail.shape
              and k_tail.stride() == v_tail.stride(), "k_tail/v_tail must share shape and strides")
        _need(k_tail.dtype in _TAIL_DTYPES and v_tail.dtype == k_tail.dtype and k_tail.dim() == 4
              and k_tail.shape[0] == B and k_tail.shape[1] == h_kv and k_tail.shape[2] >= tail_cap
              and k_tail.stride(3) == 1,
              "k_tail/v_tail must be fp16 or bf16 (B, h_kv, >=tail_cap, head_dim) with contiguous last dim")
        a.k_tail, a.v_tail = _ptr(k_tail), _ptr(v_tail)
        a.tail_dtype = _TAIL_DTYPES[k_tail.dtype]
        a.tail_stride_b, a.tail_stride_h, a.tail_stride_t = k_tail.stride(0), k_tail.stride(1), k_tail.stride(2)
    a.tail_cap = int(tail_cap)
    set_window_rows(a, B, h_kv, tail_len, tail_cap, new_kv)
    a.split_tokens = int(split_tokens)
    lib = _lib.lib()
    need = int(lib.bmx_k2b_decode_workspace_bytes(ct.byref(a)))
    ws = workspace if workspace is not None else _DEFAULT_WS.setdefault(dev, DecodeWorkspace())
    buf = ws.get(need, dev)
    a.workspace, a.workspace_bytes = buf.data_ptr(), buf.numel()
    if split_end_event is not None:
        a.split_end_event = split_end_event.cuda_event
    if _capture is not None:
        _capture(a)
        return out
    _lib.check(lib.bmx_k2b_decode(ct.byref(a), _stream(dev)), "bmx_k2b_decode")
    return out


class DecodePlan:
    """A decode call with every argument bound once: ``run()`` is one C call.

    Serving loops re-issue the same decode for a layer every step with only the
    tensors' contents changing (q, the page table, lengths, the tail); binding
    the pointers once removes the per-step host work (argument checks, struct
    fill, workspace sizing).  The bound tensors must stay alive and must not be
    reallocated while the plan is used."""

    def __init__(self, q, pages, page_table, packed_len, max_packed_len, basis16, consts,
                 sm_scale, *, rank, k_tail=None, v_tail=None, tail_len=None, tail_cap=0,
                 out=None, split_tokens=0, workspace: DecodeWorkspace | None = None,
                 page_stride: int | None = None, group: int = GROUP, k_bits: int = 3):
        self.out = torch.empty_like(q) if out is None else out
        self._keep = (q, pages, page_table, packed_len, basis16, k_tail, v_tail, tail_len)
        self.ws = workspace or DecodeWorkspace()
        captured = {}

        def capture(a):
            captured["a"] = a
        decode(q, pages, page_table, packed_len, max_packed_len, basis16, consts, sm_scale,
               rank=rank, k_tail=k_tail, v_tail=v_tail, tail_len=tail_len, tail_cap=tail_cap,
               out=self.out, split_tokens=split_tokens, workspace=self.ws, page_stride=page_stride,
               group=group, k_bits=k_bits, _capture=capture)
        self.args = captured["a"]
        self.stream = _stream(q.device)
        self._fn = _lib.lib().bmx_k2b_decode

    def run(self, split_end_event: torch.cuda.Event | None = None, *, q: torch.Tensor | None = None,
            tail_len: int | None = None, new_kv=None, out: torch.Tensor | None = None) -> torch.Tensor:
        """One call.  q: a new query tensor of the bound one's shape, dtype and
        contiguity (its pointer replaces the bound one); out: likewise, the
        tensor this call writes (default: the plan's own output buffer);
        tail_len / new_kv: the host window length and the rows given apart for
        this call (the plan must have been bound with a host tail_len)."""
        a = self.args
        if out is not None:
            _need(out.dtype == self.out.dtype and out.shape == self.out.shape and out.is_contiguous(),
                  "out must match the bound output's shape, dtype and contiguity")
        res = self.out if out is None else out
        a.out = res.data_ptr()
        a.split_end_event = None if split_end_event is None else split_end_event.cuda_event
        if q is not None:
            _need(q.dtype == self.out.dtype, "q must keep the bound query's dtype")
            a.q = q.data_ptr()
        if tail_len is not None or new_kv is not None:
            _need(not a.tail_len, "the plan was bound with a device tail_len")
            set_window_rows(a, q.shape[0] if q is not None else self.out.shape[0], self.out.shape[1],
                            a.tail_len_value if tail_len is None else tail_len, a.tail_cap, new_kv)
        rc = self._fn(ct.byref(a), self.stream)
        if rc != 0:
            _lib.check(rc, "bmx_k2b_decode")
        return res


ROPE_NONE, ROPE_EXACT, ROPE_FP16_TABLES = 0, 1, 2


def _dense_out(out, h_kv: int, n_rows: int, dtype, dev, d: int = HEAD_DIM):
    """(K, V) destinations of a dequant: new (h_kv, n_rows, d) tensors, or the
    caller's (h_kv, >= n_rows, d) views with contiguous rows; -> (K, V, rows
    between heads)."""
    if out is None:
        k = torch.empty(h_kv, n_rows, d, dtype=dtype, device=dev)
        return k, torch.empty_like(k), n_rows
    k, v = out
    _need(k.dtype == dtype and v.dtype == dtype and k.shape == v.shape and k.stride() == v.stride()
          and k.dim() == 3 and k.shape[0] == h_kv and k.shape[1] >= n_rows and k.shape[2] == d
          and k.stride(2) == 1 and k.stride(1) == d and k.stride(0) % d == 0
          and k.device == dev, f"out must be (K, V) of shape (h_kv, >= n, {d}) in dtype with contiguous rows")
    return k, v, k.stride(0) // d


def dequant_args(pages: torch.Tensor, page_table: torch.Tensor, n_tokens: int, basis16: torch.Tensor,
                 consts: CodecConsts, *, h_kv: int, rank: int, apply_rope: int = ROPE_NONE,
                 dtype: torch.dtype = torch.float32, pos0: int = 0, out: tuple | None = None,
                 group: int = GROUP, k_bits: int = 3):
    """Arguments of one bmx_k2b_dequant call and its outputs: committed pages
    of one sequence -> dense (K (h_kv, n, d), V (h_kv, n, d))
    in dtype (d = consts.head_dim; group / k_bits as in append).  apply_rope: ROPE_NONE (pre-RoPE keys), ROPE_EXACT (fp32 cos/sin)
    or ROPE_FP16_TABLES (the reference's prefill: fp16-rounded cos/sin); pos0:
    the position of the first listed token; out: (K, V) views to write into (see
    _dense_out)."""
    dev = pages.device
    _need(dtype in _V_DTYPES, "dtype must be fp16, bf16 or fp32")
    _need(int(apply_rope) in (ROPE_NONE, ROPE_EXACT, ROPE_FP16_TABLES), "apply_rope must be 0, 1 or 2")
    _need(pos0 >= 0, "pos0 must be >= 0")
    d = consts.head_dim
    k, v, rows = _dense_out(out, h_kv, n_tokens, dtype, dev, d)
    _need(page_table.dtype == torch.int32 and page_table.numel() >= n_tokens // PAGE_TOKENS,
          "page_table must hold n_tokens/16 int32 page ids")
    a = _lib.DequantArgs()
    a.geom = geom(h_kv, rank, 1, head_dim=d, group=group, k_bits=k_bits)
    a.pages, a.page_table, a.n_tokens = _ptr(pages), _ptr(page_table), int(n_tokens)
    a.n_pool_pages = pages.shape[0]
    a.basis = _ptr(basis16)
    a.inv_freq[:] = consts.inv_freq64()
    a.rope_scaling = consts.rope_scaling
    a.apply_rope = int(apply_rope)
    a.codebook[:] = consts.codebook
    a.v_sign_bits[:] = consts.sign_bits
    a.k_out, a.v_out = _ptr(k), _ptr(v)
    a.out_dtype = _V_DTYPES[dtype]
    a.pos0, a.out_rows = int(pos0), rows
    return a, k, v


def dequant_launch(a: "_lib.DequantArgs", dev: torch.device) -> None:
    """One bmx_k2b_dequant call on built arguments (dequant_args) on dev's current stream."""
    _lib.check(_lib.lib().bmx_k2b_dequant(ct.byref(a), _stream(dev)), "bmx_k2b_dequant")


def dequant(pages: torch.Tensor, page_table: torch.Tensor, n_tokens: int, basis16: torch.Tensor,
            consts: CodecConsts, *, h_kv: int, rank: int, apply_rope: int = ROPE_NONE,
            dtype: torch.dtype = torch.float32, pos0: int = 0, out: tuple | None = None,
            group: int = GROUP, k_bits: int = 3):
    """Committed pages of one sequence -> dense (K (h_kv, n, d), V (h_kv, n, d))
    in dtype: dequant_args, then one dequant_launch."""
    a, k, v = dequant_args(pages, page_table, n_tokens, basis16, consts, h_kv=h_kv, rank=rank,
                           apply_rope=apply_rope, dtype=dtype, pos0=pos0, out=out, group=group, k_bits=k_bits)
    dequant_launch(a, pages.device)
    return k, v

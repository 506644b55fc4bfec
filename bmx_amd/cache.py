"""PackedStreamingCache over the MI355X packed kernels, under HF ``generate()``.

The reference's Python API for its fused packed paths
(cache/packed_streaming.py:270-1222), kept name for name so that
``past_key_values=PackedStreamingCache(model.config, *spec_pair("k2b_ph"))``
drops in:

* ``PackedStreamingCache(model_config, k_spec, v_spec, recent_window=32,
  pack_v=True, pack_k=True)``, ``attach(model)`` / ``detach()`` / context
  manager, ``bits_per_entry()``, ``memory_report(seq_len)``
  (packed_streaming.py:1067-1222);
* ``PackedStreamingLayer`` (a transformers ``DynamicLayer``):
  ``stash_pre_rope`` (:448-457), ``update`` (:582-730) with the same flush
  schedule -- commit on the 128-token codec-page grid leaving at least
  ``recent_window`` fp16 tokens -- the same pruning of the pre-RoPE stash and
  the fp16 slab, the same blended bits-per-entry, and ``attend`` (:832-1064);
* the registered attention function (:270-307): HF's dense key/value are
  ignored; attention reads the packed pages.

What runs where:

* commit (``update``): the first codec page's truncated SVD freezes the key
  basis on the host CPU, in fp32, as the reference computes it
  (``_pack_k_block`` :507-517, decomp/lrs.py:35-41); every codec page is then
  encoded by ``bmx_k2b_append`` straight into this layer's device page pool
  (8 physical 16-token pages per codec page, logical order = table order);
* decode (one query step): ``bmx_k2b_decode`` over the pool and the fp16
  recent window, through a plan bound once per layer and rebound only at a
  commit.  The window lives in a fixed per-layer buffer of recent_window + 128
  rows; a step's new key and value are not copied into it by the host: the
  decode call is given them apart (with the window length from the host) and
  stores them itself, so a step costs the decode call alone (no slab
  concatenation, no host-to-device copy, no length upload);
* prefill (several query steps): ``bmx_k2b_dequant`` to dense pre-RoPE keys and
  values, RoPE with the fp16 tables the reference casts to
  (``_shared_rope`` :79-113, ``_dense_kv`` chunked_attention.py:148-189), the
  fp16 tail appended, then SDPA with HF's mask
  (``_prefill_dense_attention`` chunked_attention.py:320-395).

The RTN pairs (``rtn_token`` or ``rtn_channel`` keys, post-RoPE, with
``rtn_token`` values; the first is the reference's other fused path,
packed_streaming.py:904-950) take the same host logic with
the RTN kernels: each committed codec page's post-RoPE keys and values, taken
from the slab, are encoded by ``bmx_rtn_append`` (no key stash, no basis);
decode is ``bmx_rtn_decode``; prefill is ``bmx_rtn_dequant`` plus SDPA.

There is no CPU path: attention on a tensor that is not on a HIP device raises.
Values are encoded from the model's own precision (fp16, bf16 or fp32), as the
reference encodes ``values.float()``; recent-window keys/values enter the
decode kernel as fp16 (exact for fp16 and bf16 models).  Batch size 1, as in
the reference.
"""

from __future__ import annotations

import math
import weakref

import torch
import torch.nn.functional as F
from torch.nn.attention.bias import causal_lower_right
from transformers.cache_utils import Cache, DynamicLayer
from transformers.masking_utils import ALL_MASK_ATTENTION_FUNCTIONS, sdpa_mask
from transformers.modeling_utils import ALL_ATTENTION_FUNCTIONS

from . import codecs as K
from . import k2b, prefill, rtn, spectral
from .specs import CacheCodecSpec, packed_path

ATTN_NAME = "chunked_dequant"   # the reference's name (packed_streaming.py:54), set on attach
ATTN_ALIASES = ("bmx_k2b",)      # the name earlier versions of this package registered
PAGE = 128          # codec page (packed_streaming.py:438)
PAGES_PER_CODEC = PAGE // k2b.PAGE_TOKENS


# ------------------------------------------------------------------ HF helpers
# (cache/hf_compat.py:6-120, cache/collect.py:65-71)


def resolve_text_config(model_config):
    tc = getattr(model_config, "text_config", None)
    if tc is not None and hasattr(tc, "num_attention_heads"):
        return tc
    return model_config


def resolve_decoder_layers(model):
    inner = getattr(model, "model", None)
    if inner is not None:
        lm = getattr(inner, "language_model", None)
        if lm is not None and hasattr(lm, "layers"):
            return lm.layers
        if hasattr(inner, "layers"):
            return inner.layers
    tr = getattr(model, "transformer", None)
    if tr is not None and hasattr(tr, "h"):
        return tr.h
    raise ValueError(f"cannot locate the decoder layers of {type(model).__name__}")


def resolve_k_capture_module(self_attn):
    """The module whose forward output is the pre-RoPE key: ``k_norm`` when the
    attention normalises keys per head before RoPE (Qwen3), else ``k_proj``."""
    if hasattr(self_attn, "q_norm") != hasattr(self_attn, "k_norm"):
        raise ValueError("attention has only one of q_norm / k_norm: capture point ambiguous")
    for alt in ("q_layernorm", "k_layernorm", "qk_norm"):
        if hasattr(self_attn, alt):
            raise ValueError(f"attention has an unsupported pre-RoPE norm {alt!r}")
    return self_attn.k_norm if hasattr(self_attn, "k_norm") else self_attn.k_proj


def reshape_heads(out: torch.Tensor, n_head: int, d: int) -> torch.Tensor:
    """(1, S, n_head*d) or (1, S, n_head, d) -> (n_head, S, d) fp16 contiguous."""
    S = out.shape[1]
    return out.reshape(1, S, n_head, d).permute(0, 2, 1, 3).squeeze(0).contiguous().to(torch.float16)


def _rope_tables(inv_freq: torch.Tensor, scaling: float, start: int, n: int, device) -> tuple:
    """fp16 (cos, sin) (n, 128) of positions [start, start + n): HF's fp32 angle
    fl(inv_freq * pos), cos/sin in fp32 times the attention scaling, cast to
    fp16 as the reference's shared tables are."""
    pos = torch.arange(start, start + n, dtype=torch.float32, device=device)
    ang = pos[:, None] * inv_freq.to(device)[None, :]
    emb = torch.cat((ang, ang), dim=-1)
    return (emb.cos() * scaling).half(), (emb.sin() * scaling).half()


# ------------------------------------------------------------------ attention


def packed_attention_forward(module, query, key, value, attention_mask, scaling, dropout=0.0,
                             **kwargs):
    """Registered attention function (packed_streaming.py:270-300): query
    (1, n_heads, n_q, d) -> (attn_output (1, n_q, n_heads*d), None)."""
    if not hasattr(module, "_packed_layer"):
        raise RuntimeError("PackedStreamingCache.attach(model) must be called before forward")
    if query.shape[0] != 1:
        raise NotImplementedError("the packed cache serves batch size 1")
    q = query.squeeze(0)
    n_q = q.shape[1]
    out = module._packed_layer.attend(q, scaling, is_causal=n_q > 1, attention_mask=attention_mask)
    n_h, n_q, d = out.shape
    return out.transpose(0, 1).reshape(1, n_q, n_h * d).to(query.dtype), None


for _name in (ATTN_NAME, *ATTN_ALIASES):
    ALL_ATTENTION_FUNCTIONS.register(_name, packed_attention_forward)
    ALL_MASK_ATTENTION_FUNCTIONS.register(_name, sdpa_mask)


# ------------------------------------------------------------------ layer


class PackedStreamingLayer(DynamicLayer):
    """Per-layer packed cache: committed codec pages in a device page pool and
    the fp16 recent window; for k2b also the frozen key basis and the pre-RoPE
    key stash.  The spec pair picks the kernels: k2b, or RTN for rtn_token
    keys (post-RoPE) and values (the reference's two fused pairs,
    packed_streaming.py:904-975)."""

    def __init__(self, k_spec: CacheCodecSpec, v_spec: CacheCodecSpec, model_config,
                 recent_window: int = 32, pack_v: bool = True, pack_k: bool = True,
                 pack: "spectral.SpectralPack | None" = None):
        super().__init__()
        self._path = packed_path(k_spec, v_spec)
        self.k_spec, self.v_spec = k_spec, v_spec
        self.model_config = model_config
        self.recent_window = recent_window
        self.pack_v, self.pack_k = pack_v, pack_k   # always packed on this path
        tc = resolve_text_config(model_config)
        self._h_kv = getattr(tc, "num_key_value_heads", None) or tc.num_attention_heads
        self._d_head = getattr(tc, "head_dim", None) or tc.hidden_size // tc.num_attention_heads
        # the k2b kernels take head_dim 32, 64 or 128 (the general page below 128,
        # or at another rank, residual group or key width); RTN and spectral 128
        dims = k2b.HEAD_DIMS if self._path == "k2b" else (k2b.HEAD_DIM,)
        if self._d_head not in dims:
            raise NotImplementedError(f"head_dim {self._d_head}: the {self._path} kernels take head_dim "
                                      f"{' or '.join(str(x) for x in dims)}")
        recipe_page = (self._path == "k2b" and self._d_head == k2b.HEAD_DIM and k_spec.group == k2b.GROUP
                       and k_spec.bits == 3 and k_spec.rank in (16, 32))
        max_h = 16 if self._path == "k2b" and not recipe_page else 8
        if not 1 <= self._h_kv <= max_h:
            raise NotImplementedError(f"{self._h_kv} KV heads: the decode kernel takes 1..{max_h}")
        self._rank = k_spec.rank
        self._page = PAGE
        # the k2b key geometry beyond rank: residual scale group and bits
        self._kgeom = dict(group=k_spec.group, k_bits=k_spec.bits) if self._path == "k2b" else {}
        inv, scaling = K.rope_inv_freq(tc)
        self._inv_freq, self._rope_scaling = inv, scaling
        if self._path in ("k2b", "spectral"):
            self._consts = k2b.CodecConsts.make(v_bits=2, v_seed=v_spec.seed, inv_freq=inv,
                                                rope_scaling=scaling, head_dim=self._d_head)
        else:
            self._rtn = dict(k_bits=k_spec.bits, v_bits=v_spec.bits, k_group=k_spec.group,
                             v_group=v_spec.group,
                             k_arm=rtn.CHANNEL if k_spec.arm == "rtn_channel" else rtn.TOKEN)
        # pre-RoPE key stash: the captured blocks as the hook gave them (kept by
        # reference, no copy per step), rows from absolute position _k_pre_offset
        self._k_pre_parts: list = []
        self._k_pre_rows = 0
        self._k_pre_offset = 0
        # recent window: rows [0, _T) of fixed buffers (1, h_kv, recent_window + 128, d)
        # in the model dtype (fp16 and bf16 windows are the decode kernels' operands
        # as they are; an fp32 window goes in converted); _pending: the newest row's
        # (key, value) when the decode call has still to store it (the product
        # decode path only)
        self._win_k: torch.Tensor | None = None
        self._win_v: torch.Tensor | None = None
        self._T = 0
        self._pending: tuple | None = None
        self.n_rows_folded = 0    # newest rows the decode call stored (no copy of their own)
        # set while PackedStreamingCache.attach has the packed attention read this
        # layer: the one reader that takes a newest row given apart (any other
        # reader of the window lands it first, window())
        self.packed_reader = False
        self._plan = None
        self._plan_key = None
        self._empty_pool: torch.Tensor | None = None
        # committed prefix
        self._committed_S_q = 0
        self._quant_bits_k = 0.0
        self._quant_bits_v = 0.0
        self.bpe_k = float("nan")
        self.bpe_v = float("nan")
        self._frozen_svd: tuple | None = None     # (Us, V) of the first codec page, fp32 CPU
        self._basis32: torch.Tensor | None = None
        self._basis16: torch.Tensor | None = None
        # device page pool: physical page i holds logical page i of this sequence
        self._pool: torch.Tensor | None = None
        self._table: torch.Tensor | None = None   # (1, capacity) int32: 0, 1, 2, ...
        self._n_pages = 0
        self._packed_len_dev: torch.Tensor | None = None
        # spectral keys: the layer's pack, its device operands, the key pages
        # (one per 64-token group; the pool above holds the value pages)
        if self._path == "spectral" and pack is None:
            raise ValueError("the spectral path needs the layer's pack")
        # spectral values: the per-head codec, or the full-C turboquant_mse of the reference's k4 recipe
        self._v_codec = "full" if v_spec.arm == "turboquant_mse" else "perhead"
        if self._path == "spectral" and self._v_codec == "full" and self._h_kv not in (1, 2, 4, 8):
            raise NotImplementedError(f"full-C turboquant_mse values need C = 128 h_kv a power of two "
                                      f"(the reference rotates other C with a random orthogonal matrix); "
                                      f"h_kv {self._h_kv}")
        self._pack = pack
        self._dp: spectral.DevicePack | None = None
        self._kpool: torch.Tensor | None = None
        self._ktable: torch.Tensor | None = None
        self._n_kpages = 0

    # -------------------------------------------------------------- write side

    def stash_pre_rope(self, out: torch.Tensor) -> None:
        """Append captured pre-RoPE keys: (1, S, h_kv*d) or (1, S, h_kv, d)
        (packed_streaming.py:448-457); post-RoPE codecs keep none.  The block is
        kept as given (the projection's output, which the model does not write
        again) until its codec page commits: no device work per step."""
        if not self.k_spec.pre_rope:
            return
        self._k_pre_parts.append(out)
        self._k_pre_rows += out.shape[1]

    def _take_k_pre(self, start: int, end: int) -> torch.Tensor:
        """Stashed pre-RoPE keys of absolute positions [start, end) as (h_kv, n, d)
        fp16; the stash keeps what follows end."""
        if not self._k_pre_parts:
            raise RuntimeError("no pre-RoPE keys captured: call cache.attach(model) before prefill")
        lo, hi = start - self._k_pre_offset, end - self._k_pre_offset
        if lo < 0 or hi > self._k_pre_rows:
            raise RuntimeError(f"pre-RoPE stash holds positions {self._k_pre_offset}.."
                               f"{self._k_pre_offset + self._k_pre_rows}, commit needs {start}..{end}")
        raw = torch.cat(self._k_pre_parts, dim=1) if len(self._k_pre_parts) > 1 else self._k_pre_parts[0]
        block = reshape_heads(raw[:, lo:hi], self._h_kv, self._d_head)
        rest = raw[:, hi:]
        self._k_pre_parts = [rest.clone()] if rest.shape[1] else []
        self._k_pre_rows -= hi
        self._k_pre_offset = end
        return block

    # -------------------------------------------------------------- window

    def _window_dtype(self) -> torch.dtype:
        return self.dtype   # the tail in the model dtype (packed_streaming.py:849)

    def _ensure_window(self, device, committed_after: int) -> None:
        """The window buffers, made on first use (committed_after: the committed
        length this update ends with)."""
        if self._win_k is None:
            cap = self.recent_window + self._page
            self._win_k = torch.zeros(1, self._h_kv, cap, self._d_head, dtype=self._window_dtype(),
                                      device=device)
            self._win_v = torch.zeros_like(self._win_k)
            self._packed_len_dev = torch.zeros(1, dtype=torch.int32, device=device)

    def _land_pending(self) -> None:
        """Store a pending newest row into the window buffers (a copy), for a
        reader other than the decode call that would have stored it."""
        if self._pending is not None:
            k, v = self._pending
            self._pending = None
            self._win_k[:, :, self._T - 1: self._T].copy_(k)
            self._win_v[:, :, self._T - 1: self._T].copy_(v)

    def window(self) -> tuple:
        """The recent window's (keys, values), (1, h_kv, T, d) views of the buffers."""
        if self._win_k is None:
            return None, None
        self._land_pending()
        return self._win_k[:, :, : self._T], self._win_v[:, :, : self._T]

    def _fold_ok(self, key_states: torch.Tensor) -> bool:
        """A one-token step may leave its row to the decode call: the product's
        fused decode paths, an fp16 or bf16 window, on a HIP device, with the
        packed attention as the layer's reader (the tensors update() returns
        are then read by nothing else)."""
        return (self.packed_reader and self._path in ("k2b", "rtn") and key_states.is_cuda
                and self._win_k.dtype in (torch.float16, torch.bfloat16))

    def _reserve(self, n_pages: int, device) -> None:
        """Grow the pool (doubling, contents kept) to hold n_pages pages."""
        cap = 0 if self._pool is None else self._pool.shape[0]
        if n_pages <= cap:
            return
        new_cap = max(n_pages, 2 * cap, 64)
        pb = self._page_bytes()
        pool = torch.zeros(new_cap, pb, dtype=torch.uint8, device=device)
        if self._pool is not None and self._n_pages:
            pool[: self._n_pages].copy_(self._pool[: self._n_pages])
        self._pool = pool
        self._table = torch.arange(new_cap, dtype=torch.int32, device=device).unsqueeze(0)

    def _page_bytes(self) -> int:
        if self._path == "k2b":
            return k2b.page_bytes(self._h_kv, self._rank, head_dim=self._d_head, **self._kgeom)
        if self._path == "spectral":
            return spectral.v_page_bytes(self._h_kv, self._v_codec)
        return rtn.page_bytes(self._h_kv, **self._rtn)

    def _commit_spectral(self, k_pre: torch.Tensor, v: torch.Tensor) -> None:
        """Encode consecutive codec pages (h_kv, 128n, d): the spectral branch
        of _pack_k_block (packed_streaming.py:491-511) and the paired value
        pages, 2n key pages of 64 tokens and 8n value pages of 16."""
        dev = v.device
        if self._dp is None:
            self._dp = spectral.DevicePack(self._pack, self._h_kv, dev, self.k_spec.payload_quant, self._v_codec,
                                             self.v_spec.seed)
        n_grp = k_pre.shape[1] // spectral.GROUP
        kf, vf = self._n_kpages, self._n_pages
        cap = 0 if self._kpool is None else self._kpool.shape[0]
        if kf + n_grp > cap:
            new_cap = max(kf + n_grp, 2 * cap, 16)
            pool = torch.zeros(new_cap, self._dp.k_page_bytes, dtype=torch.uint8, device=dev)
            if self._kpool is not None and kf:
                pool[:kf].copy_(self._kpool[:kf])
            self._kpool = pool
            self._ktable = torch.arange(new_cap, dtype=torch.int32, device=dev)
        self._reserve(vf + 4 * n_grp, dev)
        spectral.append(k_pre.to(dev), v, self._dp, self._kpool, self._ktable[kf: kf + n_grp], self._pool,
                        self._table[0, vf: vf + 4 * n_grp], self._consts)
        self._n_kpages = kf + n_grp
        self._n_pages = vf + 4 * n_grp

    def _commit_rtn(self, k_post: torch.Tensor, v: torch.Tensor) -> None:
        """Encode consecutive codec pages of post-RoPE keys and values
        (h_kv, 128n, d) into the pool (quantize_packed("rtn_token") per side)."""
        dev = v.device
        n = k_post.shape[1] // PAGE
        first = self._n_pages
        self._reserve(first + PAGES_PER_CODEC * n, dev)
        ids = self._table[0, first: first + PAGES_PER_CODEC * n]
        rtn.append(k_post, v, self._pool, ids, **self._rtn)
        self._n_pages = first + PAGES_PER_CODEC * n

    def _commit(self, k_pre: torch.Tensor, v: torch.Tensor) -> None:
        """Encode consecutive codec pages (h_kv, 128n, d) into the pool."""
        dev = v.device
        n = k_pre.shape[1] // PAGE
        us_first = None
        if self._frozen_svd is None:
            M = k_pre[:, :PAGE].float().cpu().permute(1, 0, 2).reshape(PAGE, -1)
            U, s, Vh = torch.linalg.svd(M, full_matrices=False)
            self._frozen_svd = (U[:, : self._rank] * s[: self._rank], Vh[: self._rank].mT.contiguous())
            self._basis32 = self._frozen_svd[1].to(dev).contiguous()
            self._basis16 = self._basis32.half().contiguous()
            us_first = self._frozen_svd[0].to(dev).contiguous()
        first = self._n_pages
        self._reserve(first + PAGES_PER_CODEC * n, dev)
        ids = self._table[0, first: first + PAGES_PER_CODEC * n]
        k2b.append(k_pre.to(dev).half(), v, self._basis32, self._basis16, self._pool, ids,
                   self._consts, rank=self._rank, us_first=us_first, **self._kgeom)
        self._n_pages = first + PAGES_PER_CODEC * n

    def update(self, key_states: torch.Tensor, value_states: torch.Tensor, *args, **kwargs):
        """Append new tokens; commit codec pages on schedule; keep only the
        recent tail in the window (packed_streaming.py:582-730).  Returns views
        of the window; after a one-token step that commits nothing, its newest
        row is stored by the decode call (or by the first other reader,
        window())."""
        if not self.is_initialized:
            self.lazy_initialization(key_states, value_states)
        n = key_states.shape[2]
        T0 = self._T
        S = self._committed_S_q + T0 + n
        W = self.recent_window
        C = self._h_kv * self._d_head
        new_S_q = K.compute_flush_schedule(S, W, self._page)
        self._ensure_window(key_states.device, new_S_q)
        self._land_pending()
        if new_S_q == self._committed_S_q:   # nothing commits: the rows join the window
            if n == 1 and self._fold_ok(key_states):
                wdt = self._win_k.dtype   # the model's rows as they are (no conversion kernel)
                self._pending = (key_states.to(wdt), value_states.to(wdt))
            else:
                self._win_k[:, :, T0:T0 + n].copy_(key_states)
                self._win_v[:, :, T0:T0 + n].copy_(value_states)
            self._T = T0 + n
            self._set_bpe(S)
            self._publish()
            return self.keys, self.values
        wdt = self._win_k.dtype
        if T0:
            keys = torch.cat([self._win_k[:, :, :T0], key_states.to(wdt)], dim=2)
            values = torch.cat([self._win_v[:, :, :T0], value_states.to(wdt)], dim=2)
        else:
            keys, values = key_states, value_states
        if new_S_q > self._committed_S_q:
            start, end = self._committed_S_q, new_S_q
            v_new = values.squeeze(0)[:, : end - start, :]
            n_cp = (end - start) // self._page
            page_entries = self._page * C
            if self._path == "rtn":   # post-RoPE keys straight from the window
                self._commit_rtn(keys.squeeze(0)[:, : end - start, :], v_new)
                self._quant_bits_k += n_cp * (self.k_spec.bits + 16.0 / self.k_spec.group) * page_entries
                self._quant_bits_v += n_cp * (self.v_spec.bits + 16.0 / self.v_spec.group) * page_entries
                self._committed_S_q = end
            else:
                k_pre = self._take_k_pre(start, end)
                if self._path == "spectral":
                    self._commit_spectral(k_pre, v_new)
                    self._quant_bits_k += n_cp * spectral.payload_bpe(self._pack.bits, self._pack.group) \
                        * page_entries
                else:
                    self._commit(k_pre, v_new)
                    self._quant_bits_k += n_cp * K.bpe_k(self._rank, C, bits=self.k_spec.bits,
                                                         group=self.k_spec.group) * page_entries
                self._quant_bits_v += n_cp * K.bpe_v(1 if self._v_codec == "full" else self._h_kv, C) * page_entries
                self._committed_S_q = end
            keys = keys[..., end - start:, :]
            values = values[..., end - start:, :]
            self._packed_len_dev.fill_(end)
            self._after_commit(start, end)
        T = keys.shape[2]
        if T > self._win_k.shape[2]:
            raise RuntimeError(f"window of {T} rows exceeds its buffer ({self._win_k.shape[2]})")
        self._win_k[:, :, :T].copy_(keys)
        self._win_v[:, :, :T].copy_(values)
        self._T = T
        self._set_bpe(S)
        self._publish()
        return self.keys, self.values

    def _after_commit(self, start: int, end: int) -> None:
        """Hook: positions [start, end) were just committed."""

    def _publish(self) -> None:
        """What update() returns and the layer holds as keys/values: the window."""
        self.keys, self.values = self._win_k[:, :, : self._T], self._win_v[:, :, : self._T]

    def _set_bpe(self, S: int) -> None:
        C = self._h_kv * self._d_head
        total = S * C
        if total > 0:
            tail = self._T * C * 16.0
            self.bpe_k = (self._quant_bits_k + tail) / total
            self.bpe_v = (self._quant_bits_v + tail) / total

    def get_seq_length(self) -> int:
        return self._committed_S_q + self._T

    # -------------------------------------------------------------- DynamicLayer mutators
    # DynamicLayer's own versions slice self.keys / self.values, which here are
    # views of the window alone: they would leave the committed pages, the
    # window length and the pre-RoPE stash out of step.

    def crop(self, tokens_to_remove: int) -> None:
        """Drop the newest tokens (DynamicLayer.crop: a negative count removes
        that many, a positive one is the length to keep).  Only window rows can
        go: committed codec pages are not taken back."""
        n = self.get_seq_length()
        drop = -tokens_to_remove if tokens_to_remove <= 0 else max(n - tokens_to_remove, 0)
        if drop == 0:
            return
        if drop > self._T:
            raise NotImplementedError(f"crop of {drop} tokens reaches into the committed codec pages "
                                      f"({self._T} window rows)")
        self._land_pending()
        keep = n - drop
        if self._k_pre_rows > keep - self._k_pre_offset:   # stashed pre-RoPE rows past the new end
            raw = torch.cat(self._k_pre_parts, dim=1) if len(self._k_pre_parts) > 1 else self._k_pre_parts[0]
            raw = raw[:, : max(keep - self._k_pre_offset, 0)]
            self._k_pre_parts = [raw] if raw.shape[1] else []
            self._k_pre_rows = raw.shape[1]
        self._T -= drop
        self._set_bpe(keep)
        self._publish()

    def _one_sequence(self, what: str, ok: bool) -> None:
        if not ok:
            raise NotImplementedError(f"{what}: the packed cache serves batch size 1")

    def reorder_cache(self, beam_idx: torch.LongTensor) -> None:
        self._one_sequence("reorder_cache", beam_idx.numel() == 1 and int(beam_idx.reshape(-1)[0]) == 0)

    def batch_select_indices(self, indices: torch.Tensor) -> None:
        idx = torch.as_tensor(indices).reshape(-1)
        self._one_sequence("batch_select_indices", idx.numel() == 1 and int(idx[0]) == 0)

    def batch_repeat_interleave(self, repeats: int) -> None:
        self._one_sequence("batch_repeat_interleave", repeats == 1)

    def offload(self):
        raise NotImplementedError("the packed cache's page pool stays on the device")

    def prefetch(self):
        raise NotImplementedError("the packed cache's page pool stays on the device")

    def reset(self) -> None:
        """Forget every token (the layer object stays, as DynamicLayer.reset
        keeps it): pages, window and stash are released."""
        reader = self.packed_reader
        self.__init__(self.k_spec, self.v_spec, self.model_config, recent_window=self.recent_window,
                      pack=self._pack)
        self.packed_reader = reader

    # -------------------------------------------------------------- read side

    def attend(self, q: torch.Tensor, scaling: float, is_causal: bool = False,
               attention_mask: torch.Tensor | None = None) -> torch.Tensor:
        """q (n_q_heads, n_q, d) post-RoPE -> (n_q_heads, n_q, d)."""
        if q.device.type != "cuda":
            raise RuntimeError("the packed cache attends on a HIP device only (no CPU path)")
        n_heads, n_q, d = q.shape
        G = n_heads // self._h_kv
        if n_q == 1 and not is_causal:
            if self._path == "spectral":
                return self._decode_spectral(q, scaling, G)
            return self._decode(q, scaling, G)
        return self._dense(q, scaling, G, is_causal and n_q > 1, attention_mask)

    def _decode(self, q: torch.Tensor, scaling: float, G: int) -> torch.Tensor:
        """One query step through the layer's bound decode plan: q, the window
        length and the pending newest row are the only per-call arguments."""
        dev = q.device
        h, d = self._h_kv, self._d_head
        P, T = self._committed_S_q, self._T
        # the query goes in as the model gives it (fp32, fp16 or bf16; the kernels
        # convert on load), and the output comes back in the same dtype
        qm = q.reshape(1, h, G, d)
        if not qm.is_contiguous():
            qm = qm.contiguous()
        if self._win_k.dtype not in (torch.float16, torch.bfloat16):   # an fp32 model: the window goes in as fp16
            self._land_pending()
            kt = self._win_k[:, :, :T].half().contiguous()
            vt = self._win_v[:, :, :T].half().contiguous()
            pool, table, basis16 = self._decode_operands(dev)
            if self._path == "rtn":
                out = rtn.decode(qm, pool, table, self._packed_len_dev, P, scaling, k_tail=kt, v_tail=vt,
                                 tail_len=T, tail_cap=T, **self._rtn)
            else:
                out = k2b.decode(qm, pool, None, self._packed_len_dev, P, basis16, self._consts, scaling,
                                 rank=self._rank, k_tail=kt, v_tail=vt, tail_len=T, tail_cap=T, **self._kgeom)
            return out.reshape(h * G, 1, d)
        key = (P, G, float(scaling), qm.dtype, None if self._pool is None else self._pool.data_ptr())
        if self._plan is None or self._plan_key != key:
            pool, table, basis16 = self._decode_operands(dev)
            cap = self._win_k.shape[2]
            common = dict(k_tail=self._win_k, v_tail=self._win_v, tail_len=T, tail_cap=cap,
                          out=torch.empty_like(qm))
            if self._path == "rtn":
                self._plan = rtn.DecodePlan(qm, pool, table, self._packed_len_dev, P, scaling, **common,
                                            **self._rtn)
            else:
                self._plan = k2b.DecodePlan(qm, pool, None, self._packed_len_dev, P, basis16, self._consts,
                                            scaling, rank=self._rank, **common, **self._kgeom)
            self._plan_key = key
        pending, self._pending = self._pending, None
        # a fresh output tensor per call (an allocation, no kernel): the caller
        # may keep it past the layer's next step
        out = self._plan.run(q=qm, tail_len=T, new_kv=pending, out=torch.empty_like(qm))
        self.n_rows_folded += pending is not None
        return out.reshape(h * G, 1, d)

    def _decode_operands(self, dev) -> tuple:
        """(pool, page table, basis16) for a decode over the committed pages; with
        none committed, stand-ins that the kernel does not read."""
        if self._committed_S_q > 0:
            return self._pool, self._table, self._basis16
        if self._empty_pool is None:
            self._empty_pool = (torch.zeros(1, self._page_bytes(), dtype=torch.uint8, device=dev),
                                torch.zeros(1, 1, dtype=torch.int32, device=dev),
                                torch.zeros(self._h_kv * self._d_head, max(self._rank or 16, 16),
                                            dtype=torch.float16, device=dev))
        return self._empty_pool

    def _decode_spectral(self, q: torch.Tensor, scaling: float, G: int) -> torch.Tensor:
        """One decode step of the spectral arm: the reference's chunked step
        (every committed page dequantized, packed_streaming.py:1016-1032) with
        the keys rebuilt, scored, weighted and applied to the values inside the
        dequant kernel (one softmax partial per 64-token group, no dense rows
        written), merged with the fp16 window's partial."""
        h, d = self._h_kv, self._d_head
        P = self._committed_S_q
        if self._dp is None:   # a step before the first commit: the window alone
            self._dp = spectral.DevicePack(self._pack, self._h_kv, q.device, self.k_spec.payload_quant,
                                             self._v_codec, self.v_spec.seed)
        qg = q.reshape(h, G, d).contiguous()
        kw = vw = None
        wk, wv = self.window()
        if wk is not None and wk.shape[2]:   # fp16 / bf16 buffers are read in place (rows contiguous)
            kw, vw = wk.squeeze(0), wv.squeeze(0)
            if kw.dtype not in (torch.float16, torch.bfloat16):
                kw, vw = kw.half().contiguous(), vw.half().contiguous()
        kt = self._ktable[: P // spectral.GROUP] if P else None
        vt = self._table[0, : P // k2b.PAGE_TOKENS].contiguous() if P else None
        out = spectral.decode_attention(self._dp, self._kpool, kt, self._pool, vt, P, self._consts, qg, scaling,
                                        k_win=kw, v_win=vw, apply_rope=k2b.ROPE_FP16_TABLES)
        return out.reshape(h * G, 1, d)

    def _dense(self, q, scaling, G, causal, attention_mask):
        """Prefill (n_q > 1): _prefill_dense_attention (chunked_attention.py:
        320-395).  The page kernel dequantizes the committed pages straight to
        the model dtype (k2b keys rotated in the same pass with the fp16 RoPE
        tables, as _dense_kv does), the fp16 window follows, and one attention
        call reads the grouped heads in place (no G-fold copy of K and V).
        With no mask, or fewer queries than keys and the model's mask equal to
        the causal mask of the last n_q positions (bottom right), that is
        bmx_prefill (fp16 / bf16, head dim 128); other head dims take SDPA's
        flash kernel or its bottom-right causal bias for the same masks; any
        other mask takes SDPA's memory-efficient kernel over expanded heads."""
        dev, dt = q.device, q.dtype
        P = self._committed_S_q
        wk, wv = self.window()
        T = 0 if wk is None else wk.shape[2]
        if P > 0:
            # the committed rows dequantized straight into one buffer with the
            # window after them: no concatenation of the dense prefix
            Kd = torch.empty(self._h_kv, P + T, self._d_head, dtype=dt, device=dev)
            Vd = torch.empty_like(Kd)
            if self._path == "rtn":   # keys were committed post-RoPE
                rtn.dequant(self._pool, self._table[0, : P // rtn.PAGE_TOKENS].contiguous(), h_kv=self._h_kv,
                            dtype=dt, out=(Kd, Vd), **self._rtn)
            elif self._path == "spectral":   # keys rotated at read with the fp16 tables
                spectral.dequant(self._dp, self._kpool, self._ktable[: P // spectral.GROUP], self._pool,
                                 self._table[0, : P // k2b.PAGE_TOKENS].contiguous(), P, self._consts,
                                 apply_rope=k2b.ROPE_FP16_TABLES, dtype=dt, out=(Kd, Vd))
            else:
                k2b.dequant(self._pool, self._table[0, : P // k2b.PAGE_TOKENS].contiguous(), P, self._basis16,
                            self._consts, h_kv=self._h_kv, rank=self._rank, apply_rope=k2b.ROPE_FP16_TABLES,
                            dtype=dt, out=(Kd, Vd), **self._kgeom)
            if T:
                Kd[:, P:].copy_(wk.squeeze(0))
                Vd[:, P:].copy_(wv.squeeze(0))
        else:
            Kd, Vd = wk.squeeze(0).to(dt), wv.squeeze(0).to(dt)
        n_q, n_kv = q.shape[1], Kd.shape[1]
        lower_right = n_q != n_kv and ((causal and attention_mask is None)
                                       or _is_lower_right_causal(attention_mask, n_q, n_kv))
        if (lower_right or attention_mask is None) and prefill.supported(q, Kd, Vd):
            # bmx_prefill: grouped heads read their K/V head in place; causal
            # is the bottom-right mask (n_q == n_kv: the ordinary one)
            return prefill.attention(q, Kd, Vd, scaling, causal=causal or lower_right)
        if lower_right:
            # the queries are the last n_q positions: causal from the bottom
            # right, which ROCm's kernels take as a bias of their own (grouped
            # heads, no mask tensor: ~1.5x the memory-efficient kernel's speed
            # with the equal boolean mask)
            out = F.scaled_dot_product_attention(q.unsqueeze(0), Kd.unsqueeze(0), Vd.unsqueeze(0),
                                                 attn_mask=causal_lower_right(n_q, n_kv), scale=scaling,
                                                 enable_gqa=G > 1)
            return out.squeeze(0)
        if attention_mask is None:
            # no mask: ROCm's flash attention takes the grouped heads as they are
            out = F.scaled_dot_product_attention(q.unsqueeze(0), Kd.unsqueeze(0), Vd.unsqueeze(0),
                                                 is_causal=causal, scale=scaling, enable_gqa=G > 1)
        else:
            # with a mask only the memory-efficient kernel serves (the grouped-head
            # form would fall back to the math path, several times slower): expand
            out = F.scaled_dot_product_attention(
                q.unsqueeze(0), Kd.repeat_interleave(G, dim=0).unsqueeze(0),
                Vd.repeat_interleave(G, dim=0).unsqueeze(0), attn_mask=attention_mask, scale=scaling)
        return out.squeeze(0)


_MASK_SEEN: list = [None, -1, False]   # (weak reference to the mask, its version, the answer)


def _is_lower_right_causal(mask, n_q: int, n_kv: int) -> bool:
    """Whether a model's boolean mask (1, 1, n_q, n_kv) is exactly the causal
    mask of the last n_q positions over n_kv keys.  One device compare (the
    host waits for it) per mask: the model hands every layer the same mask
    tensor, so the answer is kept for it while it lives unmodified."""
    if mask is None or mask.dtype != torch.bool or mask.dim() != 4 or tuple(mask.shape) != (1, 1, n_q, n_kv):
        return False
    ref, version, answer = _MASK_SEEN
    if ref is not None and ref() is mask and version == mask._version:
        return answer
    i = torch.arange(n_q, device=mask.device)[:, None]
    j = torch.arange(n_kv, device=mask.device)[None, :]
    answer = bool(torch.equal(mask[0, 0], j <= i + (n_kv - n_q)))
    _MASK_SEEN[:] = [weakref.ref(mask), mask._version, answer]
    return answer


# ------------------------------------------------------------------ cache


class PackedStreamingCache(Cache):
    """Drop-in ``past_key_values=`` for ``model()`` / ``model.generate()``
    (packed_streaming.py:1067-1222).

        cache = PackedStreamingCache(model.config, *spec_pair("k2b_ph", rank=32))
        with cache.attach(model):
            out = model.generate(ids, past_key_values=cache, ...)
    """

    _layer_cls = PackedStreamingLayer

    def __init__(self, model_config, k_spec: CacheCodecSpec, v_spec: CacheCodecSpec,
                 recent_window: int = 32, pack_v: bool = True, pack_k: bool = True):
        path = packed_path(k_spec, v_spec)
        # spectral: every layer's pack, loaded once (packed_streaming.py:1094-1147)
        # decoder variants (dec_quant) applied here, once (spectral.py:1254-1326)
        self._packs = spectral.load_packs_for_spec(k_spec) if path == "spectral" else {}
        wself = weakref.proxy(self)   # no cache -> closure -> cache cycle

        def _make_layer():
            i = len(wself.layers)    # layers are made in order, layer i when len(layers) == i
            pack = None
            if path == "spectral":
                if i not in wself._packs:
                    raise KeyError(f"spectral pack file missing layer {i}")
                pack = wself._packs[i]
            return wself._layer_cls(wself.k_spec, wself.v_spec, wself.model_config,
                                    wself.recent_window, pack_v=wself.pack_v, pack_k=wself.pack_k,
                                    pack=pack)

        self._make_layer = _make_layer
        super().__init__(layer_class_to_replicate=_make_layer)
        self.model_config = model_config
        self.k_spec, self.v_spec = k_spec, v_spec
        self.recent_window = recent_window
        self.pack_v, self.pack_k = pack_v, pack_k
        self._handles: list = []
        self._saved_impl = None
        self._model = None

    def bits_per_entry(self) -> tuple:
        """(bpe_k, bpe_v): blended payload bits per entry, averaged across layers
        (cache_bits_per_entry, streaming.py:154-260).  Spectral keys, once a
        layer has committed, also pay the decoder and tier map over the whole
        sequence at the layer-mean coded and int8 column counts (the charge
        is linear in both), the int8 count read from each pack's dec_tier."""
        layers = list(self.layers)
        if not layers:
            return float("nan"), float("nan")
        bpe_k = sum(l.bpe_k for l in layers) / len(layers)
        bpe_v = sum(l.bpe_v for l in layers) / len(layers)
        last = layers[-1]
        if self.k_spec.arm == "spectral" and last._committed_S_q > 0:
            c_used = sum(l._pack.c_used for l in layers) / len(layers)
            c_int8 = sum(0 if l._pack.dec_tier is None else l._pack.c_int8(l._pack.dec_tier)
                         for l in layers) / len(layers)
            bpe_k += spectral.mixed_dec_charge(last._h_kv * last._d_head, last.get_seq_length(),
                                               last._pack.tiers, c_used, c_int8)
        return bpe_k, bpe_v

    def memory_report(self, seq_len: int) -> dict:
        """Dense fp16 bytes vs packed (bpe-derived) bytes (streaming.py:263-305)."""
        bpe_k, bpe_v = self.bits_per_entry()
        cfg = resolve_text_config(self.model_config)
        h_kv = getattr(cfg, "num_key_value_heads", None) or cfg.num_attention_heads
        d = getattr(cfg, "head_dim", None) or cfg.hidden_size // cfg.num_attention_heads
        entries = cfg.num_hidden_layers * h_kv * seq_len * d
        fp16_bytes = 2 * entries * 2
        bpe_k = 16.0 if math.isnan(bpe_k) else bpe_k
        bpe_v = 16.0 if math.isnan(bpe_v) else bpe_v
        packed_bytes = entries * (bpe_k + bpe_v) / 8.0
        return {"fp16_bytes": float(fp16_bytes), "packed_bytes": float(packed_bytes),
                "compression": fp16_bytes / max(packed_bytes, 1e-9)}

    def attach(self, model) -> "PackedStreamingCache":
        """Route the model's attention through the packed layers and capture
        pre-RoPE keys (packed_streaming.py:1150-1180)."""
        self.detach()
        self._model = model
        self._saved_impl = model.config._attn_implementation
        model.config._attn_implementation = ATTN_NAME
        decoder = resolve_decoder_layers(model)
        while len(self.layers) < len(decoder):
            self.layers.append(self._make_layer())
        for i, mlayer in enumerate(decoder):
            mlayer.self_attn._packed_layer = self.layers[i]
            self.layers[i].packed_reader = True
            layer_ref = weakref.proxy(self.layers[i])

            def k_hook(module, inp, out, layer=layer_ref):
                layer.stash_pre_rope(out)

            self._handles.append(resolve_k_capture_module(mlayer.self_attn).register_forward_hook(k_hook))
        return self

    def detach(self) -> "PackedStreamingCache":
        for h in self._handles:
            h.remove()
        self._handles = []
        for layer in self.layers:
            if isinstance(layer, PackedStreamingLayer):
                layer.packed_reader = False
                if layer._win_k is not None:
                    layer._land_pending()
        if self._model is not None:
            for mlayer in resolve_decoder_layers(self._model):
                if hasattr(mlayer.self_attn, "_packed_layer"):
                    del mlayer.self_attn._packed_layer
            if self._saved_impl is not None:
                self._model.config._attn_implementation = self._saved_impl
        self._model = None
        self._saved_impl = None
        return self

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.detach()
        return False


# ------------------------------------------------------------------ streaming twin


class StreamingQuantizedLayer(PackedStreamingLayer):
    """The reference's StreamingQuantizedLayer (cache/streaming.py:308-650) on
    the packed kernels: the same flush schedule and codecs; each committed codec
    page is encoded by the append kernel and then, once, dequantized by the
    page kernel into a write-once dense prefix in the cache dtype (k2b keys
    rotated at their true positions with fp32 cos/sin, as
    _quantize_k_block_pre_rope does at :390-453).  The layer's keys/values are
    that prefix followed by the pristine recent tail, and the model's own
    attention (SDPA) reads them.  Prefix and tail share one slab
    (1, h_kv, capacity, d) indexed by absolute position, the tail a sliding view
    of it from the committed length on: a step appends one row, a commit moves
    none, and the slab grows by doubling."""

    def __init__(self, k_spec: CacheCodecSpec, v_spec: CacheCodecSpec, model_config,
                 recent_window: int = 32, pack_v: bool = True, pack_k: bool = True,
                 pack: "spectral.SpectralPack | None" = None):
        super().__init__(k_spec, v_spec, model_config, recent_window, pack_v=pack_v, pack_k=pack_k, pack=pack)
        self._slab_k: torch.Tensor | None = None
        self._slab_v: torch.Tensor | None = None

    def _fold_ok(self, key_states: torch.Tensor) -> bool:
        return False

    def _ensure_window(self, device, committed_after: int) -> None:
        need = committed_after + self.recent_window + self._page
        have = 0 if self._slab_k is None else self._slab_k.shape[2]
        if need > have:
            rows = max(need, 2 * have, 1024)
            k = torch.zeros(1, self._h_kv, rows, self._d_head, dtype=self._window_dtype(), device=device)
            v = torch.zeros_like(k)
            used = self._committed_S_q + self._T
            if used:
                k[:, :, :used].copy_(self._slab_k[:, :, :used])
                v[:, :, :used].copy_(self._slab_v[:, :, :used])
            self._slab_k, self._slab_v = k, v
            if self._packed_len_dev is None:
                self._packed_len_dev = torch.zeros(1, dtype=torch.int32, device=device)
        self._point_window(self._committed_S_q)

    def _point_window(self, P: int) -> None:
        cap = self.recent_window + self._page
        self._win_k = self._slab_k[:, :, P:P + cap]
        self._win_v = self._slab_v[:, :, P:P + cap]

    def _after_commit(self, start: int, end: int) -> None:
        """Dequantize the pages of positions [start, end) into slab rows [start, end)."""
        dt = self._slab_k.dtype
        out = (self._slab_k[0, :, start:], self._slab_v[0, :, start:])
        p0, p1 = start // k2b.PAGE_TOKENS, end // k2b.PAGE_TOKENS
        if self._path == "rtn":
            rtn.dequant(self._pool, self._table[0, p0:p1].contiguous(), h_kv=self._h_kv, dtype=dt, out=out,
                        **self._rtn)
        elif self._path == "spectral":
            # the spectral page kernel writes from position 0: the whole prefix again
            spectral.dequant(self._dp, self._kpool, self._ktable[: end // spectral.GROUP], self._pool,
                             self._table[0, :p1].contiguous(), end, self._consts, apply_rope=k2b.ROPE_EXACT,
                             dtype=dt, out=(self._slab_k[0], self._slab_v[0]))
        else:
            k2b.dequant(self._pool, self._table[0, p0:p1].contiguous(), end - start, self._basis16, self._consts,
                        h_kv=self._h_kv, rank=self._rank, apply_rope=k2b.ROPE_EXACT, dtype=dt, pos0=start,
                        out=out, **self._kgeom)
        self._point_window(end)

    def _publish(self) -> None:
        S = self._committed_S_q + self._T
        self.keys, self.values = self._slab_k[:, :, :S], self._slab_v[:, :, :S]

    def attend(self, q, scaling, is_causal=False, attention_mask=None):
        raise RuntimeError("StreamingQuantizedLayer is read by the model's own attention")


class StreamingQuantizedCache(PackedStreamingCache):
    """Drop-in ``past_key_values=`` twin of PackedStreamingCache
    (cache/streaming.py:653-815): the same specs and flush schedule, the
    committed prefix resident dequantized, attention by the model's own
    implementation.  ``attach(model)`` only registers the pre-RoPE key capture
    (a no-op for post-RoPE key codecs)."""

    _layer_cls = StreamingQuantizedLayer

    def __init__(self, model_config, k_spec: CacheCodecSpec, v_spec: CacheCodecSpec,
                 recent_window: int = 32):
        super().__init__(model_config, k_spec, v_spec, recent_window)

    def attach(self, model) -> "StreamingQuantizedCache":
        self.detach()
        if not self.k_spec.pre_rope:
            return self
        self._model = model
        decoder = resolve_decoder_layers(model)
        while len(self.layers) < len(decoder):
            self.layers.append(self._make_layer())
        for i, mlayer in enumerate(decoder):
            layer_ref = weakref.proxy(self.layers[i])

            def k_hook(module, inp, out, layer=layer_ref):
                layer.stash_pre_rope(out)

            self._handles.append(resolve_k_capture_module(mlayer.self_attn).register_forward_hook(k_hook))
        return self

    def reconstruct_layer(self, layer_idx: int) -> tuple:
        """(keys, values) as the layer holds them, (1, h_kv, S, d): RoPE'd keys,
        dequantized prefix then the fp16 tail (streaming.py:780-786)."""
        layer = self.layers[layer_idx]
        return layer.keys, layer.values


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
  recent-window slab;
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
from transformers.cache_utils import Cache, DynamicLayer
from transformers.masking_utils import ALL_MASK_ATTENTION_FUNCTIONS, sdpa_mask
from transformers.modeling_utils import ALL_ATTENTION_FUNCTIONS

from . import codecs as K
from . import k2b, rtn, spectral
from .specs import CacheCodecSpec, packed_path

ATTN_NAME = "bmx_k2b"
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


ALL_ATTENTION_FUNCTIONS.register(ATTN_NAME, packed_attention_forward)
ALL_MASK_ATTENTION_FUNCTIONS.register(ATTN_NAME, sdpa_mask)


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
        if self._d_head != k2b.HEAD_DIM:
            raise NotImplementedError(f"head_dim {self._d_head}: the packed kernels take head_dim 128")
        if not 1 <= self._h_kv <= 8:
            raise NotImplementedError(f"{self._h_kv} KV heads: the decode kernel takes 1..8")
        self._rank = k_spec.rank
        self._page = PAGE
        inv, scaling = K.rope_inv_freq(tc)
        self._inv_freq, self._rope_scaling = inv, scaling
        if self._path in ("k2b", "spectral"):
            self._consts = k2b.CodecConsts.make(v_bits=2, v_seed=v_spec.seed, inv_freq=inv,
                                                rope_scaling=scaling)
        else:
            self._rtn = dict(k_bits=k_spec.bits, v_bits=v_spec.bits, k_group=k_spec.group,
                             v_group=v_spec.group,
                             k_arm=rtn.CHANNEL if k_spec.arm == "rtn_channel" else rtn.TOKEN)
        # pre-RoPE key stash
        self._k_pre: torch.Tensor | None = None
        self._k_pre_offset = 0
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
        self._pack = pack
        self._dp: spectral.DevicePack | None = None
        self._kpool: torch.Tensor | None = None
        self._ktable: torch.Tensor | None = None
        self._n_kpages = 0

    # -------------------------------------------------------------- write side

    def stash_pre_rope(self, out: torch.Tensor) -> None:
        """Append captured pre-RoPE keys: (1, S, h_kv*d) or (1, S, h_kv, d)
        (packed_streaming.py:448-457); post-RoPE codecs keep none."""
        if not self.k_spec.pre_rope:
            return
        block = reshape_heads(out, self._h_kv, self._d_head)
        self._k_pre = block if self._k_pre is None else torch.cat([self._k_pre, block], dim=1)

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
            return k2b.page_bytes(self._h_kv, self._rank)
        if self._path == "spectral":
            return int(_lib_v_page_bytes(self._h_kv))
        return rtn.page_bytes(self._h_kv, **self._rtn)

    def _commit_spectral(self, k_pre: torch.Tensor, v: torch.Tensor) -> None:
        """Encode consecutive codec pages (h_kv, 128n, d): the spectral branch
        of _pack_k_block (packed_streaming.py:491-511) and the paired value
        pages, 2n key pages of 64 tokens and 8n value pages of 16."""
        dev = v.device
        if self._dp is None:
            self._dp = spectral.DevicePack(self._pack, self._h_kv, dev)
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
                   self._consts, rank=self._rank, us_first=us_first)
        self._n_pages = first + PAGES_PER_CODEC * n

    def update(self, key_states: torch.Tensor, value_states: torch.Tensor, *args, **kwargs):
        """Append new tokens; commit codec pages on schedule; keep only the fp16
        tail in the slab (packed_streaming.py:582-730)."""
        keys, values = super().update(key_states, value_states, *args, **kwargs)
        S = self._committed_S_q + keys.shape[2]
        W = self.recent_window
        C = self._h_kv * self._d_head
        new_S_q = K.compute_flush_schedule(S, W, self._page)
        if new_S_q > self._committed_S_q:
            start, end = self._committed_S_q, new_S_q
            v_new = values.squeeze(0)[:, : end - start, :]
            n_cp = (end - start) // self._page
            page_entries = self._page * C
            if self._path == "rtn":   # post-RoPE keys straight from the slab
                self._commit_rtn(keys.squeeze(0)[:, : end - start, :], v_new)
                self._quant_bits_k += n_cp * (self.k_spec.bits + 16.0 / self.k_spec.group) * page_entries
                self._quant_bits_v += n_cp * (self.v_spec.bits + 16.0 / self.v_spec.group) * page_entries
                self._committed_S_q = end
            else:
                if self._k_pre is None:
                    raise RuntimeError("no pre-RoPE keys captured: call cache.attach(model) before prefill")
                lo, hi = start - self._k_pre_offset, end - self._k_pre_offset
                if self._path == "spectral":
                    self._commit_spectral(self._k_pre[:, lo:hi, :], v_new)
                    self._quant_bits_k += n_cp * spectral.payload_bpe(self._pack.bits, self._pack.group) \
                        * page_entries
                else:
                    self._commit(self._k_pre[:, lo:hi, :], v_new)
                    self._quant_bits_k += n_cp * K.bpe_k(self._rank, C) * page_entries
                self._quant_bits_v += n_cp * K.bpe_v(self._h_kv, C) * page_entries
                self._committed_S_q = end
                if hi >= self._k_pre.shape[1]:
                    self._k_pre, self._k_pre_offset = None, end
                elif hi > 0:
                    self._k_pre, self._k_pre_offset = self._k_pre[:, hi:, :].contiguous(), end
            keys = keys[..., end - start:, :].contiguous()
            values = values[..., end - start:, :].contiguous()
            self._packed_len_dev = None
        total = S * C
        if total > 0:
            tail = keys.shape[2] * C * 16.0
            self.bpe_k = (self._quant_bits_k + tail) / total
            self.bpe_v = (self._quant_bits_v + tail) / total
        self.keys, self.values = keys, values
        return keys, values

    def get_seq_length(self) -> int:
        if not self.is_initialized or self.keys is None or self.keys.numel() == 0:
            return self._committed_S_q
        return self._committed_S_q + self.keys.shape[-2]

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
        dev = q.device
        P = self._committed_S_q
        if self._packed_len_dev is None or self._packed_len_dev.device != dev:
            self._packed_len_dev = torch.tensor([P], dtype=torch.int32, device=dev)
        k_tail = self.keys.half().contiguous()
        v_tail = self.values.half().contiguous()
        T = k_tail.shape[2]
        if self._path == "rtn":
            if P > 0:
                pool, table = self._pool, self._table
            else:
                pool = torch.zeros(1, self._page_bytes(), dtype=torch.uint8, device=dev)
                table = torch.zeros(1, 1, dtype=torch.int32, device=dev)
            out = rtn.decode(
                q.reshape(1, self._h_kv, G, self._d_head).float().contiguous(), pool, table,
                self._packed_len_dev, P, scaling, k_tail=k_tail, v_tail=v_tail,
                tail_len=torch.tensor([T], dtype=torch.int32, device=dev), tail_cap=T, **self._rtn)
            return out.reshape(self._h_kv * G, 1, self._d_head)
        if P > 0:
            # the pool holds this sequence's pages in order: no table to read
            pool, basis16 = self._pool, self._basis16
        else:   # window only: the kernel reads no page
            pool = torch.zeros(1, k2b.page_bytes(self._h_kv, self._rank), dtype=torch.uint8, device=dev)
            basis16 = torch.zeros(self._h_kv * self._d_head, self._rank, dtype=torch.float16, device=dev)
        out = k2b.decode(
            q.reshape(1, self._h_kv, G, self._d_head).float().contiguous(), pool, None,
            self._packed_len_dev, P, basis16, self._consts, scaling, rank=self._rank,
            k_tail=k_tail, v_tail=v_tail,
            tail_len=torch.tensor([T], dtype=torch.int32, device=dev), tail_cap=T)
        return out.reshape(self._h_kv * G, 1, self._d_head)

    def _decode_spectral(self, q: torch.Tensor, scaling: float, G: int) -> torch.Tensor:
        """One decode step of the spectral arm: the reference's chunked step
        (every committed page dequantized, packed_streaming.py:1016-1032) with
        the keys rebuilt, scored, weighted and applied to the values inside the
        dequant kernel (one softmax partial per 64-token group, no dense rows
        written), merged with the fp16 window's partial."""
        h, d = self._h_kv, self._d_head
        P = self._committed_S_q
        if self._dp is None:   # a step before the first commit: the window alone
            self._dp = spectral.DevicePack(self._pack, self._h_kv, q.device)
        qg = q.reshape(h, G, d).contiguous()
        kw = vw = None
        if self.keys is not None and self.keys.numel():
            kw, vw = self.keys.squeeze(0).half().contiguous(), self.values.squeeze(0).half().contiguous()
        kt = self._ktable[: P // spectral.GROUP] if P else None
        vt = self._table[0, : P // k2b.PAGE_TOKENS].contiguous() if P else None
        out = spectral.decode_attention(self._dp, self._kpool, kt, self._pool, vt, P, self._consts, qg, scaling,
                                        k_win=kw, v_win=vw, apply_rope=k2b.ROPE_FP16_TABLES)
        return out.reshape(h * G, 1, d)

    def _dense(self, q, scaling, G, causal, attention_mask):
        """Prefill (n_q > 1): _prefill_dense_attention (chunked_attention.py:
        320-395).  The page kernel dequantizes the committed pages straight to
        the model dtype (k2b keys rotated in the same pass with the fp16 RoPE
        tables, as _dense_kv does), the fp16 window follows, and one SDPA
        attends: flash attention over the grouped heads (no G-fold copy of K
        and V) when no mask is needed, the memory-efficient kernel over expanded
        heads with one.  With no mask from the model and fewer queries than
        keys, the queries are the last n_q positions: the mask is causal from
        the bottom right."""
        dev, dt = q.device, q.dtype
        P = self._committed_S_q
        parts_k, parts_v = [], []
        if P > 0 and self._path == "rtn":   # keys were committed post-RoPE
            kp, vp = rtn.dequant(self._pool, self._table[0, : P // rtn.PAGE_TOKENS].contiguous(),
                                 h_kv=self._h_kv, dtype=dt, **self._rtn)
            parts_k.append(kp)
            parts_v.append(vp)
        elif P > 0 and self._path == "spectral":
            # keys rotated at read with the fp16 tables, written with room for
            # the window after them (no second copy of the dequantized rows)
            T = 0 if self.keys is None else self.keys.shape[2]
            Kd = torch.empty(self._h_kv, P + T, self._d_head, dtype=dt, device=dev)
            Vd = torch.empty_like(Kd)
            spectral.dequant(self._dp, self._kpool, self._ktable[: P // spectral.GROUP], self._pool,
                             self._table[0, : P // k2b.PAGE_TOKENS].contiguous(), P, self._consts,
                             apply_rope=k2b.ROPE_FP16_TABLES, dtype=dt, out=(Kd, Vd))
            if T:
                Kd[:, P:].copy_(self.keys.squeeze(0))
                Vd[:, P:].copy_(self.values.squeeze(0))
            parts_k, parts_v = [Kd], [Vd]
        elif P > 0:
            kp, vp = k2b.dequant(self._pool, self._table[0, : P // k2b.PAGE_TOKENS].contiguous(), P,
                                 self._basis16, self._consts, h_kv=self._h_kv, rank=self._rank,
                                 apply_rope=k2b.ROPE_FP16_TABLES, dtype=dt)
            parts_k.append(kp)
            parts_v.append(vp)
        if self.keys is not None and self.keys.numel() and not (P > 0 and self._path == "spectral"):
            parts_k.append(self.keys.squeeze(0).to(dt))
            parts_v.append(self.values.squeeze(0).to(dt))
        Kd = torch.cat(parts_k, dim=1) if len(parts_k) > 1 else parts_k[0]
        Vd = torch.cat(parts_v, dim=1) if len(parts_v) > 1 else parts_v[0]
        n_q, n_kv = q.shape[1], Kd.shape[1]
        if causal and attention_mask is None and n_q != n_kv:
            i = torch.arange(n_q, device=dev)[:, None]
            j = torch.arange(n_kv, device=dev)[None, :]
            attention_mask = (j <= i + (n_kv - n_q))[None, None]
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


def _lib_v_page_bytes(h_kv: int) -> int:
    from . import _lib
    return _lib.lib().bmx_spectral_v_page_bytes(h_kv)


# ------------------------------------------------------------------ cache


class PackedStreamingCache(Cache):
    """Drop-in ``past_key_values=`` for ``model()`` / ``model.generate()``
    (packed_streaming.py:1067-1222).

        cache = PackedStreamingCache(model.config, *spec_pair("k2b_ph", rank=32))
        with cache.attach(model):
            out = model.generate(ids, past_key_values=cache, ...)
    """

    def __init__(self, model_config, k_spec: CacheCodecSpec, v_spec: CacheCodecSpec,
                 recent_window: int = 32, pack_v: bool = True, pack_k: bool = True):
        path = packed_path(k_spec, v_spec)
        # spectral: every layer's pack, loaded once (packed_streaming.py:1094-1147)
        self._packs = spectral.load_packs(k_spec.pack_path, k_spec.budget) if path == "spectral" else {}
        wself = weakref.proxy(self)   # no cache -> closure -> cache cycle

        def _make_layer():
            i = len(wself.layers)    # layers are made in order, layer i when len(layers) == i
            pack = None
            if path == "spectral":
                if i not in wself._packs:
                    raise KeyError(f"spectral pack file missing layer {i}")
                pack = wself._packs[i]
            return PackedStreamingLayer(wself.k_spec, wself.v_spec, wself.model_config,
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
        (streaming.py:154-260)."""
        layers = list(self.layers)
        if not layers:
            return float("nan"), float("nan")
        return (sum(l.bpe_k for l in layers) / len(layers), sum(l.bpe_v for l in layers) / len(layers))

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
            layer_ref = weakref.proxy(self.layers[i])

            def k_hook(module, inp, out, layer=layer_ref):
                layer.stash_pre_rope(out)

            self._handles.append(resolve_k_capture_module(mlayer.self_attn).register_forward_hook(k_hook))
        return self

    def detach(self) -> "PackedStreamingCache":
        for h in self._handles:
            h.remove()
        self._handles = []
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

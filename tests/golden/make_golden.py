"""Write the golden vectors that pin the CPU oracle to the reference's own code.

Run in the build container only (the reference tree is not present on the GPU
box):

    python tests/golden/make_golden.py /root/reference/src

It imports pherber3/bmx from the given ``src`` directory, runs the reference's
codec / attention / cache functions on small seeded inputs, and writes the inputs
and outputs as ``.npz`` fixtures next to this script.  Only data is written.

``bmx.decomp``'s package ``__init__`` imports ``tensorly`` for the CP/Tucker
baselines, which this image does not ship.  The hot path only needs
``bmx/decomp/lrs.py`` (``truncated_svd``) and ``bmx/decomp/base.py``, so the
script registers ``bmx.decomp`` as a bare package pointing at the real directory
(its ``__init__`` is not executed) and then imports those two real modules.

Functions covered (reference file:line, paths under ``src/bmx``):
  * gaussian_codebook            cache/codecs.py:346-380
  * _hadamard_signs              cache/codecs.py:114-124
  * fwht                         quant/hadamard.py:12-25
  * quantize_packed (k2b K, V, rtn arms)  cache/codecs.py:698-796
  * PackedStreamingLayer._pack_k_block frozen-subspace logic
                                 cache/packed_streaming.py:475-542
  * pack_codes / pack_signed_codes  cache/triton_dequant_attention.py:49-165
  * rope_cos_sin                 cache/rope.py:19-58
  * naive_dense_attention / chunked_dequant_attention
                                 cache/chunked_attention.py:254-317, 398-530
  * _tail_partial + merge math   cache/triton_dequant_attention.py:324-360, 409-461
  * PackedStreamingCache under HF generate (tiny Llama, head_dim 128)
                                 cache/packed_streaming.py:1067-1222
  * spectral K codec: fit_spectral_basis, pack_from_basis,
    allocate_bits_from_variance ("round"), tier_columns,
    spectral_quantize_packed / spectral_dequant_packed (rtn quantizer,
    mse_scale)                   cache/spectral.py:238-254, 421-485, 631-645,
                                 763-841; cache/codecs.py:203-287;
                                 quant/rtn.py:10-53

  * k4 variants: int8_decoder_roundtrip, int8_decoder_certificate_tiered,
    per_layer_tier_thresholds, the Lloyd payload (_lloyd_quantize_packed /
    _lloyd_dequantize_packed through spectral_quantize_packed /
    spectral_dequant_packed with quantizer="lloyd")
                                 cache/spectral.py:648-700, 763-841, 913-1027,
                                 1176-1210

  * full-C turboquant_mse values (quantize_packed / dequant_packed, arm
    "turboquant_mse")          cache/codecs.py:616-675, 729-735, 815-818

  * k2b codecs at other geometries (head_dim 32/64, rank 64, groups 16/32/128,
    2- and 4-bit keys) and PackedStreamingCache on a head_dim-64 tiny Llama
                               cache/codecs.py:616-649, 677-695, 786-796;
                               cache/packed_streaming.py:1067-1222

``python tests/golden/make_golden.py SRC spectral`` rewrites only the named
fixture files (codecs, attention, e2e_tiny_llama, spectral, spectral_variants,
tq_full, k2b_geom, e2e_tiny_llama_d64).
"""

from __future__ import annotations

import importlib
import math
import os
import sys
import types
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent


def _import_reference(src: str):
    src = os.path.abspath(src)
    sys.path.insert(0, src)
    import bmx  # noqa: F401  (top-level package, empty __init__)

    pkg = types.ModuleType("bmx.decomp")
    pkg.__path__ = [os.path.join(src, "bmx", "decomp")]
    sys.modules["bmx.decomp"] = pkg
    importlib.import_module("bmx.decomp.base")
    importlib.import_module("bmx.decomp.lrs")


def synthetic_k2b_keys(h_kv, S, d, rank, seed):
    """Pre-RoPE keys = U c + residual (per KV head), U a seeded-QR orthonormal basis."""
    g = torch.Generator().manual_seed(seed)
    out = torch.empty(h_kv, S, d)
    for h in range(h_kv):
        A = torch.randn(d, rank, generator=g)
        Q, R = torch.linalg.qr(A)
        sgn = torch.sign(torch.diagonal(R))
        sgn[sgn == 0] = 1
        U = Q * sgn
        std = torch.arange(1, rank + 1, dtype=torch.float32) ** (-0.35)
        c = torch.randn(S, rank, generator=g) * std
        out[h] = c @ U.T + 0.05 * torch.randn(S, d, generator=g)
    return out.half()


def codec_fixtures():
    from bmx.cache import codecs
    from bmx.cache.collect import to_matrix
    from bmx.cache.streaming import compute_flush_schedule
    from bmx.cache.triton_dequant_attention import pack_codes, pack_signed_codes
    from bmx.decomp.lrs import truncated_svd
    from bmx.quant.hadamard import fwht

    out = {}
    for b in (2, 3, 4):
        out[f"codebook_b{b}"] = codecs.gaussian_codebook(b).numpy()
    for s in (0, 7):
        out[f"signs_d128_s{s}"] = codecs._hadamard_signs(128, s).numpy().astype(np.int8)
    out["signs_d64_s0"] = codecs._hadamard_signs(64, 0).numpy().astype(np.int8)

    g = torch.Generator().manual_seed(11)
    x = torch.randn(8, 128, generator=g)
    out["fwht_in"] = x.numpy()
    out["fwht_out"] = fwht(x).numpy()

    # k2b pages: 3 codec pages of 128 tokens, h_kv=2, d=128 (C=256).
    h_kv, d, S, PAGE = 2, 128, 384, 128
    for rank in (16, 32):
        kpre = synthetic_k2b_keys(h_kv, S, d, rank, seed=100 + rank)
        gv = torch.Generator().manual_seed(200 + rank)
        v = torch.randn(h_kv, S, d, generator=gv).half()
        out[f"k2b_r{rank}_kpre"] = kpre.numpy()
        out[f"k2b_r{rank}_v"] = v.numpy()
        frozen = None
        for p in range(S // PAGE):
            M = to_matrix(kpre[:, p * PAGE:(p + 1) * PAGE, :].float())
            if frozen is None:  # packed_streaming.py:513-516
                Us, V = truncated_svd(M, rank)
                frozen = (Us, V)
                out[f"k2b_r{rank}_svd_us_fp32"] = Us.numpy()
                out[f"k2b_r{rank}_svd_v_fp32"] = V.numpy()
            else:  # :517-520
                Us = M @ frozen[1]
            kp, bpe_k = codecs.quantize_packed(
                "lowrank_rtn_channel", M, bits=3, group=64, rank=rank,
                svd_factors=(Us, frozen[1]), seed=0)
            pre = f"k2b_r{rank}_p{p}_"
            out[pre + "us"] = kp["Us"].numpy()
            out[pre + "v"] = kp["V"].numpy()
            out[pre + "res"] = kp["res_Q_int"].numpy()
            out[pre + "scale"] = kp["res_scale"].numpy()
            out[pre + "bpe_k"] = np.float64(bpe_k)
            Mv = to_matrix(v[:, p * PAGE:(p + 1) * PAGE, :].float())
            vp, bpe_v = codecs.quantize_packed(
                "turboquant_mse_perhead", Mv, bits=2, seed=0, h_heads=h_kv)
            out[pre + "vidx"] = vp["indices"].numpy()
            out[pre + "vnorm"] = vp["norms"].numpy()
            out[pre + "bpe_v"] = np.float64(bpe_v)
            if p == 0:
                out[pre + "vidx_packed"] = pack_codes(vp["indices"], 2).numpy()
                out[pre + "res_packed"] = pack_signed_codes(kp["res_Q_int"], 3).numpy()
                deq = codecs.dequant_packed("lowrank_rtn_channel", kp, group=64)
                out[pre + "kdeq"] = deq.numpy()
                vdeq = codecs.dequant_packed("turboquant_mse_perhead", vp, seed=0)
                out[pre + "vdeq"] = vdeq.numpy()

    # RTN arms (config-1 analogues): rtn_channel K 4b g32, rtn_token V 4b g32.
    g = torch.Generator().manual_seed(5)
    K = torch.randn(128, 256, generator=g)
    K[:, [3, 77, 130, 201]] *= 10.0
    Vv = torch.randn(128, 256, generator=g)
    out["rtn_k_in"] = K.numpy()
    out["rtn_v_in"] = Vv.numpy()
    kp, bk = codecs.quantize_packed("rtn_channel", K, bits=4, group=32)
    vp, bv = codecs.quantize_packed("rtn_token", Vv, bits=4, group=32)
    out["rtn_channel_q"] = kp["Q_int"].numpy()
    out["rtn_channel_scale"] = kp["scale"].numpy()
    out["rtn_channel_bpe"] = np.float64(bk)
    out["rtn_channel_deq"] = codecs.dequant_packed("rtn_channel", kp, group=32).numpy()
    out["rtn_token_q"] = vp["Q_int"].numpy()
    out["rtn_token_scale"] = vp["scale"].numpy()
    out["rtn_token_bpe"] = np.float64(bv)
    out["rtn_token_deq"] = codecs.dequant_packed("rtn_token", vp, group=32).numpy()

    sched = [(S, W, gq, compute_flush_schedule(S, W, gq))
             for S in (0, 31, 32, 33, 160, 161, 300, 4096, 65536 + 200)
             for W in (32, 128) for gq in (64, 128)]
    out["flush_schedule"] = np.array(sched, dtype=np.int64)
    return out


def attention_fixtures():
    from transformers import LlamaConfig

    from bmx.cache import codecs
    from bmx.cache.chunked_attention import chunked_dequant_attention, naive_dense_attention
    from bmx.cache.collect import to_matrix
    from bmx.cache.rope import rope_cos_sin
    from bmx.cache.triton_dequant_attention import _tail_partial
    from bmx.decomp.lrs import truncated_svd

    out = {}
    h_kv, G, d, PAGE, n_pages, T = 2, 4, 128, 128, 3, 40
    S = n_pages * PAGE
    for rank, vseed in ((16, 0), (32, 7)):
        cfg = LlamaConfig(hidden_size=h_kv * G * d, num_attention_heads=h_kv * G,
                          num_key_value_heads=h_kv, head_dim=d, rope_theta=500000.0,
                          max_position_embeddings=4096)
        cos, sin = rope_cos_sin(cfg, S + T)
        kpre = synthetic_k2b_keys(h_kv, S + T, d, rank, seed=300 + rank)
        gq = torch.Generator().manual_seed(400 + rank)
        v = torch.randn(h_kv, S + T, d, generator=gq).half()
        q = torch.randn(h_kv * G, 1, d, generator=gq)
        k_blocks, v_blocks, frozen = [], [], None
        for p in range(n_pages):
            M = to_matrix(kpre[:, p * PAGE:(p + 1) * PAGE, :].float())
            if frozen is None:
                frozen = truncated_svd(M, rank)
                Us = frozen[0]
            else:
                Us = M @ frozen[1]
            kp, _ = codecs.quantize_packed("lowrank_rtn_channel", M, bits=3, group=64,
                                           rank=rank, svd_factors=(Us, frozen[1]))
            Mv = to_matrix(v[:, p * PAGE:(p + 1) * PAGE, :].float())
            vp, _ = codecs.quantize_packed("turboquant_mse_perhead", Mv, bits=2,
                                           seed=vseed, h_heads=h_kv)
            k_blocks.append((kp, p * PAGE, (p + 1) * PAGE))
            v_blocks.append((vp, p * PAGE, (p + 1) * PAGE))
        # fp16 recent window: post-RoPE keys (HF applies RoPE in fp32, slab is fp16).
        k_tail = (kpre[:, S:, :].float() * cos[S:] +
                  torch.cat([-kpre[:, S:, d // 2:].float(), kpre[:, S:, :d // 2].float()],
                            dim=-1) * sin[S:]).half()
        v_tail = v[:, S:, :]
        kw = dict(k_arm="lowrank_rtn_channel", v_arm="turboquant_mse_perhead",
                  group=64, seed=0, k_pre_rope=True, rope_cos=cos, rope_sin=sin,
                  k_tail=k_tail, v_tail=v_tail, n_q_groups=G, scale=d ** -0.5,
                  v_group=64, v_seed=vseed)
        o_naive = naive_dense_attention(q, k_blocks, v_blocks, **kw)
        o_chunk = chunked_dequant_attention(q, k_blocks, v_blocks, **kw)
        # the packed cache's fp16 tables (packed_streaming.py:106-111)
        kw16 = dict(kw, rope_cos=cos.half(), rope_sin=sin.half())
        o_chunk16 = chunked_dequant_attention(q, k_blocks, v_blocks, **kw16)
        acc_t, m_t, lse_t = _tail_partial(q.view(h_kv, G, d), k_tail, v_tail, d ** -0.5)
        pre = f"attn_r{rank}_"
        out[pre + "kpre"] = kpre.numpy()
        out[pre + "v"] = v.numpy()
        out[pre + "q"] = q.numpy()
        out[pre + "k_tail"] = k_tail.numpy()
        pos = np.arange(0, S + T, 7)
        out[pre + "rope_pos"] = pos
        out[pre + "cos"] = cos[pos].numpy()
        out[pre + "sin"] = sin[pos].numpy()
        out[pre + "vseed"] = np.int64(vseed)
        out[pre + "naive"] = o_naive.numpy()
        out[pre + "chunked"] = o_chunk.numpy()
        out[pre + "chunked_fp16rope"] = o_chunk16.numpy()
        out[pre + "tail_acc"] = acc_t.numpy()
        out[pre + "tail_m"] = m_t.numpy()
        out[pre + "tail_lse"] = lse_t.numpy()
        out[pre + "svd_us"] = frozen[0].numpy()
        out[pre + "svd_v"] = frozen[1].numpy()
    return out


def tiny_model_config():
    from transformers import LlamaConfig

    return LlamaConfig(
        vocab_size=256, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
        num_attention_heads=4, num_key_value_heads=2, head_dim=128,
        max_position_embeddings=4096, rope_theta=500000.0, initializer_range=0.1)


def e2e_fixtures():
    from transformers import LlamaForCausalLM

    from bmx.cache.packed_streaming import PackedStreamingCache
    from bmx.cache.recipes import spec_pair

    cfg = tiny_model_config()
    torch.manual_seed(0)
    model = LlamaForCausalLM(cfg).eval()
    g = torch.Generator().manual_seed(1)
    ids = torch.randint(0, cfg.vocab_size, (1, 300), generator=g)
    out = {"prompt": ids.numpy()}
    for rank in (16, 32):
        k_spec, v_spec = spec_pair("k2b_ph", rank=rank)
        cache = PackedStreamingCache(cfg, k_spec, v_spec, recent_window=32)
        cache.attach(model)
        with torch.no_grad():
            res = model.generate(ids, past_key_values=cache, max_new_tokens=140, min_new_tokens=140,
                                 do_sample=False, output_logits=True,
                                 return_dict_in_generate=True, pad_token_id=0)
        bpe = cache.bits_per_entry()
        cache.detach()
        out[f"r{rank}_tokens"] = res.sequences.numpy()
        out[f"r{rank}_logits"] = torch.stack(res.logits, 0).squeeze(1).numpy()
        out[f"r{rank}_bpe"] = np.array(bpe, dtype=np.float64)
    return out


def spectral_fixtures():
    """A spectral pack fitted by the reference on seeded synthetic keys with a
    non-identity weighting (enc != dec), h_kv 2 (C 256), group 64, and the
    packed codes, scales and dequantization of 4 groups of keys."""
    from bmx.cache import codecs
    from bmx.cache.spectral import (
        _unpack_tier_codes,
        fit_spectral_basis,
        pack_from_basis,
        spectral_dequant_packed,
        spectral_quantize_packed,
        tier_columns,
    )

    g = torch.Generator().manual_seed(23)
    C, S = 256, 256
    lam_true = 40.0 * torch.arange(1, C + 1, dtype=torch.float64) ** -1.3
    Q, _ = torch.linalg.qr(torch.randn(C, C, generator=g, dtype=torch.float64))
    mix = (Q * lam_true.sqrt()).mT            # rows of keys: z @ mix
    M_fit = (torch.randn(1024, C, generator=g, dtype=torch.float64) @ mix).float()
    w = 0.5 + torch.rand(C, generator=g, dtype=torch.float64)
    Wh, Wh_inv = torch.diag(w.sqrt()), torch.diag(w.rsqrt())
    basis = fit_spectral_basis(M_fit, Wh, Wh_inv)
    out = {"enc": basis.enc.numpy(), "dec": basis.dec.numpy(), "lam64": basis.lam64.numpy()}
    for budget in (2.0, 2.5, 3.0):
        b = codecs.allocate_bits_from_variance(basis.lam64, budget, (0, 2, 3, 4, 5, 6, 8))
        out[f"bits_b{budget}"] = b.numpy()
    pack = pack_from_basis(basis, 2.5, group=64)
    assert np.array_equal(pack.bits.numpy(), out["bits_b2.5"])
    M = (torch.randn(S, C, generator=g, dtype=torch.float64) @ mix).float()
    out["M"] = M.numpy()
    out["Y"] = (M @ pack.enc).numpy()
    cols = tier_columns(pack.bits)
    packed, bpe = spectral_quantize_packed(M, pack, mse_scale=True, cols_by_tier=cols)
    out["bpe"] = np.float64(bpe)
    for b, c in cols.items():
        out[f"cols_t{b}"] = c.numpy()
        out[f"codes_t{b}"] = _unpack_tier_codes(packed[f"t{b}_codes"], b, S).numpy()
        out[f"scale_t{b}"] = packed[f"t{b}_scale"].numpy()
    out["M_hat"] = spectral_dequant_packed(packed, pack, cols_by_tier=cols).numpy()
    return out


def spectral_variant_fixtures():
    """The k4 recipe variants on spectral.npz's pack (refitted from the same
    seeds): the int8 decoder roundtrip (blanket and tier-gated), the tiered
    int8 certificate and the per-layer thresholds it picks, and the Lloyd
    payload (Gaussian Lloyd-Max codebooks per tier, codes, scales and the
    dequantized keys of spectral.npz's keys)."""
    from bmx.cache import codecs
    from bmx.cache.spectral import (
        TIER_THRESHOLD_GRID,
        _unpack_tier_codes,
        fit_spectral_basis,
        int8_decoder_certificate_tiered,
        int8_decoder_roundtrip,
        pack_from_basis,
        per_layer_tier_thresholds,
        spectral_dequant_packed,
        spectral_quantize_packed,
        tier_columns,
    )

    g = torch.Generator().manual_seed(23)
    C, S = 256, 256
    lam_true = 40.0 * torch.arange(1, C + 1, dtype=torch.float64) ** -1.3
    Q, _ = torch.linalg.qr(torch.randn(C, C, generator=g, dtype=torch.float64))
    mix = (Q * lam_true.sqrt()).mT
    M_fit = (torch.randn(1024, C, generator=g, dtype=torch.float64) @ mix).float()
    w = 0.5 + torch.rand(C, generator=g, dtype=torch.float64)
    Wh, Wh_inv = torch.diag(w.sqrt()), torch.diag(w.rsqrt())
    basis = fit_spectral_basis(M_fit, Wh, Wh_inv)
    pack = pack_from_basis(basis, 2.5, group=64)
    pack3 = pack_from_basis(basis, 3.0, group=64)
    M = (torch.randn(S, C, generator=g, dtype=torch.float64) @ mix).float()
    out = {"M": M.numpy(), "Y": (M @ pack.enc.to(M.dtype)).numpy(),
           "dec": pack.dec.numpy(), "enc": pack.enc.numpy(), "lam": pack.lam.numpy(),
           "bits_b2.5": pack.bits.numpy(), "bits_b3.0": pack3.bits.numpy()}
    for t in (None, 3, 5):
        out[f"dec8_t{t or 'all'}"] = int8_decoder_roundtrip(pack.dec, pack.bits, tier_threshold=t).numpy()
    for t in TIER_THRESHOLD_GRID:
        cert = int8_decoder_certificate_tiered(pack, t)
        out[f"cert_b2.5_t{t}"] = np.array([cert["added"], cert["payload"], cert["implied_rel_degradation"]])
    for bar in (0.05, 0.001, 1e-5):
        thr = per_layer_tier_thresholds({0: pack, 1: pack3}, bar=bar)
        out[f"layer_thr_bar{bar:g}"] = np.array([thr[0], thr[1]], dtype=np.int64)
    for b in (2, 3, 4, 5, 6, 8):
        out[f"codebook_{b}"] = codecs.gaussian_codebook(b).numpy()
    cols = tier_columns(pack.bits)
    packed, _ = spectral_quantize_packed(M, pack, cols_by_tier=cols, quantizer="lloyd")
    for b, c in cols.items():
        out[f"lq_codes_t{b}"] = _unpack_tier_codes(packed[f"t{b}_codes"], b, S, quantizer="lloyd").numpy()
        out[f"lq_scale_t{b}"] = packed[f"t{b}_scale"].numpy()
    out["lq_M_hat"] = spectral_dequant_packed(packed, pack, cols_by_tier=cols, quantizer="lloyd").numpy()
    return out


def tq_full_fixtures():
    """The full-C turboquant_mse value codec (the k4 recipe's values): one
    Hadamard over all C = 128 h_kv channels and one norm per token, at
    h_kv 2 and 8, on fp16 values as the cache passes them; indices, norms,
    the dequantized values and the C-wide signs."""
    from bmx.cache import codecs
    from bmx.cache.collect import to_matrix

    out = {}
    g = torch.Generator().manual_seed(31)
    for h_kv in (2, 8):
        C = 128 * h_kv
        v = (torch.randn(h_kv, 96, 128, generator=g) * 1.5).half()
        M = to_matrix(v.float())
        packed, bpe = codecs.quantize_packed("turboquant_mse", M, bits=2, seed=0)
        out[f"h{h_kv}_v"] = v.numpy()
        out[f"h{h_kv}_idx"] = packed["indices"].numpy()
        out[f"h{h_kv}_norms"] = packed["norms"].numpy()
        out[f"h{h_kv}_bpe"] = np.float64(bpe)
        out[f"h{h_kv}_deq"] = codecs.dequant_packed("turboquant_mse", packed, seed=0).numpy()
        out[f"signs_d{C}_s0"] = codecs._hadamard_signs(C, 0).numpy().astype(np.int8)
    return out


# name, h_kv, head_dim, rank, residual group, key bits, value seed
GEOM_CASES = [
    ("d64_r16_g32", 2, 64, 16, 32, 3, 7),        # the reference's k2b test geometry (n_q 8, G 4)
    ("d128_r64_g64", 2, 128, 64, 64, 3, 0),      # spec_pair("k2b_ph", rank=64)
    ("d32_r16_g16_b2", 4, 32, 16, 16, 2, 3),
    ("d128_r32_g128_b4", 2, 128, 32, 128, 4, 0),
]


def k2b_geometry_fixtures():
    """The k2b codecs at geometries other than head_dim 128 / group 64 / 3 bits
    / rank 16|32: three 128-token codec pages per case, frozen basis from the
    first (packed_streaming.py:513-520), quantize_packed for keys and values
    (codecs.py:616-636, 677-695, 786-796)."""
    from bmx.cache import codecs
    from bmx.cache.collect import to_matrix
    from bmx.decomp.lrs import truncated_svd

    out = {}
    S, PAGE = 384, 128
    for name, h_kv, d, rank, group, bits, vseed in GEOM_CASES:
        kpre = synthetic_k2b_keys(h_kv, S, d, min(rank, d), seed=300 + d + rank)
        gv = torch.Generator().manual_seed(400 + d + rank)
        v = torch.randn(h_kv, S, d, generator=gv).half()
        out[f"{name}_kpre"] = kpre.numpy()
        out[f"{name}_v"] = v.numpy()
        out[f"{name}_signs"] = codecs._hadamard_signs(d, vseed).numpy().astype(np.int8)
        frozen = None
        for p in range(S // PAGE):
            M = to_matrix(kpre[:, p * PAGE:(p + 1) * PAGE].float())
            if frozen is None:
                Us, V = truncated_svd(M, rank)
                frozen = (Us, V)
                out[f"{name}_svd_us_fp32"] = Us.numpy()
                out[f"{name}_svd_v_fp32"] = V.numpy()
            else:
                Us = M @ frozen[1]
            kp, bpe_k = codecs.quantize_packed(
                "lowrank_rtn_channel", M, bits=bits, group=group, rank=rank,
                svd_factors=(Us, frozen[1]), seed=0)
            pre = f"{name}_p{p}_"
            out[pre + "us"] = kp["Us"].numpy()
            out[pre + "res"] = kp["res_Q_int"].numpy()
            out[pre + "scale"] = kp["res_scale"].numpy()
            out[pre + "bpe_k"] = np.float64(bpe_k)
            Mv = to_matrix(v[:, p * PAGE:(p + 1) * PAGE].float())
            vp, bpe_v = codecs.quantize_packed("turboquant_mse_perhead", Mv, bits=2, seed=vseed, h_heads=h_kv)
            out[pre + "vidx"] = vp["indices"].numpy()
            out[pre + "vnorm"] = vp["norms"].numpy()
            out[pre + "bpe_v"] = np.float64(bpe_v)
            if p == 0:
                out[pre + "kdeq"] = codecs.dequant_packed("lowrank_rtn_channel", kp, group=group).numpy()
                out[pre + "vdeq"] = codecs.dequant_packed("turboquant_mse_perhead", vp, seed=vseed).numpy()
    return out


def e2e_d64_fixtures():
    """The reference's PackedStreamingCache under HF generate on a tiny Llama
    with head_dim 64, k2b_ph at rank 16 and residual group 32
    (packed_streaming.py:1067-1222, recipes.py:31-42)."""
    from transformers import LlamaConfig, LlamaForCausalLM

    from bmx.cache.packed_streaming import PackedStreamingCache
    from bmx.cache.recipes import spec_pair

    cfg = LlamaConfig(vocab_size=256, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                      num_attention_heads=8, num_key_value_heads=2, head_dim=64,
                      max_position_embeddings=4096, rope_theta=500000.0, initializer_range=0.1)
    torch.manual_seed(0)
    model = LlamaForCausalLM(cfg).eval()
    g = torch.Generator().manual_seed(1)
    ids = torch.randint(0, cfg.vocab_size, (1, 300), generator=g)
    out = {"prompt": ids.numpy()}
    k_spec, v_spec = spec_pair("k2b_ph", rank=16, group=32)
    cache = PackedStreamingCache(cfg, k_spec, v_spec, recent_window=32)
    cache.attach(model)
    with torch.no_grad():
        res = model.generate(ids, past_key_values=cache, max_new_tokens=140, min_new_tokens=140,
                             do_sample=False, output_logits=True,
                             return_dict_in_generate=True, pad_token_id=0)
    bpe = cache.bits_per_entry()
    cache.detach()
    out["tokens"] = res.sequences.numpy()
    out["logits"] = torch.stack(res.logits, 0).squeeze(1).numpy()
    out["bpe"] = np.array(bpe, dtype=np.float64)
    return out


FIXTURES = {"codecs": codec_fixtures, "attention": attention_fixtures,
            "e2e_tiny_llama": e2e_fixtures, "spectral": spectral_fixtures,
            "spectral_variants": spectral_variant_fixtures, "tq_full": tq_full_fixtures,
            "k2b_geom": k2b_geometry_fixtures, "e2e_tiny_llama_d64": e2e_d64_fixtures}


def main():
    src = sys.argv[1] if len(sys.argv) > 1 else "/root/reference/src"
    names = sys.argv[2:] or list(FIXTURES)
    torch.set_num_threads(min(8, os.cpu_count() or 1))
    _import_reference(src)
    for name in names:
        np.savez_compressed(HERE / f"{name}.npz", **FIXTURES[name]())
    for f in sorted(HERE.glob("*.npz")):
        print(f.name, f.stat().st_size)


if __name__ == "__main__":
    main()

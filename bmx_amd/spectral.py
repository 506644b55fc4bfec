"""Spectral (K4) key path: host side of the C-ABI in include/bmx_spectral.h.

A corpus-fitted pack per layer (cache/spectral.py:175-215, ``SpectralPack``:
enc, dec (C x C fp32), lam, bits per direction on the tier grid, group 64)
codes the pre-RoPE keys; the values use the k2b value codec in value-only
pages (the per-head codec, or the full-C turboquant_mse of the reference's
k4 recipe).  ``DevicePack`` holds what the kernels read: the page layout of
the pack's bits, enc's columns and dec's rows in page order.  ``append`` writes
64-token groups; ``dequant`` reads them back dense (the reference's spectral
read path: chunked_attention.py:106-116, then RoPE).

Pack files: the reference's format (spectral.py:1081-1170, save_pack_file /
load_packs), a safetensors file of ``layer{i}.enc / .dec / .lam /
.bits_b{budget:g}`` and a JSON sidecar ``<path>.json`` with tiers, group and
budgets.
"""

from __future__ import annotations

import ctypes as ct
import dataclasses
import json
import math
from dataclasses import dataclass
from pathlib import Path

import numpy as np
import torch

from . import _lib
from .k2b import _V_DTYPES, HEAD_DIM, ROPE_NONE, CodecConsts, _need, _ptr, _stream

TIERS = (0, 2, 3, 4, 5, 6, 8)
GROUP = 64
_CONTAINER = {2: 2, 3: 4, 4: 4, 5: 8, 6: 8, 8: 8}
MAX_CPAD = 1072


@dataclass
class SpectralPack:
    """One layer's pack (spectral.py:175-215): Y = M enc, M_hat = Y_hat dec^T."""

    enc: torch.Tensor
    dec: torch.Tensor
    lam: torch.Tensor
    bits: torch.Tensor
    group: int = GROUP
    tiers: tuple = TIERS
    budget: float = float("nan")
    dec_tier: int | None = None       # the int8 threshold dec was roundtripped at (None: fp32 as loaded)

    @property
    def c_used(self) -> int:
        return int((self.bits != 0).sum())

    def c_int8(self, tier_threshold: int) -> int:
        """Coded directions whose tier is at most tier_threshold: the decoder
        columns an int8 decoder at that threshold stores (spectral.py:213-220)."""
        return int(((self.bits > 0) & (self.bits <= tier_threshold)).sum())


def allocate_bits(var, budget: float, tiers=TIERS, n_search: int = 40) -> torch.Tensor:
    """Reverse water-filling of a per-direction variance onto the tier grid,
    midpoint rounding (allocate_bits_from_variance, selection "round",
    codecs.py:203-287): bisect log(kappa) for the smallest kappa whose mean
    rounded rate 0.5 log2(var / kappa) stays within the budget."""
    var = np.maximum(np.asarray(torch.as_tensor(var, dtype=torch.float64)), 1e-30)
    grid = np.array(sorted(tiers), dtype=np.float64)

    def rounded(kappa):
        b = np.maximum(0.5 * np.log2(var / kappa), 0.0)
        return grid[np.abs(b[:, None] - grid[None, :]).argmin(axis=1)]

    lo_k, hi_k = float(var.min()) * 1e-6, float(var.max()) * 1e6
    lo, hi = math.log(lo_k), math.log(hi_k)
    best = rounded(hi_k)
    for _ in range(n_search):
        mid = 0.5 * (lo + hi)
        b = rounded(math.exp(mid))
        if b.mean() <= budget + 1e-12:
            best, hi = b, mid
        else:
            lo = mid
    return torch.from_numpy(best.astype(np.int64))


def payload_bpe(bits: torch.Tensor, group: int = GROUP) -> float:
    """Model-level payload bits per entry: mean(bits) + (16 / group) c_used / C
    (spectral_payload_bpe, spectral.py:602-615)."""
    C = bits.shape[0]
    return float(bits.float().mean()) + 16.0 / group * int((bits != 0).sum()) / C


TIER_THRESHOLD_GRID = (2, 3, 4, 5, 6, 8)
PER_LAYER_TIER = -1   # dec_quant "int8_tl": a threshold per layer, from each pack's certificate


def dec_quant_threshold(dec_quant: str) -> int | None:
    """The int8 tier threshold a ``dec_quant`` string names (spectral.py:
    1213-1250): "fp32" -> None (no int8 decoder), "int8" -> 8 (every coded
    column), "int8_t{T}" -> T for 2 <= T <= 8, "int8_tl" -> PER_LAYER_TIER."""
    if dec_quant == "fp32":
        return None
    if dec_quant == "int8":
        return 8
    if dec_quant == "int8_tl":
        return PER_LAYER_TIER
    t = dec_quant[len("int8_t"):] if dec_quant.startswith("int8_t") else ""
    if not t.isdigit() or not 2 <= int(t) <= 8:
        raise ValueError(f"dec_quant must be 'fp32', 'int8', 'int8_tl' or 'int8_t<T>' with 2 <= T <= 8; "
                         f"got {dec_quant!r}")
    return int(t)


def int8_decoder_roundtrip(dec: torch.Tensor, bits: torch.Tensor, tier_threshold: int | None = None) -> torch.Tensor:
    """The decoder as an int8 store would give it back (spectral.py:913-944):
    each selected column c (bits[c] != 0, and bits[c] <= tier_threshold when
    one is given) becomes q * s with s = fp16(max|dec[:, c]| / 127, floored at
    1e-12) and q = round-half-even(dec[:, c] / s) clamped to [-127, 127], all
    in fp32; the other columns are returned unchanged."""
    dec = dec.float()
    bits = bits.to(device=dec.device)
    sel = bits != 0
    if tier_threshold is not None:
        sel = sel & (bits <= tier_threshold)
    out = dec.clone()
    cols = dec[:, sel]
    s = (cols.abs().amax(dim=0) / 127.0).clamp_min(1e-12).half().float()
    out[:, sel] = torch.round(cols / s).clamp(-127.0, 127.0) * s
    return out


def int8_certificate(pack: SpectralPack, tier_threshold: int) -> dict:
    """Closed-form weighted distortion an int8 decoder at tier_threshold adds
    (spectral.py:947-960, 1004-1033), in float64: with D = dec_int8 - dec,
    added = sum_c lam_c |enc^T D[:, c]|^2, payload = sum_c lam_c 4^-bits_c,
    implied_rel_degradation = added / (payload + added)."""
    D = int8_decoder_roundtrip(pack.dec, pack.bits, tier_threshold).double() - pack.dec.double()
    lam = pack.lam.double().clamp_min(0.0)
    added = float((lam * ((pack.enc.double().T @ D) ** 2).sum(dim=0)).sum())
    payload = float((lam * torch.pow(4.0, -pack.bits.double())).sum())
    return {"tier_threshold": int(tier_threshold), "c_used": pack.c_used, "c_int8": pack.c_int8(tier_threshold),
            "added": added, "payload": payload, "noise_to_signal": added / max(payload, 1e-300),
            "implied_rel_degradation": added / max(payload + added, 1e-300)}


def per_layer_tier_thresholds(packs: dict, bar: float = 0.05) -> dict:
    """{layer: T}: the last threshold of TIER_THRESHOLD_GRID (scanned in
    ascending order) whose certificate keeps implied_rel_degradation <= bar,
    0 when none does (spectral.py:1176-1210).  Pass the packs as loaded: a
    decoder already roundtripped certifies almost anything."""
    out = {}
    for i, pack in packs.items():
        out[i] = 0
        for t in TIER_THRESHOLD_GRID:
            if int8_certificate(pack, t)["implied_rel_degradation"] <= bar:
                out[i] = t
    return out


def tier_bits(tiers, S: int) -> float:
    """The tier map's charge per entry: ceil(log2(n_tiers)) bits per channel
    over S rows (codecs.py:94-96)."""
    return math.ceil(math.log2(len(tiers))) / S


def mixed_dec_charge(C: int, S: int, tiers, c_used: float, c_int8: float) -> float:
    """Per-entry charge of the decoder and tier map over S rows with c_int8
    of the c_used coded columns stored int8 (8 bits per entry and one fp16
    scale per column) and the rest fp16 (spectral.py:1036-1064)."""
    if not 0 <= c_int8 <= c_used <= C:
        raise ValueError(f"need 0 <= c_int8 <= c_used <= C; got {c_int8}, {c_used}, {C}")
    return 8.0 * c_int8 / S + 16.0 * c_int8 / (S * C) + 16.0 * (c_used - c_int8) / S + tier_bits(tiers, S)


def load_packs_for_spec(k_spec) -> dict:
    """{layer: SpectralPack} a cache holds for a spectral key spec
    (spectral.py:1254-1326): the pack file's layers at the spec's budget,
    with each decoder int8-roundtripped once here when dec_quant asks for it
    and dec_tier set to the threshold applied.  "int8_tl" takes each layer's
    threshold from per_layer_tier_thresholds of the packs as loaded; a layer
    whose threshold is 0 keeps its fp32 decoder.  Other arms: {}."""
    thr = dec_quant_threshold(k_spec.dec_quant)
    if k_spec.arm != "spectral":
        return {}
    if not k_spec.pre_rope or not k_spec.pack_path:
        raise ValueError("a spectral key spec needs pre_rope=True and a pack_path")
    packs = load_packs(k_spec.pack_path, k_spec.budget)
    if thr is None:
        return packs
    t_map = per_layer_tier_thresholds(packs) if thr == PER_LAYER_TIER else {i: thr for i in packs}
    return {i: p if t_map[i] == 0 else
            dataclasses.replace(p, dec=int8_decoder_roundtrip(p.dec, p.bits, t_map[i]), dec_tier=t_map[i])
            for i, p in packs.items()}


def load_packs(path, budget: float) -> dict:
    """{layer: SpectralPack} of one budget from a pack file (load_packs,
    spectral.py:1137-1170); KeyError names the budgets the file holds."""
    from safetensors.torch import load_file

    side = json.loads(Path(str(path) + ".json").read_text())
    if budget not in side["budgets"]:
        raise KeyError(f"budget {budget} not in pack file; available: {side['budgets']}")
    t = load_file(str(path))
    layers = sorted({int(k.split(".")[0].removeprefix("layer")) for k in t if "." in k})
    return {i: SpectralPack(enc=t[f"layer{i}.enc"], dec=t[f"layer{i}.dec"], lam=t[f"layer{i}.lam"],
                            bits=t[f"layer{i}.bits_b{budget:g}"], group=int(side["group"]),
                            tiers=tuple(side["tiers"]), budget=float(budget))
            for i in layers}


def save_packs(path, layers: dict, budgets, *, tiers=TIERS, group: int = GROUP) -> None:
    """Write {layer: (enc, dec, lam, {budget: bits})} in the pack-file format."""
    from safetensors.torch import save_file

    t = {}
    for i, (enc, dec, lam, bits) in layers.items():
        t[f"layer{i}.enc"], t[f"layer{i}.dec"], t[f"layer{i}.lam"] = enc, dec, lam
        for b in budgets:
            t[f"layer{i}.bits_b{b:g}"] = bits[b]
    save_file({k: v.contiguous() for k, v in t.items()}, str(path))
    Path(str(path) + ".json").write_text(json.dumps({"tiers": list(tiers), "group": group,
                                                     "budgets": list(budgets)}))


V_CODECS = {"perhead": 0, "full": 1}   # BMX_SPECTRAL_V_PERHEAD, BMX_SPECTRAL_V_FULL


def v_page_bytes(h_kv: int, v_codec: str = "perhead") -> int:
    """Bytes of a 16-token value page of the value codec: "perhead"
    (turboquant_mse_perhead) or "full" (the full-C turboquant_mse)."""
    n = int(_lib.lib().bmx_spectral_v_page_bytes_codec(h_kv, V_CODECS[v_codec]))
    _need(n > 0, f"no {v_codec} value pages for h_kv {h_kv}")
    return n


def v_sign_bits_c(h_kv: int, seed: int) -> tuple:
    """The full-C codec's Hadamard signs of the C = 128 h_kv channels as 32
    uint32 words (_hadamard_signs(C, seed), codecs.py:114-124)."""
    from .codecs import hadamard_signs, sign_bits

    w = sign_bits(hadamard_signs(HEAD_DIM * h_kv, seed))
    return tuple(w + [0] * (32 - len(w)))


def _set_v_codec(a, dp) -> None:
    a.v_codec = dp.v_codec
    a.v_sign_bits_c[:] = dp.v_sign_c


LLOYD_TIERS = (2, 3, 4, 5, 6, 8)


def lloyd_levels(device) -> torch.Tensor:
    """The Lloyd payload's level table (include/bmx_spectral.h): the sorted
    levels of gaussian_codebook(b) for b = 2, 3, 4, 5, 6, 8 back to back, fp32
    (the codebook the reference's _lloyd_quantize_packed codes against,
    spectral.py:648-684)."""
    from .codecs import gaussian_codebook

    t = torch.tensor([v for b in LLOYD_TIERS for v in gaussian_codebook(b)], dtype=torch.float32)
    assert t.numel() == 380
    return t.to(device)


class DevicePack:
    """A pack's page layout and kernel operands on one device.

    Columns: the coded directions in tier order (tier ascending, direction
    ascending: tier_columns, spectral.py:631-645), each tier padded with zero
    directions to a multiple of 8 (c_pad columns).  Slice s (8 columns) of
    tier b has a w-bit container, w = 2 / 4 / 8 (tiers 2 / 3-4 / 5-8), 64 w
    bytes per page at off[s] after the fp16 scales."""

    def __init__(self, pack: SpectralPack, h_kv: int, device, payload: str = "rtn", v_codec: str = "perhead",
                 v_seed: int = 0):
        if payload not in ("rtn", "lloyd"):
            raise ValueError(f"payload must be 'rtn' or 'lloyd'; got {payload!r}")
        if v_codec not in V_CODECS:
            raise ValueError(f"v_codec must be 'perhead' or 'full'; got {v_codec!r}")
        if v_codec == "full" and h_kv not in (1, 2, 4, 8):
            # the reference rotates a non-power-of-two C with a seeded random
            # orthogonal matrix (codecs.py:104-111), which no kernel here reads
            raise NotImplementedError(f"full-C turboquant_mse values need C = 128 h_kv a power of two; h_kv {h_kv}")
        if pack.group != GROUP:
            raise NotImplementedError(f"pack group {pack.group}: the spectral kernels take 64-token groups")
        bits = pack.bits.to(torch.int64).cpu()
        C = HEAD_DIM * h_kv
        _need(tuple(pack.enc.shape) == (C, C) and tuple(pack.dec.shape) == (C, C) and bits.shape[0] == C,
              f"pack shapes must be ({C}, {C}) with {C} bits for h_kv {h_kv}")
        bad = set(bits.tolist()) - set(TIERS)
        if bad:
            raise NotImplementedError(f"tiers {sorted(bad)}: the kernels take tiers {TIERS}")
        perm, slice_bits = [], []
        for b in sorted(set(bits.tolist()) - {0}):
            cols = torch.nonzero(bits == b).flatten().tolist()
            n_pad = -(-len(cols) // 8) * 8
            perm += cols + [-1] * (n_pad - len(cols))
            slice_bits += [b] * (n_pad // 8)
        _need(len(perm) > 0, "the pack codes no direction")
        self.h_kv, self.C, self.c_pad = h_kv, C, len(perm)
        if self.c_pad > MAX_CPAD:
            raise NotImplementedError(f"c_pad {self.c_pad} above {MAX_CPAD}")
        self.c_pad32 = -(-self.c_pad // 32) * 32
        widths = [_CONTAINER[b] for b in slice_bits]
        off, o = [], 2 * self.c_pad
        for w in widths:
            off.append(o)
            o += GROUP * w
        self.k_page_bytes = o + 16
        self.v_codec = V_CODECS[v_codec]
        self.v_page_bytes = v_page_bytes(h_kv, v_codec)
        self.v_sign_c = v_sign_bits_c(h_kv, v_seed) if v_codec == "full" else (0,) * 32
        self.perm = torch.tensor(perm, dtype=torch.int64)
        self.slice_bits = slice_bits
        tab = [x | (b << 24) for x, b in zip(off, slice_bits)]
        self.slice_tab = torch.tensor(tab, dtype=torch.int32, device=device)
        keep = self.perm >= 0
        encp = torch.zeros(C, self.c_pad, dtype=torch.float32)
        encp[:, keep] = pack.enc.float().cpu()[:, self.perm[keep]]
        decp = torch.zeros(C, self.c_pad32, dtype=torch.float32)
        decp[:, : self.c_pad][:, keep] = pack.dec.float().cpu()[:, self.perm[keep]]
        self.enc_perm = encp.to(device).contiguous()
        # tiled for the dequant kernel: [h][c_pad32 / 32][8][16][32], one contiguous
        # (16 rows x 32 columns) tile per (head, 32-column step, 16-row tile)
        self.dec_perm = (decp.half().view(h_kv, 8, 16, self.c_pad32 // 32, 32).permute(0, 3, 1, 2, 4)
                         .contiguous().to(device))
        self.bpe = payload_bpe(bits, pack.group)
        self.payload = payload
        self.lloyd_levels = lloyd_levels(device) if payload == "lloyd" else None

    def layout(self) -> _lib.SpectralLayout:
        return _lib.SpectralLayout(self.h_kv, self.c_pad, self.k_page_bytes, _ptr(self.slice_tab),
                                   _ptr(self.lloyd_levels) if self.lloyd_levels is not None else None)


def append(k_pre: torch.Tensor, v: torch.Tensor, dp: DevicePack, k_pages: torch.Tensor,
           k_ids: torch.Tensor, v_pages: torch.Tensor, v_ids: torch.Tensor, consts: CodecConsts) -> None:
    """Write 64n tokens: k_pre, v (h_kv, 64n, 128) on the device (fp16, bf16 or
    fp32; innermost stride 1) into key pages k_ids (n) and value pages v_ids (4n)."""
    dev = v.device
    h_kv, S, d = k_pre.shape
    _need(d == HEAD_DIM and h_kv == dp.h_kv and tuple(v.shape) == (h_kv, S, d), "k_pre, v must be (h_kv, S, 128)")
    _need(S % GROUP == 0, "S must be a multiple of 64")
    _need(k_pre.stride(2) == 1 and v.stride(2) == 1, "innermost stride must be 1")
    _need(k_pre.dtype in _V_DTYPES and v.dtype in _V_DTYPES, "keys and values must be fp16, bf16 or fp32")
    n = S // GROUP
    _need(k_ids.dtype == torch.int32 and k_ids.numel() >= n and v_ids.dtype == torch.int32
          and v_ids.numel() >= 4 * n, "k_ids (n) and v_ids (4n) must be int32")
    _need(k_pages.shape[1] == dp.k_page_bytes and v_pages.shape[1] == dp.v_page_bytes, "pool page sizes")
    a = _lib.SpectralAppendArgs()
    a.L = dp.layout()
    a.n_groups = n
    a.k_pre, a.k_dtype, a.k_sh, a.k_st = _ptr(k_pre), _V_DTYPES[k_pre.dtype], k_pre.stride(0), k_pre.stride(1)
    a.v, a.v_dtype, a.v_sh, a.v_st = _ptr(v), _V_DTYPES[v.dtype], v.stride(0), v.stride(1)
    a.enc_perm = _ptr(dp.enc_perm)
    a.k_pages, a.k_page_ids, a.n_k_pool = _ptr(k_pages), _ptr(k_ids), k_pages.shape[0]
    a.v_pages, a.v_page_ids, a.n_v_pool = _ptr(v_pages), _ptr(v_ids), v_pages.shape[0]
    a.v_codebook[:] = consts.codebook
    a.v_sign_bits[:] = consts.sign_bits
    _set_v_codec(a, dp)
    _lib.check(_lib.lib().bmx_spectral_append(ct.byref(a), _stream(dev)), "bmx_spectral_append")


def _partial_args(dp: DevicePack, k_pages, k_table, v_pages, v_table, n_tokens: int, consts: CodecConsts,
                  q: torch.Tensor, apply_rope: int, sm_scale: float):
    """Arguments of the dequant kernel's partial form, partials not yet set."""
    _need(q.dim() == 3 and q.shape[0] == dp.h_kv and q.shape[2] == HEAD_DIM and 1 <= q.shape[1] <= 16
          and q.is_contiguous() and q.dtype in _V_DTYPES, "q must be contiguous (h_kv, 1..16, 128)")
    _need(int(apply_rope) != ROPE_NONE, "the decode form scores rotated keys")
    a = _lib.SpectralDequantArgs()
    a.L = dp.layout()
    a.n_tokens = int(n_tokens)
    a.k_pages, a.k_page_table, a.n_k_pool = _ptr(k_pages), _ptr(k_table), k_pages.shape[0]
    a.v_pages, a.v_page_table, a.n_v_pool = _ptr(v_pages), _ptr(v_table), v_pages.shape[0]
    a.dec_perm = _ptr(dp.dec_perm)
    a.apply_rope = int(apply_rope)
    a.rope_scaling = consts.rope_scaling
    a.inv_freq[:] = consts.inv_freq
    a.v_codebook[:] = consts.codebook
    a.v_sign_bits[:] = consts.sign_bits
    a.out_dtype = _V_DTYPES[torch.float16]
    a.q, a.q_dtype, a.n_q_groups = _ptr(q), _V_DTYPES[q.dtype], q.shape[1]
    a.sm_scale = float(sm_scale)
    _set_v_codec(a, dp)
    return a


def partial_count(dp: DevicePack, n_tokens: int, q: torch.Tensor, apply_rope: int = 2) -> int:
    """Softmax partials per (head, query) row that dequant's partial form
    writes for n_tokens committed tokens: one per 128-token block when the
    kernel's blocked form applies (see include/bmx_spectral.h), else one per
    64-token group."""
    a = _lib.SpectralDequantArgs()
    a.L = dp.layout()
    a.n_tokens, a.q, a.apply_rope = int(n_tokens), _ptr(q), int(apply_rope)
    _set_v_codec(a, dp)
    n = _lib.lib().bmx_spectral_partial_count(ct.byref(a))
    _need(n >= 0, "n_tokens must be a non-negative multiple of 64")
    return n


def dequant(dp: DevicePack, k_pages: torch.Tensor, k_table: torch.Tensor, v_pages: torch.Tensor,
            v_table: torch.Tensor, n_tokens: int, consts: CodecConsts, *, apply_rope: int = ROPE_NONE,
            dtype: torch.dtype = torch.float32, out: tuple | None = None, q: torch.Tensor | None = None,
            scores: torch.Tensor | None = None, partials: torch.Tensor | None = None, sm_scale: float = 1.0):
    """Pages of one sequence -> dense (K, V), each (h_kv, n_tokens, 128) in
    dtype; keys pre-RoPE (ROPE_NONE) or rotated at read (ROPE_EXACT: fp32
    cos/sin, ROPE_FP16_TABLES: the reference's fp16 tables).  ``out`` takes
    preallocated contiguous (K, V) of shape (h_kv, R, 128), R >= n_tokens, in
    dtype: rows 0 .. n_tokens - 1 of each head are written, the rest left to
    the caller (the recent window of a decode step).

    Decode form: with q (h_kv, G, 128) the kernel also writes scores
    (h_kv, G, R) fp32, q . k of the rotated keys for rows 0 .. n_tokens - 1
    (no softmax scale); out may then be (None, V) and no dense keys are
    written.  Partial form: with q and partials (h_kv, G, 130 * partial_count())
    fp32 the kernel writes each 128-token block's (or 64-token group's)
    softmax partial of the scaled scores (m, l, P.V; see include/bmx_spectral.h) and no dense rows;
    out is then unused."""
    dev = k_pages.device
    # the C-ABI carries no table lengths: a short or wrongly typed table would
    # be read past its end on the device, so every form checks them here
    _need(n_tokens % GROUP == 0, "n_tokens must be a multiple of 64")
    _need(k_table is not None and v_table is not None and k_table.dtype == torch.int32
          and k_table.numel() >= n_tokens // GROUP and v_table.dtype == torch.int32
          and v_table.numel() >= n_tokens // 16, "k_table (n/64) and v_table (n/16) must be int32")
    _need(k_table.device == dev and v_table.device == dev and k_table.is_contiguous()
          and v_table.is_contiguous(), "k_table and v_table must be contiguous on the pages' device")
    if partials is not None:
        _need(q is not None, "partials need q")
        a = _partial_args(dp, k_pages, k_table, v_pages, v_table, n_tokens, consts, q, apply_rope, sm_scale)
        n_parts = _lib.lib().bmx_spectral_partial_count(ct.byref(a))
        _need(partials.dtype == torch.float32 and partials.is_contiguous()
              and tuple(partials.shape) == (dp.h_kv, q.shape[1], 130 * n_parts),
              f"partials must be fp32 (h_kv, G, 130 * {n_parts}): partial_count() per row")
        a.partials = _ptr(partials)
        _lib.check(_lib.lib().bmx_spectral_dequant(ct.byref(a), _stream(dev)), "bmx_spectral_dequant")
        return partials
    _need(dtype in _V_DTYPES, "dtype must be fp16, bf16 or fp32")
    if out is None:
        k = torch.empty(dp.h_kv, n_tokens, HEAD_DIM, dtype=dtype, device=dev)
        v = torch.empty_like(k)
    else:
        k, v = out
        _need(v.dtype == dtype and v.shape[0] == dp.h_kv and v.shape[1] >= n_tokens and v.shape[2] == HEAD_DIM
              and v.is_contiguous() and (k is None or (k.shape == v.shape and k.dtype == dtype and k.is_contiguous())),
              "out tensors: contiguous (h_kv, >= n_tokens, 128) in dtype")
        _need(k is not None or q is not None, "keys may be left out only in the decode form (q given)")
    if q is not None:
        _need(q.dim() == 3 and q.shape[0] == dp.h_kv and q.shape[2] == HEAD_DIM and 1 <= q.shape[1] <= 16
              and q.is_contiguous() and q.dtype in _V_DTYPES, "q must be contiguous (h_kv, 1..16, 128)")
        _need(scores is not None and scores.dtype == torch.float32 and scores.is_contiguous()
              and tuple(scores.shape) == (dp.h_kv, q.shape[1], v.shape[1]), "scores must be fp32 (h_kv, G, rows)")
        _need(int(apply_rope) != ROPE_NONE, "the decode form scores rotated keys")
    a = _lib.SpectralDequantArgs()
    a.L = dp.layout()
    a.n_tokens = int(n_tokens)
    a.k_pages, a.k_page_table, a.n_k_pool = _ptr(k_pages), _ptr(k_table), k_pages.shape[0]
    a.v_pages, a.v_page_table, a.n_v_pool = _ptr(v_pages), _ptr(v_table), v_pages.shape[0]
    a.dec_perm = _ptr(dp.dec_perm)
    a.apply_rope = int(apply_rope)
    a.rope_scaling = consts.rope_scaling
    a.inv_freq[:] = consts.inv_freq
    a.v_codebook[:] = consts.codebook
    a.v_sign_bits[:] = consts.sign_bits
    a.out_dtype = _V_DTYPES[dtype]
    a.k_out, a.v_out = _ptr(k), _ptr(v)
    a.out_rows = v.shape[1]
    _set_v_codec(a, dp)
    if q is not None:
        a.q, a.q_dtype, a.n_q_groups, a.scores = _ptr(q), _V_DTYPES[q.dtype], q.shape[1], _ptr(scores)
    _lib.check(_lib.lib().bmx_spectral_dequant(ct.byref(a), _stream(dev)), "bmx_spectral_dequant")
    return k, v


def decode_attention(dp: DevicePack, k_pages: torch.Tensor, k_table: torch.Tensor, v_pages: torch.Tensor,
                     v_table: torch.Tensor, n_tokens: int, consts: CodecConsts, q: torch.Tensor, sm_scale: float,
                     k_win: torch.Tensor | None = None, v_win: torch.Tensor | None = None,
                     apply_rope: int = 2, out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """One decode step over n_tokens committed tokens and the fp16 (or bf16) window:
    q (h_kv, G, 128) post-RoPE -> (h_kv, G, 128) in out_dtype (q's by default).  The dequant
    kernel's partial form gives every 128-token block's (m, l, P.V); the merge
    kernel scores the window and folds everything by the split softmax's
    weights (m = max m_i, weights e^(m_i - m))."""
    h, G, d = q.shape
    _need(q.is_contiguous() and q.dtype in _V_DTYPES and d == HEAD_DIM, "q (h_kv, G, 128)")
    # no committed token: only the window is read, and a layer that has not
    # committed yet may have no device pack
    _need(n_tokens >= 0 and (n_tokens == 0 or (dp is not None and h == dp.h_kv)),
          "q (h_kv, G, 128) with h_kv of the pack")
    pt = None
    if n_tokens > 0:
        pt = torch.empty(h, G, 130 * partial_count(dp, n_tokens, q, apply_rope), dtype=torch.float32,
                         device=q.device)
        dequant(dp, k_pages, k_table, v_pages, v_table, n_tokens, consts, apply_rope=apply_rope,
                dtype=torch.float16, q=q, partials=pt, sm_scale=sm_scale)
    T = 0 if k_win is None else k_win.shape[1]
    if T:
        _need(k_win.dtype in (torch.float16, torch.bfloat16) and v_win.dtype == k_win.dtype
              and tuple(k_win.shape) == (h, T, d)
              and v_win.shape == k_win.shape and k_win.stride() == v_win.stride() and k_win.stride(2) == 1
              and k_win.stride(1) == d and k_win.stride(0) % 8 == 0 and k_win.data_ptr() % 16 == 0,
              "window keys and values: fp16 or bf16 (h_kv, T, 128) with contiguous rows, 16-byte aligned")
    out_dtype = q.dtype if out_dtype is None else out_dtype
    _need(out_dtype in _V_DTYPES, "out_dtype must be fp16, bf16 or fp32")
    out = torch.empty(h, G, d, dtype=out_dtype, device=q.device)
    a = _lib.SpectralMergeArgs()
    n_parts = 0 if pt is None else pt.shape[2] // 130
    a.h_kv, a.n_q_groups, a.n_groups = h, G, n_parts
    a.partials, a.q, a.q_dtype = _ptr(pt), _ptr(q), _V_DTYPES[q.dtype]
    a.k_win, a.v_win, a.win_len = (_ptr(k_win), _ptr(v_win), T) if T else (None, None, 0)
    a.win_stride_h = k_win.stride(0) if T else 0
    a.win_dtype = 1 if T and k_win.dtype == torch.bfloat16 else 0   # BMX_K2B_TAIL_BF16 / _F16
    a.sm_scale, a.out, a.out_dtype = float(sm_scale), _ptr(out), _V_DTYPES[out_dtype]
    a.v_sign_bits[:] = consts.sign_bits
    if dp is not None:
        _set_v_codec(a, dp)
    _lib.check(_lib.lib().bmx_spectral_merge(ct.byref(a), _stream(q.device)), "bmx_spectral_merge")
    return out

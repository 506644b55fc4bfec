"""CPU restatement of the reference's spectral (K4) key codec and of this
build's spectral key page (test infrastructure: only tests/, smoke() and
bench.py's cpu_baseline may use it, as the checker; the product never imports
it).

Reference algorithm (paths under src/bmx):
  * allocate_bits_from_variance, selection "round"   cache/codecs.py:203-287
    (_round_to_tiers :147-152)
  * tier_columns                                      cache/spectral.py:631-645
  * spectral_quantize_packed (quantizer "rtn", mse_scale=True):
    Y = M @ enc, then rtn_quantize_packed per tier over 64-token groups
                                                      cache/spectral.py:763-815,
                                                      quant/rtn.py:10-44
  * spectral_dequant_packed: Y_hat @ dec^T            cache/spectral.py:818-841
  * int8_decoder_roundtrip, the tiered int8 certificate and the per-layer
    thresholds it picks                               cache/spectral.py:913-1033,
                                                      1176-1210
  * the Lloyd payload (quantizer "lloyd"): _lloyd_quantize_packed /
    _lloyd_dequantize_packed                          cache/spectral.py:648-700
Pinned by tests/test_spectral_cpu.py against the reference's own outputs
(tests/golden/spectral.npz): the allocation at three budgets, the tier
columns, every code and scale of four groups given the reference's Y, and
the dequantized keys; the encode order below against a float64 product.
The Lloyd payload against the same file: the reference's level indices for
every column of every tier given the reference's Y, its steps, its
dequantized keys; and every code against the nearest-level rule it
implements.  The int8 decoder functions against tests/golden/spectral_variants.npz (the
roundtrip bit for bit at three thresholds, the certificate at every
threshold, the per-layer thresholds at three bars), and the certificate
against a Monte-Carlo estimate of the distortion it states in closed form.

The device restatement fixes two orders the reference leaves to torch:
  * encode: Y[t, j] = sum over c = 0, 1, ... of M[t, c] * enc[c, j], each
    product and each sum rounded to fp32 (no fused multiply-add);
  * the MSE scale refinement sums the 64 products of a group left to right
    in fp32.
Scales are stored as fp16 on the device page (the reference's accounting
charge, scale_bits = 16 / group); dequant(fp16_scales=True) is what the
device pages hold.

The Lloyd payload fixes its orders the same way: the initial step is the
sample deviation with the mean and the squared deviations summed left to
right in float64 (torch's float64 Welford gives the same fp32 value on
every group of the golden file), then the refits' sums left to right in
fp32.  The page stores the level index itself.

Page format (one page per 64-token group of one layer; tokens of the group
are the page's rows):
  * columns: tier_columns order (tier ascending, then column), each tier
    padded with zero columns to a multiple of 8; c_pad columns in all.
    Column k of the page is original column perm[k] (-1 = padding).
  * SCALE  [c_pad] fp16 at byte 0: the group's scale of each column.
  * slices: 8 columns each, slice s at byte offset off[s] (after SCALE, in
    order), 64 * w bytes: token t's 8 codes in the w bytes at off[s] + t * w
    (little-endian), column k of the slice at bits [k * w, (k + 1) * w).
    w is the tier's container: 2 bits for tier 2, 4 for tiers 3 and 4, 8 for
    tiers 5, 6 and 8 (the reference's containers, spectral.py:699-737); the
    stored value is code + 2^(b - 1) for tier b.
  * 16 bytes of padding end the page.
"""

from __future__ import annotations

import math

import numpy as np

TIERS = (0, 2, 3, 4, 5, 6, 8)
CONTAINER = {2: 2, 3: 4, 4: 4, 5: 8, 6: 8, 8: 8}
GROUP = 64


def round_to_tiers(b: np.ndarray, tiers: np.ndarray) -> np.ndarray:
    """Nearest tier, the lower one on a tie (codecs.py:147-152)."""
    return tiers[np.abs(b[:, None] - tiers[None, :]).argmin(axis=1)]


def allocate_bits_round(var, budget: float, tiers=TIERS, n_search: int = 40) -> np.ndarray:
    """Reverse water-filling with midpoint rounding to the tier grid: bisect
    log(kappa) for the smallest kappa whose mean rounded rate is within the
    budget (codecs.py:247-287)."""
    var = np.maximum(np.asarray(var, dtype=np.float64), 1e-30)
    tt = np.array(sorted(tiers), dtype=np.float64)
    lo_k, hi_k = float(var.min()) * 1e-6, float(var.max()) * 1e6
    lo, hi = math.log(lo_k), math.log(hi_k)
    best = round_to_tiers(np.maximum(0.5 * np.log2(var / hi_k), 0.0), tt)
    for _ in range(n_search):
        mid = 0.5 * (lo + hi)
        b = round_to_tiers(np.maximum(0.5 * np.log2(var / math.exp(mid)), 0.0), tt)
        if b.mean() <= budget + 1e-12:
            best, hi = b, mid
        else:
            lo = mid
    return best.astype(np.int64)


def tier_columns(bits) -> dict:
    """{tier: ascending column indices}, zero tier left out (spectral.py:631-645)."""
    bits = np.asarray(bits)
    return {int(b): np.nonzero(bits == b)[0] for b in sorted(set(bits.tolist())) if b != 0}


def payload_bpe(bits, group: int = GROUP) -> float:
    """mean(bits) + (16 / group) * c_used / C (spectral.py:602-615)."""
    bits = np.asarray(bits)
    return float(bits.mean()) + 16.0 / group * float((bits != 0).sum()) / bits.shape[0]


def quantize_groups(G: np.ndarray, b: int, n_iter: int = 10):
    """RTN at b bits with the MSE-refined step over each row of G (n, 64),
    fp32, sums left to right (rtn.py:10-44): scale = max|G| / qmax, then
    n_iter rounds of Q = clamp(round(G / scale)), scale = <G, Q> / <Q, Q>.
    Returns (signed codes int, fp32 scales (n,))."""
    G = np.asarray(G, dtype=np.float32)
    f32 = np.float32
    qmax = 2 ** (b - 1) - 1
    tiny = f32(1e-12)
    scale = np.maximum(np.abs(G).max(axis=1), tiny) / f32(qmax)

    def codes(s):
        return np.clip(np.rint(G / s[:, None]), -qmax - 1, qmax).astype(np.float32)

    for _ in range(n_iter):
        Q = codes(scale)
        num = np.zeros(G.shape[0], np.float32)
        den = np.zeros(G.shape[0], np.float32)
        for t in range(G.shape[1]):
            num = num + G[:, t] * Q[:, t]
            den = den + Q[:, t] * Q[:, t]
        scale = np.maximum(num / np.maximum(den, tiny), tiny)
    return codes(scale).astype(np.int64), scale.astype(np.float32)


def lloyd_quantize_groups(G: np.ndarray, levels, n_iter: int = 3):
    """The Lloyd payload over each row of G (n, 64), fp32 (spectral.py:
    648-684): step = the sample deviation (at least 1e-12), code = the number
    of midpoints (l_i + l_{i+1}) / 2 below value / step, then n_iter rounds of
    step = <G, l_code> / <l_code, l_code> and new codes.  Returns (level
    indices int, fp32 steps (n,))."""
    G = np.asarray(G, dtype=np.float32)
    f32 = np.float32
    cb = np.asarray(levels, dtype=np.float32)
    mid = ((cb[:-1] + cb[1:]) * f32(0.5)).astype(np.float32)
    tiny = f32(1e-12)
    g64 = G.astype(np.float64)
    tot = np.zeros(G.shape[0])
    for t in range(G.shape[1]):
        tot = tot + g64[:, t]
    mean = tot / 64.0
    ss = np.zeros(G.shape[0])
    for t in range(G.shape[1]):
        d = g64[:, t] - mean
        ss = ss + d * d
    scale = np.maximum(np.sqrt(ss / 63.0).astype(np.float32), tiny)

    def codes(s):
        return np.searchsorted(mid, G / s[:, None], side="left")

    q = codes(scale)
    for _ in range(n_iter):
        lv = cb[q]
        num = np.zeros(G.shape[0], np.float32)
        den = np.zeros(G.shape[0], np.float32)
        for t in range(G.shape[1]):
            num = num + G[:, t] * lv[:, t]
            den = den + lv[:, t] * lv[:, t]
        scale = np.maximum(num / np.maximum(den, tiny), tiny)
        q = codes(scale)
    return q.astype(np.int64), scale.astype(np.float32)


class Layout:
    """The page layout of a pack's bit allocation (module docstring)."""

    def __init__(self, bits):
        bits = np.asarray(bits, dtype=np.int64)
        self.C = int(bits.shape[0])
        perm, slice_bits = [], []
        for b, cols in tier_columns(bits).items():
            n_pad = -(-len(cols) // 8) * 8
            perm += list(cols) + [-1] * (n_pad - len(cols))
            slice_bits += [b] * (n_pad // 8)
        self.perm = np.array(perm, dtype=np.int64)
        self.c_pad = len(perm)
        self.slice_bits = np.array(slice_bits, dtype=np.int64)
        self.width = np.array([CONTAINER[b] for b in slice_bits], dtype=np.int64)
        sizes = GROUP * self.width
        self.off = 2 * self.c_pad + np.concatenate([[0], np.cumsum(sizes)[:-1]]).astype(np.int64)
        self.page_bytes = int(2 * self.c_pad + sizes.sum() + 16)
        self.col_bits = np.repeat(self.slice_bits, 8)

    def slice_table(self) -> np.ndarray:
        """int32 per slice: byte offset | tier bits << 24 (the kernels' table)."""
        return (self.off | (self.slice_bits << 24)).astype(np.int32)

    def permute_cols(self, X: np.ndarray) -> np.ndarray:
        """X[..., C] -> X[..., c_pad] in page column order, zero padding."""
        out = np.zeros(X.shape[:-1] + (self.c_pad,), dtype=X.dtype)
        k = self.perm >= 0
        out[..., k] = X[..., self.perm[k]]
        return out


def encode(M: np.ndarray, enc: np.ndarray, layout: Layout) -> np.ndarray:
    """Y in page column order, (S, c_pad) fp32, in the device's order."""
    M = np.asarray(M, dtype=np.float32)
    encp = layout.permute_cols(np.asarray(enc, dtype=np.float32))
    Y = np.zeros((M.shape[0], layout.c_pad), np.float32)
    for c in range(M.shape[1]):
        Y = Y + M[:, c: c + 1] * encp[c: c + 1, :]
    return Y


def quantize(Y: np.ndarray, layout: Layout, lloyd: dict | None = None):
    """Codes (n_groups, 64, c_pad) int and fp32 scales (n_groups, c_pad) of Y
    in page column order; with lloyd ({tier: levels}) the Lloyd payload's
    level indices."""
    S = Y.shape[0]
    assert S % GROUP == 0
    ng = S // GROUP
    codes = np.zeros((ng, GROUP, layout.c_pad), np.int64)
    scales = np.zeros((ng, layout.c_pad), np.float32)
    for b in sorted(set(layout.slice_bits.tolist())):
        k = np.nonzero(layout.col_bits == b)[0]
        G = Y[:, k].T.reshape(len(k), ng, GROUP).transpose(1, 0, 2).reshape(ng * len(k), GROUP)
        q, s = lloyd_quantize_groups(G, lloyd[b]) if lloyd is not None else quantize_groups(G, b)
        codes[:, :, k] = q.reshape(ng, len(k), GROUP).transpose(0, 2, 1)
        scales[:, k] = s.reshape(ng, len(k))
    return codes, scales


def code_values(codes, layout: Layout, lloyd: dict | None = None) -> np.ndarray:
    """The codes' values before the step: the signed code, or the Lloyd
    level of the index (fp32 levels; padding columns 0)."""
    if lloyd is None:
        return codes.astype(np.float64)
    out = np.zeros(codes.shape, np.float64)
    for b in sorted(set(layout.slice_bits.tolist())):
        k = layout.col_bits == b
        out[..., k] = np.asarray(lloyd[b], np.float32).astype(np.float64)[codes[..., k]]
    out[..., layout.perm < 0] = 0.0
    return out


def dequant(codes, scales, dec, layout: Layout, fp16_scales: bool = True, lloyd: dict | None = None) -> np.ndarray:
    """Pre-RoPE keys (S, C) float64 = Y_hat @ dec^T, Y_hat = code * scale
    (the Lloyd payload: level * scale)."""
    s = scales.astype(np.float16).astype(np.float64) if fp16_scales else scales.astype(np.float64)
    Yh = (code_values(codes, layout, lloyd) * s[:, None, :]).reshape(-1, layout.c_pad)
    decp = layout.permute_cols(np.asarray(dec, dtype=np.float64))
    return Yh @ decp.T


def pack_pages(codes, scales, layout: Layout, lloyd: bool = False) -> np.ndarray:
    """(n_groups, page_bytes) uint8 pages of codes (n_groups, 64, c_pad) and
    fp32 scales (stored as fp16); Lloyd level indices are stored as they are."""
    ng = codes.shape[0]
    pages = np.zeros((ng, layout.page_bytes), np.uint8)
    pages[:, : 2 * layout.c_pad] = scales.astype(np.float16).view(np.uint8).reshape(ng, -1)
    for s in range(len(layout.width)):
        w, b = int(layout.width[s]), int(layout.slice_bits[s])
        stored = (codes[:, :, 8 * s: 8 * s + 8] + (0 if lloyd else 1 << (b - 1))).astype(np.uint64)
        word = np.zeros((ng, GROUP), np.uint64)
        for k in range(8):
            word |= stored[:, :, k] << np.uint64(k * w)
        raw = word.astype("<u8").view(np.uint8).reshape(ng, GROUP, 8)[:, :, :w]
        o = int(layout.off[s])
        pages[:, o: o + GROUP * w] = raw.reshape(ng, GROUP * w)
    return pages


def unpack_pages(pages, layout: Layout, lloyd: bool = False):
    """Inverse of pack_pages: (codes, fp16 scales as fp32)."""
    ng = pages.shape[0]
    scales = pages[:, : 2 * layout.c_pad].copy().view(np.float16).astype(np.float32)
    codes = np.zeros((ng, GROUP, layout.c_pad), np.int64)
    for s in range(len(layout.width)):
        w, b = int(layout.width[s]), int(layout.slice_bits[s])
        o = int(layout.off[s])
        raw = np.zeros((ng, GROUP, 8), np.uint8)
        raw[:, :, :w] = pages[:, o: o + GROUP * w].reshape(ng, GROUP, w)
        word = raw.view("<u8")[..., 0]
        for k in range(8):
            codes[:, :, 8 * s + k] = ((word >> np.uint64(k * w)) & np.uint64((1 << w) - 1)).astype(np.int64) \
                - (0 if lloyd else 1 << (b - 1))
    return codes, scales


TIER_THRESHOLD_GRID = (2, 3, 4, 5, 6, 8)


def int8_decoder_roundtrip(dec, bits, tier_threshold=None) -> np.ndarray:
    """fp32 decoder whose columns with 0 < bits (<= tier_threshold if given)
    are stored int8 with one fp16 absmax scale per column and read back
    (spectral.py:913-944); round half to even, codes in [-127, 127]."""
    dec = np.asarray(dec, dtype=np.float32)
    bits = np.asarray(bits)
    sel = bits != 0
    if tier_threshold is not None:
        sel &= bits <= tier_threshold
    out = dec.copy()
    if sel.any():
        c = dec[:, sel]
        s = np.maximum(np.abs(c).max(axis=0) / np.float32(127.0), np.float32(1e-12))
        s = s.astype(np.float16).astype(np.float32)
        out[:, sel] = np.clip(np.rint(c / s), -127.0, 127.0).astype(np.float32) * s
    return out


def int8_certificate(enc, dec, lam, bits, tier_threshold) -> tuple:
    """(added, payload, implied_rel_degradation) in float64
    (spectral.py:947-960): the expected weighted distortion the int8 decoder
    adds for codes of second moment diag(lam), against the payload's."""
    D = int8_decoder_roundtrip(dec, bits, tier_threshold).astype(np.float64) - np.asarray(dec, np.float64)
    lam = np.maximum(np.asarray(lam, np.float64), 0.0)
    proj = np.asarray(enc, np.float64).T @ D
    added = float((lam * (proj ** 2).sum(axis=0)).sum())
    payload = float((lam * 4.0 ** -np.asarray(bits, np.float64)).sum())
    return added, payload, added / max(payload + added, 1e-300)


def per_layer_tier_thresholds(layers: dict, bar: float = 0.05) -> dict:
    """{layer: largest T of the grid whose certificate stays <= bar, else 0}
    for layers {i: (enc, dec, lam, bits)} (spectral.py:1176-1210)."""
    out = {}
    for i, (enc, dec, lam, bits) in layers.items():
        ok = [t for t in TIER_THRESHOLD_GRID if int8_certificate(enc, dec, lam, bits, t)[2] <= bar]
        out[i] = ok[-1] if ok else 0
    return out

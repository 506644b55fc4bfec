"""CPU restatement of the k2b codec family (test infrastructure only).

Every function below restates one reference function in fp32 torch on the CPU,
with the same operation order where the order decides rounding (FWHT stage
order, divide-then-round RTN, fp16 round trips).  Reference paths are under
/root/reference/src/bmx.
"""

from __future__ import annotations

import functools
import math

import torch

# ---------------------------------------------------------------------------
# bpe accounting terms — cache/codecs.py:79-96
# ---------------------------------------------------------------------------


def scale_bits(group: int) -> float:
    """fp16 group scale amortised per entry (codecs.py:79-81)."""
    return 16.0 / group


def norm_bits(h: int, C: int) -> float:
    """fp16 norm per (row, head) amortised per entry (codecs.py:84-86)."""
    return 16.0 * h / C


def factor_bits(rank: int, S: int, C: int) -> float:
    """fp16 Us (S x r) + V (C x r) amortised per entry (codecs.py:89-91)."""
    return 16.0 * rank * (S + C) / (S * C)


def compute_flush_schedule(S: int, W: int, g: int) -> int:
    """Committed-prefix length: largest multiple of g leaving >= W fp16 tokens
    (cache/streaming.py:144-151)."""
    return ((S - W) // g) * g if S > W else 0


# ---------------------------------------------------------------------------
# Layout helpers — cache/collect.py:42-51
# ---------------------------------------------------------------------------


def to_matrix(kv: torch.Tensor) -> torch.Tensor:
    """(h, S, d) -> (S, h*d) fp32 (collect.py:42-45)."""
    h, S, d = kv.shape
    return kv.permute(1, 0, 2).reshape(S, h * d).float()


def from_matrix(M: torch.Tensor, h: int) -> torch.Tensor:
    """(S, h*d) -> (h, S, d) (collect.py:48-51)."""
    S, hd = M.shape
    return M.reshape(S, h, hd // h).permute(1, 0, 2)


# ---------------------------------------------------------------------------
# Rotations — quant/hadamard.py:12-33, cache/codecs.py:104-139
# ---------------------------------------------------------------------------


def fwht(x: torch.Tensor) -> torch.Tensor:
    """Orthonormal Walsh-Hadamard transform over the last dim, Sylvester order
    (hadamard.py:12-25).  Stage h combines (i, i+h) inside blocks of 2h; the
    1/sqrt(d) is applied once at the end, as the reference does."""
    d = x.shape[-1]
    assert d > 0 and d & (d - 1) == 0
    y = x.reshape(-1, d).clone()
    h = 1
    while h < d:
        y4 = y.view(-1, d // (2 * h), 2, h)
        a, b = y4[:, :, 0, :], y4[:, :, 1, :]
        y = torch.stack((a + b, a - b), dim=2).view(-1, d)
        h *= 2
    return (y / d**0.5).view(x.shape)


@functools.lru_cache(maxsize=32)
def hadamard_signs(C: int, seed: int) -> torch.Tensor:
    """Seeded +-1 vector (int64) used by the randomized Hadamard
    (codecs.py:114-124 and hadamard.py:28-33 draw it identically)."""
    g = torch.Generator().manual_seed(seed)
    return torch.randint(0, 2, (C,), generator=g) * 2 - 1


def randomized_hadamard(x: torch.Tensor, seed: int) -> torch.Tensor:
    """fwht(x * signs) (hadamard.py:28-33)."""
    signs = hadamard_signs(x.shape[-1], seed).to(x)
    return fwht(x * signs)


def unrotate(M_rot: torch.Tensor, seed: int) -> torch.Tensor:
    """Inverse of randomized_hadamard: fwht(M) * signs (codecs.py:127-139)."""
    signs = hadamard_signs(M_rot.shape[-1], seed).to(M_rot)
    return fwht(M_rot) * signs


# ---------------------------------------------------------------------------
# Lloyd-Max codebook — cache/codecs.py:346-380
# ---------------------------------------------------------------------------


@functools.lru_cache(maxsize=16)
def gaussian_codebook(bits: int, n_samples: int = 2**18, n_iter: int = 40,
                      seed: int = 0) -> torch.Tensor:
    """Empirical 1-D Lloyd-Max codebook for N(0,1): 2**bits sorted fp32 levels
    (codecs.py:346-380).  Levels start at the empirical quantiles and are
    recentred on their cell means n_iter times."""
    n_levels = 2**bits
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(n_samples, generator=g)
    probs = torch.linspace(0, 1, n_levels + 2)[1:-1]
    levels = torch.quantile(x, probs)
    for _ in range(n_iter):
        mid = (levels[:-1] + levels[1:]) / 2
        cell = torch.bucketize(x, mid)
        new = torch.zeros(n_levels)
        for k in range(n_levels):
            sel = cell == k
            new[k] = x[sel].mean() if sel.any() else levels[k]
        levels = new
    return levels.sort().values


# ---------------------------------------------------------------------------
# RTN — quant/rtn.py:23-53
# ---------------------------------------------------------------------------


def rtn_quantize_packed(W: torch.Tensor, bits: int, group_size: int):
    """(..., d) -> (int8 codes, fp32 scale (..., d/group, 1)).  Symmetric RTN:
    scale = max|x| (clamped 1e-12) / qmax, code = clamp(round_half_even(x/scale),
    -qmax-1, qmax)  (rtn.py:23-44, max-based scale)."""
    *lead, d = W.shape
    assert d % group_size == 0
    qmax = 2 ** (bits - 1) - 1
    Gr = W.reshape(*lead, d // group_size, group_size)
    scale = Gr.abs().amax(dim=-1, keepdim=True).clamp_min(1e-12) / qmax
    Q = (Gr / scale).round().clamp(-qmax - 1, qmax)
    return Q.to(torch.int8).reshape(W.shape), scale


def rtn_dequantize_packed(Q_int: torch.Tensor, scale: torch.Tensor, group_size: int):
    """codes * group scale (rtn.py:47-53)."""
    *lead, d = Q_int.shape
    Gr = Q_int.reshape(*lead, d // group_size, group_size).to(scale.dtype)
    return (Gr * scale).reshape(Q_int.shape)


# ---------------------------------------------------------------------------
# k2b key codec: lowrank_rtn_channel — codecs.py:677-695, 786-796, 839-842
# ---------------------------------------------------------------------------


def truncated_svd(M: torch.Tensor, r: int):
    """(U*s, V) rank-r factors (decomp/lrs.py:35-41)."""
    U, s, Vh = torch.linalg.svd(M, full_matrices=False)
    return U[:, :r] * s[:r], Vh[:r, :].mT.contiguous()


def quantize_k2b_key(M: torch.Tensor, Us: torch.Tensor, V: torch.Tensor, *,
                     bits: int = 3, group: int = 64):
    """One (S, C) pre-RoPE key page -> packed dict + honest bpe.

    Us, V are the page's factors: fp16 round trip, L = Us16 @ V16^T,
    R = M - L, per-channel RTN of R with groups along tokens
    (codecs.py:677-695 and 786-796)."""
    S, C = M.shape
    rank = V.shape[1]
    assert S % group == 0
    Us16 = Us.half().float()
    V16 = V.half().float()
    L = Us16 @ V16.mT
    R = M - L
    q, scale = rtn_quantize_packed(R.mT, bits, group)
    bpe = bits + scale_bits(group) + factor_bits(rank, S, C)
    return {"Us": Us16, "V": V16, "res_Q_int": q, "res_scale": scale}, bpe


def dequant_k2b_key(packed: dict, group: int = 64) -> torch.Tensor:
    """L + RTN residual (codecs.py:839-842)."""
    L = packed["Us"] @ packed["V"].mT
    R = rtn_dequantize_packed(packed["res_Q_int"], packed["res_scale"], group).mT
    return L + R


class FrozenSubspaceKeyEncoder:
    """Per-layer write-once key encoder: the first committed page fits a rank-r
    SVD and freezes V; later pages project Us = M @ V_frozen
    (packed_streaming.py:475-542, branch at :507-530)."""

    def __init__(self, rank: int, bits: int = 3, group: int = 64):
        self.rank, self.bits, self.group = rank, bits, group
        self.frozen = None  # (Us_first, V_fp32)

    def encode(self, M: torch.Tensor, us_override=None):
        if self.frozen is None:
            Us, V = truncated_svd(M, self.rank) if us_override is None else us_override
            self.frozen = (Us, V)
        else:
            Us = M @ self.frozen[1]
        return quantize_k2b_key(M, Us, self.frozen[1], bits=self.bits, group=self.group)


# ---------------------------------------------------------------------------
# Per-head Hadamard / Lloyd value codec: turboquant_mse_perhead
# codecs.py:616-649, 734-745
# ---------------------------------------------------------------------------


def quantize_v_perhead(M: torch.Tensor, *, bits: int = 2, seed: int = 0, h: int = 1):
    """(S, C=h*d) -> (int16 codes (S, C), fp32 norms (S, h) that are fp16-exact),
    bpe.  Per (row, head): n = fp16(||v||), u = v/n, x = fwht(u * signs) * sqrt(d),
    code = bucketize(x, codebook midpoints) (codecs.py:616-636)."""
    S, C = M.shape
    d = C // h
    Mh = M.reshape(S, h, d)
    norms = Mh.norm(dim=2).clamp_min(1e-12).half().float()
    unit = Mh / norms[:, :, None]
    rot = randomized_hadamard(unit.reshape(S * h, d), seed).reshape(S, h, d)
    cb = gaussian_codebook(bits)
    mid = (cb[:-1] + cb[1:]) / 2
    idx = torch.bucketize(rot * math.sqrt(d), mid).to(torch.int16).reshape(S, C)
    return idx, norms, bits + norm_bits(h, C)


def dequant_v_perhead(idx: torch.Tensor, norms: torch.Tensor, *, bits: int = 2,
                      seed: int = 0, h: int = 1) -> torch.Tensor:
    """fwht(cb[idx]/sqrt(d)) * signs * norm (codecs.py:639-649)."""
    S, C = idx.shape
    d = C // h
    cb = gaussian_codebook(bits)
    Mq = (cb[idx.long()] / math.sqrt(d)).reshape(S, h, d)
    rec = unrotate(Mq.reshape(S * h, d), seed).reshape(S, h, d)
    return (rec * norms[:, :, None]).reshape(S, C)


# ---------------------------------------------------------------------------
# RTN arms (config-1 analogues) — codecs.py:720-725, 819-822
# ---------------------------------------------------------------------------


def quantize_rtn_token(M: torch.Tensor, bits: int, group: int):
    q, s = rtn_quantize_packed(M, bits, group)
    return {"Q_int": q, "scale": s}, bits + scale_bits(group)


def quantize_rtn_channel(M: torch.Tensor, bits: int, group: int):
    q, s = rtn_quantize_packed(M.mT, bits, group)
    return {"Q_int": q, "scale": s}, bits + scale_bits(group)


def dequant_rtn_token(p: dict, group: int) -> torch.Tensor:
    return rtn_dequantize_packed(p["Q_int"], p["scale"], group)


def dequant_rtn_channel(p: dict, group: int) -> torch.Tensor:
    return rtn_dequantize_packed(p["Q_int"], p["scale"], group).mT


# ---------------------------------------------------------------------------
# Reference sub-byte containers — cache/triton_dequant_attention.py:49-165
# ---------------------------------------------------------------------------


def pack_codes(idx: torch.Tensor, bits: int) -> torch.Tensor:
    """8/bits unsigned codes per byte, little-endian (triton_dequant_attention.py:49-82)."""
    per = 8 // bits
    C = idx.shape[-1]
    g = idx.to(torch.int32).reshape(*idx.shape[:-1], C // per, per)
    sh = torch.arange(per, dtype=torch.int32) * bits
    return (g << sh).sum(-1).to(torch.uint8)


def pack_signed_codes(code: torch.Tensor, bits: int) -> torch.Tensor:
    """Two's-complement nibbles, low nibble first (triton_dequant_attention.py:103-142)."""
    nib = code.to(torch.int32) & 0xF
    g = nib.reshape(*code.shape[:-1], code.shape[-1] // 2, 2)
    return (g[..., 0] | (g[..., 1] << 4)).to(torch.uint8)

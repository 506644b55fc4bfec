"""CPU restatement of the decode-attention side (test infrastructure only).

RoPE tables, the single-softmax oracle, the chunked online-softmax path, the
fp16-tail partial and the split-merge formula, all fp32 on the CPU.  Reference
paths are under /root/reference/src/bmx.
"""

from __future__ import annotations

import torch

from . import codecs as C

# ---------------------------------------------------------------------------
# RoPE — cache/rope.py:19-102 (HF LlamaRotaryEmbedding, default rope type)
# ---------------------------------------------------------------------------


def default_inv_freq(d: int, theta: float) -> torch.Tensor:
    """HF default-rope inverse frequencies, computed in fp32 the way
    transformers' _compute_default_rope_parameters does."""
    exps = torch.arange(0, d, 2, dtype=torch.int64).to(dtype=torch.float) / d
    return 1.0 / (theta ** exps)


def rope_cos_sin(inv_freq: torch.Tensor, positions: torch.Tensor,
                 attention_scaling: float = 1.0):
    """(S, d) fp32 cos/sin for absolute positions (rope.py:19-58).

    angle = fl32(inv_freq_j * pos) — one fp32 product per entry, exactly what
    HF's (d/2 x 1) @ (1 x S) fp32 matmul produces — then cat(angle, angle)."""
    ang = inv_freq.float()[None, :] * positions.float()[:, None]
    emb = torch.cat((ang, ang), dim=-1)
    return emb.cos() * attention_scaling, emb.sin() * attention_scaling


def rotate_half(x: torch.Tensor) -> torch.Tensor:
    """cat(-x2, x1) (rope.py:61-72)."""
    d = x.shape[-1]
    return torch.cat((-x[..., d // 2:], x[..., : d // 2]), dim=-1)


def apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """x*cos + rotate_half(x)*sin, tables broadcast over heads (rope.py:75-102)."""
    return x * cos.unsqueeze(0) + rotate_half(x) * sin.unsqueeze(0)


# ---------------------------------------------------------------------------
# Softmax pieces — chunked_attention.py:26-49, triton_dequant_attention.py:324-461
# ---------------------------------------------------------------------------


def online_softmax_update(acc, m, lse, scores_new, v_new):
    """One exact online-softmax step; lse is the raw sum of weights
    (chunked_attention.py:26-38)."""
    m_new = torch.maximum(m, scores_new.amax(dim=-1, keepdim=True))
    corr = torch.exp(m - m_new)
    p = torch.exp(scores_new - m_new)
    lse = lse * corr + p.sum(dim=-1, keepdim=True)
    acc = acc * corr + p @ v_new
    return acc, m_new, lse


def tail_partial(q_kv, k_tail, v_tail, scale):
    """fp16 recent window as one extra split partial (acc, m, lse), GQA-shaped
    (triton_dequant_attention.py:324-360).  q_kv (h_kv, G, d)."""
    s = torch.einsum("hgd,htd->hgt", q_kv.float(), k_tail.float()) * scale
    m = s.amax(dim=-1)
    p = torch.exp(s - m.unsqueeze(-1))
    return torch.einsum("hgt,htd->hgd", p, v_tail.float()), m, p.sum(dim=-1)


def merge_partials(acc, m, lse):
    """Base-e split merge (triton_dequant_attention.py:409-461):
    m* = max m_i, l = sum lse_i e^(m_i-m*), out = sum acc_i e^(m_i-m*) / l.
    acc (n, ..., d), m/lse (n, ...)."""
    mg = m.amax(dim=0)
    w = torch.exp(m - mg)
    l = (lse * w).sum(dim=0)
    return (acc * w.unsqueeze(-1)).sum(dim=0) / l.unsqueeze(-1)


def attention_diff(a, b) -> dict:
    """max_abs / max_rel / mean_abs drift (chunked_attention.py:41-49)."""
    diff = (a.double() - b.double()).abs()
    return {"max_abs": float(diff.max()),
            "max_rel": float((diff / b.double().abs().clamp_min(1e-12)).max()),
            "mean_abs": float(diff.mean())}


# ---------------------------------------------------------------------------
# k2b cache on the CPU: a list of committed 128-token codec pages + fp16 tail
# ---------------------------------------------------------------------------


class K2bOracleCache:
    """Committed k2b pages of one sequence, as the reference's block dicts hold
    them (packed_streaming.py:582-730), plus helpers to dequantize them."""

    def __init__(self, h_kv: int, d: int, rank: int, *, group: int = 64,
                 page: int = 128, k_bits: int = 3, v_bits: int = 2, v_seed: int = 0):
        self.h_kv, self.d, self.rank = h_kv, d, rank
        self.group, self.page, self.k_bits = group, page, k_bits
        self.v_bits, self.v_seed = v_bits, v_seed
        self.enc = C.FrozenSubspaceKeyEncoder(rank, k_bits, group)
        self.k_blocks: list = []   # (dict, start, end)
        self.v_blocks: list = []   # ((idx, norms), start, end)

    @property
    def n_tokens(self) -> int:
        return len(self.k_blocks) * self.page

    def commit(self, k_pre_page: torch.Tensor, v_page: torch.Tensor, us_override=None):
        """k_pre_page, v_page: (h_kv, page, d) fp16 -> one committed codec page."""
        M = C.to_matrix(k_pre_page.float())
        kp, _ = self.enc.encode(M, us_override)
        Mv = C.to_matrix(v_page.float())
        idx, norms, _ = C.quantize_v_perhead(Mv, bits=self.v_bits, seed=self.v_seed,
                                             h=self.h_kv)
        s = self.n_tokens
        self.k_blocks.append((kp, s, s + self.page))
        self.v_blocks.append(((idx, norms), s, s + self.page))

    def dense_k_pre(self) -> torch.Tensor:
        """(h_kv, S, d) fp32 dequantized pre-RoPE keys."""
        return torch.cat([C.from_matrix(C.dequant_k2b_key(kp, self.group), self.h_kv)
                          for kp, _, _ in self.k_blocks], dim=1)

    def dense_v(self) -> torch.Tensor:
        return torch.cat([C.from_matrix(
            C.dequant_v_perhead(idx, n, bits=self.v_bits, seed=self.v_seed, h=self.h_kv),
            self.h_kv) for (idx, n), _, _ in self.v_blocks], dim=1)


def naive_dense_attention(q, K_post, V, n_q_groups: int, scale: float):
    """Single-softmax oracle (chunked_attention.py:254-317): GQA expand by
    repeat_interleave, one softmax over every key.  q (n_q, 1, d) fp32,
    K_post/V (h_kv, S, d) post-RoPE keys / values."""
    Kx = K_post.float().repeat_interleave(n_q_groups, dim=0)
    Vx = V.float().repeat_interleave(n_q_groups, dim=0)
    s = (q.float() @ Kx.transpose(-1, -2)) * scale
    return torch.softmax(s, dim=-1) @ Vx


def grouped_dense_attention(q, K_post, V, n_q_groups: int, scale: float):
    """``naive_dense_attention`` for several query positions without the GQA
    copy of the keys: query head i reads KV head i // n_q_groups, the
    repeat_interleave order.  q (n_q, n, d) -> (n_q, n, d) fp32, one softmax
    over every key per (head, position)."""
    h_kv, S, d = K_post.shape
    n_q, n, _ = q.shape
    qg = q.float().reshape(h_kv, n_q_groups * n, d)
    s = (qg @ K_post.float().transpose(-1, -2)) * scale
    return (torch.softmax(s, dim=-1) @ V.float()).reshape(n_q, n, d)


def argmax_flip(r_out: torch.Tensor, r_ref: torch.Tensor) -> tuple:
    """(flip, hard) for one step of the reference's teacher-forced argmax-flip
    gate (scripts/profile_decode_ab.py:325-343, 388-395, 429-437): the step
    flips when the argmaxes differ; the flip is hard -- a real divergence, not
    accumulation-order drift -- when the reference's top-2 gap exceeds the
    step's max-abs delta.  The gate fails on any hard flip or on more than
    N // 8 flips over N steps.  r_out, r_ref: 1-D readouts of one step."""
    flip = bool(r_out.argmax() != r_ref.argmax())
    top2 = r_ref.topk(2).values
    gap = (top2[0] - top2[1]).item()
    delta = (r_out - r_ref).abs().max().item()
    return flip, flip and gap > delta


def k2b_dense_kv(cache: K2bOracleCache, inv_freq, k_tail=None, v_tail=None,
                 attention_scaling: float = 1.0):
    """Dequantize every committed page, RoPE the keys at read with fp32 tables,
    append the fp16 tail (chunked_attention.py:148-251)."""
    S = cache.n_tokens
    K = cache.dense_k_pre()
    V = cache.dense_v()
    cos, sin = rope_cos_sin(inv_freq, torch.arange(S), attention_scaling)
    K = apply_rope(K, cos, sin)
    if k_tail is not None and k_tail.shape[1] > 0:
        K = torch.cat([K, k_tail.float()], dim=1)
        V = torch.cat([V, v_tail.float()], dim=1)
    return K, V


def k2b_naive_attention(q, cache: K2bOracleCache, inv_freq, k_tail, v_tail,
                        n_q_groups: int, scale: float, attention_scaling: float = 1.0):
    """The fp32 oracle for one decode step of one sequence: (n_q, 1, d)."""
    K, V = k2b_dense_kv(cache, inv_freq, k_tail, v_tail, attention_scaling)
    return naive_dense_attention(q, K, V, n_q_groups, scale)


def k2b_chunked_attention(q, cache: K2bOracleCache, inv_freq, k_tail, v_tail,
                          n_q_groups: int, scale: float, attention_scaling: float = 1.0):
    """Chunked dequant-attention for one decode step (chunked_attention.py:398-530):
    per committed page dequantize K and V, RoPE K at its positions, grouped
    online softmax; the fp16 tail is folded in last.  This is the reference's CPU
    path and the cpu_baseline of the benchmark."""
    n_q, n, d = q.shape
    h_kv = n_q // n_q_groups
    qf = q.float()
    acc = torch.zeros(n_q, n, d)
    m = torch.full((n_q, n, 1), float("-inf"))
    lse = torch.zeros(n_q, n, 1)

    def attend(K_kv, V_kv):
        nonlocal acc, m, lse
        qg = qf.view(h_kv, n_q_groups, n, d)
        s = torch.einsum("gpnd,gbd->gpnb", qg, K_kv) * scale
        s = s.reshape(n_q, n, K_kv.shape[1])
        m_new = torch.maximum(m, s.amax(dim=-1, keepdim=True))
        corr = torch.exp(m - m_new)
        p = torch.exp(s - m_new)
        lse = lse * corr + p.sum(dim=-1, keepdim=True)
        av = torch.einsum("gpnb,gbd->gpnd", p.view(h_kv, n_q_groups, n, -1), V_kv)
        acc = acc * corr + av.reshape(n_q, n, d)
        m = m_new

    for (kp, s0, s1), ((idx, norms), _, _) in zip(cache.k_blocks, cache.v_blocks):
        K_kv = C.from_matrix(C.dequant_k2b_key(kp, cache.group), h_kv)
        cos, sin = rope_cos_sin(inv_freq, torch.arange(s0, s1), attention_scaling)
        K_kv = apply_rope(K_kv, cos, sin)
        V_kv = C.from_matrix(C.dequant_v_perhead(idx, norms, bits=cache.v_bits,
                                                 seed=cache.v_seed, h=h_kv), h_kv)
        attend(K_kv, V_kv)
    if k_tail is not None and k_tail.shape[1] > 0:
        attend(k_tail.float(), v_tail.float())
    return acc / lse


class RtnOracleCache:
    """Committed RTN pages of one sequence -- post-RoPE keys and values, each a
    quantize_packed block dict (packed_streaming.py:640-667, 544-580):
    "rtn_token" values, and "rtn_token" or (k_arm 1) "rtn_channel" keys
    (codecs.py:720-725; rtn.py:23-44) -- and their dequantization as the
    reference's fused RTN path computes it: code times the fp16 scale of its
    group, the scale stacked in fp16 by build_kv_stacked_packed
    (triton_dequant_attention.py:1436-1440), read in fp32 by the kernel
    (:670-715).  Channel-arm keys have no fused path in the reference, whose
    chunked path reads them with the fp32 scale (codecs.py:819-822); the
    pages carry that scale as the fp16 pair hi + lo (layout.scale_pair), so
    their page scale is float32(hi) + float32(lo)."""

    def __init__(self, h_kv: int, *, k_bits: int, v_bits: int, k_group: int, v_group: int,
                 k_arm: int = 0, page: int = 128):
        self.h_kv, self.page, self.k_arm = h_kv, page, k_arm
        self.k_bits, self.v_bits, self.k_group, self.v_group = k_bits, v_bits, k_group, v_group
        self.k_blocks: list = []
        self.v_blocks: list = []

    @property
    def n_tokens(self) -> int:
        return len(self.k_blocks) * self.page

    def commit(self, k_page: torch.Tensor, v_page: torch.Tensor):
        """k_page, v_page: (h_kv, page, d) post-RoPE keys / values (any float dtype)."""
        quant_k = C.quantize_rtn_channel if self.k_arm == 1 else C.quantize_rtn_token
        kp, _ = quant_k(C.to_matrix(k_page.float()), self.k_bits, self.k_group)
        vp, _ = C.quantize_rtn_token(C.to_matrix(v_page.float()), self.v_bits, self.v_group)
        s = self.n_tokens
        self.k_blocks.append((kp, s, s + self.page))
        self.v_blocks.append((vp, s, s + self.page))

    def _dense(self, blocks, group, fp16_scales, channel=False):
        out = []
        for p, _, _ in blocks:
            if not fp16_scales:
                sc = p["scale"]
            elif channel:   # the page's hi + lo pair of the fp32 scale
                hi = p["scale"].half().float()
                sc = hi + (p["scale"] - hi).half().float()
            else:
                sc = p["scale"].half().float()
            M = C.rtn_dequantize_packed(p["Q_int"], sc, group)   # (C, S) for the channel arm
            out.append(C.from_matrix(M.mT if channel else M, self.h_kv))
        return torch.cat(out, dim=1)

    def dense_kv(self, fp16_scales: bool = True):
        """(K (h_kv, S, d), V (h_kv, S, d)) fp32; fp16_scales: with the scales
        the pages hold (fp16, or the hi + lo pair for channel-arm keys), else
        with the codec's fp32 scales."""
        return (self._dense(self.k_blocks, self.k_group, fp16_scales, self.k_arm == 1),
                self._dense(self.v_blocks, self.v_group, fp16_scales))

    def codes(self):
        """(kq, ks, vq, vs): codes (h_kv, S, d) and fp32 scales -- (h_kv, S,
        d/group) per (token, channel group), or for channel-arm keys (h_kv,
        S/group, d) per (token group, channel)."""
        def per_head(blocks, channel=False):
            tr = (lambda x: x.mT) if channel else (lambda x: x)
            q = torch.cat([C.from_matrix(tr(p["Q_int"]), self.h_kv) for p, _, _ in blocks], dim=1)
            s = torch.cat([C.from_matrix(tr(p["scale"].squeeze(-1)), self.h_kv) for p, _, _ in blocks], dim=1)
            return q, s
        kq, ks = per_head(self.k_blocks, self.k_arm == 1)
        vq, vs = per_head(self.v_blocks)
        return kq, ks, vq, vs


def rtn_chunked_attention(q, cache: RtnOracleCache, k_tail, v_tail, n_q_groups: int, scale: float):
    """Chunked dequant-attention for one decode step over RTN pages
    (chunked_attention.py:398-530 with dequant_packed of the RTN arms,
    codecs.py:819-822, fp32 scales): per committed page dequantize K and V,
    grouped online softmax, the fp16 tail folded in last.  The reference's CPU
    path for these arms and the cpu_baseline of the RTN benchmark."""
    n_q, n, d = q.shape
    h_kv = n_q // n_q_groups
    qf = q.float()
    acc = torch.zeros(n_q, n, d)
    m = torch.full((n_q, n, 1), float("-inf"))
    lse = torch.zeros(n_q, n, 1)

    def attend(K_kv, V_kv):
        nonlocal acc, m, lse
        qg = qf.view(h_kv, n_q_groups, n, d)
        s = torch.einsum("gpnd,gbd->gpnb", qg, K_kv) * scale
        s = s.reshape(n_q, n, K_kv.shape[1])
        m_new = torch.maximum(m, s.amax(dim=-1, keepdim=True))
        corr = torch.exp(m - m_new)
        p = torch.exp(s - m_new)
        lse = lse * corr + p.sum(dim=-1, keepdim=True)
        av = torch.einsum("gpnb,gbd->gpnd", p.view(h_kv, n_q_groups, n, -1), V_kv)
        acc = acc * corr + av.reshape(n_q, n, d)
        m = m_new

    dq_k = C.dequant_rtn_channel if cache.k_arm == 1 else C.dequant_rtn_token
    for (kp, _, _), (vp, _, _) in zip(cache.k_blocks, cache.v_blocks):
        attend(C.from_matrix(dq_k(kp, cache.k_group), h_kv),
               C.from_matrix(C.dequant_rtn_token(vp, cache.v_group), h_kv))
    if k_tail is not None and k_tail.shape[1] > 0:
        attend(k_tail.float(), v_tail.float())
    return acc / lse


def rtn_naive_attention(q, cache: RtnOracleCache, k_tail, v_tail, n_q_groups: int, scale: float):
    """The fp32 oracle for one decode step over committed RTN pages plus the
    fp16 tail: (n_q, 1, d)."""
    K, V = cache.dense_kv()
    if k_tail is not None and k_tail.shape[1] > 0:
        K = torch.cat([K, k_tail.float()], dim=1)
        V = torch.cat([V, v_tail.float()], dim=1)
    return naive_dense_attention(q, K, V, n_q_groups, scale)

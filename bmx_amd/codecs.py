"""Codec constants of the k2b recipe, computed on the host once per process.

The write and decode kernels take the V codec's Lloyd codebook, its Hadamard
signs and the RoPE inverse frequencies as plain numbers; this module derives
them exactly as the reference defines them:
  * gaussian_codebook      cache/codecs.py:346-380 (seeded 2^18-sample Lloyd)
  * hadamard_signs         cache/codecs.py:114-124 (seeded torch.randint)
  * rope inverse frequencies: transformers' rope initialisation, as
    cache/rope.py:19-58 builds them through LlamaRotaryEmbedding.
"""

from __future__ import annotations

import functools
import math

import torch


@functools.lru_cache(maxsize=16)
def gaussian_codebook(bits: int, n_samples: int = 2**18, n_iter: int = 40,
                      seed: int = 0) -> tuple:
    """Sorted 1-D Lloyd-Max levels for N(0,1) as Python floats (fp32 values)."""
    n_levels = 2**bits
    gen = torch.Generator().manual_seed(seed)
    x = torch.randn(n_samples, generator=gen)
    levels = torch.quantile(x, torch.linspace(0, 1, n_levels + 2)[1:-1])
    for _ in range(n_iter):
        cell = torch.bucketize(x, (levels[:-1] + levels[1:]) / 2)
        nxt = levels.clone()
        for k in range(n_levels):
            sel = cell == k
            if sel.any():
                nxt[k] = x[sel].mean()
        levels = nxt
    return tuple(float(v) for v in levels.sort().values)


@functools.lru_cache(maxsize=32)
def hadamard_signs(d: int, seed: int) -> tuple:
    gen = torch.Generator().manual_seed(seed)
    return tuple(int(v) for v in (torch.randint(0, 2, (d,), generator=gen) * 2 - 1))


def sign_bits(signs) -> list:
    """+-1 vector -> uint32 words (at least 4), bit c of word c // 32 set where
    the sign is -1."""
    words = [0] * max(4, -(-len(signs) // 32))
    for c, s in enumerate(signs):
        if s < 0:
            words[c >> 5] |= 1 << (c & 31)
    return words


def rope_inv_freq(config=None, *, head_dim: int = 128, theta: float = 10000.0):
    """(inv_freq fp32 tensor (head_dim/2,), attention_scaling) for a HF config (any
    rope type transformers knows), or the default rope at ``theta``."""
    if config is not None:
        from transformers.models.llama.modeling_llama import LlamaRotaryEmbedding

        emb = LlamaRotaryEmbedding(config=config)
        return emb.inv_freq.detach().float().cpu(), float(emb.attention_scaling)
    exps = torch.arange(0, head_dim, 2, dtype=torch.int64).to(dtype=torch.float) / head_dim
    return 1.0 / (theta ** exps), 1.0


def bpe_k(rank: int, C: int, *, bits: int = 3, group: int = 64, page: int = 128) -> float:
    """Honest key bits per entry of one committed codec page
    (codecs.py:79-96): bits + 16/group + 16 r (S + C) / (S C)."""
    return bits + 16.0 / group + 16.0 * rank * (page + C) / (page * C)


def bpe_v(h: int, C: int, *, bits: int = 2) -> float:
    """Honest value bits per entry: bits + 16 h / C (codecs.py:734-745)."""
    return bits + 16.0 * h / C


def compute_flush_schedule(S: int, W: int, g: int) -> int:
    """Largest multiple of g leaving >= W recent fp16 tokens (streaming.py:144-151)."""
    return ((S - W) // g) * g if S > W else 0


SQRT_D = math.sqrt(128)

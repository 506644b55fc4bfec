"""Synthetic k2b workloads (the BASELINE configurations) and a device page pool.

Keys follow the configs' generator: per KV head a seeded-QR orthonormal basis
U (d x r, diag(R) >= 0 as quant/hadamard.py:36-46 canonicalises), coefficients
c_i ~ N(0, i^-0.7) and a N(0, 0.05^2) residual: K_pre = c U^T + e.  Values are
N(0, 1) (a Hadamard rotation of N(0, 1) is N(0, 1) again).  Everything is drawn
from a seeded CPU generator so a CPU checker can rebuild the same inputs.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import torch

from . import k2b

D = 128


def k2b_keys(h_kv: int, S: int, rank: int, gen: torch.Generator, *, res_std: float = 0.05,
             basis_rank: int | None = None, head_dim: int = D) -> torch.Tensor:
    """(h_kv, S, head_dim) fp16 pre-RoPE keys of rank-``basis_rank`` structure +
    noise (at most head_dim directions per head), on the generator's device."""
    br = min(basis_rank or rank, head_dim)
    dev = gen.device
    out = torch.empty(h_kv, S, head_dim, dtype=torch.float16, device=dev)
    std = (torch.arange(1, br + 1, dtype=torch.float32) ** (-0.35)).to(dev)
    for h in range(h_kv):
        Q, R = torch.linalg.qr(torch.randn(head_dim, br, generator=gen, device=dev).cpu())
        sgn = torch.sign(torch.diagonal(R))
        sgn[sgn == 0] = 1
        U = (Q * sgn).to(dev)
        c = torch.randn(S, br, generator=gen, device=dev) * std
        out[h] = (c @ U.T + res_std * torch.randn(S, head_dim, generator=gen, device=dev)).half()
    return out


def values(h_kv: int, S: int, gen: torch.Generator, head_dim: int = D) -> torch.Tensor:
    return torch.randn(h_kv, S, head_dim, generator=gen, device=gen.device).half()


def rope_keys(k_pre: torch.Tensor, start: int, consts: k2b.CodecConsts) -> torch.Tensor:
    """Post-RoPE fp16 keys of positions [start, start + n) from fp16 pre-RoPE keys,
    with HF's fp32 tables (angle fl32(inv_freq * pos)) — the recent-window slab."""
    dev = k_pre.device
    n = k_pre.shape[1]
    inv = torch.tensor(consts.inv_freq, dtype=torch.float32, device=dev)
    ang = inv[None, :] * torch.arange(start, start + n, device=dev, dtype=torch.float32)[:, None]
    emb = torch.cat((ang, ang), dim=-1)
    cos, sin = emb.cos() * consts.rope_scaling, emb.sin() * consts.rope_scaling
    x = k_pre.float()
    d = x.shape[-1]
    rot = torch.cat((-x[..., d // 2:], x[..., :d // 2]), dim=-1)
    return (x * cos + rot * sin).half()


def first_page_svd(k_pre: torch.Tensor, rank: int):
    """Frozen subspace from the first 128-token codec page, as
    PackedStreamingLayer._pack_k_block does (packed_streaming.py:513-516):
    (Us (128, r) fp32, V (C, r) fp32) of the truncated SVD of M = to_matrix."""
    h_kv = k_pre.shape[0]
    M = k_pre[:, :128].float().permute(1, 0, 2).reshape(128, h_kv * k_pre.shape[2]).cpu()
    U, s, Vh = torch.linalg.svd(M, full_matrices=False)
    return U[:, :rank] * s[:rank], Vh[:rank, :].mT.contiguous()


class PagePool:
    """Fixed-capacity device pool of physical pages with a host free list."""

    def __init__(self, n_pages: int, h_kv: int, rank: int, device, *, gen: torch.Generator | None = None,
                 head_dim: int = D, group: int = 64, k_bits: int = 3):
        self.h_kv, self.rank = h_kv, rank
        self.head_dim, self.group, self.k_bits = head_dim, group, k_bits
        self.page_bytes = k2b.page_bytes(h_kv, rank, head_dim=head_dim, group=group, k_bits=k_bits)
        self.pages = torch.zeros(n_pages, self.page_bytes, dtype=torch.uint8, device=device)
        order = torch.randperm(n_pages, generator=gen) if gen is not None else torch.arange(n_pages)
        self.free = order.tolist()[::-1]

    def alloc(self, n: int) -> list:
        if n > len(self.free):
            raise RuntimeError(f"page pool exhausted: need {n}, have {len(self.free)}")
        return [self.free.pop() for _ in range(n)]

    def release(self, ids) -> None:
        self.free.extend(int(i) for i in ids)


@dataclass
class PackedSeq:
    """One sequence of one layer in packed form on the device."""

    page_ids: list = field(default_factory=list)
    packed_len: int = 0
    basis32: torch.Tensor | None = None
    basis16: torch.Tensor | None = None


def encode_sequence(pool: PagePool, k_pre: torch.Tensor, v: torch.Tensor, rank: int,
                    consts: k2b.CodecConsts, svd=None, *, chunk_pages: int = 256) -> PackedSeq:
    """Quantize-on-append every full 128-token codec page of (k_pre, v) (device fp16,
    (h_kv, S, head_dim)) with the HIP write kernel, in the pool's geometry.  ``svd`` = (Us, V) of the first page;
    computed from k_pre when omitted."""
    dev = pool.pages.device
    h_kv, S, _ = k_pre.shape
    n_cp = S // 128
    if svd is None:
        svd = first_page_svd(k_pre, rank)
    us0, V = svd
    seq = PackedSeq(basis32=V.to(dev).float().contiguous(),
                    basis16=V.to(dev).half().contiguous())
    for c0 in range(0, n_cp, chunk_pages):
        c1 = min(n_cp, c0 + chunk_pages)
        ids = pool.alloc(8 * (c1 - c0))
        seq.page_ids.extend(ids)
        k2b.append(k_pre[:, c0 * 128:c1 * 128], v[:, c0 * 128:c1 * 128], seq.basis32, seq.basis16,
                   pool.pages, torch.tensor(ids, dtype=torch.int32, device=dev), consts, rank=rank,
                   us_first=us0.to(dev).float().contiguous() if c0 == 0 else None, group=pool.group,
                   k_bits=pool.k_bits)
    seq.packed_len = n_cp * 128
    return seq


def page_table(seqs, max_pages: int | None = None, device=None) -> torch.Tensor:
    mp = max_pages or max(1, max(len(s.page_ids) for s in seqs))
    t = torch.zeros(len(seqs), mp, dtype=torch.int32)
    for i, s in enumerate(seqs):
        t[i, :len(s.page_ids)] = torch.tensor(s.page_ids, dtype=torch.int32)
    return t.to(device)

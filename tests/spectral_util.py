"""Spectral packs for the tests: the reference-fitted pack of the golden
fixture, and seeded synthetic packs of the reference's form (enc = W^1/2 E,
dec = W^-1/2 E for an orthonormal E and a positive diagonal W, bits from the
allocator on a power-law spectrum whose keys have unit variance per element
on average, as model keys have a few units of norm per head)."""

from pathlib import Path

import numpy as np
import torch

from bmx_amd import spectral

GOLD = Path(__file__).parent / "golden"


def golden_pack():
    """(pack, M): the pack the reference fitted (C 256, budget 2.5) and its keys."""
    g = np.load(GOLD / "spectral.npz")
    pack = spectral.SpectralPack(enc=torch.from_numpy(g["enc"]), dec=torch.from_numpy(g["dec"]),
                                 lam=torch.from_numpy(g["lam64"]).float(),
                                 bits=torch.from_numpy(g["bits_b2.5"]), budget=2.5)
    return pack, g["M"].astype(np.float32)


def synthetic_pack(h_kv: int, budget: float, seed: int) -> spectral.SpectralPack:
    C = 128 * h_kv
    g = torch.Generator().manual_seed(seed)
    E, _ = torch.linalg.qr(torch.randn(C, C, generator=g, dtype=torch.float64))
    w = 0.5 + torch.rand(C, generator=g, dtype=torch.float64)
    lam = torch.arange(1, C + 1, dtype=torch.float64) ** -2.0
    lam *= C / lam.sum()          # unit variance per key element on average
    enc = (w.sqrt()[:, None] * E).float()
    dec = (w.rsqrt()[:, None] * E).float()
    return spectral.SpectralPack(enc=enc, dec=dec, lam=lam.float(),
                                 bits=spectral.allocate_bits(lam, budget), budget=budget)


def synthetic_keys(pack: spectral.SpectralPack, S: int, seed: int) -> np.ndarray:
    """(S, C) fp32 keys whose codes Y = M enc have variance lam per direction."""
    g = torch.Generator().manual_seed(seed)
    C = pack.enc.shape[0]
    Z = torch.randn(S, C, generator=g, dtype=torch.float64) * pack.lam.double().sqrt()
    return (Z @ pack.dec.double().T).float().numpy()

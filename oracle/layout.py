"""numpy packer / unpacker for this build's 16-token physical page (test only).

There is no reference counterpart for these bytes: the reference keeps one
stacked tensor per field (triton_dequant_attention.py:1118-1229).  This module
restates the page format the HIP write kernel produces (bmx_amd/csrc, described
in include/bmx_k2b.h), independently of the kernel, so the kernel's output bytes
can be checked exactly and decode-kernel inputs can be built on the CPU.

Page of PT=16 tokens for one layer, head_dim 128, C = 128*h_kv channels,
rank R.  Sections in order (all little-endian):
  US     [16][R] fp16                      low-rank coefficients Us per token
  VNORM  [h_kv][16] fp16                   value norm per (head, token)
  KSCALE [C/4] fp16                        slot j = (page index mod 4) of the
                                           page's 64-token scale group holds the
                                           group scales of channels [jC/4,(j+1)C/4)
  KRES   [h_kv][64 lanes][3 x u32]         3-bit two's-complement key residual
         lane = 16q + n (token n, quarter q); code k=4b+i (b<8, i<4) is channel
         16b + 4q + i of the head, at bits [3k, 3k+3) of the 96-bit lane string
  VCODE  [h_kv][64 lanes][2 x u32]         2-bit value codes
         lane = 16q + m; dword w holds channel 16b + m, b = 4w + bb (bb<4), for
         token 4q + t (t<4) at bit 16*(t&1) + 4*bb + 2*(t>>1)
"""

from __future__ import annotations

import numpy as np

PT = 16          # tokens per physical page
GROUP = 64       # tokens per key-scale group (4 pages)
CODEC_PAGE = 128  # tokens per codec page (8 physical pages)
D = 128          # head_dim


def sections(h_kv: int, rank: int) -> dict:
    C = D * h_kv
    sizes = [("us", PT * rank * 2), ("vnorm", h_kv * PT * 2), ("kscale", C // 4 * 2),
             ("kres", h_kv * 64 * 12), ("vcode", h_kv * 64 * 8)]
    off, out = 0, {}
    for name, sz in sizes:
        out[name] = (off, sz)
        off += sz
    out["total"] = (0, off)
    return out


def page_bytes(h_kv: int, rank: int) -> int:
    return sections(h_kv, rank)["total"][1]


def _kres_index(h_kv: int):
    """channel index (within head) for [q, k] lane-string slots."""
    q = np.arange(4)[:, None]
    k = np.arange(32)[None, :]
    return 16 * (k // 4) + 4 * q + (k % 4)  # (4, 32)


def pack_pages(us16, res, scale16, vidx, vnorm16, h_kv: int, rank: int) -> np.ndarray:
    """Logical codec outputs of T tokens (T multiple of 64) -> (T/16, page_bytes) u8.

    us16    (T, R)       fp16 values
    res     (C, T)       int in [-4, 3]  (per-channel residual codes, tokens last)
    scale16 (C, T/64)    fp16 group scales
    vidx    (T, C)       int in [0, 3]
    vnorm16 (T, h_kv)    fp16 norms
    """
    T = us16.shape[0]
    assert T % GROUP == 0
    C = D * h_kv
    n_pages = T // PT
    sec = sections(h_kv, rank)
    out = np.zeros((n_pages, sec["total"][1]), dtype=np.uint8)
    us16 = np.asarray(us16, dtype=np.float16)
    res = np.asarray(res).astype(np.int64)
    vidx = np.asarray(vidx).astype(np.int64)
    scale16 = np.asarray(scale16, dtype=np.float16)
    vnorm16 = np.asarray(vnorm16, dtype=np.float16)
    chan = _kres_index(h_kv)  # (4, 32)
    for p in range(n_pages):
        t0 = p * PT
        o, s = sec["us"]
        out[p, o:o + s] = us16[t0:t0 + PT].reshape(-1).view(np.uint8)
        o, s = sec["vnorm"]
        out[p, o:o + s] = np.ascontiguousarray(vnorm16[t0:t0 + PT].T).reshape(-1).view(np.uint8)
        o, s = sec["kscale"]
        g, j = p // 4, p % 4
        out[p, o:o + s] = np.ascontiguousarray(
            scale16[j * C // 4:(j + 1) * C // 4, g]).view(np.uint8)
        # KRES
        o, s = sec["kres"]
        kres = np.zeros((h_kv, 4, PT, 3), dtype=np.uint64)
        for h in range(h_kv):
            # codes[q, n, k] = res[h*128 + chan[q,k], t0+n]
            codes = res[h * D + chan[:, None, :], t0 + np.arange(PT)[None, :, None]] & 7
            for k in range(32):
                bit = 3 * k
                w, sh = bit // 32, bit % 32
                val = codes[:, :, k].astype(np.uint64)
                kres[h, :, :, w] |= (val << np.uint64(sh)) & np.uint64(0xFFFFFFFF)
                if sh > 29:
                    kres[h, :, :, w + 1] |= val >> np.uint64(32 - sh)
        out[p, o:o + s] = kres.astype(np.uint32).reshape(-1).view(np.uint8)
        # VCODE
        o, s = sec["vcode"]
        vc = np.zeros((h_kv, 4, 16, 2), dtype=np.uint64)
        for h in range(h_kv):
            for b in range(8):
                w, bb = b // 4, b % 4
                # codes[q, t, m] of channel 16b+m, token t0 + 4q + t
                cm = vidx[t0:t0 + PT, h * D + 16 * b + np.arange(16)].reshape(4, 4, 16)
                for t in range(4):
                    sh = 16 * (t & 1) + 4 * bb + 2 * (t >> 1)
                    vc[h, :, :, w] |= cm[:, t, :].astype(np.uint64) << np.uint64(sh)
        out[p, o:o + s] = vc.astype(np.uint32).reshape(-1).view(np.uint8)
    return out


def unpack_pages(pages: np.ndarray, h_kv: int, rank: int):
    """Inverse of pack_pages for a run of consecutive pages (count multiple of 4)."""
    pages = np.asarray(pages, dtype=np.uint8)
    n_pages = pages.shape[0]
    T = n_pages * PT
    C = D * h_kv
    sec = sections(h_kv, rank)
    us16 = np.zeros((T, rank), dtype=np.float16)
    vnorm16 = np.zeros((T, h_kv), dtype=np.float16)
    scale16 = np.zeros((C, T // GROUP), dtype=np.float16)
    res = np.zeros((C, T), dtype=np.int8)
    vidx = np.zeros((T, C), dtype=np.int16)
    chan = _kres_index(h_kv)
    for p in range(n_pages):
        t0 = p * PT
        o, s = sec["us"]
        us16[t0:t0 + PT] = pages[p, o:o + s].view(np.float16).reshape(PT, rank)
        o, s = sec["vnorm"]
        vnorm16[t0:t0 + PT] = pages[p, o:o + s].view(np.float16).reshape(h_kv, PT).T
        o, s = sec["kscale"]
        g, j = p // 4, p % 4
        if g < scale16.shape[1]:
            scale16[j * C // 4:(j + 1) * C // 4, g] = pages[p, o:o + s].view(np.float16)
        o, s = sec["kres"]
        kres = pages[p, o:o + s].view(np.uint32).reshape(h_kv, 4, PT, 3).astype(np.uint64)
        for k in range(32):
            bit = 3 * k
            w, sh = bit // 32, bit % 32
            val = kres[..., w] >> np.uint64(sh)
            if sh > 29:
                val |= kres[..., w + 1] << np.uint64(32 - sh)
            val = (val & np.uint64(7)).astype(np.int64)
            val = np.where(val >= 4, val - 8, val)  # sign-extend 3 bits
            for h in range(h_kv):
                res[h * D + chan[:, k][:, None], t0 + np.arange(PT)[None, :]] = val[h]
        o, s = sec["vcode"]
        vc = pages[p, o:o + s].view(np.uint32).reshape(h_kv, 4, 16, 2).astype(np.int64)
        for h in range(h_kv):
            for b in range(8):
                w, bb = b // 4, b % 4
                for t in range(4):
                    sh = 16 * (t & 1) + 4 * bb + 2 * (t >> 1)
                    vidx[t0 + 4 * np.arange(4)[:, None] + t,
                         h * D + 16 * b + np.arange(16)[None, :]] = (vc[h, :, :, w] >> sh) & 3
    return us16, res, scale16, vidx, vnorm16

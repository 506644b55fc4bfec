"""numpy packer / unpacker for this build's 16-token physical page (test only).

There is no reference counterpart for these bytes: the reference keeps one
stacked tensor per field (triton_dequant_attention.py:1118-1229).  This module
restates the page format the HIP write kernel produces (bmx_amd/csrc, described
in include/bmx_k2b.h), independently of the kernel, so the kernel's output bytes
can be checked exactly and decode-kernel inputs can be built on the CPU.

Page of PT=16 tokens for one layer, head_dim 128, C = 128*h_kv channels,
rank R.  Sections in order (all little-endian):
  US     [4][16][R/4] fp16      US[q][n][i] = Us[token n][(R/4)*q + i]
  VNORM  [h_kv][16] fp16        value norm per (head, token)
  KSCALE [C/4] fp16             the 64-token group's C scales in pair order
                                F[128h + 2j + e] = scale(channel 128h + j + 64e),
                                j < 64, e < 2; page slot s (= page index mod 4)
                                holds F[s*C/4, (s+1)*C/4)
  KRES   [h_kv][64][3] u32      lane 16q+n = token n; pair p = 4b+i (b, i < 4)
                                is channels (j, j+64), j = 16b + 4q + i, codes
                                stored offset-binary (code + 4, 3 bits); pair
                                p < 15: dword p // 5, low code at bit 3*(p % 5),
                                high code at bit 16 + 3*(p % 5); pair 15: bit k
                                of the low / high code at bit 15 / 31 of dword k
  VCODE  [h_kv][64][2] u32      lane 16q+m; the code of channel 16b + m (b < 8),
                                token 4q + t (t < 4) at dword b // 4, bit
                                8*(b % 4) + 2*t
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


def kscale_flat_index(h_kv: int) -> np.ndarray:
    """F position of each channel c (0..C-1) in the group's KSCALE order."""
    c = np.arange(D * h_kv)
    h, j = c // D, c % D
    return D * h + 2 * (j % 64) + j // 64


def kres_slots():
    """(dword, bit) of the low code of pair p < 15 (the high code is at bit + 16)."""
    p = np.arange(15)
    return p // 5, 3 * (p % 5)


def _pair_channels():
    """channel j (< 64) of pair p for lane quarter q: (4, 16) array."""
    q = np.arange(4)[:, None]
    p = np.arange(16)[None, :]
    return 16 * (p // 4) + 4 * q + (p % 4)


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
    R = rank
    n_pages = T // PT
    sec = sections(h_kv, rank)
    out = np.zeros((n_pages, sec["total"][1]), dtype=np.uint8)
    us16 = np.asarray(us16, dtype=np.float16)
    res = np.asarray(res).astype(np.int64)
    vidx = np.asarray(vidx).astype(np.int64)
    scale16 = np.asarray(scale16, dtype=np.float16)
    vnorm16 = np.asarray(vnorm16, dtype=np.float16)
    fpos = kscale_flat_index(h_kv)
    chan = _pair_channels()                      # (4, 16)
    dw, sh = kres_slots()
    for p in range(n_pages):
        t0 = p * PT
        tok = t0 + np.arange(PT)
        o, s = sec["us"]
        us = us16[t0:t0 + PT].reshape(PT, 4, R // 4).transpose(1, 0, 2)
        out[p, o:o + s] = np.ascontiguousarray(us).reshape(-1).view(np.uint8)
        o, s = sec["vnorm"]
        out[p, o:o + s] = np.ascontiguousarray(vnorm16[t0:t0 + PT].T).reshape(-1).view(np.uint8)
        o, s = sec["kscale"]
        g, j = p // 4, p % 4
        flat = np.zeros(C, dtype=np.float16)
        flat[fpos] = scale16[:, g]
        out[p, o:o + s] = np.ascontiguousarray(flat[j * C // 4:(j + 1) * C // 4]).view(np.uint8)
        # KRES
        o, s = sec["kres"]
        kres = np.zeros((h_kv, 4, PT, 3), dtype=np.uint64)
        for h in range(h_kv):
            # lo[q, n, p] = code of channel chan[q, p], hi: channel + 64; offset-binary
            lo = (res[h * D + chan[:, None, :], tok[None, :, None]] + 4).astype(np.uint64)
            hi = (res[h * D + 64 + chan[:, None, :], tok[None, :, None]] + 4).astype(np.uint64)
            for pp in range(15):
                kres[h, :, :, dw[pp]] |= (lo[:, :, pp] << np.uint64(sh[pp])) | \
                    (hi[:, :, pp] << np.uint64(16 + sh[pp]))
            for k in range(3):
                kres[h, :, :, k] |= (((lo[:, :, 15] >> np.uint64(k)) & np.uint64(1)) << np.uint64(15)) | \
                    (((hi[:, :, 15] >> np.uint64(k)) & np.uint64(1)) << np.uint64(31))
        out[p, o:o + s] = kres.astype(np.uint32).reshape(-1).view(np.uint8)
        # VCODE
        o, s = sec["vcode"]
        vc = np.zeros((h_kv, 4, 16, 2), dtype=np.uint64)
        for h in range(h_kv):
            for b in range(8):
                # cm[q, t, m]: channel 16b + m, token t0 + 4q + t
                cm = vidx[t0:t0 + PT, h * D + 16 * b + np.arange(16)].reshape(4, 4, 16)
                for t in range(4):
                    vc[h, :, :, b // 4] |= cm[:, t, :].astype(np.uint64) << np.uint64(8 * (b % 4) + 2 * t)
        out[p, o:o + s] = vc.astype(np.uint32).reshape(-1).view(np.uint8)
    return out


def unpack_pages(pages: np.ndarray, h_kv: int, rank: int):
    """Inverse of pack_pages for a run of consecutive pages (count multiple of 4)."""
    pages = np.asarray(pages, dtype=np.uint8)
    n_pages = pages.shape[0]
    T = n_pages * PT
    C = D * h_kv
    R = rank
    sec = sections(h_kv, rank)
    us16 = np.zeros((T, rank), dtype=np.float16)
    vnorm16 = np.zeros((T, h_kv), dtype=np.float16)
    scale16 = np.zeros((C, T // GROUP), dtype=np.float16)
    res = np.zeros((C, T), dtype=np.int8)
    vidx = np.zeros((T, C), dtype=np.int16)
    fpos = kscale_flat_index(h_kv)
    chan = _pair_channels()
    dw, sh = kres_slots()
    for p in range(n_pages):
        t0 = p * PT
        tok = t0 + np.arange(PT)
        o, s = sec["us"]
        us16[t0:t0 + PT] = pages[p, o:o + s].view(np.float16).reshape(4, PT, R // 4) \
            .transpose(1, 0, 2).reshape(PT, R)
        o, s = sec["vnorm"]
        vnorm16[t0:t0 + PT] = pages[p, o:o + s].view(np.float16).reshape(h_kv, PT).T
        o, s = sec["kscale"]
        g, j = p // 4, p % 4
        if g < scale16.shape[1]:
            sl = pages[p, o:o + s].view(np.float16)
            sel = (fpos >= j * C // 4) & (fpos < (j + 1) * C // 4)
            scale16[sel, g] = sl[fpos[sel] - j * C // 4]
        o, s = sec["kres"]
        kres = pages[p, o:o + s].view(np.uint32).reshape(h_kv, 4, PT, 3).astype(np.int64)
        lo = np.zeros((h_kv, 4, PT, 16), dtype=np.int64)
        hi = np.zeros_like(lo)
        for pp in range(15):
            lo[..., pp] = (kres[..., dw[pp]] >> sh[pp]) & 7
            hi[..., pp] = (kres[..., dw[pp]] >> (16 + sh[pp])) & 7
        for k in range(3):
            lo[..., 15] |= ((kres[..., k] >> 15) & 1) << k
            hi[..., 15] |= ((kres[..., k] >> 31) & 1) << k
        for h in range(h_kv):
            res[h * D + chan[:, None, :], tok[None, :, None]] = lo[h] - 4
            res[h * D + 64 + chan[:, None, :], tok[None, :, None]] = hi[h] - 4
        o, s = sec["vcode"]
        vc = pages[p, o:o + s].view(np.uint32).reshape(h_kv, 4, 16, 2).astype(np.int64)
        for h in range(h_kv):
            for b in range(8):
                for t in range(4):
                    vidx[t0 + 4 * np.arange(4)[:, None] + t,
                         h * D + 16 * b + np.arange(16)[None, :]] = \
                        (vc[h, :, :, b // 4] >> (8 * (b % 4) + 2 * t)) & 3
    return us16, res, scale16, vidx, vnorm16


# ---------------------------------------------------------------------------
# The general k2b page (include/bmx_k2b.h, "General geometry"): head_dim d,
# rank R, residual group NG, key bits b; sections 16-byte aligned:
#   US [16][R] fp16, VNORM [h][16] fp16, KSCALE [C*16/NG] fp16 (slot s = page
#   mod NG/16 holds scales [s C 16/NG, (s+1) C 16/NG)), KRES [h][16][d/2] u8
#   (offset-binary nibbles, even channel low), VCODE [h][4][d] u8 (byte (a, j):
#   tokens 4a..4a+3 of channel j at bits 2t).
# ---------------------------------------------------------------------------


def _a16(x: int) -> int:
    return (x + 15) & ~15


def general_sections(h_kv: int, rank: int, d: int, group: int) -> dict:
    C = d * h_kv
    per_slot = C // (group // PT)
    sizes = [("us", PT * rank * 2), ("vnorm", h_kv * PT * 2), ("kscale", per_slot * 2),
             ("kres", h_kv * PT * (d // 2)), ("vcode", h_kv * 4 * d)]
    off, out = 0, {}
    for name, sz in sizes:
        out[name] = (off, sz)
        off = _a16(off + sz)
    out["total"] = (0, off)
    return out


def pack_general(us16, res, scale16, vidx, vnorm16, h_kv: int, rank: int, d: int, group: int,
                 bits: int) -> np.ndarray:
    """Logical codec outputs of T tokens (T multiple of group) -> (T/16,
    page_bytes) u8 general pages; arguments as pack_pages (scale16 (C, T/group))."""
    T = us16.shape[0]
    assert T % group == 0
    C = d * h_kv
    slots = group // PT
    per = C // slots
    sec = general_sections(h_kv, rank, d, group)
    out = np.zeros((T // PT, sec["total"][1]), dtype=np.uint8)
    res = np.asarray(res).astype(np.int64) + (1 << (bits - 1))
    vidx = np.asarray(vidx).astype(np.int64)
    for p in range(T // PT):
        t0 = p * PT
        o, s = sec["us"]
        out[p, o:o + s] = np.ascontiguousarray(np.asarray(us16[t0:t0 + PT], np.float16)).reshape(-1).view(np.uint8)
        o, s = sec["vnorm"]
        out[p, o:o + s] = np.ascontiguousarray(np.asarray(vnorm16[t0:t0 + PT], np.float16).T).view(np.uint8).reshape(-1)
        o, s = sec["kscale"]
        slot = p % slots
        sc = np.asarray(scale16[:, t0 // group], np.float16)[slot * per:(slot + 1) * per]
        out[p, o:o + s] = np.ascontiguousarray(sc).view(np.uint8)
        o, s = sec["kres"]
        cr = res[:, t0:t0 + PT].T.reshape(PT, h_kv, d // 2, 2)          # (t, h, byte, nibble)
        by = (cr[..., 0] | (cr[..., 1] << 4)).transpose(1, 0, 2)        # (h, t, byte)
        out[p, o:o + s] = by.astype(np.uint8).reshape(-1)
        o, s = sec["vcode"]
        cv = vidx[t0:t0 + PT].reshape(4, 4, h_kv, d)                     # (a, t, h, j)
        vb = np.zeros((h_kv, 4, d), dtype=np.int64)
        for t in range(4):
            vb |= cv[:, t].transpose(1, 0, 2) << (2 * t)
        out[p, o:o + s] = vb.astype(np.uint8).reshape(-1)
    return out


def unpack_general(pages: np.ndarray, h_kv: int, rank: int, d: int, group: int, bits: int):
    """Inverse of pack_general for a run of consecutive pages (count a multiple
    of group / 16): (us16 (T, R), res (C, T), scale16 (C, T/group), vidx (T, C),
    vnorm16 (T, h))."""
    pages = np.asarray(pages, dtype=np.uint8)
    T = pages.shape[0] * PT
    C = d * h_kv
    slots = group // PT
    per = C // slots
    sec = general_sections(h_kv, rank, d, group)
    us16 = np.zeros((T, rank), dtype=np.float16)
    vnorm16 = np.zeros((T, h_kv), dtype=np.float16)
    scale16 = np.zeros((C, T // group), dtype=np.float16)
    res = np.zeros((C, T), dtype=np.int8)
    vidx = np.zeros((T, C), dtype=np.int16)
    for p in range(pages.shape[0]):
        t0 = p * PT
        o, s = sec["us"]
        us16[t0:t0 + PT] = pages[p, o:o + s].view(np.float16).reshape(PT, rank)
        o, s = sec["vnorm"]
        vnorm16[t0:t0 + PT] = pages[p, o:o + s].view(np.float16).reshape(h_kv, PT).T
        o, s = sec["kscale"]
        slot = p % slots
        scale16[slot * per:(slot + 1) * per, t0 // group] = pages[p, o:o + s].view(np.float16)
        o, s = sec["kres"]
        by = pages[p, o:o + s].reshape(h_kv, PT, d // 2).astype(np.int64)
        nib = np.stack([by & 15, by >> 4], axis=-1).reshape(h_kv, PT, d)   # (h, t, j)
        res[:, t0:t0 + PT] = (nib - (1 << (bits - 1))).transpose(0, 2, 1).reshape(C, PT)
        o, s = sec["vcode"]
        vb = pages[p, o:o + s].reshape(h_kv, 4, d).astype(np.int64)
        for t in range(4):
            vidx[t0 + 4 * np.arange(4)[:, None, None] + t, (np.arange(h_kv)[None, :, None] * d
                                                            + np.arange(d)[None, None, :])] = \
                ((vb >> (2 * t)) & 3).transpose(1, 0, 2)
    return us16, res, scale16, vidx, vnorm16


# ---------------------------------------------------------------------------
# RTN pages (include/bmx_rtn.h): 16 tokens, per head 4-bit offset-binary codes
# (code + 8) and fp16 scales of channel groups gk / gv (32, 64 or 128).
#   KSCALE [h][16 t][128/gk] fp16            token-arm keys
#          [2][h][4 b][4 q][8 j'] fp16       channel-arm keys: channel 32b + 8q + p(j'),
#                                            p = 0 4 1 5 2 6 3 7, scale of the page's token
#                                            group as hi = fp16(s) then lo = fp16(s - hi)
#   VSCALE [h][4 q][128/gv][4 i] fp16        token 4q + i
#   KCODE  [h][4 q][16 n][4 w] u32           channels 32w + 8q + j at nibble j
#   VCODE  [h][4 q][16 c][8 b] u16           channel 16b + c, token 4q + j at nibble j
# ---------------------------------------------------------------------------


def kchan_slot(c):
    """Position of channel c in a channel-arm KSCALE row."""
    j = c & 7
    return (c & ~7) + 2 * (j & 3) + (j >> 2)


def scale_pair(s):
    """fp32 scales -> (hi, lo) fp16 with hi = fp16(s), lo = fp16(s - hi)."""
    s = np.asarray(s, np.float32)
    hi = s.astype(np.float16)
    lo = (s - hi.astype(np.float32)).astype(np.float16)
    return hi, lo


def rtn_sections(h_kv: int, gk: int, gv: int, k_arm: int = 0) -> dict:
    ngk, ngv = 128 // gk, 128 // gv
    off = 0
    out = {}
    ksize = h_kv * 128 * 2 * 2 if k_arm == 1 else h_kv * 16 * ngk * 2
    for name, size in (("kscale", ksize), ("vscale", h_kv * 16 * ngv * 2),
                       ("kcode", h_kv * 1024), ("vcode", h_kv * 1024)):
        out[name] = (off, size)
        off += size
    return out


def rtn_page_bytes(h_kv: int, gk: int, gv: int, k_arm: int = 0) -> int:
    s = rtn_sections(h_kv, gk, gv, k_arm)
    return s["vcode"][0] + s["vcode"][1]


def pack_rtn_pages(kq, ks16, vq, vs16, h_kv: int, gk: int, gv: int, k_arm: int = 0) -> np.ndarray:
    """Codes and scales of T tokens (T multiple of 16) -> (T/16, page_bytes) u8.

    kq, vq   (h_kv, T, 128) int in [-8, 7]
    ks16     (h_kv, T, 128/gk) fp16, or for channel-arm keys (h_kv, T/gk, 128)
             fp32, stored as the pair scale_pair()
    vs16     (h_kv, T, 128/gv) fp16"""
    kq, vq = np.asarray(kq, np.int64), np.asarray(vq, np.int64)
    T = kq.shape[1]
    P = T // 16
    sec = rtn_sections(h_kv, gk, gv, k_arm)
    pages = np.zeros((P, rtn_page_bytes(h_kv, gk, gv, k_arm)), np.uint8)
    ngk, ngv = 128 // gk, 128 // gv
    slots = np.array([kchan_slot(c) for c in range(128)])
    for p in range(P):
        t0 = 16 * p
        o, n = sec["kscale"]
        if k_arm == 1:
            row = np.zeros((2, h_kv, 128), np.float16)
            row[0][:, slots], row[1][:, slots] = scale_pair(ks16[:, t0 // gk])
            pages[p, o:o + n] = row.view(np.uint8).ravel()
        else:
            pages[p, o:o + n] = np.ascontiguousarray(ks16[:, t0:t0 + 16].astype(np.float16)).view(np.uint8).ravel()
        o, n = sec["vscale"]
        vsc = vs16[:, t0:t0 + 16].astype(np.float16).reshape(h_kv, 4, 4, ngv).transpose(0, 1, 3, 2)
        pages[p, o:o + n] = np.ascontiguousarray(vsc).view(np.uint8).ravel()
        # keys: word (h, q, n, w) = channels 32w + 8q + j
        kc = (kq[:, t0:t0 + 16] + 8).reshape(h_kv, 16, 4, 4, 8)           # [h][n][w][q][j]
        words = (kc << (4 * np.arange(8))).sum(-1).astype(np.uint32)         # [h][n][w][q]
        o, n = sec["kcode"]
        pages[p, o:o + n] = np.ascontiguousarray(words.transpose(0, 3, 1, 2)).view(np.uint8).ravel()
        # values: cell (h, q, c, b) = channel 16b + c, tokens 4q + j
        vc = (vq[:, t0:t0 + 16] + 8).reshape(h_kv, 4, 4, 8, 16)           # [h][q][j][b][c]
        cells = (vc << (4 * np.arange(4))[None, None, :, None, None]).sum(2).astype(np.uint16)  # [h][q][b][c]
        o, n = sec["vcode"]
        pages[p, o:o + n] = np.ascontiguousarray(cells.transpose(0, 1, 3, 2)).view(np.uint8).ravel()
    return pages


def unpack_rtn_pages(pages: np.ndarray, h_kv: int, gk: int, gv: int, k_arm: int = 0):
    """Inverse of pack_rtn_pages: (kq, ks16, vq, vs16); channel-arm key scales
    come back per page as float32 hi + lo, (h_kv, P, 128)."""
    P = pages.shape[0]
    sec = rtn_sections(h_kv, gk, gv, k_arm)
    ngk, ngv = 128 // gk, 128 // gv
    kq = np.zeros((h_kv, 16 * P, 128), np.int64)
    vq = np.zeros_like(kq)
    ks = np.zeros((h_kv, P, 128), np.float32) if k_arm == 1 else np.zeros((h_kv, 16 * P, ngk), np.float16)
    vs = np.zeros((h_kv, 16 * P, ngv), np.float16)
    slots = np.array([kchan_slot(c) for c in range(128)])
    for p in range(P):
        t0 = 16 * p
        o, n = sec["kscale"]
        if k_arm == 1:
            pair = pages[p, o:o + n].view(np.float16).reshape(2, h_kv, 128)[:, :, slots].astype(np.float32)
            ks[:, p] = pair[0] + pair[1]
        else:
            ks[:, t0:t0 + 16] = pages[p, o:o + n].view(np.float16).reshape(h_kv, 16, ngk)
        o, n = sec["vscale"]
        vs[:, t0:t0 + 16] = pages[p, o:o + n].view(np.float16).reshape(h_kv, 4, ngv, 4) \
            .transpose(0, 1, 3, 2).reshape(h_kv, 16, ngv)
        o, n = sec["kcode"]
        words = pages[p, o:o + n].view(np.uint32).reshape(h_kv, 4, 16, 4).astype(np.int64)   # [h][q][n][w]
        nib = (words[..., None] >> (4 * np.arange(8))) & 15                                 # [h][q][n][w][j]
        kq[:, t0:t0 + 16] = nib.transpose(0, 2, 3, 1, 4).reshape(h_kv, 16, 128) - 8
        o, n = sec["vcode"]
        cells = pages[p, o:o + n].view(np.uint16).reshape(h_kv, 4, 16, 8).astype(np.int64)   # [h][q][c][b]
        nib = (cells[..., None] >> (4 * np.arange(4))) & 15                                 # [h][q][c][b][j]
        vq[:, t0:t0 + 16] = nib.transpose(0, 1, 4, 3, 2).reshape(h_kv, 16, 128) - 8
    return kq, ks, vq, vs

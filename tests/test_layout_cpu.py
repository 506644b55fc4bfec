"""The numpy page packer (oracle/layout.py) against the page format as
documented in include/bmx_k2b.h: exact bit positions of single planted codes,
and pack -> unpack round trips.  The HIP write kernel is checked byte-for-byte
against this packer in the GPU tests."""

import numpy as np
import pytest

from oracle import layout as OL

D, PT = 128, 16


def _blank(h_kv, rank, T=64):
    C = D * h_kv
    us = np.zeros((T, rank), np.float16)
    res = np.full((C, T), -4, np.int64)          # offset-binary 0: all KRES bits clear
    sc = np.zeros((C, T // 64), np.float16)
    vidx = np.zeros((T, C), np.int64)
    vn = np.zeros((T, h_kv), np.float16)
    return us, res, sc, vidx, vn


def _set_bits(page_bytes, sec, h_kv, rank):
    o, s = OL.sections(h_kv, rank)[sec]
    words = page_bytes[o:o + s].view(np.uint32)
    return {(int(w), int(b)) for w in np.nonzero(words)[0] for b in range(32) if (words[w] >> b) & 1}


@pytest.mark.parametrize("h_kv,rank", [(8, 32), (2, 16), (1, 32)])
@pytest.mark.parametrize("seed", [0, 1, 2])
def test_kres_bit_positions(h_kv, rank, seed):
    rng = np.random.default_rng(seed)
    us, res, sc, vidx, vn = _blank(h_kv, rank)
    t = int(rng.integers(64))
    c = int(rng.integers(D * h_kv))
    res[c, t] = 3                                  # offset-binary 7: three bits
    pages = OL.pack_pages(us, res, sc, vidx, vn, h_kv, rank)
    h, jj = divmod(c, D)
    j, e = jj % 64, jj // 64
    b, q, i = j // 16, (j % 16) // 4, j % 4
    p = 4 * b + i
    lane = 16 * q + (t % PT)
    base = (h * 64 + lane) * 3                     # dword index in the section
    if p < 15:
        want = {(base + p // 5, 3 * (p % 5) + 16 * e + k) for k in range(3)}
    else:
        want = {(base + k, 15 + 16 * e) for k in range(3)}
    for pg in range(pages.shape[0]):
        got = _set_bits(pages[pg], "kres", h_kv, rank)
        assert got == (want if pg == t // PT else set())


@pytest.mark.parametrize("h_kv,rank", [(8, 32), (2, 16)])
def test_vcode_us_kscale_positions(h_kv, rank):
    rng = np.random.default_rng(5)
    for _ in range(6):
        us, res, sc, vidx, vn = _blank(h_kv, rank)
        t = int(rng.integers(64))
        c = int(rng.integers(D * h_kv))
        vidx[t, c] = 3
        pages = OL.pack_pages(us, res, sc, vidx, vn, h_kv, rank)
        h, ch = divmod(c, D)
        b, m = divmod(ch, 16)
        tt = t % PT
        lane = 16 * (tt // 4) + m
        want = {((h * 64 + lane) * 2 + b // 4, 8 * (b % 4) + 2 * (tt % 4) + k) for k in range(2)}
        assert _set_bits(pages[t // PT], "vcode", h_kv, rank) == want
        # US: token tt, rank r -> half index (r // (R/4)) * 16 * (R/4) + tt * (R/4) + r % (R/4)
        us, res, sc, vidx, vn = _blank(h_kv, rank)
        r = int(rng.integers(rank))
        us[t, r] = np.float16(1.0)
        pages = OL.pack_pages(us, res, sc, vidx, vn, h_kv, rank)
        kpl = rank // 4
        o, s = OL.sections(h_kv, rank)["us"]
        halfs = pages[t // PT, o:o + s].view(np.float16)
        idx = (r // kpl) * PT * kpl + tt * kpl + r % kpl
        assert halfs[idx] == 1.0 and np.count_nonzero(halfs) == 1
        # KSCALE: channel c of group 0 -> F = 128h + 2(j % 64) + j // 64, page F // (C/4)
        us, res, sc, vidx, vn = _blank(h_kv, rank)
        sc[c, 0] = np.float16(2.5)
        pages = OL.pack_pages(us, res, sc, vidx, vn, h_kv, rank)
        F = D * h + 2 * (ch % 64) + ch // 64
        quarter = D * h_kv // 4
        o, s = OL.sections(h_kv, rank)["kscale"]
        for pg in range(4):
            halfs = pages[pg, o:o + s].view(np.float16)
            if pg == F // quarter:
                assert halfs[F % quarter] == 2.5 and np.count_nonzero(halfs) == 1
            else:
                assert np.count_nonzero(halfs) == 0


@pytest.mark.parametrize("h_kv,rank", [(8, 32), (2, 16), (4, 32)])
def test_pack_unpack_round_trip(h_kv, rank):
    rng = np.random.default_rng(11)
    T, C = 128, D * h_kv
    us = rng.standard_normal((T, rank)).astype(np.float16)
    res = rng.integers(-4, 4, (C, T))
    sc = rng.random((C, T // 64)).astype(np.float16)
    vidx = rng.integers(0, 4, (T, C))
    vn = rng.random((T, h_kv)).astype(np.float16)
    pages = OL.pack_pages(us, res, sc, vidx, vn, h_kv, rank)
    assert pages.shape == (T // PT, OL.page_bytes(h_kv, rank))
    u2, r2, s2, v2, n2 = OL.unpack_pages(pages, h_kv, rank)
    assert np.array_equal(u2, us) and np.array_equal(r2, res) and np.array_equal(s2, sc)
    assert np.array_equal(v2, vidx) and np.array_equal(n2, vn)


@pytest.mark.parametrize("h,R,d,g,b", [(2, 16, 64, 32, 3), (8, 64, 128, 64, 3), (4, 32, 32, 16, 2),
                                       (1, 128, 128, 128, 4), (16, 16, 32, 32, 3)])
def test_general_page_layout_round_trip_and_library_geometry(h, R, d, g, b):
    """The general page's numpy restatement packs and unpacks every field, and
    its sections sit where the library says (include/bmx_k2b.h)."""
    from bmx_amd import _lib

    rng = np.random.default_rng(h * 1000 + R + d + g + b)
    C, T = h * d, 256
    us = rng.standard_normal((T, R)).astype(np.float16)
    res = rng.integers(-(1 << (b - 1)), 1 << (b - 1), (C, T))
    sc = rng.random((C, T // g)).astype(np.float16)
    vi = rng.integers(0, 4, (T, C))
    vn = rng.random((T, h)).astype(np.float16)
    pages = OL.pack_general(us, res, sc, vi, vn, h, R, d, g, b)
    got = OL.unpack_general(pages, h, R, d, g, b)
    for a_, w in zip(got, (us, res, sc, vi, vn)):
        np.testing.assert_array_equal(a_, w)
    sec = OL.general_sections(h, R, d, g)
    assert pages.shape[1] == sec["total"][1] == _lib.page_bytes(h, R, head_dim=d, group=g, k_bits=b)
    lib = _lib.page_sections(h, R, head_dim=d, group=g, k_bits=b)
    for name in _lib.SECTIONS:
        assert lib[name] == sec[name] and lib[name][0] % 16 == 0
    # one residual code lands where the format says: head hh, channel 3, token 17
    # -> page 1, row (hh, token 1), byte 1, high nibble, offset binary
    hh = h - 1
    res2 = np.zeros_like(res)
    res2[hh * d + 3, 17] = 1
    p2 = OL.pack_general(us, res2, sc, vi, vn, h, R, d, g, b)
    o = sec["kres"][0] + (hh * 16 + 1) * (d // 2) + 1
    assert p2[1, o] >> 4 == 1 + (1 << (b - 1)) and p2[1, o] & 15 == 1 << (b - 1)
    # one value code: token 6 of channel 5, head hh -> byte (hh, a 1, 5), bits 4..5
    vi2 = np.zeros_like(vi)
    vi2[6, hh * d + 5] = 3
    p3 = OL.pack_general(us, res, sc, vi2, vn, h, R, d, g, b)
    assert p3[0, sec["vcode"][0] + (hh * 4 + 1) * d + 5] == 3 << 4

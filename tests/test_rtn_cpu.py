"""RTN path on the CPU: the page format (numpy packer vs the C-ABI's sizes, and
its round trip), the RTN oracle cache against the reference's golden codec
vectors, and host-side argument checks of the C-ABI (no GPU call)."""

import ctypes as ct
from pathlib import Path

import numpy as np
import pytest
import torch

from bmx_amd import _lib, rtn
from oracle import attention as A
from oracle import codecs as OC
from oracle import layout as OL

GOLD = Path(__file__).parent / "golden"


@pytest.mark.parametrize("h_kv,gk,gv", [(8, 32, 32), (8, 64, 128), (1, 128, 32), (16, 32, 64)])
def test_page_bytes_match_numpy_layout(h_kv, gk, gv):
    assert rtn.page_bytes(h_kv, k_group=gk, v_group=gv) == OL.rtn_page_bytes(h_kv, gk, gv)
    # 4-bit codes + an fp16 scale per (token, group) for K and V
    assert OL.rtn_page_bytes(h_kv, gk, gv) == 16 * h_kv * (128 + 2 * 128 // gk + 2 * 128 // gv)


def test_headline_rtn_bytes_per_token():
    assert rtn.page_bytes(8) == 16 * 1152
    # channel-arm keys: 128 channel scales per head and page
    assert rtn.page_bytes(8, k_arm=rtn.CHANNEL) == OL.rtn_page_bytes(8, 32, 32, 1) == 16 * 1344


def test_channel_arm_page_round_trip():
    rng = np.random.default_rng(2)
    h_kv, gk, gv, T = 4, 64, 32, 128
    kq, vq = rng.integers(-8, 8, (h_kv, T, 128)), rng.integers(-8, 8, (h_kv, T, 128))
    ks = (0.01 + rng.random((h_kv, T // gk, 128))).astype(np.float32)   # normal fp16 range
    vs = rng.random((h_kv, T, 128 // gv)).astype(np.float16)
    pages = OL.pack_rtn_pages(kq, ks, vq, vs, h_kv, gk, gv, k_arm=1)
    a, b, c, d = OL.unpack_rtn_pages(pages, h_kv, gk, gv, k_arm=1)
    np.testing.assert_array_equal(a, kq)
    hi, lo = OL.scale_pair(ks)
    np.testing.assert_array_equal(b, np.repeat(hi.astype(np.float32) + lo.astype(np.float32), gk // 16, axis=1))
    # hi + lo carries the fp32 scale to ~2^-22 relative (2^-21 with the fp32
    # sum's own rounding, while lo is a normal fp16: scales of 1/8 and up;
    # below, lo's subnormal step 2^-24 sets the bound); hi alone to 2^-12
    rel = np.abs(b[:, ::gk // 16] / ks - 1)
    assert rel[ks >= 0.125].max() <= 2 ** -21 and rel.max() <= 2 ** -17
    assert np.abs(hi.astype(np.float32) / ks - 1).max() > 2 ** -16
    np.testing.assert_array_equal(c, vq)
    np.testing.assert_array_equal(d, vs)
    # channel 13 = 32*0 + 8*1 + 5 sits at slot 8 + 2*1 + 1 of its row; head 0's
    # lo row follows every head's hi row
    o = OL.rtn_sections(h_kv, gk, gv, 1)["kscale"][0]
    assert pages[0, o:o + 256].view(np.float16)[8 + 3] == hi[0, 0, 13]
    assert pages[0, o + 256 * h_kv:o + 256 * h_kv + 256].view(np.float16)[8 + 3] == lo[0, 0, 13]


@pytest.mark.parametrize("h_kv,gk,gv", [(8, 32, 32), (2, 64, 128)])
def test_page_round_trip_and_layout(h_kv, gk, gv):
    rng = np.random.default_rng(0)
    T = 32
    kq, vq = rng.integers(-8, 8, (h_kv, T, 128)), rng.integers(-8, 8, (h_kv, T, 128))
    ks = rng.random((h_kv, T, 128 // gk)).astype(np.float16)
    vs = rng.random((h_kv, T, 128 // gv)).astype(np.float16)
    pages = OL.pack_rtn_pages(kq, ks, vq, vs, h_kv, gk, gv)
    got = OL.unpack_rtn_pages(pages, h_kv, gk, gv)
    for a, b in zip(got, (kq, ks, vq, vs)):
        np.testing.assert_array_equal(a, b)
    sec = OL.rtn_sections(h_kv, gk, gv)
    # key word (q 1, token 3, w 2) holds channels 72..79 of token 3, head 0, page 0
    o = sec["kcode"][0]
    w = int(pages[0, o:o + 1024].view(np.uint32)[(1 * 16 + 3) * 4 + 2])
    assert [((w >> (4 * j)) & 15) - 8 for j in range(8)] == list(kq[0, 3, 72:80])
    # value cell (q 2, c 5, b 3) holds channel 53 of tokens 8..11
    o = sec["vcode"][0]
    c = int(pages[0, o:o + 1024].view(np.uint16)[(2 * 16 + 5) * 8 + 3])
    assert [((c >> (4 * j)) & 15) - 8 for j in range(4)] == list(vq[0, 8:12, 53])
    # value scale of token 4q + i, group g at [q][g][i]
    o = sec["vscale"][0]
    vsc = pages[0, o:o + sec["vscale"][1]].view(np.float16).reshape(h_kv, 4, 128 // gv, 4)
    assert vsc[0, 2, 0, 1] == vs[0, 9, 0]


def test_oracle_cache_matches_reference_golden():
    """The RTN oracle cache codes a page with quantize_packed("rtn_token")
    exactly as the reference (golden vectors of quant/rtn.py) and dequantizes
    with the fp32 scale to the reference's own output."""
    g = np.load(GOLD / "codecs.npz")
    M = torch.from_numpy(g["rtn_v_in"])           # (128 tokens, 256 channels): h_kv 2
    c = A.RtnOracleCache(2, k_bits=4, v_bits=4, k_group=32, v_group=32)
    c.commit(OC.from_matrix(M, 2), OC.from_matrix(M, 2))
    kq, ks, vq, vs = c.codes()
    np.testing.assert_array_equal(OC.to_matrix(vq).numpy(), g["rtn_token_q"])
    np.testing.assert_array_equal(OC.to_matrix(vs).numpy(), g["rtn_token_scale"][..., 0])
    _, V32 = c.dense_kv(fp16_scales=False)
    np.testing.assert_array_equal(OC.to_matrix(V32).numpy(), g["rtn_token_deq"])
    # the fused path's fp16 scales: code * fp16(scale), exactly
    _, V16 = c.dense_kv()
    want = vq.float() * vs.half().float().repeat_interleave(32, dim=-1)
    assert torch.equal(V16, want)


def test_channel_arm_oracle_matches_reference_golden():
    """rtn_channel keys through the RTN oracle cache: the reference's golden
    codes, scales and dequantization of quantize_packed("rtn_channel")."""
    g = np.load(GOLD / "codecs.npz")
    M = torch.from_numpy(g["rtn_k_in"])            # (128 tokens, 256 channels): h_kv 2
    c = A.RtnOracleCache(2, k_bits=4, v_bits=4, k_group=32, v_group=32, k_arm=1)
    c.commit(OC.from_matrix(M, 2), OC.from_matrix(M, 2))
    kq, ks, _, _ = c.codes()
    np.testing.assert_array_equal(OC.to_matrix(kq).numpy().T, g["rtn_channel_q"])
    np.testing.assert_array_equal(OC.to_matrix(ks).numpy().T, g["rtn_channel_scale"][..., 0])
    K32, _ = c.dense_kv(fp16_scales=False)
    np.testing.assert_array_equal(OC.to_matrix(K32).numpy(), g["rtn_channel_deq"])


@pytest.mark.parametrize("k_arm", [0, 1])
def test_chunked_rtn_oracle_equals_one_softmax(k_arm):
    """The chunked restatement (per page, online softmax, fp32 scales) equals
    one softmax over the same dequantized keys and values."""
    gen = torch.Generator().manual_seed(3)
    h_kv, G = 2, 4
    c = A.RtnOracleCache(h_kv, k_bits=4, v_bits=4, k_group=32, v_group=64, k_arm=k_arm)
    for _ in range(3):
        c.commit(torch.randn(h_kv, 128, 128, generator=gen), torch.randn(h_kv, 128, 128, generator=gen))
    kt, vt = torch.randn(h_kv, 37, 128, generator=gen).half(), torch.randn(h_kv, 37, 128, generator=gen).half()
    q = torch.randn(h_kv * G, 1, 128, generator=gen)
    got = A.rtn_chunked_attention(q, c, kt, vt, G, 128 ** -0.5)
    K, V = c.dense_kv(fp16_scales=False)
    want = A.naive_dense_attention(q, torch.cat([K, kt.float()], 1), torch.cat([V, vt.float()], 1), G,
                                   128 ** -0.5)
    assert (got - want).abs().max().item() < 1e-5


def test_bad_rtn_arguments_are_rejected_with_message():
    lib = _lib.lib()
    with pytest.raises(NotImplementedError, match="2..4-bit"):
        rtn.page_bytes(8, k_bits=8)
    with pytest.raises(NotImplementedError):
        rtn.page_bytes(8, k_group=16)
    a = _lib.RtnDecodeArgs()
    a.geom = rtn.geom(8, 32, k_bits=4, v_bits=4, k_group=32, v_group=32)   # G too large
    a.batch = 1
    assert lib.bmx_rtn_decode(ct.byref(a), None) != 0 and b"n_q_groups" in lib.bmx_last_error()
    a.geom = rtn.geom(9, 4, k_bits=4, v_bits=4, k_group=32, v_group=32)    # decode takes 1..8 heads
    assert lib.bmx_rtn_decode(ct.byref(a), None) != 0 and b"h_kv" in lib.bmx_last_error()
    a.geom = rtn.geom(8, 4, k_bits=4, v_bits=4, k_group=32, v_group=32)
    a.max_packed_len = 100
    assert lib.bmx_rtn_decode(ct.byref(a), None) != 0 and b"multiple of 128" in lib.bmx_last_error()
    ap = _lib.RtnAppendArgs()
    ap.geom = rtn.geom(8, k_bits=4, v_bits=4, k_group=32, v_group=32)
    ap.n_codec_pages = 1
    assert lib.bmx_rtn_append(ct.byref(ap), None) != 0 and b"null pointer" in lib.bmx_last_error()


def test_rtn_workspace_size_formula():
    a = _lib.RtnDecodeArgs()
    a.geom = rtn.geom(8, 4, k_bits=4, v_bits=4, k_group=32, v_group=32)
    a.batch, a.max_packed_len, a.split_tokens, a.tail_cap = 2, 65536, 1024, 200
    n = _lib.lib().bmx_rtn_decode_workspace_bytes(ct.byref(a))
    # per query: 64 split records (128 fp16 channel means, fp32 max and sum), then 200 fp32 window scores
    assert n == 2 * 8 * 4 * (64 * (128 * 2 + 2 * 4) + 200 * 4)

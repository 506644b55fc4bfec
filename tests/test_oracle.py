"""Pin the CPU oracle: golden vectors from the reference's own code, closed forms,
exact identities and brute force.  CPU only."""

import math
from pathlib import Path

import numpy as np
import pytest
import scipy.linalg
import torch

from oracle import attention as A
from oracle import codecs as C

GOLD = Path(__file__).parent / "golden"


@pytest.fixture(scope="module")
def gc():
    return np.load(GOLD / "codecs.npz")


@pytest.fixture(scope="module")
def ga():
    return np.load(GOLD / "attention.npz")


# ---------------------------------------------------------------- codebook / signs


@pytest.mark.parametrize("bits", [2, 3, 4])
def test_codebook_matches_reference(gc, bits):
    np.testing.assert_array_equal(C.gaussian_codebook(bits).numpy(), gc[f"codebook_b{bits}"])


def test_codebook_properties():
    cb = C.gaussian_codebook(2)
    assert torch.all(cb[1:] > cb[:-1])
    # near the analytic Lloyd-Max levels for N(0,1) (+-0.4528, +-1.5104)
    np.testing.assert_allclose(cb.abs().sort().values.numpy(),
                               [0.4528, 0.4528, 1.5104, 1.5104], atol=2e-2)


@pytest.mark.parametrize("d,seed", [(128, 0), (128, 7), (64, 0)])
def test_signs_match_reference(gc, d, seed):
    np.testing.assert_array_equal(C.hadamard_signs(d, seed).numpy(), gc[f"signs_d{d}_s{seed}"])


# ---------------------------------------------------------------- FWHT


def test_fwht_matches_reference(gc):
    np.testing.assert_array_equal(C.fwht(torch.from_numpy(gc["fwht_in"])).numpy(), gc["fwht_out"])


@pytest.mark.parametrize("d", [2, 16, 128])
def test_fwht_is_sylvester_hadamard(d):
    H = scipy.linalg.hadamard(d) / math.sqrt(d)
    x = torch.randn(5, d, dtype=torch.float64)
    np.testing.assert_allclose(C.fwht(x).numpy(), x.numpy() @ H.T, atol=1e-12)
    # involution: fwht(fwht(x)) == x
    np.testing.assert_allclose(C.fwht(C.fwht(x)).numpy(), x.numpy(), atol=1e-12)


# ---------------------------------------------------------------- RTN


def test_rtn_closed_form_small():
    W = torch.tensor([[0.0, 1.0, -3.0, 1.5, 0.5, -0.25, 2.9, 3.0]])
    q, s = C.rtn_quantize_packed(W, 3, 8)
    assert float(s) == pytest.approx(1.0)
    # round half to even: 1.5 -> 2, 0.5 -> 0, -0.25 -> 0, 2.9 -> 3, -3 -> -3
    assert q.tolist() == [[0, 1, -3, 2, 0, 0, 3, 3]]
    q4, _ = C.rtn_quantize_packed(torch.tensor([[-4.0, 3.0, 1.0, 0.0]]) * 1.0, 3, 4)
    assert q4.min() >= -4 and q4.max() <= 3


def test_rtn_arms_match_reference(gc):
    K = torch.from_numpy(gc["rtn_k_in"])
    V = torch.from_numpy(gc["rtn_v_in"])
    kp, bk = C.quantize_rtn_channel(K, 4, 32)
    vp, bv = C.quantize_rtn_token(V, 4, 32)
    np.testing.assert_array_equal(kp["Q_int"].numpy(), gc["rtn_channel_q"])
    np.testing.assert_array_equal(kp["scale"].numpy(), gc["rtn_channel_scale"])
    np.testing.assert_array_equal(vp["Q_int"].numpy(), gc["rtn_token_q"])
    np.testing.assert_array_equal(vp["scale"].numpy(), gc["rtn_token_scale"])
    np.testing.assert_array_equal(C.dequant_rtn_channel(kp, 32).numpy(), gc["rtn_channel_deq"])
    np.testing.assert_array_equal(C.dequant_rtn_token(vp, 32).numpy(), gc["rtn_token_deq"])
    assert bk == gc["rtn_channel_bpe"] == 4 + 16 / 32
    assert bv == gc["rtn_token_bpe"]


# ---------------------------------------------------------------- k2b key codec


@pytest.mark.parametrize("rank", [16, 32])
def test_k2b_key_pages_match_reference(gc, rank):
    kpre = torch.from_numpy(gc[f"k2b_r{rank}_kpre"])
    enc = C.FrozenSubspaceKeyEncoder(rank)
    # The first page's SVD is LAPACK-dependent, so its factors are an input
    # (the reference's own SVD output); later pages project on the frozen V.
    us0 = torch.from_numpy(gc[f"k2b_r{rank}_svd_us_fp32"])
    v0 = torch.from_numpy(gc[f"k2b_r{rank}_svd_v_fp32"])
    for p in range(3):
        M = C.to_matrix(kpre[:, p * 128:(p + 1) * 128].float())
        kp, bpe = enc.encode(M, us_override=(us0, v0) if p == 0 else None)
        pre = f"k2b_r{rank}_p{p}_"
        np.testing.assert_array_equal(kp["Us"].numpy(), gc[pre + "us"])
        np.testing.assert_array_equal(kp["V"].numpy(), gc[pre + "v"])
        np.testing.assert_array_equal(kp["res_Q_int"].numpy(), gc[pre + "res"])
        np.testing.assert_array_equal(kp["res_scale"].numpy(), gc[pre + "scale"])
        assert bpe == float(gc[pre + "bpe_k"])
        if p == 0:
            np.testing.assert_array_equal(C.dequant_k2b_key(kp).numpy(), gc[pre + "kdeq"])
            np.testing.assert_array_equal(C.pack_signed_codes(kp["res_Q_int"], 3).numpy(),
                                          gc[pre + "res_packed"])


def test_k2b_bpe_closed_form():
    # 3 + 16/g + 16 r (S + C)/(S C) at S=128 (test_cache_codecs.py:78-89)
    for r, Cc in ((16, 1024), (32, 1024), (16, 256)):
        assert C.factor_bits(r, 128, Cc) == pytest.approx(16 * r * (128 + Cc) / (128 * Cc))
    M = torch.randn(128, 256)
    Us, V = C.truncated_svd(M, 16)
    _, bpe = C.quantize_k2b_key(M, Us, V)
    assert bpe == pytest.approx(3 + 16 / 64 + 16 * 16 * (128 + 256) / (128 * 256))


def test_k2b_reconstruction_error_bounded():
    """R is quantized with |err| <= scale/2 per entry (brute-force check)."""
    M = torch.randn(128, 256)
    Us, V = C.truncated_svd(M, 16)
    kp, _ = C.quantize_k2b_key(M, Us, V)
    L = kp["Us"] @ kp["V"].mT
    err = (C.dequant_k2b_key(kp) - M).abs().mT.reshape(256, 2, 64)
    R = (M - L).mT.reshape(256, 2, 64)
    scale = kp["res_scale"]
    # codes clip at -4 only below -3.5*scale, impossible since |R| <= 3*scale
    assert torch.all(err <= scale / 2 + 1e-6)
    assert torch.all(R.abs() <= 3 * scale + 1e-6)


# ---------------------------------------------------------------- V codec


@pytest.mark.parametrize("rank", [16, 32])
def test_v_codec_matches_reference(gc, rank):
    v = torch.from_numpy(gc[f"k2b_r{rank}_v"])
    for p in range(3):
        Mv = C.to_matrix(v[:, p * 128:(p + 1) * 128].float())
        idx, norms, bpe = C.quantize_v_perhead(Mv, bits=2, seed=0, h=2)
        pre = f"k2b_r{rank}_p{p}_"
        np.testing.assert_array_equal(idx.numpy(), gc[pre + "vidx"])
        np.testing.assert_array_equal(norms.numpy(), gc[pre + "vnorm"])
        assert bpe == float(gc[pre + "bpe_v"]) == 2 + 16 * 2 / 256
        if p == 0:
            np.testing.assert_array_equal(
                C.dequant_v_perhead(idx, norms, bits=2, seed=0, h=2).numpy(), gc[pre + "vdeq"])
            np.testing.assert_array_equal(C.pack_codes(idx, 2).numpy(), gc[pre + "vidx_packed"])


def test_v_codec_bucketize_ties_go_low():
    cb = C.gaussian_codebook(2)
    mid = (cb[:-1] + cb[1:]) / 2
    assert torch.bucketize(mid, mid).tolist() == [0, 1, 2]


# ---------------------------------------------------------------- schedule


def test_flush_schedule(gc):
    for S, W, g, want in gc["flush_schedule"]:
        assert C.compute_flush_schedule(int(S), int(W), int(g)) == int(want)


# ---------------------------------------------------------------- RoPE


@pytest.mark.parametrize("rank", [16, 32])
def test_rope_tables_match_hf(ga, rank):
    pre = f"attn_r{rank}_"
    inv = A.default_inv_freq(128, 500000.0)
    cos, sin = A.rope_cos_sin(inv, torch.from_numpy(ga[pre + "rope_pos"]))
    np.testing.assert_array_equal(cos.numpy(), ga[pre + "cos"])
    np.testing.assert_array_equal(sin.numpy(), ga[pre + "sin"])


# ---------------------------------------------------------------- attention


def _oracle_cache_from_fixture(ga, rank):
    pre = f"attn_r{rank}_"
    kpre = torch.from_numpy(ga[pre + "kpre"])
    v = torch.from_numpy(ga[pre + "v"])
    vseed = int(ga[pre + "vseed"])
    cache = A.K2bOracleCache(2, 128, rank, v_seed=vseed)
    svd = (torch.from_numpy(ga[pre + "svd_us"]), torch.from_numpy(ga[pre + "svd_v"]))
    for p in range(3):
        cache.commit(kpre[:, p * 128:(p + 1) * 128], v[:, p * 128:(p + 1) * 128],
                     us_override=svd if p == 0 else None)
    return cache


@pytest.mark.parametrize("rank", [16, 32])
def test_attention_matches_reference(ga, rank):
    pre = f"attn_r{rank}_"
    cache = _oracle_cache_from_fixture(ga, rank)
    q = torch.from_numpy(ga[pre + "q"])
    kt = torch.from_numpy(ga[pre + "k_tail"])
    vt = torch.from_numpy(ga[pre + "v"])[:, 384:]
    inv = A.default_inv_freq(128, 500000.0)
    o_naive = A.k2b_naive_attention(q, cache, inv, kt, vt, 4, 128 ** -0.5)
    o_chunk = A.k2b_chunked_attention(q, cache, inv, kt, vt, 4, 128 ** -0.5)
    np.testing.assert_allclose(o_naive.numpy(), ga[pre + "naive"], atol=1e-6, rtol=0)
    np.testing.assert_allclose(o_chunk.numpy(), ga[pre + "chunked"], atol=1e-6, rtol=0)
    # naive (one softmax) == chunked (online) up to fp32 reassociation
    np.testing.assert_allclose(o_naive.numpy(), o_chunk.numpy(), atol=1e-5)
    acc, m, lse = A.tail_partial(q.view(2, 4, 128), kt, vt, 128 ** -0.5)
    np.testing.assert_allclose(acc.numpy(), ga[pre + "tail_acc"], rtol=1e-6, atol=1e-5)
    np.testing.assert_allclose(m.numpy(), ga[pre + "tail_m"], rtol=1e-6)
    np.testing.assert_allclose(lse.numpy(), ga[pre + "tail_lse"], rtol=1e-6)


def test_naive_oracle_equals_hand_softmax():
    torch.manual_seed(0)
    q = torch.randn(4, 1, 8, dtype=torch.float64)
    K = torch.randn(2, 10, 8, dtype=torch.float64)
    V = torch.randn(2, 10, 8, dtype=torch.float64)
    out = A.naive_dense_attention(q, K, V, 2, 0.3).double()
    for h in range(4):
        s = [(q[h, 0] @ K[h // 2, t]).item() * 0.3 for t in range(10)]
        w = np.exp(np.array(s) - max(s))
        w /= w.sum()
        want = (torch.tensor(w)[:, None] * V[h // 2].double()).sum(0)
        np.testing.assert_allclose(out[h, 0].numpy(), want.numpy(), atol=1e-6)


def test_grouped_oracle_equals_hand_softmax():
    """The batched, copy-free form gives the hand softmax of every (head,
    position) pair, query head h reading KV head h // G."""
    torch.manual_seed(1)
    q = torch.randn(6, 3, 8, dtype=torch.float64)
    K = torch.randn(2, 10, 8, dtype=torch.float64)
    V = torch.randn(2, 10, 8, dtype=torch.float64)
    out = A.grouped_dense_attention(q, K, V, 3, 0.3).double()
    for h in range(6):
        for j in range(3):
            s = [(q[h, j] @ K[h // 3, t]).item() * 0.3 for t in range(10)]
            w = np.exp(np.array(s) - max(s))
            w /= w.sum()
            want = (torch.tensor(w)[:, None] * V[h // 3]).sum(0)
            np.testing.assert_allclose(out[h, j].numpy(), want.numpy(), atol=1e-6)


def test_argmax_flip_gate():
    """No flip; a near-tie flip (top-2 gap 0.01 below the delta 0.02) is soft;
    a flip against a top-2 gap of 1.0 with a delta of 0.7 is hard."""
    ref = torch.tensor([0.0, 3.0, 2.99, -1.0])
    assert A.argmax_flip(ref + 0.001, ref) == (False, False)
    assert A.argmax_flip(torch.tensor([0.0, 2.99, 3.01, -1.0]), ref) == (True, False)
    assert A.argmax_flip(torch.tensor([0.0, 2.6, 2.7, -1.0]), torch.tensor([0.0, 3.0, 2.0, -1.0])) \
        == (True, True)


def test_split_merge_equals_dense_union():
    """Merging per-split partials (plus a tail split) equals one softmax over the
    union (test_decode_finalize.py:165-220)."""
    torch.manual_seed(1)
    h, G, d = 2, 4, 16
    q = torch.randn(h, G, d, dtype=torch.float64)
    Ks = [torch.randn(h, n, d, dtype=torch.float64) for n in (5, 9, 1, 7)]
    Vs = [torch.randn(h, n, d, dtype=torch.float64) for n in (5, 9, 1, 7)]
    parts = [A.tail_partial(q, k, v, 0.25) for k, v in zip(Ks, Vs)]
    acc = torch.stack([p[0] for p in parts])
    m = torch.stack([p[1] for p in parts])
    lse = torch.stack([p[2] for p in parts])
    out = A.merge_partials(acc, m, lse)
    Kall, Vall = torch.cat(Ks, 1), torch.cat(Vs, 1)
    s = torch.einsum("hgd,htd->hgt", q, Kall) * 0.25
    want = torch.einsum("hgt,htd->hgd", torch.softmax(s, -1), Vall)
    # partials are fp32 (as the reference's _tail_partial), the union is fp64
    np.testing.assert_allclose(out.numpy(), want.numpy(), atol=2e-6)
    # one split collapses to acc / lse exactly
    np.testing.assert_array_equal(A.merge_partials(acc[:1], m[:1], lse[:1]).numpy(),
                                  (acc[0] / lse[0].unsqueeze(-1)).numpy())


def test_online_softmax_is_exact():
    torch.manual_seed(2)
    s = torch.randn(3, 1, 20, dtype=torch.float64)
    V = torch.randn(3, 20, 5, dtype=torch.float64)
    acc = torch.zeros(3, 1, 5, dtype=torch.float64)
    m = torch.full((3, 1, 1), float("-inf"), dtype=torch.float64)
    lse = torch.zeros(3, 1, 1, dtype=torch.float64)
    for a, b in ((0, 7), (7, 8), (8, 20)):
        acc, m, lse = A.online_softmax_update(acc, m, lse, s[..., a:b], V[:, a:b])
    np.testing.assert_allclose((acc / lse).numpy(), (torch.softmax(s, -1) @ V).numpy(), atol=1e-14)


def test_oracle_catches_a_wrong_v_seed(ga):
    """A plausible mistake (threading the K seed into V) must move the output
    far beyond the parity tolerance (test_triton_decode_k2b.py:336-403)."""
    pre = "attn_r32_"
    cache = _oracle_cache_from_fixture(ga, 32)
    cache.v_seed = 0  # fixture used v_seed 7
    q = torch.from_numpy(ga[pre + "q"])
    kt = torch.from_numpy(ga[pre + "k_tail"])
    vt = torch.from_numpy(ga[pre + "v"])[:, 384:]
    o = A.k2b_naive_attention(q, cache, A.default_inv_freq(128, 5e5), kt, vt, 4, 128 ** -0.5)
    assert (o.numpy() - ga[pre + "naive"]).__abs__().max() > 0.05


# ---------------------------------------------------------------- k2b at other geometries

# name, h_kv, head_dim, rank, residual group, key bits, value seed (tests/golden/make_golden.py)
GEOM_CASES = [
    ("d64_r16_g32", 2, 64, 16, 32, 3, 7),
    ("d128_r64_g64", 2, 128, 64, 64, 3, 0),
    ("d32_r16_g16_b2", 4, 32, 16, 16, 2, 3),
    ("d128_r32_g128_b4", 2, 128, 32, 128, 4, 0),
]


@pytest.mark.parametrize("case", GEOM_CASES, ids=[c[0] for c in GEOM_CASES])
def test_k2b_codecs_at_other_geometries_match_reference(case):
    """The oracle's key and value codecs at head_dim 32/64, rank 64, residual
    groups 16/32/128 and 2- or 4-bit keys reproduce the reference's own
    quantize_packed outputs bit for bit (the first page's SVD is an input)."""
    name, h, d, rank, group, bits, vseed = case
    g = np.load(GOLD / "k2b_geom.npz")
    np.testing.assert_array_equal(C.hadamard_signs(d, vseed).numpy(), g[f"{name}_signs"])
    kpre = torch.from_numpy(g[f"{name}_kpre"])
    v = torch.from_numpy(g[f"{name}_v"])
    enc = C.FrozenSubspaceKeyEncoder(rank, bits, group)
    us0 = torch.from_numpy(g[f"{name}_svd_us_fp32"])
    v0 = torch.from_numpy(g[f"{name}_svd_v_fp32"])
    for p in range(3):
        M = C.to_matrix(kpre[:, p * 128:(p + 1) * 128].float())
        kp, bpe = enc.encode(M, us_override=(us0, v0) if p == 0 else None)
        pre = f"{name}_p{p}_"
        np.testing.assert_array_equal(kp["Us"].numpy(), g[pre + "us"])
        np.testing.assert_array_equal(kp["res_Q_int"].numpy(), g[pre + "res"])
        np.testing.assert_array_equal(kp["res_scale"].numpy(), g[pre + "scale"])
        assert bpe == float(g[pre + "bpe_k"]) == pytest.approx(
            bits + 16 / group + 16 * rank * (128 + h * d) / (128 * h * d))
        idx, norms, bpe_v = C.quantize_v_perhead(C.to_matrix(v[:, p * 128:(p + 1) * 128].float()), bits=2,
                                                 seed=vseed, h=h)
        np.testing.assert_array_equal(idx.numpy(), g[pre + "vidx"])
        np.testing.assert_array_equal(norms.numpy(), g[pre + "vnorm"])
        assert bpe_v == float(g[pre + "bpe_v"])
        if p == 0:
            np.testing.assert_array_equal(C.dequant_k2b_key(kp, group).numpy(), g[pre + "kdeq"])
            np.testing.assert_array_equal(
                C.dequant_v_perhead(idx, norms, bits=2, seed=vseed, h=h).numpy(), g[pre + "vdeq"])
    # the residual's range is the key bits': a 3-bit restatement of a 2-bit case fails
    if bits != 3:
        kp3, _ = C.FrozenSubspaceKeyEncoder(rank, 3, group).encode(
            C.to_matrix(kpre[:, :128].float()), us_override=(us0, v0))
        assert not np.array_equal(kp3["res_Q_int"].numpy(), g[f"{name}_p0_res"])

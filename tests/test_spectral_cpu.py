"""Spectral (K4) path on the CPU: the oracle against the reference's golden
vectors (tests/golden/spectral.npz, written by make_golden.py from the
reference's own spectral.py), the host layout against the oracle's, pack
files, and the C-ABI's argument checks (no GPU call)."""

import ctypes as ct

import numpy as np
import pytest
import torch

from bmx_amd import _lib, k2b, spectral
from oracle import spectral as O
from tests.spectral_util import GOLD, golden_pack, synthetic_pack


@pytest.fixture(scope="module")
def gold():
    return np.load(GOLD / "spectral.npz")


@pytest.mark.parametrize("budget", [2.0, 2.5, 3.0])
def test_allocation_matches_reference(gold, budget):
    """Both restatements of allocate_bits_from_variance ("round") give the
    reference's bits for its fitted spectrum."""
    want = gold[f"bits_b{budget}"]
    assert np.array_equal(O.allocate_bits_round(gold["lam64"], budget), want)
    assert np.array_equal(spectral.allocate_bits(torch.from_numpy(gold["lam64"]), budget).numpy(), want)


def test_tier_columns_and_bpe_match_reference(gold):
    bits = gold["bits_b2.5"]
    cols = O.tier_columns(bits)
    assert sorted(cols) == sorted(int(k[6:]) for k in gold.files if k.startswith("cols_t"))
    for b, c in cols.items():
        assert np.array_equal(c, gold[f"cols_t{b}"])
    assert O.payload_bpe(bits) == float(gold["bpe"])
    assert spectral.payload_bpe(torch.from_numpy(bits)) == float(gold["bpe"])


def test_quantizer_matches_reference_codes(gold):
    """Given the reference's Y, every code of every tier equals the reference's
    and the steps agree to the sum order (a few fp32 ulps)."""
    bits = gold["bits_b2.5"]
    L = O.Layout(bits)
    codes, scales = O.quantize(L.permute_cols(gold["Y"]), L)
    for b, c in O.tier_columns(bits).items():
        k = np.array([np.nonzero(L.perm == x)[0][0] for x in c])
        mine = codes[:, :, k].transpose(2, 0, 1).reshape(len(c), -1)
        np.testing.assert_array_equal(mine, gold[f"codes_t{b}"])
        rs = gold[f"scale_t{b}"][..., 0]
        assert np.abs(scales[:, k].T / rs - 1).max() < 2e-6
    Mh = O.dequant(codes, scales, gold["dec"], L, fp16_scales=False)
    assert np.abs(Mh - gold["M_hat"]).max() < 1e-5


def test_quantizer_step_refinement_is_not_max_scaling(gold):
    """A planted mistake the golden codes catch: the max-based step without
    the MSE refinement changes codes."""
    bits = gold["bits_b2.5"]
    L = O.Layout(bits)
    Y = L.permute_cols(gold["Y"])
    k = np.nonzero(L.col_bits == 2)[0][:16]
    G = Y[:64, k].T
    q_ref, _ = O.quantize_groups(G, 2)
    q_max, _ = O.quantize_groups(G, 2, n_iter=0)
    assert (q_ref != q_max).any()


def test_encode_order_is_fp32_of_the_product(gold):
    L = O.Layout(gold["bits_b2.5"])
    Y = O.encode(gold["M"], gold["enc"], L)
    Y64 = L.permute_cols(gold["M"].astype(np.float64) @ gold["enc"].astype(np.float64))
    assert np.abs(Y - Y64).max() <= 1e-5 * np.abs(Y64).max()


def test_page_round_trip_and_planted_code():
    pack = synthetic_pack(2, 3.0, seed=1)
    L = O.Layout(pack.bits.numpy())
    rng = np.random.default_rng(0)
    codes = np.zeros((3, 64, L.c_pad), np.int64)
    for b in set(L.slice_bits.tolist()):
        k = L.col_bits == b
        codes[:, :, k] = rng.integers(-(1 << (b - 1)), 1 << (b - 1), (3, 64, int(k.sum())))
    scales = rng.random((3, L.c_pad)).astype(np.float32)
    pages = O.pack_pages(codes, scales, L)
    c2, s2 = O.unpack_pages(pages, L)
    np.testing.assert_array_equal(c2, codes)
    np.testing.assert_array_equal(s2, scales.astype(np.float16).astype(np.float32))
    # column 8s + 3 of token 5 in slice s sits at bits [3w, 4w) of bytes off[s] + 5w ..
    s = int(np.nonzero(L.width == 4)[0][0])
    w, b = 4, int(L.slice_bits[s])
    word = int.from_bytes(pages[1, L.off[s] + 5 * w: L.off[s] + 6 * w].tobytes(), "little")
    assert ((word >> (3 * w)) & 15) - (1 << (b - 1)) == codes[1, 5, 8 * s + 3]


@pytest.mark.parametrize("h_kv,budget", [(2, 2.5), (8, 2.5), (8, 3.0)])
def test_host_layout_matches_oracle(h_kv, budget):
    pack = synthetic_pack(h_kv, budget, seed=4)
    dp = spectral.DevicePack(pack, h_kv, "cpu")
    L = O.Layout(pack.bits.numpy())
    assert (dp.c_pad, dp.k_page_bytes) == (L.c_pad, L.page_bytes)
    np.testing.assert_array_equal(dp.slice_tab.numpy(), L.slice_table())
    np.testing.assert_array_equal(dp.perm.numpy(), L.perm)
    np.testing.assert_array_equal(dp.enc_perm.numpy(), L.permute_cols(pack.enc.numpy()))
    c32 = -(-L.c_pad // 32) * 32
    assert dp.dec_perm.shape == (h_kv, c32 // 32, 8, 16, 32)
    rows = dp.dec_perm.permute(0, 2, 3, 1, 4).reshape(128 * h_kv, c32)   # untile
    np.testing.assert_array_equal(rows[:, : L.c_pad].numpy(),
                                  L.permute_cols(pack.dec.numpy()).astype(np.float16))
    assert not rows[:, L.c_pad:].any()
    assert dp.v_page_bytes == 544 * h_kv


def test_golden_pack_layout(gold):
    pack, _ = golden_pack()
    dp = spectral.DevicePack(pack, 2, "cpu")
    assert dp.c_pad == 264 and dp.bpe == float(gold["bpe"])


def test_pack_file_round_trip(tmp_path):
    p1, p2 = synthetic_pack(1, 2.5, seed=2), synthetic_pack(1, 3.0, seed=2)
    path = tmp_path / "packs.safetensors"
    spectral.save_packs(path, {0: (p1.enc, p1.dec, p1.lam, {2.5: p1.bits, 3.0: p2.bits})}, (2.5, 3.0))
    got = spectral.load_packs(path, 3.0)[0]
    assert torch.equal(got.bits, p2.bits) and torch.equal(got.dec, p1.dec) and got.group == 64
    with pytest.raises(KeyError, match="available"):
        spectral.load_packs(path, 2.0)


def test_unsupported_packs_are_rejected():
    pack = synthetic_pack(1, 2.5, seed=3)
    with pytest.raises(NotImplementedError, match="64-token"):
        spectral.DevicePack(spectral.SpectralPack(pack.enc, pack.dec, pack.lam, pack.bits, group=32), 1, "cpu")
    bits = pack.bits.clone()
    bits[0] = 7
    with pytest.raises(NotImplementedError, match="tiers"):
        spectral.DevicePack(spectral.SpectralPack(pack.enc, pack.dec, pack.lam, bits), 1, "cpu")


def test_bad_spectral_arguments_are_rejected_with_message():
    lib = _lib.lib()
    a = _lib.SpectralAppendArgs()
    a.L = _lib.SpectralLayout(9, 64, 4096, 1)
    assert lib.bmx_spectral_append(ct.byref(a), None) != 0 and b"h_kv" in lib.bmx_last_error()
    a.L = _lib.SpectralLayout(2, 60, 4096, 1)
    assert lib.bmx_spectral_append(ct.byref(a), None) != 0 and b"c_pad" in lib.bmx_last_error()
    a.L = _lib.SpectralLayout(2, 64, 64, 1)
    assert lib.bmx_spectral_append(ct.byref(a), None) != 0 and b"k_page_bytes" in lib.bmx_last_error()
    a.L = _lib.SpectralLayout(2, 64, 4096, 1)
    a.n_groups = 1
    assert lib.bmx_spectral_append(ct.byref(a), None) != 0 and b"null pointer" in lib.bmx_last_error()
    d = _lib.SpectralDequantArgs()
    d.L = _lib.SpectralLayout(2, 64, 4096, 1)
    d.n_tokens = 100
    assert lib.bmx_spectral_dequant(ct.byref(d), None) != 0 and b"multiple of 64" in lib.bmx_last_error()
    d.n_tokens, d.apply_rope = 64, 3
    assert lib.bmx_spectral_dequant(ct.byref(d), None) != 0 and b"apply_rope" in lib.bmx_last_error()
    assert lib.bmx_spectral_v_page_bytes(8) == 4352 and lib.bmx_spectral_v_page_bytes(0) == -1


def test_recipe_and_construction_guards(tmp_path):
    """spec_pair("k4ph_b<budget>") needs a pack path; the cache asserts pre-RoPE
    keys and a pack file at construction (packed_streaming.py:336-360), loads
    every layer's pack once, and refuses the variants without kernels."""
    from transformers import LlamaConfig

    from bmx_amd.cache import PackedStreamingCache
    from bmx_amd.specs import CacheCodecSpec, spec_pair

    cfg = LlamaConfig(vocab_size=64, hidden_size=256, intermediate_size=256, num_hidden_layers=1,
                      num_attention_heads=4, num_key_value_heads=2, head_dim=128)
    p = synthetic_pack(2, 2.5, seed=1)
    path = tmp_path / "packs.safetensors"
    spectral.save_packs(path, {0: (p.enc, p.dec, p.lam, {2.5: p.bits})}, (2.5,))
    # the reference's k4 name pairs full-C turboquant_mse values: it must not
    # answer with another value codec
    for arm in ("k4_b2.5", "k4_b3"):
        with pytest.raises(NotImplementedError, match="full-C turboquant_mse"):
            spec_pair(arm, pack_path=str(path))
    with pytest.raises(ValueError, match="pack-path"):
        spec_pair("k4ph_b2.5")
    for arm in ("k4ph_b2.5_lq", "k4ph_b2.5_dec8tl"):
        with pytest.raises(NotImplementedError, match="no MI355X kernels"):
            spec_pair(arm, pack_path=str(path))
    k, v = spec_pair("k4ph_b2.5", pack_path=str(path))
    assert (k.arm, k.pre_rope, k.budget, v.arm, v.bits) == ("spectral", True, 2.5, "turboquant_mse_perhead", 2)
    with pytest.raises(AssertionError, match="pre_rope"):
        PackedStreamingCache(cfg, CacheCodecSpec(arm="spectral", pack_path=str(path), budget=2.5), v)
    with pytest.raises(AssertionError, match="pack_path"):
        PackedStreamingCache(cfg, CacheCodecSpec(arm="spectral", pre_rope=True), v)
    with pytest.raises(NotImplementedError, match="turboquant_mse_perhead"):
        PackedStreamingCache(cfg, k, CacheCodecSpec(arm="turboquant_mse", bits=2))
    cache = PackedStreamingCache(cfg, k, v)
    assert torch.equal(cache._packs[0].bits, p.bits)
    with pytest.raises(KeyError, match="available"):
        PackedStreamingCache(cfg, CacheCodecSpec(arm="spectral", pre_rope=True, pack_path=str(path),
                                                 budget=3.0), v)


def test_bad_merge_arguments_are_rejected_with_message():
    lib = _lib.lib()
    m = _lib.SpectralMergeArgs()
    m.h_kv, m.n_q_groups = 9, 4
    assert lib.bmx_spectral_merge(ct.byref(m), None) != 0 and b"h_kv" in lib.bmx_last_error()
    m.h_kv, m.n_groups, m.win_len = 8, 0, 0
    assert lib.bmx_spectral_merge(ct.byref(m), None) != 0 and b"at least one token" in lib.bmx_last_error()
    m.n_groups = 16385
    assert lib.bmx_spectral_merge(ct.byref(m), None) != 0 and b"16384" in lib.bmx_last_error()
    m.n_groups = 4
    assert lib.bmx_spectral_merge(ct.byref(m), None) != 0 and b"null pointer" in lib.bmx_last_error()


def test_dequant_table_checks_precede_every_form():
    """The C-ABI carries no table lengths: short or int64 tables, and token
    counts off the 64-token grid, are refused on the host for the partial form
    too (no device call is made)."""
    pack = synthetic_pack(2, 2.5, seed=1)
    dp = spectral.DevicePack(pack, 2, "cpu")
    consts = k2b.CodecConsts.make()
    S = 256
    kp = torch.zeros(S // 64, dp.k_page_bytes, dtype=torch.uint8)
    vp = torch.zeros(S // 16, dp.v_page_bytes, dtype=torch.uint8)
    kt, vt = torch.arange(S // 64, dtype=torch.int32), torch.arange(S // 16, dtype=torch.int32)
    q = torch.zeros(2, 4, 128)
    part = torch.zeros(2, 4, 130 * (S // 64))
    bad = [(kt[:-1], vt, S), (kt, vt[:-1], S), (kt.long(), vt, S), (kt, vt.long(), S), (kt, vt, S - 32)]
    for k_t, v_t, n in bad:
        with pytest.raises(ValueError, match="k_table|multiple of 64"):
            spectral.dequant(dp, kp, k_t, vp, v_t, n, consts, apply_rope=k2b.ROPE_EXACT, q=q,
                             partials=part if n == S else torch.zeros(2, 4, 130 * (n // 64)))
        with pytest.raises(ValueError, match="k_table|multiple of 64"):
            spectral.dequant(dp, kp, k_t, vp, v_t, n, consts)

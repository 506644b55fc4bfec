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


@pytest.fixture(scope="module")
def variants():
    return np.load(GOLD / "spectral_variants.npz")


def _variant_pack(variants, budget=2.5):
    return spectral.SpectralPack(enc=torch.from_numpy(variants["enc"]), dec=torch.from_numpy(variants["dec"]),
                                 lam=torch.from_numpy(variants["lam"]),
                                 bits=torch.from_numpy(variants[f"bits_b{budget}"]))


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
    # the reference's k4 name pairs full-C turboquant_mse values (recipes.py:138-143)
    for arm, b in (("k4_b2.5", 2.5), ("k4_b3_lq_dec8tl", 3.0)):
        k4, v4 = spec_pair(arm, pack_path=str(path))
        assert (k4.arm, k4.budget, v4.arm, v4.bits) == ("spectral", b, "turboquant_mse", 2)
    c4 = PackedStreamingCache(cfg, *spec_pair("k4_b2.5", pack_path=str(path)))
    lay = c4._make_layer()
    assert lay._v_codec == "full" and lay._page_bytes() == spectral.v_page_bytes(2, "full") == 32 + 2 * 512
    cfg3 = LlamaConfig(vocab_size=64, hidden_size=384, intermediate_size=256, num_hidden_layers=1,
                       num_attention_heads=6, num_key_value_heads=3, head_dim=128)
    from bmx_amd.cache import PackedStreamingLayer
    with pytest.raises(NotImplementedError, match="power of two"):
        PackedStreamingLayer(*spec_pair("k4_b2.5", pack_path=str(path)), cfg3, pack=p)
    with pytest.raises(ValueError, match="pack-path"):
        spec_pair("k4ph_b2.5")
    kl, vl = spec_pair("k4ph_b2.5_lq", pack_path=str(path))
    assert PackedStreamingCache(cfg, kl, vl).k_spec.payload_quant == "lloyd"
    with pytest.raises(NotImplementedError, match="lloyd payloads"):
        PackedStreamingCache(cfg, CacheCodecSpec(arm="spectral", pre_rope=True, pack_path=str(path), budget=2.5,
                                                 payload_quant="nf4"), vl)
    k, v = spec_pair("k4ph_b2.5", pack_path=str(path))
    assert (k.arm, k.pre_rope, k.budget, v.arm, v.bits) == ("spectral", True, 2.5, "turboquant_mse_perhead", 2)
    with pytest.raises(AssertionError, match="pre_rope"):
        PackedStreamingCache(cfg, CacheCodecSpec(arm="spectral", pack_path=str(path), budget=2.5), v)
    with pytest.raises(AssertionError, match="pack_path"):
        PackedStreamingCache(cfg, CacheCodecSpec(arm="spectral", pre_rope=True), v)
    with pytest.raises(NotImplementedError, match="turboquant_mse_perhead"):
        PackedStreamingCache(cfg, k, CacheCodecSpec(arm="turboquant_mse", bits=3))
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


@pytest.mark.parametrize("thr", [None, 3, 5])
def test_int8_decoder_roundtrip_matches_reference(variants, thr):
    """Both restatements of int8_decoder_roundtrip give the reference's
    decoder bit for bit; columns outside the threshold (and uncoded ones)
    are untouched."""
    dec, bits = variants["dec"], variants["bits_b2.5"]
    want = variants[f"dec8_t{thr or 'all'}"]
    got_o = O.int8_decoder_roundtrip(dec, bits, thr)
    got_p = spectral.int8_decoder_roundtrip(torch.from_numpy(dec), torch.from_numpy(bits), thr).numpy()
    assert np.array_equal(got_o.view(np.uint32), want.view(np.uint32))
    assert np.array_equal(got_p.view(np.uint32), want.view(np.uint32))
    keep = (bits == 0) | ((bits > thr) if thr is not None else False)
    assert np.array_equal(want[:, keep], dec[:, keep]) and not np.array_equal(want[:, ~keep], dec[:, ~keep])


def test_int8_certificate_matches_reference(variants):
    """The certificate's three numbers at every grid threshold, both
    restatements, against the reference's (float64, matmul order aside)."""
    pack = _variant_pack(variants)
    for t in spectral.TIER_THRESHOLD_GRID:
        want = variants[f"cert_b2.5_t{t}"]
        c = spectral.int8_certificate(pack, t)
        np.testing.assert_allclose([c["added"], c["payload"], c["implied_rel_degradation"]], want, rtol=1e-12)
        np.testing.assert_allclose(O.int8_certificate(variants["enc"], variants["dec"], variants["lam"],
                                                      variants["bits_b2.5"], t), want, rtol=1e-12)
        assert c["c_int8"] == int(((variants["bits_b2.5"] > 0) & (variants["bits_b2.5"] <= t)).sum())


def test_int8_certificate_is_the_expected_weighted_distortion(variants):
    """What the closed form states, estimated: for codes y ~ N(0, diag(lam))
    the weighted error |enc^T (dec_int8 - dec) y|^2 averages to `added`
    (a column/row swap of the perturbation or a dropped lam misses by far
    more than the 3% allowed); below the lowest coded tier nothing is
    stored int8 and `added` is exactly 0; `payload` is sum lam 4^-bits."""
    enc, dec, lam, bits = (variants[k].astype(np.float64) for k in ("enc", "dec", "lam", "bits_b2.5"))
    D = O.int8_decoder_roundtrip(variants["dec"], variants["bits_b2.5"], 5).astype(np.float64) - dec
    y = np.random.default_rng(5).standard_normal((40000, lam.size)) * np.sqrt(lam)
    est = float(((y @ D.T @ enc) ** 2).sum(axis=1).mean())
    added, payload, rel = O.int8_certificate(variants["enc"], variants["dec"], variants["lam"], variants["bits_b2.5"], 5)
    assert abs(est / added - 1) < 0.03
    assert payload == pytest.approx(float((lam * 4.0 ** -bits).sum()), rel=1e-12)
    assert rel == pytest.approx(added / (added + payload), rel=1e-12)
    low = int(bits[bits > 0].min()) - 1
    assert O.int8_certificate(variants["enc"], variants["dec"], variants["lam"], variants["bits_b2.5"], low)[0] == 0.0


@pytest.mark.parametrize("bar", [0.05, 0.001, 1e-5])
def test_per_layer_tier_thresholds_match_reference(variants, bar):
    p25, p3 = _variant_pack(variants, 2.5), _variant_pack(variants, 3.0)
    want = variants[f"layer_thr_bar{bar:g}"].tolist()
    got = spectral.per_layer_tier_thresholds({0: p25, 1: p3}, bar=bar)
    assert [got[0], got[1]] == want
    layers = {i: (variants["enc"], variants["dec"], variants["lam"], p.bits.numpy()) for i, p in enumerate((p25, p3))}
    assert list(O.per_layer_tier_thresholds(layers, bar).values()) == want


def test_k4_recipe_suffixes():
    """recipes.py:100-150: '_lq' between the budget and the decoder suffix,
    '_dec8' | '_dec8t<T>' | '_dec8tl'; a misplaced '_lq' and a threshold
    outside 2..8 raise."""
    from bmx_amd.specs import spec_pair

    want = {"k4ph_b2.5": (2.5, "rtn", "fp32"), "k4ph_b2.5_dec8": (2.5, "rtn", "int8"),
            "k4ph_b3_dec8t5": (3.0, "rtn", "int8_t5"), "k4ph_b2.5_dec8tl": (2.5, "rtn", "int8_tl"),
            "k4ph_b2.5_lq": (2.5, "lloyd", "fp32"), "k4ph_b2.5_lq_dec8t3": (2.5, "lloyd", "int8_t3")}
    for arm, (b, pq, dq) in want.items():
        k, _ = spec_pair(arm, pack_path="p")
        assert (k.budget, k.payload_quant, k.dec_quant) == (b, pq, dq), arm
    for arm in ("k4ph_b2.5_dec8tl_lq", "k4ph_b2.5_dec8_lq"):
        with pytest.raises(ValueError, match="malformed"):
            spec_pair(arm, pack_path="p")
    for arm in ("k4ph_b2.5_dec8t9", "k4ph_b2.5_dec8t1", "k4ph_b2.5_dec8t"):
        with pytest.raises(ValueError, match="int8_t<T>"):
            spec_pair(arm, pack_path="p")
    assert [spectral.dec_quant_threshold(d) for d in ("fp32", "int8", "int8_t4", "int8_tl")] == \
        [None, 8, 4, spectral.PER_LAYER_TIER]


def test_int8_decoder_packs_load_once_with_their_threshold(tmp_path):
    """load_packs_for_spec (spectral.py:1254-1326): dec8t<T> roundtrips every
    layer at T, dec8tl at each layer's certified threshold, from the packs
    as loaded; enc, lam and bits are untouched and dec_tier records T; the
    cache holds exactly these packs."""
    from transformers import LlamaConfig

    from bmx_amd.cache import PackedStreamingCache
    from bmx_amd.specs import spec_pair

    layers = {i: synthetic_pack(2, 2.5, seed=60 + i) for i in range(2)}
    path = tmp_path / "packs.safetensors"
    spectral.save_packs(path, {i: (p.enc, p.dec, p.lam, {2.5: p.bits}) for i, p in layers.items()}, (2.5,))
    t_map = spectral.per_layer_tier_thresholds(layers)
    for arm, thr in (("k4ph_b2.5_dec8t4", {0: 4, 1: 4}), ("k4ph_b2.5_dec8", {0: 8, 1: 8}),
                     ("k4ph_b2.5_dec8tl", t_map), ("k4ph_b2.5", {0: None, 1: None})):
        k, _ = spec_pair(arm, pack_path=str(path))
        packs = spectral.load_packs_for_spec(k)
        for i, p in layers.items():
            q = packs[i]
            assert q.dec_tier == thr[i] and torch.equal(q.enc, p.enc) and torch.equal(q.bits, p.bits)
            want = p.dec if thr[i] is None else O.int8_decoder_roundtrip(p.dec.numpy(), p.bits.numpy(), thr[i])
            assert np.array_equal(np.asarray(q.dec), np.asarray(want))
    cfg = LlamaConfig(vocab_size=64, hidden_size=256, intermediate_size=256, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=2, head_dim=128)
    cache = PackedStreamingCache(cfg, *spec_pair("k4ph_b2.5_dec8t4", pack_path=str(path)))
    assert cache._packs[1].dec_tier == 4


def test_mixed_decoder_charge():
    """mixed_dec_charge (spectral.py:1036-1064) at its two ends: all fp16
    columns 16 c_used / S, all int8 8 c_used / S + 16 c_used / (S C), plus
    the tier map's ceil(log2 7) / S; linear in between."""
    C, S, tiers = 256, 1000, spectral.TIERS
    tb = 3 / S
    assert spectral.mixed_dec_charge(C, S, tiers, 100, 0) == pytest.approx(16 * 100 / S + tb, rel=1e-15)
    assert spectral.mixed_dec_charge(C, S, tiers, 100, 100) == pytest.approx(8 * 100 / S + 1600 / (S * C) + tb,
                                                                            rel=1e-15)
    mid = spectral.mixed_dec_charge(C, S, tiers, 100, 50)
    assert mid == pytest.approx(0.5 * (spectral.mixed_dec_charge(C, S, tiers, 100, 0)
                                       + spectral.mixed_dec_charge(C, S, tiers, 100, 100)), rel=1e-14)
    with pytest.raises(ValueError):
        spectral.mixed_dec_charge(C, S, tiers, 100, 101)


def _lloyd_levels(variants):
    return {b: variants[f"codebook_{b}"] for b in (2, 3, 4, 5, 6, 8)}


def test_lloyd_payload_matches_reference(variants):
    """The oracle's Lloyd payload on the reference's Y: every level index of
    every tier equal, the steps within 2e-6 (the refits' fp32 sums run in a
    fixed order here), the dequantized keys (fp32 steps) within 1e-5; pages
    round-trip the indices."""
    bits = variants["bits_b2.5"]
    L = O.Layout(bits)
    lloyd = _lloyd_levels(variants)
    codes, scales = O.quantize(L.permute_cols(variants["Y"]), L, lloyd)
    for b, c in O.tier_columns(bits).items():
        k = np.array([np.nonzero(L.perm == x)[0][0] for x in c])
        mine = codes[:, :, k].transpose(2, 0, 1).reshape(len(c), -1)
        np.testing.assert_array_equal(mine, variants[f"lq_codes_t{b}"])
        assert np.abs(scales[:, k].T / variants[f"lq_scale_t{b}"][..., 0] - 1).max() < 2e-6
    Mh = O.dequant(codes, scales, variants["dec"], L, fp16_scales=False, lloyd=lloyd)
    assert np.abs(Mh - variants["lq_M_hat"]).max() < 1e-5
    c2, s2 = O.unpack_pages(O.pack_pages(codes, scales, L, lloyd=True), L, lloyd=True)
    assert np.array_equal(c2, codes) and np.array_equal(s2, scales.astype(np.float16).astype(np.float32))
    assert codes.min() >= 0 and all(codes[:, :, L.col_bits == b].max() < 2 ** b for b in set(L.slice_bits.tolist()))


def test_lloyd_codes_are_nearest_levels_and_refits_matter(variants):
    """What the payload is, checked without its formulas: each index names
    the level nearest to value / step (a midpoint off by one level, or codes
    bucketized against the levels instead of the midpoints, fails it), and
    the step is the least-squares one for the final indices up to their
    last reassignment; without the 3 refits the indices change."""
    cb = variants["codebook_3"]
    G = variants["Y"][:, :40].T.reshape(-1, 64)[:160].astype(np.float32)
    q, s = O.lloyd_quantize_groups(G, cb)
    x = G / s[:, None]
    dist = np.abs(x[..., None] - cb[None, None, :].astype(np.float64))
    assert np.all(dist[np.arange(G.shape[0])[:, None], np.arange(64)[None, :], q] <= dist.min(axis=2) + 1e-12)
    q0, _ = O.lloyd_quantize_groups(G, cb, n_iter=0)
    assert (q0 != q).any()
    lv = cb[q].astype(np.float64)
    ls = (G * lv).sum(1) / (lv * lv).sum(1)
    assert np.median(np.abs(ls / s - 1)) < 1e-3


def test_lloyd_level_table_is_the_reference_codebook(variants):
    """The device table the kernels read: gaussian_codebook(b) of b = 2, 3,
    4, 5, 6, 8 at offsets 2^b - 4 and 124, equal to the reference's."""
    t = spectral.lloyd_levels("cpu").numpy()
    for b in (2, 3, 4, 5, 6, 8):
        off = 124 if b == 8 else 2 ** b - 4
        assert np.array_equal(t[off: off + 2 ** b], variants[f"codebook_{b}"])
    dp = spectral.DevicePack(synthetic_pack(2, 2.5, seed=1), 2, "cpu", "lloyd")
    assert dp.layout().lloyd_levels == dp.lloyd_levels.data_ptr()
    assert spectral.DevicePack(synthetic_pack(2, 2.5, seed=1), 2, "cpu").layout().lloyd_levels is None


@pytest.mark.parametrize("h_kv", [2, 8])
def test_full_c_value_codec_matches_reference(h_kv):
    """The oracle's value codec at h = 1 is the reference's full-C
    turboquant_mse (tests/golden/tq_full.npz): every index and fp16 norm, the
    dequantized values, the bpe; the C-wide signs the kernels take are the
    reference's _hadamard_signs(C, 0)."""
    from oracle import codecs as OC

    z = np.load(GOLD / "tq_full.npz")
    M = OC.to_matrix(torch.from_numpy(z[f"h{h_kv}_v"]).float())
    idx, norms, bpe = OC.quantize_v_perhead(M, bits=2, seed=0, h=1)
    assert np.array_equal(idx.numpy(), z[f"h{h_kv}_idx"]) and np.array_equal(norms.numpy(), z[f"h{h_kv}_norms"])
    assert bpe == float(z[f"h{h_kv}_bpe"]) == 2 + 16 / (128 * h_kv)
    deq = OC.dequant_v_perhead(idx, norms, bits=2, seed=0, h=1)
    np.testing.assert_allclose(deq.numpy(), z[f"h{h_kv}_deq"], rtol=0, atol=1e-6)
    signs = z[f"signs_d{128 * h_kv}_s0"]
    words = spectral.v_sign_bits_c(h_kv, 0)
    assert len(words) == 32
    bits = np.array([(words[c >> 5] >> (c & 31)) & 1 for c in range(128 * h_kv)])
    assert np.array_equal(bits, (signs < 0).astype(int)) and not any(words[4 * h_kv:])


def test_full_c_value_rotation_is_the_kronecker_form():
    """What the kernels use in place of a C-point FWHT per token: the
    C-point Hadamard is H_{C/128} (x) H_128 in the index order (slice,
    channel), so head h's values are H_128 of the slices' sum signed by
    row h of H_{C/128}."""
    from oracle import codecs as OC

    h_kv = 8
    z = np.random.default_rng(3).standard_normal((5, 128 * h_kv)).astype(np.float32)
    full = OC.fwht(torch.from_numpy(z)).numpy() * np.sqrt(128 * h_kv)
    for h in range(h_kv):
        comb = sum((-1) ** bin(h & sl).count("1") * z[:, 128 * sl: 128 * (sl + 1)] for sl in range(h_kv))
        mine = OC.fwht(torch.from_numpy(comb.astype(np.float32))).numpy() * np.sqrt(128)
        np.testing.assert_allclose(mine, full[:, 128 * h: 128 * (h + 1)], rtol=1e-4, atol=1e-4)

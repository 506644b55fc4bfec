"""Spectral (K4) key path on the GPU against the CPU oracle (oracle/spectral.py,
pinned to the reference's golden vectors): the write kernel's pages byte for
byte, the dequant kernel's keys (fp16 MFMA reconstruction: bounded by the
inputs' fp16 rounding) and values, and attention over the dequantized cache."""

import numpy as np
import pytest
import torch

from bmx_amd import k2b, spectral
from oracle import attention as A
from oracle import codecs as OC
from oracle import layout as OL
from oracle import spectral as O

from tests.spectral_util import GOLD, golden_pack, synthetic_pack, synthetic_keys

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _values_of(vpages: np.ndarray, h_kv: int):
    """(codes, fp16 norms) of value-only pages through the k2b page reader."""
    sec = OL.sections(h_kv, 16)
    full = np.zeros((vpages.shape[0], sec["total"][1]), np.uint8)
    nv, nc = h_kv * 32, h_kv * 512
    full[:, sec["vnorm"][0]: sec["vnorm"][0] + nv] = vpages[:, :nv]
    full[:, sec["vcode"][0]: sec["vcode"][0] + nc] = vpages[:, nv: nv + nc]
    _, _, _, vidx, vn16 = OL.unpack_pages(full, h_kv, 16)
    return vidx, vn16


def _lloyd(payload):
    """The oracle's Lloyd levels per tier (the reference's codebooks, from the
    golden file), or None for the rtn payload."""
    if payload == "rtn":
        return None
    z = np.load(GOLD / "spectral_variants.npz")
    return {b: z[f"codebook_{b}"] for b in (2, 3, 4, 5, 6, 8)}


def _values_full_of(vpages: np.ndarray, h_kv: int):
    """(codes (16 n, C), fp16 norms (16 n,)) of n full-C value pages, in order
    (the layout of include/bmx_spectral.h)."""
    n, C = vpages.shape[0], 128 * h_kv
    norms = vpages[:, :32].copy().view(np.float16).reshape(-1)
    words = vpages[:, 32: 32 + 512 * h_kv].copy().view("<u4").reshape(n, h_kv, 64, 2)
    codes = np.zeros((n, 16, C), np.int64)
    for sl in range(h_kv):
        for lane in range(64):
            q, m = lane >> 4, lane & 15
            for w in range(2):
                dw = words[:, sl, lane, w].astype(np.int64)
                for bb in range(4):
                    for t in range(4):
                        codes[:, 4 * q + t, 128 * sl + 16 * (4 * w + bb) + m] = (dw >> (8 * bb + 2 * t)) & 3
    return codes.reshape(16 * n, C), norms


def _values_oracle(v, h_kv, v_codec):
    """The oracle's dequantized values (h_kv, S, 128) of either value codec."""
    h = 1 if v_codec == "full" else h_kv
    idx, norms, _ = OC.quantize_v_perhead(OC.to_matrix(v), bits=2, seed=0, h=h)
    return OC.from_matrix(OC.dequant_v_perhead(idx, norms, bits=2, seed=0, h=h), h_kv)


def _write(pack, h_kv, M, v, consts, shuffle_seed=None, payload="rtn", v_codec="perhead"):
    """Append keys M (S, C) and values v (h_kv, S, 128) through the C-ABI into
    pools with (optionally shuffled) page ids; returns (dp, kp, vp, k_ids, v_ids)."""
    S = M.shape[0]
    dp = spectral.DevicePack(pack, h_kv, DEV, payload, v_codec)
    ng = S // 64
    k_ids = torch.arange(ng, dtype=torch.int32)
    v_ids = torch.arange(4 * ng, dtype=torch.int32)
    if shuffle_seed is not None:
        g = torch.Generator().manual_seed(shuffle_seed)
        k_ids = k_ids[torch.randperm(ng, generator=g)].to(torch.int32)
        v_ids = v_ids[torch.randperm(4 * ng, generator=g)].to(torch.int32)
    kp = torch.zeros(ng, dp.k_page_bytes, dtype=torch.uint8, device=DEV)
    vp = torch.zeros(4 * ng, dp.v_page_bytes, dtype=torch.uint8, device=DEV)
    k_pre = OC.from_matrix(torch.from_numpy(M).float(), h_kv)
    spectral.append(k_pre.to(DEV), v.to(DEV), dp, kp, k_ids.to(DEV), vp, v_ids.to(DEV), consts)
    torch.cuda.synchronize()
    return dp, kp, vp, k_ids.to(DEV), v_ids.to(DEV)


CASES = ["golden_h2", "synthetic_h8", "synthetic_h8_b3"]


def _case(name):
    if name == "golden_h2":
        pack, M = golden_pack()
        return pack, 2, M
    budget = 3.0 if name.endswith("b3") else 2.5
    pack = synthetic_pack(8, budget, seed=5)
    return pack, 8, synthetic_keys(pack, 512, seed=6)


@pytest.mark.parametrize("payload", ["rtn", "lloyd"])
@pytest.mark.parametrize("name", CASES)
def test_append_pages_match_oracle(name, payload):
    """Every key page byte equals the oracle's page (encode in the fixed order,
    MSE-refined RTN or the Lloyd payload, container packing), and the value
    pages hold the k2b value codec's codes and fp16 norms."""
    pack, h_kv, M = _case(name)
    print(f"case {name} {payload}: h_kv {h_kv}, S {M.shape[0]}", flush=True)
    gen = torch.Generator().manual_seed(3)
    v = torch.randn(h_kv, M.shape[0], 128, generator=gen)
    consts = k2b.CodecConsts.make(v_seed=0)
    dp, kp, vp, k_ids, v_ids = _write(pack, h_kv, M, v, consts, shuffle_seed=1, payload=payload)
    L = O.Layout(pack.bits.numpy())
    assert (L.c_pad, L.page_bytes) == (dp.c_pad, dp.k_page_bytes)
    assert np.array_equal(L.slice_table(), dp.slice_tab.cpu().numpy())
    lloyd = _lloyd(payload)
    codes, scales = O.quantize(O.encode(M, pack.enc.numpy(), L), L, lloyd)
    want = O.pack_pages(codes, scales, L, lloyd=lloyd is not None)
    got = kp[k_ids.long()].cpu().numpy()
    bad = np.nonzero((got != want).any(axis=1))[0]
    print(f"key pages differing: {len(bad)}/{len(want)}; c_pad {L.c_pad}, tiers "
          f"{sorted(set(L.slice_bits.tolist()))}", flush=True)
    assert len(bad) == 0
    vidx, vn16 = _values_of(vp[v_ids.long()].cpu().numpy(), h_kv)
    idx, norms, _ = OC.quantize_v_perhead(OC.to_matrix(v), bits=2, seed=0, h=h_kv)
    np.testing.assert_array_equal(vn16.astype(np.float32), norms.numpy())
    assert int((vidx != idx.numpy()).sum()) == 0


@pytest.mark.parametrize("payload", ["rtn", "lloyd"])
@pytest.mark.parametrize("name", CASES)
def test_dequant_matches_oracle(name, payload):
    """Keys: Y_hat dec^T from the pages (fp16 steps, as stored) within the
    fp16 rounding of the MFMA inputs (code or level times step, and dec),
    pre-RoPE and rotated (fp32 and fp16 tables); values as the k2b value
    codec; dtypes rounded once from the fp32 result."""
    pack, h_kv, M = _case(name)
    S = M.shape[0]
    gen = torch.Generator().manual_seed(4)
    v = torch.randn(h_kv, S, 128, generator=gen)
    consts = k2b.CodecConsts.make(v_seed=0)
    dp, kp, vp, k_ids, v_ids = _write(pack, h_kv, M, v, consts, shuffle_seed=2, payload=payload)
    L = O.Layout(pack.bits.numpy())
    lloyd = _lloyd(payload)
    codes, scales = O.quantize(O.encode(M, pack.enc.numpy(), L), L, lloyd)
    K_or = OC.from_matrix(torch.from_numpy(O.dequant(codes, scales, pack.dec.numpy(), L, lloyd=lloyd)), h_kv)
    Kp, Vd = spectral.dequant(dp, kp, k_ids, vp, v_ids, S, consts)
    kmax = K_or.abs().max().item()
    err = (Kp.cpu().double() - K_or).abs().max().item()
    print(f"{name} {payload}: pre-RoPE keys max_abs {err:.3e} (max|K| {kmax:.3f}, rel {err / kmax:.2e})",
          flush=True)
    assert err <= 1.5e-3 * kmax
    inv = torch.tensor(consts.inv_freq)
    cos, sin = A.rope_cos_sin(inv, torch.arange(S))
    Kr, _ = spectral.dequant(dp, kp, k_ids, vp, v_ids, S, consts, apply_rope=k2b.ROPE_EXACT)
    err_r = (Kr.cpu().double() - A.apply_rope(K_or.float(), cos, sin).double()).abs().max().item()
    assert err_r <= 1.5e-3 * kmax
    idx, norms, _ = OC.quantize_v_perhead(OC.to_matrix(v), bits=2, seed=0, h=h_kv)
    V_or = OC.from_matrix(OC.dequant_v_perhead(idx, norms, bits=2, seed=0, h=h_kv), h_kv)
    assert (Vd.cpu() - V_or).abs().max().item() < 1e-4
    Kt, _ = spectral.dequant(dp, kp, k_ids, vp, v_ids, S, consts, apply_rope=k2b.ROPE_FP16_TABLES)
    for dt in (torch.float16, torch.bfloat16):
        Kh, Vh = spectral.dequant(dp, kp, k_ids, vp, v_ids, S, consts, apply_rope=k2b.ROPE_FP16_TABLES,
                                  dtype=dt)
        assert Kh.dtype == dt and torch.equal(Kh, Kt.to(dt)) and torch.equal(Vh, Vd.to(dt))


def test_attention_over_dequantized_pages():
    """Grouped decode attention over the dequantized cache (RoPE'd keys and
    the fp16 window) against the oracle's dense attention over the same
    codes: the spectral decode step's numerics, at the decode bar."""
    pack = synthetic_pack(8, 2.5, seed=8)
    S, T, G = 1024, 40, 4
    M = synthetic_keys(pack, S, seed=9)
    gen = torch.Generator().manual_seed(10)
    v = torch.randn(8, S, 128, generator=gen)
    consts = k2b.CodecConsts.make(v_seed=0)
    dp, kp, vp, k_ids, v_ids = _write(pack, 8, M, v, consts)
    Kd, Vd = spectral.dequant(dp, kp, k_ids, vp, v_ids, S, consts, apply_rope=k2b.ROPE_EXACT,
                              dtype=torch.float16)
    kt = torch.randn(8, T, 128, generator=gen).half()
    vt = torch.randn(8, T, 128, generator=gen).half()
    q = torch.randn(8 * G, 1, 128, generator=gen)
    scale = 128 ** -0.5
    K = torch.cat([Kd, kt.to(DEV)], 1)
    V = torch.cat([Vd, vt.to(DEV)], 1)
    out = torch.nn.functional.scaled_dot_product_attention(
        q.half().to(DEV).unsqueeze(0), K.unsqueeze(0), V.unsqueeze(0), scale=scale, enable_gqa=True)[0]
    L = O.Layout(pack.bits.numpy())
    codes, scales = O.quantize(O.encode(M, pack.enc.numpy(), L), L)
    K_or = OC.from_matrix(torch.from_numpy(O.dequant(codes, scales, pack.dec.numpy(), L)).float(), 8)
    cos, sin = A.rope_cos_sin(torch.tensor(consts.inv_freq), torch.arange(S))
    idx, norms, _ = OC.quantize_v_perhead(OC.to_matrix(v), bits=2, seed=0, h=8)
    V_or = OC.from_matrix(OC.dequant_v_perhead(idx, norms, bits=2, seed=0, h=8), 8)
    ref = A.naive_dense_attention(q.half().float(), torch.cat([A.apply_rope(K_or, cos, sin), kt.float()], 1),
                                  torch.cat([V_or, vt.float()], 1), G, scale)
    o = out.float().cpu().double()
    err = (o - ref.double()).abs().max().item()
    rel = ((o - ref.double()).norm() / ref.double().norm()).item()
    print(f"attention over spectral pages: max_abs {err:.3e} rel {rel:.3e}", flush=True)
    assert err <= 2e-3 and rel <= 1e-2


def test_decode_form_scores_match_keys():
    """The decode form's scores equal q . k of the kernel's own rotated keys
    (fp16 keys and queries, fp32 accumulation) and of the oracle's keys, for
    G 1 and 4 and a buffer with rows left for a window; its values equal the
    keys-and-values form's."""
    pack = synthetic_pack(8, 2.5, seed=11)
    S, extra = 512, 24
    M = synthetic_keys(pack, S, seed=12)
    gen = torch.Generator().manual_seed(13)
    v = torch.randn(8, S, 128, generator=gen)
    consts = k2b.CodecConsts.make(v_seed=0)
    dp, kp, vp, k_ids, v_ids = _write(pack, 8, M, v, consts, shuffle_seed=3)
    K, V = spectral.dequant(dp, kp, k_ids, vp, v_ids, S, consts, apply_rope=k2b.ROPE_FP16_TABLES,
                            dtype=torch.float16)
    L = O.Layout(pack.bits.numpy())
    codes, scales = O.quantize(O.encode(M, pack.enc.numpy(), L), L)
    K_or = OC.from_matrix(torch.from_numpy(O.dequant(codes, scales, pack.dec.numpy(), L)).float(), 8)
    from bmx_amd.cache import _rope_tables

    c16, s16 = _rope_tables(torch.tensor(consts.inv_freq), consts.rope_scaling, 0, S, "cpu")
    K_or = K_or * c16.float() + torch.cat((-K_or[..., 64:], K_or[..., :64]), -1) * s16.float()
    for G in (1, 4):
        q = torch.randn(8, G, 128, generator=gen).half()
        Vb = torch.zeros(8, S + extra, 128, dtype=torch.float16, device=DEV)
        Sb = torch.zeros(8, G, S + extra, dtype=torch.float32, device=DEV)
        spectral.dequant(dp, kp, k_ids, vp, v_ids, S, consts, apply_rope=k2b.ROPE_FP16_TABLES,
                         dtype=torch.float16, out=(None, Vb), q=q.to(DEV), scores=Sb)
        own = torch.bmm(q.float().to(DEV), K.float().transpose(1, 2).contiguous())
        d_own = (Sb[:, :, :S] - own).abs().max().item()
        want = q.float() @ K_or.transpose(1, 2)
        d_or = (Sb[:, :, :S].cpu() - want).abs().max().item()
        smax = want.abs().max().item()
        print(f"G {G}: scores vs own keys {d_own:.3e}, vs oracle keys {d_or:.3e} (max {smax:.2f})", flush=True)
        assert d_own <= 1e-5 * smax and d_or <= 3e-3 * smax
        assert torch.equal(Vb[:, :S], V) and not Vb[:, S:].any() and not Sb[:, :, S:].any()


PARTIAL_CASES = [
    # (h_kv, G, T, rope, S): the exact-RoPE form runs on 64-token groups; the
    # fp16-table form on 128-token blocks of 4 heads when S is a multiple of
    # 128 (ragged head counts leave waves of the last workgroup idle), else on
    # 64-token groups
    (8, 4, 40, k2b.ROPE_EXACT, 1024), (8, 1, 0, k2b.ROPE_EXACT, 1024), (8, 8, 7, k2b.ROPE_EXACT, 1024),
    (8, 16, 40, k2b.ROPE_EXACT, 1024),
    (8, 4, 40, k2b.ROPE_FP16_TABLES, 1024), (8, 16, 7, k2b.ROPE_FP16_TABLES, 2048),
    (8, 1, 0, k2b.ROPE_FP16_TABLES, 1088), (3, 8, 40, k2b.ROPE_FP16_TABLES, 512),
    (2, 5, 3, k2b.ROPE_FP16_TABLES, 256),
]


@pytest.mark.parametrize("payload", ["rtn", "lloyd"])
@pytest.mark.parametrize("h_kv,G,T,rope,S", PARTIAL_CASES)
def test_partial_form_decode_matches_oracle(h_kv, G, T, rope, S, payload):
    """The decode step through the kernel's partial form (per-block softmax
    partials) and the merge with the window: against the oracle's one-softmax
    attention over the same codes (RoPE by fp32 tables, or by the fp16-rounded
    tables of an fp16 model), and against the scores form + softmax."""
    pack = synthetic_pack(h_kv, 2.5, seed=14)
    M = synthetic_keys(pack, S, seed=15)
    gen = torch.Generator().manual_seed(16)
    v = torch.randn(h_kv, S, 128, generator=gen)
    consts = k2b.CodecConsts.make(v_seed=0)
    dp, kp, vp, k_ids, v_ids = _write(pack, h_kv, M, v, consts, shuffle_seed=4, payload=payload)
    lloyd = _lloyd(payload)
    kt = torch.randn(h_kv, T, 128, generator=gen).half()
    vt = torch.randn(h_kv, T, 128, generator=gen).half()
    q = torch.randn(h_kv, G, 128, generator=gen).half()
    scale = 128 ** -0.5
    n_parts = spectral.partial_count(dp, S, q.to(DEV), rope)
    blocked = rope == k2b.ROPE_FP16_TABLES and S % 128 == 0 and 2 * dp.k_page_bytes <= 57344
    assert n_parts == (S // 128 if blocked else S // 64)
    out = spectral.decode_attention(dp, kp, k_ids, vp, v_ids, S, consts, q.to(DEV), scale,
                                    k_win=kt.to(DEV) if T else None, v_win=vt.to(DEV) if T else None,
                                    apply_rope=rope, out_dtype=torch.float32)
    L = O.Layout(pack.bits.numpy())
    codes, scales = O.quantize(O.encode(M, pack.enc.numpy(), L), L, lloyd)
    K_or = OC.from_matrix(torch.from_numpy(O.dequant(codes, scales, pack.dec.numpy(), L, lloyd=lloyd)).float(),
                          h_kv)
    cos, sin = A.rope_cos_sin(torch.tensor(consts.inv_freq), torch.arange(S))
    if rope == k2b.ROPE_FP16_TABLES:
        cos, sin = cos.half().float(), sin.half().float()
    idx, norms, _ = OC.quantize_v_perhead(OC.to_matrix(v), bits=2, seed=0, h=h_kv)
    V_or = OC.from_matrix(OC.dequant_v_perhead(idx, norms, bits=2, seed=0, h=h_kv), h_kv)
    ref = A.naive_dense_attention(q.reshape(h_kv * G, 1, 128).float(),
                                  torch.cat([A.apply_rope(K_or, cos, sin), kt.float()], 1),
                                  torch.cat([V_or, vt.float()], 1), G, scale).reshape(h_kv, G, 128)
    o = out.cpu().double()
    err = (o - ref.double()).abs().max().item()
    rel = ((o - ref.double()).norm() / ref.double().norm()).item()
    # the scores form + one softmax + value product, same kernel inputs
    Vb = torch.empty(h_kv, S, 128, dtype=torch.float16, device=DEV)
    Sb = torch.empty(h_kv, G, S, dtype=torch.float32, device=DEV)
    spectral.dequant(dp, kp, k_ids, vp, v_ids, S, consts, apply_rope=rope, dtype=torch.float16,
                     out=(None, Vb), q=q.to(DEV), scores=Sb)
    sw = torch.cat([Sb, (q.float() @ kt.float().transpose(1, 2)).to(DEV)], -1) * scale
    Vw = torch.cat([Vb.float(), vt.float().to(DEV)], 1)
    alt = (torch.softmax(sw, -1) @ Vw).cpu().double()
    d_alt = (o - alt).abs().max().item()
    print(f"{payload} h_kv {h_kv} G {G} T {T} rope {rope} S {S} ({n_parts} partials): partial-form decode vs oracle "
          f"max_abs {err:.3e} rel {rel:.3e}; vs scores form {d_alt:.3e}", flush=True)
    assert err <= 2e-3 and rel <= 1e-2 and d_alt <= 2e-3


@pytest.mark.parametrize("G", [4, 16])
def test_window_only_decode_step(G):
    """A decode step with no committed token (a layer before its first
    commit): only the merge runs, over the fp16 window; the layer may have no
    device pack yet."""
    gen = torch.Generator().manual_seed(21)
    T = 45
    kt = torch.randn(8, T, 128, generator=gen).half()
    vt = torch.randn(8, T, 128, generator=gen).half()
    q = torch.randn(8, G, 128, generator=gen).half()
    consts = k2b.CodecConsts.make(v_seed=0)
    scale = 128 ** -0.5
    ref = A.naive_dense_attention(q.reshape(8 * G, 1, 128).float(), kt.float(), vt.float(), G,
                                  scale).reshape(8, G, 128)
    for dp in (None, spectral.DevicePack(synthetic_pack(8, 2.5, seed=14), 8, DEV)):
        out = spectral.decode_attention(dp, None, None, None, None, 0, consts, q.to(DEV), scale,
                                        k_win=kt.to(DEV), v_win=vt.to(DEV), out_dtype=torch.float32)
        err = (out.cpu().double() - ref.double()).abs().max().item()
        print(f"window only G {G} (pack {'given' if dp is not None else 'absent'}): max_abs {err:.3e}", flush=True)
        assert err <= 2e-3


@pytest.mark.parametrize("h_kv", [1, 2, 4, 8])
def test_full_c_values_pages_and_dequant(h_kv):
    """The k4 recipe's full-C turboquant_mse values: every value page's codes
    and fp16 norm equal the oracle's (the reference's codec at h = 1), on
    shuffled pages; the dense values (the prefill form) within 1e-4 of the
    oracle's, each head's channels from the Kronecker form of the C-point
    inverse rotation; the keys as with the per-head values."""
    pack = synthetic_pack(h_kv, 2.5, seed=21)
    S = 256
    M = synthetic_keys(pack, S, seed=22)
    v = (torch.randn(h_kv, S, 128, generator=torch.Generator().manual_seed(23)) * 1.3).half().float()
    consts = k2b.CodecConsts.make(v_seed=0)
    print(f"full-C values h_kv {h_kv}", flush=True)
    dp, kp, vp, k_ids, v_ids = _write(pack, h_kv, M, v, consts, shuffle_seed=5, v_codec="full")
    assert dp.v_page_bytes == 32 + 512 * h_kv
    codes, n16 = _values_full_of(vp[v_ids.long()].cpu().numpy(), h_kv)
    idx, norms, _ = OC.quantize_v_perhead(OC.to_matrix(v), bits=2, seed=0, h=1)
    assert np.array_equal(n16.astype(np.float32), norms.numpy()[:, 0])
    assert int((codes != idx.numpy()).sum()) == 0
    V_or = _values_oracle(v, h_kv, "full")
    Kp, Vd = spectral.dequant(dp, kp, k_ids, vp, v_ids, S, consts)
    err = (Vd.cpu() - V_or).abs().max().item()
    print(f"full-C values h_kv {h_kv}: dense values max_abs {err:.3e} (max {V_or.abs().max():.3f})", flush=True)
    assert err < 1e-4
    L = O.Layout(pack.bits.numpy())
    codes_k, scales = O.quantize(O.encode(M, pack.enc.numpy(), L), L)
    K_or = OC.from_matrix(torch.from_numpy(O.dequant(codes_k, scales, pack.dec.numpy(), L)), h_kv)
    assert (Kp.cpu().double() - K_or).abs().max().item() <= 1.5e-3 * K_or.abs().max().item()


FULL_CASES = [
    # (h_kv, G, T, rope, S, payload)
    (8, 4, 40, k2b.ROPE_FP16_TABLES, 1024, "rtn"), (8, 16, 7, k2b.ROPE_FP16_TABLES, 2048, "rtn"),
    (8, 4, 40, k2b.ROPE_EXACT, 1024, "rtn"), (8, 16, 0, k2b.ROPE_EXACT, 512, "lloyd"),
    (4, 8, 40, k2b.ROPE_FP16_TABLES, 512, "lloyd"), (2, 5, 3, k2b.ROPE_FP16_TABLES, 256, "rtn"),
    (1, 8, 7, k2b.ROPE_FP16_TABLES, 256, "rtn"), (8, 1, 0, k2b.ROPE_FP16_TABLES, 1088, "rtn"),
]


@pytest.mark.parametrize("h_kv,G,T,rope,S,payload", FULL_CASES)
def test_full_c_values_decode_matches_oracle(h_kv, G, T, rope, S, payload):
    """The decode step with full-C values (both partial kernels: each head's
    P.V over every slice with the weights signed by H_{C/128}, the merge's
    H16, the head's C-wide signs and 1/C) against the oracle's one-softmax
    attention over the same codes, and against the scores form + softmax."""
    pack = synthetic_pack(h_kv, 2.5, seed=24)
    M = synthetic_keys(pack, S, seed=25)
    gen = torch.Generator().manual_seed(26)
    v = torch.randn(h_kv, S, 128, generator=gen)
    consts = k2b.CodecConsts.make(v_seed=0)
    dp, kp, vp, k_ids, v_ids = _write(pack, h_kv, M, v, consts, shuffle_seed=6, payload=payload, v_codec="full")
    kt = torch.randn(h_kv, T, 128, generator=gen).half()
    vt = torch.randn(h_kv, T, 128, generator=gen).half()
    q = torch.randn(h_kv, G, 128, generator=gen).half()
    scale = 128 ** -0.5
    n_parts = spectral.partial_count(dp, S, q.to(DEV), rope)
    out = spectral.decode_attention(dp, kp, k_ids, vp, v_ids, S, consts, q.to(DEV), scale,
                                    k_win=kt.to(DEV) if T else None, v_win=vt.to(DEV) if T else None,
                                    apply_rope=rope, out_dtype=torch.float32)
    lloyd = _lloyd(payload)
    L = O.Layout(pack.bits.numpy())
    codes, scales = O.quantize(O.encode(M, pack.enc.numpy(), L), L, lloyd)
    K_or = OC.from_matrix(torch.from_numpy(O.dequant(codes, scales, pack.dec.numpy(), L, lloyd=lloyd)).float(),
                          h_kv)
    cos, sin = A.rope_cos_sin(torch.tensor(consts.inv_freq), torch.arange(S))
    if rope == k2b.ROPE_FP16_TABLES:
        cos, sin = cos.half().float(), sin.half().float()
    V_or = _values_oracle(v, h_kv, "full")
    ref = A.naive_dense_attention(q.reshape(h_kv * G, 1, 128).float(),
                                  torch.cat([A.apply_rope(K_or, cos, sin), kt.float()], 1),
                                  torch.cat([V_or, vt.float()], 1), G, scale).reshape(h_kv, G, 128)
    o = out.cpu().double()
    err = (o - ref.double()).abs().max().item()
    rel = ((o - ref.double()).norm() / ref.double().norm()).item()
    Vb = torch.empty(h_kv, S, 128, dtype=torch.float16, device=DEV)
    Sb = torch.empty(h_kv, G, S, dtype=torch.float32, device=DEV)
    spectral.dequant(dp, kp, k_ids, vp, v_ids, S, consts, apply_rope=rope, dtype=torch.float16,
                     out=(None, Vb), q=q.to(DEV), scores=Sb)
    sw = torch.cat([Sb, (q.float() @ kt.float().transpose(1, 2)).to(DEV)], -1) * scale
    Vw = torch.cat([Vb.float(), vt.float().to(DEV)], 1)
    alt = (torch.softmax(sw, -1) @ Vw).cpu().double()
    d_alt = (o - alt).abs().max().item()
    print(f"full-C {payload} h_kv {h_kv} G {G} T {T} rope {rope} S {S} ({n_parts} partials): decode vs oracle "
          f"max_abs {err:.3e} rel {rel:.3e}; vs scores form {d_alt:.3e}", flush=True)
    assert err <= 2e-3 and rel <= 1e-2 and d_alt <= 2e-3


@pytest.mark.parametrize("payload", ["rtn", "lloyd"])
def test_full_c_values_decode_long_context(payload):
    """The reference's k4_b2.5 recipe (rtn payload) and its Lloyd-payload
    variant k4_b2.5_lq at 32,768 committed tokens + a 128-token fp16 window
    (h_kv 8, G 4, the fp16 RoPE tables of an fp16 model): a bias of the
    kernels' fp16 levels or scales that is invisible over a few thousand
    tokens accumulates here.  Against the oracle's one-softmax attention over
    the same codes at the north-star bar, and against the scores form."""
    h_kv, G, T, S = 8, 4, 128, 32768
    rope = k2b.ROPE_FP16_TABLES
    pack = synthetic_pack(h_kv, 2.5, seed=34)
    M = synthetic_keys(pack, S, seed=35)
    gen = torch.Generator().manual_seed(36)
    v = torch.randn(h_kv, S, 128, generator=gen)
    consts = k2b.CodecConsts.make(v_seed=0)
    dp, kp, vp, k_ids, v_ids = _write(pack, h_kv, M, v, consts, shuffle_seed=7, payload=payload, v_codec="full")
    kt = torch.randn(h_kv, T, 128, generator=gen).half()
    vt = torch.randn(h_kv, T, 128, generator=gen).half()
    q = torch.randn(h_kv, G, 128, generator=gen).half()
    scale = 128 ** -0.5
    out = spectral.decode_attention(dp, kp, k_ids, vp, v_ids, S, consts, q.to(DEV), scale,
                                    k_win=kt.to(DEV), v_win=vt.to(DEV), apply_rope=rope, out_dtype=torch.float32)
    torch.cuda.synchronize()
    lloyd = _lloyd(payload)
    L = O.Layout(pack.bits.numpy())
    codes, scales = O.quantize(O.encode(M, pack.enc.numpy(), L), L, lloyd)
    K_or = OC.from_matrix(torch.from_numpy(O.dequant(codes, scales, pack.dec.numpy(), L, lloyd=lloyd)).float(),
                          h_kv)
    cos, sin = A.rope_cos_sin(torch.tensor(consts.inv_freq), torch.arange(S))
    cos, sin = cos.half().float(), sin.half().float()
    V_or = _values_oracle(v, h_kv, "full")
    ref = A.naive_dense_attention(q.reshape(h_kv * G, 1, 128).float(),
                                  torch.cat([A.apply_rope(K_or, cos, sin), kt.float()], 1),
                                  torch.cat([V_or, vt.float()], 1), G, scale).reshape(h_kv, G, 128)
    o = out.cpu().double()
    err = (o - ref.double()).abs().max().item()
    rel = ((o - ref.double()).norm() / ref.double().norm()).item()
    Vb = torch.empty(h_kv, S, 128, dtype=torch.float16, device=DEV)
    Sb = torch.empty(h_kv, G, S, dtype=torch.float32, device=DEV)
    spectral.dequant(dp, kp, k_ids, vp, v_ids, S, consts, apply_rope=rope, dtype=torch.float16,
                     out=(None, Vb), q=q.to(DEV), scores=Sb)
    sw = torch.cat([Sb, (q.float() @ kt.float().transpose(1, 2)).to(DEV)], -1) * scale
    Vw = torch.cat([Vb.float(), vt.float().to(DEV)], 1)
    alt = (torch.softmax(sw, -1) @ Vw).cpu().double()
    d_alt = (o - alt).abs().max().item()
    print(f"long full-C {payload} S {S} T {T}: decode vs oracle max_abs {err:.3e} rel {rel:.3e}; "
          f"vs scores form {d_alt:.3e}", flush=True)
    assert err <= 2e-3 and rel <= 1e-2 and d_alt <= 2e-3

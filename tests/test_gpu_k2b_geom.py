"""GPU tests of the k2b path on the general page: head_dim 32/64/128, rank
16..128, residual groups 16..128, 2..4-bit keys (the reference's fused path
takes any power-of-two head_dim and rank and the recipe's group,
packed_streaming.py:957-975; its own k2b test runs head_dim 64, group 32, rank
16, tests/test_triton_decode_k2b.py:156-250).

  * the append kernels against the reference's own codec outputs
    (tests/golden/k2b_geom.npz, written by make_golden.py from quantize_packed),
    and bit for bit against the oracle on dyadic inputs;
  * decode against the oracle's one-softmax attention over the same codes
    (RoPE with the reference's fp16 tables), at the north-star bar 2e-3, with and
    without a recent window, rows given apart, bf16 windows, ragged batches;
  * dequant (the prefill path) against the oracle's dense keys and values.
"""

from pathlib import Path

import numpy as np
import pytest
import torch

from bmx_amd import k2b, synth
from oracle import attention as A
from oracle import codecs as OC
from oracle import layout as OL

pytestmark = pytest.mark.gpu
DEV = "cuda"
GOLD = Path(__file__).parent / "golden"

# name, h_kv, head_dim, rank, residual group, key bits, value seed (make_golden.py)
GEOM_CASES = [
    ("d64_r16_g32", 2, 64, 16, 32, 3, 7),
    ("d128_r64_g64", 2, 128, 64, 64, 3, 0),
    ("d32_r16_g16_b2", 4, 32, 16, 16, 2, 3),
    ("d128_r32_g128_b4", 2, 128, 32, 128, 4, 0),
]


def _pool(n, h, rank, d, group, bits, gen=None):
    return synth.PagePool(n, h, rank, DEV, gen=gen, head_dim=d, group=group, k_bits=bits)


@pytest.mark.parametrize("case", GEOM_CASES, ids=[c[0] for c in GEOM_CASES])
def test_append_matches_reference_golden(case):
    name, h, d, rank, group, bits, vseed = case
    g = np.load(GOLD / "k2b_geom.npz")
    kpre = torch.from_numpy(g[f"{name}_kpre"])
    v = torch.from_numpy(g[f"{name}_v"])
    us0 = torch.from_numpy(g[f"{name}_svd_us_fp32"])
    V = torch.from_numpy(g[f"{name}_svd_v_fp32"])
    consts = k2b.CodecConsts.make(v_seed=vseed, head_dim=d)
    pool = _pool(64, h, rank, d, group, bits, gen=torch.Generator().manual_seed(3))
    seq = synth.encode_sequence(pool, kpre.to(DEV), v.to(DEV), rank, consts, svd=(us0, V))
    torch.cuda.synchronize()
    pages = pool.pages[torch.tensor(seq.page_ids, device=DEV)].cpu().numpy()
    us16, res, sc16, vidx, vn16 = OL.unpack_general(pages, h, rank, d, group, bits)
    n_us = n_res = n_sc = 0
    gpp = 128 // group
    for p in range(3):
        pre = f"{name}_p{p}_"
        sl = slice(p * 128, (p + 1) * 128)
        np.testing.assert_array_equal(vidx[sl], g[pre + "vidx"])
        np.testing.assert_array_equal(vn16[sl].astype(np.float32), g[pre + "vnorm"])
        # Us16 of later pages: a length-C fp32 dot in another order than CPU BLAS
        ulps = np.abs(us16[sl].view(np.int16).astype(np.int32)
                      - g[pre + "us"].astype(np.float16).view(np.int16).astype(np.int32))
        assert ulps.max() <= 1 and (p > 0 or ulps.max() == 0)
        n_us += int((ulps > 0).sum())
        n_res += int((res[:, sl] != g[pre + "res"]).sum())
        want_sc = g[pre + "scale"][..., 0].astype(np.float16)
        got_sc = sc16[:, p * gpp:(p + 1) * gpp]
        sc_ulps = np.abs(got_sc.view(np.int16).astype(np.int32) - want_sc.view(np.int16).astype(np.int32))
        assert sc_ulps.max() <= 1
        n_sc += int((sc_ulps > 0).sum())
    C = h * d
    print(f"{name}: Us16 mismatches {n_us}/{3 * 128 * rank}, residual codes {n_res}/{3 * 128 * C}, "
          f"scales {n_sc}/{3 * C * gpp}", flush=True)
    assert n_us <= 3 * 128 * rank // 200 and n_res <= 3 * 128 * C // 2000 and n_sc <= C // 16 + 2


@pytest.mark.parametrize("case", GEOM_CASES, ids=[c[0] for c in GEOM_CASES])
def test_append_bit_exact_on_dyadic_inputs(case):
    """Inputs whose every fp32 sum is exact in any order: the pages equal the
    numpy packing of the oracle's codes byte for byte."""
    name, h, d, rank, group, bits, vseed = case
    gen = torch.Generator().manual_seed(4)
    S, C = 256, h * d
    k_pre = (torch.randint(-24, 25, (h, S, d), generator=gen) / 8.0).half()
    v = (torch.randint(-16, 17, (h, S, d), generator=gen) / 4.0).half()
    V = (torch.randint(-2, 3, (C, rank), generator=gen) / 4.0).float()
    us0 = OC.to_matrix(k_pre[:, :128].float()) @ V
    consts = k2b.CodecConsts.make(v_seed=vseed, head_dim=d)
    pool = _pool(64, h, rank, d, group, bits)
    seq = synth.encode_sequence(pool, k_pre.to(DEV), v.to(DEV), rank, consts, svd=(us0, V))
    torch.cuda.synchronize()
    pages = pool.pages[torch.tensor(seq.page_ids, device=DEV)].cpu().numpy()
    enc = OC.FrozenSubspaceKeyEncoder(rank, bits, group)
    us_l, res_l, sc_l, vi_l, vn_l = [], [], [], [], []
    for p in range(2):
        sl = slice(p * 128, (p + 1) * 128)
        kp, _ = enc.encode(OC.to_matrix(k_pre[:, sl].float()), us_override=(us0, V) if p == 0 else None)
        us_l.append(kp["Us"].numpy().astype(np.float16))
        res_l.append(kp["res_Q_int"].numpy())
        sc_l.append(kp["res_scale"][..., 0].numpy().astype(np.float16))
        idx, norms, _ = OC.quantize_v_perhead(OC.to_matrix(v[:, sl].float()), bits=2, seed=vseed, h=h)
        vi_l.append(idx.numpy())
        vn_l.append(norms.numpy().astype(np.float16))
    want = OL.pack_general(np.concatenate(us_l), np.concatenate(res_l, 1), np.concatenate(sc_l, 1),
                           np.concatenate(vi_l), np.concatenate(vn_l), h, rank, d, group, bits)
    np.testing.assert_array_equal(pages, want)


def _case_pages(gen, h, d, rank, group, bits, S, vseed=0, pool_pages=None):
    k_pre = synth.k2b_keys(h, S, rank, gen, head_dim=d)
    v = synth.values(h, S, gen, head_dim=d)
    svd = synth.first_page_svd(k_pre, rank)
    consts = k2b.CodecConsts.make(v_seed=vseed, head_dim=d)
    pool = _pool(pool_pages or S // 16 + 8, h, rank, d, group, bits, gen=gen)
    seq = synth.encode_sequence(pool, k_pre.to(DEV), v.to(DEV), rank, consts, svd=svd)
    return k_pre, v, svd, consts, pool, seq


def _attention_ref(q, cache, consts, kt, vt, G, d):
    """The oracle's one-softmax attention, keys rotated with the reference's
    shared fp16 RoPE tables (HF's fp32 angle, cos/sin rounded to fp16, the
    rotation in fp32), as its decode reads them (packed_streaming.py:79-113)."""
    K = cache.dense_k_pre()
    cos, sin = A.rope_cos_sin(torch.tensor(consts.inv_freq), torch.arange(K.shape[1]))
    K = A.apply_rope(K, cos.half().float(), sin.half().float())
    V = cache.dense_v()
    if kt is not None:
        K, V = torch.cat([K, kt.float()], 1), torch.cat([V, vt.float()], 1)
    return A.naive_dense_attention(q, K, V, G, d ** -0.5)


def _oracle(k_pre, v, svd, consts, h, d, rank, group, bits, vseed, S):
    cache = A.K2bOracleCache(h, d, rank, group=group, k_bits=bits, v_seed=vseed)
    for p in range(S // 128):
        cache.commit(k_pre[:, p * 128:(p + 1) * 128], v[:, p * 128:(p + 1) * 128],
                     us_override=svd if p == 0 else None)
    return cache


DECODE_CASES = [  # (h_kv, head_dim, rank, group, bits, G, S, T)
    (2, 64, 16, 32, 3, 4, 1024, 40),     # the reference's test geometry
    (8, 128, 64, 64, 3, 4, 2048, 40),    # rank 64 at the recipe's other settings
    (4, 32, 16, 16, 2, 8, 1024, 0),
    (2, 128, 32, 128, 4, 1, 512, 17),
    (8, 64, 128, 32, 3, 4, 2048, 128),
    (16, 64, 32, 64, 3, 2, 1024, 24),
]


@pytest.mark.parametrize("h,d,rank,group,bits,G,S,T", DECODE_CASES)
def test_decode_matches_oracle(h, d, rank, group, bits, G, S, T):
    gen = torch.Generator().manual_seed(50 + h + d + rank + group)
    k_pre, v, svd, consts, pool, seq = _case_pages(gen, h, d, rank, group, bits, S)
    kt = vt = None
    if T:
        kx = synth.k2b_keys(h, T, rank, gen, head_dim=d)
        kt = synth.rope_keys(kx, S, consts).unsqueeze(0).to(DEV).contiguous()
        vt = synth.values(h, T, gen, head_dim=d).unsqueeze(0).to(DEV).contiguous()
    q = torch.randn(1, h, G, d, generator=gen).to(DEV)
    table = synth.page_table([seq], device=DEV)
    ln = torch.tensor([S], dtype=torch.int32, device=DEV)
    out = k2b.decode(q, pool.pages, table, ln, S, seq.basis16, consts, d ** -0.5, rank=rank,
                     k_tail=kt, v_tail=vt, tail_len=T, tail_cap=T, group=group, k_bits=bits)
    torch.cuda.synchronize()
    cache = _oracle(k_pre, v, svd, consts, h, d, rank, group, bits, 0, S)
    ref = _attention_ref(q[0].cpu().reshape(h * G, 1, d), cache, consts, kt[0].cpu() if T else None,
                         vt[0].cpu() if T else None, G, d)
    err = (out[0].cpu().reshape(h * G, 1, d) - ref).abs().max().item()
    rel = ((out[0].cpu().reshape(h * G, 1, d) - ref).norm() / ref.norm()).item()
    print(f"h {h} d {d} R {rank} group {group} bits {bits} G {G} S {S} T {T}: max_abs {err:.3e} rel {rel:.3e}",
          flush=True)
    assert err <= 2e-3 and rel <= 1e-2


def test_decode_ragged_batch_fold_and_bf16_window():
    """Two sequences of different lengths in one call (their own page tables,
    one pool), the window's newest rows given apart (attended from there and
    copied into the window buffer), the window in fp16 and in bf16, a bf16
    query: every sequence against its own oracle."""
    h, d, rank, group, bits, G, T = 2, 64, 16, 32, 3, 4, 24
    gen = torch.Generator().manual_seed(61)
    lens = (1024, 384)
    consts = k2b.CodecConsts.make(v_seed=0, head_dim=d)
    pool = _pool(200, h, rank, d, group, bits, gen=gen)
    data, seqs = [], []
    for S in lens:
        k_pre = synth.k2b_keys(h, S, rank, gen, head_dim=d)
        v = synth.values(h, S, gen, head_dim=d)
        svd = synth.first_page_svd(k_pre, rank)
        seqs.append(synth.encode_sequence(pool, k_pre.to(DEV), v.to(DEV), rank, consts, svd=svd))
        data.append((k_pre, v, svd))
    table = synth.page_table(seqs, device=DEV)
    ln = torch.tensor(lens, dtype=torch.int32, device=DEV)
    basis = torch.stack([s.basis16 for s in seqs]).contiguous()
    kt = torch.stack([synth.rope_keys(synth.k2b_keys(h, T, rank, gen, head_dim=d), S, consts)
                      for S in lens]).to(DEV).contiguous()
    vt = synth.values(2 * h, T, gen, head_dim=d).view(2, h, T, d).to(DEV).contiguous()
    q = torch.randn(2, h, G, d, generator=gen).to(DEV).bfloat16()
    for wdt in (torch.float16, torch.bfloat16):
        kw, vw = kt.to(wdt).clone(), vt.to(wdt).clone()
        new = (kw[:, :, T - 2:].clone(), vw[:, :, T - 2:].clone())
        kw[:, :, T - 2:] = 0
        vw[:, :, T - 2:] = 0
        out = k2b.decode(q, pool.pages, table, ln, max(lens), basis, consts, d ** -0.5, rank=rank,
                         k_tail=kw, v_tail=vw, tail_len=T, tail_cap=T, new_kv=new, group=group, k_bits=bits)
        torch.cuda.synchronize()
        assert out.dtype == torch.bfloat16
        assert torch.equal(kw, kt.to(wdt)) and torch.equal(vw, vt.to(wdt))   # rows given apart landed
        for b, S in enumerate(lens):
            k_pre, v, svd = data[b]
            cache = _oracle(k_pre, v, svd, consts, h, d, rank, group, bits, 0, S)
            ref = _attention_ref(q[b].float().cpu().reshape(h * G, 1, d), cache, consts, kt[b].to(wdt).cpu(),
                                 vt[b].to(wdt).cpu(), G, d)
            err = (out[b].float().cpu().reshape(h * G, 1, d) - ref).abs().max().item()
            print(f"ragged b {b} S {S} window {wdt}: max_abs {err:.3e}", flush=True)
            assert err <= 2e-3 + ref.abs().max().item() * 2 ** -8


@pytest.mark.parametrize("h,d,rank,group,bits", [(2, 64, 16, 32, 3), (8, 128, 64, 64, 3), (4, 32, 16, 16, 2)])
def test_dequant_matches_oracle(h, d, rank, group, bits):
    """Dense keys (pre-RoPE, exact-angle RoPE, fp16-table RoPE) and values of
    the committed pages against the oracle's."""
    gen = torch.Generator().manual_seed(70 + d + rank)
    S = 512
    k_pre, v, svd, consts, pool, seq = _case_pages(gen, h, d, rank, group, bits, S)
    cache = _oracle(k_pre, v, svd, consts, h, d, rank, group, bits, 0, S)
    K0 = cache.dense_k_pre()
    V0 = cache.dense_v()
    table = torch.tensor(seq.page_ids, dtype=torch.int32, device=DEV)
    cos, sin = A.rope_cos_sin(torch.tensor(consts.inv_freq), torch.arange(S))
    for mode, Kref in ((k2b.ROPE_NONE, K0), (k2b.ROPE_EXACT, A.apply_rope(K0, cos, sin)),
                       (k2b.ROPE_FP16_TABLES, A.apply_rope(K0, cos.half().float(), sin.half().float()))):
        K, V = k2b.dequant(pool.pages, table, S, seq.basis16, consts, h_kv=h, rank=rank, apply_rope=mode,
                           dtype=torch.float32, group=group, k_bits=bits)
        torch.cuda.synchronize()
        ek = (K.cpu() - Kref).abs().max().item() / Kref.abs().max().item()
        ev = (V.cpu() - V0).abs().max().item() / V0.abs().max().item()
        print(f"h {h} d {d} R {rank} group {group} bits {bits} rope {mode}: keys {ek:.2e} values {ev:.2e} "
              f"(relative to max)", flush=True)
        assert ek <= 2e-3 and ev <= 1e-5

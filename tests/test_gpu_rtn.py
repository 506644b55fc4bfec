"""GPU parity of the HIP RTN path (rtn_token keys post-RoPE and values) against
the CPU oracle, through the C-ABI (bmx_amd.rtn -> libbmx_k2b.so).

Bars: codes and fp16 scales bit-exact (the codec is element-wise: max,
divide, round half to even); dequantized pages bit-exact; attention output
max-abs <= 2e-3 and ||err||/||ref|| <= 1e-2 against the fp32 oracle
(code * fp16 scale, one softmax over packed + window tokens).
"""

import numpy as np
import pytest
import torch

from bmx_amd import rtn
from oracle import attention as A
from oracle import layout as OL

pytestmark = pytest.mark.gpu
DEV = "cuda"
MAX_ABS = 2e-3
REL = 1e-2


def _close(out, ref, what):
    out, ref = out.double().cpu(), ref.double().cpu()
    err = (out - ref).abs().max().item()
    rel = ((out - ref).norm() / ref.norm()).item()
    print(f"{what}: max_abs={err:.3e} rel={rel:.3e}", flush=True)
    assert err <= MAX_ABS and rel <= REL, f"{what}: max_abs {err:.3e} rel {rel:.3e}"


def _keys(h_kv, S, gen, outliers=True):
    """Config-1 style keys: N(0,1) with 4 fixed channels x10."""
    k = torch.randn(h_kv, S, 128, generator=gen)
    if outliers:
        k[:, :, [3, 40, 77, 101]] *= 10.0
    return k


def _encode(h_kv, k, v, codec, gen=None, n_pool=None):
    """Append every codec page of (k, v) through the HIP write kernel; returns
    (pool, page ids in logical order)."""
    S = k.shape[1]
    pool = rtn.PagePool(n_pool or S // 16, h_kv, DEV, gen=gen, **codec)
    ids = pool.alloc(S // 16)
    rtn.append(k.to(DEV), v.to(DEV), pool.pages, torch.tensor(ids, dtype=torch.int32, device=DEV), **codec)
    return pool, ids


def _oracle(h_kv, k, v, codec):
    c = A.RtnOracleCache(h_kv, **codec)
    for p in range(k.shape[1] // 128):
        c.commit(k[:, p * 128:(p + 1) * 128], v[:, p * 128:(p + 1) * 128])
    return c


@pytest.mark.parametrize("h_kv,codec,dtype", [
    (8, dict(k_bits=4, v_bits=4, k_group=32, v_group=32), torch.float16),
    (2, dict(k_bits=2, v_bits=3, k_group=64, v_group=128), torch.bfloat16),
    (16, dict(k_bits=4, v_bits=2, k_group=128, v_group=32), torch.float32),
])
def test_append_codes_bit_exact(h_kv, codec, dtype):
    gen = torch.Generator().manual_seed(1)
    S = 256
    k, v = _keys(h_kv, S, gen).to(dtype), torch.randn(h_kv, S, 128, generator=gen).to(dtype)
    pool, ids = _encode(h_kv, k, v, codec)
    torch.cuda.synchronize()
    pages = pool.pages[torch.tensor(ids, device=DEV)].cpu().numpy()
    kq, ks, vq, vs = OL.unpack_rtn_pages(pages, h_kv, codec["k_group"], codec["v_group"])
    ref = _oracle(h_kv, k, v, codec)
    rkq, rks, rvq, rvs = ref.codes()
    np.testing.assert_array_equal(kq, rkq.numpy())
    np.testing.assert_array_equal(vq, rvq.numpy())
    np.testing.assert_array_equal(ks, rks.numpy().astype(np.float16))
    np.testing.assert_array_equal(vs, rvs.numpy().astype(np.float16))


@pytest.mark.parametrize("h_kv,codec", [
    (8, dict(k_bits=4, v_bits=4, k_group=32, v_group=32, k_arm=rtn.CHANNEL)),
    (2, dict(k_bits=2, v_bits=2, k_group=64, v_group=64, k_arm=rtn.CHANNEL)),
    (16, dict(k_bits=3, v_bits=4, k_group=128, v_group=32, k_arm=rtn.CHANNEL)),
])
def test_append_channel_arm_codes_bit_exact(h_kv, codec):
    """rtn_channel keys (quantize_packed("rtn_channel"): a scale per channel
    and group of k_group tokens), written into every page of the group."""
    gen = torch.Generator().manual_seed(11)
    S = 256
    k, v = _keys(h_kv, S, gen).half(), torch.randn(h_kv, S, 128, generator=gen).half()
    pool, ids = _encode(h_kv, k, v, codec)
    torch.cuda.synchronize()
    pages = pool.pages[torch.tensor(ids, device=DEV)].cpu().numpy()
    kq, ks, vq, vs = OL.unpack_rtn_pages(pages, h_kv, codec["k_group"], codec["v_group"], k_arm=1)
    rkq, rks, rvq, rvs = _oracle(h_kv, k, v, codec).codes()
    np.testing.assert_array_equal(kq, rkq.numpy())
    hi, lo = OL.scale_pair(rks.numpy())   # the fp32 scale as the page's fp16 pair
    np.testing.assert_array_equal(ks, np.repeat(hi.astype(np.float32) + lo.astype(np.float32),
                                                codec["k_group"] // 16, axis=1))
    np.testing.assert_array_equal(vq, rvq.numpy())
    np.testing.assert_array_equal(vs, rvs.numpy().astype(np.float16))


def test_dequant_bit_exact():
    gen = torch.Generator().manual_seed(2)
    h_kv, S = 8, 384
    codec = dict(k_bits=4, v_bits=4, k_group=32, v_group=64)
    k, v = _keys(h_kv, S, gen).half(), torch.randn(h_kv, S, 128, generator=gen).half()
    pool, ids = _encode(h_kv, k, v, codec, gen=torch.Generator().manual_seed(5), n_pool=S // 16 + 7)
    K, V = rtn.dequant(pool.pages, torch.tensor(ids, dtype=torch.int32, device=DEV), h_kv=h_kv, **codec)
    rK, rV = _oracle(h_kv, k, v, codec).dense_kv()
    assert torch.equal(K.cpu(), rK) and torch.equal(V.cpu(), rV)
    codec = dict(codec, k_arm=rtn.CHANNEL)
    pool, ids = _encode(h_kv, k, v, codec, gen=torch.Generator().manual_seed(6), n_pool=S // 16 + 3)
    K, V = rtn.dequant(pool.pages, torch.tensor(ids, dtype=torch.int32, device=DEV), h_kv=h_kv, **codec)
    rK, rV = _oracle(h_kv, k, v, codec).dense_kv()
    assert torch.equal(K.cpu(), rK) and torch.equal(V.cpu(), rV)
    # in the model's dtype (the prefill form): the same values rounded once
    for dt in (torch.float16, torch.bfloat16):
        Kh, Vh = rtn.dequant(pool.pages, torch.tensor(ids, dtype=torch.int32, device=DEV), h_kv=h_kv, dtype=dt,
                             **codec)
        assert Kh.dtype == dt and torch.equal(Kh, K.to(dt)) and torch.equal(Vh, V.to(dt))
    # pages 4 .. 15 into rows 64 .. 255 of a wider buffer
    buf = torch.full((2, h_kv, S + 16, 128), 5.0, dtype=torch.float16, device=DEV)
    ids_t = torch.tensor(ids, dtype=torch.int32, device=DEV)
    rtn.dequant(pool.pages, ids_t[4:16].contiguous(), h_kv=h_kv, dtype=torch.float16,
                out=(buf[0, :, 64:], buf[1, :, 64:]), **codec)
    Kh, Vh = rtn.dequant(pool.pages, ids_t, h_kv=h_kv, dtype=torch.float16, **codec)
    assert torch.equal(buf[0, :, 64:256], Kh[:, 64:256]) and torch.equal(buf[1, :, 64:256], Vh[:, 64:256])
    assert bool((buf[:, :, :64] == 5.0).all() and (buf[:, :, 256:] == 5.0).all())


def _decode_case(h_kv, G, S, T, codec, gen, split_tokens=0, outliers=True, with_chunked=False):
    k = _keys(h_kv, S + T, gen, outliers)
    v = torch.randn(h_kv, S + T, 128, generator=gen)
    k16, v16 = k.half(), v.half()
    pool, ids = _encode(h_kv, k16[:, :S], v16[:, :S], codec, gen=torch.Generator().manual_seed(3),
                        n_pool=S // 16 + 5) if S else (rtn.PagePool(1, h_kv, DEV, **codec), [0])
    q = torch.randn(1, h_kv, G, 128, generator=gen)
    out = rtn.decode(q.to(DEV), pool.pages, torch.tensor([ids], dtype=torch.int32, device=DEV),
                     torch.tensor([S], dtype=torch.int32, device=DEV), S, 128 ** -0.5,
                     k_tail=k16[:, S:].unsqueeze(0).to(DEV), v_tail=v16[:, S:].unsqueeze(0).to(DEV),
                     tail_len=torch.tensor([T], dtype=torch.int32, device=DEV), tail_cap=T,
                     split_tokens=split_tokens, **codec)
    torch.cuda.synchronize()
    cache = _oracle(h_kv, k16[:, :S], v16[:, :S], codec) if S else None
    if cache is not None:
        ref = A.rtn_naive_attention(q.view(h_kv * G, 1, 128), cache, k16[:, S:], v16[:, S:], G, 128 ** -0.5)
    else:
        ref = A.naive_dense_attention(q.view(h_kv * G, 1, 128), k16[:, S:].float(), v16[:, S:].float(),
                                      G, 128 ** -0.5)
    if with_chunked:
        # the reference's own chunked path with fp32 scales (codecs.py:819-822)
        chunked = A.rtn_chunked_attention(q.view(h_kv * G, 1, 128), cache, k16[:, S:], v16[:, S:], G,
                                          128 ** -0.5)
        return out, ref.view(1, h_kv, G, 128), chunked.view(1, h_kv, G, 128)
    return out, ref.view(1, h_kv, G, 128)


def test_decode_config1():
    """Config 1: 32 query / 8 KV heads, d 128, ctx 4096 = 3968 packed + 128
    fp16 window tokens; keys rtn_channel 4-bit (groups of 32 tokens) with 4
    outlier channels x10, values rtn_token 4-bit (groups of 32 channels);
    seed 0.  The reference runs this pair on its chunked path only."""
    gen = torch.Generator().manual_seed(0)
    out, ref, chunked = _decode_case(8, 4, 3968, 128,
                                     dict(k_bits=4, v_bits=4, k_group=32, v_group=32, k_arm=rtn.CHANNEL), gen,
                                     with_chunked=True)
    _close(out, ref, "config1 rtn_channel K / rtn_token V, 4b g32 (fp16-scale oracle)")
    # the path the reference executes for this pair: chunked dequant-attention
    # with the fp32 scales of dequant_packed
    _close(out, chunked, "config1 vs the reference's chunked path (fp32 scales)")


def test_decode_config1_geometry_fused_pair():
    """The reference's fused pair (rtn_token keys and values) at config 1's
    geometry."""
    gen = torch.Generator().manual_seed(0)
    out, ref = _decode_case(8, 4, 3968, 128, dict(k_bits=4, v_bits=4, k_group=32, v_group=32), gen)
    _close(out, ref, "config1 geometry rtn_token K / rtn_token V, 4b g32")


def test_decode_kivi():
    """kivi recipe (recipes.py:173-177): rtn_channel keys and rtn_token values
    at 2 bits, groups of 64."""
    gen = torch.Generator().manual_seed(8)
    out, ref = _decode_case(8, 4, 8192, 200,
                            dict(k_bits=2, v_bits=2, k_group=64, v_group=64, k_arm=rtn.CHANNEL), gen)
    _close(out, ref, "kivi 2b g64")


@pytest.mark.parametrize("G", [1, 2, 8, 16])
def test_decode_query_group_sizes(G):
    gen = torch.Generator().manual_seed(30 + G)
    out, ref = _decode_case(4, G, 2048, 100, dict(k_bits=4, v_bits=4, k_group=32, v_group=32), gen)
    _close(out, ref, f"G {G}")


@pytest.mark.parametrize("codec", [dict(k_bits=2, v_bits=2, k_group=64, v_group=64),
                                   dict(k_bits=3, v_bits=4, k_group=128, v_group=32),
                                   dict(k_bits=4, v_bits=3, k_group=32, v_group=128),
                                   dict(k_bits=3, v_bits=3, k_group=128, v_group=64, k_arm=rtn.CHANNEL)])
def test_decode_bits_and_groups(codec):
    gen = torch.Generator().manual_seed(40)
    out, ref = _decode_case(8, 4, 4096, 160, codec, gen, outliers=False)
    _close(out, ref, f"bits {codec['k_bits']}/{codec['v_bits']} groups {codec['k_group']}/{codec['v_group']}")


def test_decode_split_counts_window_only_and_no_window():
    gen = torch.Generator().manual_seed(50)
    codec = dict(k_bits=4, v_bits=4, k_group=32, v_group=32)
    for st in (64, 512):
        out, ref = _decode_case(8, 4, 2048, 128, codec, gen, split_tokens=st)
        _close(out, ref, f"split_tokens {st}")
    out, ref = _decode_case(8, 4, 1024, 0, codec, gen)
    _close(out, ref, "no window")
    out, ref = _decode_case(8, 4, 0, 300, codec, gen)
    _close(out, ref, "window only")


def test_ragged_batch_shuffled_pages():
    """Batch of 4 sequences, ragged lengths and windows, shuffled physical pages."""
    gen = torch.Generator().manual_seed(60)
    h_kv, G = 8, 4
    codec = dict(k_bits=4, v_bits=4, k_group=32, v_group=32)
    lens = [128 * int(x) for x in torch.randint(2, 24, (4,), generator=gen)]
    tails = [int(x) for x in torch.randint(1, 256, (4,), generator=gen)]
    pool = rtn.PagePool(sum(lens) // 16 + 9, h_kv, DEV, gen=torch.Generator().manual_seed(4), **codec)
    tables, caches, kts, vts = [], [], [], []
    for S, T in zip(lens, tails):
        k = _keys(h_kv, S + T, gen).half()
        v = torch.randn(h_kv, S + T, 128, generator=gen).half()
        ids = pool.alloc(S // 16)
        rtn.append(k[:, :S].to(DEV), v[:, :S].to(DEV), pool.pages, torch.tensor(ids, dtype=torch.int32,
                                                                                 device=DEV), **codec)
        tables.append(ids)
        caches.append(_oracle(h_kv, k[:, :S], v[:, :S], codec))
        kts.append(k[:, S:])
        vts.append(v[:, S:])
    B, cap, mp = len(lens), max(tails), max(len(t) for t in tables)
    table = torch.zeros(B, mp, dtype=torch.int32)
    k_tail = torch.zeros(B, h_kv, cap, 128, dtype=torch.float16)
    v_tail = torch.zeros_like(k_tail)
    for i in range(B):
        table[i, :len(tables[i])] = torch.tensor(tables[i])
        k_tail[i, :, :tails[i]] = kts[i]
        v_tail[i, :, :tails[i]] = vts[i]
    q = torch.randn(B, h_kv, G, 128, generator=gen)
    out = rtn.decode(q.to(DEV), pool.pages, table.to(DEV), torch.tensor(lens, dtype=torch.int32, device=DEV),
                     max(lens), 128 ** -0.5, k_tail=k_tail.to(DEV), v_tail=v_tail.to(DEV),
                     tail_len=torch.tensor(tails, dtype=torch.int32, device=DEV), tail_cap=cap, **codec)
    torch.cuda.synchronize()
    for i in range(B):
        ref = A.rtn_naive_attention(q[i].reshape(h_kv * G, 1, 128), caches[i], kts[i], vts[i], G, 128 ** -0.5)
        _close(out[i], ref.view(h_kv, G, 128), f"ragged seq {i} len {lens[i]} tail {tails[i]}")


def test_rows_given_apart_fold_the_window_write():
    """As for k2b: the window's newest rows given apart (host tail_len) give the
    output of the call over a window that already holds them, bit for bit, and
    land in the window buffers; token and channel key arms."""
    gen = torch.Generator().manual_seed(71)
    h_kv, G, S = 8, 4, 1024
    for codec, T, n in ((dict(k_bits=4, v_bits=4, k_group=32, v_group=32), 300, 2),
                        (dict(k_bits=2, v_bits=2, k_group=128, v_group=32, k_arm=rtn.CHANNEL), 600, 1)):
        k = _keys(h_kv, S + T, gen).half()
        v = torch.randn(h_kv, S + T, 128, generator=gen).half()
        pool, ids = _encode(h_kv, k[:, :S], v[:, :S], codec, gen=torch.Generator().manual_seed(5),
                            n_pool=S // 16 + 3)
        cap = T + 3
        k_full = torch.full((1, h_kv, cap, 128), 2.0, dtype=torch.float16)
        v_full = torch.full_like(k_full, -1.0)
        k_full[0, :, :T], v_full[0, :, :T] = k[:, S:], v[:, S:]
        k_full, v_full = k_full.to(DEV), v_full.to(DEV)
        k_stale, v_stale = k_full.clone(), v_full.clone()
        k_stale[:, :, T - n:T] = 0.0
        v_stale[:, :, T - n:T] = 0.0
        q = torch.randn(1, h_kv, G, 128, generator=gen).to(DEV)
        table = torch.tensor([ids], dtype=torch.int32, device=DEV)
        ln = torch.tensor([S], dtype=torch.int32, device=DEV)
        ref = rtn.decode(q, pool.pages, table, ln, S, 128 ** -0.5, k_tail=k_full, v_tail=v_full,
                         tail_len=torch.tensor([T], dtype=torch.int32, device=DEV), tail_cap=cap, **codec)
        out = rtn.decode(q, pool.pages, table, ln, S, 128 ** -0.5, k_tail=k_stale, v_tail=v_stale, tail_len=T,
                         tail_cap=cap, new_kv=(k_full[:, :, T - n:T], v_full[:, :, T - n:T]), **codec)
        torch.cuda.synchronize()
        ok = torch.equal(out, ref) and torch.equal(k_stale, k_full) and torch.equal(v_stale, v_full)
        print(f"rtn arm {codec.get('k_arm', 0)} T {T} n {n}: folded == written and window rows stored: {ok}",
              flush=True)
        assert ok

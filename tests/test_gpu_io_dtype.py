"""GPU tests of the decode boundary's query / output dtype (io_dtype).

The reference's fused_decode_attention_k2b takes the query in the model's
dtype and returns the attention output in it
(cache/triton_dequant_attention.py:1232-1246).  A call with an fp16 or bf16
query must equal the fp32 call on the same (rounded) query, rounded once to
that dtype: the kernels convert the query on load and the output on store and
compute in between exactly as for fp32.
"""

import pytest
import torch

from bmx_amd import k2b, rtn, synth
from oracle import attention as A

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _k2b_case(gen, h_kv=8, rank=32, S=2048, T=40):
    k_pre = synth.k2b_keys(h_kv, S + T, rank, gen)
    v = synth.values(h_kv, S + T, gen)
    svd = synth.first_page_svd(k_pre, rank)
    consts = k2b.CodecConsts.make(v_seed=0)
    pool = synth.PagePool(S // 16, h_kv, rank, DEV, gen=gen)
    seq = synth.encode_sequence(pool, k_pre[:, :S].to(DEV), v[:, :S].to(DEV), rank, consts, svd=svd)
    kt = synth.rope_keys(k_pre[:, S:], S, consts).unsqueeze(0).to(DEV).contiguous()
    vt = v[:, S:].unsqueeze(0).half().to(DEV).contiguous()
    table = synth.page_table([seq], device=DEV)   # the pool hands pages out shuffled
    return k_pre, v, svd, consts, pool, seq, kt, vt, table


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
def test_k2b_decode_model_dtype_query(dt):
    gen = torch.Generator().manual_seed(21)
    h_kv, rank, S, T, G = 8, 32, 2048, 40, 4
    k_pre, v, svd, consts, pool, seq, kt, vt, table = _k2b_case(gen, h_kv, rank, S, T)
    q = torch.randn(1, h_kv, G, 128, generator=gen).to(DEV).to(dt)
    ln = torch.tensor([S], dtype=torch.int32, device=DEV)
    common = dict(rank=rank, k_tail=kt, v_tail=vt, tail_len=T, tail_cap=T)
    out_d = k2b.decode(q, pool.pages, table, ln, S, seq.basis16, consts, 128 ** -0.5, **common)
    out_f = k2b.decode(q.float().contiguous(), pool.pages, table, ln, S, seq.basis16, consts, 128 ** -0.5,
                       **common)
    torch.cuda.synchronize()
    assert out_d.dtype == dt and out_d.shape == q.shape
    assert torch.equal(out_d, out_f.to(dt)), f"{dt}: max |diff| {(out_d.float() - out_f).abs().max().item():.3e}"
    # and the oracle, at the fp32 bar plus the output's own rounding
    cache = A.K2bOracleCache(h_kv, 128, rank)
    for p in range(S // 128):
        cache.commit(k_pre[:, p * 128:(p + 1) * 128], v[:, p * 128:(p + 1) * 128],
                     us_override=svd if p == 0 else None)
    ref = A.k2b_naive_attention(q.float().cpu().view(h_kv * G, 1, 128), cache, torch.tensor(consts.inv_freq),
                                kt[0].float().cpu(), vt[0].float().cpu(), G, 128 ** -0.5).view(1, h_kv, G, 128)
    err = (out_d.float().cpu() - ref).abs().max().item()
    assert err <= 2e-3 + ref.abs().max().item() * (2 ** -8 if dt == torch.bfloat16 else 2 ** -11), err


def test_k2b_plan_fresh_output_and_dtype_guard():
    """A bound fp16 plan called with a new query and a caller's output tensor
    writes that tensor (the plan's own buffer stays untouched)."""
    gen = torch.Generator().manual_seed(22)
    h_kv, rank, S, T, G = 8, 32, 1024, 16, 4
    _, _, _, consts, pool, seq, kt, vt, table = _k2b_case(gen, h_kv, rank, S, T)
    ln = torch.tensor([S], dtype=torch.int32, device=DEV)
    q0 = torch.randn(1, h_kv, G, 128, generator=gen).to(DEV).half()
    plan = k2b.DecodePlan(q0, pool.pages, table, ln, S, seq.basis16, consts, 128 ** -0.5, rank=rank,
                          k_tail=kt, v_tail=vt, tail_len=T, tail_cap=T)
    sentinel = torch.full_like(plan.out, 7.0)
    plan.out.copy_(sentinel)
    q1 = torch.randn(1, h_kv, G, 128, generator=gen).to(DEV).half()
    mine = torch.empty_like(q1)
    got = plan.run(q=q1, out=mine)
    ref = k2b.decode(q1, pool.pages, table, ln, S, seq.basis16, consts, 128 ** -0.5, rank=rank,
                     k_tail=kt, v_tail=vt, tail_len=T, tail_cap=T)
    torch.cuda.synchronize()
    assert got.data_ptr() == mine.data_ptr() and torch.equal(mine, ref)
    assert torch.equal(plan.out, sentinel)
    with pytest.raises(ValueError):   # a query of another dtype than the bound one
        plan.run(q=q1.float().contiguous())


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
def test_rtn_decode_model_dtype_query(dt):
    gen = torch.Generator().manual_seed(23)
    h_kv, G, S, T = 8, 4, 1024, 40
    codec = dict(k_bits=4, v_bits=4, k_group=32, v_group=32)
    k = torch.randn(h_kv, S + T, 128, generator=gen).half()
    v = torch.randn(h_kv, S + T, 128, generator=gen).half()
    pool = rtn.PagePool(S // 16 + 2, h_kv, DEV, **codec)
    ids = pool.alloc(S // 16)
    rtn.append(k[:, :S].to(DEV), v[:, :S].to(DEV), pool.pages, torch.tensor(ids, dtype=torch.int32, device=DEV),
               **codec)
    table = torch.tensor([ids], dtype=torch.int32, device=DEV)
    ln = torch.tensor([S], dtype=torch.int32, device=DEV)
    kt, vt = k[:, S:].unsqueeze(0).to(DEV).contiguous(), v[:, S:].unsqueeze(0).to(DEV).contiguous()
    q = torch.randn(1, h_kv, G, 128, generator=gen).to(DEV).to(dt)
    common = dict(k_tail=kt, v_tail=vt, tail_len=T, tail_cap=T, **codec)
    out_d = rtn.decode(q, pool.pages, table, ln, S, 128 ** -0.5, **common)
    out_f = rtn.decode(q.float().contiguous(), pool.pages, table, ln, S, 128 ** -0.5, **common)
    torch.cuda.synchronize()
    assert out_d.dtype == dt
    assert torch.equal(out_d, out_f.to(dt)), f"{dt}: max |diff| {(out_d.float() - out_f).abs().max().item():.3e}"


def _bf16_exact(x):
    """Rows exactly representable in both bf16 and fp16 (bf16's 8 bits of
    mantissa, fp16's range)."""
    return x.float().bfloat16().half()


@pytest.mark.parametrize("S,T", [(1024, 40), (128, 100)])
@pytest.mark.parametrize("fold", [False, True])
def test_k2b_bf16_window_equals_fp16_window(fold, S, T):
    """The same window rows given as bf16 (tail_dtype BF16: bf16 MFMA with a
    bf16 hi/lo query, bf16 values in the merge) and as fp16: the outputs agree
    to the query split's precision; rows given apart land in the window
    buffer bit for bit.  128 packed tokens and 100 window rows: most window
    tiles are scored by workgroups with no packed tokens (a separate code
    path, whose dtype branch must be a scalar one)."""
    gen = torch.Generator().manual_seed(24)
    h_kv, rank, G = 8, 32, 4
    _, _, _, consts, pool, seq, kt, vt, table = _k2b_case(gen, h_kv, rank, S, T)
    kt, vt = _bf16_exact(kt), _bf16_exact(vt)
    q = torch.randn(1, h_kv, G, 128, generator=gen).to(DEV)
    ln = torch.tensor([S], dtype=torch.int32, device=DEV)
    outs = {}
    for dt in (torch.float16, torch.bfloat16):
        k_w, v_w = kt.to(dt).clone(), vt.to(dt).clone()
        new_kv = None
        if fold:   # the newest 2 rows given apart, their buffer rows zeroed
            new_kv = (k_w[:, :, T - 2:].clone(), v_w[:, :, T - 2:].clone())
            k_w[:, :, T - 2:] = 0
            v_w[:, :, T - 2:] = 0
        outs[dt] = k2b.decode(q, pool.pages, table, ln, S, seq.basis16, consts, 128 ** -0.5, rank=rank,
                              k_tail=k_w, v_tail=v_w, tail_len=T, tail_cap=T, new_kv=new_kv)
        torch.cuda.synchronize()
        assert torch.equal(k_w.float(), kt.float()) and torch.equal(v_w.float(), vt.float())
    err = (outs[torch.bfloat16] - outs[torch.float16]).abs().max().item()
    assert err <= 2e-5 * outs[torch.float16].abs().max().item(), err


@pytest.mark.parametrize("S,T", [(512, 40), (128, 100)])
def test_rtn_bf16_window_equals_fp16_window(S, T):
    gen = torch.Generator().manual_seed(25)
    h_kv, G = 8, 4
    codec = dict(k_bits=4, v_bits=4, k_group=32, v_group=32)
    k = torch.randn(h_kv, S + T, 128, generator=gen).half()
    v = torch.randn(h_kv, S + T, 128, generator=gen).half()
    pool = rtn.PagePool(S // 16 + 2, h_kv, DEV, **codec)
    ids = pool.alloc(S // 16)
    rtn.append(k[:, :S].to(DEV), v[:, :S].to(DEV), pool.pages, torch.tensor(ids, dtype=torch.int32, device=DEV),
               **codec)
    table = torch.tensor([ids], dtype=torch.int32, device=DEV)
    ln = torch.tensor([S], dtype=torch.int32, device=DEV)
    kt = _bf16_exact(k[:, S:]).unsqueeze(0).to(DEV).contiguous()
    vt = _bf16_exact(v[:, S:]).unsqueeze(0).to(DEV).contiguous()
    q = torch.randn(1, h_kv, G, 128, generator=gen).to(DEV)
    outs = [rtn.decode(q, pool.pages, table, ln, S, 128 ** -0.5, k_tail=kt.to(dt), v_tail=vt.to(dt), tail_len=T,
                       tail_cap=T, **codec) for dt in (torch.float16, torch.bfloat16)]
    torch.cuda.synchronize()
    assert (outs[1] - outs[0]).abs().max().item() <= 2e-5 * outs[0].abs().max().item()


def test_spectral_merge_bf16_window_equals_fp16_window():
    """The spectral decode's merge reads a bf16 window (win_dtype BF16) as the
    fp16 one: the window alone (no committed token), the same rows in both."""
    from bmx_amd import spectral
    gen = torch.Generator().manual_seed(26)
    h_kv, G, T = 8, 4, 100
    kw = _bf16_exact(torch.randn(h_kv, T, 128, generator=gen)).to(DEV)
    vw = _bf16_exact(torch.randn(h_kv, T, 128, generator=gen)).to(DEV)
    q = torch.randn(h_kv, G, 128, generator=gen).half().to(DEV)
    consts = k2b.CodecConsts.make(v_seed=0)
    outs = [spectral.decode_attention(None, None, None, None, None, 0, consts, q, 128 ** -0.5, k_win=kw.to(dt),
                                      v_win=vw.to(dt), out_dtype=torch.float32)
            for dt in (torch.float16, torch.bfloat16)]
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1])
    ref = torch.softmax((q.float() @ kw.float().transpose(1, 2)) * 128 ** -0.5, -1) @ vw.float()
    assert (outs[0] - ref).abs().max().item() <= 1e-5

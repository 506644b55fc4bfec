"""GPU tests of the torch.library operators: each equals the direct call bit
for bit, traces into one torch.compile graph without a break, passes the
library's schema and fake-tensor checks, and replays under CUDA-graph capture
(every replay checked against the eager result, with eager work between)."""

import pytest
import torch

from bmx_amd import k2b, ops, rtn, synth

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _k2b_args(gen, h_kv=8, rank=32, S=1024, T=24, G=4, dt=torch.float16):
    k_pre = synth.k2b_keys(h_kv, S + T, rank, gen)
    v = synth.values(h_kv, S + T, gen)
    svd = synth.first_page_svd(k_pre, rank)
    consts = k2b.CodecConsts.make(v_seed=0)
    pool = synth.PagePool(S // 16, h_kv, rank, DEV, gen=gen)
    seq = synth.encode_sequence(pool, k_pre[:, :S].to(DEV), v[:, :S].to(DEV), rank, consts, svd=svd)
    kt = synth.rope_keys(k_pre[:, S:], S, consts).unsqueeze(0).to(DEV).contiguous()
    vt = v[:, S:].unsqueeze(0).half().to(DEV).contiguous()
    table = synth.page_table([seq], device=DEV)
    q = torch.randn(1, h_kv, G, 128, generator=gen).to(DEV).to(dt)
    ln = torch.tensor([S], dtype=torch.int32, device=DEV)
    tl = torch.tensor([T], dtype=torch.int32, device=DEV)
    args = (q, pool.pages, table, ln, S, seq.basis16)
    kw = dict(sm_scale=128 ** -0.5, rank=rank, k_tail=kt, v_tail=vt, tail_len=tl, tail_cap=T,
              **ops.consts_args(consts))
    direct = dict(rank=rank, k_tail=kt, v_tail=vt, tail_len=tl, tail_cap=T)
    return args, kw, consts, direct


def test_k2b_decode_operator_equals_direct_call_and_compiles():
    gen = torch.Generator().manual_seed(31)
    args, kw, consts, direct = _k2b_args(gen)
    out = torch.ops.bmx.k2b_decode(*args, **kw)
    ref = k2b.decode(*args, consts, 128 ** -0.5, **direct)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)

    def layer(q):   # a decode step with work either side, as in an attention layer
        return torch.ops.bmx.k2b_decode(q * 1.0, *args[1:], **kw).float().sum(dim=2)

    compiled = torch.compile(layer, fullgraph=True, backend="aot_eager")
    got = compiled(args[0])
    torch.cuda.synchronize()
    assert torch.equal(got, layer(args[0]))
    torch.library.opcheck(torch.ops.bmx.k2b_decode.default, args, kw,
                          test_utils=("test_schema", "test_faketensor"))


def test_k2b_decode_operator_under_graph_capture():
    gen = torch.Generator().manual_seed(32)
    args, kw, consts, direct = _k2b_args(gen)
    q = args[0]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):   # warm-up: the workspace is sized outside the capture
        torch.ops.bmx.k2b_decode(*args, **kw)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = torch.ops.bmx.k2b_decode(*args, **kw)
    for i in range(3):
        q.copy_(torch.randn(q.shape, generator=gen).to(DEV).half())
        g.replay()
        torch.cuda.synchronize()
        ref = k2b.decode(*args, consts, 128 ** -0.5, **direct)
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"replay {i}"


def test_k2b_append_operator_writes_the_same_pages():
    gen = torch.Generator().manual_seed(33)
    h_kv, rank, S = 8, 32, 256
    k_pre = synth.k2b_keys(h_kv, S, rank, gen).to(DEV)
    v = synth.values(h_kv, S, gen).to(DEV)
    consts = k2b.CodecConsts.make(v_seed=3)
    basis32 = synth.first_page_svd(k_pre, rank)[1].contiguous().to(DEV)
    basis16 = basis32.half()
    pb = k2b.page_bytes(h_kv, rank)
    p1 = torch.zeros(S // 16 + 4, pb, dtype=torch.uint8, device=DEV)
    p2 = torch.zeros_like(p1)
    ids = torch.randperm(S // 16 + 4, generator=gen)[:S // 16].to(torch.int32).to(DEV)
    k2b.append(k_pre, v, basis32, basis16, p1, ids, consts, rank=rank)
    torch.ops.bmx.k2b_append(k_pre, v, basis32, basis16, p2, ids, list(consts.codebook), list(consts.sign_bits),
                             rank)
    torch.cuda.synchronize()
    assert torch.equal(p1, p2) and p2.any()


def test_rtn_operators_equal_direct_calls():
    gen = torch.Generator().manual_seed(34)
    h_kv, G, S, T = 8, 4, 512, 16
    codec = dict(k_bits=4, v_bits=4, k_group=32, v_group=32)
    k = torch.randn(h_kv, S + T, 128, generator=gen).half().to(DEV)
    v = torch.randn(h_kv, S + T, 128, generator=gen).half().to(DEV)
    pb = rtn.page_bytes(h_kv, **codec)
    p1 = torch.zeros(S // 16, pb, dtype=torch.uint8, device=DEV)
    p2 = torch.zeros_like(p1)
    ids = torch.arange(S // 16, dtype=torch.int32, device=DEV)
    rtn.append(k[:, :S], v[:, :S], p1, ids, **codec)
    torch.ops.bmx.rtn_append(k[:, :S], v[:, :S], p2, ids, 4, 4, 32, 32)
    torch.cuda.synchronize()
    assert torch.equal(p1, p2)
    table = ids.view(1, -1).contiguous()
    ln = torch.tensor([S], dtype=torch.int32, device=DEV)
    kt, vt = k[:, S:].unsqueeze(0).contiguous(), v[:, S:].unsqueeze(0).contiguous()
    q = torch.randn(1, h_kv, G, 128, generator=gen).half().to(DEV)
    out = torch.ops.bmx.rtn_decode(q, p2, table, ln, S, 128 ** -0.5, 4, 4, 32, 32, k_tail=kt, v_tail=vt,
                                   tail_len_value=T, tail_cap=T)
    ref = rtn.decode(q, p1, table, ln, S, 128 ** -0.5, k_tail=kt, v_tail=vt, tail_len=T, tail_cap=T, **codec)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)


def test_prefill_operator_equals_direct_call_and_compiles():
    from bmx_amd import prefill

    g = torch.Generator(device=DEV).manual_seed(33)
    q = torch.randn(16, 200, 128, device=DEV, generator=g).half()
    k = torch.randn(4, 1000, 128, device=DEV, generator=g).half()
    v = torch.randn(4, 1000, 128, device=DEV, generator=g).half()
    out = torch.ops.bmx.prefill_attention(q, k, v, 128 ** -0.5, True)
    ref = prefill.attention(q, k, v, 128 ** -0.5, causal=True)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)

    def layer(q):   # the attention with work either side
        return torch.ops.bmx.prefill_attention(q * 1.0, k, v, 128 ** -0.5, True).float().sum(dim=0)

    compiled = torch.compile(layer, fullgraph=True, backend="aot_eager")
    got = compiled(q)
    torch.cuda.synchronize()
    assert torch.equal(got, layer(q))
    torch.library.opcheck(torch.ops.bmx.prefill_attention.default, (q, k, v, 128 ** -0.5, True), {},
                          test_utils=("test_schema", "test_faketensor"))

"""The allocation-free decode entry point (bmx_k2b_decode_noalloc, a static
per-device scratch array in place of the caller's workspace) against the
workspace entry point (bmx_k2b_decode), through the C-ABI: the same kernels
over the same inputs, so the outputs must be identical, on two calls in a row
(the second smaller, over the scratch the first left behind), and both within
the oracle's bar.  A call whose partials exceed the scratch is refused."""

import ctypes as ct

import pytest
import torch

from bmx_amd import _lib, k2b, synth
from oracle import attention as A

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _case(S, T, seed, pool_pages):
    gen = torch.Generator().manual_seed(seed)
    h_kv, rank, G = 8, 32, 4
    k_pre = synth.k2b_keys(h_kv, S + T, rank, gen)
    v = synth.values(h_kv, S + T, gen)
    svd = synth.first_page_svd(k_pre, rank)
    consts = k2b.CodecConsts.make(v_seed=0)
    pool = synth.PagePool(pool_pages, h_kv, rank, DEV, gen=gen)
    seq = synth.encode_sequence(pool, k_pre[:, :S].to(DEV), v[:, :S].to(DEV), rank, consts, svd=svd)
    inv = torch.tensor(consts.inv_freq)
    cos, sin = A.rope_cos_sin(inv, torch.arange(S, S + T))
    k_tail = A.apply_rope(k_pre[:, S:].float(), cos, sin).half()
    v_tail = v[:, S:]
    q = torch.randn(1, h_kv, G, 128, generator=gen)
    cache = A.K2bOracleCache(h_kv, 128, rank)
    for p in range(S // 128):
        cache.commit(k_pre[:, p * 128:(p + 1) * 128], v[:, p * 128:(p + 1) * 128],
                     us_override=svd if p == 0 else None)
    ref = A.k2b_naive_attention(q.view(h_kv * G, 1, 128), cache, inv, k_tail, v_tail, G, 128 ** -0.5)
    args = dict(q=q.to(DEV), pages=pool.pages, page_table=synth.page_table([seq], device=DEV),
                packed_len=torch.tensor([S], dtype=torch.int32, device=DEV), max_packed_len=S,
                basis16=seq.basis16, consts=consts, sm_scale=128 ** -0.5, rank=rank,
                k_tail=k_tail.unsqueeze(0).to(DEV), v_tail=v_tail.unsqueeze(0).to(DEV),
                tail_len=torch.tensor([T], dtype=torch.int32, device=DEV), tail_cap=T)
    return args, ref.view(1, h_kv, G, 128), pool


def _noalloc(args):
    """The same call through bmx_k2b_decode_noalloc (workspace fields unset)."""
    out = torch.full_like(args["q"], float("nan"))
    captured = {}
    k2b.decode(**args, out=out, _capture=lambda a: captured.setdefault("a", a))
    a = captured["a"]
    a.workspace, a.workspace_bytes = None, 0
    stream = ct.c_void_p(torch.cuda.current_stream().cuda_stream)
    _lib.check(_lib.lib().bmx_k2b_decode_noalloc(ct.byref(a), stream), "bmx_k2b_decode_noalloc")
    return out


def test_noalloc_matches_workspace_entry_point_twice():
    results = []
    for S, T, seed in ((16384, 200, 61), (2048, 40, 62)):   # the second call is smaller
        args, ref, pool = _case(S, T, seed, S // 16 + 8)
        print(f"case S {S} T {T}: workspace {k2b_ws(args)} B of {_lib.DECODE_SCRATCH_BYTES}", flush=True)
        want = k2b.decode(**args)
        got = _noalloc(args)
        torch.cuda.synchronize()
        same = torch.equal(got, want)
        err = (got.cpu().double() - ref.double()).abs().max().item()
        print(f"S {S} T {T}: identical to bmx_k2b_decode: {same}; vs oracle max_abs {err:.3e}", flush=True)
        assert same
        assert err <= 2e-3
        results.append(got)
        del pool
    # a third call repeats the first shape over the second's leftovers
    args, _, _ = _case(16384, 200, 61, 16384 // 16 + 8)
    again = _noalloc(args)
    torch.cuda.synchronize()
    assert torch.equal(again, results[0])


def k2b_ws(args) -> int:
    captured = {}
    k2b.decode(**args, _capture=lambda a: captured.setdefault("a", a))
    return int(_lib.lib().bmx_k2b_decode_workspace_bytes(ct.byref(captured["a"])))


def test_noalloc_refuses_calls_above_the_scratch():
    a = _lib.DecodeArgs()
    a.geom = _lib.Geom(8, 32, 16)
    a.batch = 64
    a.max_packed_len = 1 << 20
    a.tail_cap = 4096
    # valid stand-ins for every pointer and size the argument checks look at
    # (the call must be refused on the scratch size, never launched)
    a.rope_scaling = 1.0
    a.q = a.out = a.packed_len = a.pages = a.basis = a.k_tail = a.v_tail = 1 << 20
    a.n_pool_pages, a.max_pages = 1, (1 << 20) // 16
    a.tail_len = 1 << 20
    need = int(_lib.lib().bmx_k2b_decode_workspace_bytes(ct.byref(a)))
    assert need > _lib.DECODE_SCRATCH_BYTES
    rc = _lib.lib().bmx_k2b_decode_noalloc(ct.byref(a), None)
    msg = _lib.lib().bmx_last_error().decode()
    print(f"refused: status {rc}: {msg}", flush=True)
    assert rc == 2 and "static scratch" in msg   # BMX_E_WORKSPACE, before any launch


def test_noalloc_under_graph_capture():
    """One noalloc call captured in a HIP graph, after a warm-up call outside
    the capture (it fetches the scratch's device address and raises the split
    kernel's LDS limit); nothing in the call records a memset.  Each replay,
    with a new query written eagerly and the device synchronised between
    replays, equals the workspace entry point on the same query bit for bit."""
    args, _, pool = _case(4096, 40, 63, 4096 // 16 + 8)
    q = args["q"]
    out = torch.full_like(q, float("nan"))
    captured = {}
    k2b.decode(**args, out=out, _capture=lambda a: captured.setdefault("a", a))
    a = captured["a"]
    a.workspace, a.workspace_bytes = None, 0
    lib = _lib.lib()
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        _lib.check(lib.bmx_k2b_decode_noalloc(ct.byref(a), ct.c_void_p(side.cuda_stream)), "warm-up")
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        st = torch.cuda.current_stream()
        _lib.check(lib.bmx_k2b_decode_noalloc(ct.byref(a), ct.c_void_p(st.cuda_stream)), "captured call")
    torch.cuda.synchronize()
    gen = torch.Generator().manual_seed(64)
    for rep in range(3):
        q.copy_(torch.randn(q.shape, generator=gen).to(DEV))
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        want = k2b.decode(**args)
        torch.cuda.synchronize()
        same = torch.equal(out, want)
        print(f"replay {rep}: identical to bmx_k2b_decode: {same}", flush=True)
        assert same
    del graph, pool

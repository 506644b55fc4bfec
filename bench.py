#!/usr/bin/env python3
"""Decode-attention benchmark of the k2b packed-KV path on one MI355X.

Workload (BASELINE.json configs[2] geometry at the headline 64k context):
Llama-3.1-8B attention geometry (32 layers, 32 query / 8 KV heads, head_dim
128), batch 1, k2b recipe at rank 32 (752 bytes per token per layer = 2.94
bits per entry), total context 65,536 tokens = 65,408 committed (packed) +
128 fp16 recent-window tokens, RoPE theta 5e5 applied at read.  32 distinct
synthetic layer caches (1.6 GB of pages) so a step streams from HBM, not from
the 256 MB MALL.  Inputs are resident in HBM before timing starts.

A "step" is one decode-attention call per layer for all 32 layers (the
attention part of one generated token).  A call is two kernels back to back
(k2b_decode_split_kernel, then combine_kernel<true>).  Printed: one JSON line with
the step time; the roofline of a decode call (its algorithmic bytes over the
average call duration, from HIP events around the back-to-back timed region on
the library's stream), with the measured HBM traffic per call when a rocprofv3
FETCH_SIZE / WRITE_SIZE summary for this exact workload is committed under
profiles/; and the CPU chunked-path baseline (the oracle's restatement of
chunked_dequant_attention) timed on a bounded sample.
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

METRIC = "decode-attn µs/step + % HBM roofline, k2b 3.0 bpe, 64k ctx, 1 MI355X"
HBM_PEAK_GBS = 8000.0
H_KV, G, D = 8, 4, 128
TRAFFIC_FILE = Path(__file__).resolve().parent / "profiles" / "k2b_decode_traffic.json"
SPECTRAL_TRAFFIC_FILE = Path(__file__).resolve().parent / "profiles" / "spectral_dequant_traffic.json"


def measured_traffic(workload: dict, path: Path = TRAFFIC_FILE):
    """HBM bytes per decode call from the committed rocprofv3 PMC summary, if it
    was taken on this exact workload (else None)."""
    try:
        rec = json.loads(path.read_text())
    except (OSError, ValueError):
        return None
    if rec.get("workload") != workload:
        return None
    return rec.get("bytes_per_call")


def parse():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--ctx", type=int, default=65536)
    ap.add_argument("--rank", type=int, default=32)
    ap.add_argument("--layers", type=int, default=32)
    ap.add_argument("--window", type=int, default=128)
    ap.add_argument("--split-tokens", type=int, default=0)
    ap.add_argument("--layout", choices=["contig", "paged"], default="contig",
                    help="contig: each layer's pages in order in its own pool, no page table (the "
                         "layout PackedStreamingCache allocates); paged: one shuffled pool read "
                         "through a page table")
    ap.add_argument("--cpu-sample-tokens", type=int, default=0,
                    help="committed tokens of the CPU baseline's layer call (0: the workload's own)")
    ap.add_argument("--cpu-reps", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-fp16-comparator", action="store_true",
                    help="skip timing the dense fp16 decode at the same context")
    ap.add_argument("--prefill-ctx", type=int, default=8192)
    ap.add_argument("--prefill-chunk", type=int, default=512)
    ap.add_argument("--spectral-budget", type=float, default=2.5)
    ap.add_argument("--spectral-payload", choices=["rtn", "lloyd"], default="rtn",
                    help="spectral workload: the key payload (lloyd: the recipe's _lq suffix)")
    ap.add_argument("--spectral-values", choices=["perhead", "full"], default="perhead",
                    help="spectral workload: the value codec (full: the reference's k4_b recipe, "
                         "full-C turboquant_mse; perhead: k4ph_b, turboquant_mse_perhead)")
    ap.add_argument("--workload", choices=["decode", "stream", "rtn", "prefill", "batch", "spectral", "e2e",
                                           "general"],
                    default="decode",
                    help="decode: the headline 64k decode-attention step (default); stream: "
                         "BASELINE config 5, Qwen3-8B geometry, rank 16, an 8192-token prefill "
                         "then --stream-steps steps of one-token append + decode over 36 layers; "
                         "rtn: BASELINE config 1, RTN 4-bit per-channel keys / per-token values, "
                         "ctx --rtn-ctx, --rtn-layers layers; prefill: the second block of a cached "
                         "two-block prefill, --prefill-chunk queries over --prefill-ctx + chunk keys; "
                         "batch: BASELINE config 4, 16 ragged sequences of 4k-16k; spectral: the "
                         "k4 recipe's decode step (spectral keys at --spectral-budget, one layer "
                         "of Llama-3.1-8B geometry, --ctx tokens); e2e: ms per decode token under "
                         "HF generate() on a random-init Llama-3.1-8B-geometry fp16 model, dense "
                         "DynamicCache vs the streaming twin vs the packed cache (k2b_ph rank 16); "
                         "general: the decode step on the general page (--gen-head-dim, --rank, "
                         "--gen-group, --gen-bits, --gen-kv-heads, --gen-q-groups), --ctx tokens, --layers")
    ap.add_argument("--gen-head-dim", type=int, default=64)
    ap.add_argument("--gen-group", type=int, default=32)
    ap.add_argument("--gen-bits", type=int, default=3)
    ap.add_argument("--gen-kv-heads", type=int, default=8)
    ap.add_argument("--gen-q-groups", type=int, default=4)
    ap.add_argument("--e2e-ctx", default="4096,16384,65536")
    ap.add_argument("--e2e-decode", type=int, default=64, help="decode tokens per timed generate")
    ap.add_argument("--e2e-kinds", default="dense,streaming,packed")
    ap.add_argument("--e2e-layers", type=int, default=32)
    ap.add_argument("--e2e-parity", type=int, default=32,
                    help="greedy tokens compared between the streaming twin and the packed cache")
    ap.add_argument("--rtn-ctx", type=int, default=4096)
    ap.add_argument("--rtn-layers", type=int, default=1)
    ap.add_argument("--stream-steps", type=int, default=512)
    ap.add_argument("--stream-layers", type=int, default=36)
    ap.add_argument("--copy-calib-mib", type=int, default=0,
                    help="run one untimed device copy of this many MiB first (a known-size "
                         "kernel for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE counters)")
    return ap.parse_args()


def cpu_baseline(args, packed: int, tail: int) -> dict:
    """Time the CPU chunked path (oracle restatement of chunked_dequant_attention,
    fp32 torch) on one layer call: by default the workload's own (all of its
    committed tokens + its tail), so only the layer count scales it to a step;
    with --cpu-sample-tokens, that many committed tokens, scaled linearly (the
    chunked path is per-page work)."""
    import torch

    from bmx_amd import k2b, synth
    from oracle import attention as A

    gen = torch.Generator().manual_seed(1234)
    S = args.cpu_sample_tokens or packed
    k_pre = synth.k2b_keys(H_KV, S + tail, args.rank, gen)
    v = synth.values(H_KV, S + tail, gen)
    cache = A.K2bOracleCache(H_KV, D, args.rank)
    svd = synth.first_page_svd(k_pre, args.rank)
    for p in range(S // 128):
        cache.commit(k_pre[:, p * 128:(p + 1) * 128], v[:, p * 128:(p + 1) * 128],
                     us_override=svd if p == 0 else None)
    consts = k2b.CodecConsts.make()
    inv = torch.tensor(consts.inv_freq)
    k_tail = synth.rope_keys(k_pre[:, S:], S, consts)
    q = torch.randn(H_KV * G, 1, D, generator=gen)
    threads, host = cpu_threads()
    torch.set_num_threads(threads)
    A.k2b_chunked_attention(q, cache, inv, k_tail, v[:, S:], G, D ** -0.5)  # warm-up
    times = []
    for _ in range(args.cpu_reps):
        t0 = time.perf_counter()
        A.k2b_chunked_attention(q, cache, inv, k_tail, v[:, S:], G, D ** -0.5)
        times.append(time.perf_counter() - t0)
    t = statistics.median(times)
    # the same on one thread (fewer repetitions: each call takes seconds)
    torch.set_num_threads(1)
    times1 = []
    for _ in range(3):
        t0 = time.perf_counter()
        A.k2b_chunked_attention(q, cache, inv, k_tail, v[:, S:], G, D ** -0.5)
        times1.append(time.perf_counter() - t0)
    torch.set_num_threads(threads)
    t1 = statistics.median(times1)
    tok = (packed + tail) / (S + tail)
    scale = tok * args.layers
    what = (f"the headline layer call ({S} packed + {tail} tail tokens, h_kv 8, G 4, rank {args.rank})"
            if S == packed else f"1 layer of {S} packed + {tail} tail tokens (h_kv 8, G 4, rank {args.rank})")
    scaled = f"x {args.layers} layers" if S == packed else f"scaled x{tok:.2f} tokens x {args.layers} layers"
    return {"value": round(t * scale * 1e6, 1), "unit": "us/step", "cores": threads,
            "kind": "port",
            "sample": (f"{what}, median of {args.cpu_reps} after 1 warm-up = {t * 1e3:.1f} ms/layer-call, "
                       f"{scaled}"),
            "value_1_thread": round(t1 * scale * 1e6, 1),
            "sample_1_thread": f"median of 3 = {t1 * 1e3:.1f} ms/layer-call, same scaling",
            **host}


def fp16_comparator(args, torch, dev, ctx: int, our_us: float) -> dict:
    """The measured fp16 decode at the same context, the bar the packed path
    must beat: dense fp16 K/V of all ctx tokens per layer (8 KV heads, d 128),
    one query step of 32 heads, over args.layers distinct layers (8.6 GB at
    64k and 32 layers, past the MALL).  Three forms, the fastest reported:
    torch SDPA with grouped heads (ROCm's own attention), grouped bmm ->
    softmax -> bmm with the keys stored transposed (two skinny GEMMs that read
    K and V once each), and the library's dense fp16 split-KV decode kernel
    (bmx_fp16_decode: a bandwidth kernel, every K and V byte read once)."""
    import torch.nn.functional as F

    gen = torch.Generator(device=dev).manual_seed(99)
    n_l = args.layers
    Ks = [torch.randn(1, H_KV, ctx, D, generator=gen, device=dev, dtype=torch.float16) for _ in range(n_l)]
    Vs = [torch.randn(1, H_KV, ctx, D, generator=gen, device=dev, dtype=torch.float16) for _ in range(n_l)]
    KTs = [k[0].transpose(1, 2).contiguous() for k in Ks]   # (8, 128, ctx): no transposed bmm operand
    q = torch.randn(1, H_KV * G, 1, D, generator=gen, device=dev, dtype=torch.float16)
    qg = q.view(H_KV, G, D)
    scale = D ** -0.5

    def sdpa(i):
        return F.scaled_dot_product_attention(q, Ks[i], Vs[i], enable_gqa=True, scale=scale)

    def bmm(i):
        p = torch.softmax(torch.bmm(qg, KTs[i]).float() * scale, dim=-1).half()
        return torch.bmm(p, Vs[i][0])

    # the library's dense fp16 decode kernel (include/bmx_bench.h): split-KV
    # over the CUs, every K and V byte read once with wide coalesced loads
    import ctypes as ct

    from bmx_amd import _lib

    n_split = 64
    fd_out = torch.empty(H_KV, G, D, dtype=torch.float16, device=dev)
    fd_ws = torch.empty(int(_lib.lib().bmx_fp16_decode_workspace_bytes(H_KV, G, n_split)), dtype=torch.uint8,
                        device=dev)
    fd_args = []
    for i in range(n_l):
        fa = _lib.Fp16DecodeArgs()
        fa.q, fa.k, fa.v = qg.data_ptr(), Ks[i].data_ptr(), Vs[i].data_ptr()
        fa.stride_h, fa.stride_t = ctx * D, D
        fa.h_kv, fa.n_q_groups, fa.T, fa.n_split = H_KV, G, ctx, n_split
        fa.sm_scale = scale
        fa.out, fa.workspace, fa.workspace_bytes = fd_out.data_ptr(), fd_ws.data_ptr(), fd_ws.numel()
        fd_args.append(fa)
    fd_stream = torch.cuda.current_stream(dev).cuda_stream

    def hip_kernel(i):
        rc = _lib.lib().bmx_fp16_decode(ct.byref(fd_args[i]), fd_stream)
        if rc != 0:
            raise RuntimeError(f"bmx_fp16_decode failed ({rc})")
        return fd_out

    def timed(fn, reps=10):
        for _ in range(3):
            for i in range(n_l):
                fn(i)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            for i in range(n_l):
                fn(i)
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e3 / (reps * n_l)

    res = {}
    ref = bmm(0).float().view(-1)
    try:
        d = (sdpa(0).float().view(-1) - ref).abs().max().item()
        res["sdpa_us_per_call"] = round(timed(sdpa), 3)
        res["sdpa_vs_bmm_max_abs"] = d
    except RuntimeError as e:   # a backend without grouped heads: the bmm form stands
        res["sdpa_error"] = str(e)[:200]
    res["bmm_us_per_call"] = round(timed(bmm), 3)
    res["hip_kernel_vs_bmm_max_abs"] = (hip_kernel(0).float().view(-1) - ref).abs().max().item()
    res["hip_kernel_us_per_call"] = round(timed(hip_kernel), 3)
    best = min(v for k, v in res.items() if k.endswith("_us_per_call"))
    nbytes = ctx * H_KV * D * 2 * 2
    res.update({"kind": "dense fp16 K/V decode on the same GPU (fastest of the three forms)",
                "us_per_call": best, "bytes_per_call": nbytes,
                "achieved_GBs": round(nbytes / (best * 1e-6) / 1e9, 1),
                "packed_speedup": round(best / our_us, 3),
                "fp16_roofline_us": round(nbytes / HBM_PEAK_GBS / 1e3, 3)})
    del Ks, Vs, KTs, fd_ws, fd_out
    torch.cuda.empty_cache()
    return res


def _cpu_model() -> str:
    """The host CPU as lscpu reports it: every model-name field it prints
    (a virtual machine's "Model name" can be a bare family, the "BIOS Model
    name" the full part), the vendor and the family / model / stepping; else
    /proc/cpuinfo's model name."""
    import subprocess

    fields = {}
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            key, _, val = line.partition(":")
            key, val = key.strip(), val.strip()
            if key in ("Model name", "BIOS Model name", "Vendor ID", "CPU family", "Model", "Stepping") and val:
                fields.setdefault(key, val)
    except (OSError, subprocess.SubprocessError):
        pass
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    fields.setdefault("cpuinfo model name", line.split(":", 1)[1].strip())
                    break
    except OSError:
        pass
    return "; ".join(f"{k}: {v}" for k, v in fields.items()) or "unknown"


def cpu_threads() -> tuple:
    """(threads, host fields) for the CPU baseline.  The threads are every CPU
    this process may run on (its affinity mask), capped by OMP_NUM_THREADS
    when the environment sets it (the GPU box gives one GPU's job a 16-CPU
    share of a larger host); the fields report the host's logical CPU count,
    the affinity count, the threads used and the CPU model separately."""
    host = os.cpu_count() or 1
    try:
        avail = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        avail = host
    threads = avail
    env = os.environ.get("OMP_NUM_THREADS", "")
    if env.isdigit() and int(env) > 0:
        threads = min(threads, int(env))
    return threads, {"host_logical_cpus": host, "affinity_cpus": avail, "threads": threads,
                     "omp_num_threads": env or None, "cpu_model": _cpu_model()}


STREAM_METRIC = ("append + decode-attn µs/step, k2b rank 16, Qwen3-8B geometry, "
                 "8192-token prefill + 512 one-token steps, 1 MI355X")


def gpu_sleep(torch):
    """Queue a GPU sleep so that the host enqueues a region before it starts
    and its kernels then run back to back (device time only)."""
    try:
        torch.cuda._sleep(int(2e8))
    except Exception:  # pragma: no cover - sleep helper missing in this torch build
        pass


def run_stream(args, torch, k2b, synth, dev) -> dict:
    """Qwen3-8B attention geometry (36 layers, 32q/8kv heads,
    d 128, RoPE theta 1e6), k2b rank 16, recent window 128.  Per layer an
    8192-token prefill is committed once (untimed), then each of the timed
    steps appends one token to every layer's fp16 window and decodes; when the
    flush schedule moves (every 128 steps) each layer commits one codec page
    through bmx_k2b_append, its window drops those 128 tokens, and the layer's
    decode plan is rebound to the new packed length.  Per step and layer the
    device work is the decode call alone: the token's post-RoPE key and value
    are given to it apart (new_kv, with the window length from the host), and
    it stores them into the window; at commits the append and a window shift
    come on top."""
    L, W, rank, n_pre, n_steps = args.stream_layers, 128, 16, 8192, args.stream_steps
    N = n_pre + n_steps
    flush = lambda S: ((S - W) // 128) * 128 if S > W else 0   # noqa: E731
    P0, P_end = flush(n_pre), flush(N)
    cap = 2 * 128   # the window holds at most 255 tokens between commits
    consts = k2b.CodecConsts.make(theta=1e6)
    gen = torch.Generator(device=dev).manual_seed(5)
    ws = k2b.DecodeWorkspace()
    packed_len = torch.tensor([P0], dtype=torch.int32, device=dev)
    layers = []
    for li in range(L):
        k_pre = synth.k2b_keys(H_KV, N, rank, gen)
        v = synth.values(H_KV, N, gen)
        kv_post = torch.stack([synth.rope_keys(k_pre, 0, consts), v])   # (2, h_kv, N, d)
        pool = synth.PagePool(P_end // 16, H_KV, rank, dev,
                              gen=torch.Generator().manual_seed(li) if args.layout == "paged" else None)
        seq = synth.encode_sequence(pool, k_pre[:, :P0], v[:, :P0], rank, consts)
        kvt = torch.zeros(2, 1, H_KV, cap, D, dtype=torch.float16, device=dev)
        kvt[:, 0, :, : n_pre - P0] = kv_post[:, :, P0:n_pre]
        lay = {"k_pre": k_pre, "v": v, "kv_post": kv_post, "pool": pool, "seq": seq, "kvt": kvt,
               "k_new": kv_post[0].unsqueeze(0), "v_new": kv_post[1].unsqueeze(0),
               "q": torch.randn(1, H_KV, G, D, generator=gen, device=dev),
               "out": torch.empty(1, H_KV, G, D, device=dev)}
        layers.append(lay)
    torch.cuda.synchronize()

    def bind(lay, P, T):
        if args.layout == "contig":   # the layer's pages in order (asserted), read with no table
            ids = lay["seq"].page_ids
            assert ids == list(range(ids[0], ids[0] + len(ids)))
            pages, pt = lay["pool"].pages[ids[0]:], None
        else:
            pages, pt = lay["pool"].pages, synth.page_table([lay["seq"]], max_pages=P_end // 16, device=dev)
        lay["plan"] = k2b.DecodePlan(lay["q"], pages, pt, packed_len, P, lay["seq"].basis16,
                                     consts, D ** -0.5, rank=rank, k_tail=lay["kvt"][0],
                                     v_tail=lay["kvt"][1], tail_len=T, tail_cap=cap,
                                     out=lay["out"], workspace=ws)

    for lay in layers:
        bind(lay, P0, n_pre - P0)
    for _ in range(args.warmup):
        for lay in layers:
            lay["plan"].run()
    torch.cuda.synchronize()

    P, dev_ms, commits = P0, 0.0, 0
    t_wall = time.perf_counter()
    chunk = 16
    for c0 in range(0, n_steps, chunk):
        torch.cuda.synchronize()
        gpu_sleep(torch)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for s in range(n_pre + c0, n_pre + min(n_steps, c0 + chunk)):
            T = s - P   # the window's rows before token s
            P_new = flush(s + 1)
            if P_new > P:   # commit one codec page per layer, drop it from the window
                for lay in layers:
                    ids = lay["pool"].alloc(8)
                    lay["seq"].page_ids.extend(ids)
                    k2b.append(lay["k_pre"][:, P:P_new], lay["v"][:, P:P_new], lay["seq"].basis32,
                               lay["seq"].basis16, lay["pool"].pages,
                               torch.tensor(ids, dtype=torch.int32, device=dev), consts, rank=rank)
                    lay["kvt"][:, :, :, : T - 128] = lay["kvt"][:, :, :, 128:T]
                    bind(lay, P_new, T - 128)
                packed_len.fill_(P_new)
                P, commits, T = P_new, commits + 1, T - 128
            for lay in layers:   # token s is window row T, given apart
                lay["plan"].run(tail_len=T + 1, new_kv=(lay["k_new"][:, :, s:s + 1], lay["v_new"][:, :, s:s + 1]))
        e1.record()
        torch.cuda.synchronize()
        dev_ms += e0.elapsed_time(e1)
    t_wall = time.perf_counter() - t_wall
    step_us = dev_ms * 1e3 / n_steps
    return {
        "metric": STREAM_METRIC,
        "value": round(step_us, 2),
        "unit": "us/step",
        "n_gpus": 1,
        "steps": n_steps,
        "warmup": args.warmup,
        "ms_per_step": round(step_us / 1e3, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic",
        "config": {
            "workload": (f"k2b rank-16 streaming append + decode, Qwen3-8B geometry ({L} layers, "
                         f"32q/8kv heads, d 128, RoPE theta 1e6), batch 1, {n_pre}-token prefill "
                         f"({P0} packed + {n_pre - P0} fp16 window) then {n_steps} one-token steps, "
                         f"a codec page committed every 128 steps"),
            "layers": L, "rank": rank, "prefill": n_pre, "packed_start": P0, "packed_end": P,
            "layout": args.layout,
            "commits_per_layer": commits,
        },
        "device_time": "HIP events around 16-step chunks queued behind a GPU sleep",
        "wall_us_per_step": round(t_wall * 1e6 / n_steps, 1),
    }


RTN_METRIC = ("decode-attn µs/call + % HBM roofline, RTN 4-bit (rtn_channel keys g32, rtn_token "
              "values g32), 1 MI355X")


def run_rtn(args, torch, dev) -> dict:
    """one layer, batch 1, 32 query / 8 KV heads, d 128,
    ctx 4096 = 3968 packed + 128 fp16 window tokens; keys N(0,1) with 4 fixed
    channels x10 coded rtn_channel 4-bit (groups of 32 tokens), values N(0,1)
    coded rtn_token 4-bit (groups of 32 channels); seed 0.  A call is the RTN
    split kernel and the merge kernel.  With one layer the 4.8 MB working set
    stays in the 256 MB MALL between calls (the roofline against HBM peak is
    nominal there); --rtn-layers rotates over that many layer caches."""
    from bmx_amd import k2b, rtn
    from oracle import attention as A

    ctx, L, W = args.rtn_ctx, args.rtn_layers, 128
    P = ((ctx - W) // 128) * 128
    T = ctx - P
    codec = dict(k_bits=4, v_bits=4, k_group=32, v_group=32, k_arm=rtn.CHANNEL)
    gen = torch.Generator().manual_seed(0)
    ws = k2b.DecodeWorkspace()
    layers, cpu_case = [], None
    for li in range(L):
        k = torch.randn(H_KV, ctx, D, generator=gen)
        k[:, :, [3, 40, 77, 101]] *= 10.0
        k, v = k.half(), torch.randn(H_KV, ctx, D, generator=gen).half()
        q = torch.randn(1, H_KV, G, D, generator=gen)
        pool = rtn.PagePool(P // 16, H_KV, dev, **codec)
        ids = pool.alloc(P // 16)
        rtn.append(k[:, :P].to(dev), v[:, :P].to(dev), pool.pages,
                   torch.tensor(ids, dtype=torch.int32, device=dev), **codec)
        lay = {"pool": pool, "q": q.to(dev), "kt": k[:, P:].unsqueeze(0).to(dev),
               "vt": v[:, P:].unsqueeze(0).to(dev), "table": torch.tensor([ids], dtype=torch.int32, device=dev),
               "len": torch.tensor([P], dtype=torch.int32, device=dev),
               "tl": torch.tensor([T], dtype=torch.int32, device=dev)}
        lay["plan"] = rtn.DecodePlan(lay["q"], pool.pages, lay["table"], lay["len"], P, D ** -0.5,
                                     k_tail=lay["kt"], v_tail=lay["vt"], tail_len=lay["tl"], tail_cap=T,
                                     workspace=ws, **codec)
        layers.append(lay)
        if li == 0:
            cpu_case = (k, v, q)
    torch.cuda.synchronize()
    for _ in range(args.warmup):
        for lay in layers:
            lay["plan"].run()
    calls = max(args.steps, 1) * 50
    torch.cuda.synchronize()   # no sleep kernel ahead: the host enqueues faster than a call runs
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for i in range(calls):
        layers[i % L]["plan"].run()
    e1.record()
    torch.cuda.synchronize()
    call_us = e0.elapsed_time(e1) * 1e3 / calls
    page_bytes = rtn.page_bytes(H_KV, **codec)
    C = H_KV * D
    bytes_call = P * page_bytes // 16 + T * C * 2 * 2 + 2 * H_KV * G * D * 4
    achieved = bytes_call / (call_us * 1e-6) / 1e9
    res = {
        "metric": RTN_METRIC, "value": round(call_us, 3), "unit": "us/call", "n_gpus": 1,
        "steps": calls, "warmup": args.warmup, "ms_per_step": round(call_us / 1e3, 6),
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None, "dtype": "fp16",
        "data": "synthetic",
        "config": {"workload": (f"BASELINE config 1: {L} layer(s), batch 1, 32q/8kv heads, d 128, ctx {ctx} "
                                f"= {P} packed + {T} fp16 window, rtn_channel 4b g32 keys (4 outlier "
                                f"channels x10), rtn_token 4b g32 values, seed 0"),
                   "ctx": ctx, "layers": L, "bytes_per_token_layer": page_bytes // 16},
        "roofline": {"bound": "hbm", "kernel": "RTN decode call (rtn_decode_split_kernel + combine_kernel<false>)",
                     "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                     "bytes_per_launch": bytes_call, "avg_launch_us": round(call_us, 3),
                     "note": ("working set in the 256 MB MALL" if L * bytes_call < 200e6 else "streams from HBM")},
    }
    if not args.no_cpu_baseline:
        k, v, q = cpu_case
        c = A.RtnOracleCache(H_KV, **codec)
        for p in range(P // 128):
            c.commit(k[:, p * 128:(p + 1) * 128], v[:, p * 128:(p + 1) * 128])
        threads, host = cpu_threads()
        torch.set_num_threads(threads)
        qq = q.reshape(H_KV * G, 1, D)
        A.rtn_chunked_attention(qq, c, k[:, P:], v[:, P:], G, D ** -0.5)
        times = []
        for _ in range(args.cpu_reps):
            t0 = time.perf_counter()
            A.rtn_chunked_attention(qq, c, k[:, P:], v[:, P:], G, D ** -0.5)
            times.append(time.perf_counter() - t0)
        t = statistics.median(times)
        res["cpu_baseline"] = {"value": round(t * 1e6, 1), "unit": "us/call", "cores": threads, "kind": "port",
                               "sample": (f"the whole config-1 call ({P} packed + {T} tail tokens), median of "
                                          f"{args.cpu_reps} after 1 warm-up"),
                               **host}
    return res


BATCH_METRIC = "decode-attn µs/step, k2b rank 32, batch 16 ragged 4k-16k ctx, Llama-3.1-8B geometry, 1 MI355X"


def run_batch(args, torch, dev) -> dict:
    """batched decode, 16 sequences with contexts drawn
    uniformly from 4096..16384 (seeded), k2b rank 32, Llama-3.1-8B geometry
    (32 layers, 32q/8kv heads, d 128), each sequence its own frozen key basis
    and a 128-token fp16 window, 16-token pages shuffled over the pool.  A
    step is one decode call per layer for the whole batch (two kernels: the
    split kernel over 16 workgroups per sequence, the merge)."""
    from bmx_amd import k2b, synth

    B, W = 16, 128
    gen_h = torch.Generator().manual_seed(44)
    ctxs = [int(x) for x in torch.randint(4096, 16385, (B,), generator=gen_h)]
    packed = [((c - W) // 128) * 128 for c in ctxs]
    tails = [c - p for c, p in zip(ctxs, packed)]
    cap = max(tails)
    consts = k2b.CodecConsts.make()
    gen = torch.Generator(device=dev).manual_seed(45)
    pool = synth.PagePool(sum(packed) // 16 * args.layers, H_KV, args.rank, dev,
                          gen=torch.Generator().manual_seed(46))
    ws = k2b.DecodeWorkspace()
    plans = []
    for li in range(args.layers):
        seqs = []
        k_tail = torch.zeros(B, H_KV, cap, D, dtype=torch.float16, device=dev)
        v_tail = torch.zeros_like(k_tail)
        for i in range(B):
            k_pre = synth.k2b_keys(H_KV, ctxs[i], args.rank, gen)
            v = synth.values(H_KV, ctxs[i], gen)
            seqs.append(synth.encode_sequence(pool, k_pre[:, :packed[i]], v[:, :packed[i]], args.rank, consts))
            k_tail[i, :, :tails[i]] = synth.rope_keys(k_pre[:, packed[i]:], packed[i], consts)
            v_tail[i, :, :tails[i]] = v[:, packed[i]:]
            del k_pre, v
        basis = torch.stack([sq.basis16 for sq in seqs])
        q = torch.randn(B, H_KV, G, D, generator=gen, device=dev)
        pt = synth.page_table(seqs, device=dev)
        lens = torch.tensor(packed, dtype=torch.int32, device=dev)
        tl = torch.tensor(tails, dtype=torch.int32, device=dev)
        plans.append(k2b.DecodePlan(q, pool.pages, pt, lens, max(packed), basis, consts, D ** -0.5,
                                    rank=args.rank, k_tail=k_tail, v_tail=v_tail, tail_len=tl, tail_cap=cap,
                                    workspace=ws))
    torch.cuda.synchronize()
    for _ in range(args.warmup):
        for pl in plans:
            pl.run()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()   # no sleep kernel ahead: the host enqueues faster than a call runs
    for _ in range(args.steps):
        for pl in plans:
            pl.run()
    e1.record()
    torch.cuda.synchronize()
    step_us = e0.elapsed_time(e1) * 1e3 / args.steps
    call_us = step_us / args.layers
    C = H_KV * D
    page_bytes = k2b.page_bytes(H_KV, args.rank)
    bytes_call = (sum(packed) * page_bytes // 16 + B * C * args.rank * 2 + sum(tails) * C * 2 * 2
                  + 2 * B * H_KV * G * D * 4)
    achieved = bytes_call / (call_us * 1e-6) / 1e9
    return {
        "metric": BATCH_METRIC, "value": round(step_us, 2), "unit": "us/step", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(step_us / 1e3, 4),
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None, "dtype": "fp16", "data": "synthetic",
        "config": {"workload": (f"BASELINE config 4: batch {B}, ctx uniform 4096..16384 (seeded: mean "
                                f"{sum(ctxs) / B:.0f}), k2b rank {args.rank}, {args.layers} layers, 32q/8kv heads, "
                                f"d 128, 16-token pages shuffled, per-sequence basis, 128-token fp16 windows"),
                   "batch": B, "ctx": ctxs, "layers": args.layers, "rank": args.rank},
        "per_layer_us": round(call_us, 3),
        "tokens_per_s": round(B / (step_us * 1e-6), 1),
        "roofline": {"bound": "hbm", "kernel": "k2b decode call, batch 16 (k2b_decode_split_kernel + combine_kernel<true>)",
                     "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None, "bytes_per_launch": bytes_call,
                     "avg_launch_us": round(call_us, 3)},
    }


PREFILL_METRIC = ("prefill-attn µs/layer-call (second block of a cached two-block prefill), k2b rank 32, "
                  "Llama-3.1-8B geometry, 1 MI355X")
MFMA_FP16_PEAK_TFLOPS = 2500.0


def run_prefill(args, torch, dev) -> dict:
    """The prefill row: the second forward of a cached two-block prefill, the
    case where the packed cache serves queries of a prompt chunk -- n_q =
    --prefill-chunk new tokens at positions ctx .. ctx + n_q - 1 over ctx + n_q
    keys, the model's boolean mask, one layer of Llama-3.1-8B geometry (32
    query / 8 KV heads, d 128), k2b rank 32, recent window 128, fp16.  A call
    is PackedStreamingLayer.attend: the page dequant kernel (keys rotated in
    the pass, fp16 out), the window appended, bmx_prefill (MFMA flash
    attention, the roofline's kernel).  Beside it: the dequant kernel alone
    (HBM-bound: pages in, dense fp16 K and V out), bmx_prefill alone over the
    dense rows, and SDPA over the same dense fp16 K/V (what a dense fp16 cache
    pays with torch's kernels: the model's mask, and the bottom-right bias)."""
    import torch.nn.functional as F
    from transformers import LlamaConfig

    from bmx_amd import k2b, prefill, synth
    from bmx_amd.cache import PackedStreamingLayer
    from bmx_amd.specs import spec_pair
    from oracle import attention as A

    cfg = LlamaConfig(hidden_size=4096, num_attention_heads=32, num_key_value_heads=8, head_dim=128,
                      num_hidden_layers=32, rope_theta=500000.0)
    ctx, nq, W = args.prefill_ctx, args.prefill_chunk, 128
    N = ctx + nq
    k_spec, v_spec = spec_pair("k2b_ph", rank=args.rank)
    lay = PackedStreamingLayer(k_spec, v_spec, cfg, recent_window=W)
    gen = torch.Generator().manual_seed(5)
    k_pre = synth.k2b_keys(H_KV, N, args.rank, gen)
    v = synth.values(H_KV, N, gen).half()
    cos, sin = A.rope_cos_sin(lay._inv_freq, torch.arange(N))
    k_post = A.apply_rope(k_pre.float(), cos, sin).half()
    for lo, hi in ((0, ctx), (ctx, N)):
        lay.stash_pre_rope(k_pre[:, lo:hi].transpose(0, 1).unsqueeze(0).to(dev))
        lay.update(k_post[:, lo:hi].unsqueeze(0).to(dev), v[:, lo:hi].unsqueeze(0).to(dev))
    P = lay._committed_S_q
    q = torch.randn(H_KV * G, nq, D, generator=gen).half().to(dev)
    mask = (torch.arange(N, device=dev)[None, :] <= torch.arange(nq, device=dev)[:, None] + ctx)[None, None]
    scale = D ** -0.5
    Kd, Vd = k2b.dequant(lay._pool, lay._table[0, : P // 16].contiguous(), P, lay._basis16, lay._consts,
                         h_kv=H_KV, rank=args.rank, apply_rope=k2b.ROPE_FP16_TABLES, dtype=torch.float16)
    Kf = torch.cat([Kd, lay.keys.squeeze(0).half()], 1).repeat_interleave(G, 0).unsqueeze(0)
    Vf = torch.cat([Vd, lay.values.squeeze(0).half()], 1).repeat_interleave(G, 0).unsqueeze(0)

    def timed(fn, reps):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e3 / reps

    reps = max(args.steps, 1)
    call_us = timed(lambda: lay.attend(q, scale, is_causal=True, attention_mask=mask), reps)
    # the kernel alone: arguments built once, launches back to back (the
    # wrapper's per-call argument building is host time, timed beside it)
    pt_d = lay._table[0, : P // 16].contiguous()
    da, dK, dV = k2b.dequant_args(lay._pool, pt_d, P, lay._basis16, lay._consts, h_kv=H_KV, rank=args.rank,
                                  apply_rope=k2b.ROPE_FP16_TABLES, dtype=torch.float16)
    deq_us = timed(lambda: k2b.dequant_launch(da, dev), reps)
    deq_wrap_us = timed(lambda: k2b.dequant(lay._pool, pt_d, P, lay._basis16, lay._consts, h_kv=H_KV,
                                            rank=args.rank, apply_rope=k2b.ROPE_FP16_TABLES,
                                            dtype=torch.float16), reps)
    sdpa_us = timed(lambda: F.scaled_dot_product_attention(q.unsqueeze(0), Kf, Vf, attn_mask=mask, scale=scale),
                    reps)
    # the attention kernel alone (bmx_prefill + its split combine) over the
    # same dense fp16 K/V, grouped heads: the packed call's attention, and
    # what a dense fp16 cache would pay with the same kernel
    Kg, Vg = Kf[:, ::G].contiguous().squeeze(0), Vf[:, ::G].contiguous().squeeze(0)
    attn_us = timed(lambda: prefill.attention(q, Kg, Vg, scale, causal=True), reps)
    # the same dense fp16 K/V through the bottom-right causal bias the packed
    # layer uses for this mask (grouped heads)
    from torch.nn.attention.bias import causal_lower_right

    sdpa_lr_us = timed(lambda: F.scaled_dot_product_attention(q.unsqueeze(0), Kg.unsqueeze(0), Vg.unsqueeze(0),
                                                              attn_mask=causal_lower_right(nq, N), scale=scale,
                                                              enable_gqa=True), reps)
    out = lay.attend(q, scale, is_causal=True, attention_mask=mask).float()
    ref = F.scaled_dot_product_attention(q.unsqueeze(0).float(), Kf.float(), Vf.float(), attn_mask=mask,
                                         scale=scale).squeeze(0)
    page_bytes = k2b.page_bytes(H_KV, args.rank)
    deq_bytes = P * page_bytes // 16 + H_KV * D * args.rank * 2 + 2 * P * H_KV * D * 2
    flops = 4.0 * H_KV * G * D * (nq * ctx + nq * (nq + 1) / 2)   # QK^T and PV over the visible keys
    return {
        "metric": PREFILL_METRIC, "value": round(call_us, 2), "unit": "us/layer-call", "n_gpus": 1,
        "steps": reps, "warmup": 3, "ms_per_step": round(call_us / 1e3, 4), "higher_is_better": False,
        "scaling": "weak", "vs_baseline": None, "dtype": "fp16", "data": "synthetic",
        "config": {"workload": (f"cached two-block prefill, second block: {nq} queries at positions "
                                f"{ctx}..{N - 1} over {N} keys ({P} packed + {N - P} fp16 window), "
                                f"k2b rank {args.rank}, 32q/8kv heads, d 128, model mask"),
                   "ctx": ctx, "chunk": nq, "packed_tokens": P, "rank": args.rank},
        "roofline": {"bound": "mfma", "kernel": "prefill_kernel + prefill_combine_kernel (bmx_prefill)",
                     "achieved": round(flops / (attn_us * 1e-6) / 1e12, 1), "peak": MFMA_FP16_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(flops / (attn_us * 1e-6) / 1e12 / MFMA_FP16_PEAK_TFLOPS, 4),
                     "traffic": None, "flops_per_launch": flops, "avg_launch_us": round(attn_us, 3)},
        "prefill_call": {"attention_us": round(attn_us, 2),
                         "dequant_us": round(deq_us, 2), "dequant_wrapper_us": round(deq_wrap_us, 2),
                         "dequant_gbs": round(deq_bytes / (deq_us * 1e-6) / 1e9, 1),
                         "dequant_frac_of_hbm": round(deq_bytes / (deq_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                         "dequant_bytes": deq_bytes,
                         "sdpa_dense_fp16_us": round(sdpa_us, 2),
                         "sdpa_tflops": round(flops / (sdpa_us * 1e-6) / 1e12, 1),
                         "sdpa_frac_of_fp16_mfma_peak": round(flops / (sdpa_us * 1e-6) / 1e12
                                                              / MFMA_FP16_PEAK_TFLOPS, 4),
                         "packed_over_dense_fp16": round(call_us / sdpa_us, 3),
                         "sdpa_dense_fp16_lower_right_us": round(sdpa_lr_us, 2),
                         "packed_over_dense_fp16_lower_right": round(call_us / sdpa_lr_us, 3),
                         "dense_fp16_bmx_prefill_us": round(attn_us, 2),
                         "max_abs_vs_fp32_sdpa": (out - ref).abs().max().item()},
    }


SPECTRAL_METRIC = "decode-attn µs/layer-call, spectral (K4) keys, 64k ctx, 1 MI355X"
MFMA_FP16_DENSE_TFLOPS = 2500.0


def run_spectral(args, torch, dev) -> dict:
    """The spectral (K4) row: one decode call of one layer of Llama-3.1-8B
    attention geometry (32 query / 8 KV heads, d 128) at --ctx tokens, window
    --window, fp16 model, the k4 recipe at --spectral-budget on a synthetic
    pack of the reference's form (orthonormal basis under a positive diagonal
    weighting, power-law spectrum, bits by the reference's allocator), keys
    drawn with that spectrum.  A call is PackedStreamingLayer.attend as the
    reference runs a spectral step (its chunked path, packed_streaming.py:
    1016-1032, every page dequantized): the dequant kernel's partial form (tier
    codes -> Y_hat, Y_hat dec^T on MFMA, RoPE, the scores against the step's
    queries and the weights times the dequantized values on MFMA, one softmax
    partial per 64-token group), the window's partial and the merge.
    Beside it: the dequant kernel alone (its MFMA work over the coded
    directions is the bound) and the dense fp16 decode of the same context."""
    import math

    from transformers import LlamaConfig

    from bmx_amd import k2b, spectral
    from bmx_amd.cache import PackedStreamingLayer
    from bmx_amd.specs import spec_pair

    cfg = LlamaConfig(hidden_size=4096, num_attention_heads=32, num_key_value_heads=8, head_dim=128,
                      num_hidden_layers=32, rope_theta=500000.0)
    C = H_KV * D
    gen = torch.Generator().manual_seed(5)
    E, _ = torch.linalg.qr(torch.randn(C, C, generator=gen, dtype=torch.float64))
    w = 0.5 + torch.rand(C, generator=gen, dtype=torch.float64)
    lam = torch.arange(1, C + 1, dtype=torch.float64) ** -2.0
    lam *= C / lam.sum()
    pack = spectral.SpectralPack(enc=(w.sqrt()[:, None] * E).float(), dec=(w.rsqrt()[:, None] * E).float(),
                                 lam=lam.float(), bits=spectral.allocate_bits(lam, args.spectral_budget),
                                 budget=args.spectral_budget)
    recipe = (("k4_b" if args.spectral_values == "full" else "k4ph_b") + f"{args.spectral_budget:g}"
              + ("_lq" if args.spectral_payload == "lloyd" else ""))
    k_spec, v_spec = spec_pair(recipe, pack_path="synthetic")
    lay = PackedStreamingLayer(k_spec, v_spec, cfg, recent_window=args.window, pack=pack)
    N = args.ctx
    dec = pack.dec.to(dev)
    lam_d = lam.float().sqrt().to(dev)
    g2 = torch.Generator(device=dev).manual_seed(6)
    for lo in range(0, N, 8192):      # keys with the pack's spectrum, values random, in chunks
        n = min(8192, N - lo)
        z = torch.randn(n, C, generator=g2, device=dev) * lam_d
        kp = (z @ dec.T).reshape(n, H_KV, D).half()
        vv = torch.randn(1, H_KV, n, D, generator=g2, device=dev).half()
        lay.stash_pre_rope(kp.unsqueeze(0))
        lay.update(kp.transpose(0, 1).unsqueeze(0), vv)
    torch.cuda.synchronize()
    P = lay._committed_S_q
    dp = lay._dp
    q = torch.randn(H_KV * G, 1, D, generator=gen).half().to(dev)
    scale = D ** -0.5
    kt = lay._ktable[: P // 64]
    vt = lay._table[0, : P // 16].contiguous()
    Vb = torch.empty(H_KV, P, D, dtype=torch.float16, device=dev)
    Sb = torch.empty(H_KV, G, P, dtype=torch.float32, device=dev)
    qg = q.reshape(H_KV, G, D).contiguous()

    def timed(fn, reps):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e3 / reps

    reps = max(args.steps, 1)
    call_us = timed(lambda: lay.attend(q, scale), reps)
    n_parts = spectral.partial_count(dp, P, qg, k2b.ROPE_FP16_TABLES)
    Pb = torch.empty(H_KV, G, 130 * n_parts, dtype=torch.float32, device=dev)
    deq_us = timed(lambda: spectral.dequant(dp, lay._kpool, kt, lay._pool, vt, P, lay._consts,
                                            apply_rope=k2b.ROPE_FP16_TABLES, dtype=torch.float16,
                                            q=qg, partials=Pb, sm_scale=scale), reps)
    c_used = pack.c_used
    flops = 2.0 * P * c_used * C                            # Y_hat dec^T over the coded directions
    page_bytes = P // 64 * dp.k_page_bytes + P // 16 * dp.v_page_bytes
    out_bytes = H_KV * G * n_parts * 130 * 4          # the blocks' softmax partials
    comp = {} if args.no_fp16_comparator else fp16_comparator(args, torch, dev, N, call_us)
    # CPU: the oracle's restatement of the reference's chunked spectral step on
    # a bounded sample (dequant of the sample's keys and values, RoPE, one
    # softmax), scaled to the context
    cpu = None
    if not args.no_cpu_baseline:
        import numpy as np

        from oracle import attention as A
        from oracle import codecs as OC
        from oracle import spectral as O

        S = 4096
        L = O.Layout(pack.bits.numpy())
        rng = np.random.default_rng(0)
        codes = np.zeros((S // 64, 64, L.c_pad), np.int64)
        lloyd = None
        if args.spectral_payload == "lloyd":
            lloyd = {b: OC.gaussian_codebook(b).numpy() for b in set(L.slice_bits.tolist())}
        for b in set(L.slice_bits.tolist()):
            k = L.col_bits == b
            lo = 0 if lloyd else -(1 << (b - 1))
            codes[:, :, k] = rng.integers(lo, lo + (1 << b), (S // 64, 64, int(k.sum())))
        steps = rng.random((S // 64, L.c_pad)).astype(np.float32) * 0.1
        idx = torch.randint(0, 4, (S, C), dtype=torch.int16)
        v_h = 1 if args.spectral_values == "full" else H_KV
        norms = torch.rand(S, v_h) + 0.5
        qf = q.float().cpu()
        cos, sin = A.rope_cos_sin(torch.tensor(lay._consts.inv_freq), torch.arange(S))
        threads, host = cpu_threads()
        torch.set_num_threads(threads)

        def cpu_step():
            Kc = OC.from_matrix(torch.from_numpy(O.dequant(codes, steps, pack.dec.numpy(), L, lloyd=lloyd)).float(),
                                H_KV)
            Vc = OC.from_matrix(OC.dequant_v_perhead(idx, norms, bits=2, seed=0, h=v_h), H_KV)
            return A.naive_dense_attention(qf, A.apply_rope(Kc, cos, sin), Vc, G, scale)

        cpu_step()
        times = []
        for _ in range(3):
            t0 = time.perf_counter()
            cpu_step()
            times.append(time.perf_counter() - t0)
        t = statistics.median(times)
        cpu = {"value": round(t * (P + args.window) / S * 1e6, 1), "unit": "us/layer-call", "cores": threads,
               "kind": "port",
               "sample": (f"1 layer, {S} committed tokens (h_kv 8, G 4, c_pad {L.c_pad}): the oracle's "
                          f"spectral dequant (float64 Y_hat dec^T), value dequant, RoPE and one softmax, "
                          f"median of 3 = {t * 1e3:.1f} ms, scaled x{(P + args.window) / S:.1f} tokens"),
               **host}
    return {
        "metric": SPECTRAL_METRIC, "value": round(call_us, 2), "unit": "us/layer-call", "n_gpus": 1,
        "steps": reps, "warmup": 3, "ms_per_step": round(call_us / 1e3, 4), "higher_is_better": False,
        "scaling": "weak", "vs_baseline": None, "dtype": "fp16", "data": "synthetic",
        "config": {"workload": (f"{recipe} decode call: {P} packed + "
                                f"{N - P} fp16 window tokens, 32q/8kv heads, d 128, synthetic pack "
                                f"(c_used {c_used} of {C}, c_pad {dp.c_pad}, {spectral.payload_bpe(pack.bits):.3f} "
                                f"payload bpe keys)"),
                   "ctx": N, "packed_tokens": P, "budget": args.spectral_budget, "payload": args.spectral_payload,
                   "values": args.spectral_values,
                   "c_used": c_used,
                   "c_pad": dp.c_pad, "key_page_bytes": dp.k_page_bytes},
        "roofline": {"bound": "mfma", "kernel": (("spectral_partial128_kernel (pages -> per-128-token-block softmax partials)"
                                                if n_parts == P // 128 else
                                                "spectral_dequant_kernel, partial form (pages -> per-group softmax partials)")),
                     "achieved": round(flops / (deq_us * 1e-6) / 1e12, 1), "peak": MFMA_FP16_DENSE_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(flops / (deq_us * 1e-6) / 1e12 / MFMA_FP16_DENSE_TFLOPS, 4),
                     "traffic": measured_traffic({"ctx": N, "window": args.window, "budget": args.spectral_budget,
                                                  "c_pad": dp.c_pad, "form": "partials",
                                                  **({"payload": "lloyd"} if args.spectral_payload == "lloyd" else {}),
                                                  **({"values": "full"} if args.spectral_values == "full" else {})},
                                                 SPECTRAL_TRAFFIC_FILE),
                     "flops_per_launch": flops, "avg_launch_us": round(deq_us, 3),
                     "hbm_bytes_per_launch": page_bytes + out_bytes,
                     "hbm_frac": round((page_bytes + out_bytes) / (deq_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)},
        "spectral_call": {"dequant_us": round(deq_us, 2), "window_and_merge_us": round(call_us - deq_us, 2),
                          "fp16_comparator": comp},
        "cpu_baseline": cpu,
    }


E2E_METRIC = ("ms per decode token under HF generate(), Llama-3.1-8B geometry (random init, fp16), "
              "k2b_ph rank 16, 1 MI355X")


def run_general(args, torch, dev) -> dict:
    """The decode step on the general page (any geometry off the recipe's:
    head_dim 32/64, rank 64/128, residual groups 16/32/128, 2- or 4-bit keys),
    batch 1, --ctx tokens = packed + --window fp16 window rows, --layers
    distinct layer caches in one pool, contiguous pages.  A call is
    gen_split_kernel + gen_merge_kernel; the roofline counts the pages, the
    basis, the window and q/out."""
    from bmx_amd import k2b, synth

    d, R, grp, bits = args.gen_head_dim, args.rank, args.gen_group, args.gen_bits
    H, G, L, W = args.gen_kv_heads, args.gen_q_groups, args.layers, args.window
    packed = ((args.ctx - W) // 128) * 128
    tail = args.ctx - packed
    consts = k2b.CodecConsts.make(head_dim=d)
    n_pages = packed // 16
    pool = synth.PagePool(n_pages * L, H, R, dev, head_dim=d, group=grp, k_bits=bits)
    gen = torch.Generator(device=dev).manual_seed(2025)
    ws = k2b.DecodeWorkspace()
    plans = []
    for li in range(L):
        k_pre = synth.k2b_keys(H, args.ctx, R, gen, head_dim=d)
        v = synth.values(H, args.ctx, gen, head_dim=d)
        seq = synth.encode_sequence(pool, k_pre[:, :packed], v[:, :packed], R, consts)
        base = seq.page_ids[0]
        q = torch.randn(1, H, G, d, generator=gen, device=dev)
        kt = synth.rope_keys(k_pre[:, packed:], packed, consts).unsqueeze(0).contiguous()
        vt = v[:, packed:].unsqueeze(0).contiguous()
        plans.append(k2b.DecodePlan(q, pool.pages[base: base + n_pages], None,
                                    torch.tensor([packed], dtype=torch.int32, device=dev), packed, seq.basis16,
                                    consts, d ** -0.5, rank=R, k_tail=kt, v_tail=vt, tail_len=tail, tail_cap=tail,
                                    workspace=ws, group=grp, k_bits=bits))
        del k_pre, v
    torch.cuda.synchronize()
    for _ in range(args.warmup):
        for pl in plans:
            pl.run()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for _ in range(args.steps):
        for pl in plans:
            pl.run()
    end.record()
    torch.cuda.synchronize()
    call_us = start.elapsed_time(end) * 1e3 / (args.steps * L)
    C = H * d
    bytes_call = n_pages * pool.page_bytes + C * R * 2 + tail * C * 2 * 2 + 2 * H * G * d * 4
    return {
        "metric": f"general-page k2b decode-attn us/call, head_dim {d} rank {R} group {grp} {bits}-bit keys",
        "value": round(call_us, 2), "unit": "us/call", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "higher_is_better": False, "dtype": "fp32 q/out, fp16 MFMA (high + low parts)", "data": "synthetic",
        "config": {"workload": f"k2b general page, h_kv {H}, G {G}, head_dim {d}, rank {R}, group {grp}, "
                               f"{bits}-bit keys, batch 1, ctx {args.ctx} = {packed} packed + {tail} window, "
                               f"{L} layers, contiguous pages",
                   "page_bytes": pool.page_bytes},
        "roofline": {"bound": "hbm", "kernel": "gen_split_kernel + gen_merge_kernel", "achieved":
                     round(bytes_call / (call_us * 1e-6) / 1e9, 1), "peak": 8000.0, "unit": "GB/s",
                     "frac": round(bytes_call / (call_us * 1e-6) / 8e12, 4), "traffic": None,
                     "bytes_per_launch": bytes_call},
    }


def run_e2e(args, torch, dev) -> dict:
    """End-to-end decode latency, the reference's Mode A
    (scripts/profile_decode_ab.py:113-141, 248-279): per context and cache kind,
    one warm 1-token generate, then generate(1) and generate(1 + n) timed on the
    host around device synchronisation; ms/token = (t_n - t_1) / n, which
    cancels the prefill and counts every host-side cost of a step.  The model is
    Llama-3.1-8B's geometry (32 layers, 4096 hidden, 32/8 heads, d 128, 14336
    MLP, 128256 vocabulary, llama3 RoPE scaling) with random weights in fp16
    (no checkpoint is available offline); the prompt is random token ids.
    Before timing, greedy generate through the streaming twin and through the
    packed cache are compared token for token at the smallest context (the
    reference's parity gate; reported, since random weights leave near-ties)."""
    from transformers import DynamicCache, LlamaConfig, LlamaForCausalLM

    from bmx_amd.cache import PackedStreamingCache, StreamingQuantizedCache
    from bmx_amd.specs import spec_pair

    cfg = LlamaConfig(vocab_size=128256, hidden_size=4096, intermediate_size=14336,
                      num_hidden_layers=args.e2e_layers, num_attention_heads=32, num_key_value_heads=8,
                      head_dim=128, max_position_embeddings=131072, rope_theta=500000.0,
                      rope_scaling={"rope_type": "llama3", "factor": 8.0, "low_freq_factor": 1.0,
                                    "high_freq_factor": 4.0, "original_max_position_embeddings": 8192},
                      rms_norm_eps=1e-5, tie_word_embeddings=False)
    t0 = time.perf_counter()
    torch.manual_seed(0)
    prev = torch.get_default_dtype()
    torch.set_default_dtype(torch.float16)
    try:
        with torch.device(dev):
            model = LlamaForCausalLM(cfg).eval()
    finally:
        torch.set_default_dtype(prev)
    print(f"e2e: model built in {time.perf_counter() - t0:.1f} s", file=sys.stderr, flush=True)
    k_spec, v_spec = spec_pair("k2b_ph", rank=16)
    kinds = [k for k in args.e2e_kinds.split(",") if k]
    ctxs = [int(c) for c in args.e2e_ctx.split(",") if c]

    def fresh(kind):
        if kind == "dense":
            return DynamicCache()
        cls = StreamingQuantizedCache if kind == "streaming" else PackedStreamingCache
        return cls(model.config, k_spec, v_spec)

    def generate(kind, ids, n):
        cache = fresh(kind)
        attach = getattr(cache, "attach", None)
        if attach is not None:
            attach(model)
        torch.cuda.synchronize()
        t = time.perf_counter()
        with torch.no_grad():
            out = model.generate(ids, max_new_tokens=n, min_new_tokens=n, do_sample=False, use_cache=True,
                                 past_key_values=cache, pad_token_id=0)
        torch.cuda.synchronize()
        t = time.perf_counter() - t
        if attach is not None:
            cache.detach()
        return out, t

    def prompt(ctx):
        g = torch.Generator().manual_seed(1234)
        return torch.randint(10, cfg.vocab_size - 10, (1, ctx), generator=g).to(dev)

    parity = None
    if "streaming" in kinds and "packed" in kinds and args.e2e_parity > 0:
        ids = prompt(min(ctxs))
        a, _ = generate("streaming", ids, args.e2e_parity)
        b, _ = generate("packed", ids, args.e2e_parity)
        new_a, new_b = a[0, ids.shape[1]:], b[0, ids.shape[1]:]
        agree = int((new_a == new_b).cumprod(0).sum().item())
        parity = {"ctx": min(ctxs), "tokens": args.e2e_parity, "equal": bool(torch.equal(a, b)),
                  "leading_tokens_equal": agree}
        print(f"e2e: parity {parity}", file=sys.stderr, flush=True)
    rows = []
    for ctx in ctxs:
        ids = prompt(ctx)
        for kind in kinds:
            generate(kind, ids, 1)
            _, t1 = generate(kind, ids, 1)
            out, tn = generate(kind, ids, 1 + args.e2e_decode)
            row = {"cache": kind, "ctx": ctx,
                   "ms_per_decode_token": round((tn - t1) * 1e3 / args.e2e_decode, 3),
                   "prefill_plus1_s": round(t1, 3),
                   "peak_gib": round(torch.cuda.max_memory_allocated() / 2 ** 30, 2)}
            torch.cuda.reset_peak_memory_stats()
            rows.append(row)
            print(f"e2e: {row}", file=sys.stderr, flush=True)
    packed = [r for r in rows if r["cache"] == "packed"]
    head = max(packed, key=lambda r: r["ctx"]) if packed else rows[-1]
    return {
        "metric": E2E_METRIC,
        "value": head["ms_per_decode_token"],
        "unit": "ms/token",
        "n_gpus": 1,
        "steps": args.e2e_decode,
        "warmup": 1,
        "ms_per_step": head["ms_per_decode_token"],
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic (random weights, random prompt ids)",
        "config": {"workload": f"HF generate(), Llama-3.1-8B geometry ({args.e2e_layers} layers), batch 1, "
                               f"greedy, {args.e2e_decode} decode tokens per timed run, recent window 32",
                   "value_is": f"{head['cache']} at ctx {head['ctx']}", "recipe": "k2b_ph rank 16"},
        "rows": rows,
        "parity": parity,
    }


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}); "
              "how the k2b decode path would shard across GPUs is described in DESIGN.md",
              file=sys.stderr)
        sys.exit(2)
    import torch

    from bmx_amd import k2b, synth

    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda:0")
    if args.copy_calib_mib > 0:
        n = args.copy_calib_mib << 20
        src = torch.ones(n, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    if args.workload == "stream":
        print(json.dumps(run_stream(args, torch, k2b, synth, dev)), flush=True)
        return
    if args.workload == "rtn":
        print(json.dumps(run_rtn(args, torch, dev)), flush=True)
        return
    if args.workload == "prefill":
        print(json.dumps(run_prefill(args, torch, dev)), flush=True)
        return
    if args.workload == "batch":
        print(json.dumps(run_batch(args, torch, dev)), flush=True)
        return
    if args.workload == "spectral":
        print(json.dumps(run_spectral(args, torch, dev)), flush=True)
        return
    if args.workload == "e2e":
        print(json.dumps(run_e2e(args, torch, dev)), flush=True)
        return
    if args.workload == "general":
        print(json.dumps(run_general(args, torch, dev)), flush=True)
        return
    W = args.window
    packed = ((args.ctx - W) // 128) * 128
    tail = args.ctx - packed
    consts = k2b.CodecConsts.make()
    page_bytes = k2b.page_bytes(H_KV, args.rank)
    n_pages = packed // 16

    # ---- build the 32 layer caches with the HIP write kernel ----
    t_build = time.perf_counter()
    gen = torch.Generator(device=dev).manual_seed(2024)
    layers = []
    pool = synth.PagePool(n_pages * args.layers, H_KV, args.rank, dev,
                          gen=torch.Generator().manual_seed(7) if args.layout == "paged" else None)
    for li in range(args.layers):
        k_pre = synth.k2b_keys(H_KV, args.ctx, args.rank, gen)
        v = synth.values(H_KV, args.ctx, gen)
        seq = synth.encode_sequence(pool, k_pre[:, :packed], v[:, :packed], args.rank, consts)
        if args.layout == "contig":   # the layer's own run of pages, read with no table
            base = seq.page_ids[0]
            assert seq.page_ids == list(range(base, base + n_pages))
        lay = {
            "seq": seq,
            "pt": synth.page_table([seq], device=dev) if args.layout == "paged" else None,
            "pages": pool.pages if args.layout == "paged" else pool.pages[seq.page_ids[0]: seq.page_ids[0] + n_pages],
            "len": torch.tensor([packed], dtype=torch.int32, device=dev),
            "k_tail": synth.rope_keys(k_pre[:, packed:], packed, consts).unsqueeze(0).contiguous(),
            "v_tail": v[:, packed:].unsqueeze(0).contiguous(),
            "tail_len": torch.tensor([tail], dtype=torch.int32, device=dev),
            "q": torch.randn(1, H_KV, G, D, generator=gen, device=dev),
            "out": torch.empty(1, H_KV, G, D, device=dev),
        }
        layers.append(lay)
        del k_pre, v
        if li % 8 == 7:
            torch.cuda.synchronize()
            print(f"bench: built {li + 1}/{args.layers} layer caches", file=sys.stderr, flush=True)
    torch.cuda.synchronize()
    t_build = time.perf_counter() - t_build

    ws = k2b.DecodeWorkspace()
    for lay in layers:
        lay["plan"] = k2b.DecodePlan(
            lay["q"], lay["pages"], lay["pt"], lay["len"], packed, lay["seq"].basis16, consts,
            D ** -0.5, rank=args.rank, k_tail=lay["k_tail"], v_tail=lay["v_tail"],
            tail_len=lay["tail_len"], tail_cap=tail, out=lay["out"],
            split_tokens=args.split_tokens, workspace=ws)

    for _ in range(args.warmup):
        for lay in layers:
            lay["plan"].run()
    torch.cuda.synchronize()

    # untimed wall-clock pass: host + GPU, one step after another
    t_wall = time.perf_counter()
    for _ in range(args.steps):
        for lay in layers:
            lay["plan"].run()
    torch.cuda.synchronize()
    t_wall = time.perf_counter() - t_wall

    # timed pass (the reported value): K steps back to back, bracketed by events.
    # The host enqueues a call in a few microseconds, well under its device
    # time, so the queue stays ahead of the GPU with no head start; an idle
    # head start (a sleep kernel) would let the clocks fall before the region.
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for _ in range(args.steps):
        for lay in layers:
            lay["plan"].run()
    end.record()
    torch.cuda.synchronize()
    step_us = start.elapsed_time(end) * 1e3 / args.steps

    # diagnostic pass: each call bracketed by events, one between the two
    # kernels; the event packets add gaps of several microseconds, so these
    # split / combine figures overstate kernel time (the value and the roofline
    # come from the pass above)
    n_calls = args.steps * args.layers
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(n_calls)]
    torch.cuda.synchronize()
    gpu_sleep(torch)
    i = 0
    for _ in range(args.steps):
        for lay in layers:
            e0, e1, e2 = ev[i]
            e0.record()
            e1.record()  # marks the event recorded for torch; the library re-records it
            lay["plan"].run(e1)  # after the split kernel
            e2.record()
            i += 1
    torch.cuda.synchronize()
    split_us = [e0.elapsed_time(e1) * 1e3 for e0, e1, _ in ev]
    comb_us = [e1.elapsed_time(e2) * 1e3 for _, e1, e2 in ev]
    split_avg = statistics.mean(split_us)
    comb_avg = statistics.mean(comb_us)

    C = H_KV * D
    bytes_split = packed * page_bytes // 16 + C * args.rank * 2            # pages + basis
    bytes_call = bytes_split + tail * C * 2 * 2 + 2 * H_KV * G * D * 2      # + fp16 tail, q/out
    call_us = step_us / args.layers                                          # back-to-back calls
    achieved = bytes_call / (call_us * 1e-6) / 1e9
    bpe = page_bytes * 8 / 16 / (2 * C)
    workload_key = {"ctx": args.ctx, "window": W, "rank": args.rank, "h_kv": H_KV, "G": G, "layout": args.layout}
    res = {
        "metric": METRIC,
        "value": round(step_us, 2),
        "unit": "us/step",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(step_us / 1e3, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic",
        "config": {
            "workload": (f"k2b rank-{args.rank} decode attention, Llama-3.1-8B geometry "
                         f"({args.layers} layers, 32q/8kv heads, d 128), batch 1, ctx {args.ctx} "
                         f"= {packed} packed + {tail} fp16 tail, 16-token pages "
                         + ("in order per layer, no page table (the cache's layout)" if args.layout == "contig"
                            else "shuffled over one pool, read through a page table")
                         + ", RoPE 5e5 at read"),
            "layout": args.layout,
            "ctx": args.ctx, "packed_tokens": packed, "tail_tokens": tail, "layers": args.layers,
            "batch": 1, "rank": args.rank, "bits_per_entry_kv_avg": round(bpe, 4),
            "bytes_per_token_layer": page_bytes // 16,
            "split_tokens": args.split_tokens or "auto",
        },
        "per_layer_us": round(call_us, 3),
        "roofline": {
            "bound": "hbm",
            "kernel": "k2b decode call (k2b_decode_split_kernel + combine_kernel<true>)",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": measured_traffic(workload_key),
            "bytes_per_launch": bytes_call,
            "avg_launch_us": round(call_us, 3),
        },
        "decode_call": {
            "event_bracketed_split_us": round(split_avg, 3),
            "event_bracketed_combine_us": round(comb_avg, 3),
            "split_bytes": bytes_split,
            "wall_us_per_step": round(t_wall * 1e6 / args.steps, 1),
        },
        "build_s": round(t_build, 1),
    }
    if not args.no_fp16_comparator:
        del layers, pool
        torch.cuda.empty_cache()
        print("bench: timing the fp16 comparator", file=sys.stderr, flush=True)
        res["fp16_comparator"] = fp16_comparator(args, torch, dev, args.ctx, call_us)
    if not args.no_cpu_baseline:
        print(f"bench: GPU timing done ({step_us:.1f} us/step); timing the CPU baseline",
              file=sys.stderr, flush=True)
        res["cpu_baseline"] = cpu_baseline(args, packed, tail)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()

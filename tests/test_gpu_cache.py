"""PackedStreamingCache on the GPU: every commit through bmx_k2b_append, every
decode step through bmx_k2b_decode, every prefill through bmx_k2b_dequant + SDPA.

The product cache and the oracle-backed cache (the same host logic, the CPU
oracle in place of the three kernels: tests/oracle_cache.py) run the same tiny
Llama on the same GPU, teacher-forced through the same token sequence, and
their logits are compared step by step.  The oracle-backed cache is itself
pinned to the reference's own end-to-end run on the CPU
(test_cache_cpu.test_host_logic_reproduces_reference_run).

The model's key projections are made rank 8 plus 1% noise: keys then have the
low-rank-plus-small-residual structure k2b is built for.  (With fully random
key projections the 3-bit residual is as large as the keys and one ulp of
GPU-vs-CPU activation difference flips residual codes, so two correct
implementations drift apart chaotically; that case is covered on the CPU.)
"""

import sys
from pathlib import Path

import numpy as np
import pytest
import torch

from bmx_amd import k2b
from bmx_amd.cache import PackedStreamingCache
from bmx_amd.specs import spec_pair

sys.path.insert(0, str(Path(__file__).parent))
from oracle_cache import OracleCache  # noqa: E402

pytestmark = pytest.mark.gpu
GOLD = Path(__file__).parent / "golden"


def _tiny_model(n_layers=2):
    from transformers import LlamaConfig, LlamaForCausalLM

    cfg = LlamaConfig(vocab_size=256, hidden_size=256, intermediate_size=512, num_hidden_layers=n_layers,
                      num_attention_heads=4, num_key_value_heads=2, head_dim=128,
                      max_position_embeddings=4096, rope_theta=500000.0, initializer_range=0.1)
    torch.manual_seed(0)
    model = LlamaForCausalLM(cfg).eval()
    gen = torch.Generator().manual_seed(3)
    with torch.no_grad():
        for layer in model.model.layers:
            W = layer.self_attn.k_proj.weight
            U, s, Vh = torch.linalg.svd(W, full_matrices=False)
            low = (U[:, :8] * s[:8]) @ Vh[:8]
            W.copy_(low + 0.01 * W.abs().mean() * torch.randn(W.shape, generator=gen))
    return model.to("cuda")


def _run(cache, model, tokens, n_steps):
    got = []
    with cache.attach(model), torch.no_grad():
        got.append(model(tokens[:, :300], past_key_values=cache, use_cache=True).logits[0, -1])
        for i in range(1, n_steps):
            out = model(tokens[:, 300 + i - 1: 300 + i], past_key_values=cache, use_cache=True)
            got.append(out.logits[0, -1])
    return torch.stack(got).double().cpu()


@pytest.mark.parametrize("rank", [16, 32])
def test_product_cache_matches_oracle_backed_cache(rank):
    g = np.load(GOLD / "e2e_tiny_llama.npz")
    tokens = torch.from_numpy(g[f"r{rank}_tokens"]).cuda()
    n = 140
    model = _tiny_model()
    prod = PackedStreamingCache(model.config, *spec_pair("k2b_ph", rank=rank), recent_window=32)
    got = _run(prod, model, tokens, n)
    orc = OracleCache(model.config, *spec_pair("k2b_ph", rank=rank), recent_window=32)
    ref = _run(orc, model, tokens, n)
    err = (got - ref).abs().max(dim=1).values
    scale = ref.abs().max().item()
    agree = (got.argmax(1) == ref.argmax(1)).float().mean().item()
    print(f"r{rank}: product vs oracle-backed cache, logits max|err| {err.max():.3e} (prefill "
          f"{err[0]:.3e}) of max|logit| {scale:.3f}; argmax agreement {agree:.4f}; committed "
          f"{prod.layers[0]._committed_S_q}", flush=True)
    np.testing.assert_allclose(prod.bits_per_entry(), g[f"r{rank}_bpe"], rtol=1e-12)
    assert prod.layers[0]._committed_S_q == 384
    assert err.max().item() <= 2e-3 * max(scale, 1.0)
    assert agree == 1.0


def test_fp16_model_folds_the_window_write():
    """An fp16 model: each one-token step that commits nothing leaves its new
    key and value to the decode call, which stores them into the window.  The
    logits equal, bit for bit, those of the same cache with every row written
    by a copy first (the fold turned off); against the oracle-backed cache they
    agree to fp16 model arithmetic (the two attention outputs round to fp16
    apart and the difference propagates through the fp16 layers): max |logit
    delta| <= 5e-3 of the largest logit, argmax agreement >= 0.97."""
    from bmx_amd.cache import PackedStreamingLayer

    g = np.load(GOLD / "e2e_tiny_llama.npz")
    tokens = torch.from_numpy(g["r16_tokens"]).cuda()
    n = 140
    model = _tiny_model().half()
    specs = spec_pair("k2b_ph", rank=16)
    prod = PackedStreamingCache(model.config, *specs, recent_window=32)
    got = _run(prod, model, tokens, n)
    folded = prod.layers[0].n_rows_folded
    orig = PackedStreamingLayer._fold_ok
    PackedStreamingLayer._fold_ok = lambda self, k: False
    try:
        plain = PackedStreamingCache(model.config, *specs, recent_window=32)
        ref_plain = _run(plain, model, tokens, n)
    finally:
        PackedStreamingLayer._fold_ok = orig
    orc = OracleCache(model.config, *specs, recent_window=32)
    ref = _run(orc, model, tokens, n)
    err = (got - ref).abs().max().item()
    scale = ref.abs().max().item()
    agree = (got.argmax(1) == ref.argmax(1)).float().mean().item()
    print(f"fp16: rows folded {folded}, folded == copied {torch.equal(got, ref_plain)}; vs oracle-backed "
          f"max|err| {err:.3e} of {scale:.3f}, argmax agreement {agree:.4f}", flush=True)
    assert folded == n - 1 - 1 and plain.layers[0].n_rows_folded == 0   # one step commits
    assert torch.equal(got, ref_plain)
    assert torch.equal(prod.layers[0]._pool[:24], plain.layers[0]._pool[:24])
    assert err <= 5e-3 * max(scale, 1.0) and agree >= 0.97


def _spectral_pack_file(tmp_path, n_layers):
    from bmx_amd import spectral
    from tests.spectral_util import synthetic_pack

    layers = {}
    for i in range(n_layers):
        p25, p3 = synthetic_pack(2, 2.5, seed=40 + i), synthetic_pack(2, 3.0, seed=40 + i)
        layers[i] = (p25.enc, p25.dec, p25.lam, {2.5: p25.bits, 3.0: p3.bits})
    path = tmp_path / "packs.safetensors"
    spectral.save_packs(path, layers, (2.5, 3.0))
    return str(path)


@pytest.mark.parametrize("arm", ["k4ph_b2.5", "k4ph_b3", "k4ph_b2.5_dec8t4", "k4ph_b2.5_lq_dec8tl", "k4_b2.5",
                                 "k4_b2.5_lq"])
def test_spectral_cache_matches_oracle_backed_cache(tmp_path, arm):
    """The k4 recipe through the model: every commit through
    bmx_spectral_append, every step (decode and prefill) through
    bmx_spectral_dequant + SDPA, against the same host logic with the CPU
    oracle's codes (one layer: both caches encode the same keys, so the
    logits differ by the kernels' numerics only), teacher-forced.  The
    _dec8t4 arm decodes with the int8-roundtripped decoder and pays the
    int8 decoder charge in bits_per_entry; the _lq arm codes the Lloyd
    payload (both caches: its level indices, read back through the levels);
    k4_b is the reference's recipe, full-C turboquant_mse values (value bpe
    2 + 16 / C)."""
    from bmx_amd import spectral

    g = np.load(GOLD / "e2e_tiny_llama.npz")
    tokens = torch.from_numpy(g["r16_tokens"]).cuda()
    model = _tiny_model(n_layers=1)
    path = _spectral_pack_file(tmp_path, 1)
    specs = spec_pair(arm, pack_path=path)
    budget = specs[0].budget
    prod = PackedStreamingCache(model.config, *specs, recent_window=32)
    got = _run(prod, model, tokens, 140)
    orc = OracleCache(model.config, *specs, recent_window=32)
    ref = _run(orc, model, tokens, 140)
    err = (got - ref).abs().max(dim=1).values
    scale = ref.abs().max().item()
    agree = (got.argmax(1) == ref.argmax(1)).float().mean().item()
    lay = prod.layers[0]
    print(f"{arm}: logits max|err| {err.max():.3e} of max|logit| {scale:.3f}; argmax "
          f"agreement {agree:.4f}; committed {lay._committed_S_q}; c_pad {lay._dp.c_pad}", flush=True)
    assert lay._committed_S_q == 384 and lay._n_kpages == 6 and lay._n_pages == 24
    pack = spectral.load_packs(path, budget)[0]
    if "_dec8" in arm:
        assert lay._pack.dec_tier is not None and not torch.equal(lay._pack.dec, pack.dec)
    assert (lay._dp.lloyd_levels is not None) == ("_lq" in arm)
    bpe = spectral.payload_bpe(pack.bits)
    S = lay.get_seq_length()
    c_int8 = pack.c_int8(lay._pack.dec_tier) if "_dec8" in arm else 0
    charge = 8.0 * c_int8 / S + 16.0 * c_int8 / (S * 256) + 16.0 * (pack.c_used - c_int8) / S + 3.0 / S
    assert abs(prod.bits_per_entry()[0] - ((384 * bpe + (S - 384) * 16.0) / S + charge)) < 1e-9
    bpe_v = 2 + 16.0 / 256 if arm.startswith("k4_b") else 2 + 16.0 * 2 / 256
    assert abs(prod.bits_per_entry()[1] - (384 * bpe_v + (S - 384) * 16.0) / S) < 1e-9
    assert err.max().item() <= 2e-3 * max(scale, 1.0)
    assert agree == 1.0


@pytest.mark.parametrize("arm", ["k4ph_b2.5", "k4_b2.5"])
def test_spectral_short_prompt_decodes_across_first_commit(tmp_path, arm):
    """A 100-token prompt with a 32-token window: the first decode steps run
    before any commit (the window alone, no device pack built yet), the flush
    at 160 tokens commits the first codec page mid-stream.  Teacher forced
    against the oracle-backed cache, step by step; per-head and full-C
    values."""
    g = np.load(GOLD / "e2e_tiny_llama.npz")
    tokens = torch.from_numpy(g["r16_tokens"]).cuda()
    model = _tiny_model(n_layers=1)
    specs = spec_pair(arm, pack_path=_spectral_pack_file(tmp_path, 1))

    def run(cache):
        got = []
        with cache.attach(model), torch.no_grad():
            got.append(model(tokens[:, :100], past_key_values=cache, use_cache=True).logits[0, -1])
            for i in range(100, 200):
                got.append(model(tokens[:, i:i + 1], past_key_values=cache, use_cache=True).logits[0, -1])
        return torch.stack(got).double().cpu()

    prod = PackedStreamingCache(model.config, *specs, recent_window=32)
    got = run(prod)
    ref = run(OracleCache(model.config, *specs, recent_window=32))
    err = (got - ref).abs().max().item()
    scale = ref.abs().max().item()
    agree = (got.argmax(1) == ref.argmax(1)).float().mean().item()
    print(f"{arm} short prompt: logits max|err| {err:.3e} of {scale:.3f}, argmax agreement {agree:.4f}, "
          f"committed {prod.layers[0]._committed_S_q}", flush=True)
    assert prod.layers[0]._committed_S_q == 128
    assert err <= 2e-3 * max(scale, 1.0) and agree == 1.0


def test_spectral_generate_runs(tmp_path):
    """HF generate() on the k4 recipe, two layers."""
    model = _tiny_model()
    ids = torch.randint(0, 256, (1, 200), generator=torch.Generator().manual_seed(9)).cuda()
    cache = PackedStreamingCache(model.config, *spec_pair("k4ph_b2.5", pack_path=_spectral_pack_file(tmp_path, 2)),
                                 recent_window=32)
    with cache.attach(model), torch.no_grad():
        out = model.generate(ids, past_key_values=cache, max_new_tokens=40, min_new_tokens=40,
                             do_sample=False, pad_token_id=0)
    assert out.shape == (1, 240)
    assert cache.layers[1]._committed_S_q == 128 and cache.layers[1].get_seq_length() == 239


def test_generate_runs_on_the_packed_path():
    """HF generate() end to end: 40 greedy tokens after a 200-token prompt."""
    model = _tiny_model()
    ids = torch.randint(0, 256, (1, 200), generator=torch.Generator().manual_seed(9)).cuda()
    cache = PackedStreamingCache(model.config, *spec_pair("k2b_ph", rank=16), recent_window=32)
    with cache.attach(model), torch.no_grad():
        out = model.generate(ids, past_key_values=cache, max_new_tokens=40, min_new_tokens=40,
                             do_sample=False, pad_token_id=0)
    assert out.shape == (1, 240)
    assert cache.layers[0]._committed_S_q == 128 and cache.layers[0].get_seq_length() == 239


def _generate(cache, model, ids, n):
    with cache.attach(model), torch.no_grad():
        return model.generate(ids, past_key_values=cache, max_new_tokens=n, min_new_tokens=n, do_sample=False,
                              pad_token_id=0)


@pytest.mark.parametrize("recipe,seq,dtype", [("k2b_ph", 12, torch.float32), ("k2b_ph", 200, torch.float32),
                                              ("k2b_ph", 200, torch.float16), ("rtn_token_4b", 200, torch.float32),
                                              ("kivi", 200, torch.float32), ("k4_b2.5", 200, torch.float32),
                                              ("k4ph_b2.5_lq_dec8tl", 200, torch.float16)])
def test_packed_generate_matches_streaming(recipe, seq, dtype, tmp_path):
    """The reference's parity invariant (tests/test_packed_streaming.py:23-97):
    greedy generate through PackedStreamingCache equals generate through its
    StreamingQuantizedCache twin -- the same codes, read by the fused decode
    kernel on one side and dequantized once into a dense prefix for the model's
    own SDPA on the other.  A 12-token prompt (no commit before decode) and a
    200-token prompt (a codec page commits during prefill); the packed layer's
    resident window stays within recent_window + 128 rows."""
    from bmx_amd.cache import StreamingQuantizedCache
    from bmx_amd.specs import CacheCodecSpec

    if recipe == "rtn_token_4b":
        specs = (CacheCodecSpec(arm="rtn_token", bits=4, group=32, pre_rope=False),
                 CacheCodecSpec(arm="rtn_token", bits=4, group=32))
    elif recipe == "kivi":
        specs = spec_pair("kivi", group=64)
    elif recipe.startswith("k4"):
        specs = spec_pair(recipe, pack_path=_spectral_pack_file(tmp_path, 2))
    else:
        specs = spec_pair("k2b_ph", rank=16)
    model = _tiny_model().to(dtype)
    ids = torch.randint(0, 256, (1, seq), generator=torch.Generator().manual_seed(11)).cuda()
    ref_cache = StreamingQuantizedCache(model.config, *specs)
    ref = _generate(ref_cache, model, ids, 20)
    packed = PackedStreamingCache(model.config, *specs)
    out = _generate(packed, model, ids, 20)
    lay = packed.layers[0]
    print(f"{recipe} seq {seq} {dtype}: packed == streaming {torch.equal(out, ref)}; committed "
          f"{lay._committed_S_q} (twin {ref_cache.layers[0]._committed_S_q}); window {lay.keys.shape[2]} rows",
          flush=True)
    assert lay._committed_S_q == ref_cache.layers[0]._committed_S_q == (128 if seq == 200 else 0)
    assert lay.keys.shape[2] <= lay.recent_window + lay._page + 1
    assert ref_cache.reconstruct_layer(0)[0].shape[2] == seq + 19
    assert torch.equal(out, ref)


@pytest.mark.parametrize("ctx,N", [(16384, 32), (65536, 64)])
def test_packed_vs_streaming_logit_probe(ctx, N):
    """The reference's teacher-forced packed-vs-streaming logit probe
    (scripts/profile_decode_ab.py:316-439), at 16384 tokens for 32 steps and at
    the acceptance run's 65536 tokens for 64 steps: both caches prefilled on
    the same prompt, then N steps each fed the streaming cache's greedy token;
    per step the max |logit delta| is recorded and the flip gate applied (no
    flip with the streaming top-2 gap above that step's delta, at most N // 8
    flips).  Model: fp16, Llama geometry at reduced width (2 layers, 8 query /
    2 KV heads, d 128), key projections rank 8 plus 1% noise."""
    from transformers import LlamaConfig, LlamaForCausalLM

    from bmx_amd.cache import StreamingQuantizedCache
    from oracle import attention as A

    cfg = LlamaConfig(vocab_size=4096, hidden_size=1024, intermediate_size=2048, num_hidden_layers=2,
                      num_attention_heads=8, num_key_value_heads=2, head_dim=128,
                      max_position_embeddings=2 * ctx, rope_theta=500000.0, initializer_range=0.1)
    torch.manual_seed(0)
    model = LlamaForCausalLM(cfg).eval()
    gen = torch.Generator().manual_seed(4)
    with torch.no_grad():
        for layer in model.model.layers:
            W = layer.self_attn.k_proj.weight
            U, s_, Vh = torch.linalg.svd(W, full_matrices=False)
            W.copy_((U[:, :8] * s_[:8]) @ Vh[:8] + 0.01 * W.abs().mean() * torch.randn(W.shape, generator=gen))
    model = model.half().cuda()
    ids = torch.randint(10, 4086, (1, ctx), generator=torch.Generator().manual_seed(1234)).cuda()
    specs = spec_pair("k2b_ph", rank=16)
    caches = {"streaming": StreamingQuantizedCache(model.config, *specs),
              "packed": PackedStreamingCache(model.config, *specs)}
    logits = {}
    for kind, c in caches.items():
        with c.attach(model), torch.no_grad():
            logits[kind] = model(ids, past_key_values=c, use_cache=True, logits_to_keep=1).logits[:, -1].float()
        print(f"  {kind} cache prefilled with {ctx} tokens", flush=True)
    flips = hard = 0
    envelope = 0.0
    for step in range(N):
        tok = logits["streaming"].argmax(dim=-1, keepdim=True)
        pos = torch.tensor([ctx + step], device="cuda")
        for kind, c in caches.items():
            with c.attach(model), torch.no_grad():
                logits[kind] = model(tok, past_key_values=c, use_cache=True,
                                     cache_position=pos).logits[:, -1].float()
        f, h = A.argmax_flip(logits["packed"][0].cpu(), logits["streaming"][0].cpu())
        envelope = max(envelope, (logits["packed"] - logits["streaming"]).abs().max().item())
        flips, hard = flips + f, hard + h
        if step % 16 == 15:
            print(f"  step {step + 1}/{N}: flips {flips} (hard {hard}), envelope {envelope:.4f}", flush=True)
    print(f"logit probe ctx {ctx} N {N}: flips {flips} (hard {hard}), max_abs envelope {envelope:.4f}, "
          f"committed {caches['packed'].layers[0]._committed_S_q}", flush=True)
    assert caches["packed"].layers[0]._committed_S_q == caches["streaming"].layers[0]._committed_S_q
    assert hard == 0 and flips <= N // 8


def test_config5_qwen3_streaming_append_and_decode():
    """Config 5: Qwen3-8B attention geometry (8 KV heads, G 4, d 128, RoPE theta
    1e6), k2b rank 16, recent window 128.  An 8192-token seeded prefill is
    committed once, then 512 steps each append one token -- the flush schedule
    commits a codec page through bmx_k2b_append every 128 steps -- and
    decode-attend through bmx_k2b_decode.  The product layer and the
    oracle-backed layer run the same host logic on the same inputs: the pool
    holds the oracle's codes packed (bit-exact up to fp32 reduction-order ties,
    counted), every step is within the bars of the oracle, and a seeded
    4096-way readout passes the reference's argmax-flip gate (no flip against a
    top-2 gap wider than the step's delta, at most N // 8 near-tie flips)."""
    from transformers import Qwen3Config

    from bmx_amd import k2b, synth
    from bmx_amd.cache import PackedStreamingLayer
    from oracle import attention as A
    from oracle import layout as OL
    from oracle_cache import OracleLayer

    cfg = Qwen3Config(hidden_size=4096, intermediate_size=12288, num_attention_heads=32,
                      num_key_value_heads=8, head_dim=128, num_hidden_layers=36, rope_theta=1e6)
    k_spec, v_spec = spec_pair("k2b_ph", rank=16)
    h_kv, G, d, W = 8, 4, 128, 128
    n_pre, n_steps = 8192, 512
    prod = PackedStreamingLayer(k_spec, v_spec, cfg, recent_window=W)
    orac = OracleLayer(k_spec, v_spec, cfg, recent_window=W)
    gen = torch.Generator().manual_seed(55)
    N = n_pre + n_steps
    k_pre = synth.k2b_keys(h_kv, N, 16, gen)
    v = synth.values(h_kv, N, gen).half()
    cos, sin = A.rope_cos_sin(prod._inv_freq, torch.arange(N))
    k_post = A.apply_rope(k_pre.float(), cos, sin).half()
    W_read = torch.randn(h_kv * G * d, 4096, generator=gen)

    def feed(lo, hi):
        for lay, dev in ((prod, "cuda"), (orac, "cpu")):
            lay.stash_pre_rope(k_pre[:, lo:hi].transpose(0, 1).unsqueeze(0).to(dev))
            lay.update(k_post[:, lo:hi].unsqueeze(0).to(dev), v[:, lo:hi].unsqueeze(0).to(dev))

    feed(0, n_pre)
    worst, flips, hard = 0.0, 0, 0
    for i in range(n_steps):
        feed(n_pre + i, n_pre + i + 1)
        q = torch.randn(h_kv * G, 1, d, generator=gen)
        out = prod.attend(q.to("cuda"), d ** -0.5).double().cpu()
        ref = orac.attend(q, d ** -0.5).double()
        err = (out - ref).abs().max().item()
        rel = ((out - ref).norm() / ref.norm()).item()
        worst = max(worst, err)
        assert err <= 2e-3 and rel <= 1e-2, f"step {i}: max_abs {err:.3e} rel {rel:.3e}"
        f, hf = A.argmax_flip(out.float().reshape(-1) @ W_read, ref.float().reshape(-1) @ W_read)
        flips, hard = flips + f, hard + hf
    P = prod._committed_S_q
    assert P == orac._committed_S_q == ((N - W) // 128) * 128
    assert prod.bpe_k == orac.bpe_k and prod.bpe_v == orac.bpe_v
    oc = orac._oc
    us = torch.cat([kp["Us"] for kp, _, _ in oc.k_blocks]).numpy().astype(np.float16)
    res = torch.cat([kp["res_Q_int"] for kp, _, _ in oc.k_blocks], dim=1).numpy()
    sc = torch.cat([kp["res_scale"].squeeze(-1) for kp, _, _ in oc.k_blocks], dim=1)
    vidx = torch.cat([idx for (idx, _), _, _ in oc.v_blocks]).numpy()
    vn = torch.cat([n for (_, n), _, _ in oc.v_blocks]).numpy().astype(np.float16)
    want = OL.pack_pages(us, res, sc.numpy().astype(np.float16), vidx, vn, h_kv, 16)
    got = prod._pool[: P // k2b.PAGE_TOKENS].cpu().numpy()
    bad = int((got != want).sum())
    print(f"config 5 (Qwen3, rank 16, {n_pre} + {n_steps} steps): committed {P}, worst max_abs "
          f"{worst:.3e}, argmax flips {flips} (hard {hard}), page bytes differing {bad}/{want.size}",
          flush=True)
    assert hard == 0 and flips <= n_steps // 8
    assert bad <= want.size * 1e-4


@pytest.mark.parametrize("recipe", ["rtn_token_4b", "kivi"])
def test_rtn_layer_streaming_decode_and_prefill(recipe):
    """The RTN pairs through the cache layer -- the reference's fused pair
    (rtn_token keys post-RoPE and values, 4 bits, groups of 32) and the kivi
    recipe (rtn_channel keys, 2 bits, groups of 64): a 1000-token prefill
    attended causally through bmx_rtn_dequant + SDPA, then 300 one-token steps,
    each committing on the 128-token grid through bmx_rtn_append and decoding
    through bmx_rtn_decode, against the RTN oracle fed the same committed pages
    and windows."""
    import torch.nn.functional as F
    from transformers import LlamaConfig

    from bmx_amd.cache import PackedStreamingLayer
    from bmx_amd.specs import CacheCodecSpec
    from oracle import attention as A

    cfg = LlamaConfig(hidden_size=4096, num_attention_heads=32, num_key_value_heads=8, head_dim=128,
                      num_hidden_layers=32, rope_theta=500000.0)
    if recipe == "kivi":
        k_spec, v_spec = spec_pair("kivi", group=64)
    else:
        k_spec = CacheCodecSpec(arm="rtn_token", bits=4, group=32, pre_rope=False)
        v_spec = CacheCodecSpec(arm="rtn_token", bits=4, group=32)
    h_kv, G, d, W = 8, 4, 128, 128
    lay = PackedStreamingLayer(k_spec, v_spec, cfg, recent_window=W)
    gen = torch.Generator().manual_seed(77)
    n_pre, n_steps = 1000, 300
    N = n_pre + n_steps
    k = torch.randn(h_kv, N, d, generator=gen)
    k[:, :, [3, 40, 77, 101]] *= 10.0
    k = k.half()
    v = torch.randn(h_kv, N, d, generator=gen).half()
    oc = A.RtnOracleCache(h_kv, k_bits=k_spec.bits, v_bits=v_spec.bits, k_group=k_spec.group,
                          v_group=v_spec.group, k_arm=1 if k_spec.arm == "rtn_channel" else 0)

    def sync_oracle():
        while oc.n_tokens < lay._committed_S_q:
            s = oc.n_tokens
            oc.commit(k[:, s:s + 128], v[:, s:s + 128])

    lay.update(k[:, :n_pre].unsqueeze(0).cuda(), v[:, :n_pre].unsqueeze(0).cuda())
    sync_oracle()
    P = lay._committed_S_q
    assert P == ((n_pre - W) // 128) * 128
    q = torch.randn(h_kv * G, n_pre, d, generator=gen)
    out = lay.attend(q.cuda(), d ** -0.5, is_causal=True).float().cpu()
    Kd, Vd = oc.dense_kv()
    Kx = torch.cat([Kd, k[:, P:n_pre].float()], 1).repeat_interleave(G, 0)
    Vx = torch.cat([Vd, v[:, P:n_pre].float()], 1).repeat_interleave(G, 0)
    ref = F.scaled_dot_product_attention(q.unsqueeze(0), Kx.unsqueeze(0), Vx.unsqueeze(0), is_causal=True,
                                         scale=d ** -0.5).squeeze(0)
    err = (out - ref).abs().max().item()
    print(f"{recipe} prefill {n_pre} tokens (causal): max_abs {err:.3e}", flush=True)
    assert err <= 2e-3
    worst = 0.0
    for i in range(n_steps):
        t = n_pre + i
        lay.update(k[:, t:t + 1].unsqueeze(0).cuda(), v[:, t:t + 1].unsqueeze(0).cuda())
        sync_oracle()
        P = lay._committed_S_q
        qs = torch.randn(h_kv * G, 1, d, generator=gen)
        o = lay.attend(qs.cuda(), d ** -0.5).double().cpu()
        r = A.rtn_naive_attention(qs, oc, k[:, P:t + 1], v[:, P:t + 1], G, d ** -0.5).double()
        e = (o - r).abs().max().item()
        worst = max(worst, e)
        assert e <= 2e-3 and ((o - r).norm() / r.norm()).item() <= 1e-2, f"step {i}: {e:.3e}"
    bpe_page = k_spec.bits + 16.0 / k_spec.group
    assert lay.bpe_k == pytest.approx((bpe_page * P + 16 * (N - P)) / N)
    print(f"{recipe} layer: {n_steps} decode steps, committed {P}, worst max_abs {worst:.3e}, "
          f"bpe_k {lay.bpe_k:.4f}", flush=True)


def _explicit_attention(q, K, V, G, scale, offset):
    """fp32 attention of q (H, n_q, d) over K, V (h_kv, n_kv, d): query i sits at
    position offset + i and sees keys 0 .. offset + i."""
    n_q, n_kv = q.shape[1], K.shape[1]
    Kx, Vx = K.float().repeat_interleave(G, 0), V.float().repeat_interleave(G, 0)
    s = (q.float() @ Kx.transpose(1, 2).contiguous()) * scale
    i = torch.arange(n_q)[:, None]
    j = torch.arange(n_kv)[None, :]
    s = s.masked_fill(~(j <= i + offset), float("-inf"))
    return torch.softmax(s, dim=-1) @ Vx


@pytest.mark.parametrize("path,dtype", [("k2b", torch.float16), ("k2b", torch.float32),
                                        ("rtn", torch.float16)])
def test_two_block_prefill_mask_contract(path, dtype):
    """The cached two-block prefill (test_packed_streaming.py:100-153): a first
    forward of 600 tokens, then a second of 300 -- queries at positions
    600..899 over 900 keys, fewer queries than keys, so a top-left causal mask
    would be wrong.  The second block through the layer (committed pages
    dequantized by the page kernel in the model dtype, k2b keys rotated with
    the fp16 RoPE tables in the same pass, one SDPA over grouped heads), with
    no mask from the model and with the model's own boolean mask, equals an
    explicit bottom-right-masked fp32 attention over the oracle's dequantized
    pages and the fp16 window; the top-left result is far from it."""
    from transformers import LlamaConfig

    from bmx_amd import synth
    from bmx_amd.cache import PackedStreamingLayer
    from bmx_amd.specs import CacheCodecSpec
    from oracle import attention as A
    from oracle_cache import OracleLayer

    cfg = LlamaConfig(hidden_size=4096, num_attention_heads=32, num_key_value_heads=8, head_dim=128,
                      num_hidden_layers=32, rope_theta=500000.0)
    h_kv, G, d, W = 8, 4, 128, 128
    n1, n2 = 600, 300
    N = n1 + n2
    gen = torch.Generator().manual_seed(91)
    if path == "k2b":
        k_spec, v_spec = spec_pair("k2b_ph", rank=16)
        prod = PackedStreamingLayer(k_spec, v_spec, cfg, recent_window=W)
        orac = OracleLayer(k_spec, v_spec, cfg, recent_window=W)
        orac.v_fp16 = True
        k_pre = synth.k2b_keys(h_kv, N, 16, gen)
        cos, sin = A.rope_cos_sin(prod._inv_freq, torch.arange(N))
        k_post = A.apply_rope(k_pre.float(), cos, sin).half()
    else:
        k_spec = CacheCodecSpec(arm="rtn_token", bits=4, group=32, pre_rope=False)
        v_spec = CacheCodecSpec(arm="rtn_token", bits=4, group=32)
        prod = PackedStreamingLayer(k_spec, v_spec, cfg, recent_window=W)
        oc = A.RtnOracleCache(h_kv, k_bits=4, v_bits=4, k_group=32, v_group=32)
        k_post = torch.randn(h_kv, N, d, generator=gen).half()
    v = synth.values(h_kv, N, gen).half()

    def feed(lo, hi):
        if path == "k2b":
            for lay, dev in ((prod, "cuda"), (orac, "cpu")):
                lay.stash_pre_rope(k_pre[:, lo:hi].transpose(0, 1).unsqueeze(0).to(dev))
                lay.update(k_post[:, lo:hi].unsqueeze(0).to(dev), v[:, lo:hi].unsqueeze(0).to(dev))
        else:
            prod.update(k_post[:, lo:hi].unsqueeze(0).cuda(), v[:, lo:hi].unsqueeze(0).cuda())
            while oc.n_tokens < prod._committed_S_q:
                s = oc.n_tokens
                oc.commit(k_post[:, s:s + 128], v[:, s:s + 128])

    feed(0, n1)
    feed(n1, N)
    P = prod._committed_S_q
    assert P == ((N - W) // 128) * 128 and prod.get_seq_length() == N
    if path == "k2b":
        K, V = orac._kv(torch.float32)
    else:
        Kd, Vd = oc.dense_kv()
        K, V = torch.cat([Kd, k_post[:, P:].float()], 1), torch.cat([Vd, v[:, P:].float()], 1)
    q = torch.randn(h_kv * G, n2, d, generator=gen).to(dtype)
    ref = _explicit_attention(q, K, V, G, d ** -0.5, n1)
    wrong = _explicit_attention(q, K, V, G, d ** -0.5, 0)
    mask = (torch.arange(N)[None, :] <= torch.arange(n2)[:, None] + n1)[None, None].cuda()
    tol = 2e-3 if dtype == torch.float32 else 4e-3
    for what, m in (("no mask", None), ("model mask", mask)):
        out = prod.attend(q.cuda(), d ** -0.5, is_causal=True, attention_mask=m)
        assert out.dtype == dtype
        err = (out.float().cpu() - ref).abs().max().item()
        off = (out.float().cpu() - wrong).abs().max().item()
        print(f"{path} {dtype} two-block prefill ({what}): max_abs {err:.3e} vs the bottom-right "
              f"oracle, {off:.3e} vs top-left", flush=True)
        assert err <= tol and off > 50 * tol


def test_two_block_prefill_through_the_model():
    """HF threads its mask into the packed attention: the tiny Llama's cached
    two-block prefill (200 tokens, then 200 more) through the product cache
    and through the oracle-backed cache agree at every position of the second
    block."""
    g = np.load(GOLD / "e2e_tiny_llama.npz")
    tokens = torch.from_numpy(g["r16_tokens"]).cuda()
    model = _tiny_model()

    def run(cache):
        with cache.attach(model), torch.no_grad():
            model(tokens[:, :200], past_key_values=cache, use_cache=True)
            return model(tokens[:, 200:400], past_key_values=cache, use_cache=True).logits[0].double().cpu()

    got = run(PackedStreamingCache(model.config, *spec_pair("k2b_ph", rank=16), recent_window=32))
    ref = run(OracleCache(model.config, *spec_pair("k2b_ph", rank=16), recent_window=32))
    err = (got - ref).abs().max().item()
    scale = ref.abs().max().item()
    print(f"tiny Llama two-block prefill: logits max|err| {err:.3e} of max|logit| {scale:.3f}", flush=True)
    assert err <= 2e-3 * max(scale, 1.0)
    assert bool((got.argmax(-1) == ref.argmax(-1)).all())


def test_bf16_window_keeps_the_model_rows():
    """A bf16 model's recent window stays in bf16 (the reference keeps the
    tail in the model dtype, packed_streaming.py:849, and its decode reads it
    as fp32, triton_dequant_attention.py:353): window rows beyond fp16's range
    reach the prefill's dense keys and the decode kernels as the model made
    them.  600 tokens whose last 100 key and value rows are scaled by 2^17
    (|x| up to ~6e5), a causal prefill over them, then two decode steps with
    large newest rows (each folded into the decode call), all against explicit
    fp32 attention over the oracle's pages and the bf16 rows."""
    from transformers import LlamaConfig

    from bmx_amd import synth
    from bmx_amd.cache import PackedStreamingLayer
    from oracle import attention as A
    from oracle_cache import OracleLayer

    cfg = LlamaConfig(hidden_size=4096, num_attention_heads=32, num_key_value_heads=8, head_dim=128,
                      num_hidden_layers=32, rope_theta=500000.0)
    h_kv, G, d, W, N = 8, 4, 128, 128, 600
    gen = torch.Generator().manual_seed(92)
    k_spec, v_spec = spec_pair("k2b_ph", rank=16)
    prod = PackedStreamingLayer(k_spec, v_spec, cfg, recent_window=W)
    prod.packed_reader = True   # as attach() sets it: the decode call takes the newest row
    orac = OracleLayer(k_spec, v_spec, cfg, recent_window=W)
    orac.v_fp16 = True
    k_pre = synth.k2b_keys(h_kv, N + 2, 16, gen)
    cos, sin = A.rope_cos_sin(prod._inv_freq, torch.arange(N + 2))
    k_post = A.apply_rope(k_pre.float(), cos, sin)
    v = synth.values(h_kv, N + 2, gen).float()
    k_post[:, N - 100:] *= 2.0 ** 17
    v[:, N - 100:] *= 2.0 ** 17
    k_post, v = k_post.bfloat16(), v.bfloat16()
    assert k_post.float().abs().max() > 65504 and v.float().abs().max() > 65504

    def feed(lo, hi):
        for lay, dev in ((prod, "cuda"), (orac, "cpu")):
            lay.stash_pre_rope(k_pre[:, lo:hi].transpose(0, 1).unsqueeze(0).to(dev))
            lay.update(k_post[:, lo:hi].unsqueeze(0).to(dev), v[:, lo:hi].unsqueeze(0).to(dev))

    feed(0, N)
    P = prod._committed_S_q
    assert P > 0 and prod._win_k.dtype == torch.bfloat16
    q = (1e-5 * torch.randn(h_kv * G, N, d, generator=gen)).bfloat16()
    K, V = orac._kv(torch.float32)
    assert torch.equal(K[:, P:], k_post[:, P:N].float()) and torch.equal(V[:, P:], v[:, P:N].float())
    ref = _explicit_attention(q, K, V, G, d ** -0.5, 0)
    out = prod.attend(q.cuda(), d ** -0.5, is_causal=True)
    torch.cuda.synchronize()
    err = (out.float().cpu() - ref).abs().max().item()
    top = ref.abs().max().item()
    print(f"bf16 prefill over rows up to {k_post.float().abs().max().item():.3g}: max_abs {err:.3e} "
          f"(max |out| {top:.3g})", flush=True)
    assert torch.isfinite(out).all() and err <= 1e-2 * top
    for step in range(2):
        feed(N + step, N + step + 1)
        K, V = orac._kv(torch.float32)
        qd = (1e-5 * torch.randn(h_kv * G, 1, d, generator=gen)).bfloat16()
        ref = _explicit_attention(qd, K, V, G, d ** -0.5, N + step)
        out = prod.attend(qd.cuda(), d ** -0.5)
        torch.cuda.synchronize()
        err = (out.float().cpu() - ref).abs().max().item()
        top = ref.abs().max().item()
        print(f"bf16 decode step {step}: max_abs {err:.3e} (max |out| {top:.3g}), rows folded "
              f"{prod.n_rows_folded}", flush=True)
        assert out.dtype == torch.bfloat16 and torch.isfinite(out).all() and err <= 1e-2 * top
    assert prod.n_rows_folded == 2
    assert torch.equal(prod.window()[0].cpu(), orac.window()[0])


def _tiny_model_d(head_dim, n_heads, n_kv, n_layers=2):
    """_tiny_model at another head_dim: key projections rank 8 plus 1% noise
    (with full-rank random keys the fp16 storage of the key scales and the fp16
    key operand of the score product, in the recipe's kernels as in these,
    move the random model's logits by ~0.1 against the fp32 oracle)."""
    from transformers import LlamaConfig, LlamaForCausalLM

    cfg = LlamaConfig(vocab_size=256, hidden_size=256, intermediate_size=512, num_hidden_layers=n_layers,
                      num_attention_heads=n_heads, num_key_value_heads=n_kv, head_dim=head_dim,
                      max_position_embeddings=4096, rope_theta=500000.0, initializer_range=0.1)
    torch.manual_seed(0)
    model = LlamaForCausalLM(cfg).eval()
    gen = torch.Generator().manual_seed(3)
    with torch.no_grad():
        for layer in model.model.layers:
            W = layer.self_attn.k_proj.weight
            U, s, Vh = torch.linalg.svd(W, full_matrices=False)
            W.copy_((U[:, :8] * s[:8]) @ Vh[:8] + 0.01 * W.abs().mean() * torch.randn(W.shape, generator=gen))
    return model.to("cuda")


@pytest.mark.parametrize("head_dim,n_heads,rank,group,dtype", [
    (64, 8, 16, 32, torch.float32), (64, 8, 16, 32, torch.float16), (128, 4, 64, 64, torch.float32),
    (32, 8, 16, 16, torch.float32)])
def test_general_geometry_cache_matches_oracle_backed_cache(head_dim, n_heads, rank, group, dtype):
    """Models off the recipe's page through the product cache (the general
    page's append, decode and prefill kernels): head_dim 64 with group 32 (the
    reference's k2b test geometry; the oracle-backed cache reproduces the
    reference's own run of this geometry on the CPU), rank 64 at head_dim 128
    (spec_pair("k2b_ph", rank=64)), head_dim 32 with group 16.  140
    teacher-forced steps: logits within 2e-3 of the largest (1e-2 for the fp16
    model, whose own arithmetic rounds every layer to fp16; the newest rows go
    through the decode call there), and the reference's flip gate on the greedy
    choices (no flip whose top-2 gap exceeds the step's logit delta, at most
    N // 8 flips; scripts/profile_decode_ab.py:325-343)."""
    from oracle import attention as A

    g = np.load(GOLD / "e2e_tiny_llama_d64.npz")
    tokens = torch.from_numpy(g["tokens"]).cuda()
    n = 140
    model = _tiny_model_d(head_dim, n_heads, 2).to(dtype)
    specs = spec_pair("k2b_ph", rank=rank, group=group)
    prod = PackedStreamingCache(model.config, *specs, recent_window=32)
    got = _run(prod, model, tokens, n)
    orc = OracleCache(model.config, *specs, recent_window=32)
    ref = _run(orc, model, tokens, n)
    err = (got - ref).abs().max(dim=1).values
    scale = ref.abs().max().item()
    gate = [A.argmax_flip(got[i], ref[i]) for i in range(n)]
    flips, hard = sum(f for f, _ in gate), sum(h for _, h in gate)
    folded = prod.layers[0].n_rows_folded
    print(f"head_dim {head_dim} rank {rank} group {group} {dtype}: product vs oracle-backed cache, logits "
          f"max|err| {err.max():.3e} of {scale:.3f}; flips {flips} (hard {hard}); rows folded {folded}; "
          f"committed {prod.layers[0]._committed_S_q}", flush=True)
    assert prod.layers[0]._committed_S_q == 384
    assert (folded > 100) == (dtype == torch.float16)
    np.testing.assert_allclose(prod.bits_per_entry(), orc.bits_per_entry(), rtol=1e-12)
    assert err.max().item() <= (2e-3 if dtype == torch.float32 else 1e-2) * max(scale, 1.0)
    assert hard == 0 and flips <= n // 8


def test_rank_64_generate_runs():
    """spec_pair("k2b_ph", rank=64) under HF generate on the packed path, fp16."""
    model = _tiny_model().half()
    ids = torch.randint(0, 256, (1, 300), generator=torch.Generator().manual_seed(12)).cuda()
    cache = PackedStreamingCache(model.config, *spec_pair("k2b_ph", rank=64), recent_window=32)
    with cache.attach(model), torch.no_grad():
        out = model.generate(ids, past_key_values=cache, max_new_tokens=40, min_new_tokens=40, do_sample=False,
                             pad_token_id=0)
    assert out.shape == (1, 340) and cache.layers[0]._committed_S_q >= 256
    assert cache.layers[0]._page_bytes() == k2b.page_bytes(2, 64)

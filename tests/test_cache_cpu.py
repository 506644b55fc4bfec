"""Host side of the PackedStreamingCache mirror (no GPU): recipe specs, the
bits-per-entry accounting against the reference's own end-to-end fixture,
attach/detach bookkeeping, and the fail-loud rule (no CPU attention path)."""

from pathlib import Path

import numpy as np
import pytest
import torch

from bmx_amd import codecs as K
from bmx_amd import k2b as K2B
from bmx_amd.cache import ATTN_NAME, PackedStreamingCache, resolve_decoder_layers
from bmx_amd.specs import CacheCodecSpec, check_k2b, spec_pair

GOLD = Path(__file__).parent / "golden"


def tiny_config():
    from transformers import LlamaConfig

    return LlamaConfig(vocab_size=256, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                       num_attention_heads=4, num_key_value_heads=2, head_dim=128,
                       max_position_embeddings=4096, rope_theta=500000.0, initializer_range=0.1)


def test_spec_pair_k2b_ph_matches_reference_recipe():
    """recipes.py:31-42: K lowrank_rtn_channel 3b group 64 pre-RoPE, V
    turboquant_mse_perhead 2b."""
    k, v = spec_pair("k2b_ph", rank=32)
    assert (k.arm, k.bits, k.rank, k.group, k.pre_rope) == ("lowrank_rtn_channel", 3, 32, 64, True)
    assert (v.arm, v.bits) == ("turboquant_mse_perhead", 2)
    check_k2b(k, v)


@pytest.mark.parametrize("bad", [dict(rank=8), dict(rank=48), dict(bits=5), dict(bits=1), dict(group=8),
                                 dict(group=256), dict(pre_rope=False)])
def test_unsupported_k_specs_raise(bad):
    k, v = spec_pair("k2b_ph", rank=16)
    k = CacheCodecSpec(**{**k.__dict__, **bad})
    with pytest.raises(NotImplementedError):
        check_k2b(k, v)


@pytest.mark.parametrize("good", [dict(rank=64), dict(rank=128), dict(bits=2), dict(bits=4), dict(group=32),
                                  dict(group=16), dict(group=128)])
def test_general_k_specs_taken(good):
    """The fused path's geometry (packed_streaming.py:957-975): rank, residual
    group and key bits beyond the recipe's default run on the general page."""
    k, v = spec_pair("k2b_ph", rank=16)
    check_k2b(CacheCodecSpec(**{**k.__dict__, **good}), v)


@pytest.mark.parametrize("head_dim,ok", [(64, True), (32, True), (96, False), (256, False)])
def test_k2b_layer_head_dims(head_dim, ok):
    from transformers import LlamaConfig

    from bmx_amd.cache import PackedStreamingLayer

    cfg = LlamaConfig(vocab_size=256, hidden_size=512, intermediate_size=512, num_hidden_layers=1,
                      num_attention_heads=8, num_key_value_heads=2, head_dim=head_dim)
    k, v = spec_pair("k2b_ph", rank=16, group=32)
    if ok:
        lay = PackedStreamingLayer(k, v, cfg)
        assert lay._consts.head_dim == head_dim and lay._kgeom == dict(group=32, k_bits=3)
        assert lay._page_bytes() == K2B.page_bytes(2, 16, head_dim=head_dim, group=32)
    else:
        with pytest.raises(NotImplementedError, match="head_dim"):
            PackedStreamingLayer(k, v, cfg)


def test_other_recipes_raise():
    with pytest.raises(NotImplementedError, match="k2b_ph"):
        spec_pair("turboquant_mse")


def test_kivi_recipe_and_rtn_pairs():
    """kivi = rtn_channel keys with rtn_token values, 2 bits (recipes.py:173-177);
    the RTN kernels take it and the reference's fused rtn_token pair; anything
    outside their bit widths and groups raises."""
    from bmx_amd.specs import packed_path

    k, v = spec_pair("kivi", group=64)
    assert (k.arm, k.bits, k.group, v.arm, v.bits, v.group) == ("rtn_channel", 2, 64, "rtn_token", 2, 64)
    assert packed_path(k, v) == "rtn"
    tok = CacheCodecSpec(arm="rtn_token", bits=4, group=32)
    assert packed_path(tok, tok) == "rtn"
    with pytest.raises(NotImplementedError):
        packed_path(CacheCodecSpec(arm="rtn_token", bits=8, group=32), tok)
    with pytest.raises(NotImplementedError):
        packed_path(CacheCodecSpec(arm="rtn_token", bits=4, group=8), tok)
    with pytest.raises(NotImplementedError):
        packed_path(CacheCodecSpec(arm="rtn_token", bits=4, group=32, pre_rope=True), tok)


@pytest.mark.parametrize("rank", [16, 32])
def test_blended_bpe_reproduces_reference_fixture(rank):
    """The reference's tiny-Llama run ends with 439 cached tokens (300 prompt +
    139 fed back), 384 committed in 128-token pages and 55 fp16; its
    bits_per_entry() must equal the per-page codec bpe blended with 16-bit tail
    entries (packed_streaming.py:612-619, 713-725)."""
    g = np.load(GOLD / "e2e_tiny_llama.npz")
    C = 2 * 128
    S = 300 + 139
    P = K.compute_flush_schedule(S, 32, 128)
    assert P == 384
    bk = (P * K.bpe_k(rank, C) + (S - P) * 16.0) / S
    bv = (P * K.bpe_v(2, C) + (S - P) * 16.0) / S
    np.testing.assert_allclose([bk, bv], g[f"r{rank}_bpe"], rtol=1e-12)


def test_attach_detach_and_no_cpu_path():
    from transformers import LlamaForCausalLM

    torch.manual_seed(0)
    model = LlamaForCausalLM(tiny_config()).eval()
    saved = model.config._attn_implementation
    cache = PackedStreamingCache(model.config, *spec_pair("k2b_ph", rank=16), recent_window=32)
    with cache.attach(model):
        assert model.config._attn_implementation == ATTN_NAME
        assert len(cache.layers) == 2 and len(cache._handles) == 2
        assert all(hasattr(l.self_attn, "_packed_layer") for l in resolve_decoder_layers(model))
        ids = torch.randint(0, 256, (1, 40))
        with pytest.raises(RuntimeError, match="HIP device"):
            with torch.no_grad():
                model(ids, past_key_values=cache, use_cache=True)
    assert model.config._attn_implementation == saved
    assert cache._handles == []
    assert not any(hasattr(l.self_attn, "_packed_layer") for l in resolve_decoder_layers(model))


def test_memory_report_uses_bpe():
    cache = PackedStreamingCache(tiny_config(), *spec_pair("k2b_ph", rank=16))
    rep = cache.memory_report(1000)   # nothing committed: 16 bits per entry both sides
    assert rep["fp16_bytes"] == 2 * 2 * 2 * 1000 * 128 * 2
    assert rep["compression"] == pytest.approx(1.0)


@pytest.mark.parametrize("rank", [16, 32])
def test_host_logic_reproduces_reference_run(rank):
    """The product cache's host logic (flush schedule, pre-RoPE stash and slab
    pruning, fp16 RoPE tables, prefill/decode split, bits-per-entry) with the
    CPU oracle standing in for the three kernels, teacher-forced through the
    reference's own 440-token run of the tiny Llama: every step's logits match
    the reference's (to fp32 reduction order: the reference decodes with a
    chunked online softmax, the stand-in with one softmax; 5e-4 against logits
    of magnitude ~7), every greedy choice agrees, and bits_per_entry() is equal."""
    import sys

    sys.path.insert(0, str(Path(__file__).parent))
    from oracle_cache import OracleCache
    from transformers import LlamaForCausalLM

    g = np.load(GOLD / "e2e_tiny_llama.npz")
    tokens = torch.from_numpy(g[f"r{rank}_tokens"])
    ref = torch.from_numpy(g[f"r{rank}_logits"]).double()
    torch.manual_seed(0)
    model = LlamaForCausalLM(tiny_config()).eval()
    cache = OracleCache(model.config, *spec_pair("k2b_ph", rank=rank), recent_window=32)
    got = []
    with cache.attach(model), torch.no_grad():
        got.append(model(tokens[:, :300], past_key_values=cache, use_cache=True).logits[0, -1])
        for i in range(1, ref.shape[0]):
            out = model(tokens[:, 300 + i - 1: 300 + i], past_key_values=cache, use_cache=True)
            got.append(out.logits[0, -1])
    got = torch.stack(got).double()
    err = (got - ref).abs().max().item()
    print(f"r{rank}: oracle-backed cache vs reference run, logits max|err| {err:.3e}")
    assert err <= 5e-4
    assert bool((got.argmax(1) == ref.argmax(1)).all())
    np.testing.assert_allclose(cache.bits_per_entry(), g[f"r{rank}_bpe"], rtol=1e-12)


def test_host_logic_reproduces_reference_run_head_dim_64():
    """The same teacher-forced check at a geometry off the recipe's page: a
    tiny Llama with head_dim 64 (8 query / 2 KV heads) and k2b_ph at rank 16,
    residual group 32 -- the reference's fused-kernel test geometry -- against
    the reference's own 440-token run (tests/golden/e2e_tiny_llama_d64.npz)."""
    import sys

    sys.path.insert(0, str(Path(__file__).parent))
    from oracle_cache import OracleCache
    from transformers import LlamaConfig, LlamaForCausalLM

    g = np.load(GOLD / "e2e_tiny_llama_d64.npz")
    tokens = torch.from_numpy(g["tokens"])
    ref = torch.from_numpy(g["logits"]).double()
    cfg = LlamaConfig(vocab_size=256, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                      num_attention_heads=8, num_key_value_heads=2, head_dim=64,
                      max_position_embeddings=4096, rope_theta=500000.0, initializer_range=0.1)
    torch.manual_seed(0)
    model = LlamaForCausalLM(cfg).eval()
    cache = OracleCache(model.config, *spec_pair("k2b_ph", rank=16, group=32), recent_window=32)
    got = []
    with cache.attach(model), torch.no_grad():
        got.append(model(tokens[:, :300], past_key_values=cache, use_cache=True).logits[0, -1])
        for i in range(1, ref.shape[0]):
            out = model(tokens[:, 300 + i - 1: 300 + i], past_key_values=cache, use_cache=True)
            got.append(out.logits[0, -1])
    got = torch.stack(got).double()
    err = (got - ref).abs().max().item()
    print(f"head_dim 64, group 32: oracle-backed cache vs reference run, logits max|err| {err:.3e}")
    assert err <= 5e-4
    assert bool((got.argmax(1) == ref.argmax(1)).all())
    np.testing.assert_allclose(cache.bits_per_entry(), g["bpe"], rtol=1e-12)


def test_lower_right_causal_mask_detection():
    """The prefill's bias choice: a boolean (1, 1, n_q, n_kv) mask equal to the
    causal mask of the last n_q positions is recognised (and the answer kept
    for that tensor while it is unmodified); a padded, top-left, float or
    mis-shaped mask is not."""
    from bmx_amd.cache import _is_lower_right_causal

    n_q, n_kv = 5, 12
    i = torch.arange(n_q)[:, None]
    j = torch.arange(n_kv)[None, :]
    m = (j <= i + (n_kv - n_q))[None, None].clone()
    assert _is_lower_right_causal(m, n_q, n_kv)
    assert _is_lower_right_causal(m, n_q, n_kv)          # kept for the same tensor
    m[0, 0, 2, 0] = False                                 # in place: the version moves, asked again
    assert not _is_lower_right_causal(m, n_q, n_kv)
    assert not _is_lower_right_causal((j <= i)[None, None], n_q, n_kv)   # top-left causal
    assert not _is_lower_right_causal((j <= i + (n_kv - n_q))[None, None].float(), n_q, n_kv)
    assert not _is_lower_right_causal((j <= i + (n_kv - n_q))[None, None].expand(2, 1, n_q, n_kv), n_q, n_kv)
    assert not _is_lower_right_causal(None, n_q, n_kv)


def test_attach_marks_the_packed_reader():
    """Only an attached layer leaves a step's newest row to the decode call:
    attach() marks its layers as read by the packed attention, detach() clears
    the mark (a detached layer's update() writes every row itself)."""
    from transformers import LlamaForCausalLM

    model = LlamaForCausalLM(tiny_config()).eval()
    cache = PackedStreamingCache(model.config, *spec_pair("k2b_ph", rank=16), recent_window=32)
    cache.attach(model)
    assert all(layer.packed_reader for layer in cache.layers)
    cache.detach()
    assert not any(layer.packed_reader for layer in cache.layers)


def _window_layer(n_rows, recent_window=64):
    """A k2b layer on the CPU fed n_rows tokens (fewer than its first commit
    needs: the rows stay in the window, no kernel runs)."""
    from bmx_amd.cache import PackedStreamingLayer

    cfg = tiny_config()
    layer = PackedStreamingLayer(*spec_pair("k2b_ph", rank=16), cfg, recent_window=recent_window)
    gen = torch.Generator().manual_seed(3)
    k = torch.randn(1, 2, n_rows, 128, generator=gen)
    v = torch.randn(1, 2, n_rows, 128, generator=gen)
    layer.stash_pre_rope(torch.randn(1, n_rows, 2 * 128, generator=gen))
    layer.update(k, v)
    return layer, k, v


def test_crop_drops_window_rows_and_their_stash():
    """DynamicLayer.crop semantics on the packed layer: -n drops the newest n
    rows, a positive count is the length to keep; the window length, the
    returned keys/values, the bits-per-entry and the pre-RoPE stash follow."""
    layer, k, v = _window_layer(100)
    assert layer.get_seq_length() == 100 and layer._committed_S_q == 0
    layer.crop(-10)
    assert layer.get_seq_length() == 90 and layer._k_pre_rows == 90
    assert torch.equal(layer.keys, k[:, :, :90]) and torch.equal(layer.values, v[:, :, :90])
    layer.crop(80)
    assert layer.get_seq_length() == 80 and layer._k_pre_rows == 80 and layer.keys.shape[2] == 80
    layer.crop(200)   # longer than the cache: nothing to drop
    layer.crop(0)
    assert layer.get_seq_length() == 80
    # new rows continue from the cropped length
    k2 = torch.randn(1, 2, 5, 128)
    layer.update(k2, k2)
    assert layer.get_seq_length() == 85 and torch.equal(layer.keys[:, :, 80:], k2)


def test_crop_into_committed_pages_and_batch_mutators_refused():
    layer, _, _ = _window_layer(100)
    layer._committed_S_q, layer._T = 128, 100   # as if a codec page had committed
    with pytest.raises(NotImplementedError, match="committed"):
        layer.crop(-101)
    for call in (lambda: layer.reorder_cache(torch.tensor([1, 0])),
                 lambda: layer.batch_select_indices(torch.tensor([0, 1])),
                 lambda: layer.batch_repeat_interleave(2)):
        with pytest.raises(NotImplementedError, match="batch size 1"):
            call()
    layer.reorder_cache(torch.tensor([0]))   # the one sequence in place: nothing to do
    layer.batch_select_indices(torch.tensor([0]))
    layer.batch_repeat_interleave(1)
    with pytest.raises(NotImplementedError, match="device"):
        layer.offload()


def test_reset_forgets_every_token():
    layer, _, _ = _window_layer(40)
    layer.packed_reader = True
    layer.reset()
    assert layer.get_seq_length() == 0 and layer._k_pre_rows == 0 and layer._win_k is None
    assert layer.packed_reader and not layer.is_initialized
    k = torch.randn(1, 2, 3, 128)
    layer.stash_pre_rope(torch.randn(1, 3, 256))
    layer.update(k, k)
    assert layer.get_seq_length() == 3

"""The C-ABI library loads, exports every symbol include/*.h declares,
agrees with the numpy page format, and rejects bad arguments on the host — all
without a GPU (no compute call is made)."""

import ctypes as ct
import re
from pathlib import Path

import numpy as np
import pytest
import torch

from bmx_amd import _lib, codecs as K
from oracle import codecs as OC
from oracle import layout as OL

ROOT = Path(__file__).resolve().parent.parent


def test_library_exports_every_declared_symbol():
    declared = set()
    for hdr in sorted((ROOT / "include").glob("*.h")):
        declared |= set(re.findall(r"^\s*(?:const\s+)?\w+\*?\s+\*?(bmx_\w+)\s*\(", hdr.read_text(), re.M))
    assert declared == set(_lib.EXPORTS), declared ^ set(_lib.EXPORTS)
    h = _lib.lib()
    for name in declared:
        assert getattr(h, name) is not None


@pytest.mark.parametrize("h_kv,rank", [(8, 32), (8, 16), (2, 16), (1, 32), (16, 32)])
def test_page_geometry_matches_numpy_layout(h_kv, rank):
    assert _lib.page_bytes(h_kv, rank) == OL.page_bytes(h_kv, rank)
    secs = _lib.page_sections(h_kv, rank)
    ref = OL.sections(h_kv, rank)
    for name in _lib.SECTIONS:
        assert secs[name] == ref[name]
    # bytes per token = 2R + 86 h_kv = exact k2b bits per entry
    C = 128 * h_kv
    bpt = OL.page_bytes(h_kv, rank) / 16
    bits = bpt * 8 / C
    assert bits == pytest.approx(3 + 16 / 64 + 2 + 16 * h_kv / C + 16 * rank / C)


def test_headline_bytes_per_token():
    assert OL.page_bytes(8, 32) == 16 * 752
    assert OL.page_bytes(8, 16) == 16 * 720


def test_bad_geometry_is_rejected_with_message():
    with pytest.raises(RuntimeError, match="unsupported geometry"):
        _lib.page_bytes(8, 24)
    a = _lib.DecodeArgs()
    a.geom = _lib.Geom(8, 32, 32)  # G too large
    a.batch = 1
    rc = _lib.lib().bmx_k2b_decode(ct.byref(a), None)
    assert rc != 0 and b"n_q_groups" in _lib.lib().bmx_last_error()
    a.geom = _lib.Geom(8, 32, 4)
    a.max_packed_len = 100  # not a multiple of 128
    rc = _lib.lib().bmx_k2b_decode(ct.byref(a), None)
    assert rc != 0 and b"multiple of 128" in _lib.lib().bmx_last_error()
    ap = _lib.AppendArgs()
    ap.geom = _lib.Geom(8, 7, 1)
    assert _lib.lib().bmx_k2b_append(ct.byref(ap), None) != 0
    ap.geom = _lib.Geom(8, 32, 1)
    ap.n_codec_pages = 2
    rc = _lib.lib().bmx_k2b_append(ct.byref(ap), None)
    assert rc != 0 and b"null pointer" in _lib.lib().bmx_last_error()


def test_noalloc_checks_arguments_before_the_scratch_size():
    """An invalid geometry reaches bmx_k2b_decode_noalloc's argument checks
    (BMX_E_INVALID, the field named), not its scratch-size check, which a
    wrapped size would fail with BMX_E_WORKSPACE; a valid call too large for
    the static scratch is the BMX_E_WORKSPACE case (no launch in either)."""
    E_INVALID, E_WORKSPACE = 1, 2
    L = _lib.lib()
    a = _lib.DecodeArgs()
    a.geom = _lib.Geom(-1, 32, 4)
    a.batch = 1
    assert L.bmx_k2b_decode_noalloc(ct.byref(a), None) == E_INVALID
    assert b"h_kv" in L.bmx_last_error()
    a.geom = _lib.Geom(8, 32, -3)
    assert L.bmx_k2b_decode_noalloc(ct.byref(a), None) == E_INVALID
    assert b"n_q_groups" in L.bmx_last_error()
    a.geom = _lib.Geom(8, 32, 4)
    a.rope_scaling = 1.0
    a.io_dtype = 7
    a.q = a.out = a.packed_len = 16   # non-NULL stand-ins: the call stops at the checks
    assert L.bmx_k2b_decode_noalloc(ct.byref(a), None) == E_INVALID
    assert b"io_dtype" in L.bmx_last_error()
    a.io_dtype = 0
    a.pages = a.basis = 16
    a.n_pool_pages = 1
    a.batch, a.max_packed_len, a.split_tokens = 64, 1 << 20, 128   # 8192 splits of 2048 rows: 4.4 GB
    a.max_pages = (1 << 20) // 16
    assert L.bmx_k2b_decode_noalloc(ct.byref(a), None) == E_WORKSPACE
    assert b"static scratch" in L.bmx_last_error()


def test_window_rows_given_apart_rejected_on_the_host():
    """The host window length and the rows given apart are checked before any
    device work: tail_len_value within 0..tail_cap, rows given apart only with
    tail_len NULL and n_new <= tail_len_value, 8-element strides."""
    from bmx_amd import k2b
    lib = _lib.lib()
    fake = 1 << 20   # never dereferenced: every call below fails validation
    for args_t, fn, geom in ((_lib.DecodeArgs, lib.bmx_k2b_decode, _lib.Geom(8, 32, 4)),
                             (_lib.RtnDecodeArgs, lib.bmx_rtn_decode, None)):
        a = args_t()
        if geom is not None:
            a.geom = geom
            a.rope_scaling = 1.0
        else:
            from bmx_amd import rtn
            a.geom = rtn.geom(8, 4, k_bits=4, v_bits=4, k_group=32, v_group=32)
        a.batch = 1
        a.q = a.out = a.packed_len = fake
        a.tail_cap = 128
        a.tail_len_value = 129
        assert fn(ct.byref(a), None) != 0 and b"tail_len_value" in lib.bmx_last_error()
        a.tail_len_value = 4
        a.n_new, a.new_k, a.new_v = 5, fake, fake
        assert fn(ct.byref(a), None) != 0 and b"n_new" in lib.bmx_last_error()
        a.n_new, a.tail_len = 1, fake
        assert fn(ct.byref(a), None) != 0 and b"n_new" in lib.bmx_last_error()
        a.tail_len, a.new_stride_t = None, 12
        assert fn(ct.byref(a), None) != 0 and b"multiples of 8" in lib.bmx_last_error()
        a.new_stride_t, a.tail_dtype = 128, 2
        assert fn(ct.byref(a), None) != 0 and b"tail_dtype" in lib.bmx_last_error()
    # the Python wrapper's own checks
    a = _lib.DecodeArgs()
    a.tail_cap = 128
    with pytest.raises(ValueError, match="within 0..tail_cap"):
        k2b.set_window_rows(a, 1, 8, 200, 128)
    k = torch.zeros(1, 8, 2, 128, dtype=torch.float16)
    with pytest.raises(ValueError, match="more rows than the window"):
        k2b.set_window_rows(a, 1, 8, 1, 128, (k, k))
    with pytest.raises(ValueError, match="window's dtype"):
        k2b.set_window_rows(a, 1, 8, 4, 128, (k.float(), k.float()))
    a.tail_dtype = 1   # a bf16 window takes bf16 rows only
    with pytest.raises(ValueError, match="window's dtype"):
        k2b.set_window_rows(a, 1, 8, 4, 128, (k, k))
    k2b.set_window_rows(a, 1, 8, 4, 128, (k.bfloat16(), k.bfloat16()))
    assert a.n_new == 2
    a.tail_dtype = 0
    with pytest.raises(ValueError, match="same strides"):
        k2b.set_window_rows(a, 1, 8, 4, 128, (k, k.transpose(1, 2).contiguous().transpose(1, 2)))
    k2b.set_window_rows(a, 1, 8, 4, 128, (k, k))
    assert a.tail_len is None and a.tail_len_value == 4 and a.n_new == 2 and a.new_stride_t == 128
    assert a.new_stride_b == 0 and a.new_stride_h == 256   # size-1 batch: stride unused
    # one row: its time stride is unused (any layout of the (1, h, 1, d) row)
    r = torch.zeros(1, 1, 8, 128, dtype=torch.float16).transpose(1, 2)
    k2b.set_window_rows(a, 1, 8, 4, 128, (r, torch.zeros(1, 8, 1, 128, dtype=torch.float16)))
    assert a.n_new == 1 and a.new_stride_h == 128 and a.new_stride_t == 0


def test_decode_workspace_size_formula():
    a = _lib.DecodeArgs()
    a.geom = _lib.Geom(8, 32, 4)
    a.batch = 2
    a.max_packed_len = 65536
    a.split_tokens = 1024
    n = _lib.lib().bmx_k2b_decode_workspace_bytes(ct.byref(a))
    # 64 split partials per query: a record of 128 fp16 channel means, then fp32 (max, sum)
    assert n == 2 * 64 * 8 * 4 * (128 * 2 + 2 * 4)


def test_product_codec_constants_match_reference():
    g = np.load(ROOT / "tests" / "golden" / "codecs.npz")
    assert np.array_equal(np.array(K.gaussian_codebook(2), dtype=np.float32), g["codebook_b2"])
    assert np.array_equal(np.array(K.hadamard_signs(128, 0)), g["signs_d128_s0"])
    bits = K.sign_bits(K.hadamard_signs(128, 7))
    signs = [(-1 if (bits[c >> 5] >> (c & 31)) & 1 else 1) for c in range(128)]
    assert signs == g["signs_d128_s7"].tolist()
    assert K.compute_flush_schedule(300, 32, 128) == OC.compute_flush_schedule(300, 32, 128) == 256


def test_product_inv_freq_matches_hf_config():
    from transformers import LlamaConfig

    cfg = LlamaConfig(hidden_size=4096, num_attention_heads=32, num_key_value_heads=8,
                      rope_theta=500000.0)
    inv, scale = K.rope_inv_freq(cfg)
    inv0, scale0 = K.rope_inv_freq(head_dim=128, theta=500000.0)
    assert torch.equal(inv, inv0) and scale == scale0 == 1.0

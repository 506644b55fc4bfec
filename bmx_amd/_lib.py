"""ctypes binding of libbmx_k2b.so (the C-ABI declared in include/bmx_k2b.h,
include/bmx_rtn.h, include/bmx_spectral.h, include/bmx_prefill.h and
include/bmx_bench.h).

The library is the product path: there is no fallback.  ``lib()`` raises if the
shared object was not built (python -m bmx_amd.build) and every wrapper raises
RuntimeError with the library's own message when a call returns non-zero.
"""

from __future__ import annotations

import ctypes as ct
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libbmx_k2b.so"

BMX_OK = 0
DECODE_SCRATCH_BYTES = 32 << 20   # BMX_K2B_DECODE_SCRATCH_BYTES (include/bmx_k2b.h)
SECTIONS = ("us", "vnorm", "kscale", "kres", "vcode")


class Geom(ct.Structure):
    # head_dim / k_group / k_bits 0: the recipe's 128 / 64 / 3
    _fields_ = [("h_kv", ct.c_int32), ("rank", ct.c_int32), ("n_q_groups", ct.c_int32),
                ("head_dim", ct.c_int32), ("k_group", ct.c_int32), ("k_bits", ct.c_int32)]


class DecodeArgs(ct.Structure):
    _fields_ = [
        ("geom", Geom),
        ("batch", ct.c_int32),
        ("q", ct.c_void_p),
        ("out", ct.c_void_p),
        ("pages", ct.c_void_p),
        ("n_pool_pages", ct.c_int32),
        ("page_table", ct.c_void_p),
        ("max_pages", ct.c_int32),
        ("packed_len", ct.c_void_p),
        ("max_packed_len", ct.c_int32),
        ("basis", ct.c_void_p),
        ("basis_stride", ct.c_int64),
        ("inv_freq", ct.c_float * 64),
        ("rope_scaling", ct.c_float),
        ("sm_scale", ct.c_float),
        ("codebook", ct.c_float * 4),
        ("v_sign_bits", ct.c_uint32 * 4),
        ("k_tail", ct.c_void_p),
        ("v_tail", ct.c_void_p),
        ("tail_stride_b", ct.c_int64),
        ("tail_stride_h", ct.c_int64),
        ("tail_stride_t", ct.c_int64),
        ("tail_len", ct.c_void_p),
        ("tail_cap", ct.c_int32),
        ("split_tokens", ct.c_int32),
        ("workspace", ct.c_void_p),
        ("workspace_bytes", ct.c_size_t),
        ("split_end_event", ct.c_void_p),
        ("tail_len_value", ct.c_int32),
        ("new_k", ct.c_void_p),
        ("new_v", ct.c_void_p),
        ("new_stride_b", ct.c_int64),
        ("new_stride_h", ct.c_int64),
        ("new_stride_t", ct.c_int64),
        ("n_new", ct.c_int32),
        ("io_dtype", ct.c_int32),
        ("tail_dtype", ct.c_int32),
    ]


class AppendArgs(ct.Structure):
    _fields_ = [
        ("geom", Geom),
        ("n_codec_pages", ct.c_int32),
        ("k_pre", ct.c_void_p),
        ("k_stride_h", ct.c_int64),
        ("k_stride_t", ct.c_int64),
        ("v", ct.c_void_p),
        ("v_stride_h", ct.c_int64),
        ("v_stride_t", ct.c_int64),
        ("basis32", ct.c_void_p),
        ("basis16", ct.c_void_p),
        ("us_first", ct.c_void_p),
        ("codebook", ct.c_float * 4),
        ("v_sign_bits", ct.c_uint32 * 4),
        ("pages", ct.c_void_p),
        ("n_pool_pages", ct.c_int32),
        ("page_ids", ct.c_void_p),
        ("v_dtype", ct.c_int32),
    ]


class DequantArgs(ct.Structure):
    _fields_ = [
        ("geom", Geom),
        ("pages", ct.c_void_p),
        ("n_pool_pages", ct.c_int32),
        ("page_table", ct.c_void_p),
        ("n_tokens", ct.c_int32),
        ("basis", ct.c_void_p),
        ("inv_freq", ct.c_float * 64),
        ("rope_scaling", ct.c_float),
        ("apply_rope", ct.c_int32),
        ("codebook", ct.c_float * 4),
        ("v_sign_bits", ct.c_uint32 * 4),
        ("k_out", ct.c_void_p),
        ("v_out", ct.c_void_p),
        ("out_dtype", ct.c_int32),
        ("pos0", ct.c_int32),
        ("out_rows", ct.c_int64),
    ]


class RtnGeom(ct.Structure):
    _fields_ = [("h_kv", ct.c_int32), ("n_q_groups", ct.c_int32), ("k_bits", ct.c_int32),
                ("v_bits", ct.c_int32), ("k_group", ct.c_int32), ("v_group", ct.c_int32),
                ("k_arm", ct.c_int32)]


class RtnAppendArgs(ct.Structure):
    _fields_ = [
        ("geom", RtnGeom),
        ("n_codec_pages", ct.c_int32),
        ("k", ct.c_void_p),
        ("k_stride_h", ct.c_int64),
        ("k_stride_t", ct.c_int64),
        ("k_dtype", ct.c_int32),
        ("v", ct.c_void_p),
        ("v_stride_h", ct.c_int64),
        ("v_stride_t", ct.c_int64),
        ("v_dtype", ct.c_int32),
        ("pages", ct.c_void_p),
        ("page_ids", ct.c_void_p),
        ("n_pool_pages", ct.c_int32),
    ]


class RtnDecodeArgs(ct.Structure):
    _fields_ = [
        ("geom", RtnGeom),
        ("batch", ct.c_int32),
        ("q", ct.c_void_p),
        ("out", ct.c_void_p),
        ("pages", ct.c_void_p),
        ("n_pool_pages", ct.c_int32),
        ("page_table", ct.c_void_p),
        ("max_pages", ct.c_int32),
        ("packed_len", ct.c_void_p),
        ("max_packed_len", ct.c_int32),
        ("sm_scale", ct.c_float),
        ("k_tail", ct.c_void_p),
        ("v_tail", ct.c_void_p),
        ("tail_stride_b", ct.c_int64),
        ("tail_stride_h", ct.c_int64),
        ("tail_stride_t", ct.c_int64),
        ("tail_len", ct.c_void_p),
        ("tail_cap", ct.c_int32),
        ("split_tokens", ct.c_int32),
        ("workspace", ct.c_void_p),
        ("workspace_bytes", ct.c_size_t),
        ("tail_len_value", ct.c_int32),
        ("new_k", ct.c_void_p),
        ("new_v", ct.c_void_p),
        ("new_stride_b", ct.c_int64),
        ("new_stride_h", ct.c_int64),
        ("new_stride_t", ct.c_int64),
        ("n_new", ct.c_int32),
        ("io_dtype", ct.c_int32),
        ("tail_dtype", ct.c_int32),
    ]


class RtnDequantArgs(ct.Structure):
    _fields_ = [
        ("geom", RtnGeom),
        ("pages", ct.c_void_p),
        ("n_pool_pages", ct.c_int32),
        ("page_ids", ct.c_void_p),
        ("n_pages", ct.c_int32),
        ("k_out", ct.c_void_p),
        ("v_out", ct.c_void_p),
        ("out_dtype", ct.c_int32),
        ("out_rows", ct.c_int64),
    ]


class SpectralLayout(ct.Structure):
    _fields_ = [("h_kv", ct.c_int32), ("c_pad", ct.c_int32), ("k_page_bytes", ct.c_int32),
                ("slice_tab", ct.c_void_p), ("lloyd_levels", ct.c_void_p)]


class SpectralAppendArgs(ct.Structure):
    _fields_ = [
        ("L", SpectralLayout),
        ("n_groups", ct.c_int32),
        ("k_pre", ct.c_void_p),
        ("k_dtype", ct.c_int32),
        ("k_sh", ct.c_int64),
        ("k_st", ct.c_int64),
        ("v", ct.c_void_p),
        ("v_dtype", ct.c_int32),
        ("v_sh", ct.c_int64),
        ("v_st", ct.c_int64),
        ("enc_perm", ct.c_void_p),
        ("k_pages", ct.c_void_p),
        ("k_page_ids", ct.c_void_p),
        ("n_k_pool", ct.c_int32),
        ("v_pages", ct.c_void_p),
        ("v_page_ids", ct.c_void_p),
        ("n_v_pool", ct.c_int32),
        ("v_codebook", ct.c_float * 4),
        ("v_sign_bits", ct.c_uint32 * 4),
        ("v_codec", ct.c_int32),
        ("v_sign_bits_c", ct.c_uint32 * 32),
    ]


class SpectralDequantArgs(ct.Structure):
    _fields_ = [
        ("L", SpectralLayout),
        ("n_tokens", ct.c_int32),
        ("k_pages", ct.c_void_p),
        ("k_page_table", ct.c_void_p),
        ("n_k_pool", ct.c_int32),
        ("v_pages", ct.c_void_p),
        ("v_page_table", ct.c_void_p),
        ("n_v_pool", ct.c_int32),
        ("dec_perm", ct.c_void_p),
        ("apply_rope", ct.c_int32),
        ("rope_scaling", ct.c_float),
        ("inv_freq", ct.c_float * 64),
        ("v_codebook", ct.c_float * 4),
        ("v_sign_bits", ct.c_uint32 * 4),
        ("out_dtype", ct.c_int32),
        ("k_out", ct.c_void_p),
        ("v_out", ct.c_void_p),
        ("out_rows", ct.c_int32),
        ("q", ct.c_void_p),
        ("q_dtype", ct.c_int32),
        ("n_q_groups", ct.c_int32),
        ("scores", ct.c_void_p),
        ("partials", ct.c_void_p),
        ("sm_scale", ct.c_float),
        ("v_codec", ct.c_int32),
        ("v_sign_bits_c", ct.c_uint32 * 32),
    ]


class SpectralMergeArgs(ct.Structure):
    _fields_ = [("h_kv", ct.c_int32), ("n_q_groups", ct.c_int32), ("n_groups", ct.c_int32),
                ("partials", ct.c_void_p), ("q", ct.c_void_p), ("q_dtype", ct.c_int32),
                ("k_win", ct.c_void_p), ("v_win", ct.c_void_p), ("win_len", ct.c_int32),
                ("sm_scale", ct.c_float), ("out", ct.c_void_p), ("out_dtype", ct.c_int32),
                ("v_sign_bits", ct.c_uint32 * 4), ("win_stride_h", ct.c_int64),
                ("v_codec", ct.c_int32), ("v_sign_bits_c", ct.c_uint32 * 32), ("win_dtype", ct.c_int32)]


class Fp16DecodeArgs(ct.Structure):
    """bmx_fp16_decode_args (include/bmx_bench.h): the dense fp16 comparator."""
    _fields_ = [
        ("q", ct.c_void_p), ("k", ct.c_void_p), ("v", ct.c_void_p),
        ("stride_h", ct.c_int64), ("stride_t", ct.c_int64),
        ("h_kv", ct.c_int), ("n_q_groups", ct.c_int), ("T", ct.c_int), ("n_split", ct.c_int),
        ("sm_scale", ct.c_float),
        ("out", ct.c_void_p), ("workspace", ct.c_void_p), ("workspace_bytes", ct.c_size_t),
    ]


class PrefillArgs(ct.Structure):
    """bmx_prefill_args (include/bmx_prefill.h): prefill attention over dense rows."""
    _fields_ = [
        ("q", ct.c_void_p), ("q_stride_h", ct.c_int64), ("q_stride_t", ct.c_int64),
        ("k", ct.c_void_p), ("v", ct.c_void_p), ("kv_stride_h", ct.c_int64), ("kv_stride_t", ct.c_int64),
        ("out", ct.c_void_p),
        ("h_kv", ct.c_int), ("n_q_groups", ct.c_int), ("n_q", ct.c_int), ("n_kv", ct.c_int),
        ("head_dim", ct.c_int), ("dtype", ct.c_int), ("causal", ct.c_int), ("sm_scale", ct.c_float),
        ("n_split", ct.c_int), ("workspace", ct.c_void_p), ("workspace_bytes", ct.c_size_t),
    ]


EXPORTS = {
    "bmx_last_error": (ct.c_char_p, []),
    "bmx_k2b_page_bytes": (ct.c_size_t, [ct.POINTER(Geom)]),
    "bmx_k2b_page_section": (ct.c_int, [ct.POINTER(Geom), ct.c_int, ct.POINTER(ct.c_size_t),
                                        ct.POINTER(ct.c_size_t)]),
    "bmx_k2b_decode_workspace_bytes": (ct.c_size_t, [ct.POINTER(DecodeArgs)]),
    "bmx_k2b_decode": (ct.c_int, [ct.POINTER(DecodeArgs), ct.c_void_p]),
    "bmx_k2b_decode_noalloc": (ct.c_int, [ct.POINTER(DecodeArgs), ct.c_void_p]),
    "bmx_k2b_append": (ct.c_int, [ct.POINTER(AppendArgs), ct.c_void_p]),
    "bmx_k2b_dequant": (ct.c_int, [ct.POINTER(DequantArgs), ct.c_void_p]),
    "bmx_rtn_page_bytes": (ct.c_size_t, [ct.POINTER(RtnGeom)]),
    "bmx_rtn_append": (ct.c_int, [ct.POINTER(RtnAppendArgs), ct.c_void_p]),
    "bmx_rtn_decode_workspace_bytes": (ct.c_size_t, [ct.POINTER(RtnDecodeArgs)]),
    "bmx_rtn_decode": (ct.c_int, [ct.POINTER(RtnDecodeArgs), ct.c_void_p]),
    "bmx_rtn_dequant": (ct.c_int, [ct.POINTER(RtnDequantArgs), ct.c_void_p]),
    "bmx_spectral_v_page_bytes": (ct.c_int64, [ct.c_int32]),
    "bmx_spectral_v_page_bytes_codec": (ct.c_int64, [ct.c_int32, ct.c_int32]),
    "bmx_spectral_append": (ct.c_int32, [ct.POINTER(SpectralAppendArgs), ct.c_void_p]),
    "bmx_spectral_dequant": (ct.c_int32, [ct.POINTER(SpectralDequantArgs), ct.c_void_p]),
    "bmx_spectral_merge": (ct.c_int32, [ct.POINTER(SpectralMergeArgs), ct.c_void_p]),
    "bmx_spectral_partial_count": (ct.c_int32, [ct.POINTER(SpectralDequantArgs)]),
    "bmx_fp16_decode_workspace_bytes": (ct.c_size_t, [ct.c_int, ct.c_int, ct.c_int]),
    "bmx_fp16_decode": (ct.c_int, [ct.POINTER(Fp16DecodeArgs), ct.c_void_p]),
    "bmx_prefill_workspace_bytes": (ct.c_size_t, [ct.POINTER(PrefillArgs)]),
    "bmx_prefill": (ct.c_int, [ct.POINTER(PrefillArgs), ct.c_void_p]),
}

_LIB = None


def lib():
    """Load libbmx_k2b.so once; raise if it has not been built."""
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -m bmx_amd.build` "
                "(the k2b decode path has no non-HIP fallback)")
        h = ct.CDLL(str(LIB_PATH))
        for name, (res, args) in EXPORTS.items():
            fn = getattr(h, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = h
    return _LIB


def check(rc: int, what: str) -> None:
    if rc != BMX_OK:
        msg = lib().bmx_last_error().decode()
        raise RuntimeError(f"{what} failed (status {rc}): {msg}")


def page_bytes(h_kv: int, rank: int, *, head_dim: int = 128, group: int = 64, k_bits: int = 3) -> int:
    g = Geom(h_kv, rank, 1, head_dim, group, k_bits)
    n = lib().bmx_k2b_page_bytes(ct.byref(g))
    if n == 0:
        raise RuntimeError(lib().bmx_last_error().decode())
    return int(n)


def page_sections(h_kv: int, rank: int, *, head_dim: int = 128, group: int = 64, k_bits: int = 3) -> dict:
    g = Geom(h_kv, rank, 1, head_dim, group, k_bits)
    out = {}
    for i, name in enumerate(SECTIONS):
        off, sz = ct.c_size_t(), ct.c_size_t()
        check(lib().bmx_k2b_page_section(ct.byref(g), i, ct.byref(off), ct.byref(sz)),
              "bmx_k2b_page_section")
        out[name] = (off.value, sz.value)
    return out

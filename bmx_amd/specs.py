"""Codec specification and the recipe registry subset this path serves.

Mirrors the reference's ``CacheCodecSpec`` (cache/specs.py:13-91) field for
field where the packed paths read them, and ``spec_pair`` (cache/recipes.py:
13-42) for the ``k2b_ph`` recipe.  The MI355X kernels implement the two arm
pairs the reference's attend() sends to a fused kernel
(cache/packed_streaming.py:904-975):

* k2b: K pre-RoPE ``lowrank_rtn_channel`` 3-bit residual, rank 16 or 32,
  64-token scale groups; V ``turboquant_mse_perhead`` 2-bit;
* RTN: K and V ``rtn_token`` (K post-RoPE), 2..4 bits, channel groups of
  32, 64 or 128; the keys may also be ``rtn_channel`` (token groups of 32,
  64 or 128 per channel: config 1 and the ``kivi`` recipe, which the
  reference runs on its chunked path only);
* spectral (K4): K ``spectral`` pre-RoPE from a pack file (64-token
  groups) under the reference's recipe ``k4_b<budget>``, with its full-C
  ``turboquant_mse`` 2-bit values (one C-point rotation and one norm per
  token, recipes.py:138-143; C = 128 h_kv a power of two), and under
  ``k4ph_b<budget>`` with the per-head value codec of the other pre-RoPE
  pair; both with the reference's suffixes ``_lq`` (the Lloyd payload) and
  ``_dec8``, ``_dec8t<T>``, ``_dec8tl`` (an int8 roundtrip of the decoder
  when the packs load).

Every other pair raises, naming what it got: there is no CPU or slow path to
route it to.
"""

from __future__ import annotations

import dataclasses
import re


@dataclasses.dataclass
class CacheCodecSpec:
    """Codec specification for one side (K or V) of the KV cache
    (cache/specs.py:13-91).  Only the fields the k2b path reads are kept."""

    arm: str = "fp16"
    bits: int = 3
    rank: int = 0
    group: int = 64
    seed: int = 0
    pre_rope: bool = False
    pack_path: str | None = None      # spectral: the pack file (spectral.py:1081-1170)
    budget: float | None = None       # spectral: the pack's budget label
    dec_quant: str = "fp32"           # spectral: decoder storage: fp32 | int8 | int8_t<T> | int8_tl
    payload_quant: str = "rtn"        # spectral: payload quantizer: rtn | lloyd


def spec_pair(arm: str, *, rank: int = 16, group: int = 64, seed: int = 0, pack_path: str | None = None):
    """(k_spec, v_spec) for a named recipe (cache/recipes.py:13-42, 88-143, 173-177)."""
    if arm.startswith("k4_b") or arm.startswith("k4ph_b"):
        # k4_b: the reference's recipe, full-C turboquant_mse values (recipes.py:
        # 138-143); k4ph_b: the same keys with the per-head value codec
        if not pack_path:
            raise ValueError("k4 arms require --pack-path (a fitted spectral pack file)")
        prefix = "k4_b" if arm.startswith("k4_b") else "k4ph_b"
        budget, payload_quant, dec_quant = _k4_variant(arm, prefix)
        return (CacheCodecSpec(arm="spectral", pre_rope=True, group=group, pack_path=pack_path,
                               budget=budget, seed=seed, dec_quant=dec_quant, payload_quant=payload_quant),
                CacheCodecSpec(arm="turboquant_mse" if prefix == "k4_b" else "turboquant_mse_perhead", bits=2,
                               seed=seed))
    if arm == "kivi":
        return (CacheCodecSpec(arm="rtn_channel", bits=2, group=group, seed=seed),
                CacheCodecSpec(arm="rtn_token", bits=2, group=group, seed=seed))
    if arm != "k2b_ph":
        raise NotImplementedError(
            f"recipe {arm!r} has no MI355X kernels; this package implements 'k2b_ph', 'kivi' and 'k4ph_b<budget>'")
    return (CacheCodecSpec(arm="lowrank_rtn_channel", bits=3, rank=rank, group=group, seed=seed,
                           pre_rope=True),
            CacheCodecSpec(arm="turboquant_mse_perhead", bits=2, seed=seed))


_K4_SUFFIX = re.compile(r"(?P<budget>.+?)(?P<lq>_lq)?(?P<dec>_dec8(?:tl|t[^_]*)?)?")


def _k4_variant(arm: str, prefix: str) -> tuple:
    """(budget, payload_quant, dec_quant) of a k4 recipe name
    ``<prefix><budget>[_lq][_dec8 | _dec8t<T> | _dec8tl]`` (recipes.py:
    100-150): "_lq" selects the Lloyd payload and sits between the budget and
    the decoder suffix; "_dec8" stores every coded decoder column int8,
    "_dec8t<T>" those of tiers <= T, "_dec8tl" a certificate-derived
    threshold per layer."""
    m = _K4_SUFFIX.fullmatch(arm[len(prefix):])
    dec = m.group("dec") or ""
    dec_quant = {"": "fp32", "_dec8": "int8", "_dec8tl": "int8_tl"}.get(dec, "int8_t" + dec[len("_dec8t"):])
    if "_lq" in m.group("budget") or "_dec8" in m.group("budget"):
        raise ValueError(f"malformed k4 arm {arm!r}: the form is '{prefix}<budget>[_lq][_dec8|_dec8t<T>|_dec8tl]', "
                         f"e.g. '{prefix}2.5_lq_dec8tl'")
    from .spectral import dec_quant_threshold
    dec_quant_threshold(dec_quant)   # raises on a threshold outside 2..8
    return float(m.group("budget")), ("lloyd" if m.group("lq") else "rtn"), dec_quant


def is_rtn(k_spec: CacheCodecSpec, v_spec: CacheCodecSpec) -> bool:
    """The fused RTN pair (packed_streaming.py:904-912: rtn_token keys, not
    pre-RoPE, and rtn_token values), or rtn_channel keys with rtn_token values,
    within the kernels' bit widths and groups."""
    return (k_spec.arm in ("rtn_token", "rtn_channel") and v_spec.arm == "rtn_token" and not k_spec.pre_rope
            and 2 <= k_spec.bits <= 4 and 2 <= v_spec.bits <= 4
            and k_spec.group in (32, 64, 128) and v_spec.group in (32, 64, 128))


def packed_path(k_spec: CacheCodecSpec, v_spec: CacheCodecSpec) -> str:
    """"k2b", "rtn" or "spectral" for a spec pair the MI355X kernels implement;
    raise otherwise."""
    if is_rtn(k_spec, v_spec):
        return "rtn"
    if k_spec.arm == "spectral":
        check_spectral(k_spec, v_spec)
        return "spectral"
    check_k2b(k_spec, v_spec)
    return "k2b"


def check_k2b(k_spec: CacheCodecSpec, v_spec: CacheCodecSpec) -> None:
    """Raise unless (k_spec, v_spec) is a k2b pair the kernels implement."""
    ok = (k_spec.arm == "lowrank_rtn_channel" and k_spec.bits in (2, 3, 4) and k_spec.group in (16, 32, 64, 128)
          and k_spec.pre_rope and k_spec.rank in (16, 32, 64, 128)
          and v_spec.arm == "turboquant_mse_perhead" and v_spec.bits == 2)
    if not ok:
        raise NotImplementedError(
            f"the MI355X packed paths implement K=lowrank_rtn_channel (2..4 bits, groups 16|32|64|128, "
            f"pre-RoPE, rank 16|32|64|128) with V=turboquant_mse_perhead (2 bits), and K=rtn_token|"
            f"rtn_channel with V=rtn_token (2..4 bits, groups 32|64|128, K post-RoPE); got "
            f"K={k_spec} V={v_spec}")


def check_spectral(k_spec: CacheCodecSpec, v_spec: CacheCodecSpec) -> None:
    """The construction-time guards of the spectral arm (packed_streaming.py:
    336-360: pre-RoPE keys and a pack file, asserted), then the variants the
    kernels implement."""
    assert k_spec.pre_rope, "spectral K requires pre_rope=True (RoPE is applied at read)"
    assert k_spec.pack_path, "spectral K requires pack_path (a fitted spectral pack file)"
    from .spectral import dec_quant_threshold
    dec_quant_threshold(k_spec.dec_quant)
    if k_spec.payload_quant not in ("rtn", "lloyd"):
        raise NotImplementedError(
            f"spectral payload_quant={k_spec.payload_quant!r}: the MI355X kernels implement the rtn and lloyd "
            f"payloads")
    if not (v_spec.arm in ("turboquant_mse_perhead", "turboquant_mse") and v_spec.bits == 2):
        raise NotImplementedError(
            f"spectral K pairs with V=turboquant_mse (full C) or turboquant_mse_perhead, 2 bits, on the MI355X "
            f"path; got V={v_spec}")

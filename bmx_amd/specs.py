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
  reference runs on its chunked path only).

Every other pair raises, naming what it got: there is no CPU or slow path to
route it to.
"""

from __future__ import annotations

import dataclasses


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


def spec_pair(arm: str, *, rank: int = 16, group: int = 64, seed: int = 0):
    """(k_spec, v_spec) for a named recipe (cache/recipes.py:13-42, 173-177)."""
    if arm == "kivi":
        return (CacheCodecSpec(arm="rtn_channel", bits=2, group=group, seed=seed),
                CacheCodecSpec(arm="rtn_token", bits=2, group=group, seed=seed))
    if arm != "k2b_ph":
        raise NotImplementedError(
            f"recipe {arm!r} has no MI355X kernels; this package implements 'k2b_ph' and 'kivi'")
    return (CacheCodecSpec(arm="lowrank_rtn_channel", bits=3, rank=rank, group=group, seed=seed,
                           pre_rope=True),
            CacheCodecSpec(arm="turboquant_mse_perhead", bits=2, seed=seed))


def is_rtn(k_spec: CacheCodecSpec, v_spec: CacheCodecSpec) -> bool:
    """The fused RTN pair (packed_streaming.py:904-912: rtn_token keys, not
    pre-RoPE, and rtn_token values), or rtn_channel keys with rtn_token values,
    within the kernels' bit widths and groups."""
    return (k_spec.arm in ("rtn_token", "rtn_channel") and v_spec.arm == "rtn_token" and not k_spec.pre_rope
            and 2 <= k_spec.bits <= 4 and 2 <= v_spec.bits <= 4
            and k_spec.group in (32, 64, 128) and v_spec.group in (32, 64, 128))


def packed_path(k_spec: CacheCodecSpec, v_spec: CacheCodecSpec) -> str:
    """"k2b" or "rtn" for a spec pair the MI355X kernels implement; raise otherwise."""
    if is_rtn(k_spec, v_spec):
        return "rtn"
    check_k2b(k_spec, v_spec)
    return "k2b"


def check_k2b(k_spec: CacheCodecSpec, v_spec: CacheCodecSpec) -> None:
    """Raise unless (k_spec, v_spec) is a k2b pair the kernels implement."""
    ok = (k_spec.arm == "lowrank_rtn_channel" and k_spec.bits == 3 and k_spec.group == 64
          and k_spec.pre_rope and k_spec.rank in (16, 32)
          and v_spec.arm == "turboquant_mse_perhead" and v_spec.bits == 2)
    if not ok:
        raise NotImplementedError(
            f"the MI355X packed paths implement K=lowrank_rtn_channel (3 bits, group 64, "
            f"pre-RoPE, rank 16|32) with V=turboquant_mse_perhead (2 bits), and K=rtn_token|"
            f"rtn_channel with V=rtn_token (2..4 bits, groups 32|64|128, K post-RoPE); got "
            f"K={k_spec} V={v_spec}")

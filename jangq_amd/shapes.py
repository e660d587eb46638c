"""Bit width / group size inference from packed shapes (host logic, no GPU work).

Restates the JANG loader rule ``_fix_quantized_bits``
(jang-tools/jang_tools/loader.py:1914-1981) and the Swift ``BitInference.infer``
(jang-runtime/Sources/JANGCore/BitInference.swift:15-53):
    weight [.., out, in*bits/32], scales [.., out, in/gs]  =>  w_cols*32 == bits*in,
    in == s_cols*gs.
Several (bits, gs) pairs can satisfy one shape pair; candidates are tried in the loader's
preference order and the module's logical input dimension, when known, disambiguates.
"""
from __future__ import annotations

from dataclasses import dataclass

VALID_BITS = (2, 3, 4, 5, 6, 8)


@dataclass(frozen=True)
class BitInferenceResult:
    bits: int
    in_features: int
    out_features: int


def bit_inference(qweight_shape, scales_shape, group_size: int) -> BitInferenceResult | None:
    """Fixed-gs rule of BitInference.swift:15-53 (2-D or stacked 3-D); None on mismatch."""
    q, s = list(qweight_shape), list(scales_shape)
    if len(q) < 2 or len(s) < 2 or len(q) != len(s):
        return None
    if len(q) > 2 and q[:-2] != s[:-2]:
        return None
    if q[-2] != s[-2]:
        return None
    packed_in, n_groups = q[-1], s[-1]
    if packed_in <= 0 or n_groups <= 0 or group_size <= 0:
        return None
    in_features = n_groups * group_size
    num = packed_in * 32
    if num % in_features:
        return None
    out = q[-2]
    for d in q[:-2]:
        out *= d
    return BitInferenceResult(bits=num // in_features, in_features=in_features, out_features=out)


def infer_bits_group_size(w_cols: int, s_cols: int, bits: int, group_size: int, *,
                          logical_in: int | None = None, is_router: bool = False):
    """(bits, group_size) for a module whose current settings are (bits, group_size),
    following loader.py:1914-1981. Returns the current settings when nothing fits."""
    if logical_in:
        cands: list[int] = []
        for gs in (group_size, 64, 128, 32):
            if gs not in cands and logical_in % gs == 0 and s_cols * gs == logical_in:
                cands.append(gs)
        for gs in (group_size, 64, 128, 32):
            if gs not in cands:
                cands.append(gs)
    elif is_router:
        cands = [64, group_size, 128]
    else:
        cands = [group_size] + [g for g in (64, 128) if g != group_size]
    for gs in cands:
        in_dim = s_cols * gs
        if in_dim <= 0 or (w_cols * 32) % in_dim:
            continue
        b = (w_cols * 32) // in_dim
        if b in VALID_BITS:
            if logical_in and in_dim != logical_in:
                continue
            return b, gs
    in_dim = s_cols * group_size
    if in_dim > 0:
        b = (w_cols * 32) // in_dim
        if b in VALID_BITS:
            return b, group_size
    return bits, group_size


def is_router_name(name: str) -> bool:
    """Router / gate tensors prefer gs=64 (loader.py:1941-1943)."""
    n = name.lower()
    return ".gate." in n or n.endswith(".gate") or "shared_expert_gate" in n

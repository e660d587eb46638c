"""Helpers shared by the GPU parity tests: seeded inputs built with the CPU oracle and
moved to the device, and the tolerance checks the north star states."""
from __future__ import annotations

import numpy as np
import torch

from oracle import jangq_oracle as O

# Matmul outputs vs the fp32-accumulated oracle rounded to the output dtype.
REL_L2_TOL = 1e-3
MAX_ABS_TOL = 2e-2


def bf16_tensor(a_f32: np.ndarray, device="cuda") -> torch.Tensor:
    bits = O.f32_to_bf16_bits(a_f32)
    return torch.from_numpy(bits.view(np.int16).copy()).view(torch.bfloat16).to(device)


def to_tensor(a: np.ndarray, dtype: str, device="cuda") -> torch.Tensor:
    """fp32 values -> device tensor of dtype ("bf16", "f16", "f32")."""
    if dtype == "bf16":
        return bf16_tensor(a, device)
    if dtype == "f16":
        return torch.from_numpy(np.asarray(a, np.float32).astype(np.float16)).to(device)
    return torch.from_numpy(np.asarray(a, np.float32)).to(device)


def sidecar_tensor(a, sidecar: str, device="cuda") -> torch.Tensor:
    if sidecar == "bf16":
        return torch.from_numpy(np.asarray(a, np.uint16).view(np.int16).copy()).view(
            torch.bfloat16).to(device)
    if sidecar == "f16":
        return torch.from_numpy(np.asarray(a, np.float16)).to(device)
    return torch.from_numpy(np.asarray(a, np.float32)).to(device)


def codes_tensor(packed: np.ndarray, device="cuda") -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(packed).view(np.int32)).to(device)


def values_of(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy()


class QWeight:
    """A seeded quantized matrix (or expert stack) on host and device."""

    def __init__(self, rows, K, bits, gs, seed, sidecar="bf16", std=0.02, experts=None,
                 device="cuda"):
        rng = np.random.default_rng(seed)
        shape = (rows, K) if experts is None else (experts * rows, K)
        w = O.round_bf16(rng.standard_normal(shape, dtype=np.float32) * np.float32(std))
        packed, s, b, codes = O.quantize_affine(w, bits, gs, sidecar=sidecar)
        if experts is not None:
            packed = packed.reshape(experts, rows, -1)
            s = s.reshape(experts, rows, -1)
            b = b.reshape(experts, rows, -1)
            codes = codes.reshape(experts, rows, -1)
        self.bits, self.gs, self.sidecar = bits, gs, sidecar
        self.packed, self.codes = packed, codes
        self.s_raw, self.b_raw = s, b
        self.s = O.sidecar_f32(s, sidecar)
        self.b = O.sidecar_f32(b, sidecar)
        self.dw = codes_tensor(packed, device)
        self.ds = sidecar_tensor(s, sidecar, device)
        self.db = sidecar_tensor(b, sidecar, device)

    def dequant(self):
        return O.dequantize_affine(self.packed, self.s, self.b, self.bits, self.gs)


def half_ulp(v: np.ndarray, dtype: str) -> np.ndarray:
    """Half a unit in the last place of |v| in a 16-bit float format (0 for fp32): the
    rounding every correctly rounded output of that dtype may carry."""
    if dtype not in ("bf16", "f16"):
        return np.zeros_like(np.asarray(v, dtype=np.float64))
    mant = 8 if dtype == "bf16" else 11
    e = np.floor(np.log2(np.maximum(np.abs(np.asarray(v, dtype=np.float64)), 1e-30)))
    if dtype == "f16":
        e = np.maximum(e, -14)
    return np.ldexp(1.0, (e - mant).astype(np.int64))


# Composite outputs (a MoE block, several bf16-rounded stages): rel-L2 bound. One ulp of
# bf16 is 2^-8 relative; stages that flip an intermediate rounding move ~1 in 10-20 outputs
# by one ulp, a rel-L2 of about 1e-3, so the bound is half an ulp of relative error.
COMPOSITE_REL_L2_TOL = 2e-3


def assert_close(got: np.ndarray, ref: np.ndarray, what: str,
                 rel=None, mabs=MAX_ABS_TOL, exact=None, out_dtype=None, ulps=0.5):
    """rel-L2 of got against ref (the reference rounded to the output dtype) and max-abs
    error. With `exact` (the unrounded fp32/fp64 accumulation) the max-abs bound applies to
    |got - exact| beyond the output rounding itself (ulps = half an ulp of out_dtype): an
    output that rounds the other way at a rounding boundary is then not charged a full ulp.

    Composite outputs (a MoE block: gate/up, h and each expert's output are rounded to the
    activation dtype before the next stage, as the reference's arrays are) pass ulps=1: an
    intermediate value within fp32-vs-fp64 accumulation noise of a rounding midpoint may round
    the other way, and that one-ulp step moves every output of the next matmul slightly, so
    some outputs legitimately land one ulp from the fp64 chain's rounding; their rel-L2
    bound is COMPOSITE_REL_L2_TOL. Each stage alone is held to the north-star bounds by the
    tests of its operator, and the fused launches are checked bit for bit against the
    composition of those operators."""
    if rel is None:
        rel = COMPOSITE_REL_L2_TOL if ulps >= 1 else REL_L2_TOL
    r = O.rel_l2(got, ref)
    if exact is None:
        m = O.max_abs(got, ref)
    else:
        dev = np.abs(np.asarray(got, np.float64) - np.asarray(exact, np.float64))
        m = float(np.max(dev - 2 * ulps * half_ulp(exact, out_dtype))) if dev.size else 0.0
        m = max(m, 0.0)
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    assert r <= rel and m <= mabs, f"{what}: rel_l2={r:.3e} (tol {rel}) max_abs={m:.3e} (tol {mabs})"
    return r, m


class RandQ:
    """A quantized matrix or expert stack built on the GPU from seeded random codes, for the
    configs' full sizes (a 512-expert stack is too large for the CPU quantizer). Any codes,
    scales and biases are a valid affine-quantized weight; the scales are positive and the
    biases centre each group (b ~ -s * (2^bits - 1) / 2), like quantized N(0, std) weights.
    The oracle reads back only the rows it needs (``host``)."""

    def __init__(self, rows, K, bits, gs, seed, experts=None, std=0.02, sidecar="bf16",
                 device="cuda"):
        g = torch.Generator(device=device)
        g.manual_seed(seed)
        lead = (rows,) if experts is None else (experts, rows)
        words = K * bits // 32
        # int32 words with every bit pattern: two 16-bit halves from randint
        lo = torch.randint(0, 1 << 16, (*lead, words), generator=g, device=device, dtype=torch.int32)
        hi = torch.randint(0, 1 << 16, (*lead, words), generator=g, device=device, dtype=torch.int32)
        self.dw = (hi << 16) | lo
        qmax = (1 << bits) - 1
        sdt = {"bf16": torch.bfloat16, "f16": torch.float16}[sidecar]
        # uniform codes have std qmax / sqrt(12): scales around std * sqrt(12) / qmax give
        # weights of standard deviation ~std, as a quantized N(0, std) matrix has
        s = (torch.rand((*lead, K // gs), generator=g, device=device) * 0.5 + 0.75) * (
            std * 12 ** 0.5 / qmax)
        b = -s * (qmax / 2.0) * (1.0 + 0.1 * torch.randn(s.shape, generator=g, device=device))
        self.ds, self.db = s.to(sdt), b.to(sdt)
        self.bits, self.gs, self.sidecar = bits, gs, sidecar
        self.experts = experts

    def host(self, e=None, rows=None):
        """(packed uint32, scales f32, biases f32) of expert e (or the 2-D matrix), rows sliced."""
        sel = () if e is None else (int(e),)
        if rows is not None:
            sel = sel + (rows,)
        if not sel:
            sel = (slice(None),)
        w = self.dw[sel].cpu().numpy().view(np.uint32)
        s = self.ds[sel].float().cpu().numpy()
        b = self.db[sel].float().cpu().numpy()
        return w, s, b

    def tup(self):
        return (self.dw, self.ds, self.db, self.bits)

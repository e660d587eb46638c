"""GPU parity of the batch-1 decode GEMV's launch forms at the sizes that select them, against
the oracle (fp64 accumulation of the exactly dequantized rows).

- Activation state built once per block in LDS: taken when the waves of a launch hold two or
  more row items, i.e. outputs of more rows than the resident waves cover (here 20-30k rows);
  K below a wave's two chunks per lane leaves lanes without a chunk (zero activations).
  Grouped launches of uneven problems cross problem boundaries inside a wave's item range.
- Long 2-bit rows (K > 4096) of at most 16384 output rows: one 32-code unit per lane chunk,
  8 rows per block; above 16384 rows, and above 8 waves of units, the two-unit chunks.

Weights are seeded random codes built on the GPU (tests._util.RandQ); the oracle reads back
only the rows it checks. Tolerances: rel-L2 <= 1e-3 and max-abs <= 2e-2 beyond the output
rounding (north star)."""
import numpy as np
import pytest
import torch

import jangq_amd as jq
from oracle import jangq_oracle as O
from tests._util import RandQ, assert_close, to_tensor, values_of

pytestmark = pytest.mark.gpu


def _deq(q: RandQ, rows):
    w, s, b = q.host(None, rows)
    return O.dequantize_affine(w, s, b, q.bits, q.gs).astype(np.float64)


def _slices(N, every):
    """Row slices to check: the first rows, rows around item and wave boundaries in the middle,
    and the last rows."""
    mid = (N // 2) // every * every
    return [slice(0, min(N, 96)), slice(max(0, mid - 40), min(N, mid + 40)),
            slice(max(0, N - 96), N)]


def _check(y, x, q, N, what, xdt="bf16"):
    got_all = values_of(y)
    assert got_all.shape == (1, N)
    for rows in _slices(N, 512):
        ref = x.astype(np.float64) @ _deq(q, rows).T
        assert_close(got_all[:, rows], O.round_to(ref, xdt), f"{what} rows {rows.start}:{rows.stop}",
                     exact=ref, out_dtype=xdt)


@pytest.mark.parametrize("bits,K,gs", [(3, 4096, 64), (3, 3072, 64), (3, 1024, 128), (2, 4096, 64),
                                       (2, 2048, 32), (4, 4096, 128), (6, 4096, 64), (8, 2048, 64),
                                       (5, 4096, 64)])
@pytest.mark.parametrize("xdt", ["bf16", "f16"])
def test_row_shared_state(bits, K, gs, xdt):
    """One activation row, many rows: the waves hold several items, so the block builds the
    activation state once in LDS."""
    N = 24000 + bits  # odd for odd widths: a last item of one row
    print(f"row shared state b{bits} K{K} g{gs} {xdt}", flush=True)
    q = RandQ(N, K, bits, gs, seed=700 + bits * 7 + K // 512 + gs, sidecar=xdt)
    rng = np.random.default_rng(701 + bits)
    x = O.round_to(rng.standard_normal((1, K), dtype=np.float32), xdt)
    y = jq.quantized_matmul(to_tensor(x, xdt), q.dw, q.ds, q.db, True, gs, bits)
    _check(y, x, q, N, f"shared b{bits} K{K} g{gs} {xdt}", xdt)


@pytest.mark.parametrize("bits", [3, 6])
def test_row_shared_state_grouped(bits):
    """A grouped launch of uneven problems (odd row counts, one of a single row): a wave's
    contiguous item range steps from one problem into the next."""
    K, gs = 4096, 64
    Ns = (9001, 1, 12287, 7777)
    print(f"row shared state grouped b{bits}", flush=True)
    qs = [RandQ(n, K, bits, gs, seed=720 + i + bits) for i, n in enumerate(Ns)]
    rng = np.random.default_rng(722 + bits)
    x = O.round_bf16(rng.standard_normal((1, K), dtype=np.float32))
    ys = jq.quantized_matmul_multi(to_tensor(x, "bf16"), [(q.dw, q.ds, q.db, gs, bits) for q in qs])
    for i, (q, y, n) in enumerate(zip(qs, ys, Ns)):
        _check(y, x, q, n, f"grouped b{bits} problem {i} N{n}")


@pytest.mark.parametrize("bits", [3, 8])
def test_swiglu_shared_state(bits):
    """The SwiGLU pair at one activation row over many rows (items are rows of the pair; the
    block builds the activation state once): h = silu(round(g)) * round(u), rounded."""
    N, K, gs = 20001, 4096, 64
    print(f"swiglu shared state b{bits}", flush=True)
    g = RandQ(N, K, bits, gs, seed=740 + bits)
    u = RandQ(N, K, bits, gs, seed=741 + bits)
    rng = np.random.default_rng(742)
    x = O.round_bf16(rng.standard_normal((1, K), dtype=np.float32))
    h = values_of(jq.quantized_swiglu(to_tensor(x, "bf16"), (g.dw, g.ds, g.db, bits),
                                      (u.dw, u.ds, u.db, bits), gs))
    assert h.shape == (1, N)
    for rows in _slices(N, 512):
        gv = O.round_bf16(x.astype(np.float64) @ _deq(g, rows).T).astype(np.float64)
        uv = O.round_bf16(x.astype(np.float64) @ _deq(u, rows).T).astype(np.float64)
        ref = O.silu(gv) * uv
        assert_close(h[:, rows], O.round_bf16(ref), f"swiglu b{bits} rows {rows.start}",
                     exact=ref, out_dtype="bf16", ulps=1)


@pytest.mark.parametrize("K,N", [(14336, 4096), (14336, 4099), (14336, 16384), (14336, 16385),
                                 (8192, 37), (16384, 1000), (32768, 300)])
@pytest.mark.parametrize("gs", [32, 64, 128])
def test_long_2bit_rows(K, N, gs):
    """Long 2-bit rows at one activation row on both sides of the one-unit-chunk rule (at most
    16384 rows and 8 waves of units), partial row blocks included."""
    print(f"long 2-bit K{K} N{N} g{gs}", flush=True)
    q = RandQ(N, K, 2, gs, seed=760 + K // 1024 + N % 97 + gs)
    rng = np.random.default_rng(761 + N)
    x = O.round_bf16(rng.standard_normal((1, K), dtype=np.float32))
    y = jq.quantized_matmul(to_tensor(x, "bf16"), q.dw, q.ds, q.db, True, gs, 2)
    _check(y, x, q, N, f"long 2-bit K{K} N{N} g{gs}")


@pytest.mark.parametrize("N", [96, 20000])
@pytest.mark.parametrize("gs", [32, 64, 128])
def test_8bit_f16_units_dynamic_range(N, gs):
    """8-bit codes with bf16 activations rescale each 32-value unit by a power of two into f16:
    units scaled from 2^-60 to 2^0, values spread over 2^-20 .. 1 inside a unit, an all-zero
    unit and a single-value unit; per-wave (N = 96) and block-shared (N = 20000) state. (The
    largest scale stays at 1: the north-star max-abs bound is absolute, and outputs far above
    1 carry fp32 accumulation noise beyond it on any kernel.)"""
    K = 4096
    print(f"8-bit f16 units N{N} g{gs}", flush=True)
    q = RandQ(N, K, 8, gs, seed=780 + gs + N % 7)
    rng = np.random.default_rng(781)
    units = K // 32
    x = rng.standard_normal((1, K)).astype(np.float64)
    x *= np.repeat(2.0 ** rng.integers(-60, 1, units), 32)[None, :]           # per-unit scale
    x *= 2.0 ** rng.integers(-20, 1, (1, K))                                   # spread in a unit
    x[:, 32 * 5:32 * 6] = 0.0                                                  # an all-zero unit
    x[:, 32 * 9 + 1:32 * 10] = 0.0                                             # one value left
    x = O.round_bf16(x.astype(np.float32))
    y = jq.quantized_matmul(to_tensor(x, "bf16"), q.dw, q.ds, q.db, True, gs, 8)
    _check(y, x, q, N, f"8-bit f16 units N{N} g{gs}")
    # the SwiGLU pair (the shared expert's form) on the same activations
    u = RandQ(N, K, 8, gs, seed=782 + gs)
    h = values_of(jq.quantized_swiglu(to_tensor(x, "bf16"), (q.dw, q.ds, q.db, 8),
                                      (u.dw, u.ds, u.db, 8), gs))
    for rows in _slices(N, 512):
        gv = O.round_bf16(x.astype(np.float64) @ _deq(q, rows).T).astype(np.float64)
        uv = O.round_bf16(x.astype(np.float64) @ _deq(u, rows).T).astype(np.float64)
        ref = O.silu(gv) * uv
        assert_close(h[:, rows], O.round_bf16(ref), f"8-bit swiglu N{N} g{gs} rows {rows.start}",
                     exact=ref, out_dtype="bf16", ulps=1)

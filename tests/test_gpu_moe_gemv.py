"""GPU parity of the vector-ALU expert-gathered GEMV: the gather_qmm and SwitchGLU launches
at decode sizes (a few plan rows per active expert), against the oracle's per-pair loops.

The kernel choice follows the average plan rows per active expert (upper bound of active
experts: min(pairs, E)); the cases below pin it by using every expert of a small stack the
same number of times: 1 -> tiles of one row, 2 -> two, 3..4 -> four (two at 2 bits).
Tolerances: rel-L2 <= 1e-3, max-abs <= 2e-2 beyond half an ulp of the output dtype."""
import numpy as np
import pytest
import torch

import jangq_amd as jq
from oracle import jangq_oracle as O
from tests._util import QWeight, assert_close, to_tensor, values_of

pytestmark = pytest.mark.gpu


def _pairs(E, per_expert, B, seed):
    """Each of the E experts exactly per_expert times, shuffled; x rows drawn from B."""
    rng = np.random.default_rng(seed)
    rhs = rng.permutation(np.repeat(np.arange(E), per_expert)).astype(np.int32)
    lhs = rng.integers(0, B, size=rhs.size).astype(np.int32)
    return lhs, rhs


def _run_gather(E, N, K, bits, gs, per_expert, M=1, B=5, xdt="bf16", sidecar="bf16", seed=0):
    qw = QWeight(N, K, bits, gs, seed=seed + 100, sidecar=sidecar, experts=E)
    rng = np.random.default_rng(seed)
    x = O.round_bf16(rng.standard_normal((B, M, K), dtype=np.float32))
    if xdt == "f16":
        x = x.astype(np.float16).astype(np.float32)
    lhs, rhs = _pairs(E, per_expert, B, seed)
    y = jq.gather_qmm(to_tensor(x, xdt), qw.dw, qw.ds, qw.db, torch.from_numpy(lhs).cuda(),
                      torch.from_numpy(rhs).cuda(), group_size=gs, bits=bits)
    ref = O.gather_qmm(x, qw.packed, qw.s, qw.b, lhs, rhs, bits, gs)
    assert tuple(y.shape) == (lhs.size, M, N)
    rnd = O.round_bf16 if xdt == "bf16" else (lambda v: v.astype(np.float16).astype(np.float32))
    assert_close(values_of(y), rnd(ref), f"gather b{bits} g{gs} x{per_expert} M{M} {xdt}",
                 out_dtype=xdt)


@pytest.mark.parametrize("bits", [2, 3, 4, 5, 6, 8])
@pytest.mark.parametrize("per_expert", [1, 2, 4])
def test_gather_gemv_bits_tiles(bits, per_expert):
    _run_gather(6, 45, 512, bits, 64, per_expert, seed=bits * 10 + per_expert)


@pytest.mark.parametrize("gs", [32, 64, 128])
@pytest.mark.parametrize("bits", [2, 4])
@pytest.mark.parametrize("dt", ["bf16", "f16"])
def test_gather_gemv_groups_dtypes(gs, bits, dt):
    _run_gather(5, 37, 768, bits, gs, 2, xdt=dt, sidecar=dt, seed=gs + bits)


@pytest.mark.parametrize("bits", [2, 3, 4])
def test_gather_gemv_rows_per_pair(bits):
    """x [B, M, K] with M = 2: plan rows are (pair, row) and map back to out[pair, row]."""
    _run_gather(4, 33, 256, bits, 64, 1, M=2, seed=bits)


@pytest.mark.parametrize("K", [128, 4096, 16384])
@pytest.mark.parametrize("bits", [2, 3])
def test_gather_gemv_wave_splits(K, bits):
    """One wave with idle lanes (K = 128), one to two full waves, eight waves (3-bit 16384)."""
    _run_gather(3, 9, K, bits, 64, 1, B=3, seed=K + bits)


def test_gather_gemv_unbalanced_and_many_tiles():
    """Experts with 1..4 rows in one launch, more items than resident blocks."""
    E, N, K, bits, gs = 4, 700, 512, 3, 64
    qw = QWeight(N, K, bits, gs, seed=5, experts=E)
    rng = np.random.default_rng(5)
    B = 6
    x = O.round_bf16(rng.standard_normal((B, 1, K), dtype=np.float32))
    rhs = np.array([0, 1, 1, 2, 2, 2, 3, 3, 3, 3], np.int32)
    lhs = rng.integers(0, B, size=rhs.size).astype(np.int32)
    y = jq.gather_qmm(to_tensor(x, "bf16"), qw.dw, qw.ds, qw.db, torch.from_numpy(lhs).cuda(),
                      torch.from_numpy(rhs).cuda(), group_size=gs, bits=bits)
    ref = O.gather_qmm(x, qw.packed, qw.s, qw.b, lhs, rhs, bits, gs)
    assert_close(values_of(y), O.round_bf16(ref), "unbalanced experts")


@pytest.mark.parametrize("bits,gs", [(2, 64), (4, 64)])
def test_gather_dec_kernel_band(bits, gs):
    """Ten rows per active expert: above the GEMV's tile range, inside the matrix-core decode
    kernel's (up to two 8-row tiles per expert at gs 64)."""
    _run_gather(4, 40, 256, bits, gs, 10, seed=77)


@pytest.mark.parametrize("T,k,E,gs", [(1, 4, 8, 64), (2, 4, 8, 64), (1, 10, 16, 128),
                                      (3, 4, 6, 64)])
def test_switch_glu_decode(T, k, E, gs):
    """Decode SwitchGLU (gate|up + SiLU fused, then down) on the gather GEMV, config-3 and
    config-5 style group sizes at reduced widths."""
    H, I = 1024, 512
    g = QWeight(I, H, 2, gs, seed=1, experts=E)
    u = QWeight(I, H, 2, gs, seed=2, experts=E)
    d = QWeight(H, I, 2, gs, seed=3, experts=E)
    rng = np.random.default_rng(T * 31 + k)
    x = O.round_bf16(rng.standard_normal((T, H), dtype=np.float32))
    inds = np.stack([rng.choice(E, size=k, replace=False) for _ in range(T)]).astype(np.int32)
    out = jq.switch_glu(to_tensor(x, "bf16"), torch.from_numpy(inds).cuda(),
                        (g.dw, g.ds, g.db, 2), (u.dw, u.ds, u.db, 2), (d.dw, d.ds, d.db, 2), gs)
    ref, _ = O.switch_glu(x, inds, (g.packed, g.s, g.b, 2), (u.packed, u.s, u.b, 2),
                          (d.packed, d.s, d.b, 2), gs, "bf16")
    assert tuple(out.shape) == (T, k, H)
    assert_close(values_of(out), ref, f"switch_glu decode T{T} k{k}")

"""GPU parity of the vector-ALU decode GEMV (M <= 4) against the oracle.

Covers every lane/wave split the kernel takes (K from one lane chunk up to 512 chunks per row,
with chunk counts that leave lanes of the last wave idle), row counts that are not a multiple
of the rows per block, every width, group size and 16-bit dtype, and the grouped launch.
Tolerances: rel-L2 <= 1e-3 and max-abs <= 2e-2 after rounding to the output dtype; fp32
outputs rel-L2 <= 2e-6."""
import numpy as np
import pytest
import torch

import jangq_amd as jq
from oracle import jangq_oracle as O
from tests._util import QWeight, to_tensor
from tests.test_gpu_matmul import run_case

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("bits", [2, 3, 4, 5, 6, 8])
@pytest.mark.parametrize("M", [1, 2, 3, 4])
def test_gemv_batches(bits, M):
    run_case(M, 45, 1024, bits, 64, seed=bits * 7 + M)


@pytest.mark.parametrize("K", [64, 2080, 4096, 8192, 14336, 16384])
@pytest.mark.parametrize("bits", [2, 3, 6])
def test_gemv_wave_splits(K, bits):
    """1, 2, 4 and 8 waves per block, ragged last wave (2080 = 65 chunks of 32)."""
    gs = 32 if K % 64 else 64
    run_case(1, 19, K, bits, gs, seed=K + bits)


@pytest.mark.parametrize("gs", [32, 64, 128])
@pytest.mark.parametrize("bits", [2, 3, 4, 8])
@pytest.mark.parametrize("dt", ["bf16", "f16"])
def test_gemv_groups_dtypes(gs, bits, dt):
    for M in (1, 2):
        run_case(M, 24, 768, bits, gs, xdt=dt, sidecar=dt, seed=gs + bits + M)


@pytest.mark.parametrize("ydt", ["f32", "bf16", "f16"])
def test_gemv_output_dtypes(ydt):
    run_case(1, 33, 512, 4, 64, seed=3, ydt=ydt)


def test_gemv_fallback_shapes():
    """Shapes outside the kernel's range go to the other kernels: 2-bit K % 64 != 0,
    K beyond 512 chunks, 2-bit M = 3, groups per row not a multiple of 8."""
    run_case(1, 16, 96, 2, 32, seed=1)
    run_case(1, 16, 16384 + 64, 3, 64, seed=2)
    run_case(3, 16, 512, 2, 64, seed=3)
    run_case(1, 21, 64 * 12, 3, 64, seed=4)


@pytest.mark.parametrize("N", [1, 7, 8, 9, 17, 33])
def test_gemv_row_tails(N):
    """Row blocks cut by the end of the matrix (scales window ends exactly at the view)."""
    run_case(1, N, 512, 4, 64, seed=N)
    run_case(2, N, 1024, 3, 128, seed=N + 1)


def test_gemv_grouped_launch():
    K = 2048
    ws = [QWeight(n, K, 3, 64, seed=i) for i, n in enumerate((100, 8, 33))]
    rng = np.random.default_rng(5)
    for M in (1, 2, 4):
        x = O.round_bf16(rng.standard_normal((M, K), dtype=np.float32))
        ys = jq.quantized_matmul_multi(to_tensor(x, "bf16"), [(w.dw, w.ds, w.db, 64, 3) for w in ws])
        for w, y in zip(ws, ys):
            ref = O.round_bf16(O.quantized_matmul(x, w.packed, w.s, w.b, 3, 64))
            got = y.float().cpu().numpy()
            assert O.rel_l2(got, ref) <= 1e-3 and O.max_abs(got, ref) <= 2e-2

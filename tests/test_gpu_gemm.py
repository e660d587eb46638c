"""GPU parity of the prefill matrix-core GEMM (large M) against the oracle.

Covers ragged M and N against the 256 x 256 block tile, K with one or several 16-group
batches of the bias term (and a partial last batch), group sizes 64 and 128, every width on
bf16 and f16 activations, and groups whose scale is zero (or tiny): those run with s = 1 and
codes 0 and must still give b * sum(x). Tolerances: rel-L2 <= 1e-3 and max-abs <= 2e-2 after
rounding to the output dtype; fp32 outputs rel-L2 <= 5e-4 (the kernel rounds each dequantized
weight to f16 once, 2^-11 relative, which leaves about 2e-4 rel-L2 on the outputs)."""
import numpy as np
import pytest
import torch

import jangq_amd as jq
from oracle import jangq_oracle as O
from tests._util import QWeight, assert_close, to_tensor, values_of
from tests.test_gpu_matmul import run_case

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("M,N,K", [(384, 256, 256), (400, 200, 1024), (520, 513, 2048),
                                   (600, 256, 64 * 17), (513, 96, 512)])
@pytest.mark.parametrize("bits", [2, 3, 4, 5, 6])
def test_gemm_shapes_bits(M, N, K, bits):
    run_case(M, N, K, bits, 64, seed=M + N + bits)


@pytest.mark.parametrize("bits", [2, 3, 4, 6, 8])
@pytest.mark.parametrize("gs", [64, 128])
def test_gemm_f16_and_group_sizes(bits, gs):
    run_case(390, 160, 128 * 9, bits, gs, xdt="f16", sidecar="f16", seed=bits + gs)
    if bits != 8:
        run_case(390, 160, 128 * 9, bits, gs, seed=bits + gs + 1)


@pytest.mark.parametrize("bits", [2, 3, 4, 6])
def test_gemm_fp32_output(bits):
    M, N, K, gs = 384, 256, 1024, 64
    qw = QWeight(N, K, bits, gs, seed=7)
    rng = np.random.default_rng(8)
    x = O.round_bf16(rng.standard_normal((M, K), dtype=np.float32))
    y = jq.quantized_matmul(to_tensor(x, "bf16"), qw.dw, qw.ds, qw.db, True, gs, bits,
                            out=torch.empty((M, N), dtype=torch.float32, device="cuda"))
    ref = O.quantized_matmul(x, qw.packed, qw.s, qw.b, bits, gs)
    assert_close(values_of(y), ref, f"fp32 out b{bits}", rel=5e-4, mabs=2e-3)


@pytest.mark.parametrize("scale", [0.0, 1e-35])
def test_gemm_zero_scale_groups(scale):
    """Groups with scale 0 (or below 2^-100) contribute b * sum(x) exactly."""
    M, N, K, bits, gs = 400, 64, 512, 4, 64
    qw = QWeight(N, K, bits, gs, seed=3)
    s = qw.s.copy()
    s[::3, 1::2] = scale  # every third row: odd groups
    s_t = torch.from_numpy(O.f32_to_bf16_bits(s).view(np.int16)).view(torch.bfloat16).cuda()
    rng = np.random.default_rng(4)
    x = O.round_bf16(rng.standard_normal((M, K), dtype=np.float32))
    y = jq.quantized_matmul(to_tensor(x, "bf16"), qw.dw, s_t, qw.db, True, gs, bits)
    ref = O.quantized_matmul(x, qw.packed, O.round_bf16(s), qw.b, bits, gs)
    assert_close(values_of(y), O.round_bf16(ref), "zero-scale groups", exact=ref, out_dtype="bf16")


def test_gemm_c4_shape_slice():
    """Config-4 geometry (K = 4096, N = 14336) on a 512-row slice, 4- and 3-bit."""
    for bits in (4, 3):
        run_case(512, 14336, 4096, bits, 64, seed=400 + bits)


@pytest.mark.parametrize("ydt", ["f32", "bf16"])
def test_gemm_row_and_column_ranges(ydt):
    """Activation rows and weight rows far outside f16's range (x scaled by 2^-40 .. 2^100,
    a weight row's scales and biases by 2^-30 .. 2^20): the per-row powers of two that bring
    them into f16 must leave every output at the north-star accuracy once the known scales are
    divided out."""
    M, N, K, bits, gs = 400, 160, 1024, 4, 64
    qw = QWeight(N, K, bits, gs, seed=31)
    rng = np.random.default_rng(32)
    xs = np.ones(M)
    xs[::5] = 2.0 ** -40
    xs[1::5] = 2.0 ** 100
    xs[2::7] = 2.0 ** 30
    ws = np.ones(N)
    ws[::4] = 2.0 ** -30
    ws[1::6] = 2.0 ** 20
    x = O.round_bf16(rng.standard_normal((M, K), dtype=np.float32)) * xs[:, None].astype(np.float32)
    s = (qw.s * ws[:, None]).astype(np.float32)  # powers of two: exact in bf16
    b = (qw.b * ws[:, None]).astype(np.float32)
    bits16 = lambda a: torch.from_numpy(O.f32_to_bf16_bits(a).view(np.int16)).view(torch.bfloat16).cuda()
    out = torch.empty((M, N), dtype={"f32": torch.float32, "bf16": torch.bfloat16}[ydt], device="cuda")
    y = jq.quantized_matmul(to_tensor(x, "bf16"), qw.dw, bits16(s), bits16(b), True, gs, bits, out=out)
    ref = O.quantized_matmul(x, qw.packed, s, b, bits, gs)
    norm = xs[:, None] * ws[None, :]
    got = values_of(y).astype(np.float64) / norm
    want = ref / norm
    if ydt == "bf16":
        want_r = O.round_bf16(ref).astype(np.float64) / norm
        assert_close(got, want_r, "ranges bf16", exact=want, out_dtype="bf16")
    else:
        assert_close(got, want, "ranges f32", rel=5e-4, mabs=2e-3)

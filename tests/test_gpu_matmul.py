"""GPU parity of quantized_matmul (decode GEMV and matrix-core GEMM) against the oracle.

Outputs are compared with the oracle's fp64 accumulation of the exactly dequantized
weights: rel-L2 <= 1e-3 against it rounded to the output dtype, max-abs <= 2e-2 against it
beyond the output's own rounding (half an ulp of the output dtype) (north star);
fp32 outputs are held to rel-L2 <= 2e-6 (1e-4 on the prefill GEMM path)."""
import json
from pathlib import Path

import numpy as np
import pytest
import torch

import jangq_amd as jq
from jangq_amd import _lib
from oracle import jangq_oracle as O
from tests._util import QWeight, assert_close, codes_tensor, to_tensor, values_of

pytestmark = pytest.mark.gpu
GOLD = Path(__file__).resolve().parent / "golden"


# Activation rows from which quantized_matmul runs the prefill GEMM (group sizes 64/128),
# whose fp32 outputs carry the bf16 high/low split of its bias term (~2^-17 relative).
GEMM_MIN_ROWS = 384


def run_case(M, N, K, bits, gs, xdt="bf16", sidecar="bf16", seed=0, ydt=None):
    qw = QWeight(N, K, bits, gs, seed=seed, sidecar=sidecar)
    rng = np.random.default_rng(seed + 1)
    x = O.round_to(rng.standard_normal((M, K), dtype=np.float32), xdt)
    tx = to_tensor(x, xdt)
    out = None
    if ydt is not None:
        out = torch.empty((M, N), dtype={"f32": torch.float32, "bf16": torch.bfloat16,
                                          "f16": torch.float16}[ydt], device="cuda")
    y = jq.quantized_matmul(tx, qw.dw, qw.ds, qw.db, True, gs, bits, out=out)
    ref = O.quantized_matmul(x, qw.packed, qw.s, qw.b, bits, gs)
    ydt = ydt or xdt
    if ydt == "f32":
        gemm = M >= GEMM_MIN_ROWS and gs in (64, 128)
        return assert_close(values_of(y), ref, f"M{M} N{N} K{K} b{bits} g{gs}",
                            rel=5e-4 if gemm else 2e-6, mabs=2e-3 if gemm else 1e-4)
    return assert_close(values_of(y), O.round_to(ref, ydt), f"M{M} N{N} K{K} b{bits} g{gs} {xdt}",
                        exact=ref, out_dtype=ydt)


@pytest.mark.parametrize("bits", [2, 3, 4, 5, 6, 8])
@pytest.mark.parametrize("gs", [32, 64, 128])
@pytest.mark.parametrize("M", [1, 3, 8, 32])
def test_matmul_bits_groups(bits, gs, M):
    run_case(M, 96, 512, bits, gs, seed=bits * 10 + gs + M)


@pytest.mark.parametrize("gs,tpb", [(32, 4), (64, 8), (128, 16)])
@pytest.mark.parametrize("bits", [2, 3, 4, 6, 8])
def test_decode_kernel_token_limits(gs, tpb, bits):
    """Largest batch on the decode matrix-core kernel (tokens per block = 16 / (128/gs)) and
    one more (next kernel), bf16 and f16 activations."""
    for M in (1, tpb, tpb + 1):
        run_case(M, 48, 384, bits, gs, seed=M * 31 + bits)
        run_case(M, 40, 256, bits, gs, xdt="f16", sidecar="f16", seed=M * 37 + bits)


@pytest.mark.parametrize("M", [1, 2, 4, 5, 16, 17, 64, 130])
def test_matmul_m_sweep_fp32_out(M):
    run_case(M, 200, 1024, 4, 64, seed=M, ydt="f32")


@pytest.mark.parametrize("xdt", ["f16", "f32"])
@pytest.mark.parametrize("M", [1, 6, 40])
def test_matmul_activation_dtypes(xdt, M):
    run_case(M, 64, 256, 3, 64, xdt=xdt, sidecar="f16", seed=M + 5)


@pytest.mark.parametrize("M,K,gs", [(9, 320, 64), (6, 96, 32), (2, 64, 64)])
def test_matmul_k_not_multiple_of_tile(M, K, gs):
    run_case(M, 48, K, 6, gs, seed=K)


def test_matmul_empty_and_zero_k():
    qw = QWeight(8, 64, 4, 64, seed=1)
    x = torch.zeros((0, 64), dtype=torch.bfloat16, device="cuda")
    assert jq.quantized_matmul(x, qw.dw, qw.ds, qw.db).shape == (0, 8)


def test_matmul_mlx_fixture():
    """The reference's MLX fixture: 4-bit, gs64, f16 x and sidecars, 64 -> 128."""
    from safetensors.numpy import load_file

    d = load_file(str(GOLD / "matmul_4bit_64x128.safetensors"))
    x = torch.from_numpy(d["x"][None]).cuda()
    w = codes_tensor(d["W.weight"])
    s = torch.from_numpy(d["W.scales"]).cuda()
    b = torch.from_numpy(d["W.biases"]).cuda()
    y = jq.quantized_matmul(x, w, s, b, True, 64, 4, out=torch.empty((1, 128), device="cuda"))
    got = values_of(y)[0]
    assert O.max_abs(got, d["y_ref"]) < 1e-2  # QuantizedMatmul4Tests.swift:83-84
    ref = O.quantized_matmul(d["x"].astype(np.float32)[None], d["W.weight"],
                             d["W.scales"].astype(np.float32), d["W.biases"].astype(np.float32), 4, 64)
    assert O.rel_l2(got, ref[0]) < 2e-6


@pytest.mark.parametrize("M", [1, 8, 32])
def test_c1_full_size(M):
    """Config 1 shape: 4096 x 4096, 4-bit g64 (and the decode batches of config 2)."""
    run_case(M, 4096, 4096, 4, 64, seed=101 + M)


@pytest.mark.parametrize("N,K,bits", [(14336, 4096, 3), (4096, 14336, 2), (1024, 4096, 6)])
def test_c2_projection_shapes(N, K, bits):
    run_case(1, N, K, bits, 64, seed=N + bits)
    run_case(8, N, K, bits, 64, seed=N + bits + 1)


@pytest.mark.parametrize("M", [3, 4])
@pytest.mark.parametrize("N,bits,gs", [(14336, 3, 64), (9000, 4, 128), (4096, 6, 64)])
def test_small_batches_long_outputs(M, N, bits, gs):
    """3-4 activation rows: outputs of more than 8192 rows take the matrix-core kernel, shorter
    ones the vector GEMV; both against the oracle."""
    run_case(M, N, 4096, bits, gs, seed=M * 31 + N + bits)


@pytest.mark.parametrize("bits", [2, 3, 4, 5, 6, 8])
@pytest.mark.parametrize("gs", [32, 64, 128])
def test_long_row_decode_batches(bits, gs):
    """Decode batches of long rows (K >= 8192: the 4x4x4 matrix-core GEMV, passes of 4 or 8
    rows; wider codes at K = 12288 fall to the persistent kernel), ragged N, bf16 and f16."""
    for M, N, K in ((5, 44, 8192), (8, 37, 8192), (13, 21, 12288)):
        run_case(M, N, K, bits, gs, seed=M * 7 + bits + gs)
    run_case(6, 30, 8192, bits, gs, xdt="f16", sidecar="f16", seed=bits + gs)


@pytest.mark.parametrize("M", [5, 8, 16, 32, 64])
def test_c2_down_projection_batches(M):
    """Config 2 down projection (4096 x 14336, 2-bit) at decode batches 5 to 64: K split in
    chunks over the matrix-core kernel, fp32 partials summed in a workspace."""
    run_case(M, 4096, 14336, 2, 64, seed=900 + M)


@pytest.mark.parametrize("M,N,K,bits,gs,xdt", [(8, 100, 6144, 3, 64, "bf16"),
                                               (16, 37, 8192, 6, 128, "f16"),
                                               (24, 64, 12288, 4, 64, "bf16"),
                                               (9, 48, 16384, 8, 128, "bf16")])
def test_long_row_split_k(M, N, K, bits, gs, xdt):
    """The workspace form directly: chunked K (2 to 4 chunks), ragged N, both passes."""
    qw = QWeight(N, K, bits, gs, seed=M + K, sidecar=xdt)
    rng = np.random.default_rng(K + M)
    x = O.round_to(rng.standard_normal((M, K), dtype=np.float32), xdt)
    lib = _lib.lib()
    code = {"bf16": 1, "f16": 2}[xdt]
    nws = lib.jq_quantized_matmul_workspace_size(M, N, K, bits, gs, code, code)
    assert nws > 0
    tx = to_tensor(x, xdt)
    y = torch.empty((M, N), dtype=tx.dtype, device="cuda")
    ws = torch.empty(nws, dtype=torch.uint8, device="cuda")
    st = lib.jq_quantized_matmul_ws(tx.data_ptr(), code, qw.dw.data_ptr(), qw.ds.data_ptr(),
                                    qw.db.data_ptr(), code, bits, gs, M, N, K, y.data_ptr(), code,
                                    ws.data_ptr(), nws, torch.cuda.current_stream().cuda_stream)
    assert st == 0
    assert lib.jq_quantized_matmul_ws(tx.data_ptr(), code, qw.dw.data_ptr(), qw.ds.data_ptr(),
                                      qw.db.data_ptr(), code, bits, gs, M, N, K, y.data_ptr(),
                                      code, ws.data_ptr(), nws - 1,
                                      torch.cuda.current_stream().cuda_stream) == -7
    ref = O.quantized_matmul(x, qw.packed, qw.s, qw.b, bits, gs)
    assert_close(values_of(y), O.round_to(ref, xdt), f"split-K M{M} K{K} b{bits} g{gs}",
                 exact=ref, out_dtype=xdt)


def test_multi_matches_single():
    K = 1024
    ws = [QWeight(n, K, 6, 64, seed=i) for i, n in enumerate((256, 64, 64))]
    rng = np.random.default_rng(77)
    for M in (1, 3, 8):
        x = O.round_bf16(rng.standard_normal((M, K), dtype=np.float32))
        tx = to_tensor(x, "bf16")
        ys = jq.quantized_matmul_multi(tx, [(w.dw, w.ds, w.db, 64, 6) for w in ws])
        for w, y in zip(ws, ys):
            single = jq.quantized_matmul(tx, w.dw, w.ds, w.db, True, 64, 6)
            assert torch.equal(y, single)


def test_operator_argument_checks():
    """Outputs of the wrong shape, dtype, layout or alignment, and biases whose dtype is not the
    scales', are rejected before any launch."""
    qw = QWeight(64, 256, 4, 64, seed=3)
    x = torch.zeros((2, 256), dtype=torch.bfloat16, device="cuda")
    for bad in (torch.empty((2, 63), dtype=torch.bfloat16, device="cuda"),
                torch.empty((64, 2), dtype=torch.bfloat16, device="cuda").t(),
                torch.empty(2 * 64 + 1, dtype=torch.bfloat16, device="cuda")[1:].view(2, 64),
                torch.empty((2, 64), dtype=torch.bfloat16)):
        with pytest.raises(ValueError):
            jq.quantized_matmul(x, qw.dw, qw.ds, qw.db, True, 64, 4, out=bad)
    with pytest.raises(ValueError):
        jq.quantized_matmul(x, qw.dw, qw.ds, qw.db.float(), True, 64, 4)
    with pytest.raises(ValueError):
        jq.quantized_matmul_multi(x, [(qw.dw, qw.ds, qw.db, 64, 4)],
                                  outs=[torch.empty((2, 65), dtype=torch.bfloat16, device="cuda")])
    with pytest.raises(ValueError):
        jq.quantized_matmul_multi(x, [(qw.dw, qw.ds, qw.db.half(), 64, 4)])
    st = QWeight(32, 256, 2, 64, seed=4, experts=4)
    with pytest.raises(ValueError):
        jq.gather_qmm(x[:, None, :], st.dw, st.ds, st.db.float(),
                      rhs_indices=torch.zeros(2, dtype=torch.int32, device="cuda"),
                      group_size=64, bits=2)
    d = QWeight(256, 32, 2, 32, seed=5, experts=4)
    idx = torch.zeros((2, 1), dtype=torch.int32, device="cuda")
    with pytest.raises(ValueError):  # down at group 32 with gate/up at 64
        jq.switch_glu(x, idx, (st.dw, st.ds, st.db, 2), (st.dw, st.ds, st.db, 2),
                      (d.dw, d.ds, d.db, 2), 64)


@pytest.mark.parametrize("sdt", ["f32", "bf16"])
@pytest.mark.parametrize("xdt", ["f32", "bf16"])
def test_quantized_swiglu_decode_dtypes(xdt, sdt):
    """One activation row with f32 activations or f32 scales (outside the one-launch decode
    forms) still runs: the up projection's scratch is always passed."""
    N, K, gs = 96, 512, 64
    g = QWeight(N, K, 4, gs, seed=11, sidecar=sdt)
    u = QWeight(N, K, 4, gs, seed=12, sidecar=sdt)
    rng = np.random.default_rng(13)
    x = O.round_to(rng.standard_normal((1, K), dtype=np.float32), xdt)
    h = jq.quantized_swiglu(to_tensor(x, xdt), (g.dw, g.ds, g.db, 4), (u.dw, u.ds, u.db, 4), gs)
    ref = O.swiglu_pair(x, (g.packed, g.s, g.b, 4), (u.packed, u.s, u.b, 4), gs, xdt)
    tol = dict(rel=2e-6, mabs=1e-4) if xdt == "f32" else {}
    assert_close(values_of(h), ref, f"swiglu x {xdt} scales {sdt}", **tol)

"""GPU parity of the codec kernels (unpack, dequantize, quantize): bit-exact vs the oracle."""
import numpy as np
import pytest
import torch

import jangq_amd as jq
from oracle import jangq_oracle as O
from tests._util import QWeight, codes_tensor, sidecar_tensor, to_tensor, values_of

pytestmark = pytest.mark.gpu

BITS = [2, 3, 4, 5, 6, 8]


@pytest.mark.parametrize("bits", BITS)
@pytest.mark.parametrize("rows,K", [(1, 32), (3, 96), (17, 4096)])
def test_unpack_bit_exact(bits, rows, K):
    rng = np.random.default_rng(rows * 131 + K + bits)
    codes = rng.integers(0, 1 << bits, size=(rows, K), dtype=np.uint8)
    packed = O.pack_rows(codes, bits)
    got = jq.unpack(codes_tensor(packed), bits).cpu().numpy()
    np.testing.assert_array_equal(got, codes)


@pytest.mark.parametrize("bits", BITS)
@pytest.mark.parametrize("gs", [32, 64, 128])
@pytest.mark.parametrize("sidecar", ["bf16", "f16", "f32"])
def test_dequantize_bit_exact(bits, gs, sidecar):
    qw = QWeight(33, 512, bits, gs, seed=bits * 7 + gs, sidecar=sidecar)
    ref = qw.dequant()
    for out_dt, tdt in (("f32", torch.float32), ("bf16", torch.bfloat16), ("f16", torch.float16)):
        got = jq.dequantize(qw.dw, qw.ds, qw.db, gs, bits, dtype=tdt)
        want = O.round_to(ref, out_dt)
        g = values_of(got)
        assert np.array_equal(g.view(np.uint32), want.view(np.uint32)), (
            f"{bits}-bit gs{gs} {sidecar}->{out_dt}: {(g != want).sum()} mismatches")


def test_dequantize_expert_stack_and_defaults():
    qw = QWeight(16, 256, 3, 64, seed=3, experts=5)
    got = jq.dequantize(qw.dw, qw.ds, qw.db, 64, 3)  # default dtype = scales dtype (bf16)
    assert got.dtype == torch.bfloat16 and tuple(got.shape) == (5, 16, 256)
    want = O.round_to(qw.dequant(), "bf16")
    assert np.array_equal(values_of(got), want)


@pytest.mark.parametrize("bits", BITS)
@pytest.mark.parametrize("gs", [32, 64, 128])
@pytest.mark.parametrize("wdt", ["bf16", "f16", "f32"])
def test_quantize_bit_exact(bits, gs, wdt):
    rng = np.random.default_rng(bits * 100 + gs)
    w = rng.standard_normal((24, 256)).astype(np.float32) * np.float32(0.02)
    w = O.round_to(w, wdt)
    tw = to_tensor(w, wdt)
    for sidecar, sdt in (("bf16", torch.bfloat16), ("f16", torch.float16)):
        wq, s, b = jq.quantize(tw, gs, bits, scales_dtype=sdt)
        packed, s_ref, b_ref, _ = O.quantize_affine(w, bits, gs, sidecar=sidecar)
        np.testing.assert_array_equal(wq.view(torch.int32).cpu().numpy().view(np.uint32), packed)
        np.testing.assert_array_equal(values_of(s), O.sidecar_f32(s_ref, sidecar))
        np.testing.assert_array_equal(values_of(b), O.sidecar_f32(b_ref, sidecar))


def test_quantize_edge_groups():
    """Zero, constant, all-negative, all-positive and sub-eps groups (the at_zero and eps
    branches of affine.py:236-249) match the oracle bit for bit."""
    K = 64
    rows = np.stack([
        np.zeros(K), np.full(K, 0.5), np.full(K, -0.25), -np.abs(np.linspace(0.01, 1, K)),
        np.abs(np.linspace(0.01, 1, K)), np.linspace(-3e-8, 3e-8, K), np.linspace(-1, 1, K),
        np.r_[np.full(K - 1, 1e-3), -2.0],
    ]).astype(np.float32)
    for bits in BITS:
        for sidecar, sdt in (("bf16", torch.bfloat16), ("f16", torch.float16)):
            wq, s, b = jq.quantize(to_tensor(rows, "f32"), 64, bits, scales_dtype=sdt)
            packed, s_ref, b_ref, _ = O.quantize_affine(rows, bits, 64, sidecar=sidecar)
            np.testing.assert_array_equal(wq.view(torch.int32).cpu().numpy().view(np.uint32), packed)
            np.testing.assert_array_equal(values_of(s), O.sidecar_f32(s_ref, sidecar))
            np.testing.assert_array_equal(values_of(b), O.sidecar_f32(b_ref, sidecar))


def test_quantize_dequantize_roundtrip_full_size():
    """C1 shape (4096 x 4096, 4-bit g64): GPU quantize -> GPU dequantize equals the oracle's
    dequantization of the oracle's quantization (size-independent round-trip property)."""
    rng = np.random.default_rng(101)
    w = O.round_bf16(rng.standard_normal((4096, 4096), dtype=np.float32) * np.float32(0.02))
    wq, s, b = jq.quantize(to_tensor(w, "bf16"), 64, 4)
    deq = jq.dequantize(wq, s, b, 64, 4, dtype=torch.float32)
    packed, s_ref, b_ref, _ = O.quantize_affine(w, 4, 64, sidecar="bf16")
    ref = O.dequantize_affine(packed, O.sidecar_f32(s_ref, "bf16"), O.sidecar_f32(b_ref, "bf16"), 4, 64)
    assert np.array_equal(values_of(deq), ref)


@pytest.mark.parametrize("rows,P", [(1, 1), (37, 5), (4096, 64)])
def test_expand_1bit_to_2bit(rows, P):
    """1-bit storage -> 2-bit runtime codes (affine.py:402-416): bit-exact, and the expanded
    codes dequantize to the 1-bit values q*s + b with the same sidecars."""
    rng = np.random.default_rng(rows + P)
    w = rng.integers(0, 2**32, size=(rows, P), dtype=np.uint64).astype(np.uint32)
    got = jq.expand_packed_1bit_to_2bit(codes_tensor(w))
    assert tuple(got.shape) == (rows, 2 * P)
    np.testing.assert_array_equal(got.view(torch.int32).cpu().numpy().view(np.uint32),
                                  O.expand_1bit_to_2bit(w))
    if rows == 37:
        K = 32 * P
        s = (rng.random((rows, K // 32)) * 0.1).astype(np.float32)
        b = (rng.standard_normal((rows, K // 32)) * 0.1).astype(np.float32)
        deq = jq.dequantize(got, to_tensor(s, "f32"), to_tensor(b, "f32"), 32, 2,
                            dtype=torch.float32)
        q1 = O.unpack_rows(w, 1).astype(np.float32)
        ref = (q1 * np.repeat(s, 32, axis=1)).astype(np.float32) + np.repeat(b, 32, axis=1)
        np.testing.assert_array_equal(values_of(deq), ref)


@pytest.mark.parametrize("bits", BITS)
@pytest.mark.parametrize("shape,bs", [((5, 100), 64), ((4, 256), 128), ((3, 33), 32)])
def test_dequantize_tensor_v1_flat(bits, shape, bs):
    """Flat v1 stream (quantize.py:292-326), f16 sidecars, padded last block: bit-exact."""
    rng = np.random.default_rng(bits * 7 + bs)
    total = int(np.prod(shape))
    n_blocks = -(-total // bs)
    q = O.pack_bits(rng.integers(0, 1 << bits, size=n_blocks * bs), bits)
    s = (rng.random(n_blocks) * 0.1 + 1e-3).astype(np.float16)
    b = (rng.standard_normal(n_blocks) * 0.05).astype(np.float16)
    got = jq.dequantize_tensor(torch.from_numpy(q).cuda(), torch.from_numpy(s).cuda(),
                               torch.from_numpy(b).cuda(), bits, shape, bs)
    assert got.dtype == torch.float32 and tuple(got.shape) == shape
    np.testing.assert_array_equal(values_of(got), O.dequantize_tensor_flat(q, s, b, bits, shape, bs))

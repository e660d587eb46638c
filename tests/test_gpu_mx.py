"""MX modes on the GPU (mxfp4 / mxfp8, group 32, E8M0 scales): dequantization bit-exact to the
oracle in fp32 (and correctly rounded in bf16/f16), the decode GEMV within the matmul
tolerance, the C-ABI's argument checks, and a loaded MX module's forward."""
import numpy as np
import pytest
import torch

import jangq_amd as jq
from jangq_amd import _lib
from oracle import jangq_oracle as O
from tests._util import assert_close, to_tensor, values_of

pytestmark = pytest.mark.gpu


def _mx_weight(rows, K, mode, seed, lo=110, hi=135):
    rng = np.random.default_rng(seed)
    per = 8 if mode == "mxfp4" else 4
    packed = rng.integers(0, 2**32, (rows, K // per), dtype=np.uint64).astype(np.uint32)
    if mode == "mxfp8":  # keep NaN codes (S.1111.111) out of the matmul cases
        by = packed.view(np.uint8)
        by[(by & 0x7F) == 0x7F] = 0x7E
    sc = rng.integers(lo, hi, (rows, K // 32)).astype(np.uint8)
    return packed, sc


def _dev(packed, sc):
    return (torch.from_numpy(packed.view(np.int32)).cuda(), torch.from_numpy(sc).cuda())


@pytest.mark.parametrize("mode", ["mxfp4", "mxfp8"])
@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16, torch.float16])
def test_mx_dequantize(mode, dt):
    bits = 4 if mode == "mxfp4" else 8
    packed, sc = _mx_weight(37, 256, mode, 1, lo=100, hi=150)
    w, s = _dev(packed, sc)
    got = jq.dequantize(w, s, None, group_size=32, bits=bits, mode=mode, dtype=dt)
    ref = O.mx_dequantize(packed, sc, mode)
    name = {torch.float32: "f32", torch.bfloat16: "bf16", torch.float16: "f16"}[dt]
    np.testing.assert_array_equal(values_of(got), O.round_to(ref, name))


def test_mx_special_values():
    """NaN code and scale, zero and negative zero, the smallest and largest scales."""
    packed = np.array([[0x7F, 0x80, 0, 0, 0, 0, 0, 0]], dtype=np.uint32)  # mxfp8 bytes 7F 00 00 00, 80 ...
    sc = np.array([[127]], dtype=np.uint8)
    for scale in (0, 1, 127, 254, 255):
        sc[0, 0] = scale
        w, s = _dev(packed, sc)
        got = values_of(jq.dequantize(w, s, None, group_size=32, bits=8, mode="mxfp8",
                                      dtype=torch.float32))
        ref = O.mx_dequantize(packed, sc, "mxfp8")
        np.testing.assert_array_equal(np.isnan(got), np.isnan(ref))
        ok = ~np.isnan(ref)
        np.testing.assert_array_equal(got[ok], ref[ok])
        np.testing.assert_array_equal(np.signbit(got[ok]), np.signbit(ref[ok]))


@pytest.mark.parametrize("mode", ["mxfp4", "mxfp8"])
@pytest.mark.parametrize("M,N,K,xdt", [(1, 4096, 4096, "bf16"), (3, 300, 1056, "bf16"),
                                        (2, 130, 14336, "f16"), (1, 64, 32, "bf16")])
def test_mx_quantized_matmul(mode, M, N, K, xdt):
    bits = 4 if mode == "mxfp4" else 8
    packed, sc = _mx_weight(N, K, mode, M + N + K, lo=112, hi=122)  # outputs within f16 range
    w, s = _dev(packed, sc)
    x = O.round_to(np.random.default_rng(K).standard_normal((M, K), dtype=np.float32), xdt)
    y = jq.quantized_matmul(to_tensor(x, xdt), w, s, None, True, 32, bits, mode)
    exact = O.mx_quantized_matmul(x, packed, sc, mode)
    assert tuple(y.shape) == (M, N)
    assert_close(values_of(y), O.round_to(exact, xdt), f"{mode} M{M} N{N} K{K}", exact=exact,
                 out_dtype=xdt)


def test_mx_abi_checks():
    L = _lib.lib()
    assert L.jq_mx_dequantize(None, None, 5, 1, 32, None, 0, None) == -1    # mode
    assert L.jq_mx_dequantize(None, None, 4, 1, 48, None, 0, None) == -2    # K % 32
    assert L.jq_mx_dequantize(None, None, 4, 1, 32, None, 0, None) == -5    # null
    assert L.jq_mx_quantized_matmul(None, 1, None, None, 4, 1, 8, 32 * 64 * 8 + 32, None, 1,
                                    None) == -3                              # K too long
    assert L.jq_mx_quantized_matmul(None, 0, None, None, 8, 1, 8, 64, None, 1, None) == -4


def test_mx_linear_module():
    """QuantizedLinear in mxfp4 mode (as the loader sets it) runs the MX GEMV."""
    from jangq_amd import nn as jnn
    packed, sc = _mx_weight(96, 512, "mxfp4", 7)
    lin = jnn.QuantizedLinear(512, 96, bits=4, group_size=32, device="cuda")
    lin.weight, lin.scales = _dev(packed, sc)
    lin.biases = None
    lin.bits, lin.group_size, lin.mode = 4, 32, "mxfp4"
    x = O.round_bf16(np.random.default_rng(8).standard_normal((2, 512), dtype=np.float32))
    y = lin(to_tensor(x, "bf16"))
    exact = O.mx_quantized_matmul(x, packed, sc, "mxfp4")
    assert_close(values_of(y), O.round_bf16(exact), "mx linear", exact=exact, out_dtype="bf16")

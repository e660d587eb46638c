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


def _mx_stack(E, N, K, mode, seed, lo=112, hi=122):
    packs, scs = zip(*[_mx_weight(N, K, mode, seed * 100 + e, lo, hi) for e in range(E)])
    return np.stack(packs), np.stack(scs)


@pytest.mark.parametrize("mode", ["mxfp4", "mxfp8"])
@pytest.mark.parametrize("T,k,N,K", [(1, 4, 96, 512), (5, 2, 130, 1056), (3, 3, 64, 4096)])
def test_mx_gather_qmm_decode(mode, T, k, N, K):
    """gather_qmm over an MX expert stack, one activation row per token against each of its
    experts (the SwitchGLU call shape), against the oracle's per-pair products."""
    E = 6
    bits = 4 if mode == "mxfp4" else 8
    packed, sc = _mx_stack(E, N, K, mode, T + k)
    w, s = _dev(packed, sc)
    rng = np.random.default_rng(K + T)
    x = O.round_bf16(rng.standard_normal((T, K), dtype=np.float32))
    idx = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int32)
    xt = to_tensor(x, "bf16").reshape(T, 1, 1, K)
    y = jq.gather_qmm(xt, w, s, None, rhs_indices=torch.from_numpy(idx).cuda(), transpose=True,
                      group_size=32, bits=bits, mode=mode)
    assert tuple(y.shape) == (T, k, 1, N)
    exact = np.stack([np.stack([O.mx_quantized_matmul(x[t:t + 1], packed[idx[t, j]],
                                                       sc[idx[t, j]], mode)[0]
                                for j in range(k)]) for t in range(T)])
    assert_close(values_of(y)[:, :, 0], O.round_bf16(exact), f"mx gather {mode} T{T} k{k}",
                 exact=exact, out_dtype="bf16")


@pytest.mark.parametrize("mode", ["mxfp4", "mxfp8"])
def test_mx_gather_qmm_lhs_rows(mode):
    """Explicit lhs / rhs index lists over a batch of multi-row activations (M = 3): pair i
    multiplies x[lhs[i]] by expert rhs[i]; f16 activations."""
    E, N, K, B, M = 5, 72, 256, 4, 3
    bits = 4 if mode == "mxfp4" else 8
    packed, sc = _mx_stack(E, N, K, mode, 9)
    w, s = _dev(packed, sc)
    x = O.round_to(np.random.default_rng(2).standard_normal((B, M, K), dtype=np.float32), "f16")
    lhs = np.array([0, 3, 3, 1, 2, 0, 1], dtype=np.int32)
    rhs = np.array([4, 0, 2, 2, 1, 3, 0], dtype=np.int32)
    y = jq.gather_qmm(to_tensor(x, "f16"), w, s, None, lhs_indices=torch.from_numpy(lhs).cuda(),
                      rhs_indices=torch.from_numpy(rhs).cuda(), transpose=True, group_size=32,
                      bits=bits, mode=mode)
    assert tuple(y.shape) == (7, M, N) and y.dtype == torch.float16
    exact = np.stack([O.mx_quantized_matmul(x[l], packed[r], sc[r], mode)
                      for l, r in zip(lhs, rhs)])
    assert_close(values_of(y), O.round_to(exact, "f16"), f"mx gather lhs {mode}", exact=exact,
                 out_dtype="f16")


def test_mx_gather_abi_checks():
    L = _lib.lib()
    assert L.jq_mx_gather_qmm(None, 1, 1, 1, None, None, 5, 1, 8, 32, None, None, 1, None, 1,
                              None) == -1                                    # mode
    assert L.jq_mx_gather_qmm(None, 1, 1, 1, None, None, 4, 1, 8, 48, None, None, 1, None, 1,
                              None) == -2                                    # K % 32
    assert L.jq_mx_gather_qmm(None, 1, 1, 1, None, None, 4, 1, 8, 32, None, None, 1, None, 1,
                              None) == -5                                    # null


@pytest.mark.parametrize("dt,name", [(torch.bfloat16, "bf16"), (torch.float16, "f16"),
                                     (torch.float32, "f32")])
@pytest.mark.parametrize("limit", [0.0, 1.5])
def test_swiglu_elementwise(dt, name, limit):
    rng = np.random.default_rng(3)
    g = O.round_to(rng.standard_normal(4099, dtype=np.float32) * 3, name)
    u = O.round_to(rng.standard_normal(4099, dtype=np.float32) * 3, name)
    h = jq.swiglu(to_tensor(g, name), to_tensor(u, name), limit)
    assert h.dtype == dt
    exact = O.glu(g, u, limit)
    got = values_of(h)
    ref = O.round_to(exact, name)
    if name == "f32":
        np.testing.assert_allclose(got, exact, rtol=2e-6, atol=1e-30)
    else:  # one rounding of a value computed in fp32: the correctly rounded one or a neighbour
        assert_close(got, ref, f"swiglu {name} L{limit}", exact=exact, out_dtype=name)


def _mx_switch(E, H, I, mode, seed):
    from jangq_amd import nn as jnn
    bits = 4 if mode == "mxfp4" else 8
    sw = jnn.SwitchGLU(H, I, E, group_size=32, bits=4, device="cuda")
    host = {}
    for i, (name, (n, kk)) in enumerate({"gate_proj": (I, H), "up_proj": (I, H),
                                         "down_proj": (H, I)}.items()):
        packed, sc = _mx_stack(E, n, kk, mode, seed + i)
        p = getattr(sw, name)
        p.weight, p.scales = _dev(packed, sc)
        p.biases = None
        p.bits, p.group_size, p.mode = bits, 32, mode
        host[name] = (packed, sc)
    return sw, host


def _mx_pairs(x, idx, host, mode, limit=0.0):
    """The three gathers of SwitchGLU per pair with bf16 roundings: g, u, h and y."""
    T, k = idx.shape
    out = np.zeros((T, k, host["down_proj"][0].shape[1]))
    for t in range(T):
        for j in range(k):
            e = idx[t, j]
            g = O.round_bf16(O.mx_quantized_matmul(x[t:t + 1], host["gate_proj"][0][e],
                                                   host["gate_proj"][1][e], mode))
            u = O.round_bf16(O.mx_quantized_matmul(x[t:t + 1], host["up_proj"][0][e],
                                                   host["up_proj"][1][e], mode))
            h = O.round_bf16(O.glu(g, u, limit))
            out[t, j] = O.mx_quantized_matmul(h, host["down_proj"][0][e],
                                              host["down_proj"][1][e], mode)[0]
    return out


@pytest.mark.parametrize("mode", ["mxfp4", "mxfp8"])
def test_mx_switch_glu(mode):
    E, H, I, T, k = 8, 256, 128, 3, 2
    sw, host = _mx_switch(E, H, I, mode, 20)
    rng = np.random.default_rng(5)
    x = O.round_bf16(rng.standard_normal((T, H), dtype=np.float32))
    idx = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int32)
    y = sw(to_tensor(x, "bf16"), torch.from_numpy(idx).cuda())
    assert tuple(y.shape) == (T, k, H)
    exact = _mx_pairs(x, idx, host, mode)
    assert_close(values_of(y), O.round_bf16(exact), f"mx switch_glu {mode}", exact=exact,
                 out_dtype="bf16", ulps=1)


def test_mx_sparse_moe_block():
    """A SparseMoeBlock whose experts load as mxfp4 runs routing, the three MX gathers and
    the after-down combine (mlx_lm order: round(sum_j w_j y_j) + shared)."""
    from jangq_amd import nn as jnn
    E, H, I, T, k = 8, 256, 128, 4, 2
    blk = jnn.SparseMoeBlock(H, I, E, k, group_size=64, bits=2, router_bits=8, device="cuda")
    sw, host = _mx_switch(E, H, I, "mxfp4", 30)
    blk.switch_mlp = sw
    rng = np.random.default_rng(6)
    gw = O.round_bf16(rng.standard_normal((E, H), dtype=np.float32) * 0.05)
    blk.gate = jnn.DenseRouter(H, E, device="cuda")
    with torch.no_grad():
        blk.gate.weight.copy_(torch.from_numpy(gw))
    x = O.round_bf16(rng.standard_normal((T, H), dtype=np.float32))
    y = blk(to_tensor(x, "bf16"))
    # a float32 router gate: fp32 logits (bf16 x promoted), no bf16 rounding
    logits = (x.astype(np.float64) @ gw.T.astype(np.float64)).astype(np.float32)
    idx, sc = O.route_topk(logits, k)
    ys = O.round_bf16(_mx_pairs(x, idx, host, "mxfp4"))
    exact = (ys.astype(np.float64) * sc[..., None]).sum(1)
    assert_close(values_of(y), O.round_bf16(exact), "mx moe block", exact=exact,
                 out_dtype="bf16", ulps=1)

"""Pins the CPU oracle (oracle/jangq_oracle.py, oracle/jq_oracle.c) before it is trusted as
the checker of the GPU kernels. CPU only.

Sources of truth, in order:
  * known answers of the reference's own tests (jang-tools/tests/test_pack.py:33-61) and
    their round-trip recipes (seeds 42 / 123 / 999, test_pack.py:11-22,63-87);
  * the MLX-produced fixture jang-runtime/Tests/JANGCoreMetalTests/fixtures/
    matmul_4bit_64x128.safetensors, regenerated from its recorded seed
    (jang-tools/scripts/gen_matmul_fixture.py:33-46);
  * closed forms and brute force (Python big-int bit streams, pure-Python loops);
  * agreement of two independent restatements (numpy vs bit-by-bit C).
Planted-mistake checks show each pin would catch a plausible error.
"""
import ctypes
import json
from pathlib import Path

import zlib

import numpy as np
import pytest
import torch

from oracle import jangq_oracle as O

GOLD = Path(__file__).resolve().parent / "golden"


def _bigint_stream(values, bits):
    """LSB-first definition with Python integers: value i at bit i*bits."""
    acc = 0
    for i, v in enumerate(values):
        acc |= int(v) << (i * bits)
    nbytes = (len(values) * bits + 7) // 8
    return list(acc.to_bytes(nbytes, "little"))


# ----------------------------------------------------------------------------- packing


def test_pack_known_answers_from_reference_tests():
    # jang-tools/tests/test_pack.py:33-44 (2-bit), :46-52 (1-bit), :54-61 (4-bit)
    assert O.pack_bits([0, 1, 2, 3, 0, 1, 2, 3], 2).tolist() == [0xE4, 0xE4]
    assert O.pack_bits([0, 1, 0, 1, 1, 0, 1, 0], 1).tolist() == [0b01011010]
    assert O.pack_bits([5, 10, 3, 15], 4).tolist() == [0xA5, 0xF3]
    np.testing.assert_array_equal(O.unpack_bits(np.array([0xE4, 0xE4], np.uint8), 2, 8),
                                  [0, 1, 2, 3, 0, 1, 2, 3])


def test_pack_word_straddling_vectors():
    # 3-bit: codes 2 and 5 cross byte boundaries; LSB-first value 0x8B03DD.
    assert O.pack_bits([5, 3, 7, 1, 0, 6, 2, 4], 3).tolist() == [0xDD, 0x03, 0x8B]
    # 6-bit: 63 | 42<<12 | 21<<18 = 0x56A03F.
    assert O.pack_bits([63, 0, 42, 21], 6).tolist() == [0x3F, 0xA0, 0x56]
    # Codes crossing uint32 words in a 3/5/6-bit row agree with the big-int definition.
    rng = np.random.default_rng(7)
    for bits in (3, 5, 6):
        vals = rng.integers(0, 1 << bits, size=96)
        assert O.pack_bits(vals, bits).tolist() == _bigint_stream(vals, bits)


def test_known_answers_catch_msb_first_packing():
    """Planted mistake: an MSB-first packer fails the reference known answers."""
    def msb_first(values, bits):
        v = np.asarray(values, np.uint64)
        planes = ((v[:, None] >> np.arange(bits - 1, -1, -1, dtype=np.uint64)) & 1).astype(np.uint8)
        return np.packbits(planes.reshape(-1), bitorder="big")
    assert msb_first([5, 10, 3, 15], 4).tolist() != [0xA5, 0xF3]
    assert msb_first([5, 3, 7, 1, 0, 6, 2, 4], 3).tolist() != [0xDD, 0x03, 0x8B]


@pytest.mark.parametrize("bits", [1, 2, 3, 4, 5, 6, 8])
@pytest.mark.parametrize("seed,n", [(42, 64), (123, 64), (999, 6400)])
def test_roundtrip_reference_recipes(bits, seed, n):
    # test_pack.py:11-22 / 63-74 / 76-87
    rng = np.random.default_rng(seed)
    values = rng.integers(0, (1 << bits), size=n, dtype=np.uint8)
    packed = O.pack_bits(values, bits)
    assert len(packed) == (n * bits + 7) // 8  # test_pack.py:24-31
    np.testing.assert_array_equal(O.unpack_bits(packed, bits, n), values)


@pytest.mark.parametrize("bits", [1, 2, 3, 4, 5, 6, 8])
def test_max_and_zero_values(bits):
    for fill in (0, (1 << bits) - 1):  # test_pack.py:89-104
        v = np.full(64, fill, dtype=np.uint8)
        np.testing.assert_array_equal(O.unpack_bits(O.pack_bits(v, bits), bits, 64), v)


def test_unpack_flattens_packed_matrix_view():
    values = np.array([0, 1] * 32, dtype=np.uint8)  # test_pack.py:106-110
    np.testing.assert_array_equal(O.unpack_bits(O.pack_bits(values, 1).reshape(2, 4), 1, 64), values)


@pytest.mark.parametrize("bits", [2, 3, 4, 5, 6, 8])
def test_numpy_and_bitwise_c_restatements_agree(bits, c_oracle):
    rng = np.random.default_rng(100 + bits)
    rows, K = 7, 256
    codes = rng.integers(0, 1 << bits, size=(rows, K), dtype=np.uint8)
    packed = O.pack_rows(codes, bits)
    w_c = np.zeros_like(packed)
    c_oracle.jqo_pack(codes.ctypes.data, bits, rows, K, w_c.ctypes.data)
    np.testing.assert_array_equal(w_c, packed)
    out = np.zeros((rows, K), np.uint8)
    c_oracle.jqo_unpack(packed.ctypes.data, bits, rows, K, out.ctypes.data)
    np.testing.assert_array_equal(out, codes)
    np.testing.assert_array_equal(O.unpack_rows(packed, bits), codes)


# ----------------------------------------------------------------------------- MLX fixture


def _fixture():
    from safetensors.numpy import load_file

    d = load_file(str(GOLD / "matmul_4bit_64x128.safetensors"))
    info = json.loads((GOLD / "fixture_info.json").read_text())
    rng = np.random.default_rng(info["seed"])  # gen_matmul_fixture.py:33-35
    W = rng.standard_normal((info["out_features"], info["in_features"])).astype(np.float32)
    x = rng.standard_normal((info["in_features"],)).astype(np.float16)
    return d, info, W, x


def test_fixture_inputs_regenerate_from_seed():
    d, info, W, x = _fixture()
    np.testing.assert_array_equal(x, d["x"])
    assert info["bits"] == 4 and info["group_size"] == 64


def test_quantizer_reproduces_mlx_codes_and_sidecars():
    """mx.quantize output stored by the reference: codes and f16-cast sidecars bit-equal."""
    d, info, W, _ = _fixture()
    packed, s, b, _ = O.quantize_affine(W, info["bits"], info["group_size"], sidecar="f32")
    np.testing.assert_array_equal(packed, d["W.weight"])
    np.testing.assert_array_equal(s.astype(np.float16), d["W.scales"])
    np.testing.assert_array_equal(b.astype(np.float16), d["W.biases"])


def test_dequant_matmul_reproduces_mlx_y_ref():
    """y_ref = mx.dequantize(q, s, b) @ x with MLX's fp32 sidecars (gen_matmul_fixture.py:44-46)."""
    d, info, W, x = _fixture()
    packed, s, b, _ = O.quantize_affine(W, 4, 64, sidecar="f32")
    y = O.quantized_matmul(x.astype(np.float32)[None], packed, s, b, 4, 64)[0]
    assert O.rel_l2(y, d["y_ref"]) < 1e-6
    assert O.max_abs(y, d["y_ref"]) < 1e-4
    # With the stored f16 sidecars: the reference's own acceptance bound (1e-2,
    # QuantizedMatmul4Tests.swift:83-84).
    y16 = O.quantized_matmul(x.astype(np.float32)[None], d["W.weight"],
                             d["W.scales"].astype(np.float32), d["W.biases"].astype(np.float32),
                             4, 64)[0]
    assert O.max_abs(y16, d["y_ref"]) < 1e-2


def test_fixture_catches_wrong_sign_convention():
    """Planted mistake: always-positive scale (bias = min) gives different codes."""
    d, info, W, _ = _fixture()
    g = W.reshape(128, 1, 64)
    lo, hi = g.min(-1), np.maximum(g.max(-1), 0)
    s = (hi - lo) / 15
    codes = np.clip(np.rint((g - lo[..., None]) / s[..., None]), 0, 15).astype(np.uint8)
    assert not np.array_equal(O.pack_rows(codes.reshape(128, 64), 4), d["W.weight"])


# ----------------------------------------------------------------------------- dequant


@pytest.mark.parametrize("bits", [2, 3, 4, 5, 6, 8])
def test_dequant_identity_scale_returns_codes(bits):
    # jang_tools/jangh/tests/test_jangtq2.py:19-24: dequantize(s=1, b=0) == q
    rng = np.random.default_rng(bits)
    codes = rng.integers(0, 1 << bits, size=(4, 128), dtype=np.uint8)
    packed = O.pack_rows(codes, bits)
    ones = np.ones((4, 2), np.float32)
    np.testing.assert_array_equal(O.dequantize_affine(packed, ones, 0 * ones, bits, 64), codes)


def test_dequant_rounds_product_and_sum_separately(c_oracle):
    """fl(fl(q*s)+b) (numpy's q*s + b, affine.py:458-463) differs from a fused FMA on some
    elements; the oracle and the C restatement agree with the two-rounding form."""
    rng = np.random.default_rng(5)
    rows, K, gs = 64, 256, 64
    codes = rng.integers(0, 16, size=(rows, K), dtype=np.uint8)
    packed = O.pack_rows(codes, 4)
    s = rng.standard_normal((rows, K // gs)).astype(np.float32) * np.float32(0.013)
    b = rng.standard_normal((rows, K // gs)).astype(np.float32) * np.float32(0.07)
    deq = O.dequantize_affine(packed, s, b, 4, gs)
    q = codes.astype(np.float32).reshape(rows, -1, gs)
    two = (np.float32(1) * (q * s[..., None]).astype(np.float32) + b[..., None]).reshape(rows, K)
    fused = (q.astype(np.float64) * s[..., None] + b[..., None]).astype(np.float32).reshape(rows, K)
    np.testing.assert_array_equal(deq, two)
    assert (fused != two).any(), "test inputs do not discriminate fused from two roundings"
    out = np.zeros((rows, K), np.float32)
    c_oracle.jqo_dequant(packed.ctypes.data, s.ctypes.data, b.ctypes.data, 4, gs, rows, K,
                         out.ctypes.data)
    np.testing.assert_array_equal(out, deq)


@pytest.mark.parametrize("bits", [2, 3, 6, 8])
def test_dequant_stacked_experts_flatten(bits):
    rng = np.random.default_rng(11)
    w = O.round_bf16(rng.standard_normal((3 * 8, 128)).astype(np.float32) * 0.02)
    packed, s, b, _ = O.quantize_affine(w, bits, 32)
    flat = O.dequantize_affine(packed, O.sidecar_f32(s, "bf16"), O.sidecar_f32(b, "bf16"), bits, 32)
    stacked = O.dequantize_affine(packed.reshape(3, 8, -1), O.sidecar_f32(s, "bf16").reshape(3, 8, -1),
                                  O.sidecar_f32(b, "bf16").reshape(3, 8, -1), bits, 32)
    np.testing.assert_array_equal(stacked.reshape(24, 128), flat)


@pytest.mark.parametrize("bits", [2, 3, 4, 5, 6, 8])
@pytest.mark.parametrize("gs", [32, 64, 128])
def test_quantizer_invariants(bits, gs):
    rng = np.random.default_rng(bits * 1000 + gs)
    w = O.round_bf16(rng.standard_normal((16, 256)).astype(np.float32) * 0.02)
    packed, s, b, codes = O.quantize_affine(w, bits, gs, sidecar="f32")
    assert codes.max() <= (1 << bits) - 1
    np.testing.assert_array_equal(O.unpack_rows(packed, bits), codes)
    deq = O.dequantize_affine(packed, s, b, bits, gs).reshape(16, -1, gs)
    err = np.abs(deq - w.reshape(16, -1, gs))
    # unclipped codes reconstruct within half a step; the refined scale may clip the
    # non-dominant edge to 2^b - 1 (affine.py:240-252)
    unclipped = codes.reshape(16, -1, gs) < (1 << bits) - 1
    bound = np.abs(s)[..., None] * 0.5 * (1 + 1e-5) + 1e-7
    assert np.all((err <= bound) | ~unclipped)
    # the dominant edge is hit exactly by code 0 (bias = edge)
    g = w.reshape(16, -1, gs)
    edge_idx = np.where(np.abs(g.min(-1)) > np.abs(np.maximum(g.max(-1), 0)),
                        g.argmin(-1), g.argmax(-1))
    edge_codes = np.take_along_axis(codes.reshape(16, -1, gs), edge_idx[..., None], -1)[..., 0]
    assert np.all(edge_codes == 0)


def test_f16_sidecar_guard():
    # affine.py:43-51: a zero / sub-f16 scale is stored as +-2^-14, never 0.
    w = np.zeros((1, 64), np.float32)
    _, s, _, _ = O.quantize_affine(w, 4, 64, sidecar="f16")
    assert s.dtype == np.float16 and s[0, 0] != 0
    assert abs(float(s[0, 0])) == float(np.finfo(np.float16).smallest_normal)


# ----------------------------------------------------------------------------- matmuls


def test_quantized_matmul_vs_pure_python_loop():
    rng = np.random.default_rng(3)
    w = O.round_bf16(rng.standard_normal((3, 64)).astype(np.float32) * 0.02)
    packed, s, b, codes = O.quantize_affine(w, 3, 32)
    sf, bf = O.sidecar_f32(s, "bf16"), O.sidecar_f32(b, "bf16")
    x = O.round_bf16(rng.standard_normal((2, 64)).astype(np.float32))
    y = O.quantized_matmul(x, packed, sf, bf, 3, 32)
    for m in range(2):
        for n in range(3):
            acc = 0.0
            for k in range(64):
                wq = np.float32(np.float32(codes[n, k]) * sf[n, k // 32]) + bf[n, k // 32]
                acc += float(x[m, k]) * float(np.float32(wq))
            assert abs(acc - y[m, n]) < 1e-12


def test_c_gemm_matches_numpy(c_oracle):
    rng = np.random.default_rng(4)
    x = rng.standard_normal((3, 96)).astype(np.float32)
    W = rng.standard_normal((5, 96)).astype(np.float32)
    y = np.zeros((3, 5), np.float64)
    c_oracle.jqo_gemm_f64(x.ctypes.data, W.ctypes.data, 3, 5, 96, y.ctypes.data)
    np.testing.assert_allclose(y, x.astype(np.float64) @ W.T.astype(np.float64), rtol=1e-12)


def test_gather_qmm_vs_loop_and_dense():
    rng = np.random.default_rng(9)
    E, N, K = 4, 8, 64
    w = O.round_bf16(rng.standard_normal((E * N, K)).astype(np.float32) * 0.02)
    packed, s, b, _ = O.quantize_affine(w, 4, 32)
    P = packed.reshape(E, N, -1)
    sf = O.sidecar_f32(s, "bf16").reshape(E, N, -1)
    bf = O.sidecar_f32(b, "bf16").reshape(E, N, -1)
    x = O.round_bf16(rng.standard_normal((5, 1, K)).astype(np.float32))
    lhs = np.array([0, 1, 1, 4, 2, 3])
    rhs = np.array([3, 0, 2, 2, 1, 0])
    out = O.gather_qmm(x, P, sf, bf, lhs, rhs, 4, 32)
    for i in range(len(lhs)):
        ref = O.quantized_matmul(x[lhs[i]], P[rhs[i]], sf[rhs[i]], bf[rhs[i]], 4, 32)
        np.testing.assert_array_equal(out[i], ref)


def test_switch_glu_equals_composed_gathers():
    """SwitchGLU = gather(gate), gather(up), silu*up, gather(down) (dots3/ops.py:215-223)."""
    rng = np.random.default_rng(12)
    E, H, I, T, k = 4, 64, 32, 3, 2

    def stack(rows, K, bits, seed):
        r = np.random.default_rng(seed)
        w = O.round_bf16(r.standard_normal((E * rows, K)).astype(np.float32) * 0.02)
        p, s, b, _ = O.quantize_affine(w, bits, 32)
        return (p.reshape(E, rows, -1), O.sidecar_f32(s, "bf16").reshape(E, rows, -1),
                O.sidecar_f32(b, "bf16").reshape(E, rows, -1), bits)

    g, u, d = stack(I, H, 4, 1), stack(I, H, 4, 2), stack(H, I, 2, 3)
    x = O.round_bf16(rng.standard_normal((T, H)).astype(np.float32))
    idx = np.array([[0, 3], [2, 0], [1, 1]])
    out, _ = O.switch_glu(x, idx, g, u, d, 32, "bf16")
    lhs = np.repeat(np.arange(T), k)
    gg = O.round_bf16(O.gather_qmm(x[:, None, :], *g[:3], lhs, idx.reshape(-1), 4, 32))
    uu = O.round_bf16(O.gather_qmm(x[:, None, :], *u[:3], lhs, idx.reshape(-1), 4, 32))
    h = O.round_bf16(O.silu(gg) * uu)
    dd = O.round_bf16(O.gather_qmm(h, *d[:3], np.arange(T * k), idx.reshape(-1), 2, 32))
    np.testing.assert_array_equal(out.reshape(T * k, H), dd[:, 0, :])


def test_route_topk_vs_full_sort():
    rng = np.random.default_rng(13)
    logits = rng.standard_normal((6, 32)).astype(np.float32)
    logits[0, 5] = logits[0, 9] = 9.0  # exact tie: lower id first
    idx, w = O.route_topk(logits, 4, renorm=True)
    for t in range(6):
        p = np.exp(logits[t].astype(np.float64) - logits[t].max())
        p /= p.sum()
        order = sorted(range(32), key=lambda e: (-p[e], e))[:4]
        assert idx[t].tolist() == order
        np.testing.assert_allclose(w[t], p[order] / p[order].sum(), rtol=1e-12)
    assert idx[0, 0] == 5 and idx[0, 1] == 9


def test_half_ulp_helper():
    """The test helper's rounding allowance: half an ulp of bf16 / f16 at |v|."""
    from tests._util import half_ulp
    v = np.array([1.0, 1.99, 2.0, -3.0, 6.8, 0.0], dtype=np.float32)
    assert np.array_equal(half_ulp(v, "bf16"), [2**-8, 2**-8, 2**-7, 2**-7, 2**-6, 2**-108])
    assert np.array_equal(half_ulp(np.array([1.0, 1e-6]), "f16"), [2**-11, 2**-25])
    # a bf16 rounding of any value stays within the allowance
    r = np.random.default_rng(0).standard_normal(1000).astype(np.float32) * 50
    assert np.all(np.abs(O.round_bf16(r) - r) <= half_ulp(r, "bf16"))


def test_moe_combine_vs_torch_composition():
    """The oracle's combine equals the array composition the reference's caller writes,
    (y * scores[..., None]).sum(-2) then + shared (qwen4_exp/modeling.py:594-597), evaluated
    with torch on the CPU in fp64 and rounded to bf16 at the same two points."""
    import torch

    rng = np.random.default_rng(41)
    T, k, H = 3, 5, 64
    y = O.round_bf16(rng.standard_normal((T, k, H), dtype=np.float32))
    w = rng.random((T, k)).astype(np.float32)
    sh = O.round_bf16(rng.standard_normal((T, H), dtype=np.float32))
    ty = torch.from_numpy(y).double()
    routed = (ty * torch.from_numpy(w).double().unsqueeze(-1)).sum(dim=-2).to(torch.bfloat16)
    ref = (routed.double() + torch.from_numpy(sh).double()).to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(O.moe_combine(y, w, sh), ref)
    np.testing.assert_array_equal(O.moe_combine(y, w), routed.float().numpy())
    # one-hot weights select a slot exactly
    onehot = np.zeros((T, k), np.float32)
    onehot[:, 2] = 1.0
    np.testing.assert_array_equal(O.moe_combine(y, onehot), y[:, 2, :])


def test_swiglu_pair_equals_switch_glu_single_expert():
    """A dense SwiGLU pair is SwitchGLU's gate/up stage over a one-expert stack."""
    rng = np.random.default_rng(43)
    H, I, T = 128, 64, 3
    mats = []
    for seed in (1, 2, 3):
        r = np.random.default_rng(seed)
        rows, cols = (I, H) if seed < 3 else (H, I)
        ww = O.round_bf16(r.standard_normal((rows, cols), dtype=np.float32) * np.float32(0.02))
        p, s, b, _ = O.quantize_affine(ww, 4, 64)
        mats.append((p, O.sidecar_f32(s, "bf16"), O.sidecar_f32(b, "bf16"), 4))
    x = O.round_bf16(rng.standard_normal((T, H), dtype=np.float32))
    h = O.swiglu_pair(x, mats[0], mats[1], 64)
    stack = [(m[0][None], m[1][None], m[2][None], m[3]) for m in mats]
    _, hs = O.switch_glu(x, np.zeros((T, 1), np.int64), *stack, 64, "bf16")
    np.testing.assert_array_equal(h, hs[:, 0, :])


def test_expand_1bit_to_2bit_known_answers_and_codes():
    """Known answers from the definition (source bit i -> 2-bit field i, low half of a word
    to the even output word, high half to the odd one) and the code-level identity."""
    src = np.array([[0x80000001, 0xFFFFFFFF, 0x0000FFFF, 0x00010000]], np.uint32)
    got = O.expand_1bit_to_2bit(src)
    assert got.tolist() == [[0x00000001, 0x40000000, 0x55555555, 0x55555555,
                             0x55555555, 0x00000000, 0x00000000, 0x00000001]]
    rng = np.random.default_rng(3)
    w = rng.integers(0, 2**32, size=(7, 5), dtype=np.uint64).astype(np.uint32)
    e = O.expand_1bit_to_2bit(w)
    assert e.shape == (7, 10)
    np.testing.assert_array_equal(O.unpack_rows(e, 2), O.unpack_rows(w, 1))


@pytest.mark.parametrize("bits", [2, 3, 4, 5, 6, 8])
def test_dequantize_tensor_flat_vs_loop_and_row_layout(bits):
    """quantize.py:292-326 on a padded tensor: a per-element loop over the bit stream, and the
    same bytes read as the row layout of [n_blocks, 64] (the identity the GPU path uses)."""
    rng = np.random.default_rng(bits)
    shape, bs = (3, 50), 64
    n_blocks = -(-150 // bs)
    codes = rng.integers(0, 1 << bits, size=n_blocks * bs)
    q = O.pack_bits(codes, bits)
    s = (rng.random(n_blocks) * 0.1 + 0.01).astype(np.float16)
    b = (rng.standard_normal(n_blocks) * 0.05).astype(np.float16)
    got = O.dequantize_tensor_flat(q, s, b, bits, shape, bs)
    loop = np.empty(150, np.float32)
    for i in range(150):
        v = 0
        for t in range(bits):
            bit = i * bits + t
            v |= ((int(q[bit // 8]) >> (bit % 8)) & 1) << t
        blk = i // bs
        loop[i] = np.float32(np.float32(v) * np.float32(s[blk])) + np.float32(b[blk])
    np.testing.assert_array_equal(got.reshape(-1), loop)
    rows = O.dequantize_affine(q.view(np.uint32).reshape(n_blocks, bs * bits // 32),
                               s.astype(np.float32)[:, None], b.astype(np.float32)[:, None], bits, bs)
    np.testing.assert_array_equal(got.reshape(-1), rows.reshape(-1)[:150])


# ----------------------------------------------------------------------------- MX modes


def test_e2m1_table_matches_the_format():
    """The restated mxfp4 value table against the E2M1 definition (1 sign, 2 exponent bits with
    bias 1, 1 mantissa bit; exponent 0 is subnormal)."""
    for c in range(16):
        sgn = -1.0 if c & 8 else 1.0
        e, m = (c >> 1) & 3, c & 1
        mag = m * 0.5 if e == 0 else 2.0 ** (e - 1) * (1 + m / 2)
        assert O.E2M1_TABLE[c] == sgn * mag and np.signbit(O.E2M1_TABLE[c]) == bool(c & 8)


def test_e4m3_and_e8m0_match_torch():
    b = np.arange(256, dtype=np.uint8)
    ref = torch.from_numpy(b).view(torch.float8_e4m3fn).float().numpy()
    got = O.e4m3_to_f32(b)
    np.testing.assert_array_equal(np.isnan(got), np.isnan(ref))
    np.testing.assert_array_equal(got[~np.isnan(got)], ref[~np.isnan(ref)])
    ref8 = torch.from_numpy(b).view(torch.float8_e8m0fnu).float().numpy()
    got8 = O.e8m0_to_f32(b)
    np.testing.assert_array_equal(np.isnan(got8), np.isnan(ref8))
    np.testing.assert_array_equal(got8[:255], ref8[:255])


def test_mx_layout_and_brute_force():
    """Element 2i sits in the low nibble of byte i (mxfp4_codec.py:8), bytes little-endian in
    the uint32 words; scales one per 32 elements. Checked against a pure-Python loop."""
    w = np.array([[0x00000021]], dtype=np.uint32)  # bytes 21 00 00 00
    np.testing.assert_array_equal(O.mx_codes(w, "mxfp4")[0, :4], [1, 2, 0, 0])
    np.testing.assert_array_equal(O.mx_codes(w, "mxfp8")[0], [0x21, 0, 0, 0])
    rng = np.random.default_rng(3)
    for mode, per_word in (("mxfp4", 8), ("mxfp8", 4)):
        K = 64
        packed = rng.integers(0, 2**32, (3, K // per_word), dtype=np.uint64).astype(np.uint32)
        if mode == "mxfp8":  # no NaN codes (S.1111.111)
            by = packed.view(np.uint8)
            by[(by & 0x7F) == 0x7F] = 0x7E
        sc = rng.integers(100, 140, (3, K // 32)).astype(np.uint8)
        got = O.mx_dequantize(packed, sc, mode)
        for r in range(3):
            word_bytes = [int(x) for x in packed[r].view(np.uint8)]
            for k in range(K):
                if mode == "mxfp4":
                    byte = word_bytes[k // 2]
                    code = (byte >> 4) if k % 2 else (byte & 15)
                    sgn = -1.0 if code & 8 else 1.0
                    e, m = (code >> 1) & 3, code & 1
                    v = sgn * (m * 0.5 if e == 0 else 2.0 ** (e - 1) * (1 + m / 2))
                else:
                    byte = word_bytes[k]
                    sgn = -1.0 if byte & 0x80 else 1.0
                    e, m = (byte >> 3) & 15, byte & 7
                    v = sgn * (m * 2.0 ** -9 if e == 0 else (1 + m / 8) * 2.0 ** (e - 7))
                assert got[r, k] == np.float32(v * 2.0 ** (int(sc[r, k // 32]) - 127)), (mode, r, k)


def _route_brute(logits, k, score, bias, n_group, topk_group, renorm, eps, scaling):
    """Pure-Python restatement of the reference routers, token by token (math module only)."""
    import math as m
    out_i, out_w = [], []
    for row in np.asarray(logits, np.float64).tolist():
        E = len(row)
        if score == "softmax":
            mx = max(row)
            ex = [m.exp(v - mx) for v in row]
            tot = sum(ex)
            sc = [v / tot for v in ex]
        elif score == "sigmoid":
            sc = [1.0 / (1.0 + m.exp(-v)) for v in row]
        else:
            sc = [m.sqrt(m.log1p(m.exp(-abs(v))) + max(v, 0.0)) for v in row]
        sel = [sc[e] + (0.0 if bias is None else float(bias[e])) for e in range(E)]
        if n_group > 1 and topk_group < n_group:
            gsz = E // n_group
            best = [max(sel[g * gsz:(g + 1) * gsz]) for g in range(n_group)]
            kept = sorted(range(n_group), key=lambda g: (-best[g], g))[:topk_group]
            for e in range(E):
                if e // gsz not in kept:
                    sel[e] = 0.0
                    sc[e] = 0.0
        ids = sorted(range(E), key=lambda e: (-sel[e], e))[:k]
        w = [sc[e] for e in ids]
        if renorm:
            tot = sum(w) + eps
            w = [v / tot for v in w]
        out_i.append(ids)
        out_w.append([v * scaling for v in w])
    return np.array(out_i), np.array(out_w)


@pytest.mark.parametrize("score", ["softmax", "sigmoid", "sqrtsoftplus"])
@pytest.mark.parametrize("groups", [(1, 1), (4, 2), (8, 3)])
@pytest.mark.parametrize("with_bias", [False, True])
def test_route_topk_ex_vs_brute_force(score, groups, with_bias):
    rng = np.random.default_rng(zlib.crc32(repr((score, groups, with_bias)).encode()))
    T, E, k = 5, 32, 4
    logits = rng.standard_normal((T, E)).astype(np.float32) * 2
    bias = rng.standard_normal(E).astype(np.float32) * 0.3 if with_bias else None
    ng, tg = groups
    eps = 0.0 if score == "softmax" else 1e-20
    idx, w = O.route_topk_ex(logits, k, score=score, bias=bias, n_group=ng, topk_group=tg,
                             renorm=True, scaling=2.5)
    bi, bw = _route_brute(logits, k, score, bias, ng, tg, True, eps, 2.5)
    np.testing.assert_array_equal(idx, bi)
    np.testing.assert_allclose(w, bw, rtol=1e-12)
    np.testing.assert_allclose(w.sum(-1), 2.5, rtol=1e-12)  # renormalised, then scaled
    _, w0 = O.route_topk_ex(logits, k, score=score, bias=bias, n_group=ng, topk_group=tg,
                            renorm=False)
    np.testing.assert_allclose(w0, _route_brute(logits, k, score, bias, ng, tg, False, 0, 1)[1],
                               rtol=1e-12)


def test_route_topk_ex_closed_forms():
    rng = np.random.default_rng(51)
    logits = rng.standard_normal((7, 64)).astype(np.float32) * 3
    ref_i, ref_w = O.route_topk(logits, 6)
    i0, w0 = O.route_topk_ex(logits, 6)
    np.testing.assert_array_equal(i0, ref_i)
    np.testing.assert_allclose(w0, ref_w, rtol=1e-12)
    for score in ("sigmoid", "sqrtsoftplus"):  # monotone scores without bias: the top logits
        i1, _ = O.route_topk_ex(logits, 6, score=score)
        np.testing.assert_array_equal(i1, ref_i)
    # keeping every group is no grouping at all
    i2, w2 = O.route_topk_ex(logits, 6, n_group=8, topk_group=8)
    np.testing.assert_array_equal(i2, ref_i)
    # the bias changes the selection but not the weights' source: weights are unbiased scores
    bias = np.zeros(64, np.float32)
    bias[:8] = 10.0
    i3, w3 = O.route_topk_ex(logits, 6, score="sigmoid", bias=bias, renorm=False)
    assert np.all(i3 < 8)
    np.testing.assert_allclose(w3, 1 / (1 + np.exp(-np.take_along_axis(
        logits.astype(np.float64), i3, -1))), rtol=1e-12)
    # planted mistake: weights taken from the biased values differ from the reference's
    wrong = np.take_along_axis(1 / (1 + np.exp(-logits.astype(np.float64))) + bias, i3, -1)
    assert not np.allclose(wrong, w3)
    # group-limited: only experts of the kept groups are chosen when they hold enough
    i4, _ = O.route_topk_ex(logits, 4, n_group=8, topk_group=2)
    for t in range(7):
        assert len(set((i4[t] // 8).tolist())) <= 2


def test_moe_token_forms_vs_compositions():
    """moe_token against the reference's array expressions evaluated with torch (CPU, fp64,
    rounded to bf16 where the reference's arrays are bf16): qwen4_exp/modeling.py:594-599
    ('after', sigmoid-gated shared term) and dsv41/model.py:1214-1245 ('before', clamp)."""
    import torch

    rng = np.random.default_rng(61)
    H, I, E, k = 64, 32, 6, 3
    Ws = {(c, e): rng.standard_normal((I, H) if c != "d" else (H, I)) * 0.1
          for c in "gud" for e in range(E)}
    deq = lambda c, e: Ws[(c, int(e))]  # noqa: E731
    x = O.round_bf16(rng.standard_normal(H).astype(np.float32)).astype(np.float64)
    ids = np.array([4, 1, 3])
    w = np.array([0.5, 0.3, 0.2])
    sh = O.round_bf16(rng.standard_normal(H).astype(np.float32)).astype(np.float64)
    bf = lambda t: t.to(torch.bfloat16).double()  # noqa: E731
    tx = torch.from_numpy(x)
    lim = 0.8
    for combine in ("after", "before"):
        for gate in (None, 0.7):
            if combine == "before" and gate is not None:
                continue
            got, _ = O.moe_token(x, ids, w, deq, combine, lim, sh, gate)
            ys = []
            for j, e in enumerate(ids):
                g = bf(tx @ torch.from_numpy(deq("g", e)).T).clamp(max=lim)
                u = bf(tx @ torch.from_numpy(deq("u", e)).T).clamp(-lim, lim)
                h = torch.nn.functional.silu(g) * u
                if combine == "before":
                    h = h * w[j]
                ys.append(bf(bf(h) @ torch.from_numpy(deq("d", e)).T))
            if combine == "after":
                routed = bf(sum(wj * y for wj, y in zip(w, ys)))
                term = torch.from_numpy(sh)
                if gate is not None:
                    term = bf(bf(torch.sigmoid(torch.tensor(gate, dtype=torch.float64))) * term)
                ref = bf(routed + term)
            else:
                ref = bf(sum(ys) + torch.from_numpy(sh))
            np.testing.assert_array_equal(got, ref.float().numpy())
    # the 'after' form without clamp is switch_glu's slots combined by moe_combine
    got, _ = O.moe_token(x, ids, w, deq, "after", 0.0, sh)
    slots = []
    for e in ids:
        g = O.round_bf16(x @ deq("g", e).T)
        u = O.round_bf16(x @ deq("u", e).T)
        h = O.round_bf16(O.silu(g) * u)
        slots.append(O.round_bf16(h.astype(np.float64) @ deq("d", e).T))
    np.testing.assert_array_equal(got, O.moe_combine(np.array(slots)[None], w[None], sh[None])[0])

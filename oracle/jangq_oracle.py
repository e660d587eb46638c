"""CPU oracle for the quantized-weight matmul path — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
use this module, and only as the checker / the timed CPU baseline. The product
(``jangq_amd``) never imports it.

Each function restates one reference algorithm (file:line relative to the reference
checkout) in numpy:

  pack_bits / unpack_bits      jang-tools/jang_tools/pack.py:12-82 / 85-149
  pack_rows / unpack_rows      the same stream viewed as uint32 rows (affine.py:256-265, 457)
  quantize_affine              jang-tools/jang_tools/affine.py:193-276 (mirror of mx.quantize)
  dequantize_affine            jang-tools/jang_tools/affine.py:445-463 (+ 3-D flattening of
                               quantize.py:238-239)
  quantized_matmul             mx.quantized_matmul contract, jangrt/linear.py:41-45
  gather_qmm                   naive per-pair loop of jang_tools/dots3/ops_selftest.py:18-28
  switch_glu                   mlx_lm SwitchGLU as restated at dots3/ops.py:195-223
  route_topk                   qwen4_exp/modeling.py:587-593
  route_scores / route_topk_ex softmax / sigmoid / sqrt-softplus routers with selection bias,
                               group-limited selection, renorm eps and scaling:
                               mistral4_mlx.py:355-387, dots3/ops.py:149-162,
                               laguna/model.py:50-62, dsv41/model.py:1184-1190
  glu / shared_expert / moe_token  the MoE block's expert MLPs and combine, both forms:
                               qwen4_exp/modeling.py:586-599 (weights after the down
                               projection, sigmoid-gated shared term) and dsv41/model.py:
                               1166-1245 (weights before it, SwiGLU clamp)
  mx_dequantize                OCP MX modes as MLX stores them: mxfp4 per
                               jang-tools/jang_tools/mimo_v2/mxfp4_codec.py:1-50 (E2M1 nibbles,
                               low nibble = even element, E8M0 block scales, 32 per block, the
                               bytes read as little-endian uint32 words); mxfp8 the same with
                               one E4M3 byte per element (loader.py:1877-1912 mode switch)

How each is pinned (tests/test_oracle.py):
  pack/unpack       known answers of jang-tools/tests/test_pack.py:33-61, the LSB-first 3-bit
                    straddle vector, round trips with the reference test seeds, and a
                    bit-by-bit C restatement (oracle/jq_oracle.c) agreeing on random data
  quantize_affine   the MLX-produced fixture jang-runtime/Tests/JANGCoreMetalTests/fixtures/
                    matmul_4bit_64x128.safetensors (codes, f16 sidecars) regenerated from
                    its seed; invariants (codes in range, edge code hits the edge)
  dequantize        the same fixture's y_ref (MLX dequantize @ x), dequant(s=1,b=0) == q,
                    two-rounding vs fused-FMA discrimination, C restatement agreement
  quantized_matmul  fixture y_ref; brute-force pure-Python loop on tiny shapes
  gather/switch     brute force on tiny shapes; sorted/unsorted equivalence
  route_topk        brute force (full sort) on small shapes
  route_topk_ex     a pure-Python brute force (explicit sort key, explicit group loop) on
                    small shapes; closed forms: the sigmoid/sqrt-softplus routers without
                    bias pick the top-k logits (monotone scores), group-limited selection
                    with topk_group == n_group is plain top-k, renormalised weights sum to
                    the scaling factor, softmax matches route_topk
  moe_token         a per-expert loop restating the reference's array expressions one by
                    one (tests/test_oracle.py), the "after" form equal to switch_glu +
                    moe_combine, and the "before" form equal to the "after" form's
                    per-slot outputs when every weight is 1
"""
from __future__ import annotations

import math

import numpy as np

SUPPORTED_BITS = (2, 3, 4, 5, 6, 8)

# ----------------------------------------------------------------------------- bf16 / f16


def f32_to_bf16_bits(a) -> np.ndarray:
    """Round-to-nearest-even fp32 -> bf16 bit patterns (NaN -> 0x7FC0)."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    return np.where(nan, np.uint16(0x7FC0), r)


def bf16_bits_to_f32(b) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def round_bf16(a) -> np.ndarray:
    """fp32 value of the bf16 rounding of a."""
    return bf16_bits_to_f32(f32_to_bf16_bits(a))


def round_to(a, dtype: str) -> np.ndarray:
    a = np.asarray(a, dtype=np.float32)
    if dtype == "bf16":
        return round_bf16(a)
    if dtype == "f16":
        return a.astype(np.float16).astype(np.float32)
    return a


# ----------------------------------------------------------------------------- bit stream


def pack_bits(values, bits: int) -> np.ndarray:
    """LSB-first stream: value i occupies bits [i*bits, (i+1)*bits); (n*bits+7)//8 bytes."""
    v = np.asarray(values, dtype=np.uint64).reshape(-1)
    if v.size and int(v.max()) >= (1 << bits):
        raise ValueError("value does not fit the bit width")
    bitplanes = ((v[:, None] >> np.arange(bits, dtype=np.uint64)[None, :]) & 1).astype(np.uint8)
    return np.packbits(bitplanes.reshape(-1), bitorder="little")


def unpack_bits(packed, bits: int, count: int) -> np.ndarray:
    """Inverse of pack_bits; any array shape is flattened as its row-major byte stream.
    1/2/4/8 bits: the reference's shift-and-mask fast paths (pack.py:101-130); 3/5/6 bits: a
    vectorised bit-plane unpack (the reference loops per element there, pack.py:132-149)."""
    b = np.asarray(packed, dtype=np.uint8).reshape(-1)
    if bits == 8:
        return b[:count].copy()
    if bits in (1, 2, 4):
        per = 8 // bits
        mask = (1 << bits) - 1
        out = np.empty(b.size * per, dtype=np.uint8)
        for i in range(per):
            out[i::per] = (b >> (i * bits)) & mask
        return out[:count]
    stream = np.unpackbits(b, bitorder="little")[: count * bits]
    planes = stream.reshape(count, bits).astype(np.uint16)
    return (planes << np.arange(bits, dtype=np.uint16)[None, :]).sum(axis=1).astype(np.uint8)


def pack_rows(codes: np.ndarray, bits: int) -> np.ndarray:
    """Codes [rows, K] -> uint32 [rows, K*bits/32] (each row is a whole number of words)."""
    codes = np.asarray(codes)
    rows, K = codes.shape
    if (K * bits) % 32:
        raise ValueError("row is not a whole number of uint32 words")
    return pack_bits(codes.reshape(-1), bits).view(np.uint32).reshape(rows, K * bits // 32)


def unpack_rows(w: np.ndarray, bits: int) -> np.ndarray:
    """uint32 [..., P] -> codes uint8 [..., P*32/bits]."""
    w = np.ascontiguousarray(w, dtype=np.uint32)
    K = w.shape[-1] * 32 // bits
    rows = int(np.prod(w.shape[:-1]))
    return unpack_bits(w.view(np.uint8), bits, rows * K).reshape(*w.shape[:-1], K)


# ----------------------------------------------------------------------------- quantizer

_FP16_TINY = np.float32(np.finfo(np.float16).smallest_normal)


def _to_f16_nonzero(scale: np.ndarray) -> np.ndarray:
    safe = np.where(np.abs(scale) < _FP16_TINY,
                    np.copysign(_FP16_TINY, np.where(scale == 0, 1.0, scale)), scale)
    return safe.astype(np.float16)


def quantize_affine(w, bits: int, group_size: int, sidecar: str = "bf16",
                    input_via_f16: bool = False):
    """mx.quantize affine rule. Returns (packed u32 [rows, K*bits/32], scales, biases, codes).

    sidecar: "bf16" (uint16 bf16 bit patterns), "f16" (np.float16 with the non-zero guard of
    affine.py:43-51) or "f32". input_via_f16 reproduces affine.py:212 (source cast to f16)."""
    if bits not in SUPPORTED_BITS:
        raise ValueError(f"unsupported bits={bits}")
    src = np.asarray(w)
    if input_via_f16:
        src = src.astype(np.float16)
    src = src.astype(np.float32)
    rows, K = src.shape
    if K % group_size:
        raise ValueError("K not divisible by group_size")
    g = src.reshape(rows, K // group_size, group_size)
    bins = np.float32((1 << bits) - 1)
    low = g.min(axis=-1)
    high = np.maximum(g.max(axis=-1), np.float32(0.0))
    scale = np.maximum((high - low) / bins, np.float32(1e-7)).astype(np.float32)
    dominant_low = np.abs(low) > np.abs(high)
    scale = np.where(dominant_low, scale, -scale).astype(np.float32)
    edge = np.where(dominant_low, low, high).astype(np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        edge_code = np.rint(edge / scale).astype(np.float32)
        at_zero = edge_code == 0
        refined = np.where(at_zero, scale, edge / np.where(at_zero, 1, edge_code)).astype(np.float32)
    scale = np.where(at_zero, scale, refined).astype(np.float32)
    bias = np.where(at_zero, np.float32(0.0), edge).astype(np.float32)
    q = np.rint((g - bias[..., None]) / scale[..., None])
    codes = np.clip(q, 0, bins).astype(np.uint8).reshape(rows, K)
    packed = pack_rows(codes, bits)
    if sidecar == "bf16":
        s_out, b_out = f32_to_bf16_bits(scale), f32_to_bf16_bits(bias)
    elif sidecar == "f16":
        s_out, b_out = _to_f16_nonzero(scale), bias.astype(np.float16)
    else:
        s_out, b_out = scale, bias
    return packed, s_out, b_out, codes


def sidecar_f32(a, sidecar: str) -> np.ndarray:
    """Stored sidecar as fp32 values."""
    if sidecar == "bf16":
        return bf16_bits_to_f32(a)
    return np.asarray(a).astype(np.float32)


# ----------------------------------------------------------------------------- dequant


def dequantize_affine(w, scales_f32, biases_f32, bits: int, group_size: int) -> np.ndarray:
    """fl(fl(q*s) + b) in fp32; w [..., P] (2-D or stacked), scales/biases fp32 [..., G]."""
    codes = unpack_rows(w, bits).astype(np.float32)
    lead = codes.shape[:-1]
    K = codes.shape[-1]
    q = codes.reshape(*lead, K // group_size, group_size)
    s = np.asarray(scales_f32, dtype=np.float32)[..., None]
    b = np.asarray(biases_f32, dtype=np.float32)[..., None]
    prod = (q * s).astype(np.float32)          # first rounding
    return (prod + b).astype(np.float32).reshape(*lead, K)  # second rounding


# ----------------------------------------------------------------------------- matmuls


def dequantize_tensor_flat(qweight_u8, scales, biases, bits: int, shape,
                           block_size: int = 64) -> np.ndarray:
    """Flat (v1) dequant of jang-tools/jang_tools/quantize.py:292-326: unpack the whole
    LSB-first stream (n_blocks * block_size codes), q * s + b per block in fp32 (two roundings),
    cut to prod(shape) elements."""
    s = np.asarray(scales).astype(np.float32).reshape(-1)
    b = np.asarray(biases).astype(np.float32).reshape(-1)
    n_blocks = s.size
    q = unpack_bits(np.asarray(qweight_u8, np.uint8), bits, n_blocks * block_size)
    q = q.reshape(n_blocks, block_size).astype(np.float32)
    out = (q * s[:, None]).astype(np.float32) + b[:, None]
    total = int(np.prod(shape))
    return out.reshape(-1)[:total].reshape(tuple(shape))


def expand_1bit_to_2bit(packed) -> np.ndarray:
    """1-bit -> 2-bit code expansion (jang-tools/jang_tools/affine.py:402-416), restated
    through the code stream: the 1-bit codes of each row, repacked at 2 bits."""
    w = np.asarray(packed, dtype=np.uint32)
    flat = w.reshape(-1, w.shape[-1])
    out = np.stack([pack_bits(unpack_bits(r.view(np.uint8), 1, 32 * r.size), 2).view(np.uint32)
                    for r in flat])
    return out.reshape(*w.shape[:-1], 2 * w.shape[-1])


def quantized_matmul(x_f32, w, s_f32, b_f32, bits: int, group_size: int) -> np.ndarray:
    """y = x @ dequant(W)^T accumulated in fp64 (x given as fp32 values). Returns fp64."""
    W = dequantize_affine(w, s_f32, b_f32, bits, group_size).astype(np.float64)
    x = np.asarray(x_f32, dtype=np.float64)
    return x @ W.T


def gather_qmm(x_f32, w, s_f32, b_f32, lhs, rhs, bits: int, group_size: int) -> np.ndarray:
    """out[i] = x[lhs[i]] @ dequant(W[rhs[i]])^T, fp64; x [B, M, K], w [E, N, P]."""
    x = np.asarray(x_f32, dtype=np.float64)
    lhs = np.asarray(lhs).reshape(-1)
    rhs = np.asarray(rhs).reshape(-1)
    E, N = w.shape[0], w.shape[1]
    out = np.zeros((lhs.size, x.shape[-2], N), dtype=np.float64)
    cache = {}
    for i, (l, r) in enumerate(zip(lhs, rhs)):
        if r not in cache:
            cache[r] = dequantize_affine(w[r], s_f32[r], b_f32[r], bits, group_size).astype(np.float64)
        out[i] = x[l] @ cache[r].T
    return out


def silu(v):
    v = np.asarray(v, dtype=np.float64)
    return v / (1.0 + np.exp(-v))


def switch_glu(x_f32, idx, gate, up, down, group_size: int, out_dtype: str = "bf16"):
    """Per (token t, slot j), e = idx[t, j]:
    g, u = round(x[t] @ Wg[e]^T), round(x[t] @ Wu[e]^T); h = round(silu(g) * u);
    out[t, j] = round(h @ Wd[e]^T). Each matmul accumulates in fp64. gate/up/down are
    (w, s_f32, b_f32, bits). Returns out (fp32 values of the rounded results) and h."""
    x = np.asarray(x_f32, dtype=np.float64)
    idx = np.asarray(idx)
    T, k = idx.shape
    deq = {}

    def W(which, e):
        key = (which, int(e))
        if key not in deq:
            w, s, b, bits = {"g": gate, "u": up, "d": down}[which]
            deq[key] = dequantize_affine(w[e], s[e], b[e], bits, group_size).astype(np.float64)
        return deq[key]

    H = x.shape[-1]
    I = gate[0].shape[1]
    out = np.zeros((T, k, H), dtype=np.float32)
    hs = np.zeros((T, k, I), dtype=np.float32)
    for t in range(T):
        for j in range(k):
            e = idx[t, j]
            g = round_to(x[t] @ W("g", e).T, out_dtype).astype(np.float64)
            u = round_to(x[t] @ W("u", e).T, out_dtype).astype(np.float64)
            h = round_to(silu(g) * u, out_dtype)
            hs[t, j] = h
            out[t, j] = round_to(h.astype(np.float64) @ W("d", e).T, out_dtype)
    return out, hs


def moe_combine(y, w, shared=None, out_dtype: str = "bf16") -> np.ndarray:
    """The caller-side combine of jang-tools/jang_tools/qwen4_exp/modeling.py:594-597:
    round((y * w[..., None]).sum(-2)) (+ shared, rounded again); y [T, k, H] values of
    out_dtype, w [T, k]. Products and the slot-order sum in fp64."""
    y = np.asarray(y, dtype=np.float64)
    w = np.asarray(w, dtype=np.float64)
    r = round_to((y * w[..., None]).sum(-2), out_dtype)
    if shared is not None:
        r = round_to(r.astype(np.float64) + np.asarray(shared, dtype=np.float64), out_dtype)
    return r


def swiglu_pair(x_f32, gate, up, group_size: int, out_dtype: str = "bf16") -> np.ndarray:
    """h = round(silu(round(x @ Wg^T)) * round(x @ Wu^T)) of a dense MLP (the shared expert of
    qwen4_exp/modeling.py:597; gate/up = (w, s_f32, b_f32, bits)), matmuls in fp64."""
    g = round_to(quantized_matmul(x_f32, *gate[:3], gate[3], group_size), out_dtype)
    u = round_to(quantized_matmul(x_f32, *up[:3], up[3], group_size), out_dtype)
    return round_to(silu(g) * u.astype(np.float64), out_dtype)


def route_topk(logits, k: int, renorm: bool = True):
    """softmax in fp64, top-k by descending probability (ties: lower id first)."""
    z = np.asarray(logits, dtype=np.float64)
    z = z - z.max(axis=-1, keepdims=True)
    p = np.exp(z)
    p /= p.sum(axis=-1, keepdims=True)
    order = np.lexsort((np.arange(p.shape[-1])[None, :].repeat(p.shape[0], 0), -p), axis=-1)
    idx = order[:, :k]
    w = np.take_along_axis(p, idx, axis=-1)
    if renorm:
        w = w / w.sum(axis=-1, keepdims=True)
    return idx.astype(np.int64), w


def route_scores(logits, score: str = "softmax") -> np.ndarray:
    """Router scores in fp64: softmax (qwen4_exp/modeling.py:587, mistral4_mlx.py:359),
    sigmoid (dots3/ops.py:155, laguna/model.py:52) or sqrt(softplus) (dsv41/model.py:1186)."""
    z = np.asarray(logits, dtype=np.float64)
    if score == "softmax":
        p = np.exp(z - z.max(axis=-1, keepdims=True))
        return p / p.sum(axis=-1, keepdims=True)
    if score == "sigmoid":
        return 1.0 / (1.0 + np.exp(-z))
    if score == "sqrtsoftplus":
        return np.sqrt(np.logaddexp(z, 0.0))
    raise ValueError(score)


def route_topk_ex(logits, k: int, *, score: str = "softmax", bias=None, n_group: int = 1,
                  topk_group: int = 1, renorm: bool = True, eps=None, scaling: float = 1.0):
    """The routers of the reference in fp64: selection value = score (+ bias), optionally
    group-limited (the topk_group groups of E/n_group consecutive experts with the largest
    maximum selection value stay; every other expert gets selection value 0 and score 0,
    mistral4_mlx.py:363-375), the top k in descending selection order (ties: lower id), their
    unbiased scores as weights, divided by (sum + eps) with renorm (eps 0 for softmax, 1e-20
    otherwise: dots3/ops.py:160, laguna/model.py:59) and times ``scaling``
    (mistral4_mlx.py:385)."""
    sc = route_scores(logits, score)
    T, E = sc.shape
    sel = sc + (0.0 if bias is None else np.asarray(bias, np.float64)[None, :])
    sc = sc.copy()
    if n_group > 1 and topk_group < n_group:
        gsz = E // n_group
        gmax = sel.reshape(T, n_group, gsz).max(axis=-1)
        for t in range(T):
            order = sorted(range(n_group), key=lambda g: (-gmax[t, g], g))
            for g in order[topk_group:]:
                sel[t, g * gsz:(g + 1) * gsz] = 0.0
                sc[t, g * gsz:(g + 1) * gsz] = 0.0
    idx = np.stack([np.lexsort((np.arange(E), -sel[t]))[:k] for t in range(T)])
    w = np.take_along_axis(sc, idx, axis=-1)
    if renorm:
        e = (0.0 if score == "softmax" else 1e-20) if eps is None else eps
        w = w / (w.sum(axis=-1, keepdims=True) + e)
    return idx.astype(np.int64), w * scaling


def glu(g, u, limit: float = 0.0, factor=1.0):
    """silu(g) * u * factor of rounded g, u, with the SwiGLU clamp of
    jang-tools/jang_tools/dsv41/model.py:1214-1218 (gate = min(gate, L), up = clip(up, -L, L))."""
    g = np.asarray(g, np.float64)
    u = np.asarray(u, np.float64)
    if limit > 0:
        g = np.minimum(g, limit)
        u = np.clip(u, -limit, limit)
    return silu(g) * u * factor


def shared_expert(x, Wg, Wu, Wd, limit: float = 0.0, out_dtype: str = "bf16"):
    """round(down(round(glu(round(x Wg^T), round(x Wu^T))))) of a dense SwiGLU MLP with fp64
    dequantized weights (qwen4_exp/modeling.py:599; dsv41/model.py:1237-1245)."""
    x = np.asarray(x, np.float64)
    g = round_to(x @ Wg.T, out_dtype)
    u = round_to(x @ Wu.T, out_dtype)
    h = round_to(glu(g, u, limit), out_dtype).astype(np.float64)
    return round_to(h @ Wd.T, out_dtype).astype(np.float64)


def moe_token(x, ids, w, deq, combine: str = "after", limit: float = 0.0, shared=None,
              shared_gate=None, out_dtype: str = "bf16"):
    """One token of a MoE block. deq(which, e) gives expert e's fp64 dequantized 'g', 'u' or 'd'
    matrix. Per slot: g, u rounded; h = round(glu(g, u, limit, w_j if combine == 'before'));
    y_j = round(h Wd^T). combine 'after' (qwen4_exp/modeling.py:594-599):
    round(round(sum_j w_j y_j) + s'), s' = round(round(sigmoid(gate)) * s) with a shared gate;
    'before' (dsv41/model.py:1219-1245): round(sum_j y_j + s). Returns (out, value before the
    last rounding)."""
    x = np.asarray(x, np.float64)
    acc = np.zeros(deq("d", ids[0]).shape[0], np.float64)
    for j, e in enumerate(ids):
        g = round_to(x @ deq("g", e).T, out_dtype)
        u = round_to(x @ deq("u", e).T, out_dtype)
        f = w[j] if combine == "before" else 1.0
        h = round_to(glu(g, u, limit, f), out_dtype).astype(np.float64)
        y = round_to(h @ deq("d", e).T, out_dtype).astype(np.float64)
        acc = acc + (y if combine == "before" else w[j] * y)
    if combine == "before":
        pre = acc + (0.0 if shared is None else shared)
        return round_to(pre, out_dtype), pre
    r = round_to(acc, out_dtype).astype(np.float64)
    if shared is None:
        return r, acc
    sh = np.asarray(shared, np.float64)
    if shared_gate is not None:
        gs = round_to(1.0 / (1.0 + np.exp(-float(shared_gate))), out_dtype).astype(np.float64)
        sh = round_to(gs * sh, out_dtype).astype(np.float64)
    pre = r + sh
    return round_to(pre, out_dtype), pre


# ----------------------------------------------------------------------------- MX modes

MX_BLOCK = 32
# E2M1 magnitudes of codes 0..7 (mxfp4_codec.py:22-26); code | 8 is the negative.
E2M1_TABLE = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0,
                       -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0], dtype=np.float32)


def e4m3_to_f32(b) -> np.ndarray:
    """OCP E4M3 (FN: bias 7, no infinities, S.1111.111 = NaN) bytes to fp32."""
    b = np.asarray(b, dtype=np.uint8).astype(np.int64)
    sgn = np.where(b & 0x80, -1.0, 1.0)
    e, m = (b >> 3) & 15, b & 7
    mag = np.where(e == 0, m * 2.0 ** -9, (1.0 + m / 8.0) * np.exp2(e - 7.0))
    out = sgn * mag
    return np.where((e == 15) & (m == 7), np.nan, out).astype(np.float32)


def e8m0_to_f32(e) -> np.ndarray:
    """E8M0 block scale: 2^(e - 127); 255 is NaN."""
    e = np.asarray(e, dtype=np.uint8).astype(np.float64)
    return np.where(e == 255, np.nan, np.exp2(e - 127.0)).astype(np.float32)


def mx_codes(packed, mode: str) -> np.ndarray:
    """Element codes of MX rows [rows, P] (uint32): 8 nibbles per word (mxfp4, element 2i in
    the low nibble of byte i) or 4 bytes per word (mxfp8), little-endian."""
    by = np.ascontiguousarray(np.asarray(packed, dtype=np.uint32)).view(np.uint8)
    by = by.reshape(*np.asarray(packed).shape[:-1], -1)
    if mode == "mxfp4":
        return np.stack([by & 15, by >> 4], axis=-1).reshape(*by.shape[:-1], -1)
    if mode == "mxfp8":
        return by
    raise ValueError(mode)


def mx_dequantize(packed, scales_u8, mode: str) -> np.ndarray:
    """W[n, k] = value(code[n, k]) * 2^(scale[n, k // 32] - 127) in fp32 (exact: a small
    float times a power of two)."""
    c = mx_codes(packed, mode)
    v = E2M1_TABLE[c] if mode == "mxfp4" else e4m3_to_f32(c)
    s = e8m0_to_f32(scales_u8)
    return (v.reshape(*c.shape[:-1], -1, MX_BLOCK) * s[..., None]).reshape(c.shape)


def mx_quantized_matmul(x_f32, packed, scales_u8, mode: str) -> np.ndarray:
    """y = x @ mx_dequantize(W)^T accumulated in fp64."""
    W = mx_dequantize(packed, scales_u8, mode).astype(np.float64)
    return np.asarray(x_f32, dtype=np.float64) @ W.T


# ----------------------------------------------------------------------------- metrics


def rel_l2(a, b) -> float:
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    den = math.sqrt(float((b * b).sum()))
    return math.sqrt(float(((a - b) ** 2).sum())) / (den if den > 0 else 1.0)


def max_abs(a, b) -> float:
    return float(np.max(np.abs(np.asarray(a, np.float64) - np.asarray(b, np.float64)), initial=0.0))

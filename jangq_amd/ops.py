"""Operator API of the quantized-weight matmul path, mirroring MLX's affine operators.

Signatures follow the calls the reference makes:
  quantized_matmul  jang-tools/jang_tools/jangrt/linear.py:41-45, dots3/ops.py:44-51
  gather_qmm        jang-tools/jang_tools/dsv41/model.py:855-857, dots3/ops.py:168-192
  dequantize        jang-tools/jang_tools/loader.py:469, tests/mimo_v2_affine_codec_test.py:30-38
  quantize          jang-tools/jang_tools/convert.py:622-632 (mx.quantize), affine.py:193-276
Arrays are torch tensors on the GPU; every operator runs a gfx950 kernel of
``libjangq_amd.so`` on the current stream. Shapes and dtypes are checked here; the C ABI
re-validates and its error codes surface as ValueError.
"""
from __future__ import annotations

import ctypes as _ctypes
import math

import torch

from . import _lib
from ._lib import JQ_BF16, JQ_F16, JQ_F32

SUPPORTED_BITS = (2, 3, 4, 5, 6, 8)
SUPPORTED_GROUP_SIZES = (32, 64, 128)

_DT = {torch.float32: JQ_F32, torch.bfloat16: JQ_BF16, torch.float16: JQ_F16}


def _dtype_code(t: torch.Tensor, what: str) -> int:
    try:
        return _DT[t.dtype]
    except KeyError:
        raise ValueError(f"{what}: unsupported dtype {t.dtype}") from None


# The current device's current stream as a raw handle: torch's own accessor when it has one
# (torch.cuda.current_stream() builds a Stream object and re-resolves the device, several
# microseconds of host time per launch), else the public API.
if hasattr(torch._C, "_cuda_getCurrentRawStream") and hasattr(torch._C, "_cuda_getDevice"):
    _raw_stream, _cur_dev = torch._C._cuda_getCurrentRawStream, torch._C._cuda_getDevice

    def _stream() -> int:
        return _raw_stream(_cur_dev())
else:
    def _stream() -> int:
        return torch.cuda.current_stream().cuda_stream


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _dev(t: torch.Tensor, what: str) -> torch.Tensor:
    """Contiguous GPU operand whose base address is 16-byte aligned (the kernels issue
    16-byte vector loads from it)."""
    if not t.is_cuda:
        raise ValueError(f"{what} must be a GPU tensor (got {t.device})")
    t = t.contiguous()
    if t.data_ptr() % 16:
        t = t.clone()
    return t


def _codes(w: torch.Tensor) -> torch.Tensor:
    if w.dtype not in (torch.uint32, torch.int32):
        raise ValueError(f"packed weight must be uint32 (got {w.dtype})")
    return _dev(w, "packed weight")


def _out(out: torch.Tensor | None, shape, like: torch.Tensor, what: str = "out") -> torch.Tensor:
    """The caller's output tensor, checked (shape, contiguity, device, 16-byte alignment:
    the kernels write it with vector stores), or a new one of x's dtype."""
    shape = tuple(int(d) for d in shape)
    if out is None:
        return torch.empty(shape, dtype=like.dtype, device=like.device)
    if tuple(out.shape) != shape:
        raise ValueError(f"{what} must have shape {shape}, got {tuple(out.shape)}")
    if out.dtype not in _DT:
        raise ValueError(f"{what}: unsupported dtype {out.dtype}")
    if out.device != like.device:
        raise ValueError(f"{what} must be on {like.device}, got {out.device}")
    if not out.is_contiguous() or out.data_ptr() % 16:
        raise ValueError(f"{what} must be contiguous and 16-byte aligned")
    return out


def _sidecars(scales: torch.Tensor, biases: torch.Tensor):
    """Scales and biases as GPU operands of one dtype (the kernels read both as scales.dtype)."""
    if biases is None:
        raise ValueError("affine mode needs biases")
    if scales.dtype != biases.dtype:
        raise ValueError(f"scales ({scales.dtype}) and biases ({biases.dtype}) must share a dtype")
    return _dev(scales, "scales"), _dev(biases, "biases")


MX_MODES = {"mxfp4": 4, "mxfp8": 8}


def _check_mode(mode: str, transpose: bool) -> None:
    if mode != "affine" and mode not in MX_MODES:
        raise ValueError(f"mode={mode!r}: the modes are affine, mxfp4 and mxfp8")
    if not transpose:
        raise ValueError("transpose=False is not supported (every reference call uses transpose=True)")


def _check_bits_gs(bits: int, group_size: int) -> None:
    if bits not in SUPPORTED_BITS:
        raise ValueError(f"unsupported bits={bits}; expected one of {SUPPORTED_BITS}")
    if group_size not in SUPPORTED_GROUP_SIZES:
        raise ValueError(
            f"unsupported group_size={group_size}; expected one of {SUPPORTED_GROUP_SIZES}")


def packed_in_features(w: torch.Tensor, bits: int) -> int:
    """Logical input dimension K of a packed weight: last dim * 32 / bits."""
    return w.shape[-1] * 32 // bits


def unpack(w: torch.Tensor, bits: int) -> torch.Tensor:
    """Codes as uint8 [..., K] (pack.py:85-149 applied row-wise to a uint32 matrix)."""
    if bits not in SUPPORTED_BITS:
        raise ValueError(f"unsupported bits={bits}")
    w = _codes(w)
    K = packed_in_features(w, bits)
    if (w.shape[-1] * 32) % bits:
        raise ValueError("packed width is not a whole number of codes")
    rows = math.prod(w.shape[:-1])
    out = torch.empty((*w.shape[:-1], K), dtype=torch.uint8, device=w.device)
    _lib.check(_lib.lib().jq_unpack(_ptr(w), bits, rows, K, _ptr(out), _stream()), "unpack")
    return out


def dequantize(w: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor,
               group_size: int = 64, bits: int = 4, mode: str = "affine",
               dtype: torch.dtype | None = None) -> torch.Tensor:
    """W = q*scale + bias per group, fp32 arithmetic, returned as ``dtype`` (default
    scales.dtype, as mx.dequantize). 2-D or stacked [E, N, P] weights."""
    _check_mode(mode, True)
    if mode in MX_MODES:
        return _mx_dequantize(w, scales, group_size, bits, mode, dtype or torch.bfloat16)
    _check_bits_gs(bits, group_size)
    w = _codes(w)
    scales, biases = _sidecars(scales, biases)
    K = packed_in_features(w, bits)
    if scales.shape != biases.shape or scales.shape[:-1] != w.shape[:-1]:
        raise ValueError(f"shape mismatch: w {tuple(w.shape)}, scales {tuple(scales.shape)}, "
                         f"biases {tuple(biases.shape)}")
    if scales.shape[-1] * group_size != K:
        raise ValueError(f"scales width {scales.shape[-1]} x group_size {group_size} != K {K}")
    out_dtype = dtype or scales.dtype
    rows = math.prod(w.shape[:-1])
    out = torch.empty((*w.shape[:-1], K), dtype=out_dtype, device=w.device)
    _lib.check(_lib.lib().jq_dequantize(
        _ptr(w), _ptr(scales), _ptr(biases), _dtype_code(scales, "scales"), bits, group_size,
        rows, K, _ptr(out), _dtype_code(out, "output"), _stream()), "dequantize")
    return out


def quantize(w: torch.Tensor, group_size: int = 64, bits: int = 4, mode: str = "affine",
             scales_dtype: torch.dtype | None = None):
    """Affine group quantization with mx.quantize's rule. Returns (w_q uint32 [..., K*bits/32],
    scales, biases) with scales/biases in ``scales_dtype`` (default w.dtype, as MLX)."""
    _check_mode(mode, True)
    _check_bits_gs(bits, group_size)
    w = _dev(w, "weights")
    K = w.shape[-1]
    if K % group_size:
        raise ValueError(f"input dimension {K} is not divisible by group_size={group_size}")
    sdt = scales_dtype or w.dtype
    rows = math.prod(w.shape[:-1])
    lead = tuple(w.shape[:-1])
    wq = torch.empty((*lead, K * bits // 32), dtype=torch.int32, device=w.device)
    scales = torch.empty((*lead, K // group_size), dtype=sdt, device=w.device)
    biases = torch.empty_like(scales)
    _lib.check(_lib.lib().jq_quantize(
        _ptr(w), _dtype_code(w, "weights"), bits, group_size, rows, K, _ptr(wq), _ptr(scales),
        _ptr(biases), _dtype_code(scales, "scales"), _stream()), "quantize")
    return wq.view(torch.uint32), scales, biases


def _mx_check(w, scales, group_size, bits, mode):
    if group_size != 32 or bits != MX_MODES[mode]:
        raise ValueError(f"mode={mode!r} needs group_size=32 and bits={MX_MODES[mode]}")
    w = _codes(w)
    scales = _dev(scales, "scales")
    if scales.dtype != torch.uint8:
        raise ValueError(f"{mode} scales are uint8 E8M0 exponents, got {scales.dtype}")
    K = w.shape[-1] * 32 // bits
    if tuple(scales.shape) != (*w.shape[:-1], K // 32):
        raise ValueError(f"scales must be {(*w.shape[:-1], K // 32)}, got {tuple(scales.shape)}")
    return w, scales, K


def _mx_dequantize(w, scales, group_size, bits, mode, dtype):
    """mx.dequantize for the MX modes: value(code) * 2^(scale - 127), exact in fp32."""
    w, scales, K = _mx_check(w, scales, group_size, bits, mode)
    out = torch.empty((*w.shape[:-1], K), dtype=dtype, device=w.device)
    _lib.check(_lib.lib().jq_mx_dequantize(_ptr(w), _ptr(scales), bits, math.prod(w.shape[:-1]),
                                           K, _ptr(out), _dtype_code(out, "output"), _stream()),
               "dequantize")
    return out


def _mx_matmul(x, w, scales, group_size, bits, mode, out):
    """mx.quantized_matmul for the MX modes (no biases): decode GEMVs, one per activation row."""
    w, scales, K = _mx_check(w, scales, group_size, bits, mode)
    x = _dev(x, "x")
    if w.dim() != 2 or x.shape[-1] != K:
        raise ValueError(f"x last dim {x.shape[-1]} / w {tuple(w.shape)} do not match K {K}")
    N, M = w.shape[0], math.prod(x.shape[:-1])
    out = _out(out, (*x.shape[:-1], N), x)
    _lib.check(_lib.lib().jq_mx_quantized_matmul(
        _ptr(x), _dtype_code(x, "x"), _ptr(w), _ptr(scales), bits, M, N, K, _ptr(out),
        _dtype_code(out, "output"), _stream()), "quantized_matmul")
    return out


def quantized_matmul(x: torch.Tensor, w: torch.Tensor, scales: torch.Tensor,
                     biases: torch.Tensor, transpose: bool = True, group_size: int = 64,
                     bits: int = 4, mode: str = "affine", *,
                     out: torch.Tensor | None = None) -> torch.Tensor:
    """y = x @ dequantize(w)^T with fp32 accumulation; y has x's dtype and shape [..., N]."""
    _check_mode(mode, transpose)
    if mode in MX_MODES:
        return _mx_matmul(x, w, scales, group_size, bits, mode, out)
    _check_bits_gs(bits, group_size)
    x = _dev(x, "x")
    w = _codes(w)
    scales, biases = _sidecars(scales, biases)
    if w.dim() != 2:
        raise ValueError(f"quantized_matmul expects a 2-D packed weight, got {tuple(w.shape)}")
    N = w.shape[0]
    K = packed_in_features(w, bits)
    if x.shape[-1] != K:
        raise ValueError(f"x last dim {x.shape[-1]} != K {K} (w {tuple(w.shape)}, bits {bits})")
    if tuple(scales.shape) != (N, K // group_size) or scales.shape != biases.shape:
        raise ValueError(f"scales/biases must be {(N, K // group_size)}, got "
                         f"{tuple(scales.shape)} / {tuple(biases.shape)}")
    M = math.prod(x.shape[:-1])
    out = _out(out, (*x.shape[:-1], N), x)
    lib = _lib.lib()
    xd, sd = _dtype_code(x, "x"), _dtype_code(scales, "scales")
    # Decode batches of long rows split K over the kernel's items (fp32 partials in a
    # workspace); the size query is 0 for every other shape.
    nws = lib.jq_quantized_matmul_workspace_size(M, N, K, bits, group_size, xd, sd)
    if nws > 0:
        ws = torch.empty(nws, dtype=torch.uint8, device=x.device)
        _lib.check(lib.jq_quantized_matmul_ws(
            _ptr(x), xd, _ptr(w), _ptr(scales), _ptr(biases), sd, bits, group_size, M, N, K,
            _ptr(out), _dtype_code(out, "output"), _ptr(ws), nws, _stream()), "quantized_matmul")
        return out
    _lib.check(lib.jq_quantized_matmul(
        _ptr(x), xd, _ptr(w), _ptr(scales), _ptr(biases), sd, bits, group_size, M, N, K,
        _ptr(out), _dtype_code(out, "output"), _stream()), "quantized_matmul")
    return out


def quantized_matmul_multi(x: torch.Tensor, weights, *, outs=None):
    """Several projections of the same x (q/k/v, gate/up) in one launch where they share
    bits, group_size and K; ``weights`` is a sequence of (w, scales, biases, group_size,
    bits). Returns the list of outputs [..., N_i] in x.dtype."""
    x = _dev(x, "x")
    n = len(weights)
    K = x.shape[-1]
    M = math.prod(x.shape[:-1])
    keep, ys, ws, ss, bs, bits_l, gs_l, ns = [], [], [], [], [], [], [], []
    if outs is not None and len(outs) != n:
        raise ValueError(f"outs holds {len(outs)} tensors for {n} weights")
    for i, (w, s, b, gs, bits) in enumerate(weights):
        _check_bits_gs(bits, gs)
        w = _codes(w)
        s, b = _sidecars(s, b)
        if w.dim() != 2 or packed_in_features(w, bits) != K:
            raise ValueError(f"weight {i}: K mismatch")
        if tuple(s.shape) != (w.shape[0], K // gs) or s.shape != b.shape:
            raise ValueError(f"weight {i}: scales/biases must be {(w.shape[0], K // gs)}")
        if s.dtype != weights[0][1].dtype:
            raise ValueError("all scales must share a dtype")
        y = _out(None if outs is None else outs[i], (*x.shape[:-1], w.shape[0]), x, f"outs[{i}]")
        if y.dtype != x.dtype:
            raise ValueError(f"outs[{i}] must have x's dtype {x.dtype}")
        keep += [w, s, b]
        ys.append(y)
        ws.append(w.data_ptr()); ss.append(s.data_ptr()); bs.append(b.data_ptr())
        bits_l.append(bits); gs_l.append(gs); ns.append(w.shape[0])
    ptrs = lambda vals: (_ctypes.c_void_p * n)(*vals)  # noqa: E731
    st = _lib.lib().jq_quantized_matmul_multi(
        n, ptrs([x.data_ptr()] * n), _dtype_code(x, "x"), ptrs(ws), ptrs(ss), ptrs(bs),
        _dtype_code(weights[0][1], "scales"), (_ctypes.c_int * n)(*bits_l),
        (_ctypes.c_int * n)(*gs_l), (_ctypes.c_int64 * n)(*([M] * n)),
        (_ctypes.c_int64 * n)(*ns), (_ctypes.c_int64 * n)(*([K] * n)),
        ptrs([y.data_ptr() for y in ys]), _dtype_code(x, "output"), _stream())
    _lib.check(st, "quantized_matmul_multi")
    return ys


def _expert_projs(gate, up, down, group_size):
    """The (codes, scales, biases, bits) of a SwitchGLU's three stacked projections, checked:
    gate and up share a bit width, and every scale and bias tensor shares one dtype."""
    out = []
    for what, (w, s, b, bits) in (("gate", gate), ("up", up), ("down", down)):
        _check_bits_gs(bits, group_size)
        s, b = _sidecars(s, b)
        w = _codes(w)
        if (w.dim() != 3 or s.dim() != 3 or s.shape != b.shape or s.shape[:2] != w.shape[:2]
                or s.shape[2] * group_size != packed_in_features(w, bits)):
            raise ValueError(f"{what}: stacked weights [E, N, K*bits/32] need scales/biases "
                             f"[E, N, K/{group_size}]")
        out.append((w, s, b, bits))
    if out[1][3] != out[0][3]:
        raise ValueError("gate and up projections must share a bit width")
    if len({o[1].dtype for o in out}) != 1:
        raise ValueError("the three projections' scales must share a dtype")
    return out


def _gather_workspace(n_pairs: int, E: int, M: int, device) -> torch.Tensor:
    size = _lib.lib().jq_gather_workspace_size(n_pairs, E, M)
    if size < 0:
        raise ValueError("invalid gather workspace request")
    return torch.empty(max(size, 256), dtype=torch.uint8, device=device)


def gather_qmm(x: torch.Tensor, w: torch.Tensor, scales: torch.Tensor,
               biases: torch.Tensor | None = None, lhs_indices: torch.Tensor | None = None,
               rhs_indices: torch.Tensor | None = None, transpose: bool = True,
               group_size: int = 64, bits: int = 4, mode: str = "affine",
               sorted_indices: bool = False) -> torch.Tensor:
    """out[i] = x[lhs[i]] @ dequantize(w[rhs[i]])^T, MLX broadcasting rules.

    x [*B, M, K]; w [E, N, P]; lhs indexes the flattened batch of x (default: every batch
    entry, broadcast against rhs); rhs indexes experts (default: arange(E)).
    Output [*broadcast(lhs, rhs), M, N] in x.dtype."""
    _check_mode(mode, transpose)
    if mode in MX_MODES:
        return _mx_gather(x, w, scales, lhs_indices, rhs_indices, group_size, bits, mode)
    _check_bits_gs(bits, group_size)
    x = _dev(x, "x")
    w = _codes(w)
    scales, biases = _sidecars(scales, biases)
    if w.dim() != 3:
        raise ValueError(f"gather_qmm expects stacked weights [E, N, P], got {tuple(w.shape)}")
    if x.dim() < 2:
        raise ValueError("x must have at least 2 dims [..., M, K]")
    E, N = w.shape[0], w.shape[1]
    K = packed_in_features(w, bits)
    if x.shape[-1] != K:
        raise ValueError(f"x last dim {x.shape[-1]} != K {K}")
    if tuple(scales.shape) != (E, N, K // group_size) or scales.shape != biases.shape:
        raise ValueError("scales/biases shape mismatch")
    M = x.shape[-2]
    bshape = tuple(x.shape[:-2])
    Bx = math.prod(bshape)
    dev = x.device
    if lhs_indices is None:
        lhs_indices = torch.arange(Bx, device=dev, dtype=torch.int32).reshape(bshape)
    if rhs_indices is None:
        rhs_indices = torch.arange(E, device=dev, dtype=torch.int32)
    lhs_b, rhs_b = torch.broadcast_tensors(lhs_indices.to(dev), rhs_indices.to(dev))
    ishape = tuple(lhs_b.shape)
    lhs_f = lhs_b.reshape(-1).to(torch.int32).contiguous()
    rhs_f = rhs_b.reshape(-1).to(torch.int32).contiguous()
    n_pairs = lhs_f.numel()
    out = torch.empty((*ishape, M, N), dtype=x.dtype, device=dev)
    if n_pairs == 0:
        return out
    ws = _gather_workspace(n_pairs, E, M, dev)
    _lib.check(_lib.lib().jq_gather_qmm(
        _ptr(x), _dtype_code(x, "x"), Bx, M, _ptr(w), _ptr(scales), _ptr(biases),
        _dtype_code(scales, "scales"), bits, group_size, E, N, K, _ptr(lhs_f), _ptr(rhs_f),
        n_pairs, int(sorted_indices), _ptr(out), _dtype_code(out, "output"), _ptr(ws),
        ws.numel(), _stream()), "gather_qmm")
    return out


def _route_opts(score: str, renorm: bool, renorm_eps: float | None, scaling: float,
                score_bias: torch.Tensor | None, n_group: int, topk_group: int, E: int, device):
    """(jq_route_opts, tensors to keep alive) after the host-side checks."""
    if score not in _lib.JQ_SCORE:
        raise ValueError(f"score={score!r}: expected one of {tuple(_lib.JQ_SCORE)}")
    keep = []
    bias_ptr = None
    if score_bias is not None:
        b = _dev(score_bias, "score_bias").float().contiguous()
        if b.numel() != E:
            raise ValueError(f"score_bias must hold {E} values, got {b.numel()}")
        keep.append(b)
        bias_ptr = b.data_ptr()
    if n_group > 1 and (E % n_group or not 1 <= topk_group <= n_group or n_group > 64):
        raise ValueError(f"n_group={n_group}, topk_group={topk_group} do not fit {E} experts")
    eps = (0.0 if score == "softmax" else 1e-20) if renorm_eps is None else float(renorm_eps)
    o = _lib.RouteOpts(_lib.JQ_SCORE[score], int(bool(renorm)), eps, float(scaling), bias_ptr,
                       max(int(n_group), 1), int(topk_group))
    return o, keep


def _mx_gather(x, w, scales, lhs_indices, rhs_indices, group_size, bits, mode):
    """gather_qmm over an MX-mode expert stack (no biases): one gathered GEMV launch per call,
    every (pair, activation row) its own row of the grid."""
    w, scales, K = _mx_check(w, scales, group_size, bits, mode)
    x = _dev(x, "x")
    if w.dim() != 3 or x.dim() < 2 or x.shape[-1] != K:
        raise ValueError(f"MX gather_qmm: x {tuple(x.shape)} / w {tuple(w.shape)} do not match")
    E, N = w.shape[0], w.shape[1]
    M = x.shape[-2]
    bshape = tuple(x.shape[:-2])
    Bx = math.prod(bshape)
    dev = x.device
    if lhs_indices is None:
        lhs_indices = torch.arange(Bx, device=dev, dtype=torch.int32).reshape(bshape)
    if rhs_indices is None:
        rhs_indices = torch.arange(E, device=dev, dtype=torch.int32)
    lhs_b, rhs_b = torch.broadcast_tensors(lhs_indices.to(dev), rhs_indices.to(dev))
    ishape = tuple(lhs_b.shape)
    lhs_f = lhs_b.reshape(-1).to(torch.int32).contiguous()
    rhs_f = rhs_b.reshape(-1).to(torch.int32).contiguous()
    n = lhs_f.numel()
    out = torch.empty((*ishape, M, N), dtype=x.dtype, device=dev)
    if n == 0:
        return out
    _lib.check(_lib.lib().jq_mx_gather_qmm(
        _ptr(x), _dtype_code(x, "x"), Bx, M, _ptr(w), _ptr(scales), bits, E, N, K, _ptr(lhs_f),
        _ptr(rhs_f), n, _ptr(out), _dtype_code(out, "output"), _stream()), "gather_qmm")
    return out


def swiglu(g: torch.Tensor, u: torch.Tensor, swiglu_limit: float = 0.0) -> torch.Tensor:
    """round(silu(g) * u) elementwise (g, u already in their dtype), with the optional clamp."""
    g, u = _dev(g, "g"), _dev(u, "u")
    if g.shape != u.shape or g.dtype != u.dtype:
        raise ValueError("g and u must share shape and dtype")
    h = torch.empty_like(g)
    _lib.check(_lib.lib().jq_swiglu(_ptr(g), _ptr(u), g.numel(), float(swiglu_limit), _ptr(h),
                                    _dtype_code(g, "g"), _stream()), "swiglu")
    return h


def moe_route(logits: torch.Tensor, k: int, renorm: bool = True, *, score: str = "softmax",
              score_bias: torch.Tensor | None = None, n_group: int = 1, topk_group: int = 1,
              renorm_eps: float | None = None, scaling: float = 1.0):
    """Router top-k: scores from the logits (softmax, sigmoid or sqrt-softplus), the k experts
    of largest score (+ score_bias, for the selection only; optionally group-limited) in
    descending order, and their unbiased scores, optionally divided by (sum + renorm_eps) and
    times ``scaling`` (qwen4_exp/modeling.py:587-593, mistral4_mlx.py:355-387,
    dots3/ops.py:149-162, laguna/model.py:50-62, dsv41/model.py:1184-1190). renorm_eps
    defaults to 0 for softmax and 1e-20 for the sigmoid-type routers. Logits may be the
    router's bf16/f16 output (read exactly) or f32."""
    logits = _dev(logits, "logits")
    E = logits.shape[-1]
    T = math.prod(logits.shape[:-1])
    if not 1 <= k <= min(E, 64):
        raise ValueError(f"k={k} must lie in [1, min(E, 64)]")
    o, keep = _route_opts(score, renorm, renorm_eps, scaling, score_bias, n_group, topk_group, E,
                          logits.device)
    idx = torch.empty((*logits.shape[:-1], k), dtype=torch.int32, device=logits.device)
    wts = torch.empty((*logits.shape[:-1], k), dtype=torch.float32, device=logits.device)
    _lib.check(_lib.lib().jq_moe_route_ex(_ptr(logits), _dtype_code(logits, "logits"), T, E, k,
                                          _ctypes.byref(o), _ptr(idx), _ptr(wts), _stream()),
               "moe_route")
    del keep
    return idx, wts


def switch_glu(x: torch.Tensor, indices: torch.Tensor, gate, up, down, group_size: int = 64):
    """SwitchGLU over stacked experts (mlx_lm SwitchGLU.__call__, restated at
    dots3/ops.py:195-223): out[..., j, :] = down_e(silu(gate_e(x)) * up_e(x)), e = indices[..., j].

    gate/up/down are (w, scales, biases, bits) tuples of stacked expert weights. One grouped
    launch computes gate+up+SiLU for every active expert, a second the down projection."""
    x = _dev(x, "x")
    indices = _dev(indices, "indices")
    (gw, gsc, gb, bits_gu), (uw, usc, ub, bits_u), (dw, dsc, db, bits_d) = _expert_projs(
        gate, up, down, group_size)
    E, I = gw.shape[0], gw.shape[1]
    H = x.shape[-1]
    k = indices.shape[-1]
    if packed_in_features(gw, bits_gu) != H or dw.shape[1] != H or packed_in_features(dw, bits_d) != I:
        raise ValueError("expert weight shapes do not match x / each other")
    T = math.prod(x.shape[:-1])
    if math.prod(indices.shape[:-1]) != T:
        raise ValueError("indices leading dims must match x")
    idx = indices.reshape(T, k).to(torch.int32).contiguous()
    h = torch.empty((T * k, I), dtype=x.dtype, device=x.device)
    out = torch.empty((*x.shape[:-1], k, H), dtype=x.dtype, device=x.device)
    ws = _gather_workspace(T * k, E, 1, x.device)
    sdt = _dtype_code(gsc, "scales")
    _lib.check(_lib.lib().jq_switch_glu(
        _ptr(x), _dtype_code(x, "x"), T, H, I, E, _ptr(idx), k,
        _ptr(gw), _ptr(gsc), _ptr(gb),
        _ptr(uw), _ptr(usc), _ptr(ub), bits_gu,
        _ptr(dw), _ptr(dsc), _ptr(db), bits_d, sdt, group_size,
        _ptr(h), _ptr(out), _dtype_code(out, "output"), _ptr(ws), ws.numel(), _stream()),
        "switch_glu")
    return out


def switch_glu_combine(x: torch.Tensor, indices: torch.Tensor, weights: torch.Tensor, gate, up,
                       down, group_size: int = 64,
                       shared: torch.Tensor | None = None) -> torch.Tensor:
    """moe_combine(switch_glu(x, indices, gate, up, down), weights, shared) as one call: the
    routed half of a MoE block (qwen4_exp/modeling.py:594-597; the two-dispatch fused decode
    of dsv41/metal_decode.py:334-503). Same values and roundings as the two calls; at decode
    sizes the combine runs inside the down-projection launch."""
    x = _dev(x, "x")
    indices = _dev(indices, "indices")
    (gw, gsc, gb, bits_gu), (uw, usc, ub, bits_u), (dw, dsc, db, bits_d) = _expert_projs(
        gate, up, down, group_size)
    E, I = gw.shape[0], gw.shape[1]
    H = x.shape[-1]
    k = indices.shape[-1]
    if packed_in_features(gw, bits_gu) != H or dw.shape[1] != H or packed_in_features(dw, bits_d) != I:
        raise ValueError("expert weight shapes do not match x / each other")
    T = math.prod(x.shape[:-1])
    if math.prod(indices.shape[:-1]) != T:
        raise ValueError("indices leading dims must match x")
    w = _dev(weights, "weights")
    if tuple(w.shape) != tuple(indices.shape):
        raise ValueError(f"weights must be {tuple(indices.shape)}, got {tuple(w.shape)}")
    w = w.reshape(T, k).float().contiguous()
    if shared is not None:
        shared = _dev(shared, "shared")
        if tuple(shared.shape) != tuple(x.shape) or shared.dtype != x.dtype:
            raise ValueError("shared must match x's shape and dtype")
        shared = shared.contiguous()
    idx = indices.reshape(T, k).to(torch.int32).contiguous()
    h = torch.empty((T * k, I), dtype=x.dtype, device=x.device)
    ybuf = torch.empty((T * k, H), dtype=x.dtype, device=x.device)
    out = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    ws = _gather_workspace(T * k, E, 1, x.device)
    sdt = _dtype_code(gsc, "scales")
    _lib.check(_lib.lib().jq_switch_glu_combine(
        _ptr(x), _dtype_code(x, "x"), T, H, I, E, _ptr(idx), _ptr(w), k,
        _ptr(gw), _ptr(gsc), _ptr(gb),
        _ptr(uw), _ptr(usc), _ptr(ub), bits_gu,
        _ptr(dw), _ptr(dsc), _ptr(db), bits_d, sdt, group_size,
        _ptr(h), _ptr(ybuf), _ptr(shared), _ptr(out), _dtype_code(out, "output"), _ptr(ws),
        ws.numel(), _stream()), "switch_glu_combine")
    return out


def moe_experts(x: torch.Tensor, logits: torch.Tensor, k: int, gate, up, down,
                group_size: int = 64, shared: torch.Tensor | None = None,
                renorm: bool = True):
    """moe_route(logits, k, renorm) then switch_glu_combine(x, ...) with its ids and scores:
    the MoE block after the router GEMV (qwen4_exp/modeling.py:587-597). Returns
    (out, ids, scores). At decode sizes the gate|up launch routes for itself."""
    x = _dev(x, "x")
    logits = _dev(logits, "logits")
    if logits.dtype != torch.float32:
        logits = logits.float().contiguous()
    (gw, gsc, gb, bits_gu), (uw, usc, ub, bits_u), (dw, dsc, db, bits_d) = _expert_projs(
        gate, up, down, group_size)
    E, I = gw.shape[0], gw.shape[1]
    H = x.shape[-1]
    if packed_in_features(gw, bits_gu) != H or dw.shape[1] != H or packed_in_features(dw, bits_d) != I:
        raise ValueError("expert weight shapes do not match x / each other")
    T = math.prod(x.shape[:-1])
    if tuple(logits.shape) != (*x.shape[:-1], E):
        raise ValueError(f"logits must be {(*x.shape[:-1], E)}, got {tuple(logits.shape)}")
    if shared is not None:
        shared = _dev(shared, "shared")
        if tuple(shared.shape) != tuple(x.shape) or shared.dtype != x.dtype:
            raise ValueError("shared must match x's shape and dtype")
    idx = torch.empty((*x.shape[:-1], k), dtype=torch.int32, device=x.device)
    w = torch.empty((*x.shape[:-1], k), dtype=torch.float32, device=x.device)
    h = torch.empty((T * k, I), dtype=x.dtype, device=x.device)
    ybuf = torch.empty((T * k, H), dtype=x.dtype, device=x.device)
    out = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    ws = _gather_workspace(T * k, E, 1, x.device)
    _lib.check(_lib.lib().jq_moe_experts(
        _ptr(x), _dtype_code(x, "x"), T, H, I, E, _ptr(logits), k, int(renorm), _ptr(idx),
        _ptr(w), _ptr(gw), _ptr(gsc), _ptr(gb),
        _ptr(uw), _ptr(usc), _ptr(ub), bits_gu,
        _ptr(dw), _ptr(dsc), _ptr(db), bits_d,
        _dtype_code(gsc, "scales"), group_size, _ptr(h), _ptr(ybuf), _ptr(shared), _ptr(out),
        _dtype_code(out, "output"), _ptr(ws), ws.numel(), _stream()), "moe_experts")
    return out, idx, w


def _qweight(w, s, b, bits, group_size, what, keep):
    """jq_qweight of a checked (codes, scales, biases) triple."""
    _check_bits_gs(bits, group_size)
    w = _codes(w)
    s, b = _sidecars(s, b)
    if s.shape != b.shape or s.shape[:-1] != w.shape[:-1] or \
            s.shape[-1] * group_size != packed_in_features(w, bits):
        raise ValueError(f"{what}: scales/biases must be [..., rows, K/{group_size}]")
    keep += [w, s, b]
    return _lib.QWeight(w.data_ptr(), s.data_ptr(), b.data_ptr(), _dtype_code(s, "scales"),
                        bits, group_size), w


def moe_block(x: torch.Tensor, logits: torch.Tensor, k: int, gate, up, down,
              group_size: int = 64, *, shared=None, shared_gate: torch.Tensor | None = None,
              score: str = "softmax", renorm: bool = True, renorm_eps: float | None = None,
              scaling: float = 1.0, score_bias: torch.Tensor | None = None, n_group: int = 1,
              topk_group: int = 1, combine: str = "after", swiglu_limit: float = 0.0):
    """A MoE block after its router GEMV, in one call (jq_moe_block): routing (moe_route's
    options), the routed SwitchGLU (gate/up/down = (w, scales, biases, bits) stacks sharing
    ``group_size``), the optional shared expert (``shared`` = three (w, scales, biases,
    group_size, bits) tuples: gate, up, down) with its optional sigmoid gate (``shared_gate``,
    the [..., 1] output of the 1-row shared_expert_gate linear), and the combine:
      combine="after"   round(round(sum_j w_j * y_j) + shared term)  (qwen4_exp/modeling.py:594-599)
      combine="before"  routing weights multiply h before the down projection, then
                        round(sum_j y_j + shared)                    (dsv41/model.py:1214-1245)
    swiglu_limit > 0 clamps gate <= L and up to [-L, L] (routed and shared experts).
    Returns (out [..., H], ids [..., k], weights [..., k])."""
    x = _dev(x, "x")
    logits = _dev(logits, "logits")
    if combine not in _lib.JQ_COMBINE:
        raise ValueError(f"combine={combine!r}: expected 'after' or 'before'")
    keep = []
    qg, gw = _qweight(*gate, group_size, "gate", keep)
    qu, uw = _qweight(*up, group_size, "up", keep)
    qd, dw = _qweight(*down, group_size, "down", keep)
    if gate[3] != up[3]:
        raise ValueError("gate and up projections must share a bit width")
    if gw.dim() != 3 or uw.shape != gw.shape or dw.dim() != 3 or dw.shape[0] != gw.shape[0]:
        raise ValueError("gate/up/down must be expert stacks [E, N, P] of matching E")
    E, I = gw.shape[0], gw.shape[1]
    H = x.shape[-1]
    if packed_in_features(gw, gate[3]) != H or dw.shape[1] != H or \
            packed_in_features(dw, down[3]) != I:
        raise ValueError("expert weight shapes do not match x / each other")
    T = math.prod(x.shape[:-1])
    if tuple(logits.shape) != (*x.shape[:-1], E):
        raise ValueError(f"logits must be {(*x.shape[:-1], E)}, got {tuple(logits.shape)}")
    if not 1 <= k <= min(E, 64):
        raise ValueError(f"k={k} must lie in [1, min(E, 64)]")
    ro, rkeep = _route_opts(score, renorm, renorm_eps, scaling, score_bias, n_group, topk_group,
                            E, x.device)
    keep += rkeep
    sI = 0
    sq = [None, None, None]
    if shared is not None:
        (sgw, sgs, sgb, sgg, sgbits), (suw, sus, sub, sug, subits), (sdw, sds, sdb, sdg, sdbits) = shared
        if sgbits != subits or sgg != sug:
            raise ValueError("shared gate and up must share bits and group size")
        sq[0], sgw2 = _qweight(sgw, sgs, sgb, sgbits, sgg, "shared gate", keep)
        sq[1], suw2 = _qweight(suw, sus, sub, subits, sug, "shared up", keep)
        sq[2], sdw2 = _qweight(sdw, sds, sdb, sdbits, sdg, "shared down", keep)
        sI = sgw2.shape[0]
        if sgw2.dim() != 2 or suw2.shape != sgw2.shape or packed_in_features(sgw2, sgbits) != H \
                or tuple(sdw2.shape[:1]) != (H,) or packed_in_features(sdw2, sdbits) != sI:
            raise ValueError("shared expert shapes do not match x")
    sgl = None
    if shared_gate is not None:
        if shared is None:
            raise ValueError("shared_gate needs a shared expert")
        if combine != "after":
            raise ValueError("the gated shared term belongs to combine='after'")
        sgl = _dev(shared_gate, "shared_gate")
        if sgl.numel() != T or sgl.dtype != x.dtype:
            raise ValueError(f"shared_gate must hold {T} values of {x.dtype}")
    mo = _lib.MoeOpts(_lib.JQ_COMBINE[combine], float(swiglu_limit))
    lib = _lib.lib()
    xd = _dtype_code(x, "x")
    nws = lib.jq_moe_block_workspace_size(T, H, I, E, k, sI, xd)
    if nws < 0:
        raise ValueError("moe_block: invalid sizes")
    ws = torch.empty(max(nws, 256), dtype=torch.uint8, device=x.device)
    idx = torch.empty((*x.shape[:-1], k), dtype=torch.int32, device=x.device)
    w = torch.empty((*x.shape[:-1], k), dtype=torch.float32, device=x.device)
    out = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    ref = _ctypes.byref
    _lib.check(lib.jq_moe_block(
        _ptr(x), xd, T, H, I, E, k, _ptr(logits), _dtype_code(logits, "logits"), ref(ro),
        ref(qg), ref(qu), ref(qd), sI, ref(sq[0]) if sq[0] else None,
        ref(sq[1]) if sq[1] else None, ref(sq[2]) if sq[2] else None, _ptr(sgl), ref(mo),
        _ptr(idx), _ptr(w), _ptr(out), _ptr(ws), ws.numel(), _stream()), "moe_block")
    del keep
    return out, idx, w


def moe_combine(y: torch.Tensor, weights: torch.Tensor,
                shared: torch.Tensor | None = None) -> torch.Tensor:
    """sum_j weights[..., j] * y[..., j, :] in fp32 (slot order), in y.dtype, plus ``shared``
    (rounded again): one launch for ``(y * scores[..., None]).sum(-2) (+ shared_expert(x))``
    of qwen4_exp/modeling.py:594-597."""
    y = _dev(y, "expert outputs")
    w = _dev(weights, "weights")
    if w.dtype != torch.float32:
        w = w.float().contiguous()
    k, H = y.shape[-2], y.shape[-1]
    lead = tuple(y.shape[:-2])
    if tuple(w.shape) != (*lead, k):
        raise ValueError(f"weights must be {(*lead, k)}, got {tuple(w.shape)}")
    T = math.prod(lead)
    if shared is not None:
        shared = _dev(shared, "shared")
        if tuple(shared.shape) != (*lead, H) or shared.dtype != y.dtype:
            raise ValueError("shared must match the combined output's shape and dtype")
    out = torch.empty((*lead, H), dtype=y.dtype, device=y.device)
    _lib.check(_lib.lib().jq_moe_combine(_ptr(y), _ptr(w), _ptr(shared), T, k, H, _ptr(out),
                                         _dtype_code(y, "expert outputs"), _stream()),
               "moe_combine")
    return out


def quantized_swiglu(x: torch.Tensor, gate, up, group_size: int = 64, *,
                     swiglu_limit: float = 0.0) -> torch.Tensor:
    """silu(gate(x)) * up(x) of a dense MLP, each projection rounded to x.dtype first; gate and
    up are (w, scales, biases, bits) with the same bits, N and K. With swiglu_limit > 0 the
    rounded gate is clamped to <= L and up to [-L, L] first (dsv41/model.py:1239-1244). One
    launch at decode sizes."""
    x = _dev(x, "x")
    gw, gsc, gb, bits = gate
    uw, usc, ub, bits_u = up
    if bits_u != bits:
        raise ValueError("gate and up projections must share a bit width")
    _check_bits_gs(bits, group_size)
    gw, uw = _codes(gw), _codes(uw)
    gsc, gb = _sidecars(gsc, gb)
    usc, ub = _sidecars(usc, ub)
    if usc.dtype != gsc.dtype:
        raise ValueError("gate and up scales must share a dtype")
    N, K = gw.shape[0], packed_in_features(gw, bits)
    if tuple(uw.shape) != tuple(gw.shape) or x.shape[-1] != K:
        raise ValueError("gate / up / x shapes do not match")
    if tuple(gsc.shape) != (N, K // group_size) or usc.shape != gsc.shape:
        raise ValueError(f"gate/up scales and biases must be {(N, K // group_size)}")
    M = math.prod(x.shape[:-1])
    h = torch.empty((*x.shape[:-1], N), dtype=x.dtype, device=x.device)
    # The up projection's scratch (the library uses it only outside the one-launch decode
    # forms, whose conditions include the dtypes; always passing it keeps every case valid).
    up_buf = torch.empty_like(h)
    _lib.check(_lib.lib().jq_quantized_swiglu_ex(
        _ptr(x), _dtype_code(x, "x"), M, N, K, _ptr(gw), _ptr(gsc),
        _ptr(gb), _ptr(uw), _ptr(usc), _ptr(ub),
        _dtype_code(gsc, "scales"), bits, group_size, float(swiglu_limit), _ptr(h), _ptr(up_buf),
        _dtype_code(h, "output"), _stream()), "quantized_swiglu")
    return h


def expand_packed_1bit_to_2bit(w: torch.Tensor) -> torch.Tensor:
    """1-bit storage codes [..., P] (uint32) -> the same codes as 2-bit runtime codes
    [..., 2P]; scales and biases are unchanged (affine.py:402-416, lossless)."""
    w = _codes(w)
    out = torch.empty((*w.shape[:-1], 2 * w.shape[-1]), dtype=torch.int32, device=w.device)
    _lib.check(_lib.lib().jq_expand_1bit_to_2bit(_ptr(w), w.numel(), _ptr(out), _stream()),
               "expand_packed_1bit_to_2bit")
    return out.view(torch.uint32)


def dequantize_tensor(qweight: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor,
                      bits: int, shape, block_size: int = 64) -> torch.Tensor:
    """Dequantize a flat (v1) JANG tensor to fp32 (quantize.py:292-326): the codes of all
    blocks form one LSB-first stream (uint8 ``qweight``), block b covers flat elements
    [b*block_size, (b+1)*block_size) and uses scales[b], biases[b]; the result is cut to
    prod(shape) elements. Every block is a whole number of 32-bit words, so the stream is the
    row layout of a [n_blocks, block_size] matrix and runs on the row dequant kernel."""
    _check_bits_gs(bits, block_size)
    scales = _dev(scales, "scales").reshape(-1, 1)
    biases = _dev(biases, "biases").reshape(-1, 1)
    n_blocks = scales.shape[0]
    if biases.shape[0] != n_blocks or scales.dtype != biases.dtype:
        raise ValueError("scales and biases must be [n_blocks] of one dtype")
    total = math.prod(shape)
    if total > n_blocks * block_size:
        raise ValueError(f"shape {tuple(shape)} needs more than {n_blocks} blocks")
    nbytes = n_blocks * block_size * bits // 8
    q = _dev(qweight, "qweight").reshape(-1)
    if q.dtype != torch.uint8:
        raise ValueError("qweight must be the uint8 code stream")
    if q.numel() < nbytes:
        raise ValueError(f"qweight holds {q.numel()} bytes, the blocks need {nbytes}")
    words = q[:nbytes].view(torch.int32) if q.data_ptr() % 16 == 0 else q[:nbytes].clone().view(torch.int32)
    out = torch.empty((n_blocks, block_size), dtype=torch.float32, device=q.device)
    _lib.check(_lib.lib().jq_dequantize(
        _ptr(words), _ptr(scales), _ptr(biases), _dtype_code(scales, "scales"), bits, block_size,
        n_blocks, block_size, _ptr(out), JQ_F32, _stream()), "dequantize_tensor")
    return out.reshape(-1)[:total].reshape(tuple(shape))

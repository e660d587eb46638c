// Codec kernels: unpack, dequantize (bit-exact) and the affine quantizer.
//
// One thread owns one 32-code unit (BITS whole words). The codes array of a [rows, K]
// matrix is the contiguous sequence of its units, so unit u starts at word u*BITS and its
// group is (u*32)/group_size in the flattened [rows, K/group_size] scale array.
//
// This file is compiled with -ffp-contract=off: dequantization must round the product and
// the sum separately (numpy's q*s + b in jang-tools/jang_tools/affine.py:458-463 does).
#include "jq_common.h"

namespace {

using namespace jq;

template <int BITS>
__global__ void __launch_bounds__(256) unpack_kernel(const uint32_t* __restrict__ codes,
                                                     int64_t units, uint8_t* __restrict__ out) {
  for (int64_t u = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; u < units;
       u += (int64_t)gridDim.x * blockDim.x) {
    uint32_t w[BITS];
#pragma unroll
    for (int i = 0; i < BITS; ++i) w[i] = codes[u * BITS + i];
    uint32_t packed[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      uint32_t v = 0;
#pragma unroll
      for (int b = 0; b < 4; ++b) v |= unit_code_rt<BITS>(w, q * 4 + b) << (8 * b);
      packed[q] = v;
    }
    uint4* o = (uint4*)(out + u * 32);
    o[0] = make_uint4(packed[0], packed[1], packed[2], packed[3]);
    o[1] = make_uint4(packed[4], packed[5], packed[6], packed[7]);
  }
}

template <int BITS, int SB, int OUT>
__global__ void __launch_bounds__(256) dequant_kernel(const uint32_t* __restrict__ codes,
                                                      const void* __restrict__ scales,
                                                      const void* __restrict__ biases,
                                                      int gs_shift, int64_t units,
                                                      void* __restrict__ out) {
  for (int64_t u = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; u < units;
       u += (int64_t)gridDim.x * blockDim.x) {
    uint32_t w[BITS];
#pragma unroll
    for (int i = 0; i < BITS; ++i) w[i] = codes[u * BITS + i];
    const int64_t g = (u * 32) >> gs_shift;
    const float s = load_t<SB>(scales, g);
    const float b = load_t<SB>(biases, g);
    float v[32];
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      const float q = (float)unit_code_rt<BITS>(w, i);
      v[i] = __fadd_rn(__fmul_rn(q, s), b);
    }
    if constexpr (OUT == JQ_F32) {
      float4* o = (float4*)((float*)out + u * 32);
#pragma unroll
      for (int i = 0; i < 8; ++i) o[i] = make_float4(v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]);
    } else {
      uint32_t h[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        uint32_t a, c;
        if constexpr (OUT == JQ_BF16) {
          a = f32_to_bf16_bits(v[2 * i]);
          c = f32_to_bf16_bits(v[2 * i + 1]);
        } else {
          a = f32_to_f16_bits(v[2 * i]);
          c = f32_to_f16_bits(v[2 * i + 1]);
        }
        h[i] = a | (c << 16);
      }
      uint4* o = (uint4*)((uint16_t*)out + u * 32);
#pragma unroll
      for (int i = 0; i < 4; ++i) o[i] = make_uint4(h[4 * i], h[4 * i + 1], h[4 * i + 2], h[4 * i + 3]);
    }
  }
}

// The f16 sidecar guard of jang-tools/jang_tools/affine.py:43-51: a scale whose magnitude is
// below the smallest normal f16 (2^-14) is replaced by +-2^-14 (sign of the scale, + for 0).
JQ_DEV float f16_nonzero_scale(float s) {
  const float tiny = 6.103515625e-05f;
  if (fabsf(s) < tiny) return s < 0.0f ? -tiny : tiny;
  return s;
}

// One thread per group. MLX affine rule as mirrored by jang-tools/jang_tools/affine.py:227-252:
//   low = min(w), high = max(max(w), 0), scale = max((high-low)/(2^b-1), 1e-7)
//   dominant low edge (|low| > |high|): scale > 0, edge = low; else scale < 0, edge = high
//   q0 = rint(edge/scale); if q0 != 0: scale = edge/q0, bias = edge; else bias = 0
//   code = min(rint((w - bias)/scale), 2^b - 1)
// Codes are computed from the fp32 scale/bias; the stored sidecars are their rounding.
template <int BITS, int WDT, int SB>
__global__ void __launch_bounds__(256) quantize_kernel(const void* __restrict__ w, int gs,
                                                       int64_t groups,
                                                       uint32_t* __restrict__ codes,
                                                       void* __restrict__ scales,
                                                       void* __restrict__ biases) {
  const float bins = (float)((1 << BITS) - 1);
  for (int64_t g = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; g < groups;
       g += (int64_t)gridDim.x * blockDim.x) {
    const int64_t base = g * gs;
    float lo = INFINITY, hi = 0.0f;
    for (int i = 0; i < gs; ++i) {
      const float v = load_t<WDT>(w, base + i);
      lo = fminf(lo, v);
      hi = fmaxf(hi, v);
    }
    float scale = fmaxf(__fdiv_rn(hi - lo, bins), 1e-7f);
    const bool dominant_low = fabsf(lo) > fabsf(hi);
    scale = dominant_low ? scale : -scale;
    const float edge = dominant_low ? lo : hi;
    const float q0 = rintf(__fdiv_rn(edge, scale));
    const bool at_zero = q0 == 0.0f;
    if (!at_zero) scale = __fdiv_rn(edge, q0);
    const float bias = at_zero ? 0.0f : edge;

    // Pack gs codes (gs*BITS/32 words) LSB-first.
    uint32_t* out = codes + (base * BITS) / 32;
    uint64_t acc = 0;
    int nacc = 0, wi = 0;
    for (int i = 0; i < gs; ++i) {
      const float v = load_t<WDT>(w, base + i);
      float q = rintf(__fdiv_rn(v - bias, scale));
      q = fminf(fmaxf(q, 0.0f), bins);
      acc |= (uint64_t)(uint32_t)q << nacc;
      nacc += BITS;
      if (nacc >= 32) {
        out[wi++] = (uint32_t)acc;
        acc >>= 32;
        nacc -= 32;
      }
    }
    if constexpr (SB == JQ_F16) {
      store_t<JQ_F16>(scales, g, f16_nonzero_scale(scale));
    } else {
      store_t<SB>(scales, g, scale);
    }
    store_t<SB>(biases, g, bias);
  }
}

inline unsigned grid_for(int64_t n, int block) {
  int64_t g = (n + block - 1) / block;
  if (g > (int64_t)1 << 20) g = (int64_t)1 << 20;
  return (unsigned)(g < 1 ? 1 : g);
}

template <int BITS>
int launch_unpack(const uint32_t* codes, int64_t units, uint8_t* out, hipStream_t st) {
  unpack_kernel<BITS><<<grid_for(units, 256), 256, 0, st>>>(codes, units, out);
  return jqh::launch_status();
}

template <int BITS, int SB>
int launch_dequant_sb(const uint32_t* c, const void* s, const void* b, int gsh, int64_t units,
                      void* out, int od, hipStream_t st) {
  dim3 grid(grid_for(units, 256)), block(256);
  switch (od) {
    case JQ_F32: dequant_kernel<BITS, SB, JQ_F32><<<grid, block, 0, st>>>(c, s, b, gsh, units, out); break;
    case JQ_BF16: dequant_kernel<BITS, SB, JQ_BF16><<<grid, block, 0, st>>>(c, s, b, gsh, units, out); break;
    default: dequant_kernel<BITS, SB, JQ_F16><<<grid, block, 0, st>>>(c, s, b, gsh, units, out); break;
  }
  return jqh::launch_status();
}

template <int BITS>
int launch_dequant(const uint32_t* c, const void* s, const void* b, int sb, int gsh,
                   int64_t units, void* out, int od, hipStream_t st) {
  switch (sb) {
    case JQ_F32: return launch_dequant_sb<BITS, JQ_F32>(c, s, b, gsh, units, out, od, st);
    case JQ_BF16: return launch_dequant_sb<BITS, JQ_BF16>(c, s, b, gsh, units, out, od, st);
    default: return launch_dequant_sb<BITS, JQ_F16>(c, s, b, gsh, units, out, od, st);
  }
}

template <int BITS, int WDT>
int launch_quant_w(const void* w, int gs, int64_t groups, uint32_t* c, void* s, void* b, int sb,
                   hipStream_t st) {
  dim3 grid(grid_for(groups, 256)), block(256);
  switch (sb) {
    case JQ_F32: quantize_kernel<BITS, WDT, JQ_F32><<<grid, block, 0, st>>>(w, gs, groups, c, s, b); break;
    case JQ_BF16: quantize_kernel<BITS, WDT, JQ_BF16><<<grid, block, 0, st>>>(w, gs, groups, c, s, b); break;
    default: quantize_kernel<BITS, WDT, JQ_F16><<<grid, block, 0, st>>>(w, gs, groups, c, s, b); break;
  }
  return jqh::launch_status();
}

template <int BITS>
int launch_quant(const void* w, int wd, int gs, int64_t groups, uint32_t* c, void* s, void* b,
                 int sb, hipStream_t st) {
  switch (wd) {
    case JQ_F32: return launch_quant_w<BITS, JQ_F32>(w, gs, groups, c, s, b, sb, st);
    case JQ_BF16: return launch_quant_w<BITS, JQ_BF16>(w, gs, groups, c, s, b, sb, st);
    default: return launch_quant_w<BITS, JQ_F16>(w, gs, groups, c, s, b, sb, st);
  }
}

inline int gs_shift(int gs) { return gs == 32 ? 5 : gs == 64 ? 6 : 7; }

// 1-bit storage codes -> 2-bit runtime codes, losslessly (reference
// jang-tools/jang_tools/affine.py:402-416): code i of a source word (bit i) becomes the 2-bit
// field i of the destination stream, i.e. bit 2i of destination word 2w + i/16. Each thread
// spreads one source word: its low and high halves each go to the even bits of one word.
JQ_DEV uint32_t spread_even_bits(uint32_t h) {  // bits 0..15 of h -> bits 0, 2, ..., 30
  h &= 0xFFFFu;
  h = (h | (h << 8)) & 0x00FF00FFu;
  h = (h | (h << 4)) & 0x0F0F0F0Fu;
  h = (h | (h << 2)) & 0x33333333u;
  h = (h | (h << 1)) & 0x55555555u;
  return h;
}

__global__ void __launch_bounds__(256) expand1to2_kernel(const uint32_t* __restrict__ src,
                                                         int64_t words,
                                                         uint32_t* __restrict__ dst) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < words;
       i += (int64_t)gridDim.x * blockDim.x) {
    const uint32_t v = src[i];
    uint2 o;
    o.x = spread_even_bits(v);
    o.y = spread_even_bits(v >> 16);
    *(uint2*)(dst + 2 * i) = o;
  }
}

}  // namespace

extern "C" {

int jq_expand_1bit_to_2bit(const uint32_t* src, int64_t words, uint32_t* dst,
                           jq_stream_t stream) {
  if (words < 0) return JQ_ERR_SHAPE;
  if (words == 0) return JQ_OK;
  if (!src || !dst) return JQ_ERR_NULL;
  const int64_t blocks = (words + 255) / 256;
  expand1to2_kernel<<<(unsigned)(blocks < 16384 ? blocks : 16384), 256, 0, (hipStream_t)stream>>>(
      src, words, dst);
  return jqh::launch_status();
}

int jq_abi_version(void) { return JQ_ABI_VERSION; }

const char* jq_status_string(int status) {
  switch (status) {
    case JQ_OK: return "ok";
    case JQ_ERR_BITS: return "unsupported bits (expected 2, 3, 4, 5, 6 or 8)";
    case JQ_ERR_GROUP_SIZE: return "unsupported group_size (expected 32, 64 or 128 dividing K)";
    case JQ_ERR_SHAPE: return "invalid or inconsistent shape";
    case JQ_ERR_DTYPE: return "unsupported dtype";
    case JQ_ERR_NULL: return "null pointer for a non-empty operand";
    case JQ_ERR_LAUNCH: return "HIP launch error";
    case JQ_ERR_WORKSPACE: return "workspace missing or too small";
    case JQ_ERR_INDEX: return "index out of range";
    default: return "unknown status";
  }
}

int jq_unpack(const uint32_t* codes, int bits, int64_t rows, int64_t K, uint8_t* out,
              jq_stream_t stream) {
  if (!jqh::bits_ok(bits)) return JQ_ERR_BITS;
  if (rows < 0 || K < 0 || K % 32) return JQ_ERR_SHAPE;
  const int64_t units = rows * (K / 32);
  if (units == 0) return JQ_OK;
  if (!codes || !out) return JQ_ERR_NULL;
  hipStream_t st = (hipStream_t)stream;
  switch (bits) {
    case 2: return launch_unpack<2>(codes, units, out, st);
    case 3: return launch_unpack<3>(codes, units, out, st);
    case 4: return launch_unpack<4>(codes, units, out, st);
    case 5: return launch_unpack<5>(codes, units, out, st);
    case 6: return launch_unpack<6>(codes, units, out, st);
    default: return launch_unpack<8>(codes, units, out, st);
  }
}

int jq_dequantize(const uint32_t* codes, const void* scales, const void* biases, int sb_dtype,
                  int bits, int group_size, int64_t rows, int64_t K, void* out, int out_dtype,
                  jq_stream_t stream) {
  int st0 = jqh::check_qshape(bits, group_size, rows, K);
  if (st0) return st0;
  if (!jqh::dtype_ok(sb_dtype) || !jqh::dtype_ok(out_dtype)) return JQ_ERR_DTYPE;
  const int64_t units = rows * (K / 32);
  if (units == 0) return JQ_OK;
  if (!codes || !scales || !biases || !out) return JQ_ERR_NULL;
  hipStream_t st = (hipStream_t)stream;
  const int gsh = gs_shift(group_size);
  switch (bits) {
    case 2: return launch_dequant<2>(codes, scales, biases, sb_dtype, gsh, units, out, out_dtype, st);
    case 3: return launch_dequant<3>(codes, scales, biases, sb_dtype, gsh, units, out, out_dtype, st);
    case 4: return launch_dequant<4>(codes, scales, biases, sb_dtype, gsh, units, out, out_dtype, st);
    case 5: return launch_dequant<5>(codes, scales, biases, sb_dtype, gsh, units, out, out_dtype, st);
    case 6: return launch_dequant<6>(codes, scales, biases, sb_dtype, gsh, units, out, out_dtype, st);
    default: return launch_dequant<8>(codes, scales, biases, sb_dtype, gsh, units, out, out_dtype, st);
  }
}

int jq_quantize(const void* w, int w_dtype, int bits, int group_size, int64_t rows, int64_t K,
                uint32_t* codes, void* scales, void* biases, int sb_dtype, jq_stream_t stream) {
  int st0 = jqh::check_qshape(bits, group_size, rows, K);
  if (st0) return st0;
  if (!jqh::dtype_ok(w_dtype) || !jqh::dtype_ok(sb_dtype)) return JQ_ERR_DTYPE;
  const int64_t groups = rows * (K / group_size);
  if (groups == 0) return JQ_OK;
  if (!w || !codes || !scales || !biases) return JQ_ERR_NULL;
  hipStream_t st = (hipStream_t)stream;
  switch (bits) {
    case 2: return launch_quant<2>(w, w_dtype, group_size, groups, codes, scales, biases, sb_dtype, st);
    case 3: return launch_quant<3>(w, w_dtype, group_size, groups, codes, scales, biases, sb_dtype, st);
    case 4: return launch_quant<4>(w, w_dtype, group_size, groups, codes, scales, biases, sb_dtype, st);
    case 5: return launch_quant<5>(w, w_dtype, group_size, groups, codes, scales, biases, sb_dtype, st);
    case 6: return launch_quant<6>(w, w_dtype, group_size, groups, codes, scales, biases, sb_dtype, st);
    default: return launch_quant<8>(w, w_dtype, group_size, groups, codes, scales, biases, sb_dtype, st);
  }
}

}  // extern "C"

// OCP MX modes as MLX stores them (mode "mxfp4" / "mxfp8", group size 32): dequantization and
// the decode GEMV.
//
//   W[n, k] = value(code[n, k]) * 2^(scale[n, k / 32] - 127)
//
// Codes are packed in uint32 words, little-endian bytes: mxfp4 holds two E2M1 codes per byte
// (element 2i in the low nibble, jang-tools/jang_tools/mimo_v2/mxfp4_codec.py:1-50), mxfp8
// one E4M3 (FN) byte per element; scales are one uint8 E8M0 exponent per 32 elements of a row.
// There are no biases. Reference: the mode switch of _fix_quantized_bits
// (jang-tools/jang_tools/loader.py:1877-1912) and mx.quantized_matmul / mx.dequantize with
// those modes.
//
// Values are decoded with integer operations into exact fp32 (a small float times a power of
// two is exact), so dequantization is bit-exact in fp32 and correctly rounded in bf16/f16.
//
// GEMV: a wave owns rows, a lane owns the row's 32-element blocks l, l + 64, ...; the lane's
// activations of those blocks stay in registers (as bf16/f16 pairs) while the wave walks its
// rows. Per block: the gfx950 MX conversions turn each code pair into a bf16/f16 pair of the
// activations' type (unscaled: E2M1 and E4M3 values are exact in both), v_dot2 accumulates in
// fp32, and the block scale multiplies the block's sum; a DPP wave sum ends a row. Activation
// rows are taken one launch each (decode batches).
#include <math.h>

#include "jq_common.h"
#include "jq_gemv.h"

namespace {

using namespace jq;

constexpr int kMxBlock = 32;

JQ_DEV float e2m1_f32(uint32_t c) {
  const uint32_t m = c & 7u, e = m >> 1;
  const uint32_t mag = e ? ((e + 126u) << 23) | ((m & 1u) << 22) : (m ? 0x3F000000u : 0u);
  return __uint_as_float(mag | ((c & 8u) << 28));
}

JQ_DEV float e4m3_f32(uint32_t b) {
  const uint32_t e = (b >> 3) & 15u, m = b & 7u;
  float v = e ? __uint_as_float(((e + 120u) << 23) | (m << 20)) : (float)m * 0x1p-9f;
  v = (e == 15u && m == 7u) ? __uint_as_float(0x7FC00000u) : v;
  return (b & 0x80u) ? -v : v;
}

JQ_DEV float e8m0_f32(uint32_t e) {
  return e == 255u ? __uint_as_float(0x7FC00000u) : ldexpf(1.0f, (int)e - 127);
}

// Element j (0 .. per-word count) of a code word.
template <int MODE>
JQ_DEV float mx_value(uint32_t w, int j) {
  if constexpr (MODE == 4) return e2m1_f32((w >> (4 * j)) & 15u);
  else return e4m3_f32((w >> (8 * j)) & 255u);
}

// One thread per code word (8 or 4 elements, all in one block).
template <int MODE, int OD>
__global__ void __launch_bounds__(256) mx_dequant_kernel(const uint32_t* __restrict__ codes,
                                                        const uint8_t* __restrict__ scales,
                                                        int64_t words, int64_t wpr, int64_t K,
                                                        void* __restrict__ out) {
  constexpr int PER = MODE == 4 ? 8 : 4;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < words;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / wpr, k0 = (i - r * wpr) * PER;
    const uint32_t w = codes[i];
    const float s = e8m0_f32(scales[r * (K / kMxBlock) + k0 / kMxBlock]);
#pragma unroll
    for (int j = 0; j < PER; ++j) store_t<OD>(out, r * K + k0 + j, mx_value<MODE>(w, j) * s);
  }
}

// Elements 2e, 2e + 1 of a block (code words w) as a pair of the activations' 16-bit type:
// mxfp4 byte e % 4 of word e / 4, mxfp8 bytes 2 (e % 2), + 1 of word e / 2; the lower
// element lands in the low half.
template <int MODE, int XD, int E>
JQ_DEV uint32_t mx_pair(const uint32_t* w) {
  if constexpr (MODE == 4) {
    if constexpr (XD == JQ_BF16)
      return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w[E >> 2], 1.0f, E & 3));
    else
      return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w[E >> 2], 1.0f, E & 3));
  } else {
    if constexpr (XD == JQ_BF16)
      return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w[E >> 1], 1.0f, (E & 1) != 0));
    else
      return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w[E >> 1], 1.0f, (E & 1) != 0));
  }
}

template <int MODE, int XD, int E = 0>
JQ_DEV float block_dot(const uint32_t* w, const uint32_t* xp, float part) {
  if constexpr (E == 16) {
    return part;
  } else {
    return block_dot<MODE, XD, E + 1>(w, xp, dot2<XD>(mx_pair<MODE, XD, E>(w), xp[E], part));
  }
}

// Rows per wave walk, blocks per lane XB (K <= 64 * 32 * XB), 4 waves per block.
// Gathered form (MX expert stacks): blockIdx.y is (pair, activation row) p * M + m; the pair
// reads x row lhs[p] * M + m (lhs NULL: p) and expert rhs[p]'s rows, and writes output row
// p * M + m. A pair whose expert id is >= E writes nothing.
struct MxGather {
  const uint32_t* lhs;
  const uint32_t* rhs;
  int64_t M, E, x_rows;
};

template <int MODE, int XD, int XB>
__global__ void __launch_bounds__(256) mx_gemv_kernel(const uint16_t* __restrict__ x,
                                                     const uint32_t* __restrict__ codes,
                                                     const uint8_t* __restrict__ scales,
                                                     int64_t N, int K, void* __restrict__ y,
                                                     int yd, int rows_per_wave, MxGather gt) {
  constexpr int WPB = MODE == 4 ? 4 : 8;  // code words of a 32-element block
  const int lane = threadIdx.x & 63;
  const int wave = (int)(blockIdx.x * 4 + (threadIdx.x >> 6));
  const int nb = K / kMxBlock;  // blocks per row
  if (gt.rhs) {
    const int64_t pm = blockIdx.y, p = pm / gt.M, m = pm - p * gt.M;
    const uint32_t e = gt.rhs[p];
    if (e >= (uint32_t)gt.E) return;  // whole block
    const int64_t xr = (gt.lhs ? (int64_t)gt.lhs[p] : p) * gt.M + m;
    if (xr >= gt.x_rows) return;
    x += xr * K;
    codes += (int64_t)e * N * (K / (MODE == 4 ? 8 : 4));
    scales += (int64_t)e * N * nb;
    y = (char*)y + pm * N * (yd == JQ_F32 ? 4 : 2);
  }
  // The lane's activations: XB blocks of 32 elements as 16 pairs each.
  uint32_t xa[XB][16];
#pragma unroll
  for (int q = 0; q < XB; ++q) {
    const int b = lane + 64 * q;
    const bool in = b < nb;
    const uint4* src = (const uint4*)(x + (int64_t)(in ? b : 0) * kMxBlock);
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const uint4 t = src[v];
      xa[q][4 * v] = in ? t.x : 0u;
      xa[q][4 * v + 1] = in ? t.y : 0u;
      xa[q][4 * v + 2] = in ? t.z : 0u;
      xa[q][4 * v + 3] = in ? t.w : 0u;
    }
  }
  const int64_t r0 = (int64_t)wave * rows_per_wave;
  for (int rr = 0; rr < rows_per_wave; ++rr) {
    const int64_t n = r0 + rr;
    if (n >= N) break;  // wave-uniform
    const uint32_t* crow = codes + n * (int64_t)(K / (MODE == 4 ? 8 : 4));
    const uint8_t* srow = scales + n * (int64_t)nb;
    float acc = 0.f;
#pragma unroll
    for (int q = 0; q < XB; ++q) {
      const int b = lane + 64 * q;
      if (b < nb) {
        uint32_t w[WPB];
        const uint4* cp = (const uint4*)(crow + (int64_t)b * WPB);
#pragma unroll
        for (int v = 0; v < WPB / 4; ++v) {
          const uint4 t = cp[v];
          w[4 * v] = t.x; w[4 * v + 1] = t.y; w[4 * v + 2] = t.z; w[4 * v + 3] = t.w;
        }
        const float s = e8m0_f32(srow[b]);
        acc = fmaf(block_dot<MODE, XD>(w, xa[q], 0.f), s, acc);
      }
    }
    const float tot = jqg::wave_total_lane63(acc);
    if (lane == 63) {
      if (yd == JQ_BF16) store_t<JQ_BF16>(y, n, tot);
      else if (yd == JQ_F16) store_t<JQ_F16>(y, n, tot);
      else store_t<JQ_F32>(y, n, tot);
    }
  }
}

inline unsigned grid_for(int64_t n) {
  const int64_t b = (n + 255) / 256;
  return (unsigned)(b < 8192 ? (b < 1 ? 1 : b) : 8192);
}

template <int MODE, int XD, int XB>
void gemv_launch(const uint16_t* x, const uint32_t* codes, const uint8_t* scales, int64_t N,
                 int K, void* y, int yd, const MxGather& gt, int64_t rows, hipStream_t st) {
  const int rpw = 2;
  const int64_t waves = (N + rpw - 1) / rpw;
  const dim3 grid((unsigned)((waves + 3) / 4), (unsigned)rows);
  mx_gemv_kernel<MODE, XD, XB><<<grid, 256, 0, st>>>(x, codes, scales, N, K, y, yd, rpw, gt);
}

template <int MODE, int XD>
int gemv_xb(const uint16_t* x, const uint32_t* codes, const uint8_t* scales, int64_t N, int K,
            void* y, int yd, hipStream_t st, const MxGather& gt = MxGather{nullptr, nullptr, 1, 0, 0},
            int64_t rows = 1) {
  const int nb = K / kMxBlock;
  if (nb <= 64) gemv_launch<MODE, XD, 1>(x, codes, scales, N, K, y, yd, gt, rows, st);
  else if (nb <= 128) gemv_launch<MODE, XD, 2>(x, codes, scales, N, K, y, yd, gt, rows, st);
  else if (nb <= 256) gemv_launch<MODE, XD, 4>(x, codes, scales, N, K, y, yd, gt, rows, st);
  else gemv_launch<MODE, XD, 8>(x, codes, scales, N, K, y, yd, gt, rows, st);
  return jqh::launch_status();
}

}  // namespace

extern "C" {

int jq_mx_dequantize(const uint32_t* codes, const uint8_t* scales, int mode, int64_t rows,
                     int64_t K, void* out, int out_dtype, jq_stream_t stream) {
  if (mode != 4 && mode != 8) return JQ_ERR_BITS;
  if (rows < 0 || K < 0 || K % kMxBlock || rows > ((int64_t)1 << 31) || K > ((int64_t)1 << 24))
    return K % kMxBlock ? JQ_ERR_GROUP_SIZE : JQ_ERR_SHAPE;
  if (!jqh::dtype_ok(out_dtype)) return JQ_ERR_DTYPE;
  if (rows == 0 || K == 0) return JQ_OK;
  if (!codes || !scales || !out) return JQ_ERR_NULL;
  const int64_t wpr = K / (mode == 4 ? 8 : 4), words = rows * wpr;
  hipStream_t st = (hipStream_t)stream;
#define JQ_MXD(M, OD) mx_dequant_kernel<M, OD><<<grid_for(words), 256, 0, st>>>(codes, scales, words, wpr, K, out)
  if (mode == 4) {
    if (out_dtype == JQ_BF16) JQ_MXD(4, JQ_BF16);
    else if (out_dtype == JQ_F16) JQ_MXD(4, JQ_F16);
    else JQ_MXD(4, JQ_F32);
  } else {
    if (out_dtype == JQ_BF16) JQ_MXD(8, JQ_BF16);
    else if (out_dtype == JQ_F16) JQ_MXD(8, JQ_F16);
    else JQ_MXD(8, JQ_F32);
  }
#undef JQ_MXD
  return jqh::launch_status();
}

int jq_mx_quantized_matmul(const void* x, int x_dtype, const uint32_t* codes,
                           const uint8_t* scales, int mode, int64_t M, int64_t N, int64_t K,
                           void* y, int y_dtype, jq_stream_t stream) {
  if (mode != 4 && mode != 8) return JQ_ERR_BITS;
  if (K % kMxBlock) return JQ_ERR_GROUP_SIZE;
  if (M < 0 || N < 0 || K < 0 || N >= ((int64_t)1 << 31) || K > 64 * kMxBlock * 8)
    return JQ_ERR_SHAPE;
  if (x_dtype != JQ_BF16 && x_dtype != JQ_F16) return JQ_ERR_DTYPE;
  if (!jqh::dtype_ok(y_dtype)) return JQ_ERR_DTYPE;
  if (M == 0 || N == 0) return JQ_OK;
  if (K == 0) return JQ_ERR_SHAPE;
  if (!x || !codes || !scales || !y) return JQ_ERR_NULL;
  hipStream_t st = (hipStream_t)stream;
  const int ys = jqh::dtype_size(y_dtype);
  for (int64_t m = 0; m < M; ++m) {
    const uint16_t* xm = (const uint16_t*)x + m * K;
    void* ym = (char*)y + m * N * ys;
    int s;
    if (mode == 4) s = x_dtype == JQ_BF16 ? gemv_xb<4, JQ_BF16>(xm, codes, scales, N, (int)K, ym, y_dtype, st)
                                          : gemv_xb<4, JQ_F16>(xm, codes, scales, N, (int)K, ym, y_dtype, st);
    else s = x_dtype == JQ_BF16 ? gemv_xb<8, JQ_BF16>(xm, codes, scales, N, (int)K, ym, y_dtype, st)
                                : gemv_xb<8, JQ_F16>(xm, codes, scales, N, (int)K, ym, y_dtype, st);
    if (s) return s;
  }
  return JQ_OK;
}

int jq_mx_gather_qmm(const void* x, int x_dtype, int64_t x_batch, int64_t M,
                     const uint32_t* codes, const uint8_t* scales, int mode, int64_t E,
                     int64_t N, int64_t K, const uint32_t* lhs, const uint32_t* rhs,
                     int64_t n_pairs, void* out, int y_dtype, jq_stream_t stream) {
  if (mode != 4 && mode != 8) return JQ_ERR_BITS;
  if (K % kMxBlock) return JQ_ERR_GROUP_SIZE;
  if (M <= 0 || N < 0 || K <= 0 || E <= 0 || x_batch < 0 || n_pairs < 0 ||
      N >= ((int64_t)1 << 31) || K > 64 * kMxBlock * 8 || n_pairs * M >= 65536)
    return JQ_ERR_SHAPE;
  if (!lhs && x_batch < n_pairs) return JQ_ERR_SHAPE;
  if (x_dtype != JQ_BF16 && x_dtype != JQ_F16) return JQ_ERR_DTYPE;
  if (!jqh::dtype_ok(y_dtype)) return JQ_ERR_DTYPE;
  if (n_pairs == 0 || N == 0) return JQ_OK;
  if (!x || !codes || !scales || !rhs || !out) return JQ_ERR_NULL;
  hipStream_t st = (hipStream_t)stream;
  const MxGather gt{lhs, rhs, M, E, x_batch * M};
  const uint16_t* xs = (const uint16_t*)x;
  const int64_t rows = n_pairs * M;
  if (mode == 4)
    return x_dtype == JQ_BF16 ? gemv_xb<4, JQ_BF16>(xs, codes, scales, N, (int)K, out, y_dtype, st, gt, rows)
                              : gemv_xb<4, JQ_F16>(xs, codes, scales, N, (int)K, out, y_dtype, st, gt, rows);
  return x_dtype == JQ_BF16 ? gemv_xb<8, JQ_BF16>(xs, codes, scales, N, (int)K, out, y_dtype, st, gt, rows)
                            : gemv_xb<8, JQ_F16>(xs, codes, scales, N, (int)K, out, y_dtype, st, gt, rows);
}

}  // extern "C"

// Shared device helpers for the jangq_amd gfx950 kernels.
//
// Code layout (reference: jang-tools/jang_tools/pack.py:12-149, FORMAT.md:57-90): codes of
// one matrix row form an LSB-first bitstream, code k occupying bits [k*bits, k*bits+bits)
// of the row, and the stream is stored as little-endian uint32 words. 32 consecutive codes
// therefore always occupy exactly `bits` whole words; this build calls such a run a "unit".
// Groups (32/64/128 codes) are whole units, so a unit never straddles a group, while single
// 3-, 5- and 6-bit codes do straddle words inside a unit.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/jangq_amd.h"

#define JQ_DEV __device__ __forceinline__

namespace jq {

// ----------------------------------------------------------------------------- dtypes

JQ_DEV float bf16_bits_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

// Round-to-nearest-even fp32 -> bf16 with a canonical quiet NaN (0x7FC0), the rounding of
// torch's c10::BFloat16 and numpy/ml_dtypes.
JQ_DEV uint16_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0x7FC0;
  u += 0x7FFFu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

JQ_DEV float f16_bits_to_f32(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }

// Round-to-nearest-even fp32 -> f16 (v_cvt_f16_f32).
JQ_DEV uint16_t f32_to_f16_bits(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }

// Load element i of a tensor of dtype `dt` as fp32.
JQ_DEV float load_as_f32(const void* p, int64_t i, int dt) {
  if (dt == JQ_BF16) return bf16_bits_to_f32(((const uint16_t*)p)[i]);
  if (dt == JQ_F16) return f16_bits_to_f32(((const uint16_t*)p)[i]);
  return ((const float*)p)[i];
}

template <int DT>
JQ_DEV float load_t(const void* p, int64_t i) {
  if constexpr (DT == JQ_BF16) return bf16_bits_to_f32(((const uint16_t*)p)[i]);
  else if constexpr (DT == JQ_F16) return f16_bits_to_f32(((const uint16_t*)p)[i]);
  else return ((const float*)p)[i];
}

template <int DT>
JQ_DEV void store_t(void* p, int64_t i, float v) {
  if constexpr (DT == JQ_BF16) ((uint16_t*)p)[i] = f32_to_bf16_bits(v);
  else if constexpr (DT == JQ_F16) ((uint16_t*)p)[i] = f32_to_f16_bits(v);
  else ((float*)p)[i] = v;
}

// ----------------------------------------------------------------------------- codes

// Bits [off, off+len) of the little-endian word array w (off, len compile-time after
// unrolling; len <= 32). Uses a 64-bit funnel shift (v_alignbit_b32) when the field
// crosses a word.
template <int OFF, int LEN>
JQ_DEV uint32_t field(const uint32_t* w) {
  constexpr int lo = OFF >> 5, sh = OFF & 31;
  constexpr uint32_t mask = LEN == 32 ? 0xFFFFFFFFu : ((1u << LEN) - 1u);
  if constexpr (sh + LEN <= 32) {
    return (w[lo] >> sh) & mask;
  } else {
    return __builtin_amdgcn_alignbit(w[lo + 1], w[lo], sh) & mask;
  }
}

// Code i (0..31) of a unit held in BITS words.
template <int BITS, int I>
JQ_DEV uint32_t unit_code(const uint32_t* w) {
  return field<I * BITS, BITS>(w);
}

// Runtime-index variant (used by the straightforward codec kernels).
template <int BITS>
JQ_DEV uint32_t unit_code_rt(const uint32_t* w, int i) {
  const int off = i * BITS;
  const int lo = off >> 5, sh = off & 31;
  uint64_t two = (uint64_t)w[lo];
  if (sh + BITS > 32) two |= (uint64_t)w[lo + 1] << 32;
  return (uint32_t)(two >> sh) & ((1u << BITS) - 1u);
}

// One 32-code unit (BITS words) in registers, loaded with the widest aligned vector loads.
template <int BITS>
struct UnitWords {
  uint32_t w[BITS];
};

template <int BITS>
JQ_DEV UnitWords<BITS> load_unit(const uint32_t* __restrict__ p) {
  UnitWords<BITS> u;
  if constexpr (BITS == 4) {
    const uint4 v = *(const uint4*)p;
    u.w[0] = v.x; u.w[1] = v.y; u.w[2] = v.z; u.w[3] = v.w;
  } else if constexpr (BITS == 2) {
    const uint2 v = *(const uint2*)p;
    u.w[0] = v.x; u.w[1] = v.y;
  } else if constexpr (BITS == 8) {
    const uint4 a = *(const uint4*)p, b = *(const uint4*)(p + 4);
    u.w[0] = a.x; u.w[1] = a.y; u.w[2] = a.z; u.w[3] = a.w;
    u.w[4] = b.x; u.w[5] = b.y; u.w[6] = b.z; u.w[7] = b.w;
  } else if constexpr (BITS == 6) {
    const uint2 a = *(const uint2*)p, b = *(const uint2*)(p + 2), c = *(const uint2*)(p + 4);
    u.w[0] = a.x; u.w[1] = a.y; u.w[2] = b.x; u.w[3] = b.y; u.w[4] = c.x; u.w[5] = c.y;
  } else {
#pragma unroll
    for (int i = 0; i < BITS; ++i) u.w[i] = p[i];
  }
  return u;
}

// ----------------------------------------------------------------------------- magic pairs
//
// The matmul kernels never convert codes with int->float instructions. For an 8-code chunk
// (codes c0..c7 of one group) they build four dwords, each holding two 16-bit floats
//   pair p (p = 0..3) = ( 2^B + c_p, 2^B + c_{p+4} )
// by OR-ing the code into the top B mantissa bits of the constant 2^B (B = bits), which
// makes the value exactly 2^B + c. With bf16 (7 mantissa bits) this covers B <= 6; f16
// (10 mantissa bits) covers every width including 8. A product of such a value with an
// activation of the same 16-bit format is exact in fp32, and
//   sum_k (2^B + q_k) x_k = sum_k q_k x_k + 2^B * sum_k x_k,
// so a group contributes  scale * D + (bias - 2^B * scale) * X  with D the magic dot
// product and X the plain sum of the group's activations. The activations are paired the
// same way: pair p of an 8-element chunk is (x_p, x_{p+4}).
//
// 8-bit codes with bf16 activations are split into two nibbles (code = 16*hi + lo), each a
// 4-bit magic operand: D_lo + 16*D_hi = sum q x + 272 * X.

// FMT: JQ_BF16 (exponent bias 127, 7 mantissa bits) or JQ_F16 (15, 10).
template <int FMT, int BITS>
struct Magic {
  static constexpr int mant = FMT == JQ_BF16 ? 7 : 10;
  static constexpr int ebias = FMT == JQ_BF16 ? 127 : 15;
  static constexpr uint32_t base16 = (uint32_t)(ebias + BITS) << mant;  // 2^BITS
  static constexpr uint32_t base = base16 | (base16 << 16);
  static constexpr int shift = mant - BITS;                              // code -> mantissa
  static constexpr float offset = (float)(1 << BITS);
  static_assert(shift >= 0, "code does not fit the mantissa");
};

// Four magic pairs of an 8-code chunk whose 8*BITS bits sit at the bottom of (v_hi:v).
// `base` is Magic<FMT, BITS>::base; callers that keep it in a register get one v_and_or_b32
// per pair (gfx9 VOP3 forms take no literal operand).
template <int FMT, int BITS>
JQ_DEV void chunk_to_pairs(uint32_t v, uint32_t v_hi, uint32_t out[4],
                           uint32_t base = Magic<FMT, BITS>::base) {
  using Mg = Magic<FMT, BITS>;
  constexpr uint32_t m = (1u << BITS) - 1u;
  constexpr int sh = Mg::shift;
  constexpr uint32_t fm = m << sh;
  if constexpr (BITS * 8 <= 32) {
    // lower four codes occupy 4*BITS <= 16 bits: move the upper four to bit 16.
    constexpr int half = 4 * BITS;
    constexpr uint32_t lowmask = (1u << half) - 1u;
    const uint32_t u = (v & lowmask) | ((v >> half) << 16);
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const int s = p * BITS - sh;
      const uint32_t t = s >= 0 ? (u >> s) : (u << (-s));
      out[p] = (t & (fm | (fm << 16))) | base;
    }
  } else {
    constexpr int half = 4 * BITS;  // 20, 24 or 32 bits
    const uint64_t all = (uint64_t)v | ((uint64_t)v_hi << 32);
    const uint32_t lo = (uint32_t)(all & ((1ull << half) - 1ull));
    const uint32_t hi = (uint32_t)((all >> half) & ((1ull << half) - 1ull));
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const int s = p * BITS - sh;
      const uint32_t a = s >= 0 ? (lo >> s) : (lo << (-s));
      const uint32_t b = s >= 0 ? (hi >> s) : (hi << (-s));
      out[p] = (a & fm) | ((b & fm) << 16) | base;
    }
  }
}

// Chunk c (0..3) of a unit (32 codes in BITS words): bits [8*BITS*c, 8*BITS*(c+1)).
template <int FMT, int BITS, int C>
JQ_DEV void unit_chunk_pairs(const uint32_t* w, uint32_t out[4],
                             uint32_t base = Magic<FMT, BITS>::base) {
  constexpr int off = 8 * BITS * C;
  constexpr int len = 8 * BITS;
  if constexpr (len <= 32) {
    chunk_to_pairs<FMT, BITS>(field<off, len>(w), 0u, out, base);
  } else {
    chunk_to_pairs<FMT, BITS>(field<off, 32>(w), field<off + 32, len - 32>(w), out, base);
  }
}

// 8-bit chunk c of a unit (words 2c, 2c+1) as bf16 nibble pairs: lo[p] carries the low
// nibbles of (c_p, c_{p+4}), hi[p] the high nibbles, both as 4-bit bf16 magic values.
JQ_DEV void chunk8_nibble_pairs(uint32_t w0, uint32_t w1, uint32_t lo[4], uint32_t hi[4]) {
  using Mg = Magic<JQ_BF16, 4>;
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    // bytes: [0] = byte p of w0, [2] = byte p of w1, [1] = [3] = 0
    const uint32_t sel = (uint32_t)p | (0x0Cu << 8) | ((uint32_t)(4 + p) << 16) | (0x0Cu << 24);
    const uint32_t t = __builtin_amdgcn_perm(w1, w0, sel);
    lo[p] = ((t << 3) & 0x00780078u) | Mg::base;
    hi[p] = ((t >> 1) & 0x00780078u) | Mg::base;
  }
}

// Pair a chunk of 8 16-bit activations held as 4 dwords (x0x1, x2x3, x4x5, x6x7) into
// (x0x4, x1x5, x2x6, x3x7) with byte permutes.
JQ_DEV void pair_activations(const uint32_t d[4], uint32_t out[4]) {
  out[0] = __builtin_amdgcn_perm(d[2], d[0], 0x05040100u);
  out[1] = __builtin_amdgcn_perm(d[2], d[0], 0x07060302u);
  out[2] = __builtin_amdgcn_perm(d[3], d[1], 0x05040100u);
  out[3] = __builtin_amdgcn_perm(d[3], d[1], 0x07060302u);
}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

// D = A(16x32) * B(32x16) + C with 16-bit float operands of format FMT (v_mfma_f32_16x16x32).
template <int FMT>
JQ_DEV f32x4 mfma16(u32x4 a, u32x4 b, f32x4 c) {
  if constexpr (FMT == JQ_BF16) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
}

typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2_t;
typedef __attribute__((__vector_size__(2 * sizeof(_Float16)))) _Float16 f16x2_t;

// acc + a.lo*b.lo + a.hi*b.hi for two packed 16-bit floats of format FMT.
template <int FMT>
JQ_DEV float dot2(uint32_t a, uint32_t b, float acc) {
  if constexpr (FMT == JQ_BF16) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                           __builtin_bit_cast(bf16x2_t, b), acc, false);
  } else {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, a), __builtin_bit_cast(f16x2_t, b),
                                  acc, false);
  }
}

// ----------------------------------------------------------------------------- checks

JQ_DEV bool valid_bits(int b) { return b == 2 || b == 3 || b == 4 || b == 5 || b == 6 || b == 8; }

}  // namespace jq

// Host-side validation helpers shared by the entry points.
namespace jqh {
inline bool bits_ok(int b) { return b == 2 || b == 3 || b == 4 || b == 5 || b == 6 || b == 8; }
inline bool gs_ok(int g) { return g == 32 || g == 64 || g == 128; }
inline bool dtype_ok(int d) { return d == JQ_F32 || d == JQ_BF16 || d == JQ_F16; }
inline int dtype_size(int d) { return d == JQ_F32 ? 4 : 2; }
inline int check_qshape(int bits, int gs, int64_t rows, int64_t K) {
  if (!bits_ok(bits)) return JQ_ERR_BITS;
  if (!gs_ok(gs)) return JQ_ERR_GROUP_SIZE;
  if (rows < 0 || K < 0) return JQ_ERR_SHAPE;
  if (K % gs) return JQ_ERR_GROUP_SIZE;
  if (rows > (int64_t)1 << 31 || K > (int64_t)1 << 24) return JQ_ERR_SHAPE;
  return JQ_OK;
}
inline int launch_status() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? JQ_OK : JQ_ERR_LAUNCH;
}
// Launch geometry on the host, each value queried from the runtime once per device (and
// kernel, block size, LDS bytes) and then served from a cache: the queries cost microseconds
// of host time, which is most of an eager decode launch. Defined in jq_api.hip.
int cus();  // compute units of the current device
int blocks_per_cu(const void* kern, int threads, size_t lds);  // resident blocks per CU, >= 1
// Opt a kernel in to `lds` bytes of dynamic LDS on the current device (above the 64 KB
// default); false if the runtime refuses.
bool set_lds(const void* kern, size_t lds);
}  // namespace jqh

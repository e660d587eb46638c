// Building blocks of the vector-ALU decode GEMVs (dense: jq_gemv.hip, expert-gathered:
// jq_gemv_gather.hip): activation state per 32-code unit, the unit dot product on the exact
// 16-bit code values, wave reduction, buffer views and the per-lane chunk loads.
#pragma once

#include "jq_dec.h"

namespace jqg {

using namespace jq;
using jqd::Bases;
using jqd::Dc;

template <int BITS>
constexpr int units_per_chunk() {
  return BITS == 2 ? 2 : 1;
}

// Activation state of one unit for one token: the 16 activation dwords paired as the unit's
// code dwords, X = sum x, O = -sum offset_k x_k.
struct XState {
  uint32_t pr[16];
  float X, O;
  float scl;  // F16X: 2^-k, the unit's rescaling undone (1 otherwise)
};

template <class D, int F, int P>
JQ_DEV uint32_t xpair_of(const jqd::XRaw& r) {
  return jqd::xpair<jqd::code_lo<D>(F, P), jqd::code_hi<D>(F, P)>(r);
}

template <class D>
JQ_DEV void make_xstate(const jqd::XRaw& r, XState& xs) {
  if constexpr (D::F16X) {
    // The unit's largest bf16 exponent field e; x' = x 2^k with k = 141 - e puts the largest
    // |x'| in [2^14, 2^15). bf16 values have 8 significant bits, so x' is exact in f16 unless
    // it falls below f16's normal range (|x| < 2^-28 of the largest; those truncate).
    typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
    u16x2 m = {0, 0};
#pragma unroll
    for (int i = 0; i < 16; ++i)
      m = __builtin_elementwise_max(m, __builtin_bit_cast(u16x2, r.d[i] & 0x7F807F80u));
    const int e = (int)((m[0] > m[1] ? m[0] : m[1]) >> 7);
    const int k = 141 - e;
    float X = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const float lo = __builtin_ldexpf(__uint_as_float(r.d[i] << 16), k);
      const float hi = __builtin_ldexpf(__uint_as_float(r.d[i] & 0xFFFF0000u), k);
      xs.pr[i] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(lo, hi));
      X = dot2<JQ_F16>(xs.pr[i], 0x3C003C00u, X);
    }
    xs.scl = __builtin_ldexpf(1.0f, -k);
    xs.X = X * xs.scl;      // sum of x
    if constexpr (D::BITS == 8) {
      xs.O = -1024.f * X;   // minus the codes' offset times the sum of x', in x' units
    } else {
      // 6-bit pairs (a, a + 2), a = 4m or 4m + 1: (x'_4m, x'_4m+2) are the low halves of
      // dwords 2m, 2m+1, (x'_4m+1, x'_4m+3) the high halves; offsets 64 (a) and 1024 (a + 2)
      uint32_t q[16];
#pragma unroll
      for (int m = 0; m < 8; ++m) {
        q[2 * m] = __builtin_amdgcn_perm(xs.pr[2 * m + 1], xs.pr[2 * m], 0x05040100u);
        q[2 * m + 1] = __builtin_amdgcn_perm(xs.pr[2 * m + 1], xs.pr[2 * m], 0x07060302u);
      }
      float O = 0.f;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        xs.pr[i] = q[i];
        O = dot2<JQ_F16>(q[i], 0xE400D400u, O);  // f16 (-64, -1024)
      }
      xs.O = O;
    }
  } else {
    xs.scl = 1.f;
#define JQ_XP(F, P) xs.pr[4 * F + P] = xpair_of<D, F, P>(r);
    JQ_XP(0, 0) JQ_XP(0, 1) JQ_XP(0, 2) JQ_XP(0, 3)
    JQ_XP(1, 0) JQ_XP(1, 1) JQ_XP(1, 2) JQ_XP(1, 3)
    JQ_XP(2, 0) JQ_XP(2, 1) JQ_XP(2, 2) JQ_XP(2, 3)
    JQ_XP(3, 0) JQ_XP(3, 1) JQ_XP(3, 2) JQ_XP(3, 3)
#undef JQ_XP
    float X = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) X = dot2<D::XDT>(r.d[i], D::ONE2, X);
    xs.X = X;
    if constexpr (D::SCHED) {
      float O = 0.f;
#pragma unroll
      for (int i = 0; i < 16; ++i) O = dot2<D::XDT>(jqd::bo_dword<D>(i >> 2, i & 3), xs.pr[i], O);
      xs.O = O;
    } else if constexpr (D::NIB) {
      xs.O = -272.f * X;
    } else {
      xs.O = -(float)(1 << D::BITS) * X;
    }
  }
}

// Dot product of one unit's exact code values with its paired activations.
template <class D>
JQ_DEV float unit_dot(const uint32_t* w, const Bases<D>& bs, const XState& xs) {
  if constexpr (D::F16X) {
    float d = 0.f;
    if constexpr (D::BITS == 8) {
      // Pair i = codes (2i, 2i+1), bytes 2(i%2), 2(i%2)+1 of word i/2, each under the f16
      // exponent byte 0x64: 1024 + q; the x' pairs are in the same (natural) order.
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const uint32_t b0 = 2 * (i & 1), sel = b0 | (4u << 8) | ((b0 + 1) << 16) | (4u << 24);
        d = dot2<JQ_F16>(__builtin_amdgcn_perm(bs.v[0], w[i >> 1], sel), xs.pr[i], d);
      }
    } else {
      // Pair i = codes (a, a + 2), a = 4(i/2) + i%2: the 32-bit window of the unit starting
      // at bit 6a - 4 holds code a at bits 4..9 and code a + 2 at bits 16..21.
#define JQ_P6(I)                                                                         \
  {                                                                                      \
    constexpr int a = 4 * (I >> 1) + (I & 1), s = 6 * a - 4;                             \
    uint32_t win;                                                                        \
    if constexpr (s < 0) win = w[0] << (-s);                                             \
    else win = jqd::window<6, (s < 0 ? 0 : s)>(w);                                       \
    d = dot2<JQ_F16>((win & 0x003F03F0u) | bs.v[0], xs.pr[I], d);                        \
  }
      JQ_P6(0) JQ_P6(1) JQ_P6(2) JQ_P6(3) JQ_P6(4) JQ_P6(5) JQ_P6(6) JQ_P6(7)
      JQ_P6(8) JQ_P6(9) JQ_P6(10) JQ_P6(11) JQ_P6(12) JQ_P6(13) JQ_P6(14) JQ_P6(15)
#undef JQ_P6
    }
    return d;
  } else {
    float d0 = 0.f, d1 = 0.f;
#define JQ_UF(F)                                                          \
    {                                                                       \
      u32x4 b, bh;                                                          \
      jqd::b_frag<D, F>(w, bs, b, bh);                                      \
      d0 = dot2<D::XDT>(b[0], xs.pr[4 * F + 0], d0);                        \
      d0 = dot2<D::XDT>(b[1], xs.pr[4 * F + 1], d0);                        \
      d0 = dot2<D::XDT>(b[2], xs.pr[4 * F + 2], d0);                        \
      d0 = dot2<D::XDT>(b[3], xs.pr[4 * F + 3], d0);                        \
      if constexpr (D::NIB) {                                               \
        d1 = dot2<D::XDT>(bh[0], xs.pr[4 * F + 0], d1);                     \
        d1 = dot2<D::XDT>(bh[1], xs.pr[4 * F + 1], d1);                     \
        d1 = dot2<D::XDT>(bh[2], xs.pr[4 * F + 2], d1);                     \
        d1 = dot2<D::XDT>(bh[3], xs.pr[4 * F + 3], d1);                     \
      }                                                                     \
    }
    JQ_UF(0) JQ_UF(1) JQ_UF(2) JQ_UF(3)
#undef JQ_UF
    if constexpr (D::NIB) return fmaf(16.f, d1, d0);
    return d0;
  }
}

// Sum over the 64 lanes with DPP row operations; the total lands in lane 63.
JQ_DEV float wave_total_lane63(float v) {
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));  // quad_perm 1,0,3,2
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));  // quad_perm 2,3,0,1
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x124, 0xF, 0xF, false)); // row_ror 4
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x128, 0xF, 0xF, false)); // row_ror 8
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x142, 0xA, 0xF, false)); // row_bcast 15
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x143, 0xC, 0xF, false)); // row_bcast 31
  return v;
}

template <int SB>
JQ_DEV float sb_to_f32(uint32_t h) {
  if constexpr (SB == JQ_BF16) return __uint_as_float(h << 16);
  else return f16_bits_to_f32((uint16_t)h);
}

typedef __amdgpu_buffer_rsrc_t Rsrc;
typedef uint32_t u32x3 __attribute__((ext_vector_type(3)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Raw buffer view of `bytes` bytes at p: loads past the end read zero and touch no memory.
JQ_DEV Rsrc make_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}

// The BITS*UPL code words of a lane chunk at byte voff of a row block. All offsets go into
// the vector offset: the buffer range check covers it, not the scalar offset.
template <int NW>
JQ_DEV void load_chunk(Rsrc r, uint32_t voff, uint32_t* w) {
  constexpr int soff = 0;
  if constexpr (NW == 4) {
    const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
    w[0] = v[0]; w[1] = v[1]; w[2] = v[2]; w[3] = v[3];
  } else if constexpr (NW == 8) {
    const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
    const u32x4 u = __builtin_amdgcn_raw_buffer_load_b128(r, voff + 16, soff, 0);
    w[0] = v[0]; w[1] = v[1]; w[2] = v[2]; w[3] = v[3];
    w[4] = u[0]; w[5] = u[1]; w[6] = u[2]; w[7] = u[3];
  } else if constexpr (NW == 2) {
    const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, 0);
    w[0] = v[0]; w[1] = v[1];
  } else if constexpr (NW == 3) {
    const u32x3 v = __builtin_amdgcn_raw_buffer_load_b96(r, voff, soff, 0);
    w[0] = v[0]; w[1] = v[1]; w[2] = v[2];
  } else if constexpr (NW == 6) {
#pragma unroll
    for (int i = 0; i < 3; ++i) {
      const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(r, voff + 8 * i, soff, 0);
      w[2 * i] = v[0]; w[2 * i + 1] = v[1];
    }
  } else {
#pragma unroll
    for (int i = 0; i < NW; ++i) w[i] = __builtin_amdgcn_raw_buffer_load_b32(r, voff + 4 * i, soff, 0);
  }
}

// Block = KW waves (blockDim.x = 64 * KW, KW <= kMaxWaves).
constexpr int kMaxWaves = 8;

// Waves per block for a K: the fewest (a power of two) for which each lane holds one chunk.
// (upl: units per lane chunk.)
inline int gemv_waves_upl(int64_t K, int upl, int* shift) {
  const int64_t C = K / (32 * upl);
  int kw = 1, ks = 0;
  while (64 * kw < C) kw *= 2, ++ks;
  if (shift) *shift = ks;
  return kw;
}
inline int gemv_waves(int64_t K, int bits, int* shift) {
  return gemv_waves_upl(K, bits == 2 ? 2 : 1, shift);
}

// One row of a lane's ring slot: the chunk's code words, and the scale and bias of each of
// its units (units of one group load the same element).
template <int NW, int UPL>
struct RowSlot {
  uint32_t w[NW];
  uint32_t s[UPL], b[UPL];
};

// Scale and bias words of a lane chunk's UPL units, at byte offsets vsb[t] + off of the
// sidecar rows. The two units of a 2-bit chunk lie in one group when groups hold at least 64
// codes (D::GS >= 64; 32-code groups are instantiated with GS = 32): one load each then
// serves both units.
template <class D, int NW, int UPL>
JQ_DEV void load_sb(Rsrc rs, Rsrc rb, const uint32_t* vsb, uint32_t off, RowSlot<NW, UPL>& slot) {
  if constexpr (UPL == 2 && D::GS >= 64) {
    const uint32_t sv = __builtin_amdgcn_raw_buffer_load_b16(rs, vsb[0] + off, 0, 0);
    const uint32_t bv = __builtin_amdgcn_raw_buffer_load_b16(rb, vsb[0] + off, 0, 0);
    slot.s[0] = slot.s[1] = sv;
    slot.b[0] = slot.b[1] = bv;
  } else {
#pragma unroll
    for (int t = 0; t < UPL; ++t) {
      slot.s[t] = __builtin_amdgcn_raw_buffer_load_b16(rs, vsb[t] + off, 0, 0);
      slot.b[t] = __builtin_amdgcn_raw_buffer_load_b16(rb, vsb[t] + off, 0, 0);
    }
  }
}

}  // namespace jqg

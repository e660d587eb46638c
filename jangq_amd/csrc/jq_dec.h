// Decode-shaped matrix-core kernels (few activation rows): shared device code.
//
// Work unit: RT tiles of 16 W rows over a K range, for up to TPB activation rows. Every lane
// streams its own row's codes straight from HBM into MFMA B fragments: lane (r = l%16,
// g = l/16) loads 32-code unit g of each 128-code step of row r (BITS whole words), so one
// wave load instruction reads 16 rows x 4*BITS*4 contiguous bytes and nothing is staged in
// LDS.
//
// Codes become exact 16-bit floats without int->float conversion: a code c placed at mantissa
// offset p under the exponent E makes the value 2^E' + c with the code's own offset term. For
// bf16 activations and 2/3/4-bit codes each code gets its own offset p (a "schedule"), so one
// funnel-shifted 32-bit window of the unit feeds up to three dwords with a single
// and-or each (20 / 25 / 28 instructions per 32 codes, found by exhaustive search); the
// per-slot offsets 2^(7-p) form a constant B operand. Other widths (and f16 activations) use
// one offset 2^B for every code (jq_common.h "magic pairs").
//
// A 128-code step spans GSTEP = 128/gs groups; lane group g holds codes of group
// g / (4/GSTEP). The group index is folded into the MFMA's M dimension: A row m' = GSTEP*t + j
// carries token t's activations only in the lane groups of group j (zeros elsewhere). Per
// step, with A_f the four A fragments:
//   O = sum_f A_f . BO_f   (-offsets)      X = sum_f A_f . 1   (activation sums)
//   D = O + sum_f A_f . B_f                 (= sum q*x exactly, per (token, group) row)
//   acc += s_g * D + b_g * X
// A lane's four output rows m' = 4*(l/16) + i belong to group i % GSTEP, so the scales are
// indexed at compile time per accumulator slot. Tokens per MFMA block: TPB = 16 / GSTEP.
#pragma once

#include "jq_common.h"

namespace jqd {

using namespace jq;

// ----------------------------------------------------------------------------- schedules

// Pair i (0..15) of a unit: dword i = (code a[i] as lo half, code b[i] as hi half), built
// from the window starting at bit s[i] with the codes at mantissa offsets pa[i] / pb[i].
// MFMA field f uses dwords 4f..4f+3.
struct Sched {
  int a[16], b[16], s[16], pa[16], pb[16];
};

// 2-bit: 4 shifted windows + 16 and-or.
constexpr Sched kSched2 = {
    {0, 1, 2, 3, 4, 5, 6, 7, 16, 17, 18, 19, 20, 21, 22, 23},
    {8, 9, 10, 11, 12, 13, 14, 15, 24, 25, 26, 27, 28, 29, 30, 31},
    {0, 0, 0, 3, 3, 9, 9, 9, 32, 32, 32, 35, 35, 41, 41, 41},
    {0, 2, 4, 3, 5, 1, 3, 5, 0, 2, 4, 3, 5, 1, 3, 5},
    {0, 2, 4, 3, 5, 1, 3, 5, 0, 2, 4, 3, 5, 1, 3, 5}};
// 3-bit: 9 shifted windows + 16 and-or.
constexpr Sched kSched3 = {
    {0, 1, 2, 3, 4, 5, 12, 13, 14, 15, 16, 22, 23, 24, 25, 26},
    {6, 7, 8, 9, 10, 11, 17, 18, 19, 20, 21, 27, 28, 29, 30, 31},
    {0, 1, 4, 7, 10, 13, 32, 38, 38, 44, 44, 64, 68, 68, 74, 74},
    {0, 2, 2, 2, 2, 2, 4, 1, 4, 1, 4, 2, 1, 4, 1, 4},
    {2, 4, 4, 4, 4, 4, 3, 0, 3, 0, 3, 1, 0, 3, 0, 3}};
// 4-bit: pairs (c, c+4) at offset 0, 12 shifted windows + 16 and-or.
constexpr Sched kSched4 = {
    {0, 1, 2, 3, 8, 9, 10, 11, 16, 17, 18, 19, 24, 25, 26, 27},
    {4, 5, 6, 7, 12, 13, 14, 15, 20, 21, 22, 23, 28, 29, 30, 31},
    {0, 4, 8, 12, 32, 36, 40, 44, 64, 68, 72, 76, 96, 100, 104, 108},
    {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0},
    {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0}};

template <int BITS>
constexpr const Sched& sched() {
  if constexpr (BITS == 2) return kSched2;
  else if constexpr (BITS == 3) return kSched3;
  else return kSched4;
}

// F16X_ (the vector-ALU row GEMV only, 6- and 8-bit codes, bf16 activations): the
// activations are rescaled per 32-code unit by a power of two into f16 (exact for bf16 values
// within 2^28 of the unit's largest), so that a code pair becomes one f16 pair with one
// instruction: a byte permute under the exponent of 1024 (8-bit: 1024 + q), or an and-or of a
// funnel-shifted window (6-bit, codes a and a + 2: 64 + q_a and 1024 + q_{a+2}) (see jq_gemv.h
// make_xstate / unit_dot).
template <int BITS_, int GS_, int XDT_, bool F16X_ = false>
struct Dc {
  static constexpr int BITS = BITS_, GS = GS_, XDT = XDT_;
  static constexpr int GSTEP = 128 / GS;   // groups per 128-code step
  static constexpr int TPB = 16 / GSTEP;   // activation rows per MFMA block
  static constexpr int LPG = 4 / GSTEP;    // lane groups per group
  static constexpr bool F16X = F16X_;
  static_assert(!F16X || ((BITS == 6 || BITS == 8) && XDT == JQ_BF16),
                "f16-rescaled units: 6- or 8-bit codes, bf16 x");
  static constexpr bool SCHED = XDT == JQ_BF16 && BITS >= 2 && BITS <= 4;  // per-code offsets
  static constexpr bool NIB = BITS == 8 && XDT == JQ_BF16 && !F16X;       // two nibbles
  static constexpr bool TWO = !SCHED && BITS == 2;  // f16 2-bit: pairs 8 codes apart
  static constexpr uint32_t ONE2 = XDT == JQ_BF16 ? 0x3F803F80u : 0x3C003C00u;
};

// Code indices (within the lane's 32-code unit) of dword p of field f: lo / hi halves.
template <class D>
constexpr int code_lo(int f, int p) {
  if constexpr (D::SCHED) return sched<D::BITS>().a[4 * f + p];
  else if constexpr (D::TWO) return 16 * (f >> 1) + 4 * (f & 1) + p;
  else return 8 * f + p;
}
template <class D>
constexpr int code_hi(int f, int p) {
  if constexpr (D::SCHED) return sched<D::BITS>().b[4 * f + p];
  else if constexpr (D::TWO) return 16 * (f >> 1) + 4 * (f & 1) + p + 8;
  else return 8 * f + p + 4;
}

// 16-bit value -2^e of format FMT.
template <int FMT>
constexpr uint32_t neg_pow2(int e) {
  return FMT == JQ_BF16 ? (0x8000u | ((uint32_t)(127 + e) << 7))
                        : (0x8000u | ((uint32_t)(15 + e) << 10));
}

// Constant B fragment of field f holding minus each slot's offset.
template <class D>
constexpr uint32_t bo_dword(int f, int p) {
  if constexpr (D::SCHED) {
    const Sched& S = sched<D::BITS>();
    return neg_pow2<JQ_BF16>(7 - S.pa[4 * f + p]) | (neg_pow2<JQ_BF16>(7 - S.pb[4 * f + p]) << 16);
  } else if constexpr (D::NIB) {
    return 0xC388C388u;  // bf16 -272 (= -(256 + 16)), exact
  } else {
    return neg_pow2<D::XDT>(D::BITS) | (neg_pow2<D::XDT>(D::BITS) << 16);
  }
}

// Magic bases of a scheduled unit, pinned in VGPRs (gfx9 VOP3 instructions take at most one
// scalar operand, so the and-or's mask is the scalar and the base must be a vector register).
template <class D>
struct Bases {
  uint32_t v[16];
};

// First pair index with the same (pa, pb) as pair i: equal bases share one register.
template <int BITS>
constexpr int base_rep(int i) {
  const Sched& S = sched<BITS>();
  for (int j = 0; j < i; ++j)
    if (S.pa[j] == S.pa[i] && S.pb[j] == S.pb[i]) return j;
  return i;
}

template <class D>
JQ_DEV Bases<D> make_bases() {
  Bases<D> r;
  if constexpr (D::SCHED) {
    const Sched& S = sched<D::BITS>();
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      if (base_rep<D::BITS>(i) == i) {
        r.v[i] = ((uint32_t)(134 - S.pa[i]) << 7) | ((uint32_t)(134 - S.pb[i]) << 23);
        asm volatile("" : "+v"(r.v[i]));
      } else {
        r.v[i] = r.v[base_rep<D::BITS>(i)];
      }
    }
  } else if constexpr (D::F16X) {
    // 8-bit: the exponent byte of f16 1024 beside each code byte of a pair; 6-bit: the f16
    // exponents of 64 (lo half, code at mantissa bit 4) and 1024 (hi half, bit 0)
    r.v[0] = D::BITS == 8 ? 0x64646464u : ((21u << 10) | (25u << 26));
    asm volatile("" : "+v"(r.v[0]));
  } else if constexpr (!D::NIB) {
    // The single magic base of the unscheduled forms, also pinned in a register.
    r.v[0] = Magic<D::XDT, D::BITS>::base;
    asm volatile("" : "+v"(r.v[0]));
  }
  return r;
}

// Bits [s, s+32) of the unit (zeros past its end).
template <int BITS, int S>
JQ_DEV uint32_t window(const uint32_t* w) {
  constexpr int lo = S >> 5, sh = S & 31;
  if constexpr (sh == 0) return w[lo];
  else if constexpr (lo + 1 < BITS) return __builtin_amdgcn_alignbit(w[lo + 1], w[lo], sh);
  else return w[lo] >> sh;
}

template <class D, int I>
JQ_DEV uint32_t sched_dword(const uint32_t* w, const Bases<D>& bs) {
  constexpr const Sched& S = sched<D::BITS>();
  constexpr uint32_t m = (1u << D::BITS) - 1u;
  constexpr uint32_t mask = (m << S.pa[I]) | (m << (16 + S.pb[I]));
  return (window<D::BITS, S.s[I]>(w) & mask) | bs.v[I];
}

// B fragment(s) of field F of a unit.
template <class D, int F>
JQ_DEV void b_frag(const uint32_t* w, const Bases<D>& bs, u32x4& b, u32x4& bh) {
  if constexpr (D::SCHED) {
    b = u32x4{sched_dword<D, 4 * F>(w, bs), sched_dword<D, 4 * F + 1>(w, bs),
              sched_dword<D, 4 * F + 2>(w, bs), sched_dword<D, 4 * F + 3>(w, bs)};
    bh = b;
  } else if constexpr (D::NIB) {
    uint32_t lo[4], hi[4];
    chunk8_nibble_pairs(w[2 * F], w[2 * F + 1], lo, hi);
    b = u32x4{lo[0], lo[1], lo[2], lo[3]};
    bh = u32x4{hi[0], hi[1], hi[2], hi[3]};
  } else if constexpr (D::TWO) {
    using Mg = Magic<D::XDT, 2>;
    constexpr int sh = Mg::shift;
    constexpr uint32_t pm = (3u << sh) | (3u << (sh + 16));
    const uint32_t word = w[F >> 1];
    uint32_t o[4];
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const int j = 4 * (F & 1) + p;
      const int s = 2 * j - sh;
      const uint32_t t = s >= 0 ? (word >> s) : (word << (-s));
      o[p] = (t & pm) | bs.v[0];
    }
    b = u32x4{o[0], o[1], o[2], o[3]};
    bh = b;
  } else {
    uint32_t o[4];
    unit_chunk_pairs<D::XDT, D::BITS, F>(w, o, bs.v[0]);
    b = u32x4{o[0], o[1], o[2], o[3]};
    bh = b;
  }
}

// ----------------------------------------------------------------------------- activations

// Raw activations of one step for this lane's A row: the 32 values of lane group lg,
// x[32*lg .. 32*lg+31] of the step, as 16 dwords (x_{2i}, x_{2i+1}).
struct XRaw {
  uint32_t d[16];
};

// 64 zero bytes: lanes that feed no activation read these instead of branching (a branch
// around a load makes the compiler wait for every outstanding load at the join).
static __device__ const uint4 kZeroRow[4] = {};

typedef const __attribute__((address_space(1))) u32x4 global_u32x4;

JQ_DEV void load_xraw(const uint16_t* p, XRaw& r) {
  // Global (not flat) loads: a flat load also counts against the LDS/scalar counter and
  // would force a full wait on every step.
  global_u32x4* q = (global_u32x4*)p;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const u32x4 v = q[i];
    r.d[4 * i] = v.x; r.d[4 * i + 1] = v.y; r.d[4 * i + 2] = v.z; r.d[4 * i + 3] = v.w;
  }
}

// A dword (x_a, x_b) from the raw dwords: one byte permute.
template <int A, int B>
JQ_DEV uint32_t xpair(const XRaw& r) {
  constexpr uint32_t lo = (A & 1) ? 0x0302u : 0x0100u;
  constexpr uint32_t hi = (B & 1) ? 0x0706u : 0x0504u;
  return __builtin_amdgcn_perm(r.d[B >> 1], r.d[A >> 1], lo | (hi << 16));
}

template <class D, int F>
JQ_DEV u32x4 a_frag(const XRaw& r) {
  return u32x4{xpair<code_lo<D>(F, 0), code_hi<D>(F, 0)>(r),
               xpair<code_lo<D>(F, 1), code_hi<D>(F, 1)>(r),
               xpair<code_lo<D>(F, 2), code_hi<D>(F, 2)>(r),
               xpair<code_lo<D>(F, 3), code_hi<D>(F, 3)>(r)};
}

// ----------------------------------------------------------------------------- scales

// Raw 16-bit scale / bias words of the GSTEP groups of one step.
template <class D>
struct SBRaw {
  uint32_t s[(D::GSTEP + 1) / 2], b[(D::GSTEP + 1) / 2];
};

template <class D>
JQ_DEV void load_sbraw(const uint16_t* srow, const uint16_t* brow, int g0, SBRaw<D>& r) {
  if constexpr (D::GSTEP == 1) {
    r.s[0] = srow[g0];
    r.b[0] = brow[g0];
  } else if constexpr (D::GSTEP == 2) {
    r.s[0] = *(const uint32_t*)(srow + g0);
    r.b[0] = *(const uint32_t*)(brow + g0);
  } else {
    const uint2 a = *(const uint2*)(srow + g0), c = *(const uint2*)(brow + g0);
    r.s[0] = a.x; r.s[1] = a.y; r.b[0] = c.x; r.b[1] = c.y;
  }
}

template <int SB>
JQ_DEV float half_to_f32(uint32_t w, int hi) {
  if constexpr (SB == JQ_BF16) {
    return __uint_as_float(hi ? (w & 0xFFFF0000u) : (w << 16));
  } else {
    return f16_bits_to_f32((uint16_t)(hi ? (w >> 16) : w));
  }
}

// ----------------------------------------------------------------------------- main loop

// What one step reads from HBM for RT row tiles x NB matrices: codes and their scales.
template <class D, int NB, int RT>
struct CodeStage {
  UnitWords<D::BITS> c[NB][RT];
  SBRaw<D> sb[NB][RT];
};

struct TileRows {
  const uint32_t* c;  // this lane's W row, codes
  const uint16_t* s;  // scales row
  const uint16_t* b;  // biases row
};

template <class D, int NB, int RT>
JQ_DEV void load_codes(const TileRows (&rows)[NB][RT], int s, int lg, CodeStage<D, NB, RT>& st) {
#pragma unroll
  for (int q = 0; q < NB; ++q)
#pragma unroll
    for (int r = 0; r < RT; ++r) {
      st.c[q][r] = load_unit<D::BITS>(rows[q][r].c + (s * 4 + lg) * D::BITS);
      load_sbraw<D>(rows[q][r].s, rows[q][r].b, s * D::GSTEP, st.sb[q][r]);
    }
}

template <class D, int SB, int NB, int RT>
JQ_DEV void compute_stage(const CodeStage<D, NB, RT>& st, const XRaw& xr, const Bases<D>& bs,
                          f32x4 (&acc)[NB][RT]) {
  const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
  const u32x4 ones = {D::ONE2, D::ONE2, D::ONE2, D::ONE2};
  const u32x4 A0 = a_frag<D, 0>(xr), A1 = a_frag<D, 1>(xr);
  const u32x4 A2 = a_frag<D, 2>(xr), A3 = a_frag<D, 3>(xr);
  f32x4 X = mfma16<D::XDT>(A0, ones, zero);
  X = mfma16<D::XDT>(A1, ones, X);
  X = mfma16<D::XDT>(A2, ones, X);
  X = mfma16<D::XDT>(A3, ones, X);
  constexpr u32x4 BO0 = {bo_dword<D>(0, 0), bo_dword<D>(0, 1), bo_dword<D>(0, 2), bo_dword<D>(0, 3)};
  constexpr u32x4 BO1 = {bo_dword<D>(1, 0), bo_dword<D>(1, 1), bo_dword<D>(1, 2), bo_dword<D>(1, 3)};
  constexpr u32x4 BO2 = {bo_dword<D>(2, 0), bo_dword<D>(2, 1), bo_dword<D>(2, 2), bo_dword<D>(2, 3)};
  constexpr u32x4 BO3 = {bo_dword<D>(3, 0), bo_dword<D>(3, 1), bo_dword<D>(3, 2), bo_dword<D>(3, 3)};
  f32x4 O = mfma16<D::XDT>(A0, BO0, zero);
  O = mfma16<D::XDT>(A1, BO1, O);
  O = mfma16<D::XDT>(A2, BO2, O);
  O = mfma16<D::XDT>(A3, BO3, O);
#pragma unroll
  for (int q = 0; q < NB; ++q)
#pragma unroll
    for (int r = 0; r < RT; ++r) {
      const uint32_t* w = st.c[q][r].w;
      u32x4 B, BH;
      f32x4 Dd, Dh = zero;
      b_frag<D, 0>(w, bs, B, BH);
      Dd = mfma16<D::XDT>(A0, B, O);
      if constexpr (D::NIB) Dh = mfma16<D::XDT>(A0, BH, zero);
      b_frag<D, 1>(w, bs, B, BH);
      Dd = mfma16<D::XDT>(A1, B, Dd);
      if constexpr (D::NIB) Dh = mfma16<D::XDT>(A1, BH, Dh);
      b_frag<D, 2>(w, bs, B, BH);
      Dd = mfma16<D::XDT>(A2, B, Dd);
      if constexpr (D::NIB) Dh = mfma16<D::XDT>(A2, BH, Dh);
      b_frag<D, 3>(w, bs, B, BH);
      Dd = mfma16<D::XDT>(A3, B, Dd);
      if constexpr (D::NIB) {
        Dh = mfma16<D::XDT>(A3, BH, Dh);
#pragma unroll
        for (int i = 0; i < 4; ++i) Dd[i] = fmaf(16.f, Dh[i], Dd[i]);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int j = i % D::GSTEP;
        const float sc = half_to_f32<SB>(st.sb[q][r].s[j >> 1], j & 1);
        const float bi = half_to_f32<SB>(st.sb[q][r].b[j >> 1], j & 1);
        acc[q][r][i] = fmaf(sc, Dd[i], fmaf(bi, X[i], acc[q][r][i]));
      }
    }
}

// Steps of codes kept in flight per wave: about 4 KB per row tile (even, >= 2). The grids
// of decode-shaped problems are too small to hide HBM latency with occupancy alone.
template <int BITS>
constexpr int code_depth() {
  return BITS <= 2 ? 8 : BITS <= 3 ? 6 : BITS <= 6 ? 4 : 2;
}

// Partial sums of RT 16-row tiles over steps [s0, s1) for NB weight matrices sharing the
// activations. rows: this lane's W rows. xr: this lane's activation row (token of A row
// l%16), act: whether the lane feeds A. Codes and scales are fetched DEPTH steps ahead in a
// register ring (static indices after unrolling), activations (L2-resident) one step ahead.
// Every load is unconditional (indices clamped to the last step, inactive lanes read
// zeros), so the loads of later steps stay in flight while a step is computed.
template <class D, int SB, int NB, int RT>
JQ_DEV void dec_tile(const uint16_t* xr, bool act, const TileRows (&rows)[NB][RT], int s0, int s1,
                     int lg, f32x4 (&acc)[NB][RT]) {
  constexpr int DEPTH = code_depth<D::BITS>();
  if (s0 >= s1) return;
  const int last = s1 - 1;
  const Bases<D> bs = make_bases<D>();
  const uint16_t* xl = xr + 32 * lg;
  const uint16_t* zero = (const uint16_t*)kZeroRow;
  CodeStage<D, NB, RT> ring[DEPTH];
#pragma unroll
  for (int d = 0; d < DEPTH; ++d) load_codes<D, NB, RT>(rows, min(s0 + d, last), lg, ring[d]);
  XRaw xa, xb;
  load_xraw(act ? xl + s0 * 128 : zero, xa);
  for (int s = s0;; s += DEPTH) {
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) {
      const int t = s + d;
      const uint16_t* xn = act ? xl + min(t + 1, last) * 128 : zero;
      if (d & 1) {
        load_xraw(xn, xa);
        compute_stage<D, SB, NB, RT>(ring[d], xb, bs, acc);
      } else {
        load_xraw(xn, xb);
        compute_stage<D, SB, NB, RT>(ring[d], xa, bs, acc);
      }
      load_codes<D, NB, RT>(rows, min(t + DEPTH, last), lg, ring[d]);
      if (t + 1 >= s1) return;
    }
  }
}

// Sum the partials of the KW waves of a block (each covered a K range). Returns the total
// in wave 0's registers. red: LDS scratch of (KW-1) * N4 * 256 floats (N4 = accumulators).
template <int KW, int N4>
JQ_DEV void block_reduce(f32x4* acc, float* red) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (wave > 0) {
#pragma unroll
    for (int q = 0; q < N4; ++q)
#pragma unroll
      for (int i = 0; i < 4; ++i) red[(((wave - 1) * N4 + q) * 4 + i) * 64 + lane] = acc[q][i];
  }
  __syncthreads();
  if (wave == 0) {
#pragma unroll
    for (int q = 0; q < N4; ++q)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float v = acc[q][i];
#pragma unroll
        for (int w = 1; w < KW; ++w) v += red[(((w - 1) * N4 + q) * 4 + i) * 64 + lane];
        acc[q][i] = v;
      }
  }
}

// Token outputs of a lane after the group rows are summed: lane (l%16, l/16) holds tokens
// t = TPL*(l/16) + k for k < TPL, TPL = 4 / GSTEP.
template <class D>
JQ_DEV void fold_groups(const f32x4& a, float out[4 / D::GSTEP]) {
  constexpr int TPL = 4 / D::GSTEP;
#pragma unroll
  for (int k = 0; k < TPL; ++k) {
    float v = 0.f;
#pragma unroll
    for (int j = 0; j < D::GSTEP; ++j) v += a[k * D::GSTEP + j];
    out[k] = v;
  }
}

}  // namespace jqd

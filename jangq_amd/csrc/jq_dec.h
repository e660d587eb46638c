// Decode-shaped matrix-core kernels (few activation rows): shared device code.
//
// Work unit: a 16-row tile of W over a K range, for up to TPB activation rows. Every lane
// streams its own row's codes straight from HBM into MFMA B fragments: lane (r = l%16,
// g = l/16) loads 32-code unit g of each 128-code step of row r (BITS whole words), so one
// wave load instruction reads 16 rows x 4*BITS*4 contiguous bytes and nothing is staged in
// LDS. The unit's four 8-code chunks become four B fragments (exact 16-bit "magic" values
// 2^B + q, see jq_common.h).
//
// A 128-code step spans GSTEP = 128/gs groups, and lane group g holds codes of group
// g / (4/GSTEP). Instead of splitting each MFMA by group, the group index is folded into the
// MFMA's M dimension: A row m' = GSTEP*t + j carries token t's activations only in the lane
// groups of group j (zeros elsewhere). One 16x16x32 MFMA per chunk then yields, for every
// (token, group) row, that group's magic dot product D; the constant B = 1 gives the
// activation sums X the same way. A lane's four output rows m' = 4*(l/16) + i belong to
// group i % GSTEP, so the per-group affine terms  s*D + (b - 2^B s)*X  use scales that are
// compile-time indexed per accumulator slot. Tokens per MFMA block: TPB = 16 / GSTEP.
#pragma once

#include "jq_common.h"

namespace jqd {

using namespace jq;

template <int BITS_, int GS_, int XDT_>
struct Dc {
  static constexpr int BITS = BITS_, GS = GS_, XDT = XDT_;
  static constexpr int GSTEP = 128 / GS;   // groups per 128-code step
  static constexpr int TPB = 16 / GSTEP;   // activation rows per MFMA block
  static constexpr int LPG = 4 / GSTEP;    // lane groups per group
  static constexpr bool NIB = BITS == 8 && XDT == JQ_BF16;  // 8-bit codes as two nibbles
  static constexpr bool TWO = BITS == 2;   // 2-bit: pairs 8 codes apart in one word
  static constexpr float OFF = NIB ? 272.f : (float)(1 << BITS);
  static constexpr uint32_t ONE2 = XDT == JQ_BF16 ? 0x3F803F80u : 0x3C003C00u;
};

// B fragment(s) of field C (0..3) of a unit. Field layout:
//   BITS != 2: chunk C = codes 8C..8C+7, pairs (c_p, c_{p+4})
//   BITS == 2: word C/2, pairs (c_j, c_{j+8}) for j = 4*(C%2) + p
template <class D, int C>
JQ_DEV void b_frag(const uint32_t* w, u32x4& b, u32x4& bh) {
  if constexpr (D::NIB) {
    uint32_t lo[4], hi[4];
    chunk8_nibble_pairs(w[2 * C], w[2 * C + 1], lo, hi);
    b = u32x4{lo[0], lo[1], lo[2], lo[3]};
    bh = u32x4{hi[0], hi[1], hi[2], hi[3]};
  } else if constexpr (D::TWO) {
    using Mg = Magic<D::XDT, 2>;
    constexpr int sh = Mg::shift;
    constexpr uint32_t pm = (3u << sh) | (3u << (sh + 16));
    const uint32_t word = w[C >> 1];
    uint32_t o[4];
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const int j = 4 * (C & 1) + p;
      const int s = 2 * j - sh;
      const uint32_t t = s >= 0 ? (word >> s) : (word << (-s));
      o[p] = (t & pm) | Mg::base;
    }
    b = u32x4{o[0], o[1], o[2], o[3]};
    bh = b;
  } else {
    uint32_t o[4];
    unit_chunk_pairs<D::XDT, D::BITS, C>(w, o);
    b = u32x4{o[0], o[1], o[2], o[3]};
    bh = b;
  }
}

// A fragment of field C for lane group lg from the activation row `xr` (16-bit elements,
// already offset to the step). Zero when the lane is inactive.
template <class D, int C>
JQ_DEV u32x4 a_frag(const uint16_t* xr, bool act, int lg) {
  if (!act) return u32x4{0u, 0u, 0u, 0u};
  if constexpr (D::TWO) {
    const int a = 32 * lg + 16 * (C >> 1) + 4 * (C & 1);
    const uint2 lo = *(const uint2*)(xr + a);
    const uint2 hi = *(const uint2*)(xr + a + 8);
    return u32x4{__builtin_amdgcn_perm(hi.x, lo.x, 0x05040100u),
                 __builtin_amdgcn_perm(hi.x, lo.x, 0x07060302u),
                 __builtin_amdgcn_perm(hi.y, lo.y, 0x05040100u),
                 __builtin_amdgcn_perm(hi.y, lo.y, 0x07060302u)};
  } else {
    const uint4 v = *(const uint4*)(xr + 32 * lg + 8 * C);
    const uint32_t raw[4] = {v.x, v.y, v.z, v.w};
    uint32_t pr[4];
    pair_activations(raw, pr);
    return u32x4{pr[0], pr[1], pr[2], pr[3]};
  }
}

// Scales / biases of GSTEP consecutive groups starting at element `g0` of a 16-bit sidecar row.
template <class D, int SB>
JQ_DEV void load_sb(const uint16_t* srow, const uint16_t* brow, int g0, float s[D::GSTEP],
                    float b[D::GSTEP]) {
  uint32_t sw[(D::GSTEP + 1) / 2], bw[(D::GSTEP + 1) / 2];
  if constexpr (D::GSTEP == 1) {
    sw[0] = srow[g0];
    bw[0] = brow[g0];
  } else if constexpr (D::GSTEP == 2) {
    sw[0] = *(const uint32_t*)(srow + g0);
    bw[0] = *(const uint32_t*)(brow + g0);
  } else {
    const uint2 a = *(const uint2*)(srow + g0), c = *(const uint2*)(brow + g0);
    sw[0] = a.x; sw[1] = a.y; bw[0] = c.x; bw[1] = c.y;
  }
#pragma unroll
  for (int j = 0; j < D::GSTEP; ++j) {
    const uint32_t hs = (sw[j >> 1] >> (16 * (j & 1))) & 0xFFFFu;
    const uint32_t hb = (bw[j >> 1] >> (16 * (j & 1))) & 0xFFFFu;
    if constexpr (SB == JQ_BF16) {
      s[j] = bf16_bits_to_f32(hs);
      b[j] = bf16_bits_to_f32(hb);
    } else {
      s[j] = f16_bits_to_f32((uint16_t)hs);
      b[j] = f16_bits_to_f32((uint16_t)hb);
    }
  }
}

// Partial sums of one 16-row tile over steps [s0, s1) for NB weight matrices sharing the
// activations. crow/srow/brow: this lane's W row (column of the output) per matrix.
// xr: this lane's activation row (token of A row l%16), act: whether the lane feeds A.
template <class D, int SB, int NB>
JQ_DEV void dec_tile(const uint16_t* xr, bool act, const uint32_t* const* crow,
                     const uint16_t* const* srow, const uint16_t* const* brow, int s0, int s1,
                     int lg, f32x4* acc) {
  constexpr int BITS = D::BITS;
  const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
  const u32x4 ones = {D::ONE2, D::ONE2, D::ONE2, D::ONE2};
  UnitWords<BITS> cur[NB], nxt[NB];
  if (s0 < s1) {
#pragma unroll
    for (int q = 0; q < NB; ++q) cur[q] = load_unit<BITS>(crow[q] + (s0 * 4 + lg) * BITS);
  }
  for (int s = s0; s < s1; ++s) {
    if (s + 1 < s1) {
#pragma unroll
      for (int q = 0; q < NB; ++q) nxt[q] = load_unit<BITS>(crow[q] + ((s + 1) * 4 + lg) * BITS);
    }
    const uint16_t* xs = xr + s * 128;
    const u32x4 A0 = a_frag<D, 0>(xs, act, lg), A1 = a_frag<D, 1>(xs, act, lg);
    const u32x4 A2 = a_frag<D, 2>(xs, act, lg), A3 = a_frag<D, 3>(xs, act, lg);
    f32x4 X = mfma16<D::XDT>(A0, ones, zero);
    X = mfma16<D::XDT>(A1, ones, X);
    X = mfma16<D::XDT>(A2, ones, X);
    X = mfma16<D::XDT>(A3, ones, X);
#pragma unroll
    for (int q = 0; q < NB; ++q) {
      float sc[D::GSTEP], bi[D::GSTEP];
      load_sb<D, SB>(srow[q], brow[q], s * D::GSTEP, sc, bi);
      u32x4 B, BH;
      b_frag<D, 0>(cur[q].w, B, BH);
      f32x4 Dd = mfma16<D::XDT>(A0, B, zero);
      f32x4 Dh = zero;
      if constexpr (D::NIB) Dh = mfma16<D::XDT>(A0, BH, zero);
      b_frag<D, 1>(cur[q].w, B, BH);
      Dd = mfma16<D::XDT>(A1, B, Dd);
      if constexpr (D::NIB) Dh = mfma16<D::XDT>(A1, BH, Dh);
      b_frag<D, 2>(cur[q].w, B, BH);
      Dd = mfma16<D::XDT>(A2, B, Dd);
      if constexpr (D::NIB) Dh = mfma16<D::XDT>(A2, BH, Dh);
      b_frag<D, 3>(cur[q].w, B, BH);
      Dd = mfma16<D::XDT>(A3, B, Dd);
      if constexpr (D::NIB) {
        Dh = mfma16<D::XDT>(A3, BH, Dh);
#pragma unroll
        for (int i = 0; i < 4; ++i) Dd[i] = fmaf(16.f, Dh[i], Dd[i]);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int j = i % D::GSTEP;
        const float c = fmaf(-D::OFF, sc[j], bi[j]);
        acc[q][i] = fmaf(sc[j], Dd[i], fmaf(c, X[i], acc[q][i]));
      }
    }
#pragma unroll
    for (int q = 0; q < NB; ++q) cur[q] = nxt[q];
  }
}

// Sum the partials of the 4 waves of a block (each wave covered a quarter of K). Returns
// the total in wave 0's registers. red: LDS scratch of 4 * NB * 256 floats.
template <int NB>
JQ_DEV void block_reduce4(f32x4* acc, float* red) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int q = 0; q < NB; ++q)
#pragma unroll
    for (int i = 0; i < 4; ++i) red[((wave * NB + q) * 4 + i) * 64 + lane] = acc[q][i];
  __syncthreads();
  if (wave == 0) {
#pragma unroll
    for (int q = 0; q < NB; ++q)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float v = red[((0 * NB + q) * 4 + i) * 64 + lane];
        v += red[((1 * NB + q) * 4 + i) * 64 + lane];
        v += red[((2 * NB + q) * 4 + i) * 64 + lane];
        v += red[((3 * NB + q) * 4 + i) * 64 + lane];
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

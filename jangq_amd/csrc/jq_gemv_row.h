// Whole-rows-per-wave decode GEMV body (one activation row), shared by the dense GEMV
// launches (jq_gemv.hip) and the fused MoE decode launches (jq_moe_fused_*.hip).
#pragma once

#include "jq_gemv.h"
#include "jq_qmv.h"

namespace {

using namespace jq;
using namespace jqg;
using jqk::QmvBatch;
using jqk::QmvProblem;

// Launch arguments: problems of one grouped launch share x, M, K and the dtypes; their row
// blocks are numbered 0 .. rb_begin[nprob) in problem order.
struct GemvArgs {
  QmvBatch b;
  int rb_begin[jqk::kMaxProblems + 1];
  int nprob;
  int ushift;    // log2(gs / 32)
  int kwshift;   // log2(waves per block)
  int yd;
  float glu_limit;  // SwiGLU clamp (gemv_row_kernel GLU form), 0: none
};

// The store of gemv_row_body: tot[r] (valid in lane 63) is row row0 + r's dot product; the GLU
// form holds the gate and up totals of row row0 and stores h = silu(round(g)) * round(u).
struct RowStore {
  template <int RB, bool GLU>
  JQ_DEV void finish(const GemvArgs& a, const QmvProblem& pb, int64_t row0, const float (&tot)[RB],
                     int lane) const {
    if constexpr (GLU) {
      if (lane == 63 && row0 < pb.N) {
        // g and u rounded to the output type first, as two matmuls returning it would be
        const bool bf = a.yd == JQ_BF16;
        const float g = bf ? bf16_bits_to_f32(f32_to_bf16_bits(tot[0])) : f16_bits_to_f32(f32_to_f16_bits(tot[0]));
        const float u = bf ? bf16_bits_to_f32(f32_to_bf16_bits(tot[1])) : f16_bits_to_f32(f32_to_f16_bits(tot[1]));
        const float hv = jqk::glu_value(g, u, a.glu_limit, 1.f);
        if (bf) store_t<JQ_BF16>(pb.y, row0, hv);
        else store_t<JQ_F16>(pb.y, row0, hv);
      }
    } else {
#pragma unroll
      for (int r = 0; r < RB; ++r) {
        const int64_t row = row0 + r;
        if (lane == 63 && row < pb.N) {
          if (a.yd == JQ_BF16) store_t<JQ_BF16>(pb.y, row, tot[r]);
          else if (a.yd == JQ_F16) store_t<JQ_F16>(pb.y, row, tot[r]);
          else store_t<JQ_F32>(pb.y, row, tot[r]);
        }
      }
    }
  }
};

// One activation row, whole rows per wave: lane l owns chunks l, l + 64, ... (CPL of them) of
// every row, so a row's sum is one DPP wave reduction and no LDS or barrier is involved. The
// waves (4 per block) are independent and persistent over row blocks of RB rows, with the
// same rolling register ring as gemv_kernel.
// GLU: problems 0 and 1 are the gate and up projections of a SwiGLU pair (same N); an item
// is row n of each (RB = 2), and the wave stores h[n] = silu(round(g)) * round(u) to
// problem 0's output.

template <class D, int SB, int CPL, int RB, bool GLU, class Fin>
JQ_DEV void gemv_row_body(const GemvArgs& a, int it, int nwaves, const Fin& fin) {
  static_assert(!GLU || RB == 2, "a SwiGLU item is one row of gate and one of up");
  constexpr int BITS = D::BITS;
  constexpr int UPL = units_per_chunk<BITS>();
  constexpr int NW = BITS * UPL;
  const int total = a.rb_begin[a.nprob];
  if (it >= total) return;  // this wave (no block-wide synchronisation below)
  const int K = a.b.K;
  const int lane = threadIdx.x & 63;
  const int C = K / (32 * UPL);
  const uint32_t rowbytes = (uint32_t)(K / 32) * BITS * 4;
  const uint32_t sbrow = (uint32_t)(K >> (a.ushift + 5)) * 2;
  bool act[CPL];
  uint32_t voff[CPL], vsb[CPL][UPL];
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const int c = lane + 64 * j;
    act[j] = c < C;
    const int ci = act[j] ? c : 0;
    voff[j] = (uint32_t)ci * (4 * NW);
#pragma unroll
    for (int t = 0; t < UPL; ++t) vsb[j][t] = (uint32_t)((ci * UPL + t) >> a.ushift) * 2;
  }
  jqd::XRaw xr[CPL][UPL];
#pragma unroll
  for (int j = 0; j < CPL; ++j)
#pragma unroll
    for (int t = 0; t < UPL; ++t)
      jqd::load_xraw((const uint16_t*)a.b.p[0].x + (int64_t)(voff[j] / (4 * NW) * UPL + t) * 32,
                     xr[j][t]);
  auto locate = [&](int i, int& p, int64_t& row0) {
    p = 0;
    if constexpr (GLU) {
      row0 = i;
      return;
    }
#pragma unroll
    for (int q = 1; q < jqk::kMaxProblems; ++q)
      if (q < a.nprob && i >= a.rb_begin[q]) p = q;
    row0 = (int64_t)(i - a.rb_begin[p]) * RB;
  };
  auto views = [&](int p, int64_t row0, bool live, Rsrc& rc, Rsrc& rs, Rsrc& rb) {
    const QmvProblem& pb = a.b.p[p];
    const int64_t left = pb.N - row0;
    constexpr int VR = GLU ? 1 : RB;  // rows of one view
    const uint32_t rows = live ? (uint32_t)(left < VR ? left : VR) : 0u;
    rc = make_rsrc((const char*)pb.codes + row0 * rowbytes, rows * rowbytes);
    rs = make_rsrc((const char*)pb.scales + row0 * sbrow, rows * sbrow);
    rb = make_rsrc((const char*)pb.biases + row0 * sbrow, rows * sbrow);
  };
  auto load_row = [&](Rsrc rc, Rsrc rs, Rsrc rb, int r, RowSlot<NW, UPL> (&slot)[CPL]) {
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      load_chunk<NW>(rc, voff[j] + r * rowbytes, slot[j].w);
      load_sb<D>(rs, rb, vsb[j], r * sbrow, slot[j]);
    }
  };
  int p;
  int64_t row0;
  locate(it, p, row0);
  Rsrc rc, rs, rbv, rcu, rsu, rbu;  // (up views: GLU only)
  views(p, row0, true, rc, rs, rbv);
  if constexpr (GLU) views(1, row0, true, rcu, rsu, rbu);
  RowSlot<NW, UPL> ring[RB][CPL];
#pragma unroll
  for (int r = 0; r < RB; ++r) {
    if (GLU && r == 1) load_row(rcu, rsu, rbu, 0, ring[r]);
    else load_row(rc, rs, rbv, GLU ? 0 : r, ring[r]);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
  }
  XState xs[CPL][UPL];
#pragma unroll
  for (int j = 0; j < CPL; ++j)
#pragma unroll
    for (int t = 0; t < UPL; ++t) {
      jqd::XRaw& r = xr[j][t];
#pragma unroll
      for (int i = 0; i < 16; ++i) r.d[i] = act[j] ? r.d[i] : 0u;
      make_xstate<D>(r, xs[j][t]);
    }
  const Bases<D> bs = jqd::make_bases<D>();
  for (;;) {
    const int nx = it + nwaves;
    const bool more = nx < total;
    int p2;
    int64_t row02;
    locate(more ? nx : it, p2, row02);
    Rsrc rc2, rs2, rb2, rcu2, rsu2, rbu2;
    views(p2, row02, more, rc2, rs2, rb2);
    if constexpr (GLU) views(1, row02, more, rcu2, rsu2, rbu2);
    float acc[RB];
#pragma unroll
    for (int r = 0; r < RB; ++r) {
      acc[r] = 0.f;
#pragma unroll
      for (int j = 0; j < CPL; ++j)
#pragma unroll
        for (int t = 0; t < UPL; ++t) {
          const float sv = sb_to_f32<SB>(ring[r][j].s[t]);
          const float bv = sb_to_f32<SB>(ring[r][j].b[t]);
          const float d = unit_dot<D>(ring[r][j].w + t * BITS, bs, xs[j][t]);
          acc[r] = fmaf(sv, d + xs[j][t].O, fmaf(bv, xs[j][t].X, acc[r]));
        }
      asm volatile("" : "+v"(acc[r])::"memory");
      if (GLU && r == 1) load_row(rcu2, rsu2, rbu2, 0, ring[r]);
      else load_row(rc2, rs2, rb2, GLU ? 0 : r, ring[r]);
      __builtin_amdgcn_sched_barrier(0);
    }
    const QmvProblem& pb = a.b.p[p];
    float tot[RB];
#pragma unroll
    for (int r = 0; r < RB; ++r) tot[r] = wave_total_lane63(acc[r]);
    fin.template finish<RB, GLU>(a, pb, row0, tot, lane);
    if (!more) break;
    it = nx;
    p = p2;
    row0 = row02;
  }
}

}  // namespace

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

// Lane chunks of the row body: two 32-code units for the widths in the bit mask JQ_ROW_UPL2
// (a chunk is then 16 B at 2 bits, 24 B at 3, 48 B at 6), one otherwise.
#ifndef JQ_ROW_UPL2
#define JQ_ROW_UPL2 0x4
#endif
template <int BITS>
constexpr int row_upl() {
  return ((JQ_ROW_UPL2 >> BITS) & 1) ? 2 : 1;
}
// Lane chunks per lane of a row of K codes (whole rows per wave).
inline int row_cpl(int64_t K, int bits) {
  const int64_t C = K / (32 * (((JQ_ROW_UPL2 >> bits) & 1) ? 2 : 1));
  return (int)((C + 63) / 64);
}

// The NW code words of a row-body lane chunk at byte voff of a view (16-byte loads where the
// chunk is a multiple of 8 bytes past 8; buffer loads need 4-byte alignment only).
template <int NW>
JQ_DEV void row_load_chunk(Rsrc r, uint32_t voff, uint32_t* w) {
  if constexpr (NW == 6 || NW == 12) {
#pragma unroll
    for (int i = 0; i < NW / 4; ++i) {
      const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, voff + 16 * i, 0, 0);
      w[4 * i] = v[0]; w[4 * i + 1] = v[1]; w[4 * i + 2] = v[2]; w[4 * i + 3] = v[3];
    }
    if constexpr (NW % 4) {
      const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(r, voff + 16 * (NW / 4), 0, 0);
      w[NW - 2] = v[0]; w[NW - 1] = v[1];
    }
  } else {
    load_chunk<NW>(r, voff, w);
  }
}

// The decode type of the row body: 6- and 8-bit codes with bf16 activations take the
// f16-rescaled units (one instruction per code pair).
template <class D>
struct RowD {
  using type = D;
};
template <int GS>
struct RowD<jqd::Dc<8, GS, JQ_BF16>> {
  using type = jqd::Dc<8, GS, JQ_BF16, true>;
};
template <int GS>
struct RowD<jqd::Dc<6, GS, JQ_BF16>> {
  using type = jqd::Dc<6, GS, JQ_BF16, true>;
};

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
// waves (4 per block) are independent; each walks a contiguous range of row blocks of RB rows
// with the same rolling register ring as gemv_kernel.
// GLU: problems 0 and 1 are the gate and up projections of a SwiGLU pair (same N); an item
// is row n of each (RB = 2), and the wave stores h[n] = silu(round(g)) * round(u) to
// problem 0's output.

// SHARE: the block's threads build the activation state once in LDS (blocks of at least
// CPL * 64 * UPL threads whose waves all run this body); otherwise every wave builds its own.
template <class D, int SB, int CPL, int RB, bool GLU, class Fin, bool SHARE = false>
JQ_DEV void gemv_row_body(const GemvArgs& a, int it, int nwaves, const Fin& fin) {
  static_assert(!GLU || RB == 2, "a SwiGLU item is one row of gate and one of up");
  constexpr int BITS = D::BITS;
  constexpr int UPL = row_upl<BITS>();
  constexpr int NW = BITS * UPL;
  // Both units of a chunk lie in one group (one scale and bias for the pair).
  constexpr bool SHARED = UPL == 2 && D::GS >= 64;
  const int total = a.rb_begin[a.nprob];
  // Wave w takes the contiguous items [w * per, (w + 1) * per): the problem and the row block
  // then advance by one step per item instead of being looked up again.
  const int per = (total + nwaves - 1) / nwaves;
  const int iend = (it + 1) * per < total ? (it + 1) * per : total;
  it *= per;
  // SHARE: a wave without items still takes part in building the block's activation state
  // (one barrier below); its loads go through views of 0 bytes.
  const bool has = it < total;
  if (!SHARE && !has) return;
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
      row_load_chunk<NW>(rc, voff[j] + r * rowbytes, slot[j].w);
      load_sb<D>(rs, rb, vsb[j], r * sbrow, slot[j]);
    }
  };
  // Activation state of every 32-code unit of a row, built once per block: thread u of the
  // block takes unit u (make_xstate, the arithmetic every wave would otherwise repeat) and
  // publishes it in LDS. Its activations are loaded before the weight rows (the vector-memory
  // count is in order: loaded after them, they would wait for the rows); x is read through a
  // view of K values, so units past the row read zeros and contribute exactly 0.
  constexpr int UMAX = CPL * 64 * UPL;
  const int ut = (int)threadIdx.x;  // SHARE: blockDim.x >= UMAX (the launchers' blocks)
  const Rsrc rx = make_rsrc(a.b.p[0].x, (uint32_t)K * 2);
  jqd::XRaw xr[SHARE ? 1 : CPL][SHARE ? 1 : UPL];
#pragma unroll
  for (int j = 0; j < (SHARE ? 1 : CPL); ++j)
#pragma unroll
    for (int t = 0; t < (SHARE ? 1 : UPL); ++t) {
      const uint32_t u = SHARE ? (uint32_t)ut : (uint32_t)((lane + 64 * j) * UPL + t);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rx, u * 64 + 16 * i, 0, 0);
        xr[j][t].d[4 * i] = v[0]; xr[j][t].d[4 * i + 1] = v[1];
        xr[j][t].d[4 * i + 2] = v[2]; xr[j][t].d[4 * i + 3] = v[3];
      }
    }
  int p;
  int64_t row0;
  locate(has ? it : 0, p, row0);
  Rsrc rc, rs, rbv, rcu, rsu, rbu;  // (up views: GLU only)
  views(p, row0, has, rc, rs, rbv);
  if constexpr (GLU) views(1, row0, has, rcu, rsu, rbu);
  RowSlot<NW, UPL> ring[RB][CPL];
#pragma unroll
  for (int r = 0; r < RB; ++r) {
    if (GLU && r == 1) load_row(rcu, rsu, rbu, 0, ring[r]);
    else load_row(rc, rs, rbv, GLU ? 0 : r, ring[r]);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
  }
  XState xs[CPL][UPL];
  if constexpr (SHARE) {
    __shared__ __attribute__((aligned(16))) uint32_t xsh[UMAX][20];
    if (ut < UMAX) {
      XState t;
      make_xstate<D>(xr[0][0], t);
#pragma unroll
      for (int i = 0; i < 4; ++i)
        *(u32x4*)&xsh[ut][4 * i] = u32x4{t.pr[4 * i], t.pr[4 * i + 1], t.pr[4 * i + 2], t.pr[4 * i + 3]};
      *(u32x4*)&xsh[ut][16] = u32x4{__float_as_uint(t.X), __float_as_uint(t.O),
                                    __float_as_uint(t.scl), 0u};
    }
    __syncthreads();
    if (!has) return;
#pragma unroll
    for (int j = 0; j < CPL; ++j)
#pragma unroll
      for (int t = 0; t < UPL; ++t) {
        const int u = (lane + 64 * j) * UPL + t;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const u32x4 v = *(const u32x4*)&xsh[u][4 * i];
          xs[j][t].pr[4 * i] = v[0]; xs[j][t].pr[4 * i + 1] = v[1];
          xs[j][t].pr[4 * i + 2] = v[2]; xs[j][t].pr[4 * i + 3] = v[3];
        }
        const u32x4 v = *(const u32x4*)&xsh[u][16];
        xs[j][t].X = __uint_as_float(v[0]);
        xs[j][t].O = __uint_as_float(v[1]);
        xs[j][t].scl = __uint_as_float(v[2]);
      }
  } else {
#pragma unroll
    for (int j = 0; j < CPL; ++j)
#pragma unroll
      for (int t = 0; t < UPL; ++t) make_xstate<D>(xr[j][t], xs[j][t]);
  }
  float xo[CPL], xx[CPL];  // SHARED: O and X of the chunk's two units together
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    xo[j] = xs[j][0].O + xs[j][UPL - 1].O;
    xx[j] = xs[j][0].X + xs[j][UPL - 1].X;
  }
  const Bases<D> bs = jqd::make_bases<D>();
  for (;;) {
    const int nx = it + 1;
    const bool more = nx < iend;
    int p2 = p;
    int64_t row02 = GLU ? (int64_t)nx : row0 + RB;
    if constexpr (!GLU) {
      while (p2 + 1 < a.nprob && nx >= a.rb_begin[p2 + 1]) {  // next problem (rarely taken)
        ++p2;
        row02 = (int64_t)(nx - a.rb_begin[p2]) * RB;
      }
    }
    Rsrc rc2, rs2, rb2, rcu2, rsu2, rbu2;
    views(p2, row02, more, rc2, rs2, rb2);
    if constexpr (GLU) views(1, row02, more, rcu2, rsu2, rbu2);
    float acc[RB];
#pragma unroll
    for (int r = 0; r < RB; ++r) {
      acc[r] = 0.f;
#pragma unroll
      for (int j = 0; j < CPL; ++j) {
        if constexpr (SHARED) {
          const float sv = sb_to_f32<SB>(ring[r][j].s[0]);
          const float bv = sb_to_f32<SB>(ring[r][j].b[0]);
          const float d = unit_dot<D>(ring[r][j].w, bs, xs[j][0]) +
                          unit_dot<D>(ring[r][j].w + BITS, bs, xs[j][1]);
          acc[r] = fmaf(sv, d + xo[j], fmaf(bv, xx[j], acc[r]));
        } else {
#pragma unroll
          for (int t = 0; t < UPL; ++t) {
            float sv = sb_to_f32<SB>(ring[r][j].s[t]);
            const float bv = sb_to_f32<SB>(ring[r][j].b[t]);
            const float d = unit_dot<D>(ring[r][j].w + t * BITS, bs, xs[j][t]);
            if constexpr (D::F16X) sv *= xs[j][t].scl;  // d and O are in x' units
            acc[r] = fmaf(sv, d + xs[j][t].O, fmaf(bv, xs[j][t].X, acc[r]));
          }
        }
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

// Expert-gathered decode GEMV body, shared by the gather launches (jq_gemv_gather.hip) and the
// fused MoE decode launches (jq_moe_fused_*.hip). See jq_gemv_gather.hip for the design.
#pragma once

#include "jq_gemv.h"
#include "jq_qmv.h"
#include "jq_route.h"

#include <type_traits>

namespace {

using namespace jq;
using namespace jqg;
using jqk::GatherPlan;
using jqk::QmmProblem;

constexpr int kMaxCombSlots = 16;  // expert slots (waves) of a combined-form block

struct GatherArgs {
  QmmProblem p[2];  // the projection (and up, NB == 2); output and shapes from p[0]
  GatherPlan plan;
  int nrb;          // row blocks per tile
  int ushift;       // log2(gs / 32)
  int kwshift;      // log2(waves per block)
  int yd;
  // Combined form (direct pairs t*ck + j, one row each): the k experts of a token summed in
  // slot order, then the shared expert's term (jqk::moe_final):
  //   after the down projection (cbefore = 0): round(sum_j cw[t*ck+j] * y[t*ck+j, n])
  //   before it (cbefore = 1, weights already in h):   sum_j y[t*ck+j, n]
  // with each slot output y rounded to the output dtype first.
  const float* cw;
  const void* cshared;
  const void* cgate;  // [T] logits of the shared term's sigmoid gate, or NULL
  void* cout;
  int ck, ctok, cbefore;
  // Routed form (direct pairs t*rk + j of a launch that routes for itself): pair t*rk + j
  // uses the j-th expert of the token's top-rk (jqr::route_wave on rlogits[t]); the token's
  // ids and weights go to ridx / rw (for the launches that follow). With rbefore, h of pair
  // t*rk + j is multiplied by its routing weight.
  const void* rlogits;
  uint32_t* ridx;
  float* rw;
  int rE, rk, rbefore;
  jqr::RouteOpts ro;
};

constexpr int kRouteSlots = 8;  // routed form: up to 64 * 8 = 512 experts

// No combined or routed form.
void init_forms(GatherArgs& a) {
  a.cw = nullptr;
  a.cshared = nullptr;
  a.cgate = nullptr;
  a.cout = nullptr;
  a.ck = a.ctok = a.cbefore = 0;
  a.rlogits = nullptr;
  a.ridx = nullptr;
  a.rw = nullptr;
  a.rE = a.rk = a.rbefore = 0;
  a.ro = jqr::softmax_opts(1);
}

JQ_DEV float round_out(float v, int yd) {
  if (yd == JQ_BF16) return bf16_bits_to_f32(f32_to_bf16_bits(v));
  if (yd == JQ_F16) return f16_bits_to_f32(f32_to_f16_bits(v));
  return v;
}

JQ_DEV float load_out(const void* y, int64_t i, int yd) {
  if (yd == JQ_BF16) return load_t<JQ_BF16>(y, i);
  if (yd == JQ_F16) return load_t<JQ_F16>(y, i);
  return load_t<JQ_F32>(y, i);
}

JQ_DEV void store_out(void* y, int64_t i, float v, int yd) {
  if (yd == JQ_BF16) store_t<JQ_BF16>(y, i, v);
  else if (yd == JQ_F16) store_t<JQ_F16>(y, i, v);
  else store_t<JQ_F32>(y, i, v);
}

// The activation and output rows of a tile's MT plan rows (wave-uniform). A plan row past
// the tile, or whose x row lies outside x, reads zeros; only rows inside the tile are stored.
template <int MT>
struct TileRows {
  int64_t xrow[MT];
  int64_t orow[MT];
  bool xlive[MT];
  int nrows;
};

template <int MT>
JQ_DEV void tile_rows(const GatherPlan& pl, int4 tl, TileRows<MT>& tr) {
  tr.nrows = tl.z;
#pragma unroll
  for (int m = 0; m < MT; ++m) {
    const int rr = tl.y + (m < tl.z ? m : 0);
    const int Mp = pl.M;
    const int pi = Mp == 1 ? rr : rr / Mp, mi = Mp == 1 ? 0 : rr - pi * Mp;
    const uint32_t pair = pl.order ? pl.order[tl.w + pi] : (uint32_t)(tl.w + pi);
    const int64_t xr = (int64_t)(pl.lhs ? pl.lhs[pair] : pair / (uint32_t)pl.pair_div) * Mp + mi;
    tr.xlive[m] = m < tl.z && xr < pl.x_rows;
    tr.xrow[m] = tr.xlive[m] ? xr : 0;
    tr.orow[m] = (int64_t)pair * Mp + mi;
  }
}

// Tile t of the plan, or in direct mode pairs [t*R, t*R + R) of expert rhs[t*R] (0 rows if
// the id is out of range).
JQ_DEV int4 get_tile(const GatherPlan& pl, int t) {
  if (pl.tiles) return pl.tiles[t];
  const int r0 = t * pl.direct_rows;
  const int left = pl.direct_pairs - r0;
  const uint32_t e = pl.rhs ? pl.rhs[r0] : 0u;
  const bool ok = e < (uint32_t)pl.E;
  return make_int4(ok ? (int)e : 0, 0, ok ? (left < pl.direct_rows ? left : pl.direct_rows) : 0, r0);
}

// Sum over each group of 64/RW consecutive lanes; the total lands in the group's last lane
// (RW = 1: the whole wave, lane 63).
template <int RW>
JQ_DEV float group_total(float v) {
  if constexpr (RW == 1) {
    return wave_total_lane63(v);
  } else {
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));   // quad_perm 1,0,3,2
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));   // quad_perm 2,3,0,1
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x124, 0xF, 0xF, false));  // row_ror 4
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x128, 0xF, 0xF, false));  // row_ror 8
    if constexpr (RW == 2)
      v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x142, 0xA, 0xF, false));  // row_bcast 15
    return v;
  }
}

// RW: rows per wave instruction. Rows shorter than 64 lane chunks (RW = 2, 4) split a single
// wave into RW groups of 64/RW lanes; group g loads item rows g*RBL .. g*RBL + RBL - 1, and a
// lane keeps the activations of its chunk for every row. RBL: ring slots (rows) per lane.
// COMB: the combined form above. Items are (token, row block); wave j of a block computes
// expert slot j's rows of the item over the whole of K (the waves do not split K), and wave 0
// sums the k slot outputs of each row in slot order.
// ROUTE: the routed form above; every wave computes its token's top-k (kept in its lanes,
// recomputed when the token changes) instead of reading expert ids.
template <class D, int SB, int MT, int RBL, int NB, int RW, bool COMB = false, bool ROUTE = false>
JQ_DEV void gather_body(const GatherArgs& a, int bid, int nblk) {
  constexpr int BITS = D::BITS;
  constexpr int UPL = units_per_chunk<BITS>();
  constexpr int NW = BITS * UPL;
  constexpr int RB = RBL * RW;   // rows of an item (both projections)
  constexpr int ROWS = RB / NB;  // weight rows of one projection per item
  constexpr int CL = 64 / RW;    // lanes per row group
  __shared__ float red[2][COMB ? kMaxCombSlots : kMaxWaves][RB * MT];

  const int ntiles = a.plan.n_tiles ? *a.plan.n_tiles
                                     : (a.plan.direct_pairs + a.plan.direct_rows - 1) / a.plan.direct_rows;
  int first, end;
  if constexpr (ROUTE) {
    // Routed form: nblk is a multiple of the token count (the launchers see to it) and a
    // block's items belong to one token, so each wave routes once, before its first item.
    const int T = ntiles / a.rk, bpt = nblk / T, tok = bid / bpt, sub = bid - tok * bpt;
    const int items_t = a.rk * a.nrb;
    const int per = (items_t + bpt - 1) / bpt;
    first = tok * items_t + sub * per;
    const int tend = (tok + 1) * items_t;
    end = tok < T && first + per < tend ? first + per : tend;
    if (tok >= T) end = first;
  } else {
    const int items = (COMB ? a.ctok : ntiles) * a.nrb;
    const int per = (items + nblk - 1) / nblk;
    first = bid * per;
    end = first + per < items ? first + per : items;
  }
  if (first >= end) return;  // whole block
  const int KW = COMB ? 1 : blockDim.x >> 6;  // waves over K
  const int K = (int)a.p[0].K;
  const int64_t N = a.p[0].N;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int C = K / (32 * UPL);                       // chunks per row
  const int CW = (C + KW - 1) >> a.kwshift;           // chunks per wave
  const uint32_t rowbytes = (uint32_t)(K / 32) * BITS * 4;
  const uint32_t sbrow = (uint32_t)(K >> (a.ushift + 5)) * 2;

  const int sr = RW == 1 ? 0 : lane / CL;  // row group of the lane
  const int lc = RW == 1 ? lane : lane % CL;
  const int c = (COMB ? 0 : wave) * CW + lc;
  const bool act = lc < CW && c < C;
  const int ci = act ? c : 0;
  const uint32_t voff = (uint32_t)ci * (4 * NW);
  uint32_t vsb[UPL];
#pragma unroll
  for (int t = 0; t < UPL; ++t) vsb[t] = (uint32_t)((ci * UPL + t) >> a.ushift) * 2;

  // Buffer views of an item's rows of each projection (rows past N read zero).
  auto views = [&](int4 tl, int64_t row0, bool live, Rsrc (&rc)[NB], Rsrc (&rs)[NB],
                   Rsrc (&rb)[NB]) {
    const int64_t left = N - row0;
    const uint32_t rows = live && tl.z > 0 ? (uint32_t)(left < ROWS ? left : ROWS) : 0u;
#pragma unroll
    for (int q = 0; q < NB; ++q) {
      const QmmProblem& pb = a.p[q];
      const int64_t e = tl.x;
      rc[q] = make_rsrc((const char*)(pb.codes + e * pb.expert_stride_codes) + row0 * rowbytes,
                        rows * rowbytes);
      const int64_t sb0 = e * pb.expert_stride_sb * 2 + row0 * sbrow;
      rs[q] = make_rsrc((const char*)pb.scales + sb0, rows * sbrow);
      rb[q] = make_rsrc((const char*)pb.biases + sb0, rows * sbrow);
    }
  };
  // Ring slot r of a lane holds item row ir = sr*RBL + r: row ir / NB of projection r % NB.
  auto load_row = [&](const Rsrc (&rc)[NB], const Rsrc (&rs)[NB], const Rsrc (&rb)[NB], int r,
                      RowSlot<NW, UPL>& slot) {
    const int q = r % NB, rr = (sr * RBL + r) / NB;
    load_chunk<NW>(rc[q], voff + rr * rowbytes, slot.w);
    load_sb<D>(rs[q], rb[q], vsb, rr * sbrow, slot);
  };
  XState xs[UPL][MT];
  auto load_x = [&](const TileRows<MT>& tr) {
    jqd::XRaw xr[UPL][MT];
#pragma unroll
    for (int t = 0; t < UPL; ++t)
#pragma unroll
      for (int m = 0; m < MT; ++m)
        jqd::load_xraw((const uint16_t*)a.p[0].x + tr.xrow[m] * K + (int64_t)(ci * UPL + t) * 32,
                       xr[t][m]);
#pragma unroll
    for (int t = 0; t < UPL; ++t)
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        jqd::XRaw& r = xr[t][m];
        const bool live = act && tr.xlive[m];
#pragma unroll
        for (int i = 0; i < 16; ++i) r.d[i] = live ? r.d[i] : 0u;
        make_xstate<D>(r, xs[t][m]);
      }
  };

  int it = first;
  int tile, rbi;
  int ct = 0;  // combined form: token of the item
  if constexpr (COMB) {
    ct = it / a.nrb;
    rbi = it - ct * a.nrb;
    tile = ct * a.ck + wave;  // the wave's expert slot
  } else {
    tile = it / a.nrb;
    rbi = it - tile * a.nrb;
  }
  // Routed form: lane j holds expert j (and its weight) of the block's token.
  uint32_t rt_id = 0;
  float rt_w = 0.f;
  auto tile_of = [&](int t, auto can_route) -> int4 {
    if constexpr (ROUTE) {
      const int tok = t / a.rk, j = t - tok * a.rk;
      if constexpr (decltype(can_route)::value) {  // the wave's first item only
        // Rounds up to the last slot the wave's items use; all k for the wave that publishes
        // the token's ids and weights, and for renormalised weights that enter h.
        const int last = (end - 1) / a.nrb - tok * a.rk;
        const bool all = first == tok * a.rk * a.nrb || (a.rbefore && a.ro.renorm);
        jqr::route_wave<kRouteSlots>(
            (const char*)a.rlogits + (int64_t)tok * a.rE * (a.ro.logit_dtype == JQ_F32 ? 4 : 2),
            a.rE, a.rk, a.ro, lane, rt_id, rt_w, all ? a.rk : last + 1);
      }
      const uint32_t e = (uint32_t)__builtin_amdgcn_readlane((int)rt_id, j);
      const bool ok = e < (uint32_t)a.plan.E;
      return make_int4(ok ? (int)e : 0, 0, ok ? 1 : 0, t);
    } else {
      return get_tile(a.plan, t);
    }
  };
  // The token's ids and weights, once per token: by wave 0 of the item (pair t*rk, row block 0).
  auto publish = [&](int t, int rb) {
    if constexpr (ROUTE) {
      const int tok = t / a.rk;
      if (t == tok * a.rk && rb == 0 && wave == 0 && lane < a.rk) {
        a.ridx[(int64_t)tok * a.rk + lane] = rt_id;
        a.rw[(int64_t)tok * a.rk + lane] = rt_w;
      }
    }
  };
  int4 tl = tile_of(tile, std::true_type{});
  publish(tile, rbi);
  TileRows<MT> tr;
  tile_rows<MT>(a.plan, tl, tr);
  int64_t row0 = (int64_t)rbi * ROWS;
  // Combined form: the combine's routing weights, shared row and shared-gate logit of an item
  // are requested together with the item's rows, so they sit in registers by the combine
  // instead of costing a dependent round trip at its end. Range-checked buffer loads without
  // a branch (lanes past the slots or rows read 0 or a value that is not used); 16-bit
  // halves, so every output dtype takes the same two loads.
  uint32_t pw = 0, psh = 0, psh_hi = 0, pgl = 0, pgl_hi = 0;
  auto prefetch = [&](int ctk, int64_t r0) {
    if constexpr (COMB) {
      const uint32_t es = a.yd == JQ_F32 ? 4u : 2u;
      const Rsrc rw = make_rsrc(a.cw ? a.cw + (int64_t)ctk * a.ck : nullptr,
                                a.cw && !a.cbefore ? (uint32_t)a.ck * 4u : 0u);
      pw = __builtin_amdgcn_raw_buffer_load_b32(rw, (uint32_t)lane * 4u, 0, 0);
      const int64_t nr = N - r0 < ROWS ? N - r0 : ROWS;
      const Rsrc rsh = make_rsrc(a.cshared ? (const char*)a.cshared + ((int64_t)ctk * N + r0) * es
                                           : nullptr,
                                 a.cshared ? (uint32_t)nr * es : 0u);
      psh = __builtin_amdgcn_raw_buffer_load_b16(rsh, (uint32_t)lane * es, 0, 0);
      psh_hi = __builtin_amdgcn_raw_buffer_load_b16(rsh, (uint32_t)lane * es + 2u, 0, 0);
      const Rsrc rg = make_rsrc(a.cgate ? (const char*)a.cgate + (int64_t)ctk * es : nullptr,
                                a.cgate ? es : 0u);
      pgl = __builtin_amdgcn_raw_buffer_load_b16(rg, 0u, 0, 0);
      pgl_hi = __builtin_amdgcn_raw_buffer_load_b16(rg, 2u, 0, 0);
    }
  };
  // (the halves are joined only where the value is used, so the loads need not have landed
  // when they are issued)
  auto out_value = [&](uint32_t lo, uint32_t hi) {
    return a.yd == JQ_F32 ? __uint_as_float((lo & 0xFFFFu) | (hi << 16))
           : a.yd == JQ_BF16 ? __uint_as_float(lo << 16) : f16_bits_to_f32((uint16_t)lo);
  };
  prefetch(ct, row0);
  Rsrc rc[NB], rs[NB], rbv[NB];
  views(tl, row0, true, rc, rs, rbv);
  RowSlot<NW, UPL> ring[RBL];
#pragma unroll
  for (int r = 0; r < RBL; ++r) {
    load_row(rc, rs, rbv, r, ring[r]);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
  }
  load_x(tr);
  const Bases<D> bs = jqd::make_bases<D>();

  for (int par = 0;; par ^= 1) {
    const bool more = it + 1 < end;
    const bool wrap = rbi + 1 == a.nrb;
    const int tile2 = more && wrap ? tile + (COMB ? a.ck : 1) : tile;
    const int rbi2 = more ? (wrap ? 0 : rbi + 1) : rbi;
    const int ct2 = more && wrap ? ct + 1 : ct;
    const int4 tl2 = tile_of(tile2, std::false_type{});
    if (more) publish(tile2, rbi2);
    const int64_t row02 = (int64_t)rbi2 * ROWS;
    Rsrc rc2[NB], rs2[NB], rb2[NB];
    views(tl2, row02, more, rc2, rs2, rb2);

    float acc[RBL][MT];
#pragma unroll
    for (int r = 0; r < RBL; ++r) {
#pragma unroll
      for (int m = 0; m < MT; ++m) acc[r][m] = 0.f;
#pragma unroll
      for (int t = 0; t < UPL; ++t) {
        const float sv = sb_to_f32<SB>(ring[r].s[t]);
        const float bv = sb_to_f32<SB>(ring[r].b[t]);
#pragma unroll
        for (int m = 0; m < MT; ++m) {
          const float d = unit_dot<D>(ring[r].w + t * BITS, bs, xs[t][m]);
          acc[r][m] = fmaf(sv, d + xs[t][m].O, fmaf(bv, xs[t][m].X, acc[r][m]));
        }
      }
      // Row r is consumed before its slot is reloaded (see the dense GEMV).
#pragma unroll
      for (int m = 0; m < MT; ++m) asm volatile("" : "+v"(acc[r][m])::"memory");
      load_row(rc2, rs2, rb2, r, ring[r]);
      __builtin_amdgcn_sched_barrier(0);
    }

#pragma unroll
    for (int r = 0; r < RBL; ++r)
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        const float v = group_total<RW>(acc[r][m]);
        // (an expert id outside the range gives a slot of 0 rows: it contributes 0)
        if (lc == CL - 1) red[par][wave][(sr * RBL + r) * MT + m] = COMB && tr.nrows == 0 ? 0.f : v;
      }
    __syncthreads();
    if constexpr (COMB) {
      // Each slot's output row, rounded as the expert output, joins the token's sum in slot
      // order (fp32); then the shared expert's term, and the store rounds.
      const int64_t row = row0 + lane;
      if (wave == 0 && lane < ROWS && row < N) {
        float comb = 0.f;
        for (int j = 0; j < a.ck; ++j) {
          const float y = round_out(red[par][j][lane], a.yd);
          comb = a.cbefore ? comb + y : fmaf(jqr::lane_read(__uint_as_float(pw), j), y, comb);
        }
        const float sh = out_value(psh, psh_hi), gl = out_value(pgl, pgl_hi);
        store_out(a.cout, (int64_t)ct * N + row,
                  jqk::moe_final(a.cbefore, comb, a.cshared != nullptr, sh, a.cgate != nullptr, gl,
                                 a.yd),
                  a.yd);
      }
    } else if (wave == 0 && lane < ROWS * MT) {
      const int j = lane / MT, m = lane % MT;
      int64_t orow = tr.orow[0];
      bool live = 0 < tr.nrows;
#pragma unroll
      for (int q = 1; q < MT; ++q)
        if (m == q) orow = tr.orow[q], live = q < tr.nrows;
      const int64_t row = row0 + j;
      if (live && row < N) {
        float v = 0.f;
        for (int w = 0; w < KW; ++w) v += red[par][w][(NB * j) * MT + m];
        if constexpr (NB == 2) {
          float u = 0.f;
          for (int w = 0; w < KW; ++w) u += red[par][w][(NB * j + 1) * MT + m];
          const float g = round_out(v, a.yd), up = round_out(u, a.yd);
          // the pair's routing weight when it enters before the down projection
          float f = a.p[0].glu_scale ? a.p[0].glu_scale[orow] : 1.f;
          if constexpr (ROUTE) {
            const int jj = tile - (tile / a.rk) * a.rk;
            f = a.rbefore ? jqr::lane_read(rt_w, jj) : 1.f;
          }
          v = jqk::glu_value(g, up, a.p[0].glu_limit, f);
        }
        store_out(a.p[0].y, orow * N + row, v, a.yd);
      }
    }
    if (!more) break;
    if (tile2 != tile) {
      // New tile: its activation rows replace the registers (the ring keeps the next rows).
      tile_rows<MT>(a.plan, tl2, tr);
      load_x(tr);
    }
    if constexpr (COMB) {
      // the next item's combine inputs, once this item's are consumed (after its combine)
      __builtin_amdgcn_sched_barrier(0);
      prefetch(ct2, row02);
    }
    it += 1;
    tile = tile2;
    rbi = rbi2;
    ct = ct2;
    tl = tl2;
    row0 = row02;
#pragma unroll
    for (int q = 0; q < NB; ++q) rc[q] = rc2[q], rs[q] = rs2[q], rbv[q] = rb2[q];
  }
}

}  // namespace

// Expert-gathered decode GEMV on the vector ALUs: the MoE gather_qmm and SwitchGLU launches
// when each selected expert serves only a few activation rows (decode batches).
//
//   y[o(r), n] = sum_k x[i(r), k] * (q_e[n,k] * s_e[n,k/gs] + b_e[n,k/gs])
//
// for every row r of the expert-grouped plan (expert e, x row i(r), output row o(r)), and with
// two projections (gate, up) of the same expert:  h = silu(gate) * up.
//
// Work items are (tile, row block): a tile is up to MT plan rows of one expert, a row block
// RB / NB consecutive weight rows of that expert (NB = 2: each row of gate and of up). The
// kernel reads the number of tiles from the plan, numbers the items tile-major and gives each
// block one contiguous range, so a block changes tiles rarely. Inside a block the arithmetic
// and the register ring are those of the dense GEMV: a lane holds its K slice of the tile's
// activation rows, the ring holds the next item's rows in flight while the block computes,
// reduces and stores the current one. At a tile change the block reloads the activations.
//
// Two decode-size forms over direct plans (one row per pair): the combined form runs the
// down projection with the MoE weighted combine inside (one wave per expert slot), and the
// routed form runs gate|up with each wave computing its token's top-k from the router logits
// instead of reading expert ids.
//
// Reference: gather_qmm over affine codes (mlx.core.gather_qmm as called from
// jang-tools/jang_tools/dots3/ops.py:202-214 and jangrt/switchglu_decode.py:161-183), the
// per-group affine sum s * sum q x + b * sum x (jang-tools/jang_tools/dsv41/metal_decode.py:202-233).
#include "jq_gemv.h"
#include "jq_qmv.h"
#include "jq_route.h"

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
__global__ void __launch_bounds__(64 * (COMB ? kMaxCombSlots : kMaxWaves))
gemv_gather_kernel(GatherArgs a) {
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
  {
    const int items = (COMB ? a.ctok : ntiles) * a.nrb;
    const int per = (items + (int)gridDim.x - 1) / (int)gridDim.x;
    first = blockIdx.x * per;
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
#pragma unroll
    for (int t = 0; t < UPL; ++t) {
      slot.s[t] = __builtin_amdgcn_raw_buffer_load_b16(rs[q], vsb[t] + rr * sbrow, 0, 0);
      slot.b[t] = __builtin_amdgcn_raw_buffer_load_b16(rb[q], vsb[t] + rr * sbrow, 0, 0);
    }
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
  // Routed form: lane j holds expert j (and its weight) of token rt_tok.
  int rt_tok = -1;
  uint32_t rt_id = 0;
  float rt_w = 0.f;
  auto tile_of = [&](int t) -> int4 {
    if constexpr (ROUTE) {
      const int tok = t / a.rk, j = t - tok * a.rk;
      if (tok != rt_tok) {  // wave-uniform
        jqr::route_wave<kRouteSlots>(
            (const char*)a.rlogits + (int64_t)tok * a.rE * (a.ro.logit_dtype == JQ_F32 ? 4 : 2),
            a.rE, a.rk, a.ro, lane, rt_id, rt_w);
        rt_tok = tok;
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
  int4 tl = tile_of(tile);
  publish(tile, rbi);
  TileRows<MT> tr;
  tile_rows<MT>(a.plan, tl, tr);
  int64_t row0 = (int64_t)rbi * ROWS;
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
    const int4 tl2 = tile_of(tile2);
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
          comb = a.cbefore ? comb + y : fmaf(a.cw[ct * a.ck + j], y, comb);
        }
        const float sh = a.cshared ? load_out(a.cshared, (int64_t)ct * N + row, a.yd) : 0.f;
        const float gl = a.cgate ? load_out(a.cgate, ct, a.yd) : 0.f;
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

template <class D, int SB, int MT, int RBL, int NB, int RW, bool COMB = false, bool ROUTE = false>
int launch_g(GatherArgs& a, int64_t max_tiles, hipStream_t st) {
  int kws = 0;
  int kw = RW == 1 ? gemv_waves(a.p[0].K, D::BITS, &kws) : 1;
  if (kw > kMaxWaves) return JQ_ERR_SHAPE;
  if (COMB) {
    if (kw != 1 || a.ck > kMaxCombSlots) return JQ_ERR_SHAPE;
    kw = a.ck;  // one wave per expert slot
  }
  a.kwshift = kws;
  constexpr int ROWS = RBL * RW / NB;
  const int64_t nrb = (a.p[0].N + ROWS - 1) / ROWS;
  const int64_t max_items = max_tiles * nrb;
  if (nrb == 0 || max_items == 0) return JQ_OK;
  if (max_items >= ((int64_t)1 << 31)) return JQ_ERR_SHAPE;
  a.nrb = (int)nrb;
  const int64_t units = COMB ? (int64_t)a.ctok * nrb : max_items;  // block ranges
  int nb = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
          &nb, gemv_gather_kernel<D, SB, MT, RBL, NB, RW, COMB, ROUTE>, 64 * kw, 0) != hipSuccess ||
      nb < 1)
    nb = 1;
  int dev = 0, cus = 256;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    cus = 256;
  const int64_t cap = (int64_t)nb * cus;
  const int grid = (int)(units < cap ? units : cap);
  gemv_gather_kernel<D, SB, MT, RBL, NB, RW, COMB, ROUTE><<<grid, 64 * kw, 0, st>>>(a);
  return jqh::launch_status();
}

// Rows in flight per lane: 4 rows of one projection, or 4 rows each of gate and up; rows of
// at most 16 (32) lane chunks take 4 (2) rows per wave instruction.
template <class D, int SB, int NB, int RW>
int launch_rw(GatherArgs& a, int mt, int64_t max_tiles, hipStream_t st) {
  constexpr int RBL = 4 * NB;
  if (a.rlogits) {
    if constexpr (NB == 2) return launch_g<D, SB, 1, RBL, NB, RW, false, true>(a, max_tiles, st);
    return JQ_ERR_SHAPE;
  }
  if (a.cout) {
    if constexpr (NB == 1) return launch_g<D, SB, 1, RBL, NB, RW, true>(a, max_tiles, st);
    return JQ_ERR_SHAPE;
  }
  if (mt == 1) return launch_g<D, SB, 1, RBL, NB, RW>(a, max_tiles, st);
  if (mt == 2) return launch_g<D, SB, 2, RBL, NB, RW>(a, max_tiles, st);
  if constexpr (D::BITS != 2) {
    if (mt == 4) return launch_g<D, SB, 4, RBL, NB, RW>(a, max_tiles, st);
  }
  return JQ_ERR_SHAPE;
}

template <class D, int SB, int NB>
int launch_mt(GatherArgs& a, int mt, int64_t max_tiles, hipStream_t st) {
  const int64_t C = a.p[0].K / (32 * units_per_chunk<D::BITS>());  // lane chunks per row
  if (C <= 16) return launch_rw<D, SB, NB, 4>(a, mt, max_tiles, st);
  if (C <= 32) return launch_rw<D, SB, NB, 2>(a, mt, max_tiles, st);
  return launch_rw<D, SB, NB, 1>(a, mt, max_tiles, st);
}

template <int BITS, int XDT, int NB>
int launch_sb(GatherArgs& a, int sb, int mt, int64_t max_tiles, hipStream_t st) {
  using D = Dc<BITS, 64, XDT>;  // the group size is a run-time argument of this kernel
  if (sb == JQ_BF16) return launch_mt<D, JQ_BF16, NB>(a, mt, max_tiles, st);
  return launch_mt<D, JQ_F16, NB>(a, mt, max_tiles, st);
}

template <int BITS, int NB>
int launch_x(GatherArgs& a, int xd, int sb, int mt, int64_t max_tiles, hipStream_t st) {
  if (xd == JQ_BF16) return launch_sb<BITS, JQ_BF16, NB>(a, sb, mt, max_tiles, st);
  return launch_sb<BITS, JQ_F16, NB>(a, sb, mt, max_tiles, st);
}

template <int NB>
int launch_bits(GatherArgs& a, int bits, int xd, int sb, int mt, int64_t max_tiles,
                hipStream_t st) {
  switch (bits) {
    case 2: return launch_x<2, NB>(a, xd, sb, mt, max_tiles, st);
    case 3: return launch_x<3, NB>(a, xd, sb, mt, max_tiles, st);
    case 4: return launch_x<4, NB>(a, xd, sb, mt, max_tiles, st);
    case 5: return launch_x<5, NB>(a, xd, sb, mt, max_tiles, st);
    case 6: return launch_x<6, NB>(a, xd, sb, mt, max_tiles, st);
    default: return launch_x<8, NB>(a, xd, sb, mt, max_tiles, st);
  }
}

}  // namespace

namespace jqk {

int gemv_gather_max_rows(int bits) { return bits == 2 ? 2 : 4; }

bool gemv_gather_ok(int64_t N, int64_t K, int bits, int gs, int xd, int sb) {
  if (xd != JQ_BF16 && xd != JQ_F16) return false;
  if (sb != JQ_BF16 && sb != JQ_F16) return false;
  if (gs != 32 && gs != 64 && gs != 128) return false;
  const int64_t chunk = bits == 2 ? 64 : 32;  // K of one lane chunk
  if (K <= 0 || K % chunk || gemv_waves(K, bits, nullptr) > kMaxWaves) return false;
  // Byte offsets inside an item's buffer views stay far below 2^31.
  return (N + 64) * (K / gs) * 2 < ((int64_t)1 << 31) && K * bits / 8 < ((int64_t)1 << 24);
}

int gemv_gather_launch(const QmmProblem& p, const QmmProblem* p2, const GatherPlan& plan,
                       int64_t max_tiles, int tile_rows, int bits, int gs, int xd, int sb,
                       int yd, hipStream_t st) {
  if (max_tiles == 0 || p.N == 0) return JQ_OK;
  if (!gemv_gather_ok(p.N, p.K, bits, gs, xd, sb) || tile_rows < 1 ||
      tile_rows > gemv_gather_max_rows(bits) || (tile_rows & (tile_rows - 1)))
    return JQ_ERR_SHAPE;
  GatherArgs a;
  a.p[0] = p;
  a.p[1] = p2 ? *p2 : p;
  a.plan = plan;
  a.ushift = gs == 32 ? 0 : gs == 64 ? 1 : 2;
  a.yd = yd;
  init_forms(a);
  if (p2) return launch_bits<2>(a, bits, xd, sb, tile_rows, max_tiles, st);
  return launch_bits<1>(a, bits, xd, sb, tile_rows, max_tiles, st);
}

bool gemv_gather_comb_ok(int64_t T, int k, int64_t N, int64_t K, int bits, int gs, int xd,
                         int sb) {
  // One wave per slot, each over a whole row: rows of at most 32 lane chunks, or rows that
  // take a single wave anyway.
  const int64_t C = K / (bits == 2 ? 64 : 32);
  return T > 0 && k > 0 && k <= kMaxCombSlots && gemv_gather_ok(N, K, bits, gs, xd, sb) &&
         (C <= 32 || gemv_waves(K, bits, nullptr) == 1) && T * k < ((int64_t)1 << 20);
}

int gemv_gather_comb_launch(const QmmProblem& p, const GatherPlan& plan, const MoeCombine& c,
                            int64_t T, int k, int bits, int gs, int xd, int sb, int yd,
                            hipStream_t st) {
  if (T == 0 || p.N == 0) return JQ_OK;
  if (!gemv_gather_comb_ok(T, k, p.N, p.K, bits, gs, xd, sb) || plan.tiles || plan.lhs ||
      plan.direct_rows != 1 || plan.direct_pairs != T * k || (!c.w && !c.before) || !c.out)
    return JQ_ERR_SHAPE;
  GatherArgs a;
  a.p[0] = a.p[1] = p;
  a.plan = plan;
  a.ushift = gs == 32 ? 0 : gs == 64 ? 1 : 2;
  a.yd = yd;
  init_forms(a);
  a.cw = c.w;
  a.cshared = c.shared;
  a.cgate = c.shared_gate;
  a.cout = c.out;
  a.cbefore = c.before;
  a.ck = k;
  a.ctok = (int)T;
  return launch_bits<1>(a, bits, xd, sb, 1, T * k, st);
}

bool gemv_gather_route_ok(int64_t E, int k) {
  return E >= 1 && E <= 64 * kRouteSlots && k >= 1 && k <= 64 && k <= E;
}

int gemv_gather_route_launch(const QmmProblem& g, const QmmProblem& u, const GatherPlan& plan,
                             const void* logits, int64_t E, int k, const jqr::RouteOpts& ro,
                             int before, uint32_t* idx, float* w, int64_t T, int bits, int gs,
                             int xd, int sb, int yd, hipStream_t st) {
  if (T == 0 || g.N == 0) return JQ_OK;
  if (!gemv_gather_route_ok(E, k) || !gemv_gather_ok(g.N, g.K, bits, gs, xd, sb) ||
      plan.tiles || plan.lhs || plan.direct_rows != 1 || plan.direct_pairs != T * k ||
      plan.pair_div != k || plan.E != E || !logits || !idx || !w)
    return JQ_ERR_SHAPE;
  GatherArgs a;
  a.p[0] = g;
  a.p[1] = u;
  a.plan = plan;
  a.ushift = gs == 32 ? 0 : gs == 64 ? 1 : 2;
  a.yd = yd;
  init_forms(a);
  a.rlogits = logits;
  a.ridx = idx;
  a.rw = w;
  a.rE = (int)E;
  a.rk = k;
  a.rbefore = before;
  a.ro = ro;
  return launch_bits<2>(a, bits, xd, sb, 1, T * k, st);
}

}  // namespace jqk

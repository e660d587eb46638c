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

#include "jq_gather_body.h"

namespace {

template <class D, int SB, int MT, int RBL, int NB, int RW, bool COMB = false, bool ROUTE = false>
__global__ void __launch_bounds__(64 * (COMB ? kMaxCombSlots : kMaxWaves))
gemv_gather_kernel(GatherArgs a) {
  gather_body<D, SB, MT, RBL, NB, RW, COMB, ROUTE>(a, (int)blockIdx.x, (int)gridDim.x);
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
  const int64_t cap =
      (int64_t)jqh::blocks_per_cu((const void*)gemv_gather_kernel<D, SB, MT, RBL, NB, RW, COMB, ROUTE>,
                                  64 * kw, 0) * jqh::cus();
  int64_t grid = units < cap ? units : cap;
  if constexpr (ROUTE) {  // whole tokens per block range: a multiple of the token count
    const int64_t T = max_tiles / a.rk;
    grid = (grid / T > 0 ? grid / T : 1) * T;
    if (grid >= ((int64_t)1 << 31)) return JQ_ERR_SHAPE;
  }
  gemv_gather_kernel<D, SB, MT, RBL, NB, RW, COMB, ROUTE><<<(unsigned)grid, 64 * kw, 0, st>>>(a);
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

// The group size is a run-time argument of this kernel; D::GS is 32 only for 2-bit codes in
// 32-code groups (a lane chunk's two units then hold two groups), 64 otherwise.
template <class D, int NB>
int launch_d(GatherArgs& a, int sb, int mt, int64_t max_tiles, hipStream_t st) {
  if (sb == JQ_BF16) return launch_mt<D, JQ_BF16, NB>(a, mt, max_tiles, st);
  return launch_mt<D, JQ_F16, NB>(a, mt, max_tiles, st);
}
template <int BITS, int XDT, int NB>
int launch_sb(GatherArgs& a, int sb, int mt, int64_t max_tiles, hipStream_t st) {
  if constexpr (BITS == 2)
    if (a.ushift == 0) return launch_d<Dc<2, 32, XDT>, NB>(a, sb, mt, max_tiles, st);
  return launch_d<Dc<BITS, 64, XDT>, NB>(a, sb, mt, max_tiles, st);
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

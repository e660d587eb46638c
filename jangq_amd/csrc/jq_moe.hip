// MoE path: router top-k, device-side grouping of (token, expert) pairs by expert, and the
// grouped gather_qmm / SwitchGLU launches.
//
// Caller side restated from the reference:
//   routing  softmax(logits, precise) -> top-k -> gather -> renorm
//            (jang-tools/jang_tools/qwen4_exp/modeling.py:587-593)
//   grouping mlx_lm _gather_sort / _scatter_unsort around gather_qmm(sorted_indices=True)
//            (jang-tools/jang_tools/dots3/ops.py:202-214, jangrt/switchglu_decode.py:161-183)
// Here the grouping never leaves the device and never changes values: every pair's output
// row is computed from its own activations and its expert's weights, whatever the order.
#include <math.h>

#include "jq_common.h"
#include "jq_gemv.h"
#include "jq_qmv.h"
#include "jq_route.h"

namespace {

using namespace jq;

// Rows per tile of the grouped kernels: 16 for the LDS-staged GEMM, 16/8/4 (gs 128/64/32)
// for the matrix-core decode kernel, 1/2/4 for the vector-ALU gather GEMV, which only runs
// up to kGemvRows plan rows. Workspaces are sized for the smallest tile they may get.
constexpr int kMinTileRows = 4;
constexpr int kGemmTileRows = 16;
constexpr int64_t kGemvRows = 4096;
constexpr int kMaxExperts = 4096;

// One wave per token (jqr::route_wave).
template <int SL>
__global__ void __launch_bounds__(256) route_kernel(const void* __restrict__ logits, int T, int E,
                                                    int k, jqr::RouteOpts o,
                                                    uint32_t* __restrict__ idx,
                                                    float* __restrict__ wout) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  uint32_t id;
  float w;
  const int esz = o.logit_dtype == JQ_F32 ? 4 : 2;
  jqr::route_wave<SL>((const char*)logits + (int64_t)t * E * esz, E, k, o, lane, id, w);
  if (lane < k) {
    idx[(int64_t)t * k + lane] = id;
    wout[(int64_t)t * k + lane] = w;
  }
}

JQ_DEV int block_exclusive_scan(int v, int* sh_wave, int& total) {
  // 1024 threads = 16 waves.
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int incl = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int n = __shfl_up(incl, o, 64);
    if (lane >= o) incl += n;
  }
  if (lane == 63) sh_wave[wave] = incl;
  __syncthreads();
  if (wave == 0) {
    int w = lane < 16 ? sh_wave[lane] : 0;
    int wi = w;
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) {
      const int n = __shfl_up(wi, o, 64);
      if (lane >= o) wi += n;
    }
    if (lane < 16) sh_wave[16 + lane] = wi - w;  // exclusive wave offsets
    if (lane == 15) sh_wave[32] = wi;
  }
  __syncthreads();
  total = sh_wave[32];
  const int r = sh_wave[16 + wave] + incl - v;
  __syncthreads();
  return r;
}

// Single block of 1024 threads. Builds, for the pair list rhs[n_pairs] over E experts:
//   seg_off[E+1]  exclusive offsets of each expert's segment in `order`
//   order         pair ids grouped by expert (order inside a segment is arbitrary: it does
//                 not change any value). Pairs whose expert id is >= E are left out.
//   tiles         (expert, first row, rows, segment offset) for every tile_rows-row tile of
//                 every segment (segment rows = count * M)
//   n_tiles[0]    number of tiles
__global__ void __launch_bounds__(1024) plan_kernel(const uint32_t* __restrict__ rhs, int n_pairs,
                                                    int E, int M, int tile_rows, int* seg_off,
                                                    uint32_t* order, int4* tiles, int* n_tiles) {
  __shared__ int cnt[kMaxExperts];
  __shared__ int cur[kMaxExperts];
  __shared__ int sh_wave[40];
  const int tid = threadIdx.x;
  for (int e = tid; e < E; e += 1024) cnt[e] = 0;
  __syncthreads();
  for (int i = tid; i < n_pairs; i += 1024) {
    const uint32_t e = rhs[i];
    if (e < (uint32_t)E) atomicAdd(&cnt[e], 1);
  }
  __syncthreads();
  // Each thread owns a contiguous run of ceil(E/1024) experts.
  const int per = (E + 1023) / 1024;
  const int e0 = tid * per;
  int local = 0, ltiles = 0;
  for (int e = e0; e < e0 + per && e < E; ++e) {
    local += cnt[e];
    ltiles += (cnt[e] * M + tile_rows - 1) / tile_rows;
  }
  int total;
  int base = block_exclusive_scan(local, sh_wave, total);
  int ttotal;
  int tbase = block_exclusive_scan(ltiles, sh_wave, ttotal);
  for (int e = e0; e < e0 + per && e < E; ++e) {
    seg_off[e] = base;
    cur[e] = base;
    const int rows = cnt[e] * M;
    for (int r = 0; r < rows; r += tile_rows) {
      tiles[tbase++] = make_int4(e, r, rows - r < tile_rows ? rows - r : tile_rows, base);
    }
    base += cnt[e];
  }
  if (tid == 0) {
    seg_off[E] = total;
    *n_tiles = ttotal;
  }
  __syncthreads();
  for (int i = tid; i < n_pairs; i += 1024) {
    const uint32_t e = rhs[i];
    if (e < (uint32_t)E) order[atomicAdd(&cur[e], 1)] = (uint32_t)i;
  }
}

struct WsLayout {
  int64_t seg_off, order, tiles, n_tiles, total;
};

inline int64_t align256(int64_t v) { return (v + 255) & ~(int64_t)255; }

inline int64_t max_tiles_for(int64_t n_pairs, int64_t E, int64_t M, int tile_rows) {
  const int64_t active = n_pairs < E ? n_pairs : E;
  return (n_pairs * M + tile_rows - 1) / tile_rows + active;
}

inline WsLayout ws_layout(int64_t n_pairs, int64_t E, int64_t M) {
  WsLayout L;
  int64_t o = 0;
  L.seg_off = o; o = align256(o + (E + 1) * 4);
  L.order = o; o = align256(o + n_pairs * 4);
  const int min_tile = n_pairs * M <= kGemvRows ? 1 : kMinTileRows;
  L.tiles = o; o = align256(o + max_tiles_for(n_pairs, E, M, min_tile) * 16);
  L.n_tiles = o; o = align256(o + 4);
  L.total = o;
  return L;
}

int build_plan(const uint32_t* rhs, int64_t n_pairs, int64_t E, int64_t M, int tile_rows,
               void* ws, jqk::GatherPlan& plan, const uint32_t* lhs, hipStream_t st) {
  const WsLayout L = ws_layout(n_pairs, E, M);
  char* base = (char*)ws;
  plan.seg_off = (const int*)(base + L.seg_off);
  plan.order = (const uint32_t*)(base + L.order);
  plan.tiles = (const int4*)(base + L.tiles);
  plan.n_tiles = (const int*)(base + L.n_tiles);
  plan.lhs = lhs;
  plan.M = (int)M;
  plan.pair_div = 1;
  plan.x_rows = 0;
  plan.rhs = rhs;
  plan.E = (int)E;
  plan.direct_pairs = 0;
  plan.direct_rows = 1;
  plan_kernel<<<1, 1024, 0, st>>>(rhs, (int)n_pairs, (int)E, (int)M, tile_rows,
                                  (int*)(base + L.seg_off),
                                  (uint32_t*)(base + L.order), (int4*)(base + L.tiles),
                                  (int*)(base + L.n_tiles));
  return jqh::launch_status();
}

// A plan without the plan kernel: every (one-row) pair is its own tile, read in pair order.
jqk::GatherPlan direct_plan(const uint32_t* rhs, int64_t n_pairs, int64_t E, const uint32_t* lhs) {
  jqk::GatherPlan plan;
  plan.order = nullptr;
  plan.seg_off = nullptr;
  plan.tiles = nullptr;
  plan.n_tiles = nullptr;
  plan.lhs = lhs;
  plan.M = 1;
  plan.pair_div = 1;
  plan.x_rows = 0;
  plan.rhs = rhs;
  plan.E = (int)E;
  plan.direct_pairs = (int)n_pairs;
  plan.direct_rows = 1;
  return plan;
}

// Kernel for a grouped problem of `rows` plan rows over the active experts.
//   gemv: few rows per active expert (decode); tiles of 1, 2 or 4 rows, as many as the average
//         rows per active expert, up to what the kernel holds in registers.
//   dmx:  several rows per active expert: matrix-core tiles of up to 16/(128/gs) rows with the
//         weights streamed through LDS (each expert's rows read once per tile).
//   dec:  up to two decode tiles per active expert on average (matrix cores, streaming).
//   gemm: larger problems, LDS-staged matrix-core GEMM with 16-row tiles.
enum class Kern { gemv, dmx, dec, gemm };

// The matrix-core tiles take a grouped problem from kDmxMinRows plan rows on, when the
// expected rows per selected expert (uniform routing) reach kDmxMinPerExpert. Measured on
// MI355X: 128 experts top-4 at 64 tokens (2.3 rows per expert) 334 vs 427 us per layer, 512
// experts top-10 with skewed routing at 32 tokens 252 vs 347 us; at 16 tokens (1.3 rows per
// expert, 64 rows) the one-row vector-ALU tiles stay faster (145 vs 166 us).
constexpr int64_t kDmxMinRows = 128;
constexpr double kDmxMinPerExpert = 1.25;

struct Choice {
  Kern k;
  int tile_rows;
};

// One projection per entry of bits/N/K (gate|up and down share a plan in SwitchGLU).
Choice choose(int64_t rows, int64_t E, int64_t n_pairs, int gs, int xd, int sb, int nproj,
              const int* bits, const int64_t* N, const int64_t* K) {
  const bool dt = (xd == JQ_BF16 || xd == JQ_F16) && (sb == JQ_BF16 || sb == JQ_F16);
  const int64_t active = n_pairs < E ? n_pairs : E;
  const int64_t avg = (rows + active - 1) / (active > 0 ? active : 1);
  // Distinct experts expected when n_pairs ids fall uniformly on E experts:
  // E (1 - (1 - 1/E)^n_pairs).
  const double expect = (double)E * -expm1((double)n_pairs * log1p(-1.0 / (double)E));
  const double per_expert = (double)rows / (expect > 1.0 ? expect : 1.0);
  if (dt && rows >= kDmxMinRows && per_expert >= kDmxMinPerExpert &&
      rows <= 2 * active * jqk::dmx_tokens_per_tile(gs)) {
    bool ok = true;
    for (int i = 0; i < nproj; ++i)
      ok = ok && jqk::dmx_gather_ok(N[i], K[i], bits[i], gs, xd, sb, nproj == 2 && i == 0 ? 2 : 1);
    if (ok) return {Kern::dmx, jqk::dmx_tokens_per_tile(gs)};
  }
  if (dt && rows <= kGemvRows) {
    bool ok = true;
    int maxr = 4;
    for (int i = 0; i < nproj; ++i) {
      ok = ok && jqk::gemv_gather_ok(N[i], K[i], bits[i], gs, xd, sb);
      const int m = jqk::gemv_gather_max_rows(bits[i]);
      maxr = m < maxr ? m : maxr;
    }
    if (ok && avg <= 2 * maxr) {
      const int tr = avg <= 1 ? 1 : avg <= 2 ? 2 : 4;
      return {Kern::gemv, tr < maxr ? tr : maxr};
    }
  }
  if (dt && rows <= 2 * active * jqk::dec_tokens_per_block(gs))
    return {Kern::dec, jqk::dec_tokens_per_block(gs)};
  return {Kern::gemm, kGemmTileRows};
}

int grouped_launch(const Choice& c, const jqk::QmmProblem& p, const jqk::QmmProblem* p2,
                   const jqk::GatherPlan& plan, int64_t mt, int bits, int gs, int xd, int sb,
                   int yd, hipStream_t st) {
  if (c.k == Kern::gemv)
    return jqk::gemv_gather_launch(p, p2, plan, mt, c.tile_rows, bits, gs, xd, sb, yd, st);
  if (c.k == Kern::dmx) return jqk::dmx_gather_launch(p, p2, plan, mt, bits, gs, xd, sb, yd, st);
  if (c.k == Kern::dec) return jqk::dec_gather_launch(p, p2, plan, mt, bits, gs, xd, sb, yd, st);
  return jqk::qmm_gather_launch(p, p2, plan, mt, bits, gs, xd, sb, yd, st);
}

int check_expert_shape(int bits, int gs, int64_t E, int64_t N, int64_t K) {
  int s = jqh::check_qshape(bits, gs, N, K);
  if (s) return s;
  if (E <= 0 || E > kMaxExperts) return JQ_ERR_SHAPE;
  return JQ_OK;
}

// The MoE combine (jqk::MoeCombine) of y [T, k, H] (slot outputs already rounded). One thread
// per two consecutive elements of a row (PAIR: 16-bit types, H even; one 32-bit load per slot)
// or per element; the slots summed in slot order in fp32 as before. With eight elements per
// thread (scalar 16-bit loads) config 5 at T = 32 ran 64 blocks for 14.1 us.
template <int DT, bool PAIR>
__global__ void __launch_bounds__(256) combine_kernel(const void* __restrict__ y,
                                                      jqk::MoeCombine c, int64_t T, int k,
                                                      int64_t H) {
  constexpr int VEC = PAIR ? 2 : 1;
  const int64_t per_row = H / VEC;
  const int64_t n = T * per_row;
  auto ld = [&](const void* p, int64_t e, float (&v)[VEC]) {
    if constexpr (PAIR) {
      const uint32_t w = ((const uint32_t*)p)[e >> 1];
      v[0] = DT == JQ_BF16 ? bf16_bits_to_f32(w & 0xFFFFu) : f16_bits_to_f32((uint16_t)w);
      v[1] = DT == JQ_BF16 ? bf16_bits_to_f32(w >> 16) : f16_bits_to_f32((uint16_t)(w >> 16));
    } else {
      v[0] = load_t<DT>(p, e);
    }
  };
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t t = i / per_row, col = (i - t * per_row) * VEC;
    float acc[VEC];
#pragma unroll
    for (int v = 0; v < VEC; ++v) acc[v] = 0.f;
    for (int j = 0; j < k; ++j) {
      const float wj = c.before ? 1.f : c.w[t * k + j];
      float yv[VEC];
      ld(y, (t * k + j) * H + col, yv);
#pragma unroll
      for (int v = 0; v < VEC; ++v) acc[v] = c.before ? acc[v] + yv[v] : fmaf(wj, yv[v], acc[v]);
    }
    const float gl = c.shared_gate ? load_t<DT>(c.shared_gate, t) : 0.f;
    float sh[VEC];
#pragma unroll
    for (int v = 0; v < VEC; ++v) sh[v] = 0.f;
    if (c.shared) ld(c.shared, t * H + col, sh);
#pragma unroll
    for (int v = 0; v < VEC; ++v)
      store_t<DT>(c.out, t * H + col + v,
                  jqk::moe_final(c.before, acc[v], c.shared != nullptr, sh[v],
                                 c.shared_gate != nullptr, gl, DT));
  }
}

// h = round(silu(g) * u) elementwise (g, u already rounded to the output dtype), with the
// optional clamp.
template <int DT>
__global__ void __launch_bounds__(256) swiglu_kernel(const void* __restrict__ g,
                                                     const void* __restrict__ u, int64_t n,
                                                     float limit, void* __restrict__ h) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    store_t<DT>(h, i, jqk::glu_value(load_t<DT>(g, i), load_t<DT>(u, i), limit, 1.f));
  }
}

inline unsigned grid_for(int64_t n) {
  const int64_t b = (n + 255) / 256;
  return (unsigned)(b < 8192 ? (b < 1 ? 1 : b) : 8192);
}

// Routing options from the C ABI (NULL: softmax with renormalisation, the qwen-style router).
int route_opts_of(const jq_route_opts* p, int64_t E, jqr::RouteOpts& o) {
  o = jqr::softmax_opts(1);
  if (!p) return JQ_OK;
  if (p->score < JQ_SCORE_SOFTMAX || p->score > JQ_SCORE_SQRTSOFTPLUS) return JQ_ERR_SHAPE;
  if (!(p->renorm_eps >= 0.f) || !isfinite(p->renorm_eps) || !isfinite(p->scaling))
    return JQ_ERR_SHAPE;
  const int ng = p->n_group < 1 ? 1 : p->n_group;
  if (ng > 1) {
    if (ng > 64 || E % ng || p->topk_group < 1 || p->topk_group > ng) return JQ_ERR_SHAPE;
  }
  o.score = p->score;
  o.renorm = p->renorm ? 1 : 0;
  o.eps = p->renorm_eps;
  o.scale = p->scaling;
  o.bias = p->score_bias;
  o.n_group = ng;
  o.topk_group = ng > 1 ? p->topk_group : 1;
  return JQ_OK;
}

jq_route_opts softmax_route_opts(int renorm) {
  jq_route_opts o;
  o.score = JQ_SCORE_SOFTMAX;
  o.renorm = renorm;
  o.renorm_eps = 0.f;
  o.scaling = 1.f;
  o.score_bias = nullptr;
  o.n_group = 1;
  o.topk_group = 1;
  return o;
}

}  // namespace

extern "C" {

static int combine_launch(const void* y, const jqk::MoeCombine& c, int64_t T, int k, int64_t H,
                          int dtype, hipStream_t st) {
  // (16-bit pairs need an even H and 4-byte aligned rows; the buffers are 16-byte aligned)
  const bool pair = dtype != JQ_F32 && H % 2 == 0;
  const int64_t n = T * (pair ? H / 2 : H);
  if (dtype == JQ_BF16) {
    if (pair) combine_kernel<JQ_BF16, true><<<grid_for(n), 256, 0, st>>>(y, c, T, k, H);
    else combine_kernel<JQ_BF16, false><<<grid_for(n), 256, 0, st>>>(y, c, T, k, H);
  } else if (dtype == JQ_F16) {
    if (pair) combine_kernel<JQ_F16, true><<<grid_for(n), 256, 0, st>>>(y, c, T, k, H);
    else combine_kernel<JQ_F16, false><<<grid_for(n), 256, 0, st>>>(y, c, T, k, H);
  } else {
    combine_kernel<JQ_F32, false><<<grid_for(n), 256, 0, st>>>(y, c, T, k, H);
  }
  return jqh::launch_status();
}

int jq_moe_combine(const void* y, const float* w, const void* shared, int64_t T, int k,
                   int64_t H, void* out, int dtype, jq_stream_t stream) {
  if (T < 0 || k <= 0 || H < 0) return JQ_ERR_SHAPE;
  if (!jqh::dtype_ok(dtype)) return JQ_ERR_DTYPE;
  if (T == 0 || H == 0) return JQ_OK;
  if (!y || !w || !out) return JQ_ERR_NULL;
  jqk::MoeCombine c;
  c.w = w;
  c.shared = shared;
  c.shared_gate = nullptr;
  c.out = out;
  c.before = 0;
  return combine_launch(y, c, T, k, H, dtype, (hipStream_t)stream);
}

static int swiglu_run(const void* x, int x_dtype, int64_t M, int64_t N, int64_t K,
                      const uint32_t* gate_codes, const void* gate_scales, const void* gate_biases,
                      const uint32_t* up_codes, const void* up_scales, const void* up_biases,
                      int sb_dtype, int bits, int group_size, void* h, void* up_buf, int y_dtype,
                      float limit, hipStream_t st) {
  int s = jqh::check_qshape(bits, group_size, N, K);
  if (s) return s;
  if (M < 0 || M > ((int64_t)1 << 30)) return JQ_ERR_SHAPE;
  if (!jqh::dtype_ok(x_dtype) || !jqh::dtype_ok(sb_dtype) || !jqh::dtype_ok(y_dtype))
    return JQ_ERR_DTYPE;
  if (!(limit >= 0.f)) return JQ_ERR_SHAPE;
  if (M == 0 || N == 0) return JQ_OK;
  if (!x || !gate_codes || !gate_scales || !gate_biases || !up_codes || !up_scales ||
      !up_biases || !h)
    return JQ_ERR_NULL;
  // One activation row: the whole-rows-per-wave GEMV with the SiLU * up epilogue.
  if (jqk::gemv_swiglu_ok((int)M, K, N, bits, group_size, x_dtype, sb_dtype, y_dtype)) {
    jqk::QmvBatch b;
    b.M = 1;
    b.K = (int)K;
    b.p[0].x = x; b.p[0].codes = gate_codes; b.p[0].scales = gate_scales;
    b.p[0].biases = gate_biases; b.p[0].y = h; b.p[0].N = N;
    b.p[1] = b.p[0];
    b.p[1].codes = up_codes; b.p[1].scales = up_scales; b.p[1].biases = up_biases;
    return jqk::gemv_swiglu_launch(b, bits, group_size, x_dtype, sb_dtype, y_dtype, limit, st);
  }
  // Decode sizes: one grouped launch of the expert-gathered GEMV over a single "expert" whose
  // tile holds all M rows, with the SiLU * up epilogue.
  const int maxr = jqk::gemv_gather_max_rows(bits);
  if (M <= maxr && (y_dtype == JQ_BF16 || y_dtype == JQ_F16) &&
      jqk::gemv_gather_ok(N, K, bits, group_size, x_dtype, sb_dtype)) {
    jqk::GatherPlan plan = direct_plan(nullptr, M, 1, nullptr);
    plan.direct_rows = (int)M;
    plan.x_rows = M;
    jqk::QmmProblem g, u;
    g.x = x; g.codes = gate_codes; g.scales = gate_scales; g.biases = gate_biases; g.y = h;
    g.M = 1; g.N = N; g.K = K;
    g.expert_stride_codes = 0;
    g.expert_stride_sb = 0;
    g.glu_limit = limit;
    u = g;
    u.codes = up_codes; u.scales = up_scales; u.biases = up_biases;
    const int tr = M <= 1 ? 1 : M <= 2 ? 2 : 4;
    return jqk::gemv_gather_launch(g, &u, plan, 1, tr, bits, group_size, x_dtype, sb_dtype,
                                   y_dtype, st);
  }
  // Decode batches of 5..64 rows on the matrix-core kernel: gate and up row blocks in one
  // launch with the SiLU * up epilogue (the rows the grouped dense launch would take), at
  // 8 bits or in passes of one activation block. At <= 6 bits with two-block passes the
  // grouped launch keeps its activation sums in registers, which the gate|up form cannot
  // without spilling: there the two launches are faster (3-bit 2 x 14336 x 4096 at 32 rows
  // 33.9 against 44.5 us).
  if (M >= 5 && M <= 64 && (bits > 6 || M <= jqk::dmx_tokens_per_tile(group_size)) &&
      jqk::dmx_ok((int)M, K, N, bits, group_size, x_dtype, sb_dtype, 1)) {
    jqk::QmvBatch b;
    b.M = (int)M;
    b.K = (int)K;
    b.p[0].x = x; b.p[0].codes = gate_codes; b.p[0].scales = gate_scales;
    b.p[0].biases = gate_biases; b.p[0].y = h; b.p[0].N = N;
    b.p[1] = b.p[0];
    b.p[1].codes = up_codes; b.p[1].scales = up_scales; b.p[1].biases = up_biases;
    b.p[1].y = nullptr;
    return jqk::dmx_glu_launch(b, bits, group_size, x_dtype, sb_dtype, y_dtype, limit, st);
  }
  // Otherwise: gate and up in one grouped dense launch, then the elementwise SiLU * up.
  if (!up_buf) return JQ_ERR_WORKSPACE;
  const void* xs[2] = {x, x};
  const uint32_t* cs[2] = {gate_codes, up_codes};
  const void* ss[2] = {gate_scales, up_scales};
  const void* bs[2] = {gate_biases, up_biases};
  const int bv[2] = {bits, bits}, gv[2] = {group_size, group_size};
  const int64_t Mv[2] = {M, M}, Nv[2] = {N, N}, Kv[2] = {K, K};
  void* ys[2] = {h, up_buf};
  s = jq_quantized_matmul_multi(2, xs, x_dtype, cs, ss, bs, sb_dtype, bv, gv, Mv, Nv, Kv, ys,
                                y_dtype, (jq_stream_t)st);
  if (s) return s;
  const int64_t n = M * N;
  if (y_dtype == JQ_BF16) swiglu_kernel<JQ_BF16><<<grid_for(n), 256, 0, st>>>(h, up_buf, n, limit, h);
  else if (y_dtype == JQ_F16) swiglu_kernel<JQ_F16><<<grid_for(n), 256, 0, st>>>(h, up_buf, n, limit, h);
  else swiglu_kernel<JQ_F32><<<grid_for(n), 256, 0, st>>>(h, up_buf, n, limit, h);
  return jqh::launch_status();
}

int jq_swiglu(const void* g, const void* u, int64_t n, float swiglu_limit, void* h, int dtype,
              jq_stream_t stream) {
  if (n < 0 || !(swiglu_limit >= 0.f)) return JQ_ERR_SHAPE;
  if (!jqh::dtype_ok(dtype)) return JQ_ERR_DTYPE;
  if (n == 0) return JQ_OK;
  if (!g || !u || !h) return JQ_ERR_NULL;
  hipStream_t st = (hipStream_t)stream;
  if (dtype == JQ_BF16) swiglu_kernel<JQ_BF16><<<grid_for(n), 256, 0, st>>>(g, u, n, swiglu_limit, h);
  else if (dtype == JQ_F16) swiglu_kernel<JQ_F16><<<grid_for(n), 256, 0, st>>>(g, u, n, swiglu_limit, h);
  else swiglu_kernel<JQ_F32><<<grid_for(n), 256, 0, st>>>(g, u, n, swiglu_limit, h);
  return jqh::launch_status();
}

int jq_quantized_swiglu(const void* x, int x_dtype, int64_t M, int64_t N, int64_t K,
                        const uint32_t* gate_codes, const void* gate_scales,
                        const void* gate_biases, const uint32_t* up_codes, const void* up_scales,
                        const void* up_biases, int sb_dtype, int bits, int group_size, void* h,
                        void* up_buf, int y_dtype, jq_stream_t stream) {
  return swiglu_run(x, x_dtype, M, N, K, gate_codes, gate_scales, gate_biases, up_codes,
                    up_scales, up_biases, sb_dtype, bits, group_size, h, up_buf, y_dtype, 0.f,
                    (hipStream_t)stream);
}

int jq_quantized_swiglu_ex(const void* x, int x_dtype, int64_t M, int64_t N, int64_t K,
                           const uint32_t* gate_codes, const void* gate_scales,
                           const void* gate_biases, const uint32_t* up_codes,
                           const void* up_scales, const void* up_biases, int sb_dtype, int bits,
                           int group_size, float swiglu_limit, void* h, void* up_buf,
                           int y_dtype, jq_stream_t stream) {
  return swiglu_run(x, x_dtype, M, N, K, gate_codes, gate_scales, gate_biases, up_codes,
                    up_scales, up_biases, sb_dtype, bits, group_size, h, up_buf, y_dtype,
                    swiglu_limit, (hipStream_t)stream);
}


int jq_moe_route_ex(const void* logits, int logits_dtype, int64_t T, int64_t E, int k,
                    const jq_route_opts* opts, uint32_t* idx, float* weights, jq_stream_t stream) {
  if (T < 0 || E <= 0 || E > kMaxExperts || k <= 0 || k > E || k > 64) return JQ_ERR_SHAPE;
  if (!jqh::dtype_ok(logits_dtype)) return JQ_ERR_DTYPE;
  jqr::RouteOpts o;
  int s = route_opts_of(opts, E, o);
  if (s) return s;
  o.logit_dtype = logits_dtype;
  if (T == 0) return JQ_OK;
  if (!logits || !idx || !weights) return JQ_ERR_NULL;
  const unsigned grid = (unsigned)((T + 3) / 4);
  hipStream_t st = (hipStream_t)stream;
  const int sl = (int)((E + 63) / 64);
#define JQ_R(SL) route_kernel<SL><<<grid, 256, 0, st>>>(logits, (int)T, (int)E, k, o, idx, weights)
  if (sl <= 1) JQ_R(1);
  else if (sl <= 2) JQ_R(2);
  else if (sl <= 4) JQ_R(4);
  else if (sl <= 8) JQ_R(8);
  else if (sl <= 16) JQ_R(16);
  else if (sl <= 32) JQ_R(32);
  else JQ_R(64);
#undef JQ_R
  return jqh::launch_status();
}

int jq_moe_route(const float* logits, int64_t T, int64_t E, int k, int renorm, uint32_t* idx,
                 float* weights, jq_stream_t stream) {
  const jq_route_opts o = softmax_route_opts(renorm);
  return jq_moe_route_ex(logits, JQ_F32, T, E, k, &o, idx, weights, stream);
}

int64_t jq_gather_workspace_size(int64_t n_pairs, int64_t E, int64_t M) {
  if (n_pairs < 0 || E <= 0 || M <= 0) return -1;
  return ws_layout(n_pairs, E, M).total;
}

int jq_gather_qmm(const void* x, int x_dtype, int64_t x_batch, int64_t M, const uint32_t* codes,
                  const void* scales, const void* biases, int sb_dtype, int bits, int group_size,
                  int64_t E, int64_t N, int64_t K, const uint32_t* lhs, const uint32_t* rhs,
                  int64_t n_pairs, int sorted_indices, void* out, int y_dtype, void* workspace,
                  int64_t workspace_bytes, jq_stream_t stream) {
  int s = check_expert_shape(bits, group_size, E, N, K);
  if (s) return s;
  if (x_dtype != JQ_BF16 && x_dtype != JQ_F16) return JQ_ERR_DTYPE;
  if (!jqh::dtype_ok(sb_dtype) || !jqh::dtype_ok(y_dtype)) return JQ_ERR_DTYPE;
  if (M <= 0 || x_batch < 0 || n_pairs < 0) return JQ_ERR_SHAPE;
  if (K % 128) return JQ_ERR_SHAPE;
  if (!lhs && x_batch < n_pairs) return JQ_ERR_SHAPE;
  if (n_pairs == 0 || N == 0) return JQ_OK;
  if (!x || !codes || !scales || !biases || !rhs || !out) return JQ_ERR_NULL;
  if (!workspace || workspace_bytes < ws_layout(n_pairs, E, M).total) return JQ_ERR_WORKSPACE;
  if (n_pairs * M > ((int64_t)1 << 30)) return JQ_ERR_SHAPE;
  hipStream_t st = (hipStream_t)stream;
  jqk::GatherPlan plan;
  (void)sorted_indices;  // grouping is done on the device in every case
  const int64_t Nv[1] = {N}, Kv[1] = {K};
  const Choice c = choose(n_pairs * M, E, n_pairs, group_size, x_dtype, sb_dtype, 1, &bits, Nv, Kv);
  // One row per tile on the vector-ALU kernel: the pairs are the tiles, no grouping needed.
  const bool direct = c.k == Kern::gemv && c.tile_rows == 1 && M == 1;
  if (direct) {
    plan = direct_plan(rhs, n_pairs, E, lhs);
  } else {
    s = build_plan(rhs, n_pairs, E, M, c.tile_rows, workspace, plan, lhs, st);
    if (s) return s;
  }
  plan.x_rows = x_batch * M;
  jqk::QmmProblem p;
  p.x = x;
  p.codes = codes;
  p.scales = scales;
  p.biases = biases;
  p.y = out;
  p.M = M;
  p.N = N;
  p.K = K;
  p.expert_stride_codes = N * (K * bits / 32);
  p.expert_stride_sb = N * (K / group_size);
  const int64_t mt = direct ? n_pairs : max_tiles_for(n_pairs, E, M, c.tile_rows);
  return grouped_launch(c, p, nullptr, plan, mt, bits, group_size, x_dtype, sb_dtype, y_dtype, st);
}

}  // extern "C"

namespace {

// One routed-expert call (jq_switch_glu, jq_switch_glu_combine, jq_moe_experts, jq_moe_block).
struct MoeRun {
  const void* x;
  int xd, yd, sb, gs, bits_gu, bits_d, k;
  int64_t T, H, I, E;
  const uint32_t* idx;  // [T, k] expert ids (written here when logits are given)
  const float* cw;      // [T, k] routing weights (likewise)
  const void* logits;   // [T, E] router logits (dtype ro.logit_dtype), or NULL (ids given)
  jqr::RouteOpts ro;
  const uint32_t *gc, *uc, *dc;
  const void *gsc, *gb, *usc, *ub, *dsc, *db;
  float limit;   // SwiGLU clamp
  int before;    // routing weights enter h before the down projection
  void* h_buf;   // [T*k, I]
  void* y_buf;   // [T*k, H] slot outputs (the jq_switch_glu output when comb.out is NULL)
  jqk::MoeCombine comb;  // comb.out NULL: no combine (jq_switch_glu)
  void* workspace;
  int64_t workspace_bytes;
  // shared expert inside the routed gate|up launch (jq_moe_block, one token): its
  // gate/up/down, intermediate size, h buffer and output
  const jq_qweight *sg, *su, *sd;
  int64_t sI;
  void* sh_h;
  void* sh_out;
};

int moe_run(MoeRun& r, hipStream_t st) {
  int s = check_expert_shape(r.bits_gu, r.gs, r.E, r.I, r.H);
  if (s) return s;
  s = check_expert_shape(r.bits_d, r.gs, r.E, r.H, r.I);
  if (s) return s;
  if (r.xd != JQ_BF16 && r.xd != JQ_F16) return JQ_ERR_DTYPE;
  if (!jqh::dtype_ok(r.sb) || (r.yd != JQ_BF16 && r.yd != JQ_F16)) return JQ_ERR_DTYPE;
  if (r.yd != r.xd) return JQ_ERR_DTYPE;  // h feeds the down projection as activations
  if (r.T < 0 || r.k <= 0) return JQ_ERR_SHAPE;
  if (r.H % 128 || r.I % 128) return JQ_ERR_SHAPE;
  if (!(r.limit >= 0.f)) return JQ_ERR_SHAPE;
  const int64_t n_pairs = r.T * r.k;
  if (n_pairs == 0) return JQ_OK;
  if (!r.x || !r.idx || !r.gc || !r.gsc || !r.gb || !r.uc || !r.usc || !r.ub || !r.dc ||
      !r.dsc || !r.db || !r.h_buf || !r.y_buf)
    return JQ_ERR_NULL;
  if (r.comb.out && !r.cw) return JQ_ERR_NULL;
  if (r.before && !r.cw) return JQ_ERR_NULL;
  if (!r.workspace || r.workspace_bytes < ws_layout(n_pairs, r.E, 1).total) return JQ_ERR_WORKSPACE;
  const int64_t T = r.T, H = r.H, I = r.I, E = r.E;
  const int k = r.k;
  // With logits, idx and cw are outputs: the routing of the T tokens.
  // Pair i = t*k + j uses x row t = i / k and expert idx[i]; one plan serves both launches
  // (gate+up reads x rows i / k, down reads h rows i).
  const int bv[2] = {r.bits_gu, r.bits_d};
  const int64_t Nv[2] = {I, H}, Kv[2] = {H, I};
  const Choice c = choose(n_pairs, E, n_pairs, r.gs, r.xd, r.sb, 2, bv, Nv, Kv);
  jqk::GatherPlan plan;
  const bool direct = c.k == Kern::gemv && c.tile_rows == 1;
  const bool comb_fused = r.comb.out && direct &&
                          jqk::gemv_gather_comb_ok(T, k, H, I, r.bits_d, r.gs, r.yd, r.sb);
  // Routing inside the gate|up launch: decode sizes with the combine fused into the down
  // launch, so that the three MoE launches after the router become two.
  const bool self_route = r.logits && comb_fused && jqk::gemv_gather_route_ok(E, k);
  if (r.logits && !self_route) {
    if (E > kMaxExperts || k > E || k > 64) return JQ_ERR_SHAPE;
    const int sl = (int)((E + 63) / 64);
    const unsigned grid = (unsigned)((T + 3) / 4);
#define JQ_R(SL) route_kernel<SL><<<grid, 256, 0, st>>>(r.logits, (int)T, (int)E, k, r.ro, (uint32_t*)r.idx, (float*)r.cw)
    if (sl <= 1) JQ_R(1);
    else if (sl <= 2) JQ_R(2);
    else if (sl <= 4) JQ_R(4);
    else if (sl <= 8) JQ_R(8);
    else if (sl <= 16) JQ_R(16);
    else if (sl <= 32) JQ_R(32);
    else JQ_R(64);
#undef JQ_R
    s = jqh::launch_status();
    if (s) return s;
  }
  if (direct) {
    plan = direct_plan(r.idx, n_pairs, E, nullptr);
  } else {
    s = build_plan(r.idx, n_pairs, E, 1, c.tile_rows, r.workspace, plan, nullptr, st);
    if (s) return s;
  }
  jqk::GatherPlan plan_gu = plan;
  plan_gu.lhs = nullptr;
  plan_gu.pair_div = k;  // x row = pair / k
  plan_gu.x_rows = T;
  plan.x_rows = n_pairs;  // down reads h rows = pairs
  jqk::QmmProblem g, u, d;
  g.x = r.x; g.codes = r.gc; g.scales = r.gsc; g.biases = r.gb; g.y = r.h_buf;
  g.M = 1; g.N = I; g.K = H;
  g.expert_stride_codes = I * (H * r.bits_gu / 32);
  g.expert_stride_sb = I * (H / r.gs);
  g.glu_limit = r.limit;
  // the pair weights enter h (weights before the down projection): from the routing output,
  // or from the registers of the launch that routes for itself
  g.glu_scale = r.before && !self_route ? r.cw : nullptr;
  u = g;
  u.codes = r.uc; u.scales = r.usc; u.biases = r.ub;
  const int64_t mt = direct ? n_pairs : max_tiles_for(n_pairs, E, 1, c.tile_rows);
  if (self_route)
    s = jqk::gemv_gather_route_launch(g, u, plan_gu, r.logits, E, k, r.ro, r.before,
                                      (uint32_t*)r.idx, (float*)r.cw, T, r.bits_gu, r.gs, r.xd,
                                      r.sb, r.yd, st);
  else
    s = grouped_launch(c, g, &u, plan_gu, mt, r.bits_gu, r.gs, r.xd, r.sb, r.yd, st);
  if (s) return s;
  d.x = r.h_buf; d.codes = r.dc; d.scales = r.dsc; d.biases = r.db; d.y = r.y_buf;
  d.M = 1; d.N = H; d.K = I;
  d.expert_stride_codes = H * (I * r.bits_d / 32);
  d.expert_stride_sb = H * (I / r.gs);
  jqk::MoeCombine cc = r.comb;
  cc.w = r.cw;
  if (comb_fused)
    return jqk::gemv_gather_comb_launch(d, plan, cc, T, k, r.bits_d, r.gs, r.yd, r.sb, r.yd, st);
  s = grouped_launch(c, d, nullptr, plan, mt, r.bits_d, r.gs, r.yd, r.sb, r.yd, st);
  if (s || !r.comb.out) return s;
  return combine_launch(r.y_buf, cc, T, k, H, r.yd, st);
}

MoeRun moe_args(const void* x, int x_dtype, int64_t T, int64_t H, int64_t I, int64_t E,
                       const uint32_t* idx, int k, const uint32_t* gate_codes,
                       const void* gate_scales, const void* gate_biases, const uint32_t* up_codes,
                       const void* up_scales, const void* up_biases, int bits_gu,
                       const uint32_t* down_codes, const void* down_scales,
                       const void* down_biases, int bits_d, int sb_dtype, int group_size,
                       void* h_buf, void* y_buf, int y_dtype, void* workspace,
                       int64_t workspace_bytes) {
  MoeRun r;
  r.x = x; r.xd = x_dtype; r.yd = y_dtype; r.sb = sb_dtype; r.gs = group_size;
  r.bits_gu = bits_gu; r.bits_d = bits_d; r.k = k;
  r.T = T; r.H = H; r.I = I; r.E = E;
  r.idx = idx; r.cw = nullptr; r.logits = nullptr; r.ro = jqr::softmax_opts(1);
  r.gc = gate_codes; r.gsc = gate_scales; r.gb = gate_biases;
  r.uc = up_codes; r.usc = up_scales; r.ub = up_biases;
  r.dc = down_codes; r.dsc = down_scales; r.db = down_biases;
  r.limit = 0.f; r.before = 0;
  r.h_buf = h_buf; r.y_buf = y_buf;
  r.comb.w = nullptr; r.comb.shared = nullptr; r.comb.shared_gate = nullptr;
  r.comb.out = nullptr; r.comb.before = 0;
  r.workspace = workspace; r.workspace_bytes = workspace_bytes;
  r.sg = r.su = r.sd = nullptr;
  r.sI = 0;
  r.sh_h = nullptr;
  r.sh_out = nullptr;
  return r;
}

// Whether one token's MoE block runs the shared expert's gate|up inside the routed gate|up
// launch (jq_moe_fused.h): bf16 throughout, routing in the gate|up launch, the combine in the
// down launch, and the instantiated widths (routed 2..4 bits, shared 4 or 8 bits). Measured on
// MI355X at config 5 (T = 1): one launch of 31.3 us against 24.5 + 10.4 us for the two. The
// shared down projection and the routed down-with-combine stay two launches: a single launch
// that joined them (the last wave of each row group finishing it) measured 23.0 us against
// 11.3 + 7.3 us, the routed half being latency-bound at one 16-wave block per CU.
bool fused_ok(const MoeRun& r) {
  if (r.T != 1 || r.sI <= 0 || !r.sg || !r.logits || !r.comb.out) return false;
  if (r.xd != JQ_BF16 || r.yd != JQ_BF16 || r.sb != JQ_BF16) return false;
  if (r.sg->sb_dtype != JQ_BF16 || r.su->sb_dtype != JQ_BF16) return false;
  auto lowbits = [](int b) { return b >= 2 && b <= 4; };
  if (!lowbits(r.bits_gu) || (r.sg->bits != 4 && r.sg->bits != 8)) return false;
  if (r.bits_gu == 2 && r.gs < 64) return false;  // (the fused launch has GS = 64 forms only)
  if (!jqk::gemv_gather_route_ok(r.E, r.k)) return false;
  if (!jqk::gemv_gather_ok(r.I, r.H, r.bits_gu, r.gs, r.xd, r.sb) ||
      jqk::fused_rw(r.H, r.bits_gu) > 2)
    return false;
  if (!jqk::gemv_gather_comb_ok(1, r.k, r.H, r.I, r.bits_d, r.gs, r.yd, r.sb)) return false;
  return jqk::gemv_swiglu_ok(1, r.H, r.sI, r.sg->bits, r.sg->group_size, r.xd, JQ_BF16, r.yd);
}

int moe_run_fused(MoeRun& r, hipStream_t st) {
  const int64_t H = r.H, I = r.I, E = r.E;
  const int k = r.k;
  jqk::GatherPlan plan = direct_plan(r.idx, k, E, nullptr);
  jqk::GatherPlan plan_gu = plan;
  plan_gu.pair_div = k;
  plan_gu.x_rows = 1;
  plan.x_rows = k;
  jqk::QmmProblem g, u, d;
  g.x = r.x; g.codes = r.gc; g.scales = r.gsc; g.biases = r.gb; g.y = r.h_buf;
  g.M = 1; g.N = I; g.K = H;
  g.expert_stride_codes = I * (H * r.bits_gu / 32);
  g.expert_stride_sb = I * (H / r.gs);
  g.glu_limit = r.limit;
  u = g;
  u.codes = r.uc; u.scales = r.usc; u.biases = r.ub;
  jqk::QmvProblem sg, su;
  sg.x = r.x; sg.codes = r.sg->codes; sg.scales = r.sg->scales; sg.biases = r.sg->biases;
  sg.y = r.sh_h; sg.N = r.sI;
  su = sg;
  su.codes = r.su->codes; su.scales = r.su->scales; su.biases = r.su->biases;
  int s = jqk::moe_fused_gu_launch(g, u, plan_gu, r.logits, E, k, r.ro, r.before,
                                   (uint32_t*)r.idx, (float*)r.cw, r.bits_gu, r.gs, sg, su,
                                   r.sg->bits, r.sg->group_size, r.limit, st);
  if (s) return s;
  // the shared expert's down projection, then the routed down with the combine
  s = jq_quantized_matmul(r.sh_h, r.xd, r.sd->codes, r.sd->scales, r.sd->biases,
                          r.sd->sb_dtype, r.sd->bits, r.sd->group_size, 1, H, r.sI, r.sh_out,
                          r.xd, (jq_stream_t)st);
  if (s) return s;
  d.x = r.h_buf; d.codes = r.dc; d.scales = r.dsc; d.biases = r.db; d.y = r.y_buf;
  d.M = 1; d.N = H; d.K = I;
  d.expert_stride_codes = H * (I * r.bits_d / 32);
  d.expert_stride_sb = H * (I / r.gs);
  jqk::MoeCombine c = r.comb;
  c.w = r.cw;
  c.shared = r.sh_out;
  return jqk::gemv_gather_comb_launch(d, plan, c, 1, k, r.bits_d, r.gs, r.yd, r.sb, r.yd, st);
}

// Workspace of jq_moe_block: the gather plan, then the routed h and slot outputs, then the
// shared expert's h, up scratch and output.
struct BlockWs {
  int64_t plan, h, y, sh_h, sh_up, sh_out, total;
};

BlockWs block_ws(int64_t T, int64_t H, int64_t I, int64_t E, int k, int64_t shared_I,
                        int esize) {
  BlockWs L;
  int64_t o = 0;
  L.plan = o; o = align256(o + ws_layout(T * k, E, 1).total);
  L.h = o; o = align256(o + T * k * I * esize);
  L.y = o; o = align256(o + T * k * H * esize);
  L.sh_h = o; o = align256(o + T * shared_I * esize);
  L.sh_up = o; o = align256(o + T * shared_I * esize);
  L.sh_out = o; o = align256(o + (shared_I > 0 ? T * H * esize : 0));
  L.total = o;
  return L;
}

bool qweight_ok(const jq_qweight* w) {
  return w && w->codes && w->scales && w->biases;
}

}  // namespace

extern "C" {

int jq_switch_glu(const void* x, int x_dtype, int64_t T, int64_t H, int64_t I, int64_t E,
                  const uint32_t* idx, int k, const uint32_t* gate_codes, const void* gate_scales,
                  const void* gate_biases, const uint32_t* up_codes, const void* up_scales,
                  const void* up_biases, int bits_gu, const uint32_t* down_codes,
                  const void* down_scales, const void* down_biases, int bits_d, int sb_dtype,
                  int group_size, void* h_buf, void* out, int y_dtype, void* workspace,
                  int64_t workspace_bytes, jq_stream_t stream) {
  MoeRun r = moe_args(x, x_dtype, T, H, I, E, idx, k, gate_codes, gate_scales, gate_biases,
                      up_codes, up_scales, up_biases, bits_gu, down_codes, down_scales,
                      down_biases, bits_d, sb_dtype, group_size, h_buf, out, y_dtype,
                      workspace, workspace_bytes);
  return moe_run(r, (hipStream_t)stream);
}

int jq_moe_experts(const void* x, int x_dtype, int64_t T, int64_t H, int64_t I, int64_t E,
                   const float* logits, int k, int renorm, uint32_t* idx, float* weights,
                   const uint32_t* gate_codes, const void* gate_scales, const void* gate_biases,
                   const uint32_t* up_codes, const void* up_scales, const void* up_biases,
                   int bits_gu, const uint32_t* down_codes, const void* down_scales,
                   const void* down_biases, int bits_d, int sb_dtype, int group_size,
                   void* h_buf, void* y_buf, const void* shared, void* out, int y_dtype,
                   void* workspace, int64_t workspace_bytes, jq_stream_t stream) {
  if (T > 0 && (!logits || !idx || !weights || !out)) return JQ_ERR_NULL;
  if (E <= 0 || E > kMaxExperts || k <= 0 || k > E || k > 64) return JQ_ERR_SHAPE;
  MoeRun r = moe_args(x, x_dtype, T, H, I, E, idx, k, gate_codes, gate_scales, gate_biases,
                      up_codes, up_scales, up_biases, bits_gu, down_codes, down_scales,
                      down_biases, bits_d, sb_dtype, group_size, h_buf, y_buf, y_dtype,
                      workspace, workspace_bytes);
  r.logits = logits;
  r.ro = jqr::softmax_opts(renorm);
  r.cw = weights;
  r.comb.shared = shared;
  r.comb.out = out;
  return moe_run(r, (hipStream_t)stream);
}

int jq_switch_glu_combine(const void* x, int x_dtype, int64_t T, int64_t H, int64_t I,
                          int64_t E, const uint32_t* idx, const float* weights, int k,
                          const uint32_t* gate_codes, const void* gate_scales,
                          const void* gate_biases, const uint32_t* up_codes,
                          const void* up_scales, const void* up_biases, int bits_gu,
                          const uint32_t* down_codes, const void* down_scales,
                          const void* down_biases, int bits_d, int sb_dtype, int group_size,
                          void* h_buf, void* y_buf, const void* shared, void* out, int y_dtype,
                          void* workspace, int64_t workspace_bytes, jq_stream_t stream) {
  if (T > 0 && (!weights || !out)) return JQ_ERR_NULL;
  MoeRun r = moe_args(x, x_dtype, T, H, I, E, idx, k, gate_codes, gate_scales, gate_biases,
                      up_codes, up_scales, up_biases, bits_gu, down_codes, down_scales,
                      down_biases, bits_d, sb_dtype, group_size, h_buf, y_buf, y_dtype,
                      workspace, workspace_bytes);
  r.cw = weights;
  r.comb.shared = shared;
  r.comb.out = out;
  return moe_run(r, (hipStream_t)stream);
}

int64_t jq_moe_block_workspace_size(int64_t T, int64_t H, int64_t I, int64_t E, int k,
                                    int64_t shared_I, int x_dtype) {
  if (T < 0 || H <= 0 || I <= 0 || E <= 0 || k <= 0 || shared_I < 0) return -1;
  if (x_dtype != JQ_BF16 && x_dtype != JQ_F16) return -1;
  return block_ws(T, H, I, E, k, shared_I, 2).total;
}

int jq_moe_block(const void* x, int x_dtype, int64_t T, int64_t H, int64_t I, int64_t E, int k,
                 const void* logits, int logits_dtype, const jq_route_opts* route,
                 const jq_qweight* gate,
                 const jq_qweight* up, const jq_qweight* down, int64_t shared_I,
                 const jq_qweight* shared_gate_proj, const jq_qweight* shared_up_proj,
                 const jq_qweight* shared_down_proj, const void* shared_gate_logits,
                 const jq_moe_opts* opts, uint32_t* idx, float* weights, void* out,
                 void* workspace, int64_t workspace_bytes, jq_stream_t stream) {
  if (x_dtype != JQ_BF16 && x_dtype != JQ_F16) return JQ_ERR_DTYPE;
  if (T < 0 || H <= 0 || I <= 0 || shared_I < 0) return JQ_ERR_SHAPE;
  if (E <= 0 || E > kMaxExperts || k <= 0 || k > E || k > 64) return JQ_ERR_SHAPE;
  if (!qweight_ok(gate) || !qweight_ok(up) || !qweight_ok(down)) return JQ_ERR_NULL;
  if (gate->bits != up->bits || gate->group_size != up->group_size ||
      down->group_size != gate->group_size)
    return JQ_ERR_GROUP_SIZE;
  const int before = opts ? opts->combine : JQ_COMBINE_AFTER_DOWN;
  const float limit = opts ? opts->swiglu_limit : 0.f;
  if (before != JQ_COMBINE_AFTER_DOWN && before != JQ_COMBINE_BEFORE_DOWN) return JQ_ERR_SHAPE;
  if (!(limit >= 0.f) || !isfinite(limit)) return JQ_ERR_SHAPE;
  if (before && shared_gate_logits) return JQ_ERR_SHAPE;  // the gated shared term is after-down only
  const bool has_shared = shared_I > 0;
  if (has_shared && (!qweight_ok(shared_gate_proj) || !qweight_ok(shared_up_proj) ||
                     !qweight_ok(shared_down_proj)))
    return JQ_ERR_NULL;
  if (has_shared && (shared_gate_proj->bits != shared_up_proj->bits ||
                     shared_gate_proj->group_size != shared_up_proj->group_size))
    return JQ_ERR_GROUP_SIZE;
  if (shared_gate_logits && !has_shared) return JQ_ERR_SHAPE;
  if (!jqh::dtype_ok(logits_dtype)) return JQ_ERR_DTYPE;
  jqr::RouteOpts ro;
  int s = route_opts_of(route, E, ro);
  if (s) return s;
  ro.logit_dtype = logits_dtype;
  if (T == 0) return JQ_OK;
  if (!x || !logits || !idx || !weights || !out) return JQ_ERR_NULL;
  const BlockWs L = block_ws(T, H, I, E, k, shared_I, 2);
  if (!workspace || workspace_bytes < L.total) return JQ_ERR_WORKSPACE;
  hipStream_t st = (hipStream_t)stream;
  char* ws = (char*)workspace;
  MoeRun r = moe_args(x, x_dtype, T, H, I, E, idx, k, gate->codes, gate->scales, gate->biases,
                      up->codes, up->scales, up->biases, gate->bits, down->codes, down->scales,
                      down->biases, down->bits, gate->sb_dtype, gate->group_size, ws + L.h,
                      ws + L.y, x_dtype, ws + L.plan, L.h - L.plan);
  if (up->sb_dtype != r.sb || down->sb_dtype != r.sb) return JQ_ERR_DTYPE;
  r.logits = logits;
  r.ro = ro;
  r.cw = weights;
  r.limit = limit;
  r.before = before;
  r.comb.shared_gate = shared_gate_logits;
  r.comb.out = out;
  r.comb.before = before;
  if (has_shared) {
    r.sg = shared_gate_proj;
    r.su = shared_up_proj;
    r.sd = shared_down_proj;
    r.sI = shared_I;
    r.sh_h = ws + L.sh_h;
    r.sh_out = ws + L.sh_out;
    // one token: the shared expert's gate|up runs inside the routed gate|up launch
    if (fused_ok(r)) {
      s = check_expert_shape(r.bits_gu, r.gs, E, I, H);
      if (s) return s;
      s = check_expert_shape(r.bits_d, r.gs, E, H, I);
      if (s) return s;
      if (H % 128 || I % 128) return JQ_ERR_SHAPE;
      return moe_run_fused(r, st);
    }
  }
  // Otherwise the shared expert first: its output joins the combine of the routed launch.
  void* sh_out = nullptr;
  if (has_shared) {
    const jq_qweight* sg = shared_gate_proj;
    const jq_qweight* su = shared_up_proj;
    const jq_qweight* sd = shared_down_proj;
    s = swiglu_run(x, x_dtype, T, shared_I, H, sg->codes, sg->scales, sg->biases, su->codes,
                   su->scales, su->biases, sg->sb_dtype, sg->bits, sg->group_size,
                   ws + L.sh_h, ws + L.sh_up, x_dtype, limit, st);
    if (s) return s;
    sh_out = ws + L.sh_out;
    s = jq_quantized_matmul(ws + L.sh_h, x_dtype, sd->codes, sd->scales, sd->biases,
                            sd->sb_dtype, sd->bits, sd->group_size, T, H, shared_I, sh_out,
                            x_dtype, stream);
    if (s) return s;
  }
  r.sg = r.su = r.sd = nullptr;
  r.sI = 0;
  r.comb.shared = sh_out;
  return moe_run(r, st);
}

}  // extern "C"

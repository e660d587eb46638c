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
__global__ void __launch_bounds__(256) route_kernel(const float* __restrict__ logits, int T, int E,
                                                    int k, int renorm, uint32_t* __restrict__ idx,
                                                    float* __restrict__ wout) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  uint32_t id;
  float w;
  jqr::route_wave<SL>(logits + (int64_t)t * E, E, k, renorm, lane, id, w);
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

// out[t, i] = round(sum_j w[t, j] * y[t, j, i]) (fp32, slot order), then round(+ shared[t, i]).
// One thread per 8 consecutive elements of a row (H % 8 == 0) or per element.
template <int DT, int VEC>
__global__ void __launch_bounds__(256) combine_kernel(const void* __restrict__ y,
                                                      const float* __restrict__ w,
                                                      const void* __restrict__ shared, int64_t T,
                                                      int k, int64_t H, void* __restrict__ out) {
  const int64_t per_row = H / VEC;
  const int64_t n = T * per_row;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t t = i / per_row, c = (i - t * per_row) * VEC;
    float acc[VEC];
#pragma unroll
    for (int v = 0; v < VEC; ++v) acc[v] = 0.f;
    for (int j = 0; j < k; ++j) {
      const float wj = w[t * k + j];
      const int64_t base = (t * k + j) * H + c;
#pragma unroll
      for (int v = 0; v < VEC; ++v) acc[v] = fmaf(wj, load_t<DT>(y, base + v), acc[v]);
    }
#pragma unroll
    for (int v = 0; v < VEC; ++v) {
      float r = acc[v];
      if constexpr (DT != JQ_F32) {
        r = DT == JQ_BF16 ? bf16_bits_to_f32(f32_to_bf16_bits(r))
                          : f16_bits_to_f32(f32_to_f16_bits(r));
      }
      if (shared) r += load_t<DT>(shared, t * H + c + v);
      store_t<DT>(out, t * H + c + v, r);
    }
  }
}

// h = round(silu(g) * u) elementwise (g, u already rounded to the output dtype).
template <int DT>
__global__ void __launch_bounds__(256) swiglu_kernel(const void* __restrict__ g,
                                                     const void* __restrict__ u, int64_t n,
                                                     void* __restrict__ h) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const float gv = load_t<DT>(g, i), uv = load_t<DT>(u, i);
    store_t<DT>(h, i, gv / (1.0f + expf(-gv)) * uv);
  }
}

inline unsigned grid_for(int64_t n) {
  const int64_t b = (n + 255) / 256;
  return (unsigned)(b < 8192 ? (b < 1 ? 1 : b) : 8192);
}

}  // namespace

extern "C" {

int jq_moe_combine(const void* y, const float* w, const void* shared, int64_t T, int k,
                   int64_t H, void* out, int dtype, jq_stream_t stream) {
  if (T < 0 || k <= 0 || H < 0) return JQ_ERR_SHAPE;
  if (!jqh::dtype_ok(dtype)) return JQ_ERR_DTYPE;
  if (T == 0 || H == 0) return JQ_OK;
  if (!y || !w || !out) return JQ_ERR_NULL;
  hipStream_t st = (hipStream_t)stream;
  const bool vec = H % 8 == 0;
  const int64_t n = T * (vec ? H / 8 : H);
#define JQ_C(DT)                                                                             \
  if (vec) combine_kernel<DT, 8><<<grid_for(n), 256, 0, st>>>(y, w, shared, T, k, H, out);  \
  else combine_kernel<DT, 1><<<grid_for(n), 256, 0, st>>>(y, w, shared, T, k, H, out);
  if (dtype == JQ_BF16) { JQ_C(JQ_BF16) }
  else if (dtype == JQ_F16) { JQ_C(JQ_F16) }
  else { JQ_C(JQ_F32) }
#undef JQ_C
  return jqh::launch_status();
}

int jq_quantized_swiglu(const void* x, int x_dtype, int64_t M, int64_t N, int64_t K,
                        const uint32_t* gate_codes, const void* gate_scales,
                        const void* gate_biases, const uint32_t* up_codes, const void* up_scales,
                        const void* up_biases, int sb_dtype, int bits, int group_size, void* h,
                        void* up_buf, int y_dtype, jq_stream_t stream) {
  int s = jqh::check_qshape(bits, group_size, N, K);
  if (s) return s;
  if (M < 0 || M > ((int64_t)1 << 30)) return JQ_ERR_SHAPE;
  if (!jqh::dtype_ok(x_dtype) || !jqh::dtype_ok(sb_dtype) || !jqh::dtype_ok(y_dtype))
    return JQ_ERR_DTYPE;
  if (M == 0 || N == 0) return JQ_OK;
  if (!x || !gate_codes || !gate_scales || !gate_biases || !up_codes || !up_scales ||
      !up_biases || !h)
    return JQ_ERR_NULL;
  hipStream_t st = (hipStream_t)stream;
  // One activation row: the whole-rows-per-wave GEMV with the SiLU * up epilogue.
  if (jqk::gemv_swiglu_ok((int)M, K, N, bits, group_size, x_dtype, sb_dtype, y_dtype)) {
    jqk::QmvBatch b;
    b.M = 1;
    b.K = (int)K;
    b.p[0].x = x; b.p[0].codes = gate_codes; b.p[0].scales = gate_scales;
    b.p[0].biases = gate_biases; b.p[0].y = h; b.p[0].N = N;
    b.p[1] = b.p[0];
    b.p[1].codes = up_codes; b.p[1].scales = up_scales; b.p[1].biases = up_biases;
    return jqk::gemv_swiglu_launch(b, bits, group_size, x_dtype, sb_dtype, y_dtype, st);
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
    u = g;
    u.codes = up_codes; u.scales = up_scales; u.biases = up_biases;
    const int tr = M <= 1 ? 1 : M <= 2 ? 2 : 4;
    return jqk::gemv_gather_launch(g, &u, plan, 1, tr, bits, group_size, x_dtype, sb_dtype,
                                   y_dtype, st);
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
                                y_dtype, stream);
  if (s) return s;
  const int64_t n = M * N;
  if (y_dtype == JQ_BF16) swiglu_kernel<JQ_BF16><<<grid_for(n), 256, 0, st>>>(h, up_buf, n, h);
  else if (y_dtype == JQ_F16) swiglu_kernel<JQ_F16><<<grid_for(n), 256, 0, st>>>(h, up_buf, n, h);
  else swiglu_kernel<JQ_F32><<<grid_for(n), 256, 0, st>>>(h, up_buf, n, h);
  return jqh::launch_status();
}


int jq_moe_route(const float* logits, int64_t T, int64_t E, int k, int renorm, uint32_t* idx,
                 float* weights, jq_stream_t stream) {
  if (T < 0 || E <= 0 || E > kMaxExperts || k <= 0 || k > E || k > 64) return JQ_ERR_SHAPE;
  if (T == 0) return JQ_OK;
  if (!logits || !idx || !weights) return JQ_ERR_NULL;
  const unsigned grid = (unsigned)((T + 3) / 4);
  hipStream_t st = (hipStream_t)stream;
  const int sl = (int)((E + 63) / 64);
#define JQ_R(SL) route_kernel<SL><<<grid, 256, 0, st>>>(logits, (int)T, (int)E, k, renorm, idx, weights)
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

// jq_switch_glu, and with comb_out != NULL the combine of jq_moe_combine fused into the down
// launch where the direct decode form applies (else out is written and combined after).
static int switch_glu_run(const void* x, int x_dtype, int64_t T, int64_t H, int64_t I,
                          int64_t E, const uint32_t* idx, int k, const uint32_t* gate_codes,
                          const void* gate_scales, const void* gate_biases,
                          const uint32_t* up_codes, const void* up_scales, const void* up_biases,
                          int bits_gu, const uint32_t* down_codes, const void* down_scales,
                          const void* down_biases, int bits_d, int sb_dtype, int group_size,
                          void* h_buf, void* out, int y_dtype, void* workspace,
                          int64_t workspace_bytes, const float* cw, const void* cshared,
                          void* comb_out, hipStream_t st, const float* rlogits = nullptr,
                          int renorm = 1) {
  int s = check_expert_shape(bits_gu, group_size, E, I, H);
  if (s) return s;
  s = check_expert_shape(bits_d, group_size, E, H, I);
  if (s) return s;
  if (x_dtype != JQ_BF16 && x_dtype != JQ_F16) return JQ_ERR_DTYPE;
  if (!jqh::dtype_ok(sb_dtype) || (y_dtype != JQ_BF16 && y_dtype != JQ_F16)) return JQ_ERR_DTYPE;
  if (y_dtype != x_dtype) return JQ_ERR_DTYPE;  // h feeds the down projection as activations
  if (T < 0 || k <= 0) return JQ_ERR_SHAPE;
  if (H % 128 || I % 128) return JQ_ERR_SHAPE;
  const int64_t n_pairs = T * k;
  if (n_pairs == 0) return JQ_OK;
  if (!x || !idx || !gate_codes || !gate_scales || !gate_biases || !up_codes || !up_scales ||
      !up_biases || !down_codes || !down_scales || !down_biases || !h_buf || !out)
    return JQ_ERR_NULL;
  if (comb_out && !cw) return JQ_ERR_NULL;
  if (!workspace || workspace_bytes < ws_layout(n_pairs, E, 1).total) return JQ_ERR_WORKSPACE;
  // With logits, idx and cw are outputs: the routing of the T tokens.
  // Pair i = t*k + j uses x row t = i / k and expert idx[i]; one plan serves both launches
  // (gate+up reads x rows i / k, down reads h rows i).
  const int bv[2] = {bits_gu, bits_d};
  const int64_t Nv[2] = {I, H}, Kv[2] = {H, I};
  const Choice c = choose(n_pairs, E, n_pairs, group_size, x_dtype, sb_dtype, 2, bv, Nv, Kv);
  jqk::GatherPlan plan;
  const bool direct = c.k == Kern::gemv && c.tile_rows == 1;
  // Routing inside the gate|up launch: decode sizes with the combine fused into the down
  // launch, so that the three MoE launches after the router become two.
  const bool self_route = rlogits && direct && comb_out && jqk::gemv_gather_route_ok(E, k) &&
                          jqk::gemv_gather_comb_ok(T, k, H, I, bits_d, group_size, y_dtype, sb_dtype);
  if (rlogits && !self_route) {
    s = jq_moe_route(rlogits, T, E, k, renorm, (uint32_t*)idx, (float*)cw, (jq_stream_t)st);
    if (s) return s;
  }
  if (direct) {
    plan = direct_plan(idx, n_pairs, E, nullptr);
  } else {
    s = build_plan(idx, n_pairs, E, 1, c.tile_rows, workspace, plan, nullptr, st);
    if (s) return s;
  }
  jqk::GatherPlan plan_gu = plan;
  plan_gu.lhs = nullptr;
  plan_gu.pair_div = k;  // x row = pair / k
  plan_gu.x_rows = T;
  plan.x_rows = n_pairs;  // down reads h rows = pairs
  jqk::QmmProblem g, u, d;
  g.x = x; g.codes = gate_codes; g.scales = gate_scales; g.biases = gate_biases; g.y = h_buf;
  g.M = 1; g.N = I; g.K = H;
  g.expert_stride_codes = I * (H * bits_gu / 32);
  g.expert_stride_sb = I * (H / group_size);
  u = g;
  u.codes = up_codes; u.scales = up_scales; u.biases = up_biases;
  const int64_t mt = direct ? n_pairs : max_tiles_for(n_pairs, E, 1, c.tile_rows);
  if (self_route)
    s = jqk::gemv_gather_route_launch(g, u, plan_gu, rlogits, E, k, renorm, (uint32_t*)idx,
                                      (float*)cw, T, bits_gu, group_size, x_dtype, sb_dtype,
                                      y_dtype, st);
  else
    s = grouped_launch(c, g, &u, plan_gu, mt, bits_gu, group_size, x_dtype, sb_dtype, y_dtype, st);
  if (s) return s;
  d.x = h_buf; d.codes = down_codes; d.scales = down_scales; d.biases = down_biases; d.y = out;
  d.M = 1; d.N = H; d.K = I;
  d.expert_stride_codes = H * (I * bits_d / 32);
  d.expert_stride_sb = H * (I / group_size);
  if (comb_out && direct &&
      jqk::gemv_gather_comb_ok(T, k, H, I, bits_d, group_size, y_dtype, sb_dtype))
    return jqk::gemv_gather_comb_launch(d, plan, cw, cshared, comb_out, T, k, bits_d,
                                        group_size, y_dtype, sb_dtype, y_dtype, st);
  s = grouped_launch(c, d, nullptr, plan, mt, bits_d, group_size, y_dtype, sb_dtype, y_dtype, st);
  if (s || !comb_out) return s;
  return jq_moe_combine(out, cw, cshared, T, k, H, comb_out, y_dtype, (jq_stream_t)st);
}

int jq_switch_glu(const void* x, int x_dtype, int64_t T, int64_t H, int64_t I, int64_t E,
                  const uint32_t* idx, int k, const uint32_t* gate_codes, const void* gate_scales,
                  const void* gate_biases, const uint32_t* up_codes, const void* up_scales,
                  const void* up_biases, int bits_gu, const uint32_t* down_codes,
                  const void* down_scales, const void* down_biases, int bits_d, int sb_dtype,
                  int group_size, void* h_buf, void* out, int y_dtype, void* workspace,
                  int64_t workspace_bytes, jq_stream_t stream) {
  return switch_glu_run(x, x_dtype, T, H, I, E, idx, k, gate_codes, gate_scales, gate_biases,
                        up_codes, up_scales, up_biases, bits_gu, down_codes, down_scales,
                        down_biases, bits_d, sb_dtype, group_size, h_buf, out, y_dtype,
                        workspace, workspace_bytes, nullptr, nullptr, nullptr,
                        (hipStream_t)stream);
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
  return switch_glu_run(x, x_dtype, T, H, I, E, idx, k, gate_codes, gate_scales, gate_biases,
                        up_codes, up_scales, up_biases, bits_gu, down_codes, down_scales,
                        down_biases, bits_d, sb_dtype, group_size, h_buf, y_buf, y_dtype,
                        workspace, workspace_bytes, weights, shared, out, (hipStream_t)stream,
                        logits, renorm);
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
  return switch_glu_run(x, x_dtype, T, H, I, E, idx, k, gate_codes, gate_scales, gate_biases,
                        up_codes, up_scales, up_biases, bits_gu, down_codes, down_scales,
                        down_biases, bits_d, sb_dtype, group_size, h_buf, y_buf, y_dtype,
                        workspace, workspace_bytes, weights, shared, out, (hipStream_t)stream);
}

}  // extern "C"

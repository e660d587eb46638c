// Internal launch descriptors shared by the matmul translation units (not part of the ABI).
#pragma once

#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "jq_common.h"

namespace jqr {

enum { kSoftmax = 0, kSigmoid = 1, kSqrtSoftplus = 2 };

// Device copy of the routing options (jq_route_opts of the C ABI): scores, selection bias,
// group-limited selection, renormalisation and scaling (jq_route.h).
struct RouteOpts {
  int score;          // kSoftmax / kSigmoid / kSqrtSoftplus
  int renorm;         // divide the k weights by (their sum + eps)
  float eps;
  float scale;        // routed scaling factor, applied last
  const float* bias;  // [E] selection bias or NULL
  int n_group, topk_group;
  int logit_dtype;    // JQ_F32 / JQ_BF16 / JQ_F16 logits
};

inline __host__ __device__ RouteOpts softmax_opts(int renorm) {
  RouteOpts o;
  o.score = kSoftmax;
  o.renorm = renorm;
  o.eps = 0.f;
  o.scale = 1.f;
  o.bias = nullptr;
  o.n_group = 1;
  o.topk_group = 1;
  o.logit_dtype = 0;
  return o;
}

}  // namespace jqr

namespace jqk {

constexpr int kMaxProblems = 8;

struct QmvProblem {
  const void* x;          // [M, K]
  const uint32_t* codes;  // [N, K*bits/32]
  const void* scales;     // [N, K/gs]
  const void* biases;     // [N, K/gs]
  void* y;                // [M, N]
  int64_t N;
};

struct QmvBatch {
  QmvProblem p[kMaxProblems];
  int M;
  int K;
};

// Decode GEMV (VALU) for M <= 4, any K % 32 == 0. Returns a jq_status.
int qmv_launch(const QmvBatch& b, int nprob, int bits, int gs, int xd, int sb, int yd,
               hipStream_t st);

// Decode GEMV on the vector ALUs (jq_gemv.hip): M <= 4, bf16/f16 activations and scales.
// SwiGLU pair at one activation row (b.p[0] gate, b.p[1] up, same x and N): whole rows per
// wave, h = silu(round(g)) * round(u) written to b.p[0].y (bf16/f16).
bool gemv_swiglu_ok(int M, int64_t K, int64_t N, int bits, int gs, int xd, int sb, int yd);
int gemv_swiglu_launch(const QmvBatch& b, int bits, int gs, int xd, int sb, int yd, float limit,
                       hipStream_t st);
bool gemv_ok(int M, int64_t K, int64_t maxN, int bits, int gs, int xd, int sb);
int gemv_launch(const QmvBatch& b, int nprob, int bits, int gs, int xd, int sb, int yd,
                hipStream_t st);

// Prefill GEMM on the matrix cores (jq_gemm.hip): gs 64/128, bf16/f16 activations
// (8-bit codes only with f16 activations).
bool gemm_ok(int64_t M, int64_t K, int bits, int gs, int xd, int sb);

// Row-gathered operand description for the grouped (MoE) matrix-core launches.
// Pairs are processed in expert-grouped order `order`; A row r of segment e is
//   pair p = order[seg_off[e] + r / M], token row m = r % M
//   ->  x row (lhs ? lhs[p] : p / pair_div)*M + m
// and its output goes to out row p*M + m.
struct GatherPlan {
  const uint32_t* order;     // [n_pairs] pair ids grouped by expert
  const int* seg_off;        // [E + 1] segment offsets into order
  const int4* tiles;         // [max_tiles] (expert, first row, rows, seg_off[expert])
  const int* n_tiles;        // [1] number of valid tiles
  const uint32_t* lhs;       // [n_pairs] or NULL
  int M;                     // rows per pair
  int pair_div;              // without lhs: x row of pair p is p / pair_div
  int64_t x_rows;            // rows of x; a pair mapping outside reads zeros
  // Direct tiles (tiles == NULL; vector-ALU gather GEMV only, M == 1): tile t holds pairs
  // [t*direct_rows, t*direct_rows + direct_rows) of expert rhs[t*direct_rows] (expert 0 when
  // rhs is NULL; with rhs, direct_rows is 1); an id >= E reads nothing and is not stored.
  const uint32_t* rhs;
  int E;
  int direct_pairs;
  int direct_rows;
};

struct QmmProblem {
  const void* x;
  const uint32_t* codes;
  const void* scales;
  const void* biases;
  void* y;
  int64_t M, N, K;
  int64_t expert_stride_codes;  // words between experts (gather mode)
  int64_t expert_stride_sb;     // elements between experts' scale rows (gather mode)
  // SwiGLU pair (gate problem of a gate|up launch): with glu_limit > 0 the rounded gate is
  // clamped to <= L and the rounded up to [-L, L]; with glu_scale, h = silu(g) * u is
  // multiplied by glu_scale[output row] before its rounding (routing weights applied before
  // the down projection).
  float glu_limit = 0.f;
  const float* glu_scale = nullptr;
};

// h = silu(g) * u of a SwiGLU pair whose g and u are already rounded to the output dtype:
// the optional clamp (jang-tools/jang_tools/dsv41/model.py:1214-1218: up = clip(up, -L, L),
// gate = min(gate, L)) and the optional per-row factor (the routing weight, model.py:1219-1222).
// h is rounded to fp32 here (the empty asm makes it an opaque register value): a caller that
// rounds h to f16 at a compile-time dtype would otherwise get the last product and the f16
// rounding fused into one v_fma_mix (one rounding instead of two), and outputs an f16 ulp
// away from the same h computed in a kernel whose output dtype is a run-time value.
JQ_DEV float glu_value(float g, float u, float limit, float factor) {
  if (limit > 0.f) {
    g = fminf(g, limit);
    u = fminf(fmaxf(u, -limit), limit);
  }
  float h = g / (1.0f + expf(-g)) * u;
  if (factor != 1.f) h *= factor;
  asm("" : "+v"(h));
  return h;
}

// Decode batches on matrix cores with LDS-streamed weights (jq_dmx.hip): M <= 2*16/(128/gs),
// gs 64/128, scales of the activation dtype, K % 256 == 0 and K <= 4096 (or K = 1024..2048
// in 2-step waves), the ring within the LDS budget (rt: 16-row tiles per item).
bool dmx_ok(int M, int64_t K, int64_t maxN, int bits, int gs, int xd, int sb, int rt);
int dmx_tokens_per_tile(int gs);
int dmx_launch(const QmvBatch& b, int nprob, int bits, int gs, int xd, int sb, int yd,
               hipStream_t st);
// Gate (b.p[0]) and up (b.p[1]) of one shape over the same activations in one launch:
// b.p[0].y = silu(round(g)) * round(u), rounded (glu_value with `limit`); same limits as
// dmx_ok with rt = 1.
int dmx_glu_launch(const QmvBatch& b, int bits, int gs, int xd, int sb, int yd, float limit,
                   hipStream_t st);
// Expert-gathered form: plan tiles (plan.tiles != NULL) of up to dmx_tokens_per_tile rows;
// with p2, gate (p) and up (p2) rows of each tile give h = silu(g) * u.
bool dmx_gather_ok(int64_t N, int64_t K, int bits, int gs, int xd, int sb, int nb);
// Long rows (K > 4096) of one problem: K split into chunks over the items, fp32 partials in a
// workspace (the returned size, 0 when the split does not apply), then one summing launch.
int64_t dmx_split_workspace(int M, int64_t K, int64_t N, int bits, int gs, int xd, int sb);
int dmx_split_launch(const QmvBatch& b, int bits, int gs, int xd, int sb, int yd, void* ws,
                     int64_t ws_bytes, hipStream_t st);
int dmx_gather_launch(const QmmProblem& p, const QmmProblem* p2, const GatherPlan& plan,
                      int64_t max_tiles, int bits, int gs, int xd, int sb, int yd,
                      hipStream_t st);

// Matrix-core GEMM y = x @ deq(W)^T. K % 128 == 0 required. Returns a jq_status.
int qmm_launch(const QmmProblem& p, int bits, int gs, int xd, int sb, int yd, hipStream_t st);
int gemm_launch(const QmmProblem& p, int bits, int gs, int xd, int sb, int yd, hipStream_t st);

// Prefill GEMM on the f16 matrix cores (jq_gemm16.hip): gs 64/128, bf16/f16 activations, every
// width. Its workspace holds the f16 activation rows of a pass; a smaller one (at least 256
// rows' worth) runs the rows in passes.
bool gemm16_ok(int64_t M, int64_t K, int bits, int gs, int xd, int sb);
int64_t gemm16_workspace(int64_t rows, int64_t N, int64_t K, int gs);
int gemm16_launch(const QmmProblem& p, int bits, int gs, int xd, int sb, int yd, void* ws,
                  int64_t ws_bytes, hipStream_t st);

// Grouped matrix-core GEMM over expert segments described by `plan` (device data). With
// p2 != NULL, p is the gate and p2 the up projection (same shapes) and the output is
// silu(gate) * up (the SwitchGLU activation).
int qmm_gather_launch(const QmmProblem& p, const QmmProblem* p2, const GatherPlan& plan,
                      int64_t max_tiles, int bits, int gs, int xd, int sb, int yd,
                      hipStream_t st);

// Decode-shaped matrix-core kernels (jq_dec.hip): activation rows per MFMA block for a
// group size, eligibility of a dense problem, dense and grouped launches.
int dec_tokens_per_block(int gs);
bool dec_dense_ok(int M, int64_t K, int gs, int xd, int sb);
int dec_dense_launch(const QmvBatch& b, int nprob, int bits, int gs, int xd, int sb, int yd,
                     hipStream_t st);
int dec_gather_launch(const QmmProblem& p, const QmmProblem* p2, const GatherPlan& plan,
                      int64_t max_tiles, int bits, int gs, int xd, int sb, int yd,
                      hipStream_t st);

// Decode GEMV on 4x4x4 matrix-core blocks (jq_qmv4.hip): passes of up to 8 activation rows,
// K % 32 == 0, bf16/f16 activations and scales.
bool qmv4_ok(int M, int64_t K, int64_t maxN, int bits, int gs, int xd, int sb);
int qmv4_launch(const QmvBatch& b, int nprob, int bits, int gs, int xd, int sb, int yd,
                hipStream_t st);

// Persistent decode-batch matrix-core kernel (jq_decp.hip): any M (passes of up to
// 2 * 16/(128/gs) activation rows), K % 128 == 0, bf16/f16 activations and scales.
bool decp_ok(int M, int64_t K, int64_t maxN, int xd, int sb);
int decp_launch(const QmvBatch& b, int nprob, int bits, int gs, int xd, int sb, int yd,
                hipStream_t st);

// Expert-gathered decode GEMV on the vector ALUs (jq_gemv_gather.hip): plan tiles of
// tile_rows (1, 2 or 4, at most gemv_gather_max_rows) rows; p2 as for qmm_gather_launch.
int gemv_gather_max_rows(int bits);
bool gemv_gather_ok(int64_t N, int64_t K, int bits, int gs, int xd, int sb);
int gemv_gather_launch(const QmmProblem& p, const QmmProblem* p2, const GatherPlan& plan,
                       int64_t max_tiles, int tile_rows, int bits, int gs, int xd, int sb,
                       int yd, hipStream_t st);
// The MoE combine of a token's k slot outputs y_j (each rounded to the output dtype), the
// shared expert's output and its optional sigmoid gate:
//   after the down projection (before = 0): r = round(sum_j w_j * y_j)   (fp32, slot order)
//     shared term  s' = round(round(sigmoid(gate)) * s)  with a gate, else s;  out = r + s'
//   before it (before = 1, the weights were applied to h):  out = (sum_j y_j) + s
// out is rounded by its store. Follows jang-tools/jang_tools/qwen4_exp/modeling.py:594-599
// and jang-tools/jang_tools/dsv41/model.py:1219-1245 (and the down dispatch of
// dsv41/metal_decode.py:395-420).
struct MoeCombine {
  const float* w;           // [T, k] routing weights (after-down form)
  const void* shared;       // [T, N] shared expert output, or NULL
  const void* shared_gate;  // [T] logits of the shared term's gate, or NULL
  void* out;                // [T, N]
  int before;
};

JQ_DEV float round_to_dtype(float v, int yd) {
  if (yd == 1) return __uint_as_float((uint32_t)jq::f32_to_bf16_bits(v) << 16);
  if (yd == 2) return jq::f16_bits_to_f32(jq::f32_to_f16_bits(v));
  return v;
}

// acc: fp32 slot-order sum (weighted in the after-down form).
JQ_DEV float moe_final(int before, float acc, bool has_shared, float sh, bool has_gate, float gl,
                       int yd) {
  if (before) return has_shared ? acc + sh : acc;
  const float r = round_to_dtype(acc, yd);
  if (!has_shared) return r;
  if (has_gate) {
    float p = round_to_dtype(1.0f / (1.0f + expf(-gl)), yd) * sh;
    asm("" : "+v"(p));  // an fp32 product, then its rounding (as in glu_value)
    sh = round_to_dtype(p, yd);
  }
  return r + sh;
}

// The same GEMV over a direct plan of T * k pairs (pair t*k + j reads x row t*k + j) with the
// MoE combine fused in (MoeCombine, slot order in fp32); an expert id outside [0, E)
// contributes 0. One wave per slot (k <= 16), each over whole rows: K of at most 32 lane
// chunks or of a single wave.
bool gemv_gather_comb_ok(int64_t T, int k, int64_t N, int64_t K, int bits, int gs, int xd,
                         int sb);
int gemv_gather_comb_launch(const QmmProblem& p, const GatherPlan& plan, const MoeCombine& c,
                            int64_t T, int k, int bits, int gs, int xd, int sb, int yd,
                            hipStream_t st);
// The gate|up launch over a direct plan of T * k pairs (x row = pair / k) that routes for
// itself: pair t*k + j takes the j-th expert of the token's top-k (jqr::route_wave, E <= 512),
// and the token's ids and weights are written to idx / w [T, k] as jq_moe_route_ex writes
// them; with before, h of each pair is multiplied by its weight.
bool gemv_gather_route_ok(int64_t E, int k);
int gemv_gather_route_launch(const QmmProblem& g, const QmmProblem& u, const GatherPlan& plan,
                             const void* logits, int64_t E, int k, const jqr::RouteOpts& ro,
                             int before, uint32_t* idx, float* w, int64_t T, int bits, int gs,
                             int xd, int sb, int yd, hipStream_t st);

// The gate|up launch of one token's MoE block with the shared expert inside (jq_moe_fused.h):
// the routed gate|up pairs of a launch that routes for itself and the shared expert's gate|up
// rows (sg, su: [Is, H]) in one grid. bf16 activations and scales; routed bits 2..4 on rows of
// at least 32 lane chunks, shared bits 4 or 8 on rows of at most two waves of chunks.
// fused_rw: rows per wave instruction of a gathered projection with K inputs.
int fused_rw(int64_t K, int bits);
int moe_fused_gu_launch(const QmmProblem& g, const QmmProblem& u, const GatherPlan& plan,
                        const void* logits, int64_t E, int k, const jqr::RouteOpts& ro,
                        int before, uint32_t* idx, float* w, int bits_r, int gs_r,
                        const QmvProblem& sg, const QmvProblem& su, int bits_s, int gs_s,
                        float limit, hipStream_t st);


}  // namespace jqk

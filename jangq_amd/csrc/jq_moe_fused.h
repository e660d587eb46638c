// The gate|up launch of one token's MoE block with the shared expert inside: blocks [0, nA)
// run the routed gate|up pairs, each wave routing for itself (gather_body, routed form);
// blocks [nA, grid) run the shared expert's gate|up rows (gemv_row_body, SwiGLU form), every
// wave on its own. The two halves stream their weights side by side, so the shared expert's
// rows keep the memory system busy while the routed waves compute their top-k; the grid is
// split between them in proportion to their bytes. (The reference's two-dispatch fused decode
// puts the shared expert into the routed gate|up dispatch as slot TOPK the same way,
// jang-tools/jang_tools/dsv41/metal_decode.py:334-371.)
#pragma once

#include "jq_gather_body.h"
#include "jq_gemv_row.h"

namespace {

struct FusedGuArgs {
  GatherArgs g;  // routed gate|up (routed form)
  GemvArgs s;    // shared gate|up (SwiGLU form)
  int nA;        // routed blocks
};

template <class DR, int RW, class DS, int CPLS>
__global__ void __launch_bounds__(64 * jqg::kMaxWaves) moe_gu_fused_kernel(FusedGuArgs a) {
  if ((int)blockIdx.x < a.nA) {
    gather_body<DR, JQ_BF16, 1, 4, 2, RW, false, true>(a.g, (int)blockIdx.x, a.nA);
  } else {
    const int wpb = (int)(blockDim.x >> 6);
    const int w = __builtin_amdgcn_readfirstlane(((int)blockIdx.x - a.nA) * wpb +
                                                 (int)(threadIdx.x >> 6));
    gemv_row_body<DS, JQ_BF16, CPLS, 2, true>(a.s, w, ((int)gridDim.x - a.nA) * wpb, RowStore());
  }
}

// Split `cap` resident blocks between the routed half (itemsA items, bytesA bytes) and the
// shared half (wavesB waves of work at wpb waves per block, bytesB bytes).
inline void split_grid(int64_t cap, int64_t itemsA, double bytesA, int64_t wavesB, int wpb,
                       double bytesB, int& nA, int& nB) {
  const double fa = bytesA / (bytesA + bytesB);
  int64_t a = (int64_t)(cap * fa + 0.5);
  a = a < 1 ? 1 : a;
  a = a > itemsA ? itemsA : a;
  const int64_t needB = (wavesB + wpb - 1) / wpb;
  int64_t b = cap - a;
  b = b < 1 ? 1 : b;
  b = b > needB ? needB : b;
  nA = (int)a;
  nB = (int)b;
}

// Row blocks of a one-problem row GEMV (RB rows each; GLU: rows of the pair).
inline void row_args(GemvArgs& s, const jqk::QmvProblem& p0, const jqk::QmvProblem* p1, int K,
                     int gs, int yd, float limit, int RB, bool glu) {
  s.b.M = 1;
  s.b.K = K;
  s.b.p[0] = p0;
  s.b.p[1] = p1 ? *p1 : p0;
  s.nprob = glu ? 2 : 1;
  s.ushift = gs == 32 ? 0 : gs == 64 ? 1 : 2;
  s.kwshift = 0;
  s.yd = yd;
  s.glu_limit = limit;
  const int total = glu ? (int)p0.N : (int)((p0.N + RB - 1) / RB);
  s.rb_begin[0] = 0;
  for (int i = 1; i <= jqk::kMaxProblems; ++i) s.rb_begin[i] = total;
}

}  // namespace

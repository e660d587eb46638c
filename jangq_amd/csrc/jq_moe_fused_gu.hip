// The gate|up launch of one token's MoE block with the shared expert inside (jq_moe_fused.h).
#include "jq_moe_fused.h"

namespace {

template <class DR, int RW, class DS, int CPLS>
int gu_launch(FusedGuArgs& a, int kwR, int64_t itemsA, double bytesA, int64_t wavesB,
              double bytesB, hipStream_t st) {
  const int threads = 64 * kwR;
  const int64_t cap =
      (int64_t)jqh::blocks_per_cu((const void*)moe_gu_fused_kernel<DR, RW, DS, CPLS>, threads, 0) *
      jqh::cus();
  int nA = 0, nB = 0;
  split_grid(cap, itemsA, bytesA, wavesB, kwR, bytesB, nA, nB);
  a.nA = nA;
  moe_gu_fused_kernel<DR, RW, DS, CPLS><<<nA + nB, threads, 0, st>>>(a);
  return jqh::launch_status();
}

template <class DR, int RW>
int gu_shared(FusedGuArgs& a, int bits_s, int cpls, int kwR, int64_t itemsA, double bytesA,
              int64_t wavesB, double bytesB, hipStream_t st) {
#define JQ_GU(BS, C)                                                                       \
  if (bits_s == BS && cpls == C)                                                           \
    return gu_launch<DR, RW, typename RowD<jqd::Dc<BS, 64, JQ_BF16>>::type, C>(            \
        a, kwR, itemsA, bytesA, wavesB, bytesB, st);
  JQ_GU(8, 2) JQ_GU(8, 1) JQ_GU(4, 2) JQ_GU(4, 1)
#undef JQ_GU
  return JQ_ERR_SHAPE;
}

}  // namespace

namespace jqk {

// Routed row width (rows per wave instruction) of a gathered projection with K inputs.
int fused_rw(int64_t K, int bits) {
  const int64_t C = K / (bits == 2 ? 64 : 32);
  return C <= 16 ? 4 : C <= 32 ? 2 : 1;
}

int moe_fused_gu_launch(const QmmProblem& g, const QmmProblem& u, const GatherPlan& plan,
                        const void* logits, int64_t E, int k, const jqr::RouteOpts& ro,
                        int before, uint32_t* idx, float* w, int bits_r, int gs_r,
                        const QmvProblem& sg, const QmvProblem& su, int bits_s, int gs_s,
                        float limit, hipStream_t st) {
  const int64_t H = g.K, I = g.N, Is = sg.N;
  const int rw = fused_rw(H, bits_r);
  int kws = 0;
  const int kwR = rw == 1 ? jqg::gemv_waves(H, bits_r, &kws) : 1;
  const int cpls = row_cpl(H, bits_s);
  // (2-bit routed codes in 32-code groups would need the GS = 32 instantiation)
  if (rw > 2 || kwR > jqg::kMaxWaves || cpls > 2 || (bits_r == 2 && gs_r < 64) ||
      (((JQ_ROW_UPL2 >> bits_s) & 1) && gs_s < 64))
    return JQ_ERR_SHAPE;
  FusedGuArgs a;
  GatherArgs& ga = a.g;
  ga.p[0] = g;
  ga.p[1] = u;
  ga.plan = plan;
  ga.ushift = gs_r == 32 ? 0 : gs_r == 64 ? 1 : 2;
  ga.kwshift = kws;
  ga.yd = JQ_BF16;
  init_forms(ga);
  ga.rlogits = logits;
  ga.ridx = idx;
  ga.rw = w;
  ga.rE = (int)E;
  ga.rk = k;
  ga.rbefore = before;
  ga.ro = ro;
  const int rows = 2 * rw;  // rows of one projection per item (4 ring rows of gate and up)
  ga.nrb = (int)((I + rows - 1) / rows);
  row_args(a.s, sg, &su, (int)H, gs_s, JQ_BF16, limit, 2, true);
  const int64_t itemsA = (int64_t)k * ga.nrb;
  // The routed half's bytes weigh 1.5x in the grid split: its waves first run the top-k and
  // look up their experts. Measured at config 5 (T = 1): weights 1.0 / 1.2 / 1.4-1.6 / 1.8 of
  // the bytes gave the layer 44.1 / 42.9 / 42.3 / 44.8 us.
  const double bytesA = 1.5 * 2.0 * k * I * (H * bits_r / 8 + H / gs_r * 4);
  const double bytesB = 2.0 * Is * (H * bits_s / 8 + H / gs_s * 4);
#define JQ_R(BR, RW)                                                                          \
  if (bits_r == BR && rw == RW)                                                               \
    return gu_shared<jqd::Dc<BR, 64, JQ_BF16>, RW>(a, bits_s, cpls, kwR, itemsA, bytesA, Is,  \
                                                   bytesB, st);
  JQ_R(2, 1) JQ_R(2, 2) JQ_R(3, 1) JQ_R(3, 2) JQ_R(4, 1) JQ_R(4, 2)
#undef JQ_R
  return JQ_ERR_SHAPE;
}

}  // namespace jqk

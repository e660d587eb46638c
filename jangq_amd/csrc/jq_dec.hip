// Decode-shaped quantized matmuls on matrix cores: dense (one or several problems sharing
// activations) and expert-grouped (MoE gather / fused gate|up + SwiGLU). See jq_dec.h.
//
// Block = KW waves over RT 16-row tiles of W; wave w covers the w-th 1/KW of K's 128-code
// steps for all RT tiles, and the block sums the partials in LDS. Grid: one block per
// (row-tile group, problem) for dense launches; a persistent loop over (expert tile,
// row-tile group) items for grouped launches.
#include "jq_dec.h"
#include "jq_qmv.h"

namespace {

using namespace jq;
using namespace jqd;
using jqk::GatherPlan;
using jqk::QmmProblem;
using jqk::QmvBatch;

JQ_DEV void store_out(void* y, int64_t idx, float v, int yd) {
  if (yd == JQ_BF16) ((uint16_t*)y)[idx] = f32_to_bf16_bits(v);
  else if (yd == JQ_F16) ((uint16_t*)y)[idx] = f32_to_f16_bits(v);
  else ((float*)y)[idx] = v;
}

JQ_DEV float round_to(float v, int yd) {
  if (yd == JQ_BF16) return bf16_bits_to_f32(f32_to_bf16_bits(v));
  if (yd == JQ_F16) return f16_bits_to_f32(f32_to_f16_bits(v));
  return v;
}

// A row m' = l%16 of the MFMA block feeds token t = m' / GSTEP from the lane groups of
// group m' % GSTEP.
template <class D>
JQ_DEV bool a_active(int lr, int lg, int rows) {
  const int t = lr / D::GSTEP, j = lr % D::GSTEP;
  return t < rows && j == lg / D::LPG;
}

template <class D, int SB, int RT, int KW>
__global__ void __launch_bounds__(64 * KW) dec_dense_kernel(QmvBatch batch, int yd) {
  __shared__ float red[(KW > 1 ? KW - 1 : 1) * RT * 4 * 64];
  const auto& pb = batch.p[blockIdx.y];
  const int64_t N = pb.N;
  const int64_t nb = (int64_t)blockIdx.x * 16 * RT;
  if (nb >= N) return;
  const int K = batch.K, M = batch.M;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  const int lr = lane & 15, lg = lane >> 4;
  const int S = K / 128;
  const int s0 = (S * wave) / KW, s1 = (S * (wave + 1)) / KW;
  const int64_t P = (int64_t)K * D::BITS / 32, G = K / D::GS;
  TileRows rows[1][RT];
#pragma unroll
  for (int r = 0; r < RT; ++r) {
    int64_t row = nb + 16 * r + lr;
    row = row < N ? row : N - 1;  // rows past N compute junk that is never stored
    rows[0][r].c = pb.codes + row * P;
    rows[0][r].s = (const uint16_t*)pb.scales + row * G;
    rows[0][r].b = (const uint16_t*)pb.biases + row * G;
  }
  const bool act = a_active<D>(lr, lg, M);
  const int t = lr / D::GSTEP;
  const uint16_t* xr = (const uint16_t*)pb.x + (int64_t)(act ? t : 0) * K;
  f32x4 acc[1][RT];
#pragma unroll
  for (int r = 0; r < RT; ++r) acc[0][r] = f32x4{0.f, 0.f, 0.f, 0.f};
  dec_tile<D, SB, 1, RT>(xr, act, rows, s0, s1, lg, acc);
  block_reduce<KW, RT>(&acc[0][0], red);
  if (wave == 0) {
    constexpr int TPL = 4 / D::GSTEP;
#pragma unroll
    for (int r = 0; r < RT; ++r) {
      const int64_t n = nb + 16 * r + lr;
      if (n < N) {
        float v[TPL];
        fold_groups<D>(acc[0][r], v);
#pragma unroll
        for (int k = 0; k < TPL; ++k) {
          const int tok = TPL * lg + k;
          if (tok < M) store_out(pb.y, (int64_t)tok * N + n, v[k], yd);
        }
      }
    }
  }
}

// Grouped over expert tiles of <= TPB rows; NB == 2 computes gate (p) and up (p2) and
// writes silu(gate) * up.
template <class D, int SB, int NB, int KW>
__global__ void __launch_bounds__(64 * KW) dec_gather_kernel(QmmProblem p, QmmProblem p2,
                                                             GatherPlan plan, int yd) {
  __shared__ float red[(KW > 1 ? KW - 1 : 1) * NB * 4 * 64];
  const int64_t N = p.N;
  const int K = (int)p.K;
  const int64_t nrt = (N + 15) / 16;
  const int64_t items = (int64_t)(*plan.n_tiles) * nrt;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  const int lr = lane & 15, lg = lane >> 4;
  const int S = K / 128;
  const int s0 = (S * wave) / KW, s1 = (S * (wave + 1)) / KW;
  const int64_t P = (int64_t)K * D::BITS / 32, G = K / D::GS;
  const int Mp = plan.M;
  for (int64_t item = blockIdx.x; item < items; item += gridDim.x) {
    const int4 tile = plan.tiles[item / nrt];
    const int e = tile.x, r0 = tile.y, nrows = tile.z;
    const int seg = plan.seg_off[e];
    const int64_t n0 = (item % nrt) * 16;
    const int64_t row = n0 + lr < N ? n0 + lr : N - 1;
    TileRows rows[NB][1];
    rows[0][0].c = p.codes + e * p.expert_stride_codes + row * P;
    rows[0][0].s = (const uint16_t*)p.scales + e * p.expert_stride_sb + row * G;
    rows[0][0].b = (const uint16_t*)p.biases + e * p.expert_stride_sb + row * G;
    if constexpr (NB == 2) {
      rows[1][0].c = p2.codes + e * p.expert_stride_codes + row * P;
      rows[1][0].s = (const uint16_t*)p2.scales + e * p.expert_stride_sb + row * G;
      rows[1][0].b = (const uint16_t*)p2.biases + e * p.expert_stride_sb + row * G;
    }
    bool act = a_active<D>(lr, lg, nrows);
    int64_t xrow = 0;
    if (act) {
      const int rr = r0 + lr / D::GSTEP;
      const uint32_t pair = plan.order[seg + rr / Mp];
      xrow = (int64_t)(plan.lhs ? plan.lhs[pair] : pair / plan.pair_div) * Mp + rr % Mp;
      if (xrow >= plan.x_rows) {
        act = false;
        xrow = 0;
      }
    }
    const uint16_t* xr = (const uint16_t*)p.x + xrow * K;
    f32x4 acc[NB][1];
#pragma unroll
    for (int q = 0; q < NB; ++q) acc[q][0] = f32x4{0.f, 0.f, 0.f, 0.f};
    dec_tile<D, SB, NB, 1>(xr, act, rows, s0, s1, lg, acc);
    block_reduce<KW, NB>(&acc[0][0], red);
    if (wave == 0 && n0 + lr < N) {
      constexpr int TPL = 4 / D::GSTEP;
      float v[TPL], u[TPL];
      fold_groups<D>(acc[0][0], v);
      if constexpr (NB == 2) fold_groups<D>(acc[NB - 1][0], u);
#pragma unroll
      for (int k = 0; k < TPL; ++k) {
        const int tok = TPL * lg + k;
        if (tok < nrows) {
          const int rr = r0 + tok;
          const uint32_t pair = plan.order[seg + rr / Mp];
          const int64_t orow = (int64_t)pair * Mp + rr % Mp;
          float val = v[k];
          if constexpr (NB == 2) {
            const float g = round_to(v[k], yd), up = round_to(u[k], yd);
            val = jqk::glu_value(g, up, p.glu_limit, p.glu_scale ? p.glu_scale[orow] : 1.f);
          }
          store_out(p.y, orow * N + n0 + lr, val, yd);
        }
      }
    }
    __syncthreads();  // red is reused by the next item
  }
}

// Launch shape: enough waves to fill 256 CUs several times over, enough steps per wave to
// amortise the block reduction. RT = 2 row tiles per wave for tall problems; K is split
// across KW = 8 waves when there are few row tiles.
template <int BITS, int GS, int XDT, int SB>
int dense_t(const QmvBatch& b, int nprob, int64_t maxN, int yd, hipStream_t st) {
  using D = Dc<BITS, GS, XDT>;
  int64_t rows_total = 0;
  for (int i = 0; i < nprob; ++i) rows_total += b.p[i].N;
  const int64_t tiles = (rows_total + 15) / 16;
  const int S = b.K / 128;
  if (tiles >= 2048 && S >= 16) {
    dim3 grid((unsigned)((maxN + 31) / 32), (unsigned)nprob);
    dec_dense_kernel<D, SB, 2, 4><<<grid, 256, 0, st>>>(b, yd);
  } else if (tiles < 1024 && S >= 16) {
    dim3 grid((unsigned)((maxN + 15) / 16), (unsigned)nprob);
    dec_dense_kernel<D, SB, 1, 8><<<grid, 512, 0, st>>>(b, yd);
  } else {
    dim3 grid((unsigned)((maxN + 15) / 16), (unsigned)nprob);
    dec_dense_kernel<D, SB, 1, 4><<<grid, 256, 0, st>>>(b, yd);
  }
  return jqh::launch_status();
}

template <int BITS, int GS, int XDT, int SB, int NB>
int gather_t(const QmmProblem& p, const QmmProblem& p2, const GatherPlan& plan, int64_t max_tiles,
             int yd, hipStream_t st) {
  using D = Dc<BITS, GS, XDT>;
  const int64_t items = max_tiles * ((p.N + 15) / 16);
  const int64_t grid = items < 4096 ? (items < 1 ? 1 : items) : 4096;
  dec_gather_kernel<D, SB, NB, 4><<<(unsigned)grid, 256, 0, st>>>(p, p2, plan, yd);
  return jqh::launch_status();
}

template <int XDT, int SB>
int dense_bits(int bits, int gs, const QmvBatch& b, int nprob, int64_t maxN, int yd,
               hipStream_t st) {
#define JQ_D(B)                                                          \
  switch (gs) {                                                          \
    case 32: return dense_t<B, 32, XDT, SB>(b, nprob, maxN, yd, st);     \
    case 64: return dense_t<B, 64, XDT, SB>(b, nprob, maxN, yd, st);     \
    default: return dense_t<B, 128, XDT, SB>(b, nprob, maxN, yd, st);    \
  }
  switch (bits) {
    case 2: JQ_D(2)
    case 3: JQ_D(3)
    case 4: JQ_D(4)
    case 5: JQ_D(5)
    case 6: JQ_D(6)
    default: JQ_D(8)
  }
#undef JQ_D
}

template <int XDT, int SB, int NB>
int gather_bits(int bits, int gs, const QmmProblem& p, const QmmProblem& p2,
                const GatherPlan& plan, int64_t mt, int yd, hipStream_t st) {
#define JQ_G(B)                                                                     \
  switch (gs) {                                                                     \
    case 32: return gather_t<B, 32, XDT, SB, NB>(p, p2, plan, mt, yd, st);          \
    case 64: return gather_t<B, 64, XDT, SB, NB>(p, p2, plan, mt, yd, st);          \
    default: return gather_t<B, 128, XDT, SB, NB>(p, p2, plan, mt, yd, st);         \
  }
  switch (bits) {
    case 2: JQ_G(2)
    case 3: JQ_G(3)
    case 4: JQ_G(4)
    case 5: JQ_G(5)
    case 6: JQ_G(6)
    default: JQ_G(8)
  }
#undef JQ_G
}

}  // namespace

namespace jqk {

int dec_tokens_per_block(int gs) { return 16 / (128 / gs); }

bool dec_dense_ok(int M, int64_t K, int gs, int xd, int sb) {
  return M >= 1 && M <= dec_tokens_per_block(gs) && K % 128 == 0 && K > 0 &&
         (xd == JQ_BF16 || xd == JQ_F16) && (sb == JQ_BF16 || sb == JQ_F16);
}

int dec_dense_launch(const QmvBatch& b, int nprob, int bits, int gs, int xd, int sb, int yd,
                     hipStream_t st) {
  int64_t maxN = 0;
  for (int i = 0; i < nprob; ++i) maxN = b.p[i].N > maxN ? b.p[i].N : maxN;
  if (maxN == 0) return JQ_OK;
  if (xd == JQ_BF16) {
    return sb == JQ_BF16 ? dense_bits<JQ_BF16, JQ_BF16>(bits, gs, b, nprob, maxN, yd, st)
                         : dense_bits<JQ_BF16, JQ_F16>(bits, gs, b, nprob, maxN, yd, st);
  }
  return sb == JQ_BF16 ? dense_bits<JQ_F16, JQ_BF16>(bits, gs, b, nprob, maxN, yd, st)
                       : dense_bits<JQ_F16, JQ_F16>(bits, gs, b, nprob, maxN, yd, st);
}

int dec_gather_launch(const QmmProblem& p, const QmmProblem* p2, const GatherPlan& plan,
                      int64_t max_tiles, int bits, int gs, int xd, int sb, int yd,
                      hipStream_t st) {
  if (max_tiles == 0 || p.N == 0) return JQ_OK;
  const QmmProblem& q2 = p2 ? *p2 : p;
#define JQ_X(XD, SBT)                                                                   \
  return p2 ? gather_bits<XD, SBT, 2>(bits, gs, p, q2, plan, max_tiles, yd, st)         \
            : gather_bits<XD, SBT, 1>(bits, gs, p, q2, plan, max_tiles, yd, st);
  if (xd == JQ_BF16) {
    if (sb == JQ_BF16) { JQ_X(JQ_BF16, JQ_BF16) }
    JQ_X(JQ_BF16, JQ_F16)
  }
  if (sb == JQ_BF16) { JQ_X(JQ_F16, JQ_BF16) }
  JQ_X(JQ_F16, JQ_F16)
#undef JQ_X
}

}  // namespace jqk

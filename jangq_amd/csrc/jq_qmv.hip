// Decode GEMV: y[m, n] = sum_k x[m, k] * (q[n, k] * s[n, k/gs] + b[n, k/gs]) for M <= 4.
//
// Memory-bound design for gfx950 (no matrix cores):
//   * a wave owns RW consecutive output rows; lane l walks the 32-code units l, l+64, ...
//     of every row, so each load instruction of the wave reads 64 consecutive units
//     (64 * 4*BITS bytes) of one row: fully coalesced, 8-32 bytes per lane;
//   * the unit's activations (32 per token) are loaded once per lane and reused for the RW
//     rows; they are paired (x_p, x_{p+4}) with byte permutes;
//   * codes are turned into exact 16-bit float "magic" values 2^B + q in registers and
//     multiplied with v_dot2_f32_{bf16,f16}; per unit the partial is
//       s * D + (b - 2^B s) * X      (D = magic dot product, X = sum of activations),
//     the factorisation of the reference's qdot (jang-tools/jang_tools/dsv41/metal_decode.py:202-233);
//   * a wave-wide butterfly reduction (DPP/permute) finishes each (row, token) sum.
// Accumulation is fp32 throughout; summation order differs from MLX's (allowed: outputs are
// checked against an fp32-accumulated oracle within rel-L2 1e-3).
#include "jq_common.h"
#include "jq_qmv.h"

namespace {

using namespace jq;
using jqk::QmvBatch;
using jqk::QmvProblem;

constexpr int kWaves = 4;  // waves per block

// Activations of one unit for one token: 32 values as 16 paired dwords plus their fp32 sum.
template <int XDT>
struct XUnit {
  uint32_t pr[16];  // for 16-bit x: chunk c pairs at pr[4c..4c+3]
  float xf[32];     // for f32 x: plain values (unused otherwise)
  float sum;
};

template <int XDT>
JQ_DEV void load_x_unit(const void* __restrict__ x, int64_t off, XUnit<XDT>& xu) {
  if constexpr (XDT == JQ_F32) {
    const float4* p = (const float4*)((const float*)x + off);
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float4 v = p[i];
      xu.xf[4 * i] = v.x; xu.xf[4 * i + 1] = v.y; xu.xf[4 * i + 2] = v.z; xu.xf[4 * i + 3] = v.w;
      s += (v.x + v.y) + (v.z + v.w);
    }
    xu.sum = s;
  } else {
    const uint4* p = (const uint4*)((const uint16_t*)x + off);
    uint32_t raw[16];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint4 v = p[i];
      raw[4 * i] = v.x; raw[4 * i + 1] = v.y; raw[4 * i + 2] = v.z; raw[4 * i + 3] = v.w;
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) pair_activations(&raw[4 * c], &xu.pr[4 * c]);
    // Plain sum via dot2 with (1, 1).
    constexpr uint32_t one2 = XDT == JQ_BF16 ? 0x3F803F80u : 0x3C003C00u;
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) s = dot2<XDT>(raw[i], one2, s);
    xu.sum = s;
  }
}

// Contribution of one unit of one row to one token: returns (D, offset) such that the unit
// adds  s*D + (b - offset*s)*X.
template <int BITS, int XDT>
JQ_DEV float unit_dot(const UnitWords<BITS>& u, const XUnit<XDT>& xu, float& offset) {
  if constexpr (XDT == JQ_F32) {
    // Exact int -> float through the 2^23 magic, then fp32 FMAs.
    float d = 0.f;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      const uint32_t q = unit_code_rt<BITS>(u.w, i);
      d = fmaf(__uint_as_float(0x4B000000u | q) - 8388608.0f, xu.xf[i], d);
    }
    offset = 0.f;
    return d;
  } else if constexpr (BITS == 8 && XDT == JQ_BF16) {
    float dl = 0.f, dh = 0.f;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      uint32_t lo[4], hi[4];
      chunk8_nibble_pairs(u.w[2 * c], u.w[2 * c + 1], lo, hi);
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        dl = dot2<XDT>(lo[p], xu.pr[4 * c + p], dl);
        dh = dot2<XDT>(hi[p], xu.pr[4 * c + p], dh);
      }
    }
    offset = 272.f;
    return fmaf(16.f, dh, dl);
  } else {
    float d0 = 0.f, d1 = 0.f;
    uint32_t pr[4];
    unit_chunk_pairs<XDT, BITS, 0>(u.w, pr);
#pragma unroll
    for (int p = 0; p < 4; ++p) d0 = dot2<XDT>(pr[p], xu.pr[p], d0);
    unit_chunk_pairs<XDT, BITS, 1>(u.w, pr);
#pragma unroll
    for (int p = 0; p < 4; ++p) d1 = dot2<XDT>(pr[p], xu.pr[4 + p], d1);
    unit_chunk_pairs<XDT, BITS, 2>(u.w, pr);
#pragma unroll
    for (int p = 0; p < 4; ++p) d0 = dot2<XDT>(pr[p], xu.pr[8 + p], d0);
    unit_chunk_pairs<XDT, BITS, 3>(u.w, pr);
#pragma unroll
    for (int p = 0; p < 4; ++p) d1 = dot2<XDT>(pr[p], xu.pr[12 + p], d1);
    offset = Magic<XDT, BITS>::offset;
    return d0 + d1;
  }
}

JQ_DEV float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// One launch computes `nprob` problems (same BITS, gs, M, K, dtypes); blockIdx.y selects
// the problem, blockIdx.x a block of kWaves*RW rows of it.
template <int BITS, int MT, int RW, int XDT>
__global__ void __launch_bounds__(64 * kWaves) qmv_kernel(QmvBatch batch, int gs_shift, int sb,
                                                          int yd) {
  const QmvProblem& pb = batch.p[blockIdx.y];
  const int64_t N = pb.N;
  const int K = batch.K;
  const int M = batch.M;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t row0 = ((int64_t)blockIdx.x * kWaves + wave) * RW;
  if (row0 >= N) return;
  const int upr = K >> 5;  // units per row
  const int G = K >> gs_shift;
  const uint32_t* __restrict__ codes = pb.codes;

  float acc[RW][MT];
#pragma unroll
  for (int r = 0; r < RW; ++r)
#pragma unroll
    for (int m = 0; m < MT; ++m) acc[r][m] = 0.f;

  for (int u = lane; u < upr; u += 64) {
    XUnit<XDT> xu[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      if (m < M) load_x_unit<XDT>(pb.x, (int64_t)m * K + (int64_t)u * 32, xu[m]);
    }
    const int g = (u * 32) >> gs_shift;
#pragma unroll
    for (int r = 0; r < RW; ++r) {
      const int64_t row = row0 + r;
      if (row < N) {
        const UnitWords<BITS> uw = load_unit<BITS>(codes + (row * upr + u) * BITS);
        const float s = load_as_f32(pb.scales, row * G + g, sb);
        const float b = load_as_f32(pb.biases, row * G + g, sb);
#pragma unroll
        for (int m = 0; m < MT; ++m) {
          if (m < M) {
            float off;
            const float d = unit_dot<BITS, XDT>(uw, xu[m], off);
            const float cb = fmaf(-off, s, b);
            acc[r][m] = fmaf(s, d, fmaf(cb, xu[m].sum, acc[r][m]));
          }
        }
      }
    }
  }

#pragma unroll
  for (int r = 0; r < RW; ++r) {
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      const float v = wave_sum(acc[r][m]);
      const int64_t row = row0 + r;
      if (lane == r * MT + m && row < N && m < M) {
        const int64_t o = (int64_t)m * N + row;
        if (yd == JQ_BF16) store_t<JQ_BF16>(pb.y, o, v);
        else if (yd == JQ_F16) store_t<JQ_F16>(pb.y, o, v);
        else store_t<JQ_F32>(pb.y, o, v);
      }
    }
  }
}

template <int BITS, int MT, int RW, int XDT>
int launch_qmv_t(const QmvBatch& b, int nprob, int64_t maxN, int gsh, int sb, int yd,
                 hipStream_t st) {
  const int64_t rows_per_block = kWaves * RW;
  dim3 grid((unsigned)((maxN + rows_per_block - 1) / rows_per_block), (unsigned)nprob);
  qmv_kernel<BITS, MT, RW, XDT><<<grid, 64 * kWaves, 0, st>>>(b, gsh, sb, yd);
  return jqh::launch_status();
}

template <int BITS, int MT, int XDT>
int launch_qmv_rw(const QmvBatch& b, int nprob, int64_t maxN, int gsh, int sb, int yd,
                  hipStream_t st) {
  // Rows per wave: enough loads in flight per lane, enough waves to fill 256 CUs.
  if (maxN >= 8192) return launch_qmv_t<BITS, MT, 4, XDT>(b, nprob, maxN, gsh, sb, yd, st);
  return launch_qmv_t<BITS, MT, 2, XDT>(b, nprob, maxN, gsh, sb, yd, st);
}

template <int BITS, int XDT>
int launch_qmv_m(const QmvBatch& b, int nprob, int64_t maxN, int gsh, int sb, int yd,
                 hipStream_t st) {
  if (b.M == 1) return launch_qmv_rw<BITS, 1, XDT>(b, nprob, maxN, gsh, sb, yd, st);
  if (b.M == 2) return launch_qmv_rw<BITS, 2, XDT>(b, nprob, maxN, gsh, sb, yd, st);
  return launch_qmv_rw<BITS, 4, XDT>(b, nprob, maxN, gsh, sb, yd, st);
}

template <int XDT>
int launch_qmv_b(int bits, const QmvBatch& b, int nprob, int64_t maxN, int gsh, int sb, int yd,
                 hipStream_t st) {
  switch (bits) {
    case 2: return launch_qmv_m<2, XDT>(b, nprob, maxN, gsh, sb, yd, st);
    case 3: return launch_qmv_m<3, XDT>(b, nprob, maxN, gsh, sb, yd, st);
    case 4: return launch_qmv_m<4, XDT>(b, nprob, maxN, gsh, sb, yd, st);
    case 5: return launch_qmv_m<5, XDT>(b, nprob, maxN, gsh, sb, yd, st);
    case 6: return launch_qmv_m<6, XDT>(b, nprob, maxN, gsh, sb, yd, st);
    default: return launch_qmv_m<8, XDT>(b, nprob, maxN, gsh, sb, yd, st);
  }
}

}  // namespace

namespace jqk {

int qmv_launch(const QmvBatch& b, int nprob, int bits, int gs, int xd, int sb, int yd,
               hipStream_t st) {
  int64_t maxN = 0;
  for (int i = 0; i < nprob; ++i) maxN = b.p[i].N > maxN ? b.p[i].N : maxN;
  if (maxN == 0 || b.M == 0) return JQ_OK;
  const int gsh = gs == 32 ? 5 : gs == 64 ? 6 : 7;
  if (b.M > 4) return JQ_ERR_SHAPE;
  switch (xd) {
    case JQ_F32: return launch_qmv_b<JQ_F32>(bits, b, nprob, maxN, gsh, sb, yd, st);
    case JQ_BF16: return launch_qmv_b<JQ_BF16>(bits, b, nprob, maxN, gsh, sb, yd, st);
    default: return launch_qmv_b<JQ_F16>(bits, b, nprob, maxN, gsh, sb, yd, st);
  }
}

}  // namespace jqk

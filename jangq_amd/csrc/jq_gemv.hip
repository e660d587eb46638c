// Decode GEMV on the vector ALUs: y[m, n] = sum_k x[m, k] * (q[n,k] * s[n,k/gs] + b[n,k/gs])
// for a few activation rows (M <= 4; M <= 2 at 2 bits), bf16 or f16 activations, K up to 512
// lane chunks. No matrix cores.
//
// Work split. A block of KW waves owns RB consecutive output rows. The row's packed codes are
// cut into lane chunks of UPL whole 32-code units (UPL = 2 for 2-bit, so that every chunk is
// 16 bytes; 1 otherwise: 12, 16, 20, 24 or 32 bytes). Wave w takes a contiguous range of
// chunks and lane l the chunks l, l+64, ... of that range (J per lane), so each load
// instruction of a wave reads one contiguous run of a row, and the lane's K slice is the same
// for every row of the block.
//
// Activation-stationary. The lane loads its K slice of x once per block and keeps it in
// registers in the pairing the code unpack produces, together with two per-unit constants,
// X = sum x and O = -sum offset_k x_k. The codes of all RB rows (plus their scales and biases)
// are issued up front, in the order they are consumed, so one wave keeps RB rows of loads in
// flight and waits on them one row at a time.
//
// Arithmetic. Codes become exact 16-bit floats (offset_k + q_k) with mask-and-or only (the
// per-code offset schedules for bf16 2/3/4-bit, the uniform 2^bits offset otherwise; 8-bit bf16
// splits into two nibbles); v_dot2_f32_{bf16,f16} multiplies them with the activation pairs.
// Per unit and row:  acc += s * (D + O) + b * X  with D the dot product of the exact values,
// i.e. the reference's  s * sum q x + b * sum x  (jang-tools/jang_tools/dsv41/metal_decode.py:202-233).
// Accumulation is fp32. Each (row, token) partial is summed over the wave with DPP row
// operations and over the block's waves through LDS.
#include "jq_dec.h"
#include "jq_qmv.h"

namespace {

using namespace jq;
using jqd::Bases;
using jqd::Dc;
using jqk::QmvBatch;
using jqk::QmvProblem;

template <int BITS>
constexpr int units_per_chunk() {
  return BITS == 2 ? 2 : 1;
}

// Activation state of one unit for one token: the 16 activation dwords paired as the unit's
// code dwords, X = sum x, O = -sum offset_k x_k.
struct XState {
  uint32_t pr[16];
  float X, O;
};

template <class D, int F, int P>
JQ_DEV uint32_t xpair_of(const jqd::XRaw& r) {
  return jqd::xpair<jqd::code_lo<D>(F, P), jqd::code_hi<D>(F, P)>(r);
}

template <class D>
JQ_DEV void make_xstate(const jqd::XRaw& r, XState& xs) {
#define JQ_XP(F, P) xs.pr[4 * F + P] = xpair_of<D, F, P>(r);
  JQ_XP(0, 0) JQ_XP(0, 1) JQ_XP(0, 2) JQ_XP(0, 3)
  JQ_XP(1, 0) JQ_XP(1, 1) JQ_XP(1, 2) JQ_XP(1, 3)
  JQ_XP(2, 0) JQ_XP(2, 1) JQ_XP(2, 2) JQ_XP(2, 3)
  JQ_XP(3, 0) JQ_XP(3, 1) JQ_XP(3, 2) JQ_XP(3, 3)
#undef JQ_XP
  float X = 0.f;
#pragma unroll
  for (int i = 0; i < 16; ++i) X = dot2<D::XDT>(r.d[i], D::ONE2, X);
  xs.X = X;
  if constexpr (D::SCHED) {
    float O = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) O = dot2<D::XDT>(jqd::bo_dword<D>(i >> 2, i & 3), xs.pr[i], O);
    xs.O = O;
  } else if constexpr (D::NIB) {
    xs.O = -272.f * X;
  } else {
    xs.O = -(float)(1 << D::BITS) * X;
  }
}

// Dot product of one unit's exact code values with its paired activations.
template <class D>
JQ_DEV float unit_dot(const uint32_t* w, const Bases<D>& bs, const XState& xs) {
  float d0 = 0.f, d1 = 0.f;
#define JQ_UF(F)                                                          \
  {                                                                       \
    u32x4 b, bh;                                                          \
    jqd::b_frag<D, F>(w, bs, b, bh);                                      \
    d0 = dot2<D::XDT>(b[0], xs.pr[4 * F + 0], d0);                        \
    d0 = dot2<D::XDT>(b[1], xs.pr[4 * F + 1], d0);                        \
    d0 = dot2<D::XDT>(b[2], xs.pr[4 * F + 2], d0);                        \
    d0 = dot2<D::XDT>(b[3], xs.pr[4 * F + 3], d0);                        \
    if constexpr (D::NIB) {                                               \
      d1 = dot2<D::XDT>(bh[0], xs.pr[4 * F + 0], d1);                     \
      d1 = dot2<D::XDT>(bh[1], xs.pr[4 * F + 1], d1);                     \
      d1 = dot2<D::XDT>(bh[2], xs.pr[4 * F + 2], d1);                     \
      d1 = dot2<D::XDT>(bh[3], xs.pr[4 * F + 3], d1);                     \
    }                                                                     \
  }
  JQ_UF(0) JQ_UF(1) JQ_UF(2) JQ_UF(3)
#undef JQ_UF
  if constexpr (D::NIB) return fmaf(16.f, d1, d0);
  return d0;
}

// Sum over the 64 lanes with DPP row operations; the total lands in lane 63.
JQ_DEV float wave_total_lane63(float v) {
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));  // quad_perm 1,0,3,2
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));  // quad_perm 2,3,0,1
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x124, 0xF, 0xF, false)); // row_ror 4
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x128, 0xF, 0xF, false)); // row_ror 8
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x142, 0xA, 0xF, false)); // row_bcast 15
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x143, 0xC, 0xF, false)); // row_bcast 31
  return v;
}

template <int SB>
JQ_DEV float sb_to_f32(uint32_t h) {
  if constexpr (SB == JQ_BF16) return __uint_as_float(h << 16);
  else return f16_bits_to_f32((uint16_t)h);
}

// Codes, scales and biases of one row for one lane: J chunks of UPL units (a scale and a
// bias per unit; units of one group load the same element).
template <int BITS, int UPL, int J>
struct RowLoad {
  uint32_t w[J][BITS * UPL];
  uint32_t s[J][UPL], b[J][UPL];
};

template <int N>
JQ_DEV void load_words(const uint32_t* __restrict__ p, uint32_t* w) {
  if constexpr (N == 4) {
    const u32x4 v = *(const u32x4*)p;
    w[0] = v[0]; w[1] = v[1]; w[2] = v[2]; w[3] = v[3];
  } else if constexpr (N == 8) {
    const u32x4 a = *(const u32x4*)p, c = *(const u32x4*)(p + 4);
    w[0] = a[0]; w[1] = a[1]; w[2] = a[2]; w[3] = a[3];
    w[4] = c[0]; w[5] = c[1]; w[6] = c[2]; w[7] = c[3];
  } else if constexpr (N == 6) {
    const uint2 a = *(const uint2*)p, b = *(const uint2*)(p + 2), c = *(const uint2*)(p + 4);
    w[0] = a.x; w[1] = a.y; w[2] = b.x; w[3] = b.y; w[4] = c.x; w[5] = c.y;
  } else {
#pragma unroll
    for (int i = 0; i < N; ++i) w[i] = p[i];
  }
}

// Block = KW waves (blockDim.x = 64 * KW, KW <= kMaxWaves); ushift = log2(gs / 32).
constexpr int kMaxWaves = 8;

template <class D, int SB, int MT, int RB, int J>
__global__ void __launch_bounds__(64 * kMaxWaves) gemv_kernel(QmvBatch batch, int ushift, int yd) {
  constexpr int BITS = D::BITS;
  constexpr int UPL = units_per_chunk<BITS>();
  __shared__ float red[kMaxWaves][RB * MT];
  const int KW = blockDim.x >> 6;

  const QmvProblem& pb = batch.p[blockIdx.y];
  const int64_t N = pb.N;
  const int64_t row0 = (int64_t)blockIdx.x * RB;
  if (row0 >= N) return;  // whole block
  const int K = batch.K, M = batch.M;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int C = K / (32 * UPL);                  // chunks per row
  const int CW = (C + KW - 1) / KW;              // chunks per wave
  const int64_t P = (int64_t)K * BITS / 32;      // words per row
  const int G = K >> (ushift + 5);

  // Lane chunks: active flag and clamped chunk index.
  int cidx[J];
  bool act[J];
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int loc = lane + 64 * j;
    const int c = wave * CW + loc;
    act[j] = loc < CW && c < C;
    cidx[j] = act[j] ? c : 0;
  }

  // Activations first (so waiting for them does not wait for the codes).
  jqd::XRaw xr[J][UPL][MT];
#pragma unroll
  for (int j = 0; j < J; ++j)
#pragma unroll
    for (int t = 0; t < UPL; ++t)
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        const int mm = m < M ? m : M - 1;
        jqd::load_xraw((const uint16_t*)pb.x + (int64_t)mm * K + (int64_t)(cidx[j] * UPL + t) * 32,
                       xr[j][t][m]);
      }

  // All RB rows of codes, scales and biases, in consumption order.
  RowLoad<BITS, UPL, J> rl[RB];
  const uint32_t* __restrict__ codes = pb.codes;
  const uint16_t* __restrict__ sc = (const uint16_t*)pb.scales;
  const uint16_t* __restrict__ bi = (const uint16_t*)pb.biases;
#pragma unroll
  for (int r = 0; r < RB; ++r) {
    const int64_t row = row0 + r < N ? row0 + r : N - 1;
#pragma unroll
    for (int j = 0; j < J; ++j) {
      load_words<BITS * UPL>(codes + row * P + (int64_t)cidx[j] * UPL * BITS, rl[r].w[j]);
#pragma unroll
      for (int t = 0; t < UPL; ++t) {
        const int64_t gi = row * G + ((cidx[j] * UPL + t) >> ushift);
        rl[r].s[j][t] = sc[gi];
        rl[r].b[j][t] = bi[gi];
      }
    }
  }

  XState xs[J][UPL][MT];
#pragma unroll
  for (int j = 0; j < J; ++j)
#pragma unroll
    for (int t = 0; t < UPL; ++t)
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        jqd::XRaw& r = xr[j][t][m];
        const bool live = act[j] && m < M;
#pragma unroll
        for (int i = 0; i < 16; ++i) r.d[i] = live ? r.d[i] : 0u;
        make_xstate<D>(r, xs[j][t][m]);
      }

  const Bases<D> bs = jqd::make_bases<D>();
  float acc[RB][MT];
#pragma unroll
  for (int r = 0; r < RB; ++r) {
#pragma unroll
    for (int m = 0; m < MT; ++m) acc[r][m] = 0.f;
#pragma unroll
    for (int j = 0; j < J; ++j)
#pragma unroll
      for (int t = 0; t < UPL; ++t) {
        const float s = sb_to_f32<SB>(rl[r].s[j][t]);
        const float b = sb_to_f32<SB>(rl[r].b[j][t]);
#pragma unroll
        for (int m = 0; m < MT; ++m) {
          const float d = unit_dot<D>(rl[r].w[j] + t * BITS, bs, xs[j][t][m]);
          acc[r][m] = fmaf(s, d + xs[j][t][m].O, fmaf(b, xs[j][t][m].X, acc[r][m]));
        }
      }
  }

#pragma unroll
  for (int r = 0; r < RB; ++r)
#pragma unroll
    for (int m = 0; m < MT; ++m) acc[r][m] = wave_total_lane63(acc[r][m]);

  void* y = pb.y;
  if (KW == 1) {
    if (lane == 63) {
#pragma unroll
      for (int r = 0; r < RB; ++r)
#pragma unroll
        for (int m = 0; m < MT; ++m) {
          const int64_t row = row0 + r;
          if (row < N && m < M) {
            const int64_t o = (int64_t)m * N + row;
            if (yd == JQ_BF16) store_t<JQ_BF16>(y, o, acc[r][m]);
            else if (yd == JQ_F16) store_t<JQ_F16>(y, o, acc[r][m]);
            else store_t<JQ_F32>(y, o, acc[r][m]);
          }
        }
    }
  } else {
    if (lane == 63) {
#pragma unroll
      for (int r = 0; r < RB; ++r)
#pragma unroll
        for (int m = 0; m < MT; ++m) red[wave][r * MT + m] = acc[r][m];
    }
    __syncthreads();
    const int t = threadIdx.x;
    if (t < RB * MT) {
      float v = 0.f;
      for (int w = 0; w < KW; ++w) v += red[w][t];
      const int r = t / MT, m = t % MT;
      const int64_t row = row0 + r;
      if (row < N && m < M) {
        const int64_t o = (int64_t)m * N + row;
        if (yd == JQ_BF16) store_t<JQ_BF16>(y, o, v);
        else if (yd == JQ_F16) store_t<JQ_F16>(y, o, v);
        else store_t<JQ_F32>(y, o, v);
      }
    }
  }
}

// Launch shape: the fewest waves per block (a power of two, at most kMaxWaves) for which
// every lane holds one chunk of a row.
template <class D, int SB, int MT, int RB>
int launch_kw(const QmvBatch& b, int nprob, int64_t maxN, int ushift, int yd, hipStream_t st) {
  constexpr int UPL = units_per_chunk<D::BITS>();
  const int C = b.K / (32 * UPL);
  int kw = 1;
  while (64 * kw < C) kw *= 2;
  if (kw > kMaxWaves) return JQ_ERR_SHAPE;
  dim3 grid((unsigned)((maxN + RB - 1) / RB), (unsigned)nprob);
  gemv_kernel<D, SB, MT, RB, 1><<<grid, 64 * kw, 0, st>>>(b, ushift, yd);
  return jqh::launch_status();
}

// Rows per block: all of a block's rows are loaded before the first is used, so RB is set by
// the registers left after the activations (18 per unit and token).
template <class D, int SB>
int launch_m(const QmvBatch& b, int nprob, int64_t maxN, int ushift, int yd, hipStream_t st) {
  constexpr bool two = D::BITS == 2;  // two units per lane chunk
  if (b.M == 1) return launch_kw<D, SB, 1, 8>(b, nprob, maxN, ushift, yd, st);
  if (b.M == 2) return launch_kw<D, SB, 2, two ? 4 : 8>(b, nprob, maxN, ushift, yd, st);
  if constexpr (!two) return launch_kw<D, SB, 4, 4>(b, nprob, maxN, ushift, yd, st);
  return JQ_ERR_SHAPE;
}

template <int BITS, int XDT>
int launch_sb(const QmvBatch& b, int nprob, int64_t maxN, int ushift, int sb, int yd,
              hipStream_t st) {
  using D = Dc<BITS, 64, XDT>;  // the group size is a run-time argument of this kernel
  if (sb == JQ_BF16) return launch_m<D, JQ_BF16>(b, nprob, maxN, ushift, yd, st);
  return launch_m<D, JQ_F16>(b, nprob, maxN, ushift, yd, st);
}

template <int BITS>
int launch_x(const QmvBatch& b, int nprob, int64_t maxN, int ushift, int xd, int sb, int yd,
             hipStream_t st) {
  if (xd == JQ_BF16) return launch_sb<BITS, JQ_BF16>(b, nprob, maxN, ushift, sb, yd, st);
  return launch_sb<BITS, JQ_F16>(b, nprob, maxN, ushift, sb, yd, st);
}

}  // namespace

namespace jqk {

bool gemv_ok(int M, int64_t K, int bits, int gs, int xd, int sb) {
  if (M < 1 || M > (bits == 2 ? 2 : 4)) return false;
  if (xd != JQ_BF16 && xd != JQ_F16) return false;
  if (sb != JQ_BF16 && sb != JQ_F16) return false;
  const int64_t chunk = bits == 2 ? 64 : 32;  // K of one lane chunk
  if (K <= 0 || K % chunk || K / chunk > 64 * kMaxWaves) return false;
  (void)gs;
  return true;
}

int gemv_launch(const QmvBatch& b, int nprob, int bits, int gs, int xd, int sb, int yd,
                hipStream_t st) {
  int64_t maxN = 0;
  for (int i = 0; i < nprob; ++i) maxN = b.p[i].N > maxN ? b.p[i].N : maxN;
  if (maxN == 0 || b.M == 0) return JQ_OK;
  if (!gemv_ok(b.M, b.K, bits, gs, xd, sb)) return JQ_ERR_SHAPE;
  const int us = gs == 32 ? 0 : gs == 64 ? 1 : 2;
  switch (bits) {
    case 2: return launch_x<2>(b, nprob, maxN, us, xd, sb, yd, st);
    case 3: return launch_x<3>(b, nprob, maxN, us, xd, sb, yd, st);
    case 4: return launch_x<4>(b, nprob, maxN, us, xd, sb, yd, st);
    case 5: return launch_x<5>(b, nprob, maxN, us, xd, sb, yd, st);
    case 6: return launch_x<6>(b, nprob, maxN, us, xd, sb, yd, st);
    default: return launch_x<8>(b, nprob, maxN, us, xd, sb, yd, st);
  }
}

}  // namespace jqk

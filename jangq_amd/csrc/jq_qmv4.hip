// Decode GEMV on 4x4x4 matrix-core blocks: y[m, n] = sum_k x[m, k] * (q[n,k] s[n,k/gs] + b[n,k/gs])
// for up to 8 activation rows per pass (more in passes), bf16 or f16 activations.
//
// Why this shape. v_mfma_f32_4x4x4_16b multiplies 16 independent 4x4x4 blocks; block b lives in
// lanes 4b..4b+3, lane 4b+j holds row j of its A operand, column j of its B operand and column
// j of its result. Here column j is W row (4q + j) of a row quad and block b is a 32-code unit
// of that row, so one wave load instruction reads 4 W rows x 16 consecutive units: long
// contiguous runs, as few cache lines per instruction as a plain row-streaming GEMV (the
// 16-row fragments of the larger MFMA shapes touch 16+ lines per instruction and leave the
// texture-address unit as the bottleneck). A row i is token i of the pass, so the matrix core
// does every token's multiply-adds and the vector ALUs only unpack codes and apply scales.
//
// Per lane (block b = unit, j = row of the quad): the lane holds its units' activations for
// its own token j (the pairs the code unpack yields, jq_gemv.h make_xstate) and, for all four
// tokens of a set, X = sum x and O = -sum offset*x of each unit (from its quad neighbours).
// Per unit and row:  D_i = O_i + sum_k x_ik (offset_k + q_k) = sum_k x_ik q_k  by 8 MFMAs (4
// codes each; 16 with the two nibbles of 8-bit codes and bf16 activations), then
//   acc_i += s * D_i + b * X_i
// which is the reference's s * sum q x + b * sum x (jang-tools/jang_tools/dsv41/metal_decode.py:202-233).
//
// Pipeline (that of jq_gemv.hip): a block of KW waves covers K (wave w: units
// [16 UPL w, 16 UPL (w+1))), blocks are persistent over items of RQ row quads, the RQ quads'
// codes, scales and biases sit in a register ring and quad q of the next item is issued as soon
// as quad q of the current one has been consumed. Each item ends with a reduction over the 16
// unit lanes (DPP within rows of 16 lanes, lane swizzles across them), one LDS exchange between
// the waves and the stores.
#include "jq_gemv.h"
#include "jq_qmv.h"

namespace {

using namespace jq;
using namespace jqg;
using jqk::QmvBatch;
using jqk::QmvProblem;

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));

// D + A(4x4) * B(4x4) in each of the 16 blocks; a0:a1 and b0:b1 hold four 16-bit values each.
template <int FMT>
JQ_DEV f32x4 mfma4(uint32_t a0, uint32_t a1, uint32_t b0, uint32_t b1, f32x4 c) {
  const u32x2 a = {a0, a1}, b = {b0, b1};
  if constexpr (FMT == JQ_BF16) {
    return __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(__builtin_bit_cast(s16x4, a),
                                                  __builtin_bit_cast(s16x4, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_4x4x4f16(__builtin_bit_cast(f16x4, a),
                                              __builtin_bit_cast(f16x4, b), c, 0, 0, 0);
  }
}

// v broadcast from lane 4*(l/4) + I of each quad (DPP quad_perm I,I,I,I).
template <int I>
JQ_DEV float quad_bcast(float v) {
  constexpr int ctrl = I | (I << 2) | (I << 4) | (I << 6);
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v),
                                                               ctrl, 0xF, 0xF, false));
}

// Sum of v over the 16 lanes with the same l % 4 (every such lane receives the total).
JQ_DEV float unit_lanes_total(float v) {
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x124, 0xF, 0xF, false));  // row_ror 4
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x128, 0xF, 0xF, false));  // row_ror 8
  v += __shfl_xor(v, 16, 64);
  v += __shfl_xor(v, 32, 64);
  return v;
}

struct Qmv4Args {
  QmvBatch b;
  int rb_begin[jqk::kMaxProblems + 1];  // first item of each problem
  int nprob;
  int ushift;  // log2(gs / 32)
  int m0;      // first activation row of this pass
  int mrows;   // activation rows of this pass
  int yd;
};

// One row quad of a lane's ring: its UPL units of codes and their scale / bias.
template <int BITS, int UPL>
struct QuadSlot {
  uint32_t w[UPL][BITS];
  uint32_t s[UPL], b[UPL];
};

// MT: activation rows of the pass rounded up (1, 2, 4 or 8); NT = token sets of 4.
template <class D, int SB, int MT, int RQ, int UPL>
__global__ void __launch_bounds__(64 * kMaxWaves) qmv4_kernel(Qmv4Args a) {
  constexpr int BITS = D::BITS;
  constexpr int NT = (MT + 3) / 4;
  constexpr int TS = MT < 4 ? MT : 4;          // live token slots per set
  constexpr int NV = NT * TS * RQ;             // partial values per lane per item
  __shared__ float red[2][kMaxWaves][NV][4];

  const int total = a.rb_begin[a.nprob];
  int it = blockIdx.x;
  if (it >= total) return;  // whole block
  const int KW = blockDim.x >> 6;
  const int K = a.b.K;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int ub = lane >> 2, j = lane & 3;
  const int U = K / 32;  // units per row
  const uint32_t rowbytes = (uint32_t)U * BITS * 4;
  const uint32_t sbrow = (uint32_t)(U >> a.ushift) * 2;

  // This lane's units and their offsets.
  uint32_t voff[UPL], vsb[UPL];
  bool ulive[UPL];
#pragma unroll
  for (int t = 0; t < UPL; ++t) {
    const int u = (wave * UPL + t) * 16 + ub;
    ulive[t] = u < U;
    const int uc = ulive[t] ? u : 0;
    voff[t] = (uint32_t)uc * BITS * 4;
    vsb[t] = (uint32_t)(uc >> a.ushift) * 2;
  }

  // Activations of token 4s + j for the lane's units, paired as the code unpack yields them.
  jqd::XRaw xr[NT][UPL];
#pragma unroll
  for (int s = 0; s < NT; ++s)
#pragma unroll
    for (int t = 0; t < UPL; ++t) {
      int tok = 4 * s + j;
      tok = tok < a.mrows ? tok : a.mrows - 1;
      const int u = ulive[t] ? (wave * UPL + t) * 16 + ub : 0;
      jqd::load_xraw((const uint16_t*)a.b.p[0].x + (int64_t)(a.m0 + tok) * K + (int64_t)u * 32,
                     xr[s][t]);
    }

  auto locate = [&](int i, int& p, int64_t& row0) {
    p = 0;
#pragma unroll
    for (int q = 1; q < jqk::kMaxProblems; ++q)
      if (q < a.nprob && i >= a.rb_begin[q]) p = q;
    row0 = (int64_t)(i - a.rb_begin[p]) * (4 * RQ);
  };
  auto views = [&](int p, int64_t row0, bool live, Rsrc& rc, Rsrc& rs, Rsrc& rb) {
    const QmvProblem& pb = a.b.p[p];
    const int64_t left = pb.N - row0;
    const uint32_t rows = live ? (uint32_t)(left < 4 * RQ ? left : 4 * RQ) : 0u;
    rc = make_rsrc((const char*)pb.codes + row0 * rowbytes, rows * rowbytes);
    rs = make_rsrc((const char*)pb.scales + row0 * sbrow, rows * sbrow);
    rb = make_rsrc((const char*)pb.biases + row0 * sbrow, rows * sbrow);
  };
  auto load_quad = [&](Rsrc rc, Rsrc rs, Rsrc rb, int q, QuadSlot<BITS, UPL>& sl) {
    const uint32_t r = (uint32_t)(4 * q + j);
#pragma unroll
    for (int t = 0; t < UPL; ++t) {
      load_chunk<BITS>(rc, voff[t] + r * rowbytes, sl.w[t]);
      sl.s[t] = __builtin_amdgcn_raw_buffer_load_b16(rs, vsb[t] + r * sbrow, 0, 0);
      sl.b[t] = __builtin_amdgcn_raw_buffer_load_b16(rb, vsb[t] + r * sbrow, 0, 0);
    }
  };

  int p;
  int64_t row0;
  locate(it, p, row0);
  Rsrc rc, rs, rbv;
  views(p, row0, true, rc, rs, rbv);
  QuadSlot<BITS, UPL> ring[RQ];
#pragma unroll
  for (int q = 0; q < RQ; ++q) {
    load_quad(rc, rs, rbv, q, ring[q]);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
  }

  // Paired activations, and X / O of the four tokens of each set (from the quad neighbours).
  uint32_t pr[NT][UPL][16];
  float Xq[NT][UPL][TS], Oq[NT][UPL][TS];
#pragma unroll
  for (int s = 0; s < NT; ++s)
#pragma unroll
    for (int t = 0; t < UPL; ++t) {
      jqd::XRaw& r = xr[s][t];
      const bool live = ulive[t] && 4 * s + j < a.mrows;
#pragma unroll
      for (int i = 0; i < 16; ++i) r.d[i] = live ? r.d[i] : 0u;
      XState xs;
      make_xstate<D>(r, xs);
#pragma unroll
      for (int i = 0; i < 16; ++i) pr[s][t][i] = xs.pr[i];
      Xq[s][t][0] = quad_bcast<0>(xs.X);
      Oq[s][t][0] = quad_bcast<0>(xs.O);
      if constexpr (TS > 1) { Xq[s][t][1] = quad_bcast<1>(xs.X); Oq[s][t][1] = quad_bcast<1>(xs.O); }
      if constexpr (TS > 2) {
        Xq[s][t][2] = quad_bcast<2>(xs.X); Oq[s][t][2] = quad_bcast<2>(xs.O);
        Xq[s][t][3] = quad_bcast<3>(xs.X); Oq[s][t][3] = quad_bcast<3>(xs.O);
      }
    }
  const Bases<D> bs = jqd::make_bases<D>();

  for (int par = 0;; par ^= 1) {
    const int nx = it + gridDim.x;
    const bool more = nx < total;
    int p2;
    int64_t row02;
    locate(more ? nx : it, p2, row02);
    Rsrc rc2, rs2, rb2;
    views(p2, row02, more, rc2, rs2, rb2);

    float acc[NT][RQ][TS];
#pragma unroll
    for (int q = 0; q < RQ; ++q) {
#pragma unroll
      for (int s = 0; s < NT; ++s)
#pragma unroll
        for (int i = 0; i < TS; ++i) acc[s][q][i] = 0.f;
#pragma unroll
      for (int t = 0; t < UPL; ++t) {
        const float sv = sb_to_f32<SB>(ring[q].s[t]);
        const float bv = sb_to_f32<SB>(ring[q].b[t]);
        f32x4 Dd[NT], Dh[NT];
#pragma unroll
        for (int s = 0; s < NT; ++s) {
          Dd[s] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int i = 0; i < TS; ++i) Dd[s][i] = Oq[s][t][i];  // D starts at -sum offset*x
          Dh[s] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
#define JQ_F(F)                                                                        \
        {                                                                              \
          u32x4 B, BH;                                                                 \
          jqd::b_frag<D, F>(ring[q].w[t], bs, B, BH);                                  \
          _Pragma("unroll") for (int s = 0; s < NT; ++s) {                             \
            const uint32_t* x = pr[s][t];                                              \
            Dd[s] = mfma4<D::XDT>(x[4 * F], x[4 * F + 1], B[0], B[1], Dd[s]);          \
            Dd[s] = mfma4<D::XDT>(x[4 * F + 2], x[4 * F + 3], B[2], B[3], Dd[s]);      \
            if constexpr (D::NIB) {                                                    \
              Dh[s] = mfma4<D::XDT>(x[4 * F], x[4 * F + 1], BH[0], BH[1], Dh[s]);      \
              Dh[s] = mfma4<D::XDT>(x[4 * F + 2], x[4 * F + 3], BH[2], BH[3], Dh[s]);  \
            }                                                                          \
          }                                                                            \
        }
        JQ_F(0) JQ_F(1) JQ_F(2) JQ_F(3)
#undef JQ_F
#pragma unroll
        for (int s = 0; s < NT; ++s)
#pragma unroll
          for (int i = 0; i < TS; ++i) {
            const float d = D::NIB ? fmaf(16.f, Dh[s][i], Dd[s][i]) : Dd[s][i];
            acc[s][q][i] = fmaf(sv, d, fmaf(bv, Xq[s][t][i], acc[s][q][i]));
          }
      }
      // Quad q is consumed before its slot is reloaded (results first, then memory).
#pragma unroll
      for (int s = 0; s < NT; ++s)
#pragma unroll
        for (int i = 0; i < TS; ++i) asm volatile("" : "+v"(acc[s][q][i])::"memory");
      load_quad(rc2, rs2, rb2, q, ring[q]);
      __builtin_amdgcn_sched_barrier(0);
    }

    // Totals over the unit lanes; value v = (s, q, i) goes to LDS from lane unit v % 16.
#pragma unroll
    for (int s = 0; s < NT; ++s)
#pragma unroll
      for (int q = 0; q < RQ; ++q)
#pragma unroll
        for (int i = 0; i < TS; ++i) {
          const int v = (s * RQ + q) * TS + i;
          const float tot = unit_lanes_total(acc[s][q][i]);
          if (ub == v % 16) red[par][wave][v][j] = tot;
        }
    __syncthreads();
    {
      const QmvProblem& pb = a.b.p[p];
      for (int o = threadIdx.x; o < NV * 4; o += blockDim.x) {
        const int v = o >> 2, jj = o & 3;
        float tot = 0.f;
        for (int w = 0; w < KW; ++w) tot += red[par][w][v][jj];
        const int i = v % TS, q = (v / TS) % RQ, s = v / (TS * RQ);
        const int tok = 4 * s + i;
        const int64_t n = row0 + 4 * q + jj;
        if (tok < a.mrows && n < pb.N) {
          const int64_t oi = (int64_t)(a.m0 + tok) * pb.N + n;
          if (a.yd == JQ_BF16) store_t<JQ_BF16>(pb.y, oi, tot);
          else if (a.yd == JQ_F16) store_t<JQ_F16>(pb.y, oi, tot);
          else store_t<JQ_F32>(pb.y, oi, tot);
        }
      }
    }
    if (!more) break;
    it = nx;
    p = p2;
    row0 = row02;
  }
}

template <class D, int SB, int MT, int RQ, int UPL>
int launch_cfg(Qmv4Args& a, int kw, hipStream_t st) {
  int total = 0;
  for (int i = 0; i < a.nprob; ++i) {
    a.rb_begin[i] = total;
    total += (int)((a.b.p[i].N + 4 * RQ - 1) / (4 * RQ));
  }
  for (int i = a.nprob; i <= jqk::kMaxProblems; ++i) a.rb_begin[i] = total;
  if (total == 0) return JQ_OK;
  auto kern = qmv4_kernel<D, SB, MT, RQ, UPL>;
  const int64_t cap = (int64_t)jqh::blocks_per_cu((const void*)kern, 64 * kw, 0) * jqh::cus();
  const int64_t iters = (total + cap - 1) / cap;
  const int grid = (int)((total + iters - 1) / iters);
  kern<<<grid, 64 * kw, 0, st>>>(a);
  return jqh::launch_status();
}

// Units per lane: the fewest (1, 2 or 4) for which at most kMaxWaves waves cover a row.
inline int qmv4_upl(int64_t K, int* kw) {
  const int64_t U = K / 32;
  for (int upl = 1; upl <= 4; upl *= 2) {
    const int64_t w = (U + 16 * upl - 1) / (16 * upl);
    if (w <= kMaxWaves) {
      *kw = (int)w;
      return upl;
    }
  }
  return 0;
}

// Row quads per item (the ring depth): 4, fewer where the ring would not fit the registers.
template <class D, int SB, int MT>
int launch_mt(Qmv4Args& a, hipStream_t st) {
  int kw = 0;
  const int upl = qmv4_upl(a.b.K, &kw);
  constexpr bool wide = D::BITS > 4 || MT > 4;  // large code or activation state
  if (upl == 1) return launch_cfg<D, SB, MT, 4, 1>(a, kw, st);
  if (upl == 2) {
    if constexpr (wide) return launch_cfg<D, SB, MT, 2, 2>(a, kw, st);
    else return launch_cfg<D, SB, MT, 4, 2>(a, kw, st);
  }
  if (upl == 4) {
    if constexpr (MT <= 4 && D::BITS <= 4) return launch_cfg<D, SB, MT, 2, 4>(a, kw, st);
  }
  return JQ_ERR_SHAPE;
}

template <class D, int SB>
int launch_pass(Qmv4Args& a, hipStream_t st) {
  if (a.mrows == 1) return launch_mt<D, SB, 1>(a, st);
  if (a.mrows == 2) return launch_mt<D, SB, 2>(a, st);
  if (a.mrows <= 4) return launch_mt<D, SB, 4>(a, st);
  return launch_mt<D, SB, 8>(a, st);
}

template <int BITS, int XDT, int SB>
int launch_t(const QmvBatch& b, int nprob, int ushift, int yd, hipStream_t st) {
  using D = jqd::Dc<BITS, 64, XDT>;  // the group size is a run-time argument of this kernel
  int kw = 0;
  const int upl = qmv4_upl(b.K, &kw);
  const int pass = upl == 4 ? 4 : 8;  // activation rows per pass
  for (int m0 = 0; m0 < b.M; m0 += pass) {
    Qmv4Args a;
    a.b = b;
    a.nprob = nprob;
    a.ushift = ushift;
    a.m0 = m0;
    a.mrows = b.M - m0 < pass ? b.M - m0 : pass;
    a.yd = yd;
    const int s = launch_pass<D, SB>(a, st);
    if (s) return s;
  }
  return JQ_OK;
}

template <int BITS>
int launch_bits(const QmvBatch& b, int nprob, int ushift, int xd, int sb, int yd, hipStream_t st) {
  if (xd == JQ_BF16) {
    return sb == JQ_BF16 ? launch_t<BITS, JQ_BF16, JQ_BF16>(b, nprob, ushift, yd, st)
                         : launch_t<BITS, JQ_BF16, JQ_F16>(b, nprob, ushift, yd, st);
  }
  return sb == JQ_BF16 ? launch_t<BITS, JQ_F16, JQ_BF16>(b, nprob, ushift, yd, st)
                       : launch_t<BITS, JQ_F16, JQ_F16>(b, nprob, ushift, yd, st);
}

}  // namespace

namespace jqk {

bool qmv4_ok(int M, int64_t K, int64_t maxN, int bits, int gs, int xd, int sb) {
  (void)gs;
  int kw = 0;
  if (M < 1 || K <= 0 || K % 32) return false;
  const int upl = qmv4_upl(K, &kw);
  if (upl == 0 || (upl == 4 && bits > 4)) return false;
  return (xd == JQ_BF16 || xd == JQ_F16) && (sb == JQ_BF16 || sb == JQ_F16) &&
         (maxN + 64) * (K / 32) * 2 < ((int64_t)1 << 31) && K * bits / 8 < ((int64_t)1 << 24);
}

int qmv4_launch(const QmvBatch& b, int nprob, int bits, int gs, int xd, int sb, int yd,
                hipStream_t st) {
  int64_t maxN = 0;
  for (int i = 0; i < nprob; ++i) maxN = b.p[i].N > maxN ? b.p[i].N : maxN;
  if (maxN == 0 || b.M == 0) return JQ_OK;
  if (!qmv4_ok(b.M, b.K, maxN, bits, gs, xd, sb)) return JQ_ERR_SHAPE;
  // Problems of one launch must share the activations (they stay in registers).
  for (int i = 1; i < nprob; ++i) {
    if (b.p[i].x != b.p[0].x) {
      for (int k = 0; k < nprob; ++k) {
        QmvBatch one = b;
        one.p[0] = b.p[k];
        const int s = qmv4_launch(one, 1, bits, gs, xd, sb, yd, st);
        if (s) return s;
      }
      return JQ_OK;
    }
  }
  const int ushift = gs == 32 ? 0 : gs == 64 ? 1 : 2;
  switch (bits) {
    case 2: return launch_bits<2>(b, nprob, ushift, xd, sb, yd, st);
    case 3: return launch_bits<3>(b, nprob, ushift, xd, sb, yd, st);
    case 4: return launch_bits<4>(b, nprob, ushift, xd, sb, yd, st);
    case 5: return launch_bits<5>(b, nprob, ushift, xd, sb, yd, st);
    case 6: return launch_bits<6>(b, nprob, ushift, xd, sb, yd, st);
    default: return launch_bits<8>(b, nprob, ushift, xd, sb, yd, st);
  }
}

}  // namespace jqk

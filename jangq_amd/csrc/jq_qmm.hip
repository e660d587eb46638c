// Matrix-core GEMM for quantized weights: y = x @ deq(W)^T, bf16/f16 activations.
//
// Exact factorised form. Per group g of a row n, with codes in the B operand as the 16-bit
// floats 2^B + q (exact, see jq_common.h "magic pairs"):
//   y[m, n] += s[n,g] * P[m, n, g] + (b[n,g] - 2^B s[n,g]) * X[m, g]
//   P[m, n, g] = sum_{k in g} (2^B + q[n,k]) x[m,k]      (v_mfma_f32_16x16x32_{bf16,f16})
//   X[m, g]    = sum_{k in g} x[m,k]
// Every product inside the MFMA is exact and accumulates in fp32, so the result carries
// fp32 accumulation error only (no bf16 rounding of dequantized weights). The reference's
// own dequantized weights are the fp32 values q*s+b (jang-tools/jang_tools/affine.py:445-463).
//
// Tiling: a block of 4 waves computes a BM x BN output tile, walking K in tiles of 128
// codes. Each k-tile stages through LDS:
//   xs    activations [BM][128] as (x_p, x_{p+4}) pairs, one 16-byte chunk per 8 values
//   xsum  per-group activation sums [groups][BM]
//   ws    packed code words [BN][128*BITS/32] (+ padding)
//   sc/cb per-group scale and bias - 2^B*scale [groups][BN]
// Global loads of tile t+1 are issued into registers before tile t is computed.
// MFMA fragment layout (16x16x32): lane l holds row l%16 of A / column l%16 of B, and the
// 8 consecutive k-slots of lane group l/16; C/D hold rows 4*(l/16)+i, column l%16.
// A and B use the same slot -> k assignment (chunk l/16 of the slice, pair order), so the
// permutation inside a chunk cancels.
#include "jq_common.h"
#include "jq_qmv.h"

namespace {

using namespace jq;
using jqk::GatherPlan;
using jqk::QmmProblem;

constexpr int KT = 128;  // codes per k-tile

template <int BITS_, int GS_, int BM_, int BN_, int WGM_, int WGN_, int XDT_, int NB_ = 1>
struct Cfg {
  static constexpr int BITS = BITS_, GS = GS_, BM = BM_, BN = BN_, WGM = WGM_, WGN = WGN_;
  static constexpr int NB = NB_;  // weight matrices sharing the A tile (2 = gate+up)
  static constexpr int XDT = XDT_;
  static constexpr int WM = BM / WGM, WN = BN / WGN;
  static constexpr int FM = WM / 16, FN = WN / 16;
  static constexpr int WPR = KT * BITS / 32;  // code words per row per k-tile
  static constexpr int WST = WPR + 4;         // LDS row stride in words
  static constexpr int XST = KT / 2 + 4;      // LDS activation row stride in dwords
  static constexpr int GT = KT / GS;          // groups per k-tile
  static constexpr int SPG = GS / 32;         // MFMA slices per group
  static constexpr bool NIB = (BITS == 8 && XDT == JQ_BF16);
  static constexpr bool F16X = false;
  static constexpr int XCH = BM * (KT / 8);   // 16-byte activation chunks per tile
  static constexpr int XIT = (XCH + 255) / 256;
  static constexpr int CVEC = BN * WPR / 4;   // 16-byte code vectors per tile
  static constexpr int CIT = (CVEC + 255) / 256;
  static constexpr int SCN = BN * GT;         // (row, group) scale entries per tile
  static constexpr int SIT = (SCN + 255) / 256;
  static_assert(WGM * WGN == 4, "4 waves per block");
  static_assert(FM >= 1 && FN >= 1, "wave tile must hold whole 16x16 blocks");
  static_assert(WPR % 4 == 0, "code rows must be whole 16-byte vectors");
};

template <class C>
struct Smem {
  uint32_t xs[C::BM][C::XST];
  float xsum[C::GT][C::BM];
  uint32_t ws[C::NB][C::BN][C::WST];
  float sc[C::NB][C::GT][C::BN];
  float cb[C::NB][C::GT][C::BN];
};

// Registers holding one k-tile's global loads (prefetch stage).
template <class C>
struct Stage {
  uint4 x[C::XIT];
  uint4 c[C::NB][C::CIT];
  float s[C::NB][C::SIT];
  float b[C::NB][C::SIT];
};

template <class C>
struct TileCtx {
  // A row pointers (element offsets into x) for the rows this thread loads, -1 = zero row.
  int64_t xoff[C::XIT];
  const uint32_t* codes[C::NB];  // expert base of each weight matrix
  const void* scales[C::NB];
  const void* biases[C::NB];
  int64_t n0;              // first output column (row of W) of the tile
  int64_t N;
  int64_t P;               // words per W row
  int64_t G;               // groups per W row
};

template <class C>
JQ_DEV void load_stage(const TileCtx<C>& t, const void* __restrict__ x, int kt, int sb,
                       Stage<C>& st) {
  const int tid = threadIdx.x;
#pragma unroll
  for (int it = 0; it < C::XIT; ++it) {
    const int ci = tid + 256 * it;
    uint4 v = make_uint4(0, 0, 0, 0);
    if (ci < C::XCH && t.xoff[it] >= 0) {
      const int ch = ci % (KT / 8);
      v = *(const uint4*)((const uint16_t*)x + t.xoff[it] + (int64_t)kt * KT + ch * 8);
    }
    st.x[it] = v;
  }
#pragma unroll
  for (int q = 0; q < C::NB; ++q) {
#pragma unroll
    for (int it = 0; it < C::CIT; ++it) {
      const int vi = tid + 256 * it;
      uint4 v = make_uint4(0, 0, 0, 0);
      if (vi < C::CVEC) {
        const int n = vi / (C::WPR / 4), c4 = vi % (C::WPR / 4);
        const int64_t row = t.n0 + n;
        if (row < t.N)
          v = *(const uint4*)(t.codes[q] + row * t.P + (int64_t)kt * C::WPR + c4 * 4);
      }
      st.c[q][it] = v;
    }
#pragma unroll
    for (int it = 0; it < C::SIT; ++it) {
      const int si = tid + 256 * it;
      float s = 0.f, b = 0.f;
      if (si < C::SCN) {
        const int n = si / C::GT, g = si % C::GT;
        const int64_t row = t.n0 + n;
        if (row < t.N) {
          const int64_t idx = row * t.G + (int64_t)kt * C::GT + g;
          s = load_as_f32(t.scales[q], idx, sb);
          b = load_as_f32(t.biases[q], idx, sb);
        }
      }
      st.s[q][it] = s;
      st.b[q][it] = b;
    }
  }
}

template <class C>
JQ_DEV void store_stage(const Stage<C>& st, Smem<C>& sm) {
  const int tid = threadIdx.x;
  constexpr uint32_t one2 = C::XDT == JQ_BF16 ? 0x3F803F80u : 0x3C003C00u;
  constexpr float off = C::NIB ? 272.f : (float)(1 << C::BITS);
#pragma unroll
  for (int it = 0; it < C::XIT; ++it) {
    const int ci = tid + 256 * it;
    const int r = ci / (KT / 8), ch = ci % (KT / 8);
    const uint32_t raw[4] = {st.x[it].x, st.x[it].y, st.x[it].z, st.x[it].w};
    uint32_t pr[4];
    pair_activations(raw, pr);
    float sum = dot2<C::XDT>(raw[0], one2, 0.f);
    sum = dot2<C::XDT>(raw[1], one2, sum);
    sum = dot2<C::XDT>(raw[2], one2, sum);
    sum = dot2<C::XDT>(raw[3], one2, sum);
    // Reduce over the GS/8 consecutive lanes (chunks) of one group.
#pragma unroll
    for (int o = 1; o < C::GS / 8; o <<= 1) sum += __shfl_xor(sum, o, 64);
    if (ci < C::XCH) {
      *(u32x4*)&sm.xs[r][ch * 4] = u32x4{pr[0], pr[1], pr[2], pr[3]};
      if ((ch % (C::GS / 8)) == 0) sm.xsum[ch / (C::GS / 8)][r] = sum;
    }
  }
#pragma unroll
  for (int q = 0; q < C::NB; ++q) {
#pragma unroll
    for (int it = 0; it < C::CIT; ++it) {
      const int vi = tid + 256 * it;
      if (vi < C::CVEC) {
        const int n = vi / (C::WPR / 4), c4 = vi % (C::WPR / 4);
        *(uint4*)&sm.ws[q][n][c4 * 4] = st.c[q][it];
      }
    }
#pragma unroll
    for (int it = 0; it < C::SIT; ++it) {
      const int si = tid + 256 * it;
      if (si < C::SCN) {
        const int n = si / C::GT, g = si % C::GT;
        sm.sc[q][g][n] = st.s[q][it];
        sm.cb[q][g][n] = fmaf(-off, st.s[q][it], st.b[q][it]);
      }
    }
  }
}

// B fragment of slice `slc` (32 codes) of LDS row `wr` for lane group lg: 4 magic pairs
// (or low/high nibble pairs for 8-bit codes with bf16 activations).
template <class C>
JQ_DEV void load_b(const uint32_t* wr, int slc, int lg, u32x4& b, u32x4& bh) {
  const uint32_t* u = wr + slc * C::BITS;
  if constexpr (C::NIB) {
    uint32_t lo[4], hi[4];
    chunk8_nibble_pairs(u[2 * lg], u[2 * lg + 1], lo, hi);
    b = u32x4{lo[0], lo[1], lo[2], lo[3]};
    bh = u32x4{hi[0], hi[1], hi[2], hi[3]};
  } else {
    const int off = 8 * C::BITS * lg;
    const int lo = off >> 5, sh = off & 31;
    const uint32_t w0 = u[lo], w1 = u[lo + 1];
    const uint32_t v = __builtin_amdgcn_alignbit(w1, w0, sh);
    uint32_t vh = 0;
    if constexpr (C::BITS > 4) vh = __builtin_amdgcn_alignbit(u[lo + 2], w1, sh);
    uint32_t pr[4];
    chunk_to_pairs<C::XDT, C::BITS>(v, vh, pr);
    b = u32x4{pr[0], pr[1], pr[2], pr[3]};
    bh = b;
  }
}

template <class C>
JQ_DEV void compute_tile(const Smem<C>& sm, f32x4 (&acc)[C::NB][C::FM][C::FN]) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int lr = lane & 15, lg = lane >> 4;
  const int mb = (wave / C::WGN) * C::WM, nb = (wave % C::WGN) * C::WN;
  const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int g = 0; g < C::GT; ++g) {
    u32x4 A[C::FM][C::SPG];
    f32x4 X[C::FM];
#pragma unroll
    for (int i = 0; i < C::FM; ++i) {
#pragma unroll
      for (int t = 0; t < C::SPG; ++t) {
        const int slc = g * C::SPG + t;
        A[i][t] = *(const u32x4*)&sm.xs[mb + 16 * i + lr][slc * 16 + lg * 4];
      }
      X[i] = *(const f32x4*)&sm.xsum[g][mb + 16 * i + 4 * lg];
    }
#pragma unroll
    for (int q = 0; q < C::NB; ++q)
#pragma unroll
    for (int j = 0; j < C::FN; ++j) {
      const int n = nb + 16 * j + lr;
      const float s = sm.sc[q][g][n], c = sm.cb[q][g][n];
      u32x4 B[C::SPG], BH[C::SPG];
#pragma unroll
      for (int t = 0; t < C::SPG; ++t) load_b<C>(sm.ws[q][n], g * C::SPG + t, lg, B[t], BH[t]);
#pragma unroll
      for (int i = 0; i < C::FM; ++i) {
        f32x4 part = mfma16<C::XDT>(A[i][0], B[0], zero);
#pragma unroll
        for (int t = 1; t < C::SPG; ++t) part = mfma16<C::XDT>(A[i][t], B[t], part);
        if constexpr (C::NIB) {
          f32x4 ph = mfma16<C::XDT>(A[i][0], BH[0], zero);
#pragma unroll
          for (int t = 1; t < C::SPG; ++t) ph = mfma16<C::XDT>(A[i][t], BH[t], ph);
#pragma unroll
          for (int r = 0; r < 4; ++r) part[r] = fmaf(16.f, ph[r], part[r]);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r)
          acc[q][i][j][r] = fmaf(s, part[r], fmaf(c, X[i][r], acc[q][i][j][r]));
      }
    }
  }
}

JQ_DEV void store_out(void* y, int64_t idx, float v, int yd) {
  if (yd == JQ_BF16) ((uint16_t*)y)[idx] = f32_to_bf16_bits(v);
  else if (yd == JQ_F16) ((uint16_t*)y)[idx] = f32_to_f16_bits(v);
  else ((float*)y)[idx] = v;
}

// Full K loop for one output tile; acc returned to the caller for the epilogue.
template <class C>
JQ_DEV void mainloop(const TileCtx<C>& t, const void* __restrict__ x, int nkt, int sb,
                     Smem<C>& sm, f32x4 (&acc)[C::NB][C::FM][C::FN]) {
#pragma unroll
  for (int q = 0; q < C::NB; ++q)
#pragma unroll
    for (int i = 0; i < C::FM; ++i)
#pragma unroll
      for (int j = 0; j < C::FN; ++j) acc[q][i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  Stage<C> st;
  load_stage<C>(t, x, 0, sb, st);
  for (int kt = 0; kt < nkt; ++kt) {
    __syncthreads();  // previous compute done before LDS is overwritten
    store_stage<C>(st, sm);
    __syncthreads();
    if (kt + 1 < nkt) load_stage<C>(t, x, kt + 1, sb, st);
    compute_tile<C>(sm, acc);
  }
}

template <class C>
__global__ void __launch_bounds__(256) qmm_dense_kernel(QmmProblem p, int sb, int yd) {
  __shared__ Smem<C> sm;
  TileCtx<C> t;
  const int64_t m0 = (int64_t)blockIdx.y * C::BM;
  t.n0 = (int64_t)blockIdx.x * C::BN;
  t.N = p.N;
  t.P = p.K * C::BITS / 32;
  t.G = p.K / C::GS;
  t.codes[0] = p.codes;
  t.scales[0] = p.scales;
  t.biases[0] = p.biases;
#pragma unroll
  for (int it = 0; it < C::XIT; ++it) {
    const int ci = threadIdx.x + 256 * it;
    const int64_t m = m0 + ci / (KT / 8);
    t.xoff[it] = (ci < C::XCH && m < p.M) ? m * p.K : -1;
  }
  f32x4 acc[C::NB][C::FM][C::FN];
  mainloop<C>(t, p.x, (int)(p.K / KT), sb, sm, acc);

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int lr = lane & 15, lg = lane >> 4;
  const int mb = (wave / C::WGN) * C::WM, nb = (wave % C::WGN) * C::WN;
#pragma unroll
  for (int i = 0; i < C::FM; ++i)
#pragma unroll
    for (int j = 0; j < C::FN; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t m = m0 + mb + 16 * i + 4 * lg + r;
        const int64_t n = t.n0 + nb + 16 * j + lr;
        if (m < p.M && n < p.N) store_out(p.y, m * p.N + n, acc[0][i][j][r], yd);
      }
}

// Value of v after rounding to dtype yd (the dtype a standalone projection would return).
JQ_DEV float round_to(float v, int yd) {
  if (yd == JQ_BF16) return bf16_bits_to_f32(f32_to_bf16_bits(v));
  if (yd == JQ_F16) return f16_bits_to_f32(f32_to_f16_bits(v));
  return v;
}

// silu(g) * u in fp32 (MLX nn.silu = x * sigmoid(x)).

// Grouped launch over expert segments. Persistent: block b handles items b, b+grid, ...
// item = (tile, n-block); tile = (expert, first row, rows) from the device plan.
// NB == 2: weight 0 = gate, weight 1 = up; the epilogue writes silu(gate) * up with both
// projections first rounded to yd, as two gather_qmm calls returning yd would give.
template <class C>
__global__ void __launch_bounds__(256) qmm_gather_kernel(QmmProblem p, QmmProblem p2,
                                                         GatherPlan plan, int sb, int yd) {
  __shared__ Smem<C> sm;
  const int64_t nblk = (p.N + C::BN - 1) / C::BN;
  const int64_t items = (int64_t)(*plan.n_tiles) * nblk;
  const int Mp = plan.M;
  const int esz = sb == JQ_F32 ? 4 : 2;
  for (int64_t item = blockIdx.x; item < items; item += gridDim.x) {
    const int4 tile = plan.tiles[item / nblk];
    const int e = tile.x, r0 = tile.y, rows = tile.z;
    const int seg = plan.seg_off[e];
    TileCtx<C> t;
    t.n0 = (item % nblk) * C::BN;
    t.N = p.N;
    t.P = p.K * C::BITS / 32;
    t.G = p.K / C::GS;
    const int64_t sboff = (int64_t)e * p.expert_stride_sb * esz;
    t.codes[0] = p.codes + (int64_t)e * p.expert_stride_codes;
    t.scales[0] = (const char*)p.scales + sboff;
    t.biases[0] = (const char*)p.biases + sboff;
    if constexpr (C::NB == 2) {
      t.codes[1] = p2.codes + (int64_t)e * p.expert_stride_codes;
      t.scales[1] = (const char*)p2.scales + sboff;
      t.biases[1] = (const char*)p2.biases + sboff;
    }
#pragma unroll
    for (int it = 0; it < C::XIT; ++it) {
      const int ci = threadIdx.x + 256 * it;
      const int r = ci / (KT / 8);
      int64_t off = -1;
      if (ci < C::XCH && r < rows) {
        const int rr = r0 + r;
        const uint32_t pair = plan.order[seg + rr / Mp];
        const int64_t xr =
            (int64_t)(plan.lhs ? plan.lhs[pair] : pair / plan.pair_div) * Mp + rr % Mp;
        off = xr < plan.x_rows ? xr * p.K : -1;
      }
      t.xoff[it] = off;
    }
    f32x4 acc[C::NB][C::FM][C::FN];
    mainloop<C>(t, p.x, (int)(p.K / KT), sb, sm, acc);

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int lr = lane & 15, lg = lane >> 4;
    const int mb = (wave / C::WGN) * C::WM, nb = (wave % C::WGN) * C::WN;
#pragma unroll
    for (int i = 0; i < C::FM; ++i)
#pragma unroll
      for (int rr4 = 0; rr4 < 4; ++rr4) {
        const int r = mb + 16 * i + 4 * lg + rr4;
        if (r < rows) {
          const int rr = r0 + r;
          const uint32_t pair = plan.order[seg + rr / Mp];
          const int64_t orow = (int64_t)pair * Mp + rr % Mp;
#pragma unroll
          for (int j = 0; j < C::FN; ++j) {
            const int64_t n = t.n0 + nb + 16 * j + lr;
            if (n < p.N) {
              float v = acc[0][i][j][rr4];
              if constexpr (C::NB == 2)
                v = jqk::glu_value(round_to(v, yd), round_to(acc[1][i][j][rr4], yd), p.glu_limit,
                                   p.glu_scale ? p.glu_scale[orow] : 1.f);
              store_out(p.y, orow * p.N + n, v, yd);
            }
          }
        }
      }
  }
}

// ----------------------------------------------------------------------------- dispatch

template <int BITS, int GS, int XDT>
int dense_bg(const QmmProblem& p, int sb, int yd, hipStream_t st) {
  if (p.M <= 16) {
    using C = Cfg<BITS, GS, 16, 64, 1, 4, XDT>;
    dim3 grid((unsigned)((p.N + C::BN - 1) / C::BN), (unsigned)((p.M + C::BM - 1) / C::BM));
    qmm_dense_kernel<C><<<grid, 256, 0, st>>>(p, sb, yd);
  } else if (p.M <= 64) {
    using C = Cfg<BITS, GS, 32, 128, 1, 4, XDT>;
    dim3 grid((unsigned)((p.N + C::BN - 1) / C::BN), (unsigned)((p.M + C::BM - 1) / C::BM));
    qmm_dense_kernel<C><<<grid, 256, 0, st>>>(p, sb, yd);
  } else {
    using C = Cfg<BITS, GS, 128, 128, 2, 2, XDT>;
    dim3 grid((unsigned)((p.N + C::BN - 1) / C::BN), (unsigned)((p.M + C::BM - 1) / C::BM));
    qmm_dense_kernel<C><<<grid, 256, 0, st>>>(p, sb, yd);
  }
  return jqh::launch_status();
}

template <int BITS, int GS, int XDT, int NB>
int gather_bg(const QmmProblem& p, const QmmProblem& p2, const GatherPlan& plan,
              int64_t max_tiles, int sb, int yd, hipStream_t st) {
  // Decode-sized segments: 16-row tiles, 64 columns per block.
  using C = Cfg<BITS, GS, 16, 64, 1, 4, XDT, NB>;
  const int64_t nblk = (p.N + C::BN - 1) / C::BN;
  const int64_t items = max_tiles * nblk;
  int64_t grid = items < 2048 ? items : 2048;
  if (grid < 1) grid = 1;
  qmm_gather_kernel<C><<<(unsigned)grid, 256, 0, st>>>(p, p2, plan, sb, yd);
  return jqh::launch_status();
}

template <int XDT>
int dense_x(int bits, int gs, const QmmProblem& p, int sb, int yd, hipStream_t st) {
#define JQ_GS(B)                                                   \
  switch (gs) {                                                    \
    case 32: return dense_bg<B, 32, XDT>(p, sb, yd, st);           \
    case 64: return dense_bg<B, 64, XDT>(p, sb, yd, st);           \
    default: return dense_bg<B, 128, XDT>(p, sb, yd, st);          \
  }
  switch (bits) {
    case 2: JQ_GS(2)
    case 3: JQ_GS(3)
    case 4: JQ_GS(4)
    case 5: JQ_GS(5)
    case 6: JQ_GS(6)
    default: JQ_GS(8)
  }
#undef JQ_GS
}

template <int XDT, int NB>
int gather_x(int bits, int gs, const QmmProblem& p, const QmmProblem& p2, const GatherPlan& plan,
             int64_t mt, int sb, int yd, hipStream_t st) {
#define JQ_GS(B)                                                                \
  switch (gs) {                                                                 \
    case 32: return gather_bg<B, 32, XDT, NB>(p, p2, plan, mt, sb, yd, st);     \
    case 64: return gather_bg<B, 64, XDT, NB>(p, p2, plan, mt, sb, yd, st);     \
    default: return gather_bg<B, 128, XDT, NB>(p, p2, plan, mt, sb, yd, st);    \
  }
  switch (bits) {
    case 2: JQ_GS(2)
    case 3: JQ_GS(3)
    case 4: JQ_GS(4)
    case 5: JQ_GS(5)
    case 6: JQ_GS(6)
    default: JQ_GS(8)
  }
#undef JQ_GS
}

}  // namespace

namespace jqk {

int qmm_launch(const QmmProblem& p, int bits, int gs, int xd, int sb, int yd, hipStream_t st) {
  if (p.M == 0 || p.N == 0) return JQ_OK;
  if (p.K % KT) return JQ_ERR_SHAPE;
  if (xd == JQ_BF16) return dense_x<JQ_BF16>(bits, gs, p, sb, yd, st);
  if (xd == JQ_F16) return dense_x<JQ_F16>(bits, gs, p, sb, yd, st);
  return JQ_ERR_DTYPE;
}

int qmm_gather_launch(const QmmProblem& p, const QmmProblem* p2, const GatherPlan& plan,
                      int64_t max_tiles, int bits, int gs, int xd, int sb, int yd,
                      hipStream_t st) {
  if (max_tiles == 0 || p.N == 0) return JQ_OK;
  if (p.K % KT) return JQ_ERR_SHAPE;
  if (p2) {
    if (xd == JQ_BF16) return gather_x<JQ_BF16, 2>(bits, gs, p, *p2, plan, max_tiles, sb, yd, st);
    if (xd == JQ_F16) return gather_x<JQ_F16, 2>(bits, gs, p, *p2, plan, max_tiles, sb, yd, st);
  } else {
    if (xd == JQ_BF16) return gather_x<JQ_BF16, 1>(bits, gs, p, p, plan, max_tiles, sb, yd, st);
    if (xd == JQ_F16) return gather_x<JQ_F16, 1>(bits, gs, p, p, plan, max_tiles, sb, yd, st);
  }
  return JQ_ERR_DTYPE;
}

}  // namespace jqk

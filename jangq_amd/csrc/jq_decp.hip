// Decode-batch quantized matmul on matrix cores, persistent: y = x @ deq(W)^T for a few
// activation rows (passes of up to 2 * 16/(128/gs) rows), one or several problems per launch.
//
// Arithmetic (jq_dec.h): lane (r = l%16, g = l/16) streams unit g of each 128-code step of W
// row r straight into v_mfma_f32_16x16x32 B fragments; the step's 128/gs groups are folded
// into the MFMA M dimension, so every accumulator slot belongs to one (token, group) and
// takes  acc += s_g * D + b_g * X  with D = sum q*x exactly (the per-group affine sum
// s * sum q x + b * sum x of jang-tools/jang_tools/dsv41/metal_decode.py:202-233).
//
// Structure (that of the vector-ALU GEMV, jq_gemv.hip). A block of KW waves splits K: wave w
// owns SW consecutive 128-code steps of every item (RT 16-row tiles of one problem). The
// pass's activations are staged once per block into LDS as ready A fragments, so the
// matrix loop reads them with LDS loads, which the vector-memory counter does not track.
// Blocks are persistent and walk items b, b + grid, ...; each lane holds the SW positions of
// its item in a register ring (codes, scales, biases), and position d of the next item is
// issued as soon as position d of the current one has been consumed, so a whole item of
// loads stays in flight through the reduction and the stores. Loads are consumed in the
// order they were issued and no branch separates a slot's use from its reload. At the end
// of an item each wave writes its folded partials to LDS (double-buffered); after one
// barrier the waves sum the KW partials, one output slot per wave in turn, and store them.
#include "jq_gemv.h"
#include "jq_qmv.h"

namespace {

using namespace jq;
using namespace jqd;
using jqg::Rsrc;
using jqg::make_rsrc;
using jqk::QmvBatch;
using jqk::QmvProblem;

constexpr int kMaxKW = 8;                 // 512 threads: up to 256 VGPRs per wave
constexpr int kXLdsMax = 140 * 1024;      // activation bytes staged per pass (LDS)
constexpr int kTokStride = 4 * 64 + 16;   // LDS bytes per (step, token): 4 lane groups + pad

struct DecpArgs {
  QmvBatch b;
  int rb_begin[jqk::kMaxProblems + 1];  // first item of each problem
  int nprob;
  int m0;        // first activation row of this pass
  int mrows;     // activation rows of this pass (<= NA * TPB)
  int yd;
};

JQ_DEV void store_out(void* y, int64_t idx, float v, int yd) {
  if (yd == JQ_BF16) ((uint16_t*)y)[idx] = f32_to_bf16_bits(v);
  else if (yd == JQ_F16) ((uint16_t*)y)[idx] = f32_to_f16_bits(v);
  else ((float*)y)[idx] = v;
}

// One position of a lane's ring: the unit of codes and the step's scale / bias words of
// each of the item's RT tiles.
template <class D, int RT>
struct Slot {
  uint32_t c[RT][D::BITS];
  uint32_t s[RT][(D::GSTEP + 1) / 2], b[RT][(D::GSTEP + 1) / 2];
};

template <int GSTEP>
JQ_DEV void load_sb(Rsrc r, uint32_t voff, uint32_t* w) {
  if constexpr (GSTEP == 1) {
    w[0] = __builtin_amdgcn_raw_buffer_load_b16(r, voff, 0, 0);
  } else if constexpr (GSTEP == 2) {
    w[0] = __builtin_amdgcn_raw_buffer_load_b32(r, voff, 0, 0);
  } else {
    const jqg::u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(r, voff, 0, 0);
    w[0] = v[0];
    w[1] = v[1];
  }
}

// MFMAs and scale terms of one position: RT tiles x NA activation blocks.
template <class D, int SB, int RT, int NA>
JQ_DEV void compute_pos(const Slot<D, RT>& st, const u32x4 (&A)[NA][4], const Bases<D>& bs,
                        f32x4 (&acc)[NA][RT]) {
  const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
  const u32x4 ones = {D::ONE2, D::ONE2, D::ONE2, D::ONE2};
  constexpr u32x4 BO0 = {bo_dword<D>(0, 0), bo_dword<D>(0, 1), bo_dword<D>(0, 2), bo_dword<D>(0, 3)};
  constexpr u32x4 BO1 = {bo_dword<D>(1, 0), bo_dword<D>(1, 1), bo_dword<D>(1, 2), bo_dword<D>(1, 3)};
  constexpr u32x4 BO2 = {bo_dword<D>(2, 0), bo_dword<D>(2, 1), bo_dword<D>(2, 2), bo_dword<D>(2, 3)};
  constexpr u32x4 BO3 = {bo_dword<D>(3, 0), bo_dword<D>(3, 1), bo_dword<D>(3, 2), bo_dword<D>(3, 3)};
  f32x4 X[NA], O[NA];
#pragma unroll
  for (int a = 0; a < NA; ++a) {
    X[a] = mfma16<D::XDT>(A[a][0], ones, zero);
    X[a] = mfma16<D::XDT>(A[a][1], ones, X[a]);
    X[a] = mfma16<D::XDT>(A[a][2], ones, X[a]);
    X[a] = mfma16<D::XDT>(A[a][3], ones, X[a]);
    O[a] = mfma16<D::XDT>(A[a][0], BO0, zero);
    O[a] = mfma16<D::XDT>(A[a][1], BO1, O[a]);
    O[a] = mfma16<D::XDT>(A[a][2], BO2, O[a]);
    O[a] = mfma16<D::XDT>(A[a][3], BO3, O[a]);
  }
#pragma unroll
  for (int r = 0; r < RT; ++r) {
    const uint32_t* w = st.c[r];
    f32x4 Dd[NA], Dh[NA];
#pragma unroll
    for (int a = 0; a < NA; ++a) { Dd[a] = O[a]; Dh[a] = zero; }
#define JQ_F(F)                                                            \
    {                                                                      \
      u32x4 B, BH;                                                         \
      b_frag<D, F>(w, bs, B, BH);                                          \
      _Pragma("unroll") for (int a = 0; a < NA; ++a) {                     \
        Dd[a] = mfma16<D::XDT>(A[a][F], B, Dd[a]);                         \
        if constexpr (D::NIB) Dh[a] = mfma16<D::XDT>(A[a][F], BH, Dh[a]);  \
      }                                                                    \
    }
    JQ_F(0) JQ_F(1) JQ_F(2) JQ_F(3)
#undef JQ_F
    float sc[4], bi[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int j = i % D::GSTEP;
      sc[i] = half_to_f32<SB>(st.s[r][j >> 1], j & 1);
      bi[i] = half_to_f32<SB>(st.b[r][j >> 1], j & 1);
    }
#pragma unroll
    for (int a = 0; a < NA; ++a)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float d = D::NIB ? fmaf(16.f, Dh[a][i], Dd[a][i]) : Dd[a][i];
        acc[a][r][i] = fmaf(sc[i], d, fmaf(bi[i], X[a][i], acc[a][r][i]));
      }
  }
}

// LDS layout: [zero fragment: 64 B][x: S steps x mrows tokens x kTokStride B]
// [partials: 2 x KW x NOUT x 64 floats]. The 64 B at (s, t) + 64 g are the four A fragments
// of lane group g for token t at step s (jq_dec.h a_frag order); the 16 B pad per (s, t)
// puts the tokens that one LDS read serves in different banks.
template <class D, int SB, int RT, int NA, int SW>
__global__ void __launch_bounds__(64 * kMaxKW) decp_kernel(DecpArgs a) {
  constexpr int BITS = D::BITS, TPB = D::TPB, TPL = 4 / D::GSTEP;
  constexpr int MP = NA * TPB;          // activation rows of a pass
  constexpr int NOUT = RT * NA * TPL;   // partial outputs per lane per item
  constexpr int SBW = (D::GSTEP + 1) / 2;
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];

  const int total = a.rb_begin[a.nprob];
  int it = blockIdx.x;
  if (it >= total) return;  // whole block
  const int KW = blockDim.x >> 6;
  const int K = a.b.K;
  const int S = K / 128;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lr = lane & 15, lg = lane >> 4;
  const uint32_t rowbytes = (uint32_t)(K / 32) * BITS * 4;
  const uint32_t sbrow = (uint32_t)(K / D::GS) * 2;
  const int mp = a.mrows;  // staged activation rows (<= MP)
  u32x4* zfrag = (u32x4*)lds;
  uint8_t* xs = lds + 64;
  float* red = (float*)(lds + 64 + (size_t)S * mp * kTokStride);

  // LDS byte offset of this lane's fragments for activation block ab at step 0 (-1: the
  // lane feeds no activation and reads the zero fragment).
  int xbase[NA];
#pragma unroll
  for (int ab = 0; ab < NA; ++ab) {
    const int t = ab * TPB + lr / D::GSTEP;
    const bool act = (lr % D::GSTEP) == lg / D::LPG && t < a.mrows;
    xbase[ab] = act ? t * kTokStride + lg * 64 : -1;
  }
  const int s0 = wave * SW;

  auto locate = [&](int item, int& p, int64_t& row0) {
    p = 0;
#pragma unroll
    for (int q = 1; q < jqk::kMaxProblems; ++q)
      if (q < a.nprob && item >= a.rb_begin[q]) p = q;
    row0 = (int64_t)(item - a.rb_begin[p]) * (16 * RT);
  };
  // Buffer views of an item's codes / scales / biases rows (rows past N and dead items read
  // zero without touching memory).
  auto views = [&](int p, int64_t row0, bool live, Rsrc& rc, Rsrc& rs, Rsrc& rb) {
    const QmvProblem& pb = a.b.p[p];
    const int64_t left = pb.N - row0;
    const uint32_t rows = live ? (uint32_t)(left < 16 * RT ? left : 16 * RT) : 0u;
    rc = make_rsrc((const char*)pb.codes + row0 * rowbytes, rows * rowbytes);
    rs = make_rsrc((const char*)pb.scales + row0 * sbrow, rows * sbrow);
    rb = make_rsrc((const char*)pb.biases + row0 * sbrow, rows * sbrow);
  };
  auto load_slot = [&](Rsrc rc, Rsrc rs, Rsrc rb, int d, Slot<D, RT>& sl) {
    const int s = s0 + d < S ? s0 + d : S - 1;
#pragma unroll
    for (int r = 0; r < RT; ++r) {
      const uint32_t row = (uint32_t)(16 * r + lr);
      jqg::load_chunk<BITS>(rc, row * rowbytes + (uint32_t)(s * 4 + lg) * BITS * 4, sl.c[r]);
      const uint32_t so = row * sbrow + (uint32_t)s * D::GSTEP * 2;
      load_sb<D::GSTEP>(rs, so, sl.s[r]);
      load_sb<D::GSTEP>(rb, so, sl.b[r]);
    }
  };

  int p;
  int64_t row0;
  locate(it, p, row0);
  Rsrc rc, rs, rbv;
  views(p, row0, true, rc, rs, rbv);
  Slot<D, RT> ring[SW];
#pragma unroll
  for (int d = 0; d < SW; ++d) {
    load_slot(rc, rs, rbv, d, ring[d]);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
  }

  // Stage the pass's activations (every problem of a launch shares them) as A fragments,
  // while the first item's codes are in flight: four slots' loads are issued per round.
  {
    const uint16_t* x = (const uint16_t*)a.b.p[0].x;
    const int slots = S * mp * 4;
    if (threadIdx.x < 4) zfrag[threadIdx.x] = u32x4{0u, 0u, 0u, 0u};
    for (int i0 = threadIdx.x; i0 < slots; i0 += 4 * blockDim.x) {
      XRaw r[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        int i = i0 + u * (int)blockDim.x;
        i = i < slots ? i : slots - 1;
        const int g = i & 3, t = (i >> 2) % mp, s = (i >> 2) / mp;
        load_xraw(x + (int64_t)(a.m0 + t) * K + s * 128 + 32 * g, r[u]);
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int i = i0 + u * (int)blockDim.x;
        if (i < slots) {
          const int g = i & 3, t = (i >> 2) % mp, s = (i >> 2) / mp;
          u32x4* dst = (u32x4*)(xs + (size_t)(s * mp + t) * kTokStride + g * 64);
          dst[0] = a_frag<D, 0>(r[u]);
          dst[1] = a_frag<D, 1>(r[u]);
          dst[2] = a_frag<D, 2>(r[u]);
          dst[3] = a_frag<D, 3>(r[u]);
        }
      }
    }
    __syncthreads();
  }
  const Bases<D> bs = make_bases<D>();

  for (int par = 0;; par ^= 1) {
    const int nx = it + gridDim.x;
    const bool more = nx < total;
    int p2;
    int64_t row02;
    locate(more ? nx : it, p2, row02);
    Rsrc rc2, rs2, rb2;
    views(p2, row02, more, rc2, rs2, rb2);

    f32x4 acc[NA][RT];
#pragma unroll
    for (int ab = 0; ab < NA; ++ab)
#pragma unroll
      for (int r = 0; r < RT; ++r) acc[ab][r] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int d = 0; d < SW; ++d) {
      const int s = s0 + d;
      u32x4 A[NA][4];
#pragma unroll
      for (int ab = 0; ab < NA; ++ab) {
        const u32x4* f = (xbase[ab] >= 0 && s < S)
                             ? (const u32x4*)(xs + (size_t)s * mp * kTokStride + xbase[ab])
                             : zfrag;
        A[ab][0] = f[0];
        A[ab][1] = f[1];
        A[ab][2] = f[2];
        A[ab][3] = f[3];
      }
      compute_pos<D, SB, RT, NA>(ring[d], A, bs, acc);
      // The slot is consumed before it is reloaded (results first, then memory), so it keeps
      // its registers across the loop.
#pragma unroll
      for (int ab = 0; ab < NA; ++ab)
#pragma unroll
        for (int r = 0; r < RT; ++r) asm volatile("" : "+v"(acc[ab][r])::"memory");
      load_slot(rc2, rs2, rb2, d, ring[d]);
      __builtin_amdgcn_sched_barrier(0);
    }

    float* mine = red + ((size_t)(par * KW + wave) * NOUT) * 64;
#pragma unroll
    for (int ab = 0; ab < NA; ++ab)
#pragma unroll
      for (int r = 0; r < RT; ++r) {
        float v[TPL];
        fold_groups<D>(acc[ab][r], v);
#pragma unroll
        for (int k = 0; k < TPL; ++k) mine[((ab * RT + r) * TPL + k) * 64 + lane] = v[k];
      }
    __syncthreads();
    {
      const QmvProblem& pb = a.b.p[p];
      for (int o = wave; o < NOUT; o += KW) {
        float v = 0.f;
        for (int w = 0; w < KW; ++w) v += red[((size_t)(par * KW + w) * NOUT + o) * 64 + lane];
        const int k = o % TPL, r = (o / TPL) % RT, ab = o / (TPL * RT);
        const int tok = ab * TPB + TPL * lg + k;
        const int64_t n = row0 + 16 * r + lr;
        if (tok < a.mrows && n < pb.N) store_out(pb.y, (int64_t)(a.m0 + tok) * pb.N + n, v, a.yd);
      }
    }
    if (!more) break;
    it = nx;
    p = p2;
    row0 = row02;
  }
  (void)SBW;
}

template <class D, int SB, int RT, int NA, int SW>
int launch_cfg(DecpArgs& a, int kw, hipStream_t st) {
  constexpr int TPL = 4 / D::GSTEP;
  int total = 0;
  for (int i = 0; i < a.nprob; ++i) {
    a.rb_begin[i] = total;
    total += (int)((a.b.p[i].N + 16 * RT - 1) / (16 * RT));
  }
  for (int i = a.nprob; i <= jqk::kMaxProblems; ++i) a.rb_begin[i] = total;
  if (total == 0) return JQ_OK;
  const int S = a.b.K / 128;
  const size_t lds =
      64 + (size_t)S * a.mrows * kTokStride + (size_t)2 * kw * RT * NA * TPL * 64 * 4;
  auto kern = decp_kernel<D, SB, RT, NA, SW>;
  if (!jqh::set_lds((const void*)kern, lds)) return JQ_ERR_LAUNCH;
  const int64_t cap = (int64_t)jqh::blocks_per_cu((const void*)kern, 64 * kw, lds) * jqh::cus();
  const int64_t iters = (total + cap - 1) / cap;
  const int grid = (int)((total + iters - 1) / iters);
  kern<<<grid, 64 * kw, lds, st>>>(a);
  return jqh::launch_status();
}

// Steps per wave SW (the ring depth, one item): 4, 8 or 16, the smallest for which at most
// kMaxKW waves cover K.
template <class D, int SB, int RT, int NA>
int launch_sw(DecpArgs& a, hipStream_t st) {
  const int S = a.b.K / 128;
  if (S <= 4 * kMaxKW) return launch_cfg<D, SB, RT, NA, 4>(a, (S + 3) / 4, st);
  if (S <= 8 * kMaxKW) return launch_cfg<D, SB, RT, NA, 8>(a, (S + 7) / 8, st);
  return launch_cfg<D, SB, RT, NA, 16>(a, (S + 15) / 16, st);
}

template <int BITS, int GS, int XDT, int SB>
int launch_t(const QmvBatch& b, int nprob, int yd, hipStream_t st) {
  using D = Dc<BITS, GS, XDT>;
  int64_t rows = 0;
  for (int i = 0; i < nprob; ++i) rows += b.p[i].N;
  const int64_t tiles = (rows + 15) / 16;
  // Rows per pass: two activation blocks when their fragments fit the LDS budget.
  const int64_t xrow = (int64_t)(b.K / 128) * kTokStride;  // LDS bytes per activation row
  const bool two = b.M > D::TPB && 2 * D::TPB * xrow <= kXLdsMax;
  const int pass = two ? 2 * D::TPB : D::TPB * xrow <= kXLdsMax ? D::TPB : (int)(kXLdsMax / xrow);
  if (pass < 1) return JQ_ERR_SHAPE;
  for (int m0 = 0; m0 < b.M; m0 += pass) {
    DecpArgs a;
    a.b = b;
    a.nprob = nprob;
    a.m0 = m0;
    a.mrows = b.M - m0 < pass ? b.M - m0 : pass;
    a.yd = yd;
    int s;
    const bool big = tiles >= 1024 && D::BITS <= 4 && b.K / 128 <= 4 * kMaxKW;
    if (two) s = launch_sw<D, SB, 1, 2>(a, st);
    else if (big) s = launch_sw<D, SB, 2, 1>(a, st);
    else s = launch_sw<D, SB, 1, 1>(a, st);
    if (s) return s;
  }
  return JQ_OK;
}

template <int XDT, int SB>
int launch_bits(int bits, int gs, const QmvBatch& b, int nprob, int yd, hipStream_t st) {
#define JQ_D(B)                                                      \
  switch (gs) {                                                      \
    case 32: return launch_t<B, 32, XDT, SB>(b, nprob, yd, st);      \
    case 64: return launch_t<B, 64, XDT, SB>(b, nprob, yd, st);      \
    default: return launch_t<B, 128, XDT, SB>(b, nprob, yd, st);     \
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

}  // namespace

namespace jqk {

bool decp_ok(int M, int64_t K, int64_t maxN, int xd, int sb) {
  // K up to 16 steps x kMaxKW waves x 128 codes; 32-bit buffer offsets inside a tile.
  return M >= 1 && K % 128 == 0 && K > 0 && K <= 16 * kMaxKW * 128 &&
         (xd == JQ_BF16 || xd == JQ_F16) && (sb == JQ_BF16 || sb == JQ_F16) &&
         maxN < ((int64_t)1 << 30);
}

int decp_launch(const QmvBatch& b, int nprob, int bits, int gs, int xd, int sb, int yd,
                hipStream_t st) {
  int64_t maxN = 0;
  for (int i = 0; i < nprob; ++i) maxN = b.p[i].N > maxN ? b.p[i].N : maxN;
  if (maxN == 0 || b.M == 0) return JQ_OK;
  if (!decp_ok(b.M, b.K, maxN, xd, sb)) return JQ_ERR_SHAPE;
  // The staged activations are those of problem 0: every problem must share them.
  for (int i = 1; i < nprob; ++i) {
    if (b.p[i].x != b.p[0].x) {
      for (int j = 0; j < nprob; ++j) {
        QmvBatch one = b;
        one.p[0] = b.p[j];
        const int s = decp_launch(one, 1, bits, gs, xd, sb, yd, st);
        if (s) return s;
      }
      return JQ_OK;
    }
  }
  if (xd == JQ_BF16) {
    return sb == JQ_BF16 ? launch_bits<JQ_BF16, JQ_BF16>(bits, gs, b, nprob, yd, st)
                         : launch_bits<JQ_BF16, JQ_F16>(bits, gs, b, nprob, yd, st);
  }
  return sb == JQ_BF16 ? launch_bits<JQ_F16, JQ_BF16>(bits, gs, b, nprob, yd, st)
                       : launch_bits<JQ_F16, JQ_F16>(bits, gs, b, nprob, yd, st);
}

}  // namespace jqk

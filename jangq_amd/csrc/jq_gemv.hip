// Decode GEMV on the vector ALUs: y[m, n] = sum_k x[m, k] * (q[n,k] * s[n,k/gs] + b[n,k/gs])
// for a few activation rows (M <= 4; M <= 2 at 2 bits), bf16 or f16 activations, K up to 512
// lane chunks. No matrix cores.
//
// Work split. A block of KW waves works on row blocks of RB consecutive output rows. A row's
// packed codes are cut into lane chunks of UPL whole 32-code units (UPL = 2 for 2-bit, so that
// every chunk is 16 bytes; 1 otherwise: 12, 16, 20, 24 or 32 bytes). Wave w takes a contiguous
// range of chunks and lane l chunk l of that range, so each load instruction of a wave reads
// one contiguous run of a row (buffer loads of 16 / 12 / 8 bytes per lane), and the lane's K
// slice is the same for every row.
//
// For one activation row whose rows take at most two waves of chunks, gemv_row_kernel instead
// gives each wave whole rows (a lane takes chunks l, l + 64): one DPP sum per row, no LDS.
//
// Activation-stationary and persistent. Blocks stay resident and walk row blocks b,
// b + gridDim.x, ...; a lane loads its K slice of x once and keeps it in registers in the
// pairing the code unpack produces, with two per-unit constants, X = sum x and
// O = -sum offset_k x_k. The codes, scales and biases of the RB rows live in a rolling
// register ring: row r of the next row block is issued as soon as row r of the current one
// has been consumed, so RB rows of loads stay in flight through the reduction and the store.
//
// Arithmetic. Codes become exact 16-bit floats (offset_k + q_k) with mask-and-or only (the
// per-code offset schedules for bf16 2/3/4-bit, the uniform 2^bits offset otherwise; 8-bit bf16
// splits into two nibbles); v_dot2_f32_{bf16,f16} multiplies them with the activation pairs.
// Per unit and row:  acc += s * (D + O) + b * X  with D the dot product of the exact values,
// i.e. the reference's  s * sum q x + b * sum x  (jang-tools/jang_tools/dsv41/metal_decode.py:202-233).
// Accumulation is fp32. Each (row, token) partial is summed over the wave with DPP row
// operations and over the block's waves through LDS.
#include "jq_gemv.h"
#include "jq_gemv_row.h"
#include "jq_qmv.h"

namespace {

using namespace jq;
using namespace jqg;
using jqk::QmvBatch;
using jqk::QmvProblem;


// Persistent: block b handles row blocks b, b + gridDim.x, ... Each lane keeps a rolling
// ring of the RB rows of its current row block in registers; row r of the next row block is
// issued right after row r of the current one has been consumed, so RB rows of loads stay in
// flight while the block computes, reduces and stores.
// UPL_: units per lane chunk (0: units_per_chunk; 1 for long 2-bit rows, so that the row's
// 32-code units spread over twice the waves).
template <class D, int SB, int MT, int RB, int UPL_ = 0>
__global__ void __launch_bounds__(64 * kMaxWaves) gemv_kernel(GemvArgs a) {
  constexpr int BITS = D::BITS;
  constexpr int UPL = UPL_ ? UPL_ : units_per_chunk<BITS>();
  constexpr int NW = BITS * UPL;
  __shared__ float red[2][kMaxWaves][RB * MT];

  const int total = a.rb_begin[a.nprob];
  int it = blockIdx.x;
  if (it >= total) return;  // whole block
  const int KW = blockDim.x >> 6;
  const int K = a.b.K, M = a.b.M;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int C = K / (32 * UPL);                       // chunks per row
  const int CW = (C + KW - 1) >> a.kwshift;           // chunks per wave
  const uint32_t rowbytes = (uint32_t)(K / 32) * BITS * 4;
  const uint32_t sbrow = (uint32_t)(K >> (a.ushift + 5)) * 2;

  const int c = wave * CW + lane;
  const bool act = lane < CW && c < C;
  const int ci = act ? c : 0;
  const uint32_t voff = (uint32_t)ci * (4 * NW);
  uint32_t vsb[UPL];
#pragma unroll
  for (int t = 0; t < UPL; ++t) vsb[t] = (uint32_t)((ci * UPL + t) >> a.ushift) * 2;

  // Activations first (waiting for them does not wait for the codes).
  jqd::XRaw xr[UPL][MT];
#pragma unroll
  for (int t = 0; t < UPL; ++t)
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      const int mm = m < M ? m : M - 1;
      jqd::load_xraw((const uint16_t*)a.b.p[0].x + (int64_t)mm * K + (int64_t)(ci * UPL + t) * 32,
                     xr[t][m]);
    }

  // Row block `i`: its problem, first row and buffer views of its RB rows (rows past the
  // problem's end read zero).
  auto locate = [&](int i, int& p, int64_t& row0) {
    p = 0;
#pragma unroll
    for (int q = 1; q < jqk::kMaxProblems; ++q)
      if (q < a.nprob && i >= a.rb_begin[q]) p = q;
    row0 = (int64_t)(i - a.rb_begin[p]) * RB;
  };
  auto views = [&](int p, int64_t row0, bool live, Rsrc& rc, Rsrc& rs, Rsrc& rb) {
    const QmvProblem& pb = a.b.p[p];
    const int64_t left = pb.N - row0;
    const uint32_t rows = live ? (uint32_t)(left < RB ? left : RB) : 0u;
    rc = make_rsrc((const char*)pb.codes + row0 * rowbytes, rows * rowbytes);
    rs = make_rsrc((const char*)pb.scales + row0 * sbrow, rows * sbrow);
    rb = make_rsrc((const char*)pb.biases + row0 * sbrow, rows * sbrow);
  };
  auto load_row = [&](Rsrc rc, Rsrc rs, Rsrc rb, int r, RowSlot<NW, UPL>& slot) {
    load_chunk<NW>(rc, voff + r * rowbytes, slot.w);
    load_sb<D>(rs, rb, vsb, r * sbrow, slot);
  };

  int p;
  int64_t row0;
  locate(it, p, row0);
  Rsrc rc, rs, rbv;
  views(p, row0, true, rc, rs, rbv);
  RowSlot<NW, UPL> ring[RB];
#pragma unroll
  for (int r = 0; r < RB; ++r) {
    load_row(rc, rs, rbv, r, ring[r]);
    // Keep the issue order row by row, as in the loop below: the wait counts at the loop
    // head are the worse of the two orders.
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
  }

  XState xs[UPL][MT];
#pragma unroll
  for (int t = 0; t < UPL; ++t)
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      jqd::XRaw& r = xr[t][m];
      const bool live = act && m < M;
#pragma unroll
      for (int i = 0; i < 16; ++i) r.d[i] = live ? r.d[i] : 0u;
      make_xstate<D>(r, xs[t][m]);
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

    float acc[RB][MT];
#pragma unroll
    for (int r = 0; r < RB; ++r) {
#pragma unroll
      for (int m = 0; m < MT; ++m) acc[r][m] = 0.f;
#pragma unroll
      for (int t = 0; t < UPL; ++t) {
        const float sv = sb_to_f32<SB>(ring[r].s[t]);
        const float bv = sb_to_f32<SB>(ring[r].b[t]);
#pragma unroll
        for (int m = 0; m < MT; ++m) {
          const float d = unit_dot<D>(ring[r].w + t * BITS, bs, xs[t][m]);
          acc[r][m] = fmaf(sv, d + xs[t][m].O, fmaf(bv, xs[t][m].X, acc[r][m]));
        }
      }
      // Row r is consumed before its slot is reloaded (compiler barrier: the row's results
      // first, then memory). The slot thus keeps its registers across the loop; a reload
      // hoisted above the use would need a second ring and a full wait to copy it back.
#pragma unroll
      for (int m = 0; m < MT; ++m) asm volatile("" : "+v"(acc[r][m])::"memory");
      load_row(rc2, rs2, rb2, r, ring[r]);
      __builtin_amdgcn_sched_barrier(0);
    }

#pragma unroll
    for (int r = 0; r < RB; ++r)
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        const float v = wave_total_lane63(acc[r][m]);
        if (lane == 63) red[par][wave][r * MT + m] = v;
      }
    __syncthreads();
    if (wave == 0 && lane < RB * MT) {
      float v = 0.f;
      for (int w = 0; w < KW; ++w) v += red[par][w][lane];
      const int r = lane / MT, m = lane % MT;
      const QmvProblem& pb = a.b.p[p];
      const int64_t row = row0 + r;
      if (row < pb.N && m < M) {
        const int64_t o = (int64_t)m * pb.N + row;
        if (a.yd == JQ_BF16) store_t<JQ_BF16>(pb.y, o, v);
        else if (a.yd == JQ_F16) store_t<JQ_F16>(pb.y, o, v);
        else store_t<JQ_F32>(pb.y, o, v);
      }
    }
    if (!more) break;
    it = nx;
    p = p2;
    row0 = row02;
  }
}

template <class D, int SB, int CPL, int RB, bool GLU = false, bool SHARE = false>
__global__ void __launch_bounds__(256) gemv_row_kernel(GemvArgs a) {
  static_assert(CPL * 64 * row_upl<D::BITS>() <= 256, "one unit of x per thread");
  gemv_row_body<D, SB, CPL, RB, GLU, RowStore, SHARE>(
      a, __builtin_amdgcn_readfirstlane((int)blockIdx.x * 4 + (int)(threadIdx.x >> 6)),
      (int)gridDim.x * 4, RowStore());
}

template <class D, int SB, int CPL, int RB, bool GLU = false>
int launch_row(GemvArgs& a, hipStream_t st) {
  a.kwshift = 0;
  int total = 0;
  if constexpr (GLU) {  // items are rows of the pair
    total = (int)a.b.p[0].N;
    a.rb_begin[0] = 0;
    for (int i = 1; i <= jqk::kMaxProblems; ++i) a.rb_begin[i] = total;
  } else {
    for (int i = 0; i < a.nprob; ++i) {
      a.rb_begin[i] = total;
      total += (int)((a.b.p[i].N + RB - 1) / RB);
    }
    for (int i = a.nprob; i <= jqk::kMaxProblems; ++i) a.rb_begin[i] = total;
  }
  if (total == 0) return JQ_OK;
  // Waves (all resident at once) and items per wave for one form of the kernel.
  auto shape = [&](auto kern, int64_t& waves, int64_t& iters) {
    const int64_t cap = (int64_t)jqh::blocks_per_cu((const void*)kern, 256, 0) * jqh::cus() * 4;
    iters = (total + cap - 1) / cap;
    waves = (total + iters - 1) / iters;
  };
  // Waves with several items build the activation state once per block (measured at config 2:
  // gate|up, 3 items per wave, 13.0 -> 12.6 us); with one item per wave the barrier is only
  // latency (q|k|v, o and config 1 each 0.1-0.2 us slower), so every wave builds its own,
  // except for the f16-rescaled 8-bit units, whose state costs about twice as much to build
  // (config-5 8-bit attention T=1 14.5 -> 14.1 us, the config-5 layer T=1 41.3 -> 40.7 us).
  int64_t waves = 0, iters = 0;
  shape(gemv_row_kernel<D, SB, CPL, RB, GLU, false>, waves, iters);
  if (iters >= 2 || D::F16X) {
    shape(gemv_row_kernel<D, SB, CPL, RB, GLU, true>, waves, iters);
    gemv_row_kernel<D, SB, CPL, RB, GLU, true><<<(unsigned)((waves + 3) / 4), 256, 0, st>>>(a);
  } else {
    gemv_row_kernel<D, SB, CPL, RB, GLU, false><<<(unsigned)((waves + 3) / 4), 256, 0, st>>>(a);
  }
  return jqh::launch_status();
}

// Grid: as many blocks as fit the GPU at once, but no more than there are row blocks, with
// the row blocks spread evenly (every block takes the same number, up to one).
template <class D, int SB, int MT, int RB, int UPL_ = 0>
int launch_rb(GemvArgs& a, hipStream_t st) {
  int kws = 0;
  const int kw = UPL_ ? gemv_waves_upl(a.b.K, UPL_, &kws) : gemv_waves(a.b.K, D::BITS, &kws);
  if (kw > kMaxWaves) return JQ_ERR_SHAPE;
  a.kwshift = kws;
  int total = 0;
  for (int i = 0; i < a.nprob; ++i) {
    a.rb_begin[i] = total;
    total += (int)((a.b.p[i].N + RB - 1) / RB);
  }
  for (int i = a.nprob; i <= jqk::kMaxProblems; ++i) a.rb_begin[i] = total;
  if (total == 0) return JQ_OK;
  const int64_t cap =
      (int64_t)jqh::blocks_per_cu((const void*)gemv_kernel<D, SB, MT, RB, UPL_>, 64 * kw, 0) *
      jqh::cus();
  const int64_t iters = (total + cap - 1) / cap;
  const int grid = (int)((total + iters - 1) / iters);
  gemv_kernel<D, SB, MT, RB, UPL_><<<grid, 64 * kw, 0, st>>>(a);
  return jqh::launch_status();
}

// Rows per block (the ring depth). Measured on MI355X: long rows (four or more waves, e.g. a
// 14336-wide down projection) do best in gemv_kernel with 16 rows; M = 2, 4 take 4 rows
// (registers: 18 per unit and token go to x). One activation row with rows of at most two
// waves of chunks runs gemv_row_kernel (whole rows per wave, 2 rows in flight), measured
// against gemv_kernel: 4096 x 4096 4-bit 5.48 -> 5.03 us, config-2 q|k|v (6-bit) 7.40 ->
// 7.02 us, o 5.96 -> 5.83 us, gate|up (3-bit) 13.98 -> 13.69 us; with 4 or 8 rows in flight
// it was slower, and so were long rows (the down projection 9.12 -> 10.54 us). Outputs of at
// most kFewRows rows take one row per item: an 8-bit 128- or 512-expert router at K = 4096
// 4.3 -> 3.6 us (at 4096 rows one row per item was slower, 5.2 -> 5.7 us).
constexpr int64_t kFewRows = 1024;
constexpr int64_t kLongFewRows = 16384;
template <class D, int SB>
int launch_m(GemvArgs& a, hipStream_t st) {
  constexpr bool two = D::BITS == 2;  // two units per lane chunk
  const int kw = gemv_waves(a.b.K, D::BITS, nullptr);
  if (a.b.M == 1) {
    // Long 2-bit rows of a short output (config 2's down projection, 4096 x 14336): one
    // 32-code unit per lane chunk, so the row spreads over twice the waves (8 per block, two
    // per SIMD instead of one), 8 rows per block: 8.8 -> 8.0 us. With many rows the extra
    // load instructions per byte cost more than the second wave gains (57344 rows: 61 -> 71 us).
    if constexpr (two)
      if (kw >= 4 && gemv_waves_upl(a.b.K, 1, nullptr) <= kMaxWaves) {
        int64_t rows = 0;
        for (int i = 0; i < a.nprob; ++i) rows += a.b.p[i].N;
        if (rows <= kLongFewRows) return launch_rb<D, SB, 1, 8, 1>(a, st);
      }
    if (kw >= 4) return launch_rb<D, SB, 1, 16>(a, st);
    int64_t rows = 0;
    for (int i = 0; i < a.nprob; ++i) rows += a.b.p[i].N;
    const int cpl = row_cpl(a.b.K, D::BITS);
    using DR = typename RowD<D>::type;
    if (rows <= kFewRows) {  // short outputs (routers): one row per item, twice the waves
      if (cpl == 1) return launch_row<DR, SB, 1, 1>(a, st);
      return launch_row<DR, SB, 2, 1>(a, st);
    }
    if (cpl == 1) return launch_row<DR, SB, 1, 2>(a, st);
    return launch_row<DR, SB, 2, 2>(a, st);
  }
  if (a.b.M == 2) return launch_rb<D, SB, 2, 4>(a, st);
  if constexpr (!two) return launch_rb<D, SB, 4, 4>(a, st);
  return JQ_ERR_SHAPE;
}

template <class D, int SB>
int launch_glu(GemvArgs& a, hipStream_t st) {
  const int cpl = row_cpl(a.b.K, D::BITS);
  if (a.b.M != 1 || cpl > 2) return JQ_ERR_SHAPE;
  using DR = typename RowD<D>::type;
  if (cpl == 1) return launch_row<DR, SB, 1, 2, true>(a, st);
  return launch_row<DR, SB, 2, 2, true>(a, st);
}

// The group size is a run-time argument of these kernels; D::GS is 32 only for codes in
// 32-code groups whose lane chunks hold two units (two groups then), 64 otherwise.
template <class D>
int launch_glu_d(GemvArgs& a, int sb, hipStream_t st) {
  if (sb == JQ_BF16) return launch_glu<D, JQ_BF16>(a, st);
  return launch_glu<D, JQ_F16>(a, st);
}
template <int BITS, int XDT>
int launch_glu_sb(GemvArgs& a, int sb, hipStream_t st) {
  if constexpr (row_upl<BITS>() == 2)
    if (a.ushift == 0) return launch_glu_d<Dc<BITS, 32, XDT>>(a, sb, st);
  return launch_glu_d<Dc<BITS, 64, XDT>>(a, sb, st);
}

template <class D>
int launch_d(GemvArgs& a, int sb, hipStream_t st) {
  if (sb == JQ_BF16) return launch_m<D, JQ_BF16>(a, st);
  return launch_m<D, JQ_F16>(a, st);
}
template <int BITS, int XDT>
int launch_sb(GemvArgs& a, int sb, hipStream_t st) {
  if constexpr (BITS == 2 || row_upl<BITS>() == 2)
    if (a.ushift == 0) return launch_d<Dc<BITS, 32, XDT>>(a, sb, st);
  return launch_d<Dc<BITS, 64, XDT>>(a, sb, st);
}

template <int BITS>
int launch_x(GemvArgs& a, int xd, int sb, hipStream_t st) {
  if (xd == JQ_BF16) return launch_sb<BITS, JQ_BF16>(a, sb, st);
  return launch_sb<BITS, JQ_F16>(a, sb, st);
}

}  // namespace

namespace jqk {

bool gemv_ok(int M, int64_t K, int64_t maxN, int bits, int gs, int xd, int sb) {
  if (M < 1 || M > (bits == 2 ? 2 : 4)) return false;
  if (xd != JQ_BF16 && xd != JQ_F16) return false;
  if (sb != JQ_BF16 && sb != JQ_F16) return false;
  const int64_t chunk = bits == 2 ? 64 : 32;  // K of one lane chunk
  if (K <= 0 || K % chunk || gemv_waves(K, bits, nullptr) > kMaxWaves) return false;
  // Byte offsets inside a row block's buffer views stay far below 2^31.
  return (maxN + 64) * (K / gs) * 2 < ((int64_t)1 << 31) && K * bits / 8 < ((int64_t)1 << 24);
}

int gemv_launch(const QmvBatch& b, int nprob, int bits, int gs, int xd, int sb, int yd,
                hipStream_t st) {
  int64_t maxN = 0;
  for (int i = 0; i < nprob; ++i) maxN = b.p[i].N > maxN ? b.p[i].N : maxN;
  if (maxN == 0 || b.M == 0) return JQ_OK;
  if (!gemv_ok(b.M, b.K, maxN, bits, gs, xd, sb)) return JQ_ERR_SHAPE;
  // Problems of one launch must share the activations (x stays in registers).
  for (int i = 1; i < nprob; ++i) {
    if (b.p[i].x != b.p[0].x) {
      for (int j = 0; j < nprob; ++j) {
        QmvBatch one = b;
        one.p[0] = b.p[j];
        const int s = gemv_launch(one, 1, bits, gs, xd, sb, yd, st);
        if (s) return s;
      }
      return JQ_OK;
    }
  }
  GemvArgs a;
  a.b = b;
  a.nprob = nprob;
  a.ushift = gs == 32 ? 0 : gs == 64 ? 1 : 2;
  a.yd = yd;
  a.glu_limit = 0.f;
  switch (bits) {
    case 2: return launch_x<2>(a, xd, sb, st);
    case 3: return launch_x<3>(a, xd, sb, st);
    case 4: return launch_x<4>(a, xd, sb, st);
    case 5: return launch_x<5>(a, xd, sb, st);
    case 6: return launch_x<6>(a, xd, sb, st);
    default: return launch_x<8>(a, xd, sb, st);
  }
}

bool gemv_swiglu_ok(int M, int64_t K, int64_t N, int bits, int gs, int xd, int sb, int yd) {
  return M == 1 && (yd == JQ_BF16 || yd == JQ_F16) && gemv_ok(1, K, N, bits, gs, xd, sb) &&
         gemv_waves(K, bits, nullptr) <= 2;
}

int gemv_swiglu_launch(const QmvBatch& b, int bits, int gs, int xd, int sb, int yd, float limit,
                       hipStream_t st) {
  if (b.p[0].N == 0) return JQ_OK;
  if (!gemv_swiglu_ok(b.M, b.K, b.p[0].N, bits, gs, xd, sb, yd) || b.p[1].N != b.p[0].N ||
      b.p[1].x != b.p[0].x)
    return JQ_ERR_SHAPE;
  GemvArgs a;
  a.b = b;
  a.nprob = 2;
  a.ushift = gs == 32 ? 0 : gs == 64 ? 1 : 2;
  a.yd = yd;
  a.glu_limit = limit;
#define JQ_GLU(B)                                                     \
  if (xd == JQ_BF16) return launch_glu_sb<B, JQ_BF16>(a, sb, st);     \
  return launch_glu_sb<B, JQ_F16>(a, sb, st);
  switch (bits) {
    case 2: { JQ_GLU(2) }
    case 3: { JQ_GLU(3) }
    case 4: { JQ_GLU(4) }
    case 5: { JQ_GLU(5) }
    case 6: { JQ_GLU(6) }
    default: { JQ_GLU(8) }
  }
#undef JQ_GLU
}

}  // namespace jqk

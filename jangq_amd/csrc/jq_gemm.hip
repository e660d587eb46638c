// Prefill GEMM on the matrix cores: y = x @ deq(W)^T for many activation rows (the
// reference's large-M quantized_matmul, jang-tools/jang_tools/jangrt/linear.py:41-45;
// algebra of jang-tools/jang_tools/dsv41/metal_decode.py:202-233).
//
// Exactness. Codes enter the B operand as exact 16-bit floats OFF + q (magic values, no
// int->float conversion; OFF = 2^bits, the smallest offset that holds the code), so every
// MFMA product is exact and accumulates in fp32. Per group
// g of a row n, with P_g = sum_{k in g} x_k (OFF + q_k) and X_g = sum_{k in g} x_k:
//   y = sum_g s_g P_g + sum_g c_g X_g,      c_g = b_g - OFF s_g.
// The first sum is accumulated in Horner form: before group g's MFMAs the accumulator is
// multiplied by s_{g-1}/s_g (one multiply per accumulator element per group), so the MFMAs
// add P_g unscaled and the result is s_last * acc. The second sum is a rank-G product; it is
// added in batches of 16 groups by three extra MFMA k-steps (X and c/s_batch-end each split
// into bf16 high and low parts: hi*hi + lo*hi + hi*lo), about 5% more matrix work; its
// rounding (about 2^-17 of c*X, where c*X partly cancels s*P) leaves results within ~1e-4 of
// an fp32 accumulation, the reason OFF is kept small. A group whose scale is 0 (or below
// 2^-100) is run with codes 0 and a stand-in scale s' (c = b - OFF s'), which gives b * X.
//
// Tiling. A block of 8 waves computes a 256 x 256 tile (waves 2 x 4, 128 x 64 each, as 4 x 2
// tiles of v_mfma_f32_32x32x16). K advances in stages of 32 (one 32-code unit per row of W):
// waves 0-3 stage the activations (one row each: permute into the code order of the unit,
// partial X), waves 4-7 the codes (one column each: unpack to magic values, scales at group
// starts); both write double-buffered LDS, one barrier per stage, global loads two stages
// ahead in a register ring.
// MFMA operand mapping: lane half h of k-step t takes unit fragment F = 2h + t (8 codes), for
// A and B alike, so the fragment order inside a unit cancels.
#include <type_traits>

#include "jq_dec.h"
#include "jq_qmv.h"

namespace {

using namespace jq;

typedef float f32x16 __attribute__((ext_vector_type(16)));

// Unpack traits for this kernel: one offset for every code (OFF = 2^bits, the "magic pairs"
// of jq_common.h) keeps the offset term a multiple of X.
template <int BITS_, int XDT_>
struct Dg {
  static constexpr int BITS = BITS_, XDT = XDT_, GS = 64;
  static constexpr bool SCHED = false;
  static constexpr bool NIB = false;
  static constexpr bool F16X = false;
  static constexpr bool TWO = BITS == 2;
  static constexpr uint32_t ONE2 = XDT == JQ_BF16 ? 0x3F803F80u : 0x3C003C00u;
  static constexpr float OFF = (float)(1 << BITS);
};

template <int FMT>
JQ_DEV f32x16 mfma32(u32x4 a, u32x4 b, f32x16 c) {
  if constexpr (FMT == JQ_BF16) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
}

constexpr int BM = 256, BN = 256, NTH = 512;
constexpr int WM = 128, WN = 64;           // wave tile
constexpr int FM = WM / 32, FN = WN / 32;  // 32x32 tiles per wave
constexpr int ROWB = 80;                   // LDS bytes per staged row: 4 fragments x 16 + pad
constexpr int BATCH = 16;                  // groups per bias-term batch

struct Smem {
  uint8_t a[2][BM][ROWB];  // activation stage, [row][fragment F][8 values]
  uint8_t b[2][BN][ROWB];  // code stage as magic values, [column][F][8 values]
  float r[2][BN];          // Horner ratio s_{g-1}/s_g, written with a group's first stage
  uint8_t xa[BM][ROWB];    // batch: X_hi[16] | X_lo[16] (16-bit floats) per row
  uint8_t xb[BN][ROWB];    // batch: (c/s_end)_hi[16] | (c/s_end)_lo[16] per column
  float sl[BN];            // s of the last group per column
  float cb[BN][BATCH];     // c = b - OFF s of the batch's groups per column (fp32)
};

struct GemmArgs {
  const void* x;
  const uint32_t* codes;
  const void* scales;
  const void* biases;
  void* y;
  int64_t M, N;
  int K, gs, yd;
};

template <int FMT>
JQ_DEV uint16_t to16(float v) {
  return FMT == JQ_BF16 ? f32_to_bf16_bits(v) : f32_to_f16_bits(v);
}
template <int FMT>
JQ_DEV float from16(uint32_t h) {
  return FMT == JQ_BF16 ? __uint_as_float(h << 16) : f16_bits_to_f32((uint16_t)h);
}

// 16 values v[0..15] as 16-bit high parts followed by 16 low parts (v - high).
template <int FMT>
JQ_DEV void write_hilo(uint8_t* dst, const float* v) {
  uint32_t hi[8], lo[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint16_t h0 = to16<FMT>(v[2 * i]), h1 = to16<FMT>(v[2 * i + 1]);
    const uint16_t l0 = to16<FMT>(v[2 * i] - from16<FMT>(h0));
    const uint16_t l1 = to16<FMT>(v[2 * i + 1] - from16<FMT>(h1));
    hi[i] = (uint32_t)h0 | ((uint32_t)h1 << 16);
    lo[i] = (uint32_t)l0 | ((uint32_t)l1 << 16);
  }
  u32x4* d = (u32x4*)dst;
  d[0] = u32x4{hi[0], hi[1], hi[2], hi[3]};
  d[1] = u32x4{hi[4], hi[5], hi[6], hi[7]};
  d[2] = u32x4{lo[0], lo[1], lo[2], lo[3]};
  d[3] = u32x4{lo[4], lo[5], lo[6], lo[7]};
}

template <class D, int SB, int SPG>
__global__ void __launch_bounds__(NTH, 1) gemm_kernel(GemmArgs a) {
  constexpr int BITS = D::BITS;
  extern __shared__ __attribute__((aligned(16))) uint8_t gemm_lds[];
  Smem& sm = *reinterpret_cast<Smem*>(gemm_lds);

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 2, wn = wave & 3;
  const int lr = lane & 31, lh = lane >> 5;
  const int64_t m0 = (int64_t)blockIdx.y * BM, n0 = (int64_t)blockIdx.x * BN;
  const int K = a.K;
  const int S = K / 32;          // stages
  const int G = K / a.gs;        // groups
  const int64_t P = (int64_t)K * BITS / 32;
  // Staging: thread t owns activation row and code column sr = t / 2, half hh = t % 2 of the
  // stage's 32-code unit (16 codes = fragments F = 2hh, 2hh+1). Every thread issues the same
  // loads, so the hardware wait counters track the prefetch ring exactly.
  const int sr = tid >> 1, hh = tid & 1;
  const int64_t arow = m0 + sr, bcol = n0 + sr;
  const bool alive = arow < a.M, blive = bcol < a.N;

  // Prefetch ring: the loads of stage k land in slot k % 2, two stages ahead of use.
  struct Slot {
    u32x4 x[2];      // 16 activations of the row half
    uint32_t w[BITS];  // the column's unit (both halves load it)
    uint32_t s, b;   // raw scale and bias of the stage's group
  };
  Slot pf[2];
  uint32_t zmask = ~0u;
  float sprev = 1.f, xg = 0.f;

  const uint16_t* __restrict__ xrow = (const uint16_t*)a.x + (alive ? arow : 0) * (int64_t)K + 16 * hh;
  const uint32_t* __restrict__ crow = a.codes + (blive ? bcol : 0) * P;
  const uint16_t* __restrict__ srow = (const uint16_t*)a.scales + (blive ? bcol : 0) * (int64_t)G;
  const uint16_t* __restrict__ brow = (const uint16_t*)a.biases + (blive ? bcol : 0) * (int64_t)G;

  auto load_stage = [&](int k, Slot& sl) {
    const u32x4* p = (const u32x4*)(xrow + 32 * k);
    sl.x[0] = p[0];
    sl.x[1] = p[1];
    const uint32_t* c = crow + (int64_t)k * BITS;
#pragma unroll
    for (int i = 0; i < BITS; ++i) sl.w[i] = c[i];
    sl.s = srow[k / SPG];
    sl.b = brow[k / SPG];
  };

  const jqd::Bases<D> bs = jqd::make_bases<D>();

  // Bits [16*BITS*hh, 16*BITS*(hh+1)) of a unit, moved to bit 0: the codes of this thread's
  // half. Fragments F = 2hh + t of the unit are fragments t of that half (the code order
  // inside fragments 2 and 3 is that of 0 and 1, shifted by 16).
  auto half_words = [&](const uint32_t* w, uint32_t* hw) {
    constexpr int HB = 16 * BITS;  // bits per half
#pragma unroll
    for (int i = 0; i < (HB + 31) / 32; ++i) {
      const int lo_w = (HB >> 5) + i, sh = HB & 31;  // upper half starts at bit HB
      uint32_t up;
      if constexpr ((HB & 31) == 0) {
        up = lo_w < BITS ? w[lo_w] : 0u;
      } else {
        const uint32_t a0 = lo_w < BITS ? w[lo_w] : 0u;
        const uint32_t a1 = lo_w + 1 < BITS ? w[lo_w + 1] : 0u;
        up = __builtin_amdgcn_alignbit(a1, a0, sh);
      }
      hw[i] = hh ? up : w[i];
    }
  };

  // Staging of stage k (in-group position KIN, compile time) from its prefetch slot. Both
  // halves of a row or column compute the shared values and write them alike, so no lane
  // predication splits the stage's code.
  auto stage = [&](int k, const Slot& sl, auto kin_c) {
    constexpr int KIN = decltype(kin_c)::value;
    constexpr bool gfirst = KIN == 0, glast = KIN == SPG - 1;
    const int buf = k & 1;
    const int g = k / SPG;
    const int gb = g % BATCH;
    // Activations: fragments 2hh, 2hh+1 of the row, and the half's sum.
    jqd::XRaw xr;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      xr.d[4 * i] = sl.x[i][0]; xr.d[4 * i + 1] = sl.x[i][1];
      xr.d[4 * i + 2] = sl.x[i][2]; xr.d[4 * i + 3] = sl.x[i][3];
    }
    u32x4* adst = (u32x4*)&sm.a[buf][sr][32 * hh];
    adst[0] = jqd::a_frag<D, 0>(xr);
    adst[1] = jqd::a_frag<D, 1>(xr);
    float u = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) u = dot2<D::XDT>(xr.d[i], D::ONE2, u);
    u += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, u), 0xB1, 0xF, 0xF, false));  // + partner half (lane ^ 1)
    xg = gfirst ? u : xg + u;
    if constexpr (glast) {
      // X of the group as 16-bit high and low parts into its batch slot.
      uint16_t* row = (uint16_t*)&sm.xa[sr][0];
      const uint16_t h = to16<D::XDT>(xg);
      row[gb] = h;
      row[BATCH + gb] = to16<D::XDT>(xg - from16<D::XDT>(h));
    }
    // Codes: fragments 2hh, 2hh+1 of the column as magic values; scales at group starts.
    if constexpr (gfirst) {
      const float sv = SB == JQ_BF16 ? __uint_as_float(sl.s << 16) : f16_bits_to_f32((uint16_t)sl.s);
      const float bv = SB == JQ_BF16 ? __uint_as_float(sl.b << 16) : f16_bits_to_f32((uint16_t)sl.b);
      // A zero (or below 2^-100) scale runs with codes 0 and a stand-in scale: the previous
      // group's (Horner ratio 1), or |b|/OFF for the first group, so that s*P = s*OFF*X
      // stays of the size of the group's true term b*X.
      const bool zero = fabsf(sv) < 7.8886091e-31f;  // NaN keeps its scale
      const float sp = !zero ? sv : g > 0 ? sprev : fmaxf(fabsf(bv), 8.6736174e-19f) / D::OFF;
      zmask = zero || !blive ? 0u : ~0u;
      sm.r[buf][sr] = sprev * __builtin_amdgcn_rcpf(sp);  // ratio to ~1 ulp
      sm.cb[sr][gb] = blive ? fmaf(-D::OFF, sp, bv) : 0.f;
      sm.sl[sr] = sp;  // the last group's value remains
      sprev = sp;
    }
    uint32_t w[BITS], hw[BITS];
#pragma unroll
    for (int i = 0; i < BITS; ++i) w[i] = sl.w[i] & zmask;
    half_words(w, hw);
    u32x4 f0, f1, h;
    jqd::b_frag<D, 0>(hw, bs, f0, h);
    jqd::b_frag<D, 1>(hw, bs, f1, h);
    u32x4* bdst = (u32x4*)&sm.b[buf][sr][32 * hh];
    bdst[0] = f0;
    bdst[1] = f1;
    if constexpr (glast) {
      if (gb == BATCH - 1 || g == G - 1) {
        // Batch end: clear the unused X slots, write the coefficients c / s_end.
        uint16_t* row = (uint16_t*)&sm.xa[sr][0];
        for (int q = gb + 1; q < BATCH; ++q) row[q] = row[BATCH + q] = 0;
        const float inv = 1.f / sprev;
        float v[BATCH];
#pragma unroll
        for (int q = 0; q < BATCH; ++q) v[q] = q <= gb ? sm.cb[sr][q] * inv : 0.f;
        write_hilo<D::XDT>(&sm.xb[sr][0], v);
      }
    }
  };

  f32x16 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  // MFMAs of stage k. At a group's first stage each tile is first scaled by the Horner
  // ratio (zero accumulators on the first group), tile by tile so that the multiplies of one
  // tile overlap the matrix work of the previous.
  auto compute = [&](int k, auto kin_c) {
    constexpr int KIN = decltype(kin_c)::value;
    const int buf = k & 1;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int fo = (2 * lh + t) * 16;
      u32x4 A[FM], B[FN];
#pragma unroll
      for (int i = 0; i < FM; ++i) A[i] = *(const u32x4*)&sm.a[buf][wm * WM + 32 * i + lr][fo];
#pragma unroll
      for (int j = 0; j < FN; ++j) B[j] = *(const u32x4*)&sm.b[buf][wn * WN + 32 * j + lr][fo];
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        float rj = 1.f;
        if constexpr (KIN == 0) rj = sm.r[buf][wn * WN + 32 * j + lr];
#pragma unroll
        for (int i = 0; i < FM; ++i) {
          if constexpr (KIN == 0) {
            if (t == 0) {
#pragma unroll
              for (int r = 0; r < 16; ++r) acc[i][j][r] *= rj;
            }
          }
          acc[i][j] = mfma32<D::XDT>(A[i], B[j], acc[i][j]);
        }
      }
    }
  };

  // Bias terms of a batch: X_hi*c_hi + X_lo*c_hi + X_hi*c_lo.
  auto batch_mfma = [&]() {
#pragma unroll
    for (int t = 0; t < 3; ++t) {
      const int ao = (t == 1 ? 32 : 0) + 16 * lh, bo = (t == 2 ? 32 : 0) + 16 * lh;
      u32x4 A[FM], B[FN];
#pragma unroll
      for (int i = 0; i < FM; ++i) A[i] = *(const u32x4*)&sm.xa[wm * WM + 32 * i + lr][ao];
#pragma unroll
      for (int j = 0; j < FN; ++j) B[j] = *(const u32x4*)&sm.xb[wn * WN + 32 * j + lr][bo];
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = mfma32<D::XDT>(A[i], B[j], acc[i][j]);
    }
  };

  // Pipeline: stage k+1 is written to LDS while stage k is multiplied; its loads were issued
  // two stages earlier into ring slot (k+1) % 2. The loop runs 4 stages per trip so that
  // slots and in-group positions are compile-time.
  using I0 = std::integral_constant<int, 0>;
  load_stage(0, pf[0]);
  load_stage(S > 1 ? 1 : S - 1, pf[1]);
  stage(0, pf[0], I0{});
  __syncthreads();
  load_stage(S > 2 ? 2 : S - 1, pf[0]);
  // One step: the MFMAs of stage k, the staging of stage k+1, the rare batch work.
  auto step = [&](int k, auto j_c) {
    constexpr int J = decltype(j_c)::value;
    constexpr int KIN = J % SPG, NKIN = (J + 1) % SPG;
    compute(k, std::integral_constant<int, KIN>{});
    if (k + 1 < S) stage(k + 1, pf[(J + 1) & 1], std::integral_constant<int, NKIN>{});
    if (KIN == SPG - 1) {
      const int g = k / SPG;
      if ((g % BATCH) == BATCH - 1 || g == G - 1) batch_mfma();
    }
    __syncthreads();
    // Past the last stage the slot is refilled with stage S-1 again and never staged.
    load_stage(k + 3 < S ? k + 3 : S - 1, pf[(J + 1) & 1]);
  };
  for (int k0 = 0; k0 < S; k0 += 4) {
    step(k0, I0{});
    if (k0 + 1 < S) step(k0 + 1, std::integral_constant<int, 1>{});
    if (k0 + 2 < S) step(k0 + 2, std::integral_constant<int, 2>{});
    if (k0 + 3 < S) step(k0 + 3, std::integral_constant<int, 3>{});
  }

  // y = s_last * acc.
#pragma unroll
  for (int j = 0; j < FN; ++j) {
    const int nl = wn * WN + 32 * j + lr;
    const int64_t n = n0 + nl;
    const float sj = sm.sl[nl];
    if (n < a.N) {
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int64_t m = m0 + wm * WM + 32 * i + 8 * (r >> 2) + 4 * lh + (r & 3);
          if (m < a.M) {
            const float v = acc[i][j][r] * sj;
            const int64_t o = m * a.N + n;
            if (a.yd == JQ_BF16) ((uint16_t*)a.y)[o] = f32_to_bf16_bits(v);
            else if (a.yd == JQ_F16) ((uint16_t*)a.y)[o] = f32_to_f16_bits(v);
            else ((float*)a.y)[o] = v;
          }
        }
    }
  }
}

template <class D, int SB, int SPG>
int launch_g(const GemmArgs& a, hipStream_t st) {
  const size_t lds = sizeof(Smem);  // above the 64 KB default: opt in (per device)
  if (!jqh::set_lds((const void*)gemm_kernel<D, SB, SPG>, lds)) return JQ_ERR_LAUNCH;
  dim3 grid((unsigned)((a.N + BN - 1) / BN), (unsigned)((a.M + BM - 1) / BM));
  gemm_kernel<D, SB, SPG><<<grid, NTH, lds, st>>>(a);
  return jqh::launch_status();
}

template <class D, int SB>
int launch(const GemmArgs& a, hipStream_t st) {
  return a.gs == 64 ? launch_g<D, SB, 2>(a, st) : launch_g<D, SB, 4>(a, st);
}

template <int BITS, int XDT>
int launch_sb(const GemmArgs& a, int sb, hipStream_t st) {
  using D = Dg<BITS, XDT>;
  if (sb == JQ_BF16) return launch<D, JQ_BF16>(a, st);
  return launch<D, JQ_F16>(a, st);
}

template <int BITS>
int launch_x(const GemmArgs& a, int xd, int sb, hipStream_t st) {
  if (xd == JQ_BF16) {
    if constexpr (BITS == 8) return JQ_ERR_SHAPE;  // 8-bit magic values need f16
    else return launch_sb<BITS, JQ_BF16>(a, sb, st);
  }
  return launch_sb<BITS, JQ_F16>(a, sb, st);
}

}  // namespace

namespace jqk {

bool gemm_ok(int64_t M, int64_t K, int bits, int gs, int xd, int sb) {
  if (xd != JQ_BF16 && xd != JQ_F16) return false;
  if (sb != JQ_BF16 && sb != JQ_F16) return false;
  if (bits == 8 && xd == JQ_BF16) return false;
  if (gs != 64 && gs != 128) return false;
  return M >= 1 && K > 0 && K % gs == 0 && K <= (1 << 24);
}

int gemm_launch(const QmmProblem& p, int bits, int gs, int xd, int sb, int yd, hipStream_t st) {
  if (!gemm_ok(p.M, p.K, bits, gs, xd, sb)) return JQ_ERR_SHAPE;
  if (p.M == 0 || p.N == 0) return JQ_OK;
  GemmArgs a;
  a.x = p.x;
  a.codes = p.codes;
  a.scales = p.scales;
  a.biases = p.biases;
  a.y = p.y;
  a.M = p.M;
  a.N = p.N;
  a.K = (int)p.K;
  a.gs = gs;
  a.yd = yd;
  switch (bits) {
    case 2: return launch_x<2>(a, xd, sb, st);
    case 3: return launch_x<3>(a, xd, sb, st);
    case 4: return launch_x<4>(a, xd, sb, st);
    case 5: return launch_x<5>(a, xd, sb, st);
    case 6: return launch_x<6>(a, xd, sb, st);
    default: return launch_x<8>(a, xd, sb, st);
  }
}

}  // namespace jqk

// Prefill GEMM on the f16 matrix cores: y = x @ deq(W)^T for many activation rows (the
// reference's large-M quantized_matmul, jang-tools/jang_tools/jangrt/linear.py:41-45).
//
// Arithmetic. The weights are dequantized tile by tile into f16, w' = f16(s' q + b') with one
// rounding (v_pk_fma_f16), where s' = s 2^-f_n and b' = b 2^-f_n carry a power-of-two scale per
// weight row n chosen so that the row's largest |s q + b| lies in [2^13, 2^14); the activations
// enter as x' = f16(x 2^-e_m) with a power of two per activation row (exact for bf16 inputs in
// range: both formats hold 8 significant bits). The matrix cores multiply x' by w' exactly
// and accumulate in fp32, and y = acc 2^(e_m + f_n). The only rounding beyond fp32
// accumulation is that of w' to f16 (2^-11 relative): about 2e-4 rel-L2 on the outputs, where
// dequantizing to bf16 would give 1.5e-3. No per-group rescale touches the accumulators.
//
// Codes become f16 values without an int-to-float conversion: one and-or places code a at
// mantissa bit pa of a dword's low half and code b at bit pb of its high half under the
// exponent of 1024 (the schedules of jq_sched16.h, one funnel shift per few pairs); one
// v_pk_fma_f16 with constants 2^-p and -1024 2^-p turns 1024 + q 2^p into q exactly, and a
// second applies s' and b'. The x' rows are written in the schedules' pair order by a pre-pass
// (prep_kernel), so the natural-order copies of x' line up with the codes.
//
// The pre-pass also writes each weight row's (s', b') per group as one f16 pair, group-major,
// so a stage's pairs for 256 rows are 1 KB of contiguous memory.
//
// Tiling. A block of 8 waves computes 256 x 256 outputs (waves 2 x 4, 128 x 64 each, as 4 x 2
// tiles of v_mfma_f32_32x32x16_f16). K advances in stages of 64 (two 32-code units per weight
// row). Each stage's x' tile (256 rows x 128 B) goes into a 3-slot LDS ring, copied 2 stages
// ahead, and its code tile (256 rows x 8 BITS B) with the (s', b') pairs into a ring of 4
// slots (3 for 8-bit codes), copied 3 (2) stages ahead, all with buffer_load ... lds: every
// x' copy instruction reads whole 128-byte lines (8 rows; the chunks of a row XOR-swizzled by
// the row, so that the fragment reads spread over the banks). A wave unpacks its own B
// fragments from the code tile (lane half h takes unit h, k-step t its chunk t, as the A
// fragments): the two waves of a column pair both unpack it, and no second LDS pass is
// needed. The fragments of stage s + 1 are unpacked while stage s is multiplied, one code pair
// per matrix instruction, so vector and matrix work interleave in every wave. One barrier per
// stage. The 16-bit outputs leave through LDS as whole 16-byte row pieces.
#include <utility>

#include "jq_common.h"
#include "jq_gemv.h"
#include "jq_qmv.h"
#include "jq_sched16.h"

#define JQ_LDS __attribute__((address_space(3)))

namespace {

using namespace jq;
using jqg::Rsrc;

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));

constexpr int BM = 256, BN = 256, BK = 64, NTH = 512;
constexpr int kMaxK = 1 << 22;  // 256 rows of x' stay below 2^31 bytes in one buffer view

template <int BITS>
struct G16 {
  static constexpr int RB = 8 * BITS;                // code bytes per weight row per stage
  static constexpr int CB = RB % 32 == 0 ? 16 : 4;   // copy bytes per lane
  static constexpr int BI = RB / (2 * CB);           // code copies per wave per stage
  static constexpr int A_BYTES = BM * 128;           // x' tile of a stage
  static constexpr int C_BYTES = BN * RB;            // code tile of a stage
  static constexpr int CSLOT = C_BYTES + BN * 4;     // + the (s', b') f16 pair per weight row
  static constexpr int EXP_BYTES = (BM + BN) * 4;    // row / column exponents
  static constexpr int NAS = 3;                      // x' ring slots (copies 2 stages ahead)
  // code ring slots: 4 (copies 3 stages ahead) where the LDS holds them, else 3
  static constexpr int NCS = NAS * A_BYTES + 4 * CSLOT + EXP_BYTES <= 160 * 1024 ? 4 : 3;
  static constexpr int C_OFF = NAS * A_BYTES;
  static constexpr int E_OFF = C_OFF + NCS * CSLOT;
  static constexpr int LDS = E_OFF + EXP_BYTES;
  static constexpr int NA = 4;       // x' copies per wave per stage
  static constexpr int NC = BI + 1;  // code and sidecar copies per wave per stage
};

// Pair p of a 32-code unit: (window shift, code a, code b, bit pa, bit pb).
template <int BITS>
struct Pair {
  static constexpr int s(int p) {
    if constexpr (BITS == 2) return jq16::kSched16_2.s[p];
    else if constexpr (BITS == 3) return jq16::kSched16_3.s[p];
    else if constexpr (BITS == 4) return jq16::kSched16_4.s[p];
    else if constexpr (BITS == 5) return jq16::kSched16_5.s[p];
    else if constexpr (BITS == 6) return jq16::kSched16_6.s[p];
    else return 32 * (p >> 1);
  }
  static constexpr int a(int p) {
    if constexpr (BITS == 2) return jq16::kSched16_2.a[p];
    else if constexpr (BITS == 3) return jq16::kSched16_3.a[p];
    else if constexpr (BITS == 4) return jq16::kSched16_4.a[p];
    else if constexpr (BITS == 5) return jq16::kSched16_5.a[p];
    else if constexpr (BITS == 6) return jq16::kSched16_6.a[p];
    else return 4 * (p >> 1) + (p & 1);  // 8-bit: bytes (0, 2) and (1, 3) of word p / 2
  }
  static constexpr int b(int p) {
    if constexpr (BITS == 2) return jq16::kSched16_2.b[p];
    else if constexpr (BITS == 3) return jq16::kSched16_3.b[p];
    else if constexpr (BITS == 4) return jq16::kSched16_4.b[p];
    else if constexpr (BITS == 5) return jq16::kSched16_5.b[p];
    else if constexpr (BITS == 6) return jq16::kSched16_6.b[p];
    else return 4 * (p >> 1) + (p & 1) + 2;
  }
  static constexpr int pa(int p) {
    if constexpr (BITS == 2) return jq16::kSched16_2.pa[p];
    else if constexpr (BITS == 3) return jq16::kSched16_3.pa[p];
    else if constexpr (BITS == 4) return jq16::kSched16_4.pa[p];
    else if constexpr (BITS == 5) return jq16::kSched16_5.pa[p];
    else if constexpr (BITS == 6) return jq16::kSched16_6.pa[p];
    else return 0;
  }
  static constexpr int pb(int p) {
    if constexpr (BITS == 2) return jq16::kSched16_2.pb[p];
    else if constexpr (BITS == 3) return jq16::kSched16_3.pb[p];
    else if constexpr (BITS == 4) return jq16::kSched16_4.pb[p];
    else if constexpr (BITS == 5) return jq16::kSched16_5.pb[p];
    else if constexpr (BITS == 6) return jq16::kSched16_6.pb[p];
    else return 0;
  }
  // x' slot 2p holds code a(p)'s activation, slot 2p + 1 code b(p)'s.
  static constexpr int code_of_slot(int slot) { return slot & 1 ? b(slot >> 1) : a(slot >> 1); }
};

constexpr uint16_t f16_pow2(int e) { return (uint16_t)((15 + e) << 10); }  // 2^e, normal

// Window of a unit: the unit's bits [s, s + 32).
template <int BITS>
JQ_DEV uint32_t window(const uint32_t (&u)[BITS], int s) {
  const int lo = s >> 5, sh = s & 31;
  if (sh == 0) return u[lo];
  const uint32_t hi = lo + 1 < BITS ? u[lo + 1] : 0u;
  return __builtin_amdgcn_alignbit(hi, u[lo], sh);
}

// f16 pair (s' q_a + b', s' q_b + b') of pair p of a unit.
template <int BITS, int P>
JQ_DEV uint32_t dq_pair(const uint32_t (&u)[BITS], h2 s2, h2 b2, uint32_t magic) {
  using S = Pair<BITS>;
  uint32_t v;
  if constexpr (BITS == 8) {
    // [byte a, 0x64, byte b, 0x64] of word P / 2 (v_perm: selectors 0-3 pick the word's bytes,
    // 4-7 the constant's)
    constexpr uint32_t sel = (uint32_t)(P & 1) | (4u << 8) | ((uint32_t)((P & 1) + 2) << 16) | (4u << 24);
    v = __builtin_amdgcn_perm(0x64646464u, u[P >> 1], sel);
  } else {
    constexpr uint32_t m = (1u << BITS) - 1u;
    constexpr uint32_t mask = (m << S::pa(P)) | (m << (16 + S::pb(P)));
    v = (window<BITS>(u, S::s(P)) & mask) | magic;  // one v_and_or_b32
  }
  constexpr uint32_t c1 = (uint32_t)f16_pow2(-S::pa(P)) | ((uint32_t)f16_pow2(-S::pb(P)) << 16);
  constexpr uint32_t c2 = (uint32_t)(0x8000u | f16_pow2(10 - S::pa(P))) |
                          ((uint32_t)(0x8000u | f16_pow2(10 - S::pb(P))) << 16);
  const h2 q = __builtin_elementwise_fma(__builtin_bit_cast(h2, v), __builtin_bit_cast(h2, c1),
                                         __builtin_bit_cast(h2, c2));
  return __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(s2, q, b2));
}

struct G16Args {
  const uint16_t* xp;     // x' f16 [M, K] in pair order
  const int* erow;        // e_m [M]
  const int* ecol;        // f_n [N]
  const uint32_t* codes;  // [N, K * BITS / 32]
  const uint32_t* sbp;    // [G, N]: f16 s' (low half) and b' (high half) of group g, row n
  void* y;                // [M, N]
  int64_t M, N;
  int K, G, gs, yd;
};

// Row swizzle of the 16-byte chunks of an x' row in LDS.
JQ_DEV int swz(int row) { return (row & 7) ^ ((row >> 3) & 1); }

template <int N>
JQ_DEV void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

JQ_DEV void lds_barrier() {
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// The x' copies of stage st into its ring slot (4 instructions per wave, 8 rows each).
JQ_DEV void issue_a(JQ_LDS uint8_t* slot, int st, int wave, Rsrc rx, const uint32_t* xoff) {
  const uint32_t kb = (uint32_t)st * BK;
#pragma unroll
  for (int j = 0; j < 4; ++j)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (JQ_LDS void*)(slot + (32 * wave + 8 * j) * 128),
                                             16, xoff[j], kb * 2u, 0, 0);
}

// The code copies of stage st (BI instructions per wave) and the (s', b') words of the
// stage's group for the block's 256 weight rows, 1 KB contiguous in the group-major pair
// array (32 rows per wave, lanes 0-31).
template <int BITS>
JQ_DEV void issue_c(JQ_LDS uint8_t* slot, int st, int wave, int lane, Rsrc rc, Rsrc rsb,
                    const uint32_t* coff, uint32_t sboff, uint32_t gstride, int g) {
  using L = G16<BITS>;
  // (literal sizes: the host pass rejects a size argument that depends on the template)
#pragma unroll
  for (int j = 0; j < L::BI; ++j) {
    JQ_LDS void* dst = (JQ_LDS void*)(slot + (L::BI * wave + j) * 64 * L::CB);
    const uint32_t so = (uint32_t)st * L::RB;
    if constexpr (L::CB == 16) __builtin_amdgcn_raw_ptr_buffer_load_lds(rc, dst, 16, coff[j], so, 0, 0);
    else __builtin_amdgcn_raw_ptr_buffer_load_lds(rc, dst, 4, coff[j], so, 0, 0);
  }
  if (lane < 32)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsb, (JQ_LDS void*)(slot + L::C_BYTES + 128 * wave), 4,
                                             sboff, (uint32_t)g * gstride, 0, 0);
}

// The unit words and the scaled (s', b') pairs of column tile j of a stage, from its code slot.
template <int BITS, int SB>
struct TileSrc {
  uint32_t u[BITS];
  h2 s2, b2;
};

template <int BITS, int SB>
JQ_DEV void tile_src(const JQ_LDS uint8_t* cslot, int nl, int h, TileSrc<BITS, SB>& ts) {
  using L = G16<BITS>;
  const JQ_LDS uint32_t* src = (const JQ_LDS uint32_t*)(cslot + nl * L::RB + 4 * BITS * h);
#pragma unroll
  for (int i = 0; i < BITS; ++i) ts.u[i] = src[i];
  const uint32_t sb = ((const JQ_LDS uint32_t*)(cslot + L::C_BYTES))[nl];
  ts.s2 = __builtin_bit_cast(h2, __builtin_amdgcn_perm(sb, sb, 0x01000100u));  // (s', s')
  ts.b2 = __builtin_bit_cast(h2, __builtin_amdgcn_perm(sb, sb, 0x03020302u));  // (b', b')
}

template <int... I, class F>
JQ_DEV void static_for_impl(std::integer_sequence<int, I...>, F&& f) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, class F>
JQ_DEV void static_for(F&& f) {
  static_for_impl(std::make_integer_sequence<int, N>{}, f);
}

template <int BITS, int SB>
__global__ void __launch_bounds__(NTH, 1) gemm16_kernel(G16Args a) {
  using L = G16<BITS>;
  extern __shared__ __attribute__((aligned(1024))) uint8_t g16_lds[];
  JQ_LDS uint8_t* lds = (JQ_LDS uint8_t*)g16_lds;
  JQ_LDS int* rexp = (JQ_LDS int*)(lds + L::E_OFF);
  JQ_LDS int* cexp = rexp + BM;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 2, wn = wave & 3;
  const int r = lane & 31, h = lane >> 5;
  const int64_t m0 = (int64_t)blockIdx.y * BM, n0 = (int64_t)blockIdx.x * BN;
  const int K = a.K, G = a.G;
  const int S = K / BK;
  const uint32_t rowbytes = (uint32_t)(K / 32) * BITS * 4;
  const int mrows = (int)(a.M - m0 < BM ? a.M - m0 : BM);
  const int nrows = (int)(a.N - n0 < BN ? a.N - n0 : BN);
  const int gsh = a.gs == 128 ? 1 : 0;  // stages per group: 1 (gs 64) or 2 (gs 128)

  // Buffer views of the block's x' rows, code rows and sidecar rows (reads past them are 0).
  const Rsrc rx = jqg::make_rsrc(a.xp + m0 * K, (uint32_t)mrows * (uint32_t)K * 2u);
  const Rsrc rc = jqg::make_rsrc((const uint8_t*)a.codes + n0 * rowbytes, (uint32_t)nrows * rowbytes);
  const Rsrc rsb = jqg::make_rsrc(a.sbp, (uint32_t)G * (uint32_t)a.N * 4u);

  // Per-lane copy offsets. x': wave w copies rows [32w, 32w + 32), 8 rows per instruction,
  // lane -> (row, physical chunk lane % 8) holding logical chunk (lane % 8) ^ swz(row).
  uint32_t xoff[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int row = 32 * wave + 8 * j + (lane >> 3);
    xoff[j] = (uint32_t)row * (uint32_t)K * 2u + (uint32_t)(((lane & 7) ^ swz(row)) * 16);
  }
  // codes: the stage's code tile is 256 rows x RB bytes, copied in CB-byte pieces.
  uint32_t coff[L::BI];
#pragma unroll
  for (int j = 0; j < L::BI; ++j) {
    const int f = (L::BI * wave + j) * 64 + lane;
    const int row = f * L::CB / L::RB, byte = f * L::CB % L::RB;
    coff[j] = (uint32_t)row * rowbytes + (uint32_t)byte;
  }
  const uint32_t sboff = (uint32_t)(n0 + 32 * wave + (lane & 31)) * 4u;  // pair word, group 0

  auto aslot = [&](int st) { return lds + (st % L::NAS) * L::A_BYTES; };
  auto cslot = [&](int st) { return lds + L::C_OFF + (st % L::NCS) * L::CSLOT; };
  auto copy_a = [&](int st) { issue_a(aslot(st), st, wave, rx, xoff); };
  auto copy_c = [&](int st) {
    issue_c<BITS>(cslot(st), st, wave, lane, rc, rsb, coff, sboff, (uint32_t)a.N * 4u, st >> gsh);
  };

  // Exponents of the block's rows and columns (rows past the matrix: 0).
  if (tid < BM) rexp[tid] = tid < mrows ? a.erow[m0 + tid] : 0;
  else cexp[tid - BM] = tid - BM < nrows ? a.ecol[n0 + tid - BM] : 0;

  // Prologue: codes of stages 0, 1 (and 2), x' of stages 0, 1; wait for C0, A0, C1.
  copy_c(0);
  copy_a(0);
  if (S > 1) {
    copy_c(1);
    copy_a(1);
    if (L::NCS == 4 && S > 2) {
      copy_c(2);
      wait_vm<L::NA + L::NC>();
    } else {
      wait_vm<L::NA>();
    }
  } else {
    wait_vm<0>();
  }
  lds_barrier();

  f32x16 acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int q = 0; q < 16; ++q) acc[i][j][q] = 0.f;

  // The exponent pair of 1024 pinned in a register: gfx9 VOP3 takes no literal, so the
  // and-or of a pair takes its mask as the scalar operand and this base as a vector one.
  uint32_t magic = 0x64006400u;
  asm volatile("" : "+v"(magic));
  const int sw = swz(r);  // rows wm*128 + 32 i + r share r's swizzle
  int fcol[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) fcol[j] = cexp[wn * 64 + 32 * j + r];

  // B fragments of the stage being multiplied (dword 4t + d of tile j: k-step t), and those
  // of the next stage, unpacked between its matrix instructions: 32 chunks of one MFMA and
  // one code pair each, fenced so that the two waves of a SIMD always hold matrix and vector
  // work to interleave. Two register sets alternate between the stages of a trip.
  uint32_t B0[2][16], B1[2][16];
  {
    TileSrc<BITS, SB> ts[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) tile_src<BITS, SB>(cslot(0), wn * 64 + 32 * j + r, h, ts[j]);
    static_for<32>([&](auto kc) {
      constexpr int K = decltype(kc)::value, jd = K >> 4, p = K & 15;
      B0[jd][p] = dq_pair<BITS, p>(ts[jd].u, ts[jd].s2, ts[jd].b2, magic);
    });
  }

  auto stage = [&](int st, const uint32_t (&Bc)[2][16], uint32_t (&Bn)[2][16]) {
    constexpr int CD = L::NCS - 1;  // code copies run CD stages ahead
    if (st + CD < S) copy_c(st + CD);
    if (st + 2 < S) copy_a(st + 2);
    const JQ_LDS uint8_t* as = aslot(st);
    auto afrag = [&](int i, int t) {
      return *(const JQ_LDS u32x4*)(as + (wm * 128 + 32 * i + r) * 128 + (((4 * h + t) ^ sw) * 16));
    };
    u32x4 A[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) A[i] = afrag(i, 0);
    // (past the last stage this unpacks a stale slot; the result is not used)
    TileSrc<BITS, SB> ts[2];
#pragma unroll
    for (int j = 0; j < 2; ++j)
      tile_src<BITS, SB>(cslot(st + 1), wn * 64 + 32 * j + r, h, ts[j]);
    __builtin_amdgcn_sched_barrier(0);
    static_for<32>([&](auto kc) {
      constexpr int K = decltype(kc)::value;
      constexpr int t = K >> 3, i = (K >> 1) & 3, j = K & 1;  // MFMA (k-step, row tile, col tile)
      constexpr int jd = K >> 4, p = K & 15;                  // code pair unpacked alongside
      const u32x4 b = {Bc[j][4 * t], Bc[j][4 * t + 1], Bc[j][4 * t + 2], Bc[j][4 * t + 3]};
      acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, A[i]),
                                                         __builtin_bit_cast(f16x8, b), acc[i][j],
                                                         0, 0, 0);
      if constexpr (j == 1 && t < 3) A[i] = afrag(i, t + 1);  // row tile i's next k-step
      Bn[jd][p] = dq_pair<BITS, p>(ts[jd].u, ts[jd].s2, ts[jd].b2, magic);
      __builtin_amdgcn_sched_barrier(0);
    });
    // The next stage's fragments are complete here (kept from being sunk into the next stage).
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int q = 0; q < 16; ++q) asm volatile("" : "+v"(Bn[j][q]));
    // Before the barrier: x' of stage st + 1 and codes of stage st + 2 landed (the copies
    // issued in this trip may still run: in the 3-slot code ring the codes of st + 2 were
    // issued first, before the x' of st + 2).
    if (L::NCS == 4) {
      if (st + CD < S && st + 2 < S) wait_vm<L::NA + L::NC>();
      else if (st + 2 < S) wait_vm<L::NA>();
      else wait_vm<0>();
    } else {
      if (st + 2 < S) wait_vm<L::NA>();
      else wait_vm<0>();
    }
    lds_barrier();
  };
  int st = 0;
  for (; st + 1 < S; st += 2) {
    stage(st, B0, B1);
    stage(st + 1, B1, B0);
  }
  if (st < S) stage(st, B0, B1);

  // y = acc 2^(e_m + f_n).
  if (a.yd == JQ_F32) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int nl = wn * 64 + 32 * j + r;
      if (nl >= nrows) continue;
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int q = 0; q < 16; ++q) {
          const int ml = wm * 128 + 32 * i + 8 * (q >> 2) + 4 * h + (q & 3);
          if (ml < mrows)
            ((float*)a.y)[(m0 + ml) * a.N + n0 + nl] = __builtin_ldexpf(acc[i][j][q], rexp[ml] + fcol[j]);
        }
    }
    return;
  }
  // 16-bit outputs go through LDS (the ring is free after the last barrier): each wave
  // stages 64 of its rows x 64 columns (8 KB) at a time and writes them back as whole 16-byte
  // row pieces, 8 rows x 128 B per store instruction.
  JQ_LDS uint16_t* stg = (JQ_LDS uint16_t*)(lds + wave * 8192);
  const bool bf = a.yd == JQ_BF16;
  const bool vec = (a.N & 7) == 0 && (((uintptr_t)a.y) & 15) == 0;
#pragma unroll
  for (int hf = 0; hf < 2; ++hf) {
#pragma unroll
    for (int ii = 0; ii < 2; ++ii) {
      const int i = 2 * hf + ii;
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int q = 0; q < 16; ++q) {
          const int rl = 32 * ii + 8 * (q >> 2) + 4 * h + (q & 3);  // row within the half
          const float v = __builtin_ldexpf(acc[i][j][q], rexp[wm * 128 + 32 * i + 8 * (q >> 2) + 4 * h + (q & 3)] + fcol[j]);
          stg[rl * 64 + 32 * j + r] = bf ? f32_to_bf16_bits(v) : f32_to_f16_bits(v);
        }
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's staging writes done
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int rl = 8 * k + (lane >> 3), c8 = lane & 7;
      const int ml = wm * 128 + 64 * hf + rl;
      const int nl = wn * 64 + 8 * c8;
      if (ml >= mrows || nl >= nrows) continue;
      const u32x4 v = *(const JQ_LDS u32x4*)(stg + rl * 64 + 8 * c8);
      uint16_t* dst = (uint16_t*)a.y + (m0 + ml) * a.N + n0 + nl;
      if (vec && nl + 8 <= nrows) {
        *(u32x4*)dst = v;
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e)
          if (nl + e < nrows) dst[e] = (uint16_t)(v[e >> 1] >> (16 * (e & 1)));
      }
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);  // reads done before the next half overwrites
  }
}

// ----------------------------------------------------------------------------- pre-pass

struct PrepArgs {
  const void* x;     // [M, K] bf16 / f16
  uint16_t* xp;      // x' [M, K]
  int* erow;         // [M]
  const void* scales;
  const void* biases;
  int* ecol;         // [N]
  uint32_t* sbp;     // [G, N] (s', b') f16 pairs
  int64_t M, N;
  int K, G, qmax, xd, sb;
  int xblocks;       // blocks [0, xblocks) convert activation rows, the rest weight rows
};

JQ_DEV int exp_for(float mx, int top) {
  // 2^-e brings mx into [2^(top-1), 2^top); 0 for zero or non-finite maxima.
  if (!(mx > 0.f) || !__builtin_isfinite(mx)) return 0;
  int E;
  (void)__builtin_frexpf(mx, &E);  // mx = f 2^E, f in [0.5, 1)
  return E - top;
}

JQ_DEV float wave_max(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
}

// Activation rows: one wave per row. Pass 1 takes the row's largest finite |x| (bf16 only;
// f16 rows keep e = 0), pass 2 writes x' = f16(x 2^-e) in each unit's pair order.
// Weight rows: 8 threads per row; f = exponent of the max over groups of |b| and |b + s qmax|,
// then the row's (s', b') pairs into the group-major array.
template <int BITS>
__global__ void __launch_bounds__(256) prep_kernel(PrepArgs a) {
  using S = Pair<BITS>;
  if ((int)blockIdx.x < a.xblocks) {
    const int64_t m = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (m >= a.M) return;
    const int lane = threadIdx.x & 63;
    const int U = a.K / 32;
    const u32x4* row = (const u32x4*)((const uint16_t*)a.x + m * a.K);
    int e = 0;
    if (a.xd == JQ_BF16) {
      float mx = 0.f;
      for (int u = lane; u < U; u += 64)
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const u32x4 v = row[4 * u + c];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float lo = fabsf(__uint_as_float(v[i] << 16));
            const float hi = fabsf(__uint_as_float(v[i] & 0xFFFF0000u));
            mx = __builtin_isfinite(lo) ? fmaxf(mx, lo) : mx;
            mx = __builtin_isfinite(hi) ? fmaxf(mx, hi) : mx;
          }
        }
      e = exp_for(wave_max(mx), 14);
    }
    if (lane == 0) a.erow[m] = e;
    u32x4* out = (u32x4*)(a.xp + m * a.K);
    for (int u = lane; u < U; u += 64) {
      uint32_t in[16];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const u32x4 v = row[4 * u + c];
        in[4 * c] = v[0]; in[4 * c + 1] = v[1]; in[4 * c + 2] = v[2]; in[4 * c + 3] = v[3];
      }
      uint32_t o[16];
#pragma unroll
      for (int p = 0; p < 16; ++p) {
        uint16_t hv[2];
#pragma unroll
        for (int k = 0; k < 2; ++k) {
          const int c = S::code_of_slot(2 * p + k);
          const uint32_t bits = (in[c >> 1] >> (16 * (c & 1))) & 0xFFFFu;
          if (a.xd == JQ_BF16)
            hv[k] = f32_to_f16_bits(__builtin_ldexpf(__uint_as_float(bits << 16), -e));
          else
            hv[k] = (uint16_t)bits;
        }
        o[p] = (uint32_t)hv[0] | ((uint32_t)hv[1] << 16);
      }
#pragma unroll
      for (int c = 0; c < 4; ++c) out[4 * u + c] = u32x4{o[4 * c], o[4 * c + 1], o[4 * c + 2], o[4 * c + 3]};
    }
  } else {
    // 8 threads per weight row, thread k taking groups [k * gc, (k + 1) * gc)
    const int64_t n = (int64_t)((int)blockIdx.x - a.xblocks) * 32 + (threadIdx.x >> 3);
    const int k = threadIdx.x & 7;
    const int gc = (a.G + 7) >> 3, g0 = k * gc, g1 = g0 + gc < a.G ? g0 + gc : a.G;
    const bool live = n < a.N;
    const uint16_t* s = (const uint16_t*)a.scales + (live ? n : 0) * a.G;
    const uint16_t* b = (const uint16_t*)a.biases + (live ? n : 0) * a.G;
    auto f32_of = [&](uint32_t h) {
      return a.sb == JQ_BF16 ? bf16_bits_to_f32(h) : f16_bits_to_f32((uint16_t)h);
    };
    float mx = 0.f;
    for (int g = g0; live && g < g1; ++g) {
      const float sv = f32_of(s[g]), bv = f32_of(b[g]);
      mx = fmaxf(mx, fmaxf(fabsf(bv), fabsf(fmaf(sv, (float)a.qmax, bv))));
    }
#pragma unroll
    for (int o = 1; o < 8; o <<= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
    if (!live) return;
    const int f = exp_for(mx, 14);
    if (k == 0) a.ecol[n] = f;
    // (s', b') = (s, b) 2^-f in f16 (exact for bf16 and f16 sidecars in range), group-major
    for (int g = g0; g < g1; ++g)
      a.sbp[(int64_t)g * a.N + n] = (uint32_t)f32_to_f16_bits(__builtin_ldexpf(f32_of(s[g]), -f)) |
                                   ((uint32_t)f32_to_f16_bits(__builtin_ldexpf(f32_of(b[g]), -f)) << 16);
  }
}

template <int BITS, int SB>
int launch_g16(const G16Args& a, hipStream_t st) {
  using L = G16<BITS>;
  const void* kern = (const void*)gemm16_kernel<BITS, SB>;
  if (!jqh::set_lds(kern, L::LDS)) return JQ_ERR_LAUNCH;
  dim3 grid((unsigned)((a.N + BN - 1) / BN), (unsigned)((a.M + BM - 1) / BM));
  gemm16_kernel<BITS, SB><<<grid, NTH, L::LDS, st>>>(a);
  return jqh::launch_status();
}

template <int BITS>
int run_bits(const PrepArgs& p, const G16Args& g, bool cols, int sb, hipStream_t st) {
  PrepArgs q = p;
  q.xblocks = (int)((p.M + 3) / 4);
  const int cblocks = cols ? (int)((p.N + 31) / 32) : 0;
  prep_kernel<BITS><<<(unsigned)(q.xblocks + cblocks), 256, 0, st>>>(q);
  int s = jqh::launch_status();
  if (s) return s;
  return sb == JQ_BF16 ? launch_g16<BITS, JQ_BF16>(g, st) : launch_g16<BITS, JQ_F16>(g, st);
}

inline int64_t align256(int64_t v) { return (v + 255) & ~(int64_t)255; }

}  // namespace

namespace jqk {

bool gemm16_ok(int64_t M, int64_t K, int bits, int gs, int xd, int sb) {
  if (xd != JQ_BF16 && xd != JQ_F16) return false;
  if (sb != JQ_BF16 && sb != JQ_F16) return false;
  if (gs != 64 && gs != 128) return false;
  if (bits < 2 || bits > 8 || bits == 7) return false;
  return M >= 1 && K > 0 && K % gs == 0 && K <= kMaxK;
}

// Workspace of a pass over `rows` activation rows: x' [rows, K] f16, e [rows], f [N] and the
// (s', b') pairs [K / gs, N].
int64_t gemm16_workspace(int64_t rows, int64_t N, int64_t K, int gs) {
  return align256(rows * K * 2) + align256(rows * 4) + align256(N * 4) + align256(K / gs * N * 4);
}

int gemm16_launch(const QmmProblem& p, int bits, int gs, int xd, int sb, int yd, void* ws,
                  int64_t ws_bytes, hipStream_t st) {
  if (!gemm16_ok(p.M, p.K, bits, gs, xd, sb)) return JQ_ERR_SHAPE;
  if (p.M == 0 || p.N == 0) return JQ_OK;
  // Rows per pass: all of them when the workspace holds them, else whole 256-row tiles.
  int64_t rows = p.M;
  const int64_t fixed = align256(p.N * 4) + align256(p.K / gs * p.N * 4);
  if (gemm16_workspace(rows, p.N, p.K, gs) > ws_bytes) {
    const int64_t per = p.K * 2 + 4;
    rows = ((ws_bytes - fixed - 512) / per) / BM * BM;
    if (rows < BM) return JQ_ERR_WORKSPACE;
  }
  if (!ws) return JQ_ERR_NULL;
  uint8_t* base = (uint8_t*)ws;
  uint16_t* xp = (uint16_t*)base;
  int* erow = (int*)(base + align256(rows * p.K * 2));
  int* ecol = (int*)(base + align256(rows * p.K * 2) + align256(rows * 4));
  uint32_t* sbp = (uint32_t*)(base + align256(rows * p.K * 2) + align256(rows * 4) + align256(p.N * 4));
  const int G = (int)(p.K / gs);
  const int xs = 2, ys = jqh::dtype_size(yd);
  for (int64_t m0 = 0; m0 < p.M; m0 += rows) {
    const int64_t mr = p.M - m0 < rows ? p.M - m0 : rows;
    PrepArgs pa;
    pa.x = (const uint8_t*)p.x + m0 * p.K * xs;
    pa.xp = xp;
    pa.erow = erow;
    pa.scales = p.scales;
    pa.biases = p.biases;
    pa.ecol = ecol;
    pa.sbp = sbp;
    pa.M = mr;
    pa.N = p.N;
    pa.K = (int)p.K;
    pa.G = G;
    pa.qmax = (1 << bits) - 1;
    pa.xd = xd;
    pa.sb = sb;
    G16Args ga;
    ga.xp = xp;
    ga.erow = erow;
    ga.ecol = ecol;
    ga.sbp = sbp;
    ga.codes = p.codes;
    ga.y = (uint8_t*)p.y + m0 * p.N * ys;
    ga.M = mr;
    ga.N = p.N;
    ga.K = (int)p.K;
    ga.G = G;
    ga.gs = gs;
    ga.yd = yd;
    const bool cols = m0 == 0;
    int s;
    switch (bits) {
      case 2: s = run_bits<2>(pa, ga, cols, sb, st); break;
      case 3: s = run_bits<3>(pa, ga, cols, sb, st); break;
      case 4: s = run_bits<4>(pa, ga, cols, sb, st); break;
      case 5: s = run_bits<5>(pa, ga, cols, sb, st); break;
      case 6: s = run_bits<6>(pa, ga, cols, sb, st); break;
      default: s = run_bits<8>(pa, ga, cols, sb, st); break;
    }
    if (s) return s;
  }
  return JQ_OK;
}

}  // namespace jqk

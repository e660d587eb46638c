// Decode-batch quantized matmul on matrix cores with the weights streamed through LDS by
// direct-to-LDS buffer loads: y = x @ deq(W)^T for up to 2 * 16/(128/gs) activation rows per
// pass, dense (one or several problems sharing x) or expert-gathered (MoE tiles of a plan).
//
// Arithmetic (jq_dec.h, as the register-streamed decode kernel): lane (r = l%16, g = l/16)
// feeds unit g of each 128-code step of W row r into v_mfma_f32_16x16x32 B fragments; the
// step's 128/gs groups are folded into the MFMA M dimension, so every accumulator slot
// belongs to one (token, group) and takes  acc += s_g * D + b_g * X,  D = sum q*x exactly
// (the per-group affine sum s * sum q x + b * sum x, jang-tools/jang_tools/dsv41/metal_decode.py:202-233).
//
// Memory path. Wave w of a block owns SW consecutive 128-code steps of every item (RT tiles
// of 16 W rows). Per item it copies its piece of each row (SW*16*BITS bytes, contiguous in
// HBM) and of the rows' scales and biases straight into its own LDS ring with
// buffer_load ... lds: one instruction moves 1 KB as 8 rows x 128 B runs (16 B per lane), so
// address and cache-line work per byte is that of a contiguous stream, where register
// fragments would make every load instruction touch 16 rows. Rows sit at a stride of piece +
// 16 B in LDS, which spreads the 16 rows of a fragment read over the banks. The ring holds
// NSLOT items; the copy of item k + NSLOT - 1 is issued before item k is computed, and the
// wave waits only for its own copies of item k (a vector-memory count, no barrier), so
// NSLOT - 1 items of HBM traffic stay in flight. The activations of the wave's steps are
// held in registers as A fragments (loaded once per pass, or per tile when gathering), with
// their MFMA row sums X and offset sums O.
//
// One barrier per item: each wave writes its folded partials to LDS, then the waves sum the
// KW partials, one output slot per wave in turn, and store them (gathered gate|up pairs:
// h = silu(g) * u with the bf16 roundings of the stock path).
#include "jq_gemv.h"
#include "jq_qmv.h"

#define JQ_LDS __attribute__((address_space(3)))

namespace {

using namespace jq;
using namespace jqd;
using jqg::Rsrc;
using jqg::make_rsrc;
using jqk::GatherPlan;
using jqk::QmmProblem;
using jqk::QmvBatch;
using jqk::QmvProblem;

constexpr int kMaxKW = 8;
constexpr int kLdsMax = 156 * 1024;

struct DmxArgs {
  // dense
  QmvBatch b;
  int rb_begin[jqk::kMaxProblems + 1];
  int nprob;
  int mpass, mtotal;  // activation rows per pass (blockIdx.y is the pass) and in all

  // gathered
  QmmProblem g[2];
  GatherPlan plan;
  // dense with K split into chunks of `split` steps: fp32 partials [chunk][mtotal][N]
  int split;
  float* part;
  // both
  int nrb;     // gathered: row blocks per tile (split: row blocks of the matrix)
  int items;   // dense: total items (gathered: read from the plan)
  int K;
  int yd;
};

// Compile-time layout of one wave's ring.
template <class D, int RT, int SW, int NSLOT>
struct Ring {
  static constexpr int PB = SW * 16 * D::BITS;                  // piece bytes per row
  static constexpr int RS = PB + 16;                            // LDS row stride
  // A tile's rows fill 16 * RS bytes exactly: copies of 16 B per lane (1 KB each), then
  // copies of 4 B per lane (256 B each) for the rest.
  static constexpr int CODE_INSTR = 16 * RS / 1024;             // b128 copies per tile
  static constexpr int TAIL_INSTR = (16 * RS - 1024 * CODE_INSTR) / 256;  // b32 copies
  static constexpr int CODE_AREA = 16 * RS;
  static_assert((16 * RS) % 256 == 0, "whole b32 copies");
  static constexpr int SBP = SW * D::GSTEP * 2;                 // scale bytes per row piece
  static constexpr int SB_INSTR = (16 * SBP + 255) / 256;       // b32 copies per tile and array
  static constexpr int SB_AREA = SB_INSTR * 256;
  static constexpr int TILE = CODE_AREA + 2 * SB_AREA;
  static constexpr int SLOT = RT * TILE;
  static constexpr int WAVE = NSLOT * SLOT;
  static constexpr int ND = RT * (CODE_INSTR + TAIL_INSTR + 2 * SB_INSTR);  // copies per item
};

// Wave-uniform reads of plan data through the constant address space: scalar loads, counted
// by the LDS/scalar counter, so they never wait for the ring's copies.
template <class T>
JQ_DEV T ldc(const T* p) {
  return *(const __attribute__((address_space(4))) T*)p;
}

JQ_DEV float round_to(float v, int yd) {
  if (yd == JQ_BF16) return bf16_bits_to_f32(f32_to_bf16_bits(v));
  if (yd == JQ_F16) return f16_bits_to_f32(f32_to_f16_bits(v));
  return v;
}

JQ_DEV void store_out(void* y, int64_t idx, float v, int yd) {
  if (yd == JQ_BF16) ((uint16_t*)y)[idx] = f32_to_bf16_bits(v);
  else if (yd == JQ_F16) ((uint16_t*)y)[idx] = f32_to_f16_bits(v);
  else ((float*)y)[idx] = v;
}

// s_waitcnt with only the vector-memory count set (expcnt and lgkmcnt left free).
template <int N>
JQ_DEV void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// Workgroup barrier after this wave's LDS writes have landed. No memory fence: the fence of
// __syncthreads would also wait for every outstanding copy into the ring.
JQ_DEV void lds_barrier() {
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// An item's source rows: per tile, a buffer view of its 16 code rows and of the scale and
// bias rows (rows past the matrix, dead items and empty tiles are views of 0 bytes).
template <int RT>
struct ItemSrc {
  Rsrc c[RT], s[RT], b[RT];
};

// Token rows of a gathered tile, per lane: the x row this lane's A fragments read (slot
// xt = lr / GSTEP) and the output rows of the TPL token slots it stores (TPL * lg + k).
template <int TPL>
struct LaneToks {
  int64_t xrow;
  bool xlive;
  int64_t orow[TPL];
  bool olive[TPL];
};

template <int MP, int TPL>
JQ_DEV void lane_toks(const GatherPlan& pl, int4 tl, int xt, int lg, LaneToks<TPL>& lt) {
  lt.xrow = 0;
  lt.xlive = false;
#pragma unroll
  for (int k = 0; k < TPL; ++k) lt.orow[k] = 0, lt.olive[k] = false;
#pragma unroll
  for (int m = 0; m < MP; ++m) {
    if (m < tl.z) {  // wave-uniform
      const int rr = tl.y + m;
      const int Mp = pl.M;
      const int pi = Mp == 1 ? rr : rr / Mp, mi = Mp == 1 ? 0 : rr - pi * Mp;
      const uint32_t pair = ldc(pl.order + tl.w + pi);
      const int64_t xr = (int64_t)(pl.lhs ? ldc(pl.lhs + pair) : pair / (uint32_t)pl.pair_div) * Mp + mi;
      const bool live = xr < pl.x_rows;
      if (xt == m) lt.xrow = live ? xr : 0, lt.xlive = live;
#pragma unroll
      for (int k = 0; k < TPL; ++k)
        if (TPL * lg + k == m) lt.orow[k] = (int64_t)pair * Mp + mi, lt.olive[k] = true;
    }
  }
}

// SPLIT (dense, one problem): unit u of the item walk is a K chunk of a.split steps; its
// partial sums go to a.part and a second kernel adds the chunks.
// DGLU (dense, problems 0 = gate and 1 = up of one shape): items alternate gate and up of one
// row block (item 2j: gate rows of block j, 2j + 1: up rows), both in the same block; the
// reducing wave of an output keeps the rounded gate value in a register and the up item
// stores silu(g) * u (glu_value with a.g[0].glu_limit) into problem 0's output.
template <class D, int SB, int RT, int NA, int SW, int NSLOT, bool GATHER, int NB, bool SPLIT = false,
          bool DGLU = false>
struct Dmx {
  using R = Ring<D, RT, SW, NSLOT>;
  static constexpr int BITS = D::BITS, TPB = D::TPB, TPL = 4 / D::GSTEP;
  static constexpr int MP = NA * TPB;            // token slots of a pass or tile
  static constexpr int NOUT = RT * NA * TPL;     // partial outputs per lane per item
  // X and O kept per step in registers: always up to 4 steps of activation blocks, and up to
  // 8 in the plain dense form at <= 6 bits (<= 5 with the K split), where the gfx950 build's
  // resource report shows no spill; elsewhere they are recomputed per item.
  static constexpr bool PRE =
      NA * SW <= 4 || (NA * SW <= 8 && !GATHER && !DGLU && BITS <= (SPLIT ? 5 : 6));

  // Per-lane byte offsets of the copies inside a tile's rows (the same for every item):
  // copy j, lane i lands at LDS byte 1024 j + 16 i of the tile = (row f / RS, byte f % RS);
  // pad lanes and lanes past the 16 rows repeat row 0's first chunk.
  struct Offs {
    uint32_t c[R::CODE_INSTR];
    uint32_t tail[R::TAIL_INSTR];  // the 4-byte copies of the rest
    uint32_t s[R::SB_INSTR];
  };

  static JQ_DEV void offsets(int lane, uint32_t rowbytes, uint32_t sbrow, int s0, Offs& o) {
#pragma unroll
    for (int j = 0; j < R::CODE_INSTR; ++j) {
      const int f = 1024 * j + 16 * lane;
      const int row = f / R::RS, byte = f % R::RS;
      const bool ok = row < 16 && byte < R::PB;
      o.c[j] = ok ? (uint32_t)row * rowbytes + (uint32_t)(s0 * 16 * BITS + byte)
                  : (uint32_t)(s0 * 16 * BITS);
    }
#pragma unroll
    for (int j = 0; j < R::TAIL_INSTR; ++j) {
      const int f = 1024 * R::CODE_INSTR + 256 * j + 4 * lane;
      const int row = f / R::RS, byte = f % R::RS;
      const bool ok = row < 16 && byte < R::PB;
      o.tail[j] = ok ? (uint32_t)row * rowbytes + (uint32_t)(s0 * 16 * BITS + byte)
                     : (uint32_t)(s0 * 16 * BITS);
    }
#pragma unroll
    for (int j = 0; j < R::SB_INSTR; ++j) {
      const int f = 256 * j + 4 * lane;
      const int row = f / R::SBP, byte = f % R::SBP;
      const bool ok = row < 16;
      o.s[j] = ok ? (uint32_t)row * sbrow + (uint32_t)(s0 * D::GSTEP * 2 + byte)
                  : (uint32_t)(s0 * D::GSTEP * 2);
    }
  }

  // Copy an item into a ring slot (always the same number of copies).
  static JQ_DEV void copy(const ItemSrc<RT>& src, const Offs& o, JQ_LDS uint8_t* __restrict__ slot) {
#pragma unroll
    for (int r = 0; r < RT; ++r) {
      JQ_LDS uint8_t* t = slot + r * R::TILE;
#pragma unroll
      for (int j = 0; j < R::CODE_INSTR; ++j)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(src.c[r], (JQ_LDS void*)(t + 1024 * j), 16, o.c[j], 0, 0, 0);
#pragma unroll
      for (int j = 0; j < R::TAIL_INSTR; ++j)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(src.c[r], (JQ_LDS void*)(t + 1024 * R::CODE_INSTR + 256 * j), 4, o.tail[j], 0, 0, 0);
#pragma unroll
      for (int j = 0; j < R::SB_INSTR; ++j) {
        __builtin_amdgcn_raw_ptr_buffer_load_lds(src.s[r], (JQ_LDS void*)(t + R::CODE_AREA + 256 * j), 4, o.s[j], 0, 0, 0);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(src.b[r], (JQ_LDS void*)(t + R::CODE_AREA + R::SB_AREA + 256 * j), 4, o.s[j], 0, 0, 0);
      }
    }
  }

  // A fragments of the wave's steps for the token slots of a pass / tile, and their sums.
  struct Act {
    u32x4 A[NA][SW][4];
    f32x4 X[PRE ? NA : 1][PRE ? SW : 1], O[PRE ? NA : 1][PRE ? SW : 1];
  };

  static JQ_DEV void sums(const u32x4 (&A)[4], f32x4& X, f32x4& O) {
    const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
    const u32x4 ones = {D::ONE2, D::ONE2, D::ONE2, D::ONE2};
    constexpr u32x4 BO0 = {bo_dword<D>(0, 0), bo_dword<D>(0, 1), bo_dword<D>(0, 2), bo_dword<D>(0, 3)};
    constexpr u32x4 BO1 = {bo_dword<D>(1, 0), bo_dword<D>(1, 1), bo_dword<D>(1, 2), bo_dword<D>(1, 3)};
    constexpr u32x4 BO2 = {bo_dword<D>(2, 0), bo_dword<D>(2, 1), bo_dword<D>(2, 2), bo_dword<D>(2, 3)};
    constexpr u32x4 BO3 = {bo_dword<D>(3, 0), bo_dword<D>(3, 1), bo_dword<D>(3, 2), bo_dword<D>(3, 3)};
    X = mfma16<D::XDT>(A[0], ones, zero);
    X = mfma16<D::XDT>(A[1], ones, X);
    X = mfma16<D::XDT>(A[2], ones, X);
    X = mfma16<D::XDT>(A[3], ones, X);
    O = mfma16<D::XDT>(A[0], BO0, zero);
    O = mfma16<D::XDT>(A[1], BO1, O);
    O = mfma16<D::XDT>(A[2], BO2, O);
    O = mfma16<D::XDT>(A[3], BO3, O);
  }

  // Lane (lr, lg) of activation block ab feeds token slot ab*TPB + lr/GSTEP in the lane
  // groups of group lr % GSTEP; other lanes hold zeros. Only the lanes of live token slots
  // load (the others are masked off and send no request), so a block moves each activation
  // value once.
  template <class XRow>
  static JQ_DEV void issue_act(const uint16_t* x, int K, int s0, int lr, int lg, XRow xrow,
                               XRaw (&raw)[NA][SW]) {
#pragma unroll
    for (int ab = 0; ab < NA; ++ab) {
      const int t = ab * TPB + lr / D::GSTEP;
      int64_t row;
      const bool act = (lr % D::GSTEP) == lg / D::LPG && xrow(t, row);
#pragma unroll
      for (int d = 0; d < SW; ++d) {
        if (act) {
          load_xraw(x + row * K + (int64_t)(s0 + d) * 128 + 32 * lg, raw[ab][d]);
        } else {
#pragma unroll
          for (int q = 0; q < 16; ++q) raw[ab][d].d[q] = 0u;
        }
      }
    }
  }

  static JQ_DEV void finish_act(const XRaw (&raw)[NA][SW], Act& ac) {
#pragma unroll
    for (int ab = 0; ab < NA; ++ab)
#pragma unroll
      for (int d = 0; d < SW; ++d) {
        ac.A[ab][d][0] = a_frag<D, 0>(raw[ab][d]);
        ac.A[ab][d][1] = a_frag<D, 1>(raw[ab][d]);
        ac.A[ab][d][2] = a_frag<D, 2>(raw[ab][d]);
        ac.A[ab][d][3] = a_frag<D, 3>(raw[ab][d]);
      }
    if constexpr (PRE) {
#pragma unroll
      for (int ab = 0; ab < NA; ++ab)
#pragma unroll
        for (int d = 0; d < SW; ++d) sums(ac.A[ab][d], ac.X[ab][d], ac.O[ab][d]);
    }
  }

  template <class XRow>
  static JQ_DEV void load_act(const uint16_t* x, int K, int s0, int lr, int lg, XRow xrow, Act& ac) {
    XRaw raw[NA][SW];
    issue_act(x, K, s0, lr, lg, xrow, raw);
    finish_act(raw, ac);
  }

  // The MFMAs and scale terms of one item from its ring slot.
  static JQ_DEV void compute(const JQ_LDS uint8_t* __restrict__ slot, const Act& ac, const Bases<D>& bs,
                             int lr, int lg, f32x4 (&acc)[NA][RT]) {
    const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ab = 0; ab < NA; ++ab)
#pragma unroll
      for (int r = 0; r < RT; ++r) acc[ab][r] = zero;
#pragma unroll
    for (int d = 0; d < SW; ++d) {
      f32x4 X[NA], O[NA];
#pragma unroll
      for (int ab = 0; ab < NA; ++ab) {
        if constexpr (PRE) {
          X[ab] = ac.X[ab][d];
          O[ab] = ac.O[ab][d];
        } else {
          sums(ac.A[ab][d], X[ab], O[ab]);
        }
      }
#pragma unroll
      for (int r = 0; r < RT; ++r) {
        const JQ_LDS uint8_t* t = slot + r * R::TILE;
        uint32_t w[BITS];
        const JQ_LDS uint32_t* cw = (const JQ_LDS uint32_t*)(t + lr * R::RS + (4 * d + lg) * 4 * BITS);
#pragma unroll
        for (int q = 0; q < BITS; ++q) w[q] = cw[q];
        uint32_t sw[(D::GSTEP + 1) / 2], bw[(D::GSTEP + 1) / 2];
        const int sbo = lr * R::SBP + d * D::GSTEP * 2;
        if constexpr (D::GSTEP == 1) {
          sw[0] = *(const JQ_LDS uint16_t*)(t + R::CODE_AREA + sbo);
          bw[0] = *(const JQ_LDS uint16_t*)(t + R::CODE_AREA + R::SB_AREA + sbo);
        } else {
#pragma unroll
          for (int q = 0; q < (D::GSTEP + 1) / 2; ++q) {
            sw[q] = *(const JQ_LDS uint32_t*)(t + R::CODE_AREA + sbo + 4 * q);
            bw[q] = *(const JQ_LDS uint32_t*)(t + R::CODE_AREA + R::SB_AREA + sbo + 4 * q);
          }
        }
        f32x4 Dd[NA], Dh[NA];
#pragma unroll
        for (int ab = 0; ab < NA; ++ab) { Dd[ab] = O[ab]; Dh[ab] = zero; }
#define JQ_F(F)                                                                  \
        {                                                                        \
          u32x4 B, BH;                                                           \
          b_frag<D, F>(w, bs, B, BH);                                            \
          _Pragma("unroll") for (int ab = 0; ab < NA; ++ab) {                    \
            Dd[ab] = mfma16<D::XDT>(ac.A[ab][d][F], B, Dd[ab]);                  \
            if constexpr (D::NIB) Dh[ab] = mfma16<D::XDT>(ac.A[ab][d][F], BH, Dh[ab]); \
          }                                                                      \
        }
        JQ_F(0) JQ_F(1) JQ_F(2) JQ_F(3)
#undef JQ_F
        float sc[4], bi[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int j = i % D::GSTEP;
          sc[i] = half_to_f32<SB>(sw[j >> 1], j & 1);
          bi[i] = half_to_f32<SB>(bw[j >> 1], j & 1);
        }
#pragma unroll
        for (int ab = 0; ab < NA; ++ab)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float dv = D::NIB ? fmaf(16.f, Dh[ab][i], Dd[ab][i]) : Dd[ab][i];
            acc[ab][r][i] = fmaf(sc[i], dv, fmaf(bi[i], X[ab][i], acc[ab][r][i]));
          }
      }
    }
  }

  // Rows of W per item, and between the tiles of an item (gate|up pairs share their rows).
  static constexpr int IROWS = NB == 2 ? 16 : 16 * RT;
  static constexpr int TSTEP = NB == 2 ? 0 : 16;

  // Wave-uniform walk over items in order: unit u (a plan tile when gathering, a problem
  // otherwise) and row block rb inside it, with the unit's source base pointers. Moving to
  // the next item needs no division; a new unit reloads its tile and bases.
  struct Cursor {
    int it, u, rb, nrb;
    int64_t N;              // rows of the unit's matrices
    int ez;                 // gathered: the tile has rows (0: nothing to read or store)
    const char* cb[RT];     // codes of the unit's row 0 (per tile)
    const char* sb[RT];     // scales
    const char* bb[RT];     // biases
    const char *ocb, *osb, *obb;  // DGLU: the other unit's codes, scales and biases
  };

  static JQ_DEV void unit_bases(const DmxArgs& a, Cursor& c, int4* tlo) {
    if constexpr (GATHER) {
      int4 tl = make_int4(0, 0, 0, 0);
      if (c.u < ldc(a.plan.n_tiles)) {
        const int* tp = (const int*)(a.plan.tiles + c.u);
        tl = make_int4(ldc(tp), ldc(tp + 1), ldc(tp + 2), ldc(tp + 3));
      }
      if (tlo) *tlo = tl;
      c.ez = tl.z > 0;
      c.N = a.g[0].N;
      c.nrb = a.nrb;
#pragma unroll
      for (int r = 0; r < RT; ++r) {
        const QmmProblem& pb = a.g[NB == 2 ? r : 0];
        const int64_t e = tl.x;
        c.cb[r] = (const char*)(pb.codes + e * pb.expert_stride_codes);
        c.sb[r] = (const char*)pb.scales + e * pb.expert_stride_sb * 2;
        c.bb[r] = (const char*)pb.biases + e * pb.expert_stride_sb * 2;
      }
    } else if constexpr (SPLIT) {
      if (tlo) *tlo = make_int4(0, 0, 0, 0);
      const QmvProblem& pb = a.b.p[0];
      c.ez = 1;
      c.N = pb.N;
      c.nrb = a.nrb;
      const int64_t cbyte = (int64_t)c.u * a.split * 16 * BITS;  // chunk start inside a row
      const int64_t sbyte = (int64_t)c.u * a.split * D::GSTEP * 2;
#pragma unroll
      for (int r = 0; r < RT; ++r) {
        c.cb[r] = (const char*)pb.codes + cbyte;
        c.sb[r] = (const char*)pb.scales + sbyte;
        c.bb[r] = (const char*)pb.biases + sbyte;
      }
    } else {
      if (tlo) *tlo = make_int4(0, 0, 0, 0);
      const int u = c.u < a.nprob ? c.u : a.nprob - 1;
      const QmvProblem& pb = a.b.p[u];
      c.ez = 1;
      c.N = pb.N;
      c.nrb = a.rb_begin[u + 1] - a.rb_begin[u];
#pragma unroll
      for (int r = 0; r < RT; ++r) {
        c.cb[r] = (const char*)pb.codes;
        c.sb[r] = (const char*)pb.scales;
        c.bb[r] = (const char*)pb.biases;
      }
    }
  }

  static JQ_DEV void cursor_at(const DmxArgs& a, int it, Cursor& c, int4* tlo) {
    c.it = it;
    if constexpr (DGLU) {
      c.u = it & 1;
      c.rb = it >> 1;
      const QmvProblem& po = a.b.p[c.u ^ 1];
      c.ocb = (const char*)po.codes;
      c.osb = (const char*)po.scales;
      c.obb = (const char*)po.biases;
    } else if constexpr (GATHER || SPLIT) {
      c.u = it / a.nrb;
      c.rb = it - c.u * a.nrb;
    } else {
      int u = 0;
#pragma unroll
      for (int q = 1; q < jqk::kMaxProblems; ++q)
        if (q < a.nprob && it >= a.rb_begin[q]) u = q;
      c.u = u;
      c.rb = it - a.rb_begin[u];
    }
    unit_bases(a, c, tlo);
  }

  // Returns whether the unit changed.
  static JQ_DEV bool advance(const DmxArgs& a, Cursor& c, int4* tlo) {
    ++c.it;
    if constexpr (DGLU) {
      // gate and up share N: swap the two units' bases instead of reading them again
      c.u ^= 1;
      c.rb += c.u ^ 1;
      const char* t = c.cb[0]; c.cb[0] = c.ocb; c.ocb = t;
      t = c.sb[0]; c.sb[0] = c.osb; c.osb = t;
      t = c.bb[0]; c.bb[0] = c.obb; c.obb = t;
      return true;
    }
    if (++c.rb < c.nrb) return false;
    c.rb = 0;
    ++c.u;
    if constexpr (!GATHER && !SPLIT) {
      while (c.u < a.nprob && a.rb_begin[c.u + 1] == a.rb_begin[c.u]) ++c.u;  // empty problems
    }
    unit_bases(a, c, tlo);
    return true;
  }

  // Buffer views of the cursor's item (0 bytes when dead or empty).
  static JQ_DEV void sources(const Cursor& c, bool live, uint32_t rowbytes, uint32_t sbrow,
                             ItemSrc<RT>& src) {
#pragma unroll
    for (int r = 0; r < RT; ++r) {
      const int64_t r0 = (int64_t)c.rb * IROWS + TSTEP * r;
      const int64_t left = c.N - r0;
      const uint32_t rows = live && c.ez && left > 0 ? (uint32_t)(left < 16 ? left : 16) : 0u;
      src.c[r] = make_rsrc(c.cb[r] + r0 * rowbytes, rows * rowbytes);
      src.s[r] = make_rsrc(c.sb[r] + r0 * sbrow, rows * sbrow);
      src.b[r] = make_rsrc(c.bb[r] + r0 * sbrow, rows * sbrow);
    }
  }

  static JQ_DEV void run(const DmxArgs& a, JQ_LDS uint8_t* __restrict__ ring0,
                         JQ_LDS uint8_t* __restrict__ ring1, JQ_LDS uint8_t* __restrict__ ring2,
                         JQ_LDS uint8_t* __restrict__ ring3, JQ_LDS float* __restrict__ red) {
    const int items = GATHER ? ldc(a.plan.n_tiles) * a.nrb : a.items;
    int per = (items + (int)gridDim.x - 1) / (int)gridDim.x;
    if constexpr (DGLU) per += per & 1;  // whole (gate, up) pairs per block
    const int first = blockIdx.x * per;
    const int end = first + per < items ? first + per : items;
    if (first >= end) return;  // whole block
    const int KW = blockDim.x >> 6;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lr = lane & 15, lg = lane >> 4;
    const int s0 = wave * SW;
    // Dense: the pass of this block (all passes share the weights, read again from the cache).
    const int pm0 = GATHER ? 0 : (int)blockIdx.y * a.mpass;
    const int pmr = GATHER ? 0 : (a.mtotal - pm0 < a.mpass ? a.mtotal - pm0 : a.mpass);
    const uint32_t rowbytes = (uint32_t)(a.K / 32) * BITS * 4;
    const uint32_t sbrow = (uint32_t)(a.K / D::GS) * 2;
    Offs o;
    offsets(lane, rowbytes, sbrow, s0, o);

    // Ring prologue: items first .. first + NSLOT - 2 (the copy cursor ends on the next).
    Cursor cc, wc;  // copy cursor (NSLOT - 1 items ahead) and work cursor
    int4 tl;
    cursor_at(a, first, wc, &tl);
    cc = wc;
    // The first item's activations are requested before the ring's first copies and turned
    // into A fragments after them, so that both round trips overlap.
    Act ac;
    LaneToks<TPL> tk;
    {
      XRaw raw[NA][SW];
      if constexpr (GATHER) {
        lane_toks<MP, TPL>(a.plan, tl, lr / D::GSTEP, lg, tk);
        issue_act((const uint16_t*)a.g[0].x, a.K, s0, lr, lg,
                  [&](int, int64_t& row) { row = tk.xrow; return tk.xlive; }, raw);
      } else {
        issue_act((const uint16_t*)a.b.p[0].x, a.K, s0 + (SPLIT ? wc.u * a.split : 0), lr, lg,
                  [&](int t, int64_t& row) { row = pm0 + t; return t < pmr; }, raw);
      }
#pragma unroll
      for (int k = 0; k < NSLOT - 1; ++k) {
        ItemSrc<RT> src;
        sources(cc, cc.it < end, rowbytes, sbrow, src);
        copy(src, o, k == 0 ? ring0 : k == 1 ? ring1 : ring2);  // k < NSLOT - 1 <= 3
        asm volatile("" ::: "memory");
        advance(a, cc, nullptr);
      }
      finish_act(raw, ac);
    }
    const Bases<D> bs = make_bases<D>();
    float gk[NOUT];  // DGLU: rounded gate values of the wave's outputs, kept for the up item

    auto step = [&](int it, JQ_LDS uint8_t* __restrict__ cur, JQ_LDS uint8_t* __restrict__ fill) {
      const int par = (it - first) & 1;  // partials double-buffered across consecutive items
      // Copy of item it + NSLOT - 1 (the copy cursor) into the slot freed by item it - 1.
      {
        ItemSrc<RT> s2;
        sources(cc, cc.it < end, rowbytes, sbrow, s2);
        copy(s2, o, fill);
        advance(a, cc, nullptr);
      }
      const int64_t row0 = (int64_t)wc.rb * IROWS;
      static_assert((NSLOT - 1) * R::ND <= 63, "vmcnt range");
      wait_vm<(NSLOT - 1) * R::ND>();
      asm volatile("" ::: "memory");
      f32x4 acc[NA][RT];
      compute(cur, ac, bs, lr, lg, acc);
      JQ_LDS float* mine = red + ((par * KW + wave) * NOUT) * 64;
#pragma unroll
      for (int ab = 0; ab < NA; ++ab)
#pragma unroll
        for (int r = 0; r < RT; ++r) {
          float v[TPL];
          fold_groups<D>(acc[ab][r], v);
#pragma unroll
          for (int k = 0; k < TPL; ++k) mine[((ab * RT + r) * TPL + k) * 64 + lane] = v[k];
        }
      lds_barrier();
      // Sum the waves' partials and store: output slot o = (ab, r, k); gathered gate|up
      // pairs take r = 0 (gate) and r = 1 (up) together.
      constexpr int NO = NB == 2 ? NOUT / 2 : NOUT;
      if constexpr (DGLU) {
        static_assert(RT == 1 && NB == 1 && !GATHER && !SPLIT, "dense gate|up pairs");
        const bool up = wc.u == 1;
#pragma unroll
        for (int j = 0; j < NOUT; ++j) {
          const int oi = wave + j * KW;  // output slot (ab, k) = (oi / TPL, oi % TPL)
          if (oi < NOUT) {
            float v = 0.f;
#pragma unroll
            for (int w = 0; w < kMaxKW; ++w)
              if (w < KW) v += red[((par * KW + w) * NOUT + oi) * 64 + lane];
            const float rv = round_to(v, a.yd);
            if (!up) {
              gk[j] = rv;
            } else {
              const int tok = (oi / TPL) * TPB + TPL * lg + oi % TPL;
              const int64_t n = row0 + lr;
              if (tok < pmr && n < wc.N)
                store_out(a.b.p[0].y, (int64_t)(pm0 + tok) * wc.N + n,
                          jqk::glu_value(gk[j], rv, a.g[0].glu_limit, 1.f), a.yd);
            }
          }
        }
      }
      for (int oi = wave; oi < (DGLU ? 0 : NO); oi += KW) {
        const int k = oi % TPL;
        const int rr = NB == 2 ? 0 : (oi / TPL) % RT;
        const int ab = NB == 2 ? oi / TPL : oi / (TPL * RT);
        const int slot0 = (ab * RT + rr) * TPL + k;
        float v = 0.f;
#pragma unroll
        for (int w = 0; w < kMaxKW; ++w)
          if (w < KW) v += red[((par * KW + w) * NOUT + slot0) * 64 + lane];
        const int tok = ab * TPB + TPL * lg + k;
        if constexpr (GATHER) {
          const int64_t N = wc.N;
          const int64_t n = row0 + TSTEP * rr + lr;
          int64_t orow = tk.orow[0];
          bool live = tk.olive[0];
#pragma unroll
          for (int q = 1; q < TPL; ++q)
            if (k == q) orow = tk.orow[q], live = tk.olive[q];
          if constexpr (NB == 2) {
            float u = 0.f;
            const int slot1 = (ab * RT + 1) * TPL + k;
#pragma unroll
            for (int w = 0; w < kMaxKW; ++w)
              if (w < KW) u += red[((par * KW + w) * NOUT + slot1) * 64 + lane];
            const float gg = round_to(v, a.yd), uu = round_to(u, a.yd);
            const jqk::QmmProblem& gp = a.g[0];
            v = jqk::glu_value(gg, uu, gp.glu_limit,
                               gp.glu_scale && live ? gp.glu_scale[orow] : 1.f);
          }
          if (live && n < N) store_out(a.g[0].y, orow * N + n, v, a.yd);
        } else {
          const int64_t n = row0 + 16 * rr + lr;
          if constexpr (SPLIT) {
            if (tok < pmr && n < wc.N) a.part[((int64_t)wc.u * a.mtotal + pm0 + tok) * wc.N + n] = v;
          } else {
            const QmvProblem& pb = a.b.p[wc.u < a.nprob ? wc.u : a.nprob - 1];
            if (tok < pmr && n < wc.N) store_out(pb.y, (int64_t)(pm0 + tok) * wc.N + n, v, a.yd);
          }
        }
      }
      // Next item (and, when its tile differs, its activations).
      if (it + 1 < end) {
        if (advance(a, wc, &tl)) {
          if constexpr (GATHER) {
            lane_toks<MP, TPL>(a.plan, tl, lr / D::GSTEP, lg, tk);
            load_act((const uint16_t*)a.g[0].x, a.K, s0, lr, lg, [&](int, int64_t& row) { row = tk.xrow; return tk.xlive; }, ac);
          } else if constexpr (SPLIT) {
            load_act((const uint16_t*)a.b.p[0].x, a.K, s0 + wc.u * a.split, lr, lg,
                     [&](int t, int64_t& row) { row = pm0 + t; return t < pmr; }, ac);
          }
        }
      }
    };

    // Items in ring order (slot = k % NSLOT at compile time): item k computes from slot
    // k % NSLOT and refills slot (k - 1) % NSLOT.
    for (int it = first; it < end; it += NSLOT) {
      if constexpr (NSLOT == 2) {
        step(it, ring0, ring1);
        if (it + 1 >= end) break;
        step(it + 1, ring1, ring0);
      } else if constexpr (NSLOT == 3) {
        step(it, ring0, ring2);
        if (it + 1 >= end) break;
        step(it + 1, ring1, ring0);
        if (it + 2 >= end) break;
        step(it + 2, ring2, ring1);
      } else {
        step(it, ring0, ring3);
        if (it + 1 >= end) break;
        step(it + 1, ring1, ring0);
        if (it + 2 >= end) break;
        step(it + 2, ring2, ring1);
        if (it + 3 >= end) break;
        step(it + 3, ring3, ring2);
      }
    }
  }
};

template <class D, int SB, int RT, int NA, int SW, int NSLOT, bool GATHER, int NB, bool SPLIT,
          bool DGLU>
__global__ void __launch_bounds__(64 * kMaxKW) dmx_kernel(DmxArgs a) {
  using K = Dmx<D, SB, RT, NA, SW, NSLOT, GATHER, NB, SPLIT, DGLU>;
  using R = typename K::R;
  extern __shared__ __attribute__((aligned(1024))) uint8_t dmx_lds[];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int KW = blockDim.x >> 6;
  JQ_LDS uint8_t* base = (JQ_LDS uint8_t*)dmx_lds;
  JQ_LDS uint8_t* w0 = base + wave * R::WAVE;
  JQ_LDS float* red = (JQ_LDS float*)(base + KW * R::WAVE);
  JQ_LDS uint8_t* s1 = w0 + R::SLOT;
  JQ_LDS uint8_t* s2 = w0 + (NSLOT >= 3 ? 2 : 0) * R::SLOT;
  JQ_LDS uint8_t* s3 = w0 + (NSLOT >= 4 ? 3 : 0) * R::SLOT;
  K::run(a, w0, s1, s2, s3, red);
}

template <class D, int RT, int NA, int SW, int NSLOT>
constexpr size_t dmx_lds_bytes(int kw) {
  using R = Ring<D, RT, SW, NSLOT>;
  return (size_t)kw * R::WAVE + (size_t)2 * kw * RT * NA * (4 / D::GSTEP) * 64 * 4;
}

template <class D, int SB, int RT, int NA, int SW, int NSLOT, bool GATHER, int NB, bool SPLIT,
          bool DGLU>
int launch_cfg(DmxArgs& a, int kw, int64_t max_items, hipStream_t st) {
  const size_t lds = dmx_lds_bytes<D, RT, NA, SW, NSLOT>(kw);
  if (lds > (size_t)kLdsMax) return JQ_ERR_SHAPE;
  auto kern = dmx_kernel<D, SB, RT, NA, SW, NSLOT, GATHER, NB, SPLIT, DGLU>;
  if (!jqh::set_lds((const void*)kern, lds)) return JQ_ERR_LAUNCH;
  int64_t cap = (int64_t)jqh::blocks_per_cu((const void*)kern, 64 * kw, lds) * jqh::cus();
  int64_t grid;
  int ny = 1;
  if constexpr (GATHER) {
    grid = max_items < cap ? max_items : cap;  // items are read from the plan on the device
  } else {
    // Passes of activation rows side by side (grid y), sharing the resident-block capacity.
    ny = (a.mtotal + a.mpass - 1) / a.mpass;
    cap = cap / ny > 0 ? cap / ny : 1;
    const int64_t iters = (max_items + cap - 1) / cap;
    grid = (max_items + iters - 1) / iters;
  }
  if (grid < 1 || ny < 1) return JQ_OK;
  kern<<<dim3((unsigned)grid, (unsigned)ny), 64 * kw, lds, st>>>(a);
  return jqh::launch_status();
}

// Ring depth: the most items (4, 3 or 2) that fit the LDS budget at kMaxKW waves and the
// vector-memory count.
template <class D, int RT, int NA, int SW>
constexpr int ring_slots() {
  constexpr int nd = Ring<D, RT, SW, 2>::ND;
  if (dmx_lds_bytes<D, RT, NA, SW, 4>(kMaxKW) <= (size_t)kLdsMax && 3 * nd <= 63) return 4;
  if (dmx_lds_bytes<D, RT, NA, SW, 3>(kMaxKW) <= (size_t)kLdsMax && 2 * nd <= 63) return 3;
  return 2;
}

// Steps per wave: 4 when K has a multiple of 4 steps that at most kMaxKW waves cover, else 2.
inline int dmx_sw(int K) {
  const int S = K / 128;
  if (S % 4 == 0 && S / 4 <= kMaxKW) return 4;
  if (S % 2 == 0 && S / 2 <= kMaxKW) return 2;
  return 0;
}

template <class D, int SB, int RT, int NA, bool GATHER, int NB, bool SPLIT = false,
          bool DGLU = false>
int launch_sw(DmxArgs& a, int64_t max_items, hipStream_t st) {
  const int kc = SPLIT ? a.split * 128 : a.K;  // codes of K one block covers
  const int sw = dmx_sw(kc);
  const int kw = sw ? kc / 128 / sw : 0;
  if (sw == 2)
    return launch_cfg<D, SB, RT, NA, 2, ring_slots<D, RT, NA, 2>(), GATHER, NB, SPLIT, DGLU>(a, kw, max_items, st);
  if (sw == 4)
    return launch_cfg<D, SB, RT, NA, 4, ring_slots<D, RT, NA, 4>(), GATHER, NB, SPLIT, DGLU>(a, kw, max_items, st);
  return JQ_ERR_SHAPE;
}

// Dense: passes of TPB (one activation block) or 2 TPB rows, all in one launch. Passes of
// one block are taken when every (pass, row block) item still gets a CU of its own (short
// outputs such as a router: the one-block form keeps its activation sums in registers, and
// the extra passes run on CUs that would sit idle).
template <int BITS, int GS, int XDT, int SB>
int dense_t(const QmvBatch& b, int nprob, int yd, hipStream_t st) {
  using D = Dc<BITS, GS, XDT>;
  constexpr int RT = 1;
  int64_t rows16 = 0;
  for (int i = 0; i < nprob; ++i) rows16 += (b.p[i].N + 15) / 16;
  const int64_t passes1 = (b.M + D::TPB - 1) / D::TPB;
  const bool wide = b.M > D::TPB && rows16 * passes1 > jqh::cus();
  const int pass = wide ? 2 * D::TPB : D::TPB;
  DmxArgs a;
  a.b = b;
  a.nprob = nprob;
  a.mpass = pass;
  a.mtotal = b.M;
  a.K = b.K;
  a.yd = yd;
  a.nrb = 0;
  a.split = 0;
  a.part = nullptr;
  int total = 0;
  for (int i = 0; i < nprob; ++i) {
    a.rb_begin[i] = total;
    total += (int)((b.p[i].N + 16 * RT - 1) / (16 * RT));
  }
  for (int i = nprob; i <= jqk::kMaxProblems; ++i) a.rb_begin[i] = total;
  a.items = total;
  if (total == 0) return JQ_OK;
  if (pass > D::TPB) return launch_sw<D, SB, RT, 2, false, 1>(a, total, st);
  return launch_sw<D, SB, RT, 1, false, 1>(a, total, st);
}

// Dense gate|up pairs with the SiLU * up epilogue: items (gate, up) per 16-row block, passes
// as in dense_t.
template <int BITS, int GS, int XDT, int SB>
int dense_glu_t(const QmvBatch& b, float limit, int yd, hipStream_t st) {
  using D = Dc<BITS, GS, XDT>;
  const int pass = b.M > D::TPB ? 2 * D::TPB : D::TPB;
  DmxArgs a;
  a.b = b;
  a.nprob = 2;
  a.mpass = pass;
  a.mtotal = b.M;
  a.K = b.K;
  a.yd = yd;
  a.nrb = 0;
  a.split = 0;
  a.part = nullptr;
  a.g[0].glu_limit = limit;
  const int nrb = (int)((b.p[0].N + 15) / 16);
  for (int i = 0; i <= jqk::kMaxProblems; ++i) a.rb_begin[i] = i == 0 ? 0 : i == 1 ? nrb : 2 * nrb;
  a.items = 2 * nrb;
  if (nrb == 0) return JQ_OK;
  if (pass > D::TPB) return launch_sw<D, SB, 1, 2, false, 1, false, true>(a, a.items, st);
  return launch_sw<D, SB, 1, 1, false, 1, false, true>(a, a.items, st);
}

template <int XDT, int SB>
int glu_bits(int bits, int gs, const QmvBatch& b, float limit, int yd, hipStream_t st) {
#define JQ_D(B)                                                        \
  switch (gs) {                                                        \
    case 64: return dense_glu_t<B, 64, XDT, SB>(b, limit, yd, st);     \
    default: return dense_glu_t<B, 128, XDT, SB>(b, limit, yd, st);    \
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

// Chunk partials summed in chunk order and rounded: y[m0 + m, n] = sum_c part[c, m, n].
__global__ void split_sum_kernel(const float* __restrict__ part, int nchunk, int64_t mn,
                                 void* __restrict__ y, int64_t y0, int yd) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < mn;
       i += (int64_t)gridDim.x * blockDim.x) {
    float v = 0.f;
    for (int c = 0; c < nchunk; ++c) v += part[(int64_t)c * mn + i];
    store_out(y, y0 + i, v, yd);
  }
}

// K chunks for a split launch: the fewest chunks of at most 4 * kMaxKW steps, each a whole
// number of steps per wave. Returns the chunk count (0: no split fits) and its steps.
inline int split_chunks(int64_t K, int& cs) {
  const int S = (int)(K / 128);
  for (int nc = 2; nc <= 64; ++nc) {
    if (S % nc) continue;
    cs = S / nc;
    if (cs <= 4 * kMaxKW && dmx_sw(cs * 128)) return nc;
  }
  return 0;
}

template <int BITS, int GS, int XDT, int SB>
int split_t(const QmvBatch& b, int yd, float* part, int nchunk, int cs, hipStream_t st) {
  using D = Dc<BITS, GS, XDT>;
  const int pass = b.M > D::TPB ? 2 * D::TPB : D::TPB;
  const int64_t N = b.p[0].N;
  DmxArgs a;
  a.b = b;
  a.nprob = 1;
  a.mpass = pass;
  a.mtotal = b.M;
  a.K = b.K;
  a.yd = JQ_F32;
  a.split = cs;
  a.part = part;
  a.nrb = (int)((N + 15) / 16);
  a.items = nchunk * a.nrb;
  for (int i = 0; i <= jqk::kMaxProblems; ++i) a.rb_begin[i] = i == 0 ? 0 : a.nrb;
  int s;
  if (pass > D::TPB) s = launch_sw<D, SB, 1, 2, false, 1, true>(a, a.items, st);
  else s = launch_sw<D, SB, 1, 1, false, 1, true>(a, a.items, st);
  if (s) return s;
  const int64_t mn = (int64_t)b.M * N;
  const int64_t blocks = (mn + 255) / 256;
  split_sum_kernel<<<(unsigned)(blocks < 4096 ? blocks : 4096), 256, 0, st>>>(part, nchunk, mn,
                                                                              b.p[0].y, 0, yd);
  return jqh::launch_status();
}

template <int XDT, int SB>
int split_bits(int bits, int gs, const QmvBatch& b, int yd, float* part, int nchunk, int cs,
               hipStream_t st) {
#define JQ_S(B)                                                                       \
  switch (gs) {                                                                       \
    case 64: return split_t<B, 64, XDT, SB>(b, yd, part, nchunk, cs, st);             \
    default: return split_t<B, 128, XDT, SB>(b, yd, part, nchunk, cs, st);            \
  }
  switch (bits) {
    case 2: JQ_S(2)
    case 3: JQ_S(3)
    case 4: JQ_S(4)
    case 5: JQ_S(5)
    case 6: JQ_S(6)
    default: JQ_S(8)
  }
#undef JQ_S
}

template <int XDT, int SB>
int dense_bits(int bits, int gs, const QmvBatch& b, int nprob, int yd, hipStream_t st) {
#define JQ_D(B)                                                    \
  switch (gs) {                                                    \
    case 64: return dense_t<B, 64, XDT, SB>(b, nprob, yd, st);     \
    default: return dense_t<B, 128, XDT, SB>(b, nprob, yd, st);    \
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

// Gathered: tiles of up to TPB token rows (one activation block).
template <int BITS, int GS, int XDT, int SB, int NB>
int gather_t(DmxArgs& a, int64_t max_tiles, hipStream_t st) {
  using D = Dc<BITS, GS, XDT>;
  constexpr int RT = NB;
  const int64_t N = a.g[0].N;
  a.nrb = (int)((N + (NB == 2 ? 16 : 16 * RT) - 1) / (NB == 2 ? 16 : 16 * RT));
  const int64_t max_items = max_tiles * a.nrb;
  if (max_items == 0) return JQ_OK;
  if (max_items >= ((int64_t)1 << 31)) return JQ_ERR_SHAPE;
  return launch_sw<D, SB, RT, 1, true, NB>(a, max_items, st);
}

template <int XDT, int SB, int NB>
int gather_bits(int bits, int gs, DmxArgs& a, int64_t max_tiles, hipStream_t st) {
#define JQ_G(B)                                                         \
  switch (gs) {                                                         \
    case 64: return gather_t<B, 64, XDT, SB, NB>(a, max_tiles, st);     \
    default: return gather_t<B, 128, XDT, SB, NB>(a, max_tiles, st);    \
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

// LDS bytes of the smallest ring (two items) of one block, as Ring lays it out.
size_t dmx_min_lds(int bits, int gs, int K, int rt, int na) {
  const int sw = dmx_sw(K), kw = K / 128 / sw, gstep = 128 / gs;
  const int pb = sw * 16 * bits, rs = pb + 16;
  const int code = 16 * rs;
  const int sbp = sw * gstep * 2;
  const int sbarea = (16 * sbp + 255) / 256 * 256;
  const size_t wave = (size_t)2 * rt * (code + 2 * sbarea);
  return (size_t)kw * wave + (size_t)2 * kw * rt * na * (4 / gstep) * 64 * 4;
}

bool dmx_ok(int M, int64_t K, int64_t maxN, int bits, int gs, int xd, int sb, int rt) {
  if ((xd != JQ_BF16 && xd != JQ_F16) || sb != xd) return false;
  if (gs != 64 && gs != 128) return false;
  if (bits < 2 || bits > 8 || bits == 7) return false;
  if (K <= 0 || K % 128 || K > 4 * kMaxKW * 128 || dmx_sw((int)K) == 0) return false;
  const int tpb = 16 / (128 / gs);
  if (M < 1 || maxN >= ((int64_t)1 << 30)) return false;  // passes of up to 2 * tpb rows
  return dmx_min_lds(bits, gs, (int)K, rt, M > tpb ? 2 : 1) <= (size_t)kLdsMax;
}

int dmx_tokens_per_tile(int gs) { return 16 / (128 / gs); }

int dmx_launch(const QmvBatch& b, int nprob, int bits, int gs, int xd, int sb, int yd,
               hipStream_t st) {
  int64_t maxN = 0;
  for (int i = 0; i < nprob; ++i) maxN = b.p[i].N > maxN ? b.p[i].N : maxN;
  if (maxN == 0 || b.M == 0) return JQ_OK;
  if (!dmx_ok(b.M, b.K, maxN, bits, gs, xd, sb, 1)) return JQ_ERR_SHAPE;
  for (int i = 1; i < nprob; ++i) {
    if (b.p[i].x != b.p[0].x) {  // the activations are those of problem 0
      for (int j = 0; j < nprob; ++j) {
        QmvBatch one = b;
        one.p[0] = b.p[j];
        const int s = dmx_launch(one, 1, bits, gs, xd, sb, yd, st);
        if (s) return s;
      }
      return JQ_OK;
    }
  }
  if (xd == JQ_BF16) return dense_bits<JQ_BF16, JQ_BF16>(bits, gs, b, nprob, yd, st);
  return dense_bits<JQ_F16, JQ_F16>(bits, gs, b, nprob, yd, st);
}

int dmx_glu_launch(const QmvBatch& b, int bits, int gs, int xd, int sb, int yd, float limit,
                   hipStream_t st) {
  const int64_t N = b.p[0].N;
  if (N == 0 || b.M == 0) return JQ_OK;
  if (b.p[1].N != N || b.p[1].x != b.p[0].x) return JQ_ERR_SHAPE;
  if (!dmx_ok(b.M, b.K, N, bits, gs, xd, sb, 1)) return JQ_ERR_SHAPE;
  if (xd == JQ_BF16) return glu_bits<JQ_BF16, JQ_BF16>(bits, gs, b, limit, yd, st);
  return glu_bits<JQ_F16, JQ_F16>(bits, gs, b, limit, yd, st);
}

int64_t dmx_split_workspace(int M, int64_t K, int64_t N, int bits, int gs, int xd, int sb) {
  if ((xd != JQ_BF16 && xd != JQ_F16) || sb != xd || (gs != 64 && gs != 128)) return 0;
  if (bits < 2 || bits > 8 || bits == 7 || M < 1 || N < 1 || N >= ((int64_t)1 << 30)) return 0;
  if (K <= 4 * kMaxKW * 128 || K % 128 || K > ((int64_t)1 << 20)) return 0;
  int cs = 0;
  const int nc = split_chunks(K, cs);
  if (nc == 0) return 0;
  const int tpb = 16 / (128 / gs);
  if (dmx_min_lds(bits, gs, cs * 128, 1, M > tpb ? 2 : 1) > (size_t)kLdsMax) return 0;
  return (int64_t)nc * M * N * 4;  // fp32 partials of every chunk and activation row
}

int dmx_split_launch(const QmvBatch& b, int bits, int gs, int xd, int sb, int yd, void* ws,
                     int64_t ws_bytes, hipStream_t st) {
  const int64_t need = dmx_split_workspace(b.M, b.K, b.p[0].N, bits, gs, xd, sb);
  if (need == 0) return JQ_ERR_SHAPE;
  if (!ws || ws_bytes < need) return JQ_ERR_WORKSPACE;
  int cs = 0;
  const int nc = split_chunks(b.K, cs);
  float* part = (float*)ws;
  if (xd == JQ_BF16) return split_bits<JQ_BF16, JQ_BF16>(bits, gs, b, yd, part, nc, cs, st);
  return split_bits<JQ_F16, JQ_F16>(bits, gs, b, yd, part, nc, cs, st);
}

bool dmx_gather_ok(int64_t N, int64_t K, int bits, int gs, int xd, int sb, int nb) {
  return dmx_ok(1, K, N, bits, gs, xd, sb, nb);
}

int dmx_gather_launch(const QmmProblem& p, const QmmProblem* p2, const GatherPlan& plan,
                      int64_t max_tiles, int bits, int gs, int xd, int sb, int yd,
                      hipStream_t st) {
  if (max_tiles == 0 || p.N == 0) return JQ_OK;
  if (!dmx_gather_ok(p.N, p.K, bits, gs, xd, sb, p2 ? 2 : 1) || plan.tiles == nullptr)
    return JQ_ERR_SHAPE;
  DmxArgs a;
  a.g[0] = p;
  a.g[1] = p2 ? *p2 : p;
  a.plan = plan;
  a.K = (int)p.K;
  a.yd = yd;
  a.nprob = 0;
  a.items = 0;
  a.split = 0;
  a.part = nullptr;
  if (xd == JQ_BF16)
    return p2 ? gather_bits<JQ_BF16, JQ_BF16, 2>(bits, gs, a, max_tiles, st)
              : gather_bits<JQ_BF16, JQ_BF16, 1>(bits, gs, a, max_tiles, st);
  return p2 ? gather_bits<JQ_F16, JQ_F16, 2>(bits, gs, a, max_tiles, st)
            : gather_bits<JQ_F16, JQ_F16, 1>(bits, gs, a, max_tiles, st);
}

}  // namespace jqk

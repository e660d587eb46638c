// Router top-k of one token in one wave, shared by the route kernel and the expert launch
// that routes for itself (jq_moe.hip, jq_gemv_gather.hip).
//
// softmax(logits) in fp32 (max-subtracted) and the top k by probability, ties to the lower
// expert id, optionally renormalised to sum 1: the caller-side routing of
// jang-tools/jang_tools/qwen4_exp/modeling.py:587-593.
#pragma once
#include <math.h>

#include "jq_common.h"
#include "jq_gemv.h"

namespace jqr {

// Order-preserving u32 key of a float (a larger float has a larger key; -0 is taken as +0
// by the caller); 0 lies below every float's key and marks chosen or padding slots.
JQ_DEV uint32_t ord_key(float v) {
  const uint32_t b = __float_as_uint(v);
  return b ^ ((uint32_t)((int32_t)b >> 31) | 0x80000000u);
}
JQ_DEV float ord_val(uint32_t k) {
  return __uint_as_float(k & 0x80000000u ? k ^ 0x80000000u : ~k);
}

// One DPP step of a wave maximum (lanes outside row_mask, and lanes whose source is out of
// range, see the neutral value and keep theirs).
template <int CTRL, int ROWS>
JQ_DEV uint64_t max_step(uint64_t k) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)k, CTRL, ROWS, 0xF, false);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(k >> 32), CTRL, ROWS, 0xF, false);
  const uint64_t o = ((uint64_t)hi << 32) | lo;
  return o > k ? o : k;
}
template <int CTRL, int ROWS>
JQ_DEV float fmax_step(float v) {
  return fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
                      __builtin_bit_cast(int, -INFINITY), __builtin_bit_cast(int, v), CTRL, ROWS, 0xF, false)));
}

// Wave maxima, broadcast to every lane: DPP row operations carry the maximum into lane 63
// (as a wave sum would), a scalar read hands it to all lanes.
JQ_DEV uint64_t wave_max_u64(uint64_t k) {
  k = max_step<0xB1, 0xF>(k);   // quad_perm 1,0,3,2
  k = max_step<0x4E, 0xF>(k);   // quad_perm 2,3,0,1
  k = max_step<0x124, 0xF>(k);  // row_ror 4
  k = max_step<0x128, 0xF>(k);  // row_ror 8
  k = max_step<0x142, 0xA>(k);  // row_bcast 15
  k = max_step<0x143, 0xC>(k);  // row_bcast 31
  const uint32_t lo = __builtin_amdgcn_readlane((int)(uint32_t)k, 63);
  const uint32_t hi = __builtin_amdgcn_readlane((int)(uint32_t)(k >> 32), 63);
  return ((uint64_t)hi << 32) | lo;
}
JQ_DEV float wave_max_f32(float v) {
  v = fmax_step<0xB1, 0xF>(v);
  v = fmax_step<0x4E, 0xF>(v);
  v = fmax_step<0x124, 0xF>(v);
  v = fmax_step<0x128, 0xF>(v);
  v = fmax_step<0x142, 0xA>(v);
  v = fmax_step<0x143, 0xC>(v);
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

// Lane l holds the order keys of logits l, l + 64, ... (SL = ceil(E/64) of them). Top-k in
// k rounds on the logits (softmax is monotone): each lane offers its largest remaining key
// and the wave maximum of (key, ~id) picks the round's expert (ties -> lowest id), whose key
// is then cleared. Lane j < k returns round j's expert and its probability (renormalised over
// the k when renorm). Every lane of the wave must take part.
template <int SL>
JQ_DEV void route_wave(const float* __restrict__ row, int E, int k, int renorm, int lane,
                       uint32_t& id, float& w) {
  uint32_t key[SL];
  float mx = -INFINITY;
#pragma unroll
  for (int i = 0; i < SL; ++i) {
    const int e = lane + 64 * i;
    const float v = e < E ? row[e] + 0.0f : -INFINITY;  // + 0: -0 becomes +0
    key[i] = e < E ? ord_key(v) : 0u;
    mx = fmaxf(mx, v);
  }
  mx = wave_max_f32(mx);
  float sum = 0.f;
#pragma unroll
  for (int i = 0; i < SL; ++i) sum += key[i] ? expf(ord_val(key[i]) - mx) : 0.f;
  sum = __builtin_bit_cast(float, __builtin_amdgcn_readlane(
                                      __builtin_bit_cast(int, jqg::wave_total_lane63(sum)), 63));
  const float inv = 1.0f / sum;

  uint64_t mine = 0;  // lane j: round j's (key, ~id)
  for (int j = 0; j < k; ++j) {
    // The lane's largest remaining key; a strict > in slot order keeps the lowest id.
    uint32_t bk = 0;
    int bi = 0;
#pragma unroll
    for (int i = 0; i < SL; ++i) {
      const bool better = key[i] > bk;
      bk = better ? key[i] : bk;
      bi = better ? i : bi;
    }
    const uint64_t offer = bk ? ((uint64_t)bk << 32) | (uint32_t)~(uint32_t)(lane + 64 * bi) : 0ull;
    const uint64_t best = wave_max_u64(offer);
    const uint32_t bid = ~(uint32_t)best;
#pragma unroll
    for (int i = 0; i < SL; ++i) key[i] = (uint32_t)(lane + 64 * i) == bid ? 0u : key[i];
    mine = lane == j ? best : mine;
  }
  const float p = expf(ord_val((uint32_t)(mine >> 32)) - mx) * inv;
  float wsum = 0.f;  // the k probabilities in round order
  for (int j = 0; j < k; ++j)
    wsum += __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, p), j));
  id = ~(uint32_t)mine;
  w = renorm ? p / wsum : p;
}

}  // namespace jqr

// Router top-k of one token in one wave, shared by the route kernel and the expert launch
// that routes for itself (jq_moe.hip, jq_gemv_gather.hip).
//
// Scores from the router logits, then the k experts of largest selection value (ties to the
// lower expert id), in descending order, with their weights:
//   softmax       p = softmax(logits) in fp32, max-subtracted ("precise")
//                   jang-tools/jang_tools/qwen4_exp/modeling.py:587-593,
//                   jang-tools/jang_tools/mistral4_mlx.py:359-387
//   sigmoid       s = sigmoid(logits)
//                   jang-tools/jang_tools/dots3/ops.py:149-162, laguna/model.py:50-62
//   sqrt-softplus s = sqrt(softplus(logits))
//                   jang-tools/jang_tools/dsv41/model.py:1184-1190
// The selection value is the score plus an optional per-expert bias (e_score_correction_bias;
// the weights keep the unbiased score). Group-limited selection (n_group > 1) keeps the
// topk_group groups of E / n_group consecutive experts with the largest maximum selection
// value and gives every other expert the selection value 0 and the score 0
// (mistral4_mlx.py:363-375). The weights are the scores of the chosen experts, optionally
// divided by (their sum + eps), then multiplied by the routed scaling factor.
#pragma once
#include <math.h>

#include "jq_common.h"
#include "jq_gemv.h"
#include "jq_qmv.h"

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

// A pointer that every lane holds, moved to scalar registers so that buffer descriptors built
// from it are wave-uniform.
template <class T>
JQ_DEV const T* uniform_ptr(const T* p) {
  const uint64_t v = (uint64_t)p;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return (const T*)(((uint64_t)hi << 32) | lo);
}

JQ_DEV float lane_read(float v, int l) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}

// Score of a logit for the sigmoid-type routers (softmax scores need the row's max and sum).
JQ_DEV float gate_score(int score, float v) {
  if (score == kSigmoid) return 1.0f / (1.0f + expf(-v));
  // softplus(v) = max(v, 0) + log1p(exp(-|v|)), then its square root
  return sqrtf(fmaxf(v, 0.f) + log1pf(expf(-fabsf(v))));
}

// Lane l holds logits l, l + 64, ... (SL = ceil(E/64) of them). Top-k in k rounds: each lane
// offers its largest remaining selection key and the wave maximum of (key, ~id) picks the
// round's expert (ties -> lowest id), whose key is then cleared. Lane j < k returns round j's
// expert and its weight. Every lane of the wave must take part.
// row: the token's E logits of o.logit_dtype (converted exactly to fp32).
template <int SL>
JQ_DEV void route_wave(const void* __restrict__ row, int E, int k, const RouteOpts& o, int lane,
                       uint32_t& id, float& w, int rounds = 64) {
  // All SL logits (and biases) of a lane are requested before any is used: range-checked
  // buffer loads (slots past E read 0 and touch no memory) under a wave-uniform dtype branch,
  // so the loads stay in flight together instead of one round trip each.
  float v[SL];
  float bias[SL];
  {
    const bool f32 = o.logit_dtype == JQ_F32;
    const jqg::Rsrc rl = jqg::make_rsrc(uniform_ptr(row), (uint32_t)E * (f32 ? 4u : 2u));
    uint32_t raw[SL];
    if (f32) {
#pragma unroll
      for (int i = 0; i < SL; ++i)
        raw[i] = __builtin_amdgcn_raw_buffer_load_b32(rl, (uint32_t)(lane + 64 * i) * 4u, 0, 0);
    } else {
#pragma unroll
      for (int i = 0; i < SL; ++i)
        raw[i] = __builtin_amdgcn_raw_buffer_load_b16(rl, (uint32_t)(lane + 64 * i) * 2u, 0, 0);
    }
    const jqg::Rsrc rbias = jqg::make_rsrc(uniform_ptr(o.bias), o.bias ? (uint32_t)E * 4u : 0u);
#pragma unroll
    for (int i = 0; i < SL; ++i)
      bias[i] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rbias, (uint32_t)(lane + 64 * i) * 4u, 0, 0));
#pragma unroll
    for (int i = 0; i < SL; ++i) {
      const float x = f32 ? __uint_as_float(raw[i])
                      : o.logit_dtype == JQ_BF16 ? __uint_as_float(raw[i] << 16)
                                                 : jq::f16_bits_to_f32((uint16_t)raw[i]);
      v[i] = lane + 64 * i < E ? x + 0.0f : -INFINITY;  // -0 becomes +0
    }
  }
  float mx = -INFINITY;
#pragma unroll
  for (int i = 0; i < SL; ++i) mx = fmaxf(mx, v[i]);
  const bool soft = o.score == kSoftmax;
  float inv = 1.f;
  if (soft) {
    mx = wave_max_f32(mx);
    float sum = 0.f;
#pragma unroll
    for (int i = 0; i < SL; ++i) sum += lane + 64 * i < E ? expf(v[i] - mx) : 0.f;
    sum = lane_read(jqg::wave_total_lane63(sum), 63);
    inv = 1.0f / sum;
  }
  auto score_of = [&](float x) { return soft ? expf(x - mx) * inv : gate_score(o.score, x); };
  const bool grouped = o.n_group > 1 && o.topk_group < o.n_group;
  // Selection on the logits themselves when they order the experts as the scores do
  // (softmax is monotone); otherwise on score + bias.
  const bool by_logit = soft && !o.bias && !grouped;
  uint32_t key[SL];
#pragma unroll
  for (int i = 0; i < SL; ++i) {
    const int e = lane + 64 * i;
    float sel = v[i];
    if (!by_logit) sel = score_of(v[i]) + bias[i] + 0.0f;  // (0 without a bias or past E)
    key[i] = e < E ? ord_key(sel) : 0u;
  }
  if (grouped) {
    // Group maxima (lane g holds group g's), the topk_group largest groups kept (ties -> the
    // lower group), every expert of another group set to selection value 0 and score 0.
    const int gsz = E / o.n_group;
    uint32_t gkey = 0;
    for (int g = 0; g < o.n_group; ++g) {
      uint32_t m = 0;
#pragma unroll
      for (int i = 0; i < SL; ++i) {
        const int e = lane + 64 * i;
        m = (e < E && e / gsz == g && key[i] > m) ? key[i] : m;
      }
      const uint64_t best = wave_max_u64((uint64_t)m << 32);
      gkey = lane == g ? (uint32_t)(best >> 32) : gkey;
    }
    bool kept = false;
    for (int r = 0; r < o.topk_group; ++r) {
      const uint64_t offer = lane < o.n_group && !kept
                                 ? ((uint64_t)gkey << 32) | (uint32_t)~(uint32_t)lane : 0ull;
      const uint32_t gid = ~(uint32_t)wave_max_u64(offer);
      kept = kept || (uint32_t)lane == gid;
    }
    const int kept_i = kept ? 1 : 0;
#pragma unroll
    for (int i = 0; i < SL; ++i) {
      const int e = lane + 64 * i;
      const int g = e < E ? e / gsz : 0;
      const int kg = __shfl(kept_i, g, 64);
      if (e < E && !kg) {
        key[i] = ord_key(0.0f);
        v[i] = -INFINITY;  // score 0
      }
    }
  }

  uint64_t mine = 0;  // lane j: round j's (key, ~id)
  float sc = 0.f;     // lane j: round j's score
  // Only the first `rounds` experts when the caller needs no more (their ids and unrenormalised
  // weights are final after their own rounds; renormalised weights need all k).
  const int nr = rounds < k ? rounds : k;
  for (int j = 0; j < nr; ++j) {
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
    float vb = -INFINITY;  // the chosen expert's logit, from its lane
#pragma unroll
    for (int i = 0; i < SL; ++i) {
      const bool hit = (uint32_t)(lane + 64 * i) == bid;
      vb = hit ? v[i] : vb;
      key[i] = hit ? 0u : key[i];
    }
    vb = lane_read(vb, (int)(bid & 63u));
    mine = lane == j ? best : mine;
    sc = lane == j ? vb : sc;
  }
  const float p = lane < k ? score_of(sc) : 0.f;
  float wsum = 0.f;  // the k scores in round order
  for (int j = 0; j < k; ++j) wsum += lane_read(p, j);
  id = ~(uint32_t)mine;
  float r = o.renorm ? p / (wsum + o.eps) : p;
  w = o.scale == 1.f ? r : r * o.scale;
}

}  // namespace jqr

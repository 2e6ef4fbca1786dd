// Router top-k of one token's fp32 logits by one wave (gfx950), shared by the
// router (router.hip) and the decode kernels that select their own experts
// (qmv.hip).
//
// Semantics: the reference's fused router
// (engine/patches/decode-fusion/fused_kernels.py:288-330 kernel source,
// :363-371 router_topk): the k largest logits in descending order, ties to
// the lower expert index, and the scores
//   norm:  exp(l_j - l_0) / sum_{j<k} exp(l_j - l_0)   -- softmax renormalised
//          over the chosen experts (qwen3_5_moe/language.py:65-71);
//   else:  exp(l_j - max) / sum_e exp(l_e - max)        -- the full softmax.
// Softmax is monotonic, so selecting on logits selects the same experts as
// selecting on softmax probabilities, without rounding them to bf16 first
// (the stock path's bf16 gates can tie where the logits do not).  Logits are
// expected finite; a NaN, outside that contract, ranks below every number.
//
// Lane l holds experts l, l + 64, ... (PER per lane, coalesced loads).  Each
// round takes the wave maximum of the lanes' best untaken values, then the
// lowest expert index holding it (one ballot per column of 64 experts), and
// retires that expert in its owner lane.
#pragma once

#include <math.h>
#include <stdint.h>

namespace qmoe_topk {

constexpr int kMaxK = 64;
constexpr int kMaxPer = 16;  // E <= 1024

// Whole-wave reductions that leave the result in every lane, without the
// LDS crossbar (__shfl_xor lowers to ds_bpermute, whose latency dominated a
// k-round top-k): two quad_perm steps, row_half_mirror and row_ror:8 cover a
// 16-lane row with DPP, then v_permlane16_swap and v_permlane32_swap combine
// the rows.
template <class Op>
__device__ __forceinline__ float wave_all(float v, Op op) {
  auto dpp = [](float x, int ctrl) {
    switch (ctrl) {  // the control word must be a constant
      case 0xB1: return __uint_as_float(__builtin_amdgcn_update_dpp(0u, __float_as_uint(x), 0xB1, 0xf, 0xf, false));
      case 0x4E: return __uint_as_float(__builtin_amdgcn_update_dpp(0u, __float_as_uint(x), 0x4E, 0xf, 0xf, false));
      case 0x141: return __uint_as_float(__builtin_amdgcn_update_dpp(0u, __float_as_uint(x), 0x141, 0xf, 0xf, false));
      default: return __uint_as_float(__builtin_amdgcn_update_dpp(0u, __float_as_uint(x), 0x128, 0xf, 0xf, false));
    }
  };
  v = op(v, dpp(v, 0xB1));   // quad_perm 1,0,3,2
  v = op(v, dpp(v, 0x4E));   // quad_perm 2,3,0,1
  v = op(v, dpp(v, 0x141));  // row_half_mirror
  v = op(v, dpp(v, 0x128));  // row_ror:8
  auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = op(__uint_as_float(r16[0]), __uint_as_float(r16[1]));
  auto r32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return op(__uint_as_float(r32[0]), __uint_as_float(r32[1]));
}
__device__ __forceinline__ float wave_max(float v) {
  return wave_all(v, [](float a, float b) { return fmaxf(a, b); });
}
__device__ __forceinline__ float wave_sum(float v) {
  return wave_all(v, [](float a, float b) { return a + b; });
}

// Unsigned maximum over the wave, left in every lane.  The DPP moves start
// from 0, the identity of the maximum, so the compiler folds each into its
// v_max_u32 (one instruction per step).
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xf, 0xf, false));   // quad_perm 1,0,3,2
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xf, 0xf, false));   // quad_perm 2,3,0,1
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x141, 0xf, 0xf, false));  // row_half_mirror
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x128, 0xf, 0xf, false));  // row_ror:8
  auto r16 = __builtin_amdgcn_permlane16_swap(v, v, false, false);
  v = max(r16[0], r16[1]);
  auto r32 = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return max(r32[0], r32[1]);
}

// Order-preserving unsigned key of a logit: equal keys for equal values (-0
// folded into +0), a larger key for a larger value, and 1, below every
// number, for NaN.  Key 0 marks an expert already chosen (or absent).
__device__ __forceinline__ uint32_t logit_key(float x) {
  const uint32_t b = __float_as_uint(x + 0.0f);
  const uint32_t k = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  return x != x ? 1u : k;
}
__device__ __forceinline__ float key_logit(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}

// The top-k of the E logits at lp (E <= 64 * PER, k <= min(E, 64)), called by
// every lane of one wave (want_scores wave-uniform).  Lane j < k returns choice
// j in idx and its score in score (0 unless want_scores); lanes j >= k return
// idx 0 and score 0.  The rounds select on
// logit_key, which orders the logits as their values do (NaN last), so a
// round is integer work without branches: the wave maximum of the keys, one
// ballot per column of 64 experts for that maximum, and scalar selects for
// the first non-empty column.  A chosen expert's key becomes 0; while an
// expert is left the maximum is at least 1, so no other bookkeeping is needed.
template <int PER>
__device__ __forceinline__ void wave_topk(const float* __restrict__ lp, int E, int k, int norm, int& idx,
                                          float& score, bool want_scores = true) {
  const int lane = threadIdx.x & 63;
  float v[PER];
  uint32_t key[PER];
#pragma unroll
  for (int c = 0; c < PER; ++c) {
    const int e = c * 64 + lane;
    v[c] = e < E ? lp[e] : -INFINITY;
    key[c] = e < E ? logit_key(v[c]) : 0u;
  }
  float lmax = v[0];
#pragma unroll
  for (int c = 1; c < PER; ++c) lmax = fmaxf(lmax, v[c]);
  const float gmax = wave_max(lmax);
  float all = 0.f;  // sum over every expert of exp(l - max), for the full softmax (absent: exp(-inf) = 0)
  if (want_scores && !norm) {
#pragma unroll
    for (int c = 0; c < PER; ++c) all += expf(v[c] - gmax);
    all = wave_sum(all);
  }

  float mine = -INFINITY;  // lane j keeps the j-th chosen logit
  idx = 0;
  for (int j = 0; j < k; ++j) {
    uint32_t bv = key[0];
#pragma unroll
    for (int c = 1; c < PER; ++c) bv = max(bv, key[c]);
    const uint32_t wm = wave_max_u32(bv);
    // the lowest expert index holding the maximum: column c = e / 64 first,
    // then the lowest lane of that column
    uint64_t m[PER];
#pragma unroll
    for (int c = 0; c < PER; ++c) m[c] = __ballot(key[c] == wm);
    int col = PER - 1;
    uint64_t mc = m[PER - 1];
#pragma unroll
    for (int c = PER - 2; c >= 0; --c) {
      col = m[c] ? c : col;
      mc = m[c] ? m[c] : mc;
    }
    const int sel = 64 * col + (int)__builtin_ctzll(mc);
    const bool owner = lane == (sel & 63);
#pragma unroll
    for (int c = 0; c < PER; ++c) key[c] = owner && c == col ? 0u : key[c];
    mine = lane == j ? key_logit(wm) : mine;
    idx = lane == j ? sel : idx;
  }
  score = 0.f;
  if (!want_scores) return;
  if (norm) {
    const float top0 = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(mine), 0));
    const float p = lane < k ? expf(mine - top0) : 0.f;
    const float denom = wave_sum(p);
    if (lane < k) score = p / denom;
  } else {
    if (lane < k) score = expf(mine - gmax) / all;
  }
}

}  // namespace qmoe_topk

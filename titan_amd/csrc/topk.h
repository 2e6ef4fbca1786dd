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
// Lane l holds experts l, l + 64, ... (PER per lane, coalesced loads).
#pragma once

#include <math.h>
#include <stdint.h>

namespace qmoe_topk {

constexpr int kMaxK = 64;
constexpr int kMaxPer = 16;  // E <= 1024

// Whole-wave reductions that leave the result in every lane, without the
// LDS crossbar (__shfl_xor lowers to ds_bpermute): two quad_perm steps,
// row_half_mirror and row_ror:8 cover a 16-lane row with DPP, then
// v_permlane16_swap and v_permlane32_swap combine the rows.
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

// Lane l's keys of experts l, l + 64, ... (absent experts: key 0) and logits.
template <int PER>
__device__ __forceinline__ void load_keys(const float* __restrict__ lp, int E, float (&v)[PER],
                                          uint32_t (&key)[PER]) {
  const int lane = threadIdx.x & 63;
  // every load issued before any is used (a guarded load would wait alone)
#pragma unroll
  for (int c = 0; c < PER; ++c) v[c] = lp[min(c * 64 + lane, E - 1)];
#pragma unroll
  for (int c = 0; c < PER; ++c) {
    const bool live = c * 64 + lane < E;
    key[c] = live ? logit_key(v[c]) : 0u;
    v[c] = live ? v[c] : -INFINITY;
  }
}

// Wave maximum of v, wave-uniform: DPP steps leave each 16-lane row's maximum
// in its lanes, and the four rows meet in scalar registers.
__device__ __forceinline__ uint32_t wave_max_key(uint32_t v) {
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xf, 0xf, false));   // quad_perm 1,0,3,2
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xf, 0xf, false));   // quad_perm 2,3,0,1
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x141, 0xf, 0xf, false));  // row_half_mirror
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x128, 0xf, 0xf, false));  // row_ror:8
  const uint32_t r0 = __builtin_amdgcn_readlane(v, 0), r1 = __builtin_amdgcn_readlane(v, 16);
  const uint32_t r2 = __builtin_amdgcn_readlane(v, 32), r3 = __builtin_amdgcn_readlane(v, 48);
  return max(max(r0, r1), max(r2, r3));
}

// A lane's remaining experts as a list, best first.  For PER <= 8 the lane's
// keys are sorted once (descending, equal keys in column order: odd-even
// transposition swapping on strict order only) with their columns packed one
// per byte, and taking the head shifts the list.  For PER = 16 the keys stay
// in place and the head (largest key, lowest column among equals) is found
// again after each take.
template <int PER>
struct LaneList {
  static constexpr bool kSorted = PER <= 8;
  uint32_t key[PER];
  uint64_t cols;  // sorted: column of key[i] in byte i
  uint32_t hk;    // head key
  int hc;         // head column

  __device__ __forceinline__ void init() {
    if constexpr (kSorted) {
      int col[PER];
#pragma unroll
      for (int c = 0; c < PER; ++c) col[c] = c;
#pragma unroll
      for (int r = 0; r < PER; ++r)
#pragma unroll
        for (int a = r & 1; a + 1 < PER; a += 2) {
          const bool sw = key[a + 1] > key[a];
          const uint32_t ka = key[a], kb = key[a + 1];
          const int ca = col[a], cb = col[a + 1];
          key[a] = sw ? kb : ka;
          key[a + 1] = sw ? ka : kb;
          col[a] = sw ? cb : ca;
          col[a + 1] = sw ? ca : cb;
        }
      cols = 0;
#pragma unroll
      for (int c = 0; c < PER; ++c) cols |= (uint64_t)col[c] << (8 * c);
    }
    head();
  }
  __device__ __forceinline__ void head() {
    if constexpr (kSorted) {
      hk = key[0];
      hc = (int)(cols & 0xFF);
    } else {
      hk = key[0];
#pragma unroll
      for (int c = 1; c < PER; ++c) hk = max(hk, key[c]);
      hc = PER - 1;
#pragma unroll
      for (int c = PER - 2; c >= 0; --c) hc = key[c] == hk ? c : hc;
    }
  }
  // the owner lane gives up its head
  __device__ __forceinline__ void take(bool owner) {
    if constexpr (kSorted) {
#pragma unroll
      for (int c = 0; c + 1 < PER; ++c) key[c] = owner ? key[c + 1] : key[c];
      key[PER - 1] = owner ? 0u : key[PER - 1];
      cols = owner ? cols >> 8 : cols;
    } else {
#pragma unroll
      for (int c = 0; c < PER; ++c) key[c] = owner && c == hc ? 0u : key[c];
    }
    head();
  }
};

// One round: the lane holding the wave's best head, ties to the lowest expert
// index 64 * hc + lane.  Wave-uniform.
template <int PER>
__device__ __forceinline__ int round_owner(const LaneList<PER>& L) {
  const uint32_t wm = wave_max_key(L.hk);
  const uint64_t m = __ballot(L.hk == wm);
  if (__builtin_expect(__popcll(m) == 1, 1)) return (int)__builtin_ctzll(m);
  int ol = 0;
  bool found = false;
#pragma unroll
  for (int c = 0; c < PER; ++c) {
    const uint64_t mc = __ballot(L.hk == wm && L.hc == c);
    ol = (!found && mc) ? (int)__builtin_ctzll(mc) : ol;
    found = found || mc != 0;
  }
  return ol;
}

// Choice k - 1 alone (1 <= k <= min(E, 64)), wave-uniform: k - 1 rounds taken,
// then the k-th round's winner.
template <int PER>
__device__ __forceinline__ int wave_topk_last(const float* __restrict__ lp, int E, int k) {
  const int lane = threadIdx.x & 63;
  float v[PER];
  LaneList<PER> L;
  load_keys<PER>(lp, E, v, L.key);
  L.init();
  for (int j = 0; j + 1 < k; ++j) L.take(lane == round_owner<PER>(L));
  const int ol = round_owner<PER>(L);
  return 64 * __builtin_amdgcn_readlane(L.hc, ol) + ol;
}

// The top-k of the E logits at lp (E <= 64 * PER, k <= min(E, 64)), called by
// every lane of one wave, in two parts.  wave_topk_select leaves choice j in
// lane j's idx and its key in key_j (lanes j >= k: 0 and 0), and the lane's
// logits in v (absent experts -inf); wave_topk_scores then gives lane j < k
// its score (0 in lanes j >= k).  The rounds select on logit_key, which orders
// the logits as their values do (NaN last), so a round is integer work: the
// wave maximum of the lanes' heads, one ballot for the lane holding it, and
// that lane's take.  A taken or absent expert has key 0; while an expert is
// left the maximum is at least 1.
template <int PER>
__device__ __forceinline__ void wave_topk_select(const float* __restrict__ lp, int E, int k, float (&v)[PER],
                                                 int& idx, uint32_t& key_j) {
  const int lane = threadIdx.x & 63;
  LaneList<PER> L;
  load_keys<PER>(lp, E, v, L.key);
  L.init();
  key_j = 0;
  idx = 0;
  for (int j = 0; j < k; ++j) {
    const int ol = round_owner<PER>(L);
    const int e = 64 * __builtin_amdgcn_readlane(L.hc, ol) + ol;
    const uint32_t kk = __builtin_amdgcn_readlane(L.hk, ol);
    idx = lane == j ? e : idx;
    key_j = lane == j ? kk : key_j;
    L.take(lane == ol);
  }
}

template <int PER>
__device__ __forceinline__ float wave_topk_scores(const float (&v)[PER], int k, int norm, uint32_t key_j) {
  const int lane = threadIdx.x & 63;
  const float mine = lane < k ? key_logit(key_j) : -INFINITY;  // lane j's chosen logit
  if (norm) {
    const float top0 = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(mine), 0));
    const float p = lane < k ? expf(mine - top0) : 0.f;
    const float denom = wave_sum(p);
    return lane < k ? p / denom : 0.f;
  }
  float lmax = v[0];
#pragma unroll
  for (int c = 1; c < PER; ++c) lmax = fmaxf(lmax, v[c]);
  const float gmax = wave_max(lmax);
  float all = 0.f;  // sum over every expert of exp(l - max), for the full softmax (absent: exp(-inf) = 0)
#pragma unroll
  for (int c = 0; c < PER; ++c) all += expf(v[c] - gmax);
  all = wave_sum(all);
  return lane < k ? expf(mine - gmax) / all : 0.f;
}

template <int PER>
__device__ __forceinline__ void wave_topk(const float* __restrict__ lp, int E, int k, int norm, int& idx,
                                          float& score) {
  float v[PER];
  uint32_t key_j;
  wave_topk_select<PER>(lp, E, k, v, idx, key_j);
  score = wave_topk_scores<PER>(v, k, norm, key_j);
}

}  // namespace qmoe_topk

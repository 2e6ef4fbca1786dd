// Router top-k over fp32 logits, one wave per token (gfx950).
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
// (the stock path's bf16 gates can tie where the logits do not).
//
// Lane l holds experts l, l + 64, ... (PER per lane, coalesced loads).  Each
// round takes the wave maximum of the lanes' best untaken values, then the
// lowest expert index holding it (one ballot per column of 64 experts), and
// retires that expert in its owner lane.
#include <limits.h>

#include "common.h"

namespace {

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

template <int PER>
__global__ __launch_bounds__(256) void router_topk_kernel(const float* __restrict__ logits, int64_t T, int E, int k,
                                                         int norm, int32_t* __restrict__ idx,
                                                         float* __restrict__ scores) {
  const int64_t t = (int64_t)blockIdx.x * 4 + threadIdx.x / 64;
  const int lane = threadIdx.x % 64;
  if (t >= T) return;
  const float* lp = logits + t * E;
  float v[PER];
  uint32_t taken = 0;  // bit c: expert c * 64 + lane already chosen (or absent)
#pragma unroll
  for (int c = 0; c < PER; ++c) {
    const int e = c * 64 + lane;
    v[c] = e < E ? lp[e] : -INFINITY;
    if (e >= E) taken |= 1u << c;
  }
  float lmax = -INFINITY;
#pragma unroll
  for (int c = 0; c < PER; ++c)
    if (!(taken >> c & 1)) lmax = fmaxf(lmax, v[c]);
  const float gmax = wave_max(lmax);
  float all = 0.f;  // sum over every expert of exp(l - max), for the full softmax
  if (!norm) {
#pragma unroll
    for (int c = 0; c < PER; ++c)
      if (!(taken >> c & 1)) all += expf(v[c] - gmax);
    all = wave_sum(all);
  }

  float mine = -INFINITY;  // lane j keeps the j-th chosen logit
  for (int j = 0; j < k; ++j) {
    float bv = -INFINITY;
#pragma unroll
    for (int c = 0; c < PER; ++c)
      if (!(taken >> c & 1)) bv = fmaxf(bv, v[c]);
    const float wm = wave_max(bv);
    // the lowest expert index holding the maximum: column c = e / 64 first,
    // then the lowest lane of that column (one ballot per column)
    int sel = 0;  // no comparable candidate (NaN logits): stay in range
#pragma unroll
    for (int c = 0; c < PER; ++c) {
      const uint64_t m = __ballot(!(taken >> c & 1) && v[c] == wm);
      if (m) {
        sel = 64 * c + __builtin_ctzll(m);
        break;
      }
    }
    if (lane == (sel & 63)) taken |= 1u << (sel >> 6);
    if (lane == 0) idx[t * k + j] = sel;
    if (lane == j) mine = wm;
  }
  if (norm) {
    const float top0 = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(mine), 0));
    const float p = lane < k ? expf(mine - top0) : 0.f;
    const float denom = wave_sum(p);
    if (lane < k) scores[t * k + lane] = p / denom;
  } else {
    if (lane < k) scores[t * k + lane] = expf(mine - gmax) / all;
  }
}

// Router logits over a dense bf16 router weight: logits[t, e] = x[t] . W[e]
// in fp32 (v_dot2_f32_bf16), one wave per (token, expert) row, each lane
// taking 16-byte units u = lane, lane + 64, ... of both rows.
__global__ __launch_bounds__(256) void router_logits_dense_kernel(const uint16_t* __restrict__ x, int64_t T,
                                                                 int K, const uint16_t* __restrict__ w, int E,
                                                                 float* __restrict__ logits) {
  const int64_t row = (int64_t)blockIdx.x * 4 + threadIdx.x / 64;
  const int lane = threadIdx.x % 64;
  if (row >= T * E) return;
  const int64_t t = row / E;
  const int64_t e = row - t * E;
  const uint4* xp = reinterpret_cast<const uint4*>(x + t * K);
  const uint4* wp = reinterpret_cast<const uint4*>(w + e * K);
  const int units = K / 8;
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  int u = lane;
  for (; u + 192 < units; u += 256) {  // four units in flight per lane
    uint4 xv[4], wv[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      xv[j] = xp[u + 64 * j];
      wv[j] = wp[u + 64 * j];
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      acc[j] = dot2_bf16(xv[j].x, wv[j].x, acc[j]);
      acc[j] = dot2_bf16(xv[j].y, wv[j].y, acc[j]);
      acc[j] = dot2_bf16(xv[j].z, wv[j].z, acc[j]);
      acc[j] = dot2_bf16(xv[j].w, wv[j].w, acc[j]);
    }
  }
  for (; u < units; u += 64) {
    const uint4 xv = xp[u], wv = wp[u];
    acc[0] = dot2_bf16(xv.x, wv.x, acc[0]);
    acc[0] = dot2_bf16(xv.y, wv.y, acc[0]);
    acc[0] = dot2_bf16(xv.z, wv.z, acc[0]);
    acc[0] = dot2_bf16(xv.w, wv.w, acc[0]);
  }
  const float v = wave_sum((acc[0] + acc[1]) + (acc[2] + acc[3]));
  if (lane == 0) logits[row] = v;
}

}  // namespace

extern "C" int qmoe_router_logits_dense(const uint16_t* x, int64_t T, int64_t K, const uint16_t* w, int64_t E,
                                        float* logits, void* stream) {
  if (T < 0 || K <= 0 || E <= 0) return qmoe::fail(QMOE_ERR_INVALID, "bad sizes");
  if (T == 0) return QMOE_OK;
  if (!x || !w || !logits) return qmoe::fail(QMOE_ERR_INVALID, "null pointer");
  if (K % 8) return qmoe::fail(QMOE_ERR_UNSUPPORTED, "K=%lld: must be a multiple of 8", (long long)K);
  if (K > 0x7FFFFFFF || E > 0x7FFFFFFF) return qmoe::fail(QMOE_ERR_UNSUPPORTED, "sizes too large");
  if (!qmoe::aligned16(x) || !qmoe::aligned16(w)) return qmoe::fail(QMOE_ERR_UNSUPPORTED, "x and w must be 16-byte aligned");
  const int64_t blocks = (T * E + 3) / 4;
  if (blocks > 0x7FFFFFFF) return qmoe::fail(QMOE_ERR_UNSUPPORTED, "too many rows");
  router_logits_dense_kernel<<<dim3((unsigned)blocks), dim3(256), 0, qmoe::as_stream(stream)>>>(x, T, (int)K, w,
                                                                                               (int)E, logits);
  return qmoe::launch_status("router_logits_dense_kernel");
}

extern "C" int qmoe_router_topk(const float* logits, int64_t T, int64_t E, int64_t k, int norm, int32_t* idx,
                                float* scores, void* stream) {
  if (T < 0 || E <= 0 || k <= 0) return qmoe::fail(QMOE_ERR_INVALID, "bad sizes");
  if (k > E) return qmoe::fail(QMOE_ERR_INVALID, "k=%lld > E=%lld", (long long)k, (long long)E);
  if (T == 0) return QMOE_OK;
  if (!logits || !idx || !scores) return qmoe::fail(QMOE_ERR_INVALID, "null pointer");
  if (k > kMaxK || E > 64 * kMaxPer)
    return qmoe::fail(QMOE_ERR_UNSUPPORTED, "k=%lld, E=%lld: the router takes k <= %d, E <= %d", (long long)k,
                      (long long)E, kMaxK, 64 * kMaxPer);
  const int64_t blocks = (T + 3) / 4;
  if (blocks > 0x7FFFFFFF) return qmoe::fail(QMOE_ERR_UNSUPPORTED, "too many tokens");
  const dim3 grid((unsigned)blocks), block(256);
  hipStream_t st = qmoe::as_stream(stream);
  const int per = (int)((E + 63) / 64);
  const int e = (int)E, kk = (int)k;
  if (per <= 1) router_topk_kernel<1><<<grid, block, 0, st>>>(logits, T, e, kk, norm, idx, scores);
  else if (per <= 2) router_topk_kernel<2><<<grid, block, 0, st>>>(logits, T, e, kk, norm, idx, scores);
  else if (per <= 4) router_topk_kernel<4><<<grid, block, 0, st>>>(logits, T, e, kk, norm, idx, scores);
  else if (per <= 8) router_topk_kernel<8><<<grid, block, 0, st>>>(logits, T, e, kk, norm, idx, scores);
  else router_topk_kernel<16><<<grid, block, 0, st>>>(logits, T, e, kk, norm, idx, scores);
  return qmoe::launch_status("router_topk_kernel");
}

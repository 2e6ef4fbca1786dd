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
// lowest expert index holding it, and retires that expert in its owner lane.
#include <limits.h>

#include "common.h"

namespace {

constexpr int kMaxK = 64;
constexpr int kMaxPer = 16;  // E <= 1024

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, 64));
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  return v;
}
__device__ __forceinline__ int wave_min(int v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = min(v, __shfl_xor(v, m, 64));
  return v;
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
    int bc = -1;
#pragma unroll
    for (int c = 0; c < PER; ++c)
      if (!(taken >> c & 1) && (bc < 0 || v[c] > bv)) {
        bv = v[c];
        bc = c;
      }
    const float wm = wave_max(bc >= 0 ? bv : -INFINITY);
    const int cand = (bc >= 0 && bv == wm) ? bc * 64 + lane : INT_MAX;
    int sel = wave_min(cand);
    if (sel == INT_MAX) sel = 0;  // no comparable candidate (NaN logits): stay in range
    if (cand == sel) taken |= 1u << bc;
    if (lane == 0) idx[t * k + j] = sel;
    if (lane == j) mine = wm;
  }
  if (norm) {
    const float top0 = __shfl(mine, 0, 64);
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

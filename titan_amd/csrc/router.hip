// Router top-k over fp32 logits, one wave per token, and the router logits
// (gfx950).  The selection itself (semantics, tie order, scores) is
// qmoe_topk::wave_topk in topk.h, which the decode kernels that pick their own
// experts share.
#include <limits.h>

#include "common.h"
#include "gemm_common.h"
#include "topk.h"

namespace {

using qmoe_topk::kMaxK;
using qmoe_topk::kMaxPer;
using qmoe_topk::wave_sum;

template <int PER>
__global__ __launch_bounds__(256) void router_topk_kernel(const float* __restrict__ logits, int64_t T, int E, int k,
                                                         int norm, int32_t* __restrict__ idx,
                                                         float* __restrict__ scores) {
  const int64_t t = (int64_t)blockIdx.x * 4 + threadIdx.x / 64;
  const int lane = threadIdx.x % 64;
  if (t >= T) return;
  int sel;
  float sc;
  qmoe_topk::wave_topk<PER>(logits + t * E, E, k, norm, sel, sc);
  if (lane < k) {
    idx[t * k + lane] = sel;
    scores[t * k + lane] = sc;
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

// Router logits for many tokens on the matrix cores: the same
// logits[t, e] = x[t] . W[e] in fp32 (bf16 products exact), as a tiled GEMM.
// A block computes TOK tokens x EXP experts (64 x 64, or 32 x 32 when the
// larger tiles would leave CUs idle).  K goes through an LDS ring of
// kRlStages chunks of 128 columns: per chunk the block copies its token and
// expert rows (256 bytes each) with global_load_lds, 16-byte unit u of row r
// at position u ^ (r & 7), so the 16-byte fragment reads are conflict-free.
// A chunk is eight k-steps of 16 columns; wave w takes k-steps 2w and 2w + 1
// for the whole tile (one v_mfma_f32_32x32x16_bf16 accumulator per 32 x 32
// piece, tokens the first operand's rows, experts the second's columns), so
// each fragment read from LDS feeds EXP / 32 or TOK / 32 MFMAs.  At k-step s,
// lane l feeds unit 8 * (l / 32) + s of its row: the MFMAs' K order is a
// permutation of the chunk's columns, the same for both operands, so each
// product x[t, k] * w[e, k] is summed exactly once.  The four waves' partial
// tiles are added through LDS in wave order.  Rows past T or E repeat the
// last row and are not stored.
//
// The copies bound it: a copies-only variant (no fragment reads, no MFMAs)
// took 7 of the kernel's 9.3 us per call with one 64 x 64 tile per block at
// K = 2048 (512 KiB), and a fifth ring stage changed nothing, so the tile
// size trades copy bytes per CU against CUs in use.
constexpr int kRlChunk = 128;              // K columns per stage
constexpr int kRlStages = 4;
constexpr int kRlRowBytes = 2 * kRlChunk;  // 256
// The tiled kernel from this many tokens (and experts) on; below, the
// one-wave-per-logit kernel above, whose x and W reads stay in L2.
constexpr int64_t kRlMinT = 48;
constexpr int64_t kRlMinE = 32;

template <int TOK, int EXP>
struct RlCfg {
  static constexpr int kStageBytes = (TOK + EXP) * kRlRowBytes;
  static constexpr int kCopies = kStageBytes / 1024 / 4;  // 16-byte copies per lane, wave and chunk
  static constexpr int kTokCopies = TOK * kRlRowBytes / 1024;  // wave-wide copies of token rows
  static_assert(kTokCopies % kCopies == 0, "a wave copies token rows or expert rows, not both");
  static_assert(4 * TOK * EXP * 4 <= kRlStages * kStageBytes, "partial tiles fit the ring");
};

template <int TOK, int EXP>
__global__ __launch_bounds__(256) void router_logits_mfma_kernel(const uint16_t* __restrict__ x, int64_t T, int K,
                                                                const uint16_t* __restrict__ w, int E,
                                                                int n_tok_tiles, int n_exp_tiles,
                                                                float* __restrict__ logits) {
  using C = RlCfg<TOK, EXP>;
  constexpr int MI = TOK / 32, NJ = EXP / 32;
  __shared__ __attribute__((aligned(1024))) char smem[kRlStages * C::kStageBytes];
  // Blocks b and b + 8 run on one XCD (dispatch goes round-robin over the
  // eight): a token tile's expert tiles share an XCD, so its x rows are
  // fetched into one L2.
  const int b = blockIdx.x;
  const int tt = b % 8 + 8 * (b / (8 * n_exp_tiles));
  const int et = (b / 8) % n_exp_tiles;
  if (tt >= n_tok_tiles) return;
  const int64_t t0 = (int64_t)tt * TOK;
  const int e0 = et * EXP;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid / 64);
  const int lane = tid % 64;
  const uint32_t lds = (uint32_t)(uintptr_t)smem;

  // Copy d of wave w is wave-wide copy j = kCopies * w + d, four rows of 256
  // bytes at stage bytes j * 1024: token rows 4j .. 4j + 3 for j < TOK / 4,
  // else expert rows 4j - TOK ..; lane i writes position i % 16 of row
  // 4j + i / 16 (tokens first, then experts).
  const char* src[C::kCopies];
#pragma unroll
  for (int d = 0; d < C::kCopies; ++d) {
    const int j = C::kCopies * wave + d;
    const int r = 4 * j + lane / 16;
    const int unit = (lane % 16) ^ (r & 7);
    if (j < C::kTokCopies)
      src[d] = reinterpret_cast<const char*>(x + min(t0 + r, T - 1) * K + unit * 8);
    else
      src[d] = reinterpret_cast<const char*>(w + (int64_t)min(e0 + r - TOK, E - 1) * K + unit * 8);
  }
  const int nchunks = K / kRlChunk;
  // A chunk past the last copies the last one again, onto the same bytes.
  auto issue = [&](int c) {
    c = min(c, nchunks - 1);
    const uint32_t st = lds + (uint32_t)(c % kRlStages) * C::kStageBytes + (uint32_t)(C::kCopies * wave) * 1024;
#pragma unroll
    for (int d = 0; d < C::kCopies; ++d) qmoe_gemm::dma16(src[d] + (size_t)c * kRlRowBytes, st + d * 1024);
  };

  const int l32 = lane % 32, h = lane / 32;
  f32x16_t acc[MI][NJ];
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

#pragma unroll
  for (int c = 0; c < kRlStages - 1; ++c) issue(c);
  for (int c = 0; c < nchunks; ++c) {
    // chunk c has landed once only the next kRlStages - 2 chunks' copies are
    // outstanding; the stage refilled below was last read in iteration c - 1,
    // which every wave has left once past the barrier
    qmoe_gemm::wait_vmem<(kRlStages - 2) * C::kCopies>();
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");  // no LDS read moves above the barrier
    issue(c + kRlStages - 1);
    const char* st = smem + (c % kRlStages) * C::kStageBytes;
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      // rows 32i + l32 all have (row & 7) == (l32 & 7)
      const int pos = ((8 * h + 2 * wave + s) ^ (l32 & 7)) * 16;
      i32x4_t fa[MI], fb[NJ];
#pragma unroll
      for (int i = 0; i < MI; ++i) fa[i] = *reinterpret_cast<const i32x4_t*>(st + (32 * i + l32) * kRlRowBytes + pos);
#pragma unroll
      for (int j = 0; j < NJ; ++j)
        fb[j] = *reinterpret_cast<const i32x4_t*>(st + (TOK + 32 * j + l32) * kRlRowBytes + pos);
#pragma unroll
      for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NJ; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, fa[i]),
                                                              __builtin_bit_cast(bf16x8_t, fb[j]), acc[i][j], 0, 0, 0);
    }
  }
  qmoe_gemm::wait_vmem<0>();  // the trailing repeat copies
  __syncthreads();            // every wave is done with the ring

  // Wave w's partial tile at float offset w * TOK * EXP as [token][expert]:
  // acc[i][j] register 4q + r of lane l holds token 32i + 8q + 4(l / 32) + r,
  // expert 32j + l % 32.
  float* part = reinterpret_cast<float*>(smem) + wave * TOK * EXP;
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) part[(32 * i + 8 * (r / 4) + 4 * h + r % 4) * EXP + 32 * j + l32] = acc[i][j][r];
  __syncthreads();
  const float* p = reinterpret_cast<const float*>(smem);
#pragma unroll
  for (int it = 0; it < TOK * EXP / 256; ++it) {
    const int o = it * 256 + tid;
    const int64_t t = t0 + o / EXP;
    const int e = e0 + o % EXP;
    const float v = ((p[o] + p[o + TOK * EXP]) + p[o + 2 * TOK * EXP]) + p[o + 3 * TOK * EXP];
    if (t < T && e < E) logits[t * E + e] = v;
  }
}

template <int TOK, int EXP>
int launch_router_logits_mfma(const uint16_t* x, int64_t T, int64_t K, const uint16_t* w, int64_t E, float* logits,
                              hipStream_t st) {
  const int64_t nt = (T + TOK - 1) / TOK, ne = (E + EXP - 1) / EXP;
  const int64_t blocks = 8 * ne * ((nt + 7) / 8);  // token tiles rounded up to the eight XCDs
  if (blocks > 0x7FFFFFFF) return qmoe::fail(QMOE_ERR_UNSUPPORTED, "too many tokens");
  router_logits_mfma_kernel<TOK, EXP><<<dim3((unsigned)blocks), dim3(256), 0, st>>>(x, T, (int)K, w, (int)E, (int)nt,
                                                                                   (int)ne, logits);
  return qmoe::launch_status("router_logits_mfma_kernel");
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
  if (T >= kRlMinT && E >= kRlMinE && K % kRlChunk == 0) {
    // 64 x 64 tiles once they number half the CUs or more (fewer copy bytes
    // per logit), else 32 x 32 (four times the blocks)
    if (((T + 63) / 64) * ((E + 63) / 64) >= 128)
      return launch_router_logits_mfma<64, 64>(x, T, K, w, E, logits, qmoe::as_stream(stream));
    return launch_router_logits_mfma<32, 32>(x, T, K, w, E, logits, qmoe::as_stream(stream));
  }
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

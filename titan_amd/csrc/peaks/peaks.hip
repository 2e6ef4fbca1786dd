// Ceiling probes for the bench's measured-peak denominators (qmoe_peaks.h):
// a streaming read over a buffer larger than the caches and dense MFMA loops.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "qmoe_peaks.h"

namespace {

constexpr int kStreamThreads = 256;
constexpr int kStreamBlocks = 256 * 8;  // eight blocks per CU
constexpr int kUnroll = 8;              // 16-byte loads in flight per thread

typedef __attribute__((__vector_size__(4 * sizeof(int)))) int i32x4_t;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16_t;
typedef __attribute__((__vector_size__(16 * sizeof(int)))) int i32x16_t;
typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;

__global__ __launch_bounds__(kStreamThreads) void stream_read_kernel(const i32x4_t* __restrict__ p, int64_t n,
                                                                     uint32_t* __restrict__ sink) {
  const int64_t stride = (int64_t)gridDim.x * kStreamThreads;
  int64_t i = (int64_t)blockIdx.x * kStreamThreads + threadIdx.x;
  uint32_t acc = 0;
  for (; i + (kUnroll - 1) * stride < n; i += kUnroll * stride) {
    i32x4_t v[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) v[u] = __builtin_nontemporal_load(p + i + u * stride);
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) acc ^= (uint32_t)(v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3]);
  }
  for (; i < n; i += stride) {
    const i32x4_t v = __builtin_nontemporal_load(p + i);
    acc ^= (uint32_t)(v[0] ^ v[1] ^ v[2] ^ v[3]);
  }
  // one word per block: the block's xor, written by thread 0
  __shared__ uint32_t red[kStreamThreads / 64];
  for (int m = 32; m >= 1; m >>= 1) acc ^= (uint32_t)__shfl_xor((int)acc, m, 64);
  if (threadIdx.x % 64 == 0) red[threadIdx.x / 64] = acc;
  __syncthreads();
  if (threadIdx.x == 0) sink[blockIdx.x] = red[0] ^ red[1] ^ red[2] ^ red[3];
}

constexpr int kMfmaThreads = 256;
constexpr int kMfmaBlocks = 256 * 2;  // two blocks of four waves per CU: two waves per SIMD

__device__ __forceinline__ uint32_t mix(uint32_t x) {
  x ^= x >> 16;
  x *= 0x7feb352dU;
  x ^= x >> 15;
  x *= 0x846ca68bU;
  x ^= x >> 16;
  return x;
}

// Random bf16 operands in [-2, 2) (exponent kept in range so no value is
// special): the matrix core's power, and so the sustained clock, depends on
// the data it multiplies.
__device__ __forceinline__ bf16x8_t rand_bf16x8(uint32_t seed) {
  i32x4_t r;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t h = mix(seed * 4 + j);
    r[j] = (int)((h & 0x807F807Fu) | 0x3F003F00u);  // sign, 7 mantissa bits, exponents 2^-1 .. 2^0
  }
  return __builtin_bit_cast(bf16x8_t, r);
}

__global__ __launch_bounds__(kMfmaThreads) void mfma_bf16_kernel(int iters, uint32_t* __restrict__ sink) {
  const uint32_t gid = blockIdx.x * kMfmaThreads + threadIdx.x;
  const bf16x8_t a0 = rand_bf16x8(gid * 4 + 0), a1 = rand_bf16x8(gid * 4 + 1);
  const bf16x8_t b0 = rand_bf16x8(gid * 4 + 2), b1 = rand_bf16x8(gid * 4 + 3);
  f32x16_t c0 = {}, c1 = {}, c2 = {}, c3 = {};
  for (int it = 0; it < iters; ++it) {
    c0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, b0, c0, 0, 0, 0);
    c1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, b0, c1, 0, 0, 0);
    c2 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, b1, c2, 0, 0, 0);
    c3 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, b1, c3, 0, 0, 0);
  }
  float s = 0.f;
#pragma unroll
  for (int r = 0; r < 16; ++r) s += c0[r] + c1[r] + c2[r] + c3[r];
  if (threadIdx.x % 64 == 0) sink[gid / 64] = __float_as_uint(s);
}

__global__ __launch_bounds__(kMfmaThreads) void mfma_i8_kernel(int iters, uint32_t* __restrict__ sink) {
  const uint32_t gid = blockIdx.x * kMfmaThreads + threadIdx.x;
  i32x4_t a0, a1, b0, b1;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    a0[j] = (int)mix(gid * 16 + j);
    a1[j] = (int)mix(gid * 16 + 4 + j);
    b0[j] = (int)mix(gid * 16 + 8 + j);
    b1[j] = (int)mix(gid * 16 + 12 + j);
  }
  i32x16_t c0 = {}, c1 = {}, c2 = {}, c3 = {};
  for (int it = 0; it < iters; ++it) {
    c0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a0, b0, c0, 0, 0, 0);
    c1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a1, b0, c1, 0, 0, 0);
    c2 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a0, b1, c2, 0, 0, 0);
    c3 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a1, b1, c3, 0, 0, 0);
  }
  int s = 0;
#pragma unroll
  for (int r = 0; r < 16; ++r) s += c0[r] ^ c1[r] ^ c2[r] ^ c3[r];
  if (threadIdx.x % 64 == 0) sink[gid / 64] = (uint32_t)s;
}

// Per-call floor of a one-launch decode step, in two parts.  The launch
// alone: blocks of W waves that do nothing.  The dependent chain: each wave
// (work item blockIdx.x * W + wave) reads its kernel arguments, then the
// expert id of its slot, then one 16-byte unit per lane of the first weight
// row of its row block (one row of 64 units, as the decode kernel's first
// row), and stores one word -- the three memory round trips a decode wave
// cannot overlap.  W = 1, 2, 4: the same waves in fewer, wider workgroups.
template <int W>
__global__ __launch_bounds__(64 * W) void launch_probe_kernel() {}

template <int W>
__global__ __launch_bounds__(64 * W) void chain_probe_kernel(const int32_t* __restrict__ ids, int blocks_per_slot,
                                                             int num_experts, const i32x4_t* __restrict__ w,
                                                             int64_t expert_units, int64_t block_units,
                                                             uint32_t* __restrict__ sink) {
  const int lane = threadIdx.x % 64;
  const uint32_t b = blockIdx.x * W + threadIdx.x / 64;  // the wave's work item
  const uint32_t slot = b / (uint32_t)blocks_per_slot;
  const uint32_t rb = b - slot * (uint32_t)blocks_per_slot;
  int e = ids[slot];
  e = min(max(e, 0), num_experts - 1);
  const i32x4_t v = __builtin_nontemporal_load(w + (int64_t)e * expert_units + (int64_t)rb * block_units + lane);
  uint32_t acc = (uint32_t)(v[0] ^ v[1] ^ v[2] ^ v[3]);
  for (int m = 32; m >= 1; m >>= 1) acc ^= (uint32_t)__shfl_xor((int)acc, m, 64);
  if (lane == 0) sink[b] = acc;
}

// chain_probe_kernel's waves, each reading all of its contiguous rows,
// LOADS KiB (one 16-byte unit per lane and KiB, all in flight together),
// and its rows' scale and bias units (lanes below sbu) after the id.
template <int W, int LOADS>
__global__ __launch_bounds__(64 * W) void burst_probe_kernel(const int32_t* __restrict__ ids, int blocks_per_slot,
                                                             int num_experts, const i32x4_t* __restrict__ w,
                                                             const i32x4_t* __restrict__ s,
                                                             const i32x4_t* __restrict__ b, int64_t expert_units,
                                                             int64_t sexpert_units, int sbu,
                                                             uint32_t* __restrict__ sink) {
  const int lane = threadIdx.x % 64;
  const uint32_t item = blockIdx.x * W + threadIdx.x / 64;
  const uint32_t slot = item / (uint32_t)blocks_per_slot;
  const uint32_t rb = item - slot * (uint32_t)blocks_per_slot;
  int e = ids[slot];
  e = min(max(e, 0), num_experts - 1);
  const i32x4_t* wp = w + (int64_t)e * expert_units + (int64_t)rb * (LOADS * 64) + lane;
  i32x4_t v[LOADS];
#pragma unroll
  for (int r = 0; r < LOADS; ++r) v[r] = __builtin_nontemporal_load(wp + r * 64);
  const int su = min(lane, sbu - 1);
  const int64_t so = (int64_t)e * sexpert_units + (int64_t)rb * sbu + su;
  const i32x4_t sv = __builtin_nontemporal_load(s + so), bv = __builtin_nontemporal_load(b + so);
  uint32_t acc = lane < sbu ? (uint32_t)(sv[0] ^ sv[1] ^ bv[2] ^ bv[3]) : 0u;
#pragma unroll
  for (int r = 0; r < LOADS; ++r) acc ^= (uint32_t)(v[r][0] ^ v[r][1] ^ v[r][2] ^ v[r][3]);
  for (int m = 32; m >= 1; m >>= 1) acc ^= (uint32_t)__shfl_xor((int)acc, m, 64);
  if (lane == 0) sink[item] = acc;
}

// One wave writes the GPU's constant 100 MHz clock (s_memrealtime) to
// stamps[slot] with a vector store: placed between the timed windows of one
// graph, it times each window from the GPU without a graph launch inside it.
__global__ __launch_bounds__(64) void stamp_kernel(uint64_t* __restrict__ stamps, int slot) {
  const uint64_t t = __builtin_amdgcn_s_memrealtime();
  if (threadIdx.x == 0) stamps[slot] = t;
}

int status() { return hipGetLastError() == hipSuccess ? 0 : 3; }

}  // namespace

extern "C" int qmoe_peak_stream_blocks(void) { return kStreamBlocks; }

extern "C" int qmoe_peak_stream_read(const void* buf, size_t bytes, uint32_t* sink, void* stream) {
  if (!buf || !sink || bytes % 16 || (reinterpret_cast<uintptr_t>(buf) & 15)) return 1;
  stream_read_kernel<<<dim3(kStreamBlocks), dim3(kStreamThreads), 0, reinterpret_cast<hipStream_t>(stream)>>>(
      static_cast<const i32x4_t*>(buf), (int64_t)(bytes / 16), sink);
  return status();
}

extern "C" int qmoe_peak_mfma_waves(void) { return kMfmaBlocks * kMfmaThreads / 64; }

extern "C" int qmoe_peak_mfma_bf16(int iters, uint32_t* sink, void* stream) {
  if (iters <= 0 || !sink) return 1;
  mfma_bf16_kernel<<<dim3(kMfmaBlocks), dim3(kMfmaThreads), 0, reinterpret_cast<hipStream_t>(stream)>>>(iters, sink);
  return status();
}

extern "C" int qmoe_peak_launch(int waves, int waves_per_block, void* stream) {
  if (waves <= 0 || (waves_per_block != 1 && waves_per_block != 2 && waves_per_block != 4) ||
      waves % waves_per_block)
    return 1;
  const dim3 grid(waves / waves_per_block), block(64 * waves_per_block);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (waves_per_block == 1) launch_probe_kernel<1><<<grid, block, 0, st>>>();
  else if (waves_per_block == 2) launch_probe_kernel<2><<<grid, block, 0, st>>>();
  else launch_probe_kernel<4><<<grid, block, 0, st>>>();
  return status();
}

extern "C" int qmoe_peak_chain(const int32_t* ids, int slots, int num_experts, const void* w, int rows_per_expert,
                               int row_bytes, int rows_per_block, int waves_per_block, uint32_t* sink,
                               void* stream) {
  // every wave reads units [0, 64) of row rb * rows_per_block of its expert:
  // in bounds when a row holds at least 64 units and the row blocks tile the
  // rows; the waves' work items are exactly 0 .. slots * blocks_per_slot - 1
  // when the blocks of waves_per_block waves divide them
  if (!ids || !w || !sink || slots <= 0 || num_experts <= 0 || rows_per_expert <= 0 || rows_per_block <= 0 ||
      row_bytes % 16 || row_bytes / 16 < 64 || rows_per_expert % rows_per_block ||
      (reinterpret_cast<uintptr_t>(w) & 15) ||
      (waves_per_block != 1 && waves_per_block != 2 && waves_per_block != 4))
    return 1;
  const int blocks_per_slot = rows_per_expert / rows_per_block;
  const int64_t items = (int64_t)slots * blocks_per_slot;
  if (items % waves_per_block || items > 0x7FFFFFFF) return 1;
  const int64_t row_units = row_bytes / 16;
  const dim3 grid((uint32_t)(items / waves_per_block)), block(64 * waves_per_block);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int64_t eu = (int64_t)rows_per_expert * row_units, bu = (int64_t)rows_per_block * row_units;
  const i32x4_t* wp = static_cast<const i32x4_t*>(w);
  if (waves_per_block == 1) chain_probe_kernel<1><<<grid, block, 0, st>>>(ids, blocks_per_slot, num_experts, wp, eu, bu, sink);
  else if (waves_per_block == 2) chain_probe_kernel<2><<<grid, block, 0, st>>>(ids, blocks_per_slot, num_experts, wp, eu, bu, sink);
  else chain_probe_kernel<4><<<grid, block, 0, st>>>(ids, blocks_per_slot, num_experts, wp, eu, bu, sink);
  return status();
}

template <int LOADS>
int launch_burst(dim3 grid, int waves_per_block, hipStream_t st, const int32_t* ids, int blocks_per_slot,
                 int num_experts, const i32x4_t* wp, const i32x4_t* sp, const i32x4_t* bp, int64_t eu, int64_t seu,
                 int sbu, uint32_t* sink) {
  const dim3 block(64 * waves_per_block);
  switch (waves_per_block) {
    case 1: burst_probe_kernel<1, LOADS><<<grid, block, 0, st>>>(ids, blocks_per_slot, num_experts, wp, sp, bp, eu, seu, sbu, sink); break;
    case 2: burst_probe_kernel<2, LOADS><<<grid, block, 0, st>>>(ids, blocks_per_slot, num_experts, wp, sp, bp, eu, seu, sbu, sink); break;
    case 4: burst_probe_kernel<4, LOADS><<<grid, block, 0, st>>>(ids, blocks_per_slot, num_experts, wp, sp, bp, eu, seu, sbu, sink); break;
    default: burst_probe_kernel<10, LOADS><<<grid, block, 0, st>>>(ids, blocks_per_slot, num_experts, wp, sp, bp, eu, seu, sbu, sink); break;
  }
  return status();
}

extern "C" int qmoe_peak_burst(const int32_t* ids, int slots, int num_experts, const void* w, const void* s,
                               const void* b, int rows_per_expert, int row_bytes, int srow_bytes, int rows_per_block,
                               int waves_per_block, uint32_t* sink, void* stream) {
  // wave (slot, rb) reads code units [rb * 64 L, rb * 64 L + 64 L) of its
  // expert's rows_per_expert * row_bytes / 16 (L = rows_per_block * row_bytes
  // / 1024 = 4, 8 or 16) and units [rb * sbu, rb * sbu + sbu) of its expert's
  // scale and bias units: in bounds when the row blocks tile the rows; the
  // work items are 0 .. slots * blocks_per_slot - 1 exactly
  if (!ids || !w || !s || !b || !sink || slots <= 0 || num_experts <= 0 || rows_per_expert <= 0 ||
      rows_per_block <= 0 || row_bytes <= 0 || row_bytes % 16 || rows_per_expert % rows_per_block ||
      srow_bytes <= 0 || (rows_per_block * srow_bytes) % 16 || rows_per_block * srow_bytes > 1024 ||
      ((int64_t)rows_per_expert * srow_bytes) % 16 ||
      ((reinterpret_cast<uintptr_t>(w) | reinterpret_cast<uintptr_t>(s) | reinterpret_cast<uintptr_t>(b)) & 15) ||
      (waves_per_block != 1 && waves_per_block != 2 && waves_per_block != 4 && waves_per_block != 10))
    return 1;
  const int64_t block_bytes = (int64_t)rows_per_block * row_bytes;
  if (block_bytes != 4096 && block_bytes != 8192 && block_bytes != 16384) return 1;
  const int blocks_per_slot = rows_per_expert / rows_per_block;
  const int64_t items = (int64_t)slots * blocks_per_slot;
  if (items % waves_per_block || items > 0x7FFFFFFF) return 1;
  const int sbu = rows_per_block * srow_bytes / 16;
  const int64_t eu = (int64_t)rows_per_expert * row_bytes / 16, seu = (int64_t)rows_per_expert * srow_bytes / 16;
  const dim3 grid((uint32_t)(items / waves_per_block));
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const i32x4_t* wp = static_cast<const i32x4_t*>(w);
  const i32x4_t* sp = static_cast<const i32x4_t*>(s);
  const i32x4_t* bp = static_cast<const i32x4_t*>(b);
  if (block_bytes == 4096)
    return launch_burst<4>(grid, waves_per_block, st, ids, blocks_per_slot, num_experts, wp, sp, bp, eu, seu, sbu, sink);
  if (block_bytes == 8192)
    return launch_burst<8>(grid, waves_per_block, st, ids, blocks_per_slot, num_experts, wp, sp, bp, eu, seu, sbu, sink);
  return launch_burst<16>(grid, waves_per_block, st, ids, blocks_per_slot, num_experts, wp, sp, bp, eu, seu, sbu, sink);
}

extern "C" int qmoe_peak_stamp(uint64_t* stamps, int slot, void* stream) {
  if (!stamps || slot < 0) return 1;
  stamp_kernel<<<dim3(1), dim3(64), 0, reinterpret_cast<hipStream_t>(stream)>>>(stamps, slot);
  return status();
}

extern "C" int qmoe_peak_mfma_i8(int iters, uint32_t* sink, void* stream) {
  if (iters <= 0 || !sink) return 1;
  mfma_i8_kernel<<<dim3(kMfmaBlocks), dim3(kMfmaThreads), 0, reinterpret_cast<hipStream_t>(stream)>>>(iters, sink);
  return status();
}

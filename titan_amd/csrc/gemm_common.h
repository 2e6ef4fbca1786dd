// Pieces shared by the grouped GEMMs over expert-sorted rows (gemm_bf16.hip,
// int8.hip): asynchronous global->LDS copies with explicit wait counts, the
// tile table's per-tile row counts, the heavy-first ranking of tiles and the
// persistent snake schedule over (tile, column block) units.
#pragma once

#include <stdint.h>

#include "common.h"

namespace qmoe_gemm {

// Rows per routing tile and 32-row subtiles per tile: the tile table of
// qmoe_route / qmoe_build_tiles uses tile_rows == kTileRows
// (qmoe_gemm_tile_rows()).
constexpr int kTileRows = 128;
constexpr int kMaxSub = kTileRows / 32;
constexpr int kThreads = 256;  // four waves per block (the bf16 GEMM)
constexpr int kBlocksPerCU = 2;
constexpr int kMaxOrder = 512;  // tiles ranked in LDS; more fall back to tile order

// Asynchronous 16- and 4-byte copies into LDS: lane i writes
// lds_base + i * size.  M0 carries the LDS base (declared clobbered).
__device__ __forceinline__ void dma16(const void* g, uint32_t lds_base) {
  asm volatile(
      "s_mov_b32 m0, %0\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %1, off"
      :
      : "s"(lds_base), "v"(g)
      : "memory", "m0");
}
__device__ __forceinline__ void dma4(const void* g, uint32_t lds_base) {
  asm volatile(
      "s_mov_b32 m0, %0\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dword %1, off"
      :
      : "s"(lds_base), "v"(g)
      : "memory", "m0");
}
// The same copies from a wave-uniform base (an SGPR pair) plus a 32-bit
// per-lane byte offset: lane i copies from sbase + voff_i.  (No instruction
// offset: an LDS-DMA load applies it to the LDS address as well.)
__device__ __forceinline__ void dma16s(const void* sbase, uint32_t voff, uint32_t lds_base) {
  asm volatile(
      "s_mov_b32 m0, %0\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %1, %2"
      :
      : "s"(lds_base), "v"(voff), "s"(sbase)
      : "memory", "m0");
}
__device__ __forceinline__ void dma4s(const void* sbase, uint32_t voff, uint32_t lds_base) {
  asm volatile(
      "s_mov_b32 m0, %0\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dword %1, %2"
      :
      : "s"(lds_base), "v"(voff), "s"(sbase)
      : "memory", "m0");
}
// Wait until at most N vector-memory operations of this wave are outstanding.
template <int N>
__device__ __forceinline__ void wait_vmem() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// A 64-bit value every lane holds alike, moved to scalar registers, so that
// stores address base + 32-bit lane offset (SGPR base) and keep no 64-bit
// per-lane pointers live.
__device__ __forceinline__ int64_t uniform64(int64_t v) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)v);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)((uint64_t)v >> 32));
  return (int64_t)(((uint64_t)hi << 32) | lo);
}

// 16-byte LDS reads whose results are only waited for together: an epilogue
// reads all of a pass's staged row pieces, then stores them.  (Written as
// plain loads, the compiler sinks each read next to its row-guarded store,
// and every read's latency is exposed.)  The reads and their
// s_waitcnt lgkmcnt(0) are one asm statement, so no output register is read
// or copied before the data has arrived; the outputs are early-clobber so no
// address register of a later read shares a destination of an earlier one.
// a[i] are LDS byte addresses.
__device__ __forceinline__ void lds_read16x4(i32x4_t (&v)[4], const uint32_t (&a)[4]) {
  asm volatile(
      "ds_read_b128 %0, %4\n\t"
      "ds_read_b128 %1, %5\n\t"
      "ds_read_b128 %2, %6\n\t"
      "ds_read_b128 %3, %7\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3])
      : "v"(a[0]), "v"(a[1]), "v"(a[2]), "v"(a[3])
      : "memory");
}
__device__ __forceinline__ void lds_read16x8(i32x4_t (&v)[8], const uint32_t (&a)[8]) {
  asm volatile(
      "ds_read_b128 %0, %8\n\t"
      "ds_read_b128 %1, %9\n\t"
      "ds_read_b128 %2, %10\n\t"
      "ds_read_b128 %3, %11\n\t"
      "ds_read_b128 %4, %12\n\t"
      "ds_read_b128 %5, %13\n\t"
      "ds_read_b128 %6, %14\n\t"
      "ds_read_b128 %7, %15\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3]), "=&v"(v[4]), "=&v"(v[5]), "=&v"(v[6]), "=&v"(v[7])
      : "v"(a[0]), "v"(a[1]), "v"(a[2]), "v"(a[3]), "v"(a[4]), "v"(a[5]), "v"(a[6]), "v"(a[7])
      : "memory");
}
template <int N>
__device__ __forceinline__ void lds_read16_all(i32x4_t (&v)[N], const uint32_t (&a)[N]) {
  static_assert(N == 4 || N == 8, "4 or 8 reads");
  if constexpr (N == 4) lds_read16x4(v, a);
  else lds_read16x8(v, a);
}

typedef __attribute__((__vector_size__(2 * sizeof(float)))) float f32x2_t;

// Two floats -> packed bf16 pair (low half = a), round to nearest even.
__device__ __forceinline__ uint32_t cvt_pk_bf16(float a, float b) {
  f32x2_t v = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

// The tile table: tile t covers rows tile_row[t] .. of expert tile_exp[t],
// at most kTileRows of them, ending at the expert's segment end offsets[e+1]
// (titan/kernels/moe_gather_ws.py:133-178).
struct Tiles {
  const int32_t* offsets;
  const int32_t* tile_row;
  const int32_t* tile_exp;
  const int32_t* ntiles;
  int64_t n_rows;
  int num_experts;
};

struct TileRows {
  int e;
  int64_t row0;
  int valid;  // rows of the tile (0: nothing to do)
};

__device__ __forceinline__ TileRows tile_rows_of(const Tiles& t, int tile) {
  TileRows r;
  r.e = min(max(t.tile_exp[tile], 0), t.num_experts - 1);
  r.row0 = t.tile_row[tile];
  const int64_t rowend = min((int64_t)t.offsets[r.e + 1], t.n_rows);
  r.valid = (int)max((int64_t)0, min((int64_t)kTileRows, rowend - r.row0));
  return r;
}

// Ranks the ntiles (<= kMaxOrder) tiles by subtile count, largest first and
// stable in tile order: order[rank] = tile.  cls is scratch LDS of kMaxOrder
// ints.  Called by the whole block.
__device__ inline void rank_tiles(const Tiles& t, int ntiles, int* order, int* cls) {
  for (int i = threadIdx.x; i < ntiles; i += blockDim.x) cls[i] = (tile_rows_of(t, i).valid + 31) / 32;
  __syncthreads();
  if (threadIdx.x < 64) {
    const int lane = threadIdx.x;
    const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    int total[kMaxSub + 1];
#pragma unroll
    for (int m = 0; m <= kMaxSub; ++m) total[m] = 0;
    for (int t0 = 0; t0 < ntiles; t0 += 64) {
      const int m = t0 + lane < ntiles ? cls[t0 + lane] : -1;
#pragma unroll
      for (int k = 0; k <= kMaxSub; ++k) total[k] += __popcll(__ballot(m == k));
    }
    int start[kMaxSub + 1];
    int acc = 0;
#pragma unroll
    for (int k = kMaxSub; k >= 0; --k) {
      start[k] = acc;
      acc += total[k];
    }
    for (int t0 = 0; t0 < ntiles; t0 += 64) {
      const int m = t0 + lane < ntiles ? cls[t0 + lane] : -1;
      int r = 0;
#pragma unroll
      for (int k = 0; k <= kMaxSub; ++k) {
        const uint64_t bal = __ballot(m == k);
        if (m == k) r = start[k] + __popcll(bal & below);
        start[k] += __popcll(bal);
      }
      if (m >= 0) order[r] = t0 + lane;
    }
  }
  __syncthreads();
}

// Persistent schedule.  Units are u = rank * NB + column block over the
// ranked tiles; P blocks (a multiple of 8) take them in a snake over their
// slots -- round k gives unit k * P + q to slot q on even rounds and
// k * P + P - 1 - q on odd ones -- which balances the largest units first and
// leaves the smallest for the tail.  Slot q sits on XCD q / (P / 8) (block
// ids are dealt round-robin to the 8 XCDs), so the column blocks of one tile,
// consecutive units, share an XCD's L2.
struct Snake {
  int64_t units;
  int P, q;
  __device__ __forceinline__ Snake(int64_t units_) : units(units_) {
    P = gridDim.x;
    const int b = blockIdx.x;
    q = (b % 8) * (P / 8) + b / 8;
  }
  // unit of round k, or -1 past the end
  __device__ __forceinline__ int64_t unit(int64_t k) const {
    const int64_t u = k * P + ((k & 1) ? P - 1 - q : q);
    return u < units ? u : -1;
  }
};

// Persistent grid size: blocks_per_cu blocks per CU, a multiple of 8, no
// more than the units (rounded up to 8).
int grid_blocks(int64_t units, int blocks_per_cu = kBlocksPerCU);

}  // namespace qmoe_gemm

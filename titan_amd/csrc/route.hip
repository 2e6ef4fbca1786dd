// Routing on the device: stable counting sort of expert ids, inverse
// permutation, per-expert segment offsets and the ragged tile list.
//
// Replaces _gather_sort (switch_layers.py:13-18: two mx.argsort calls and a
// gather) and the single-threadgroup tile walk of build_tiles
// (titan/kernels/moe_gather_ws.py:133-156).  Up to 4096 pairs and 512
// experts, one single-block launch does it all (route_fused_kernel); beyond,
// two launches up to 2048 experts:
//   count   one block per 1024-row chunk: per-chunk expert histogram in LDS
//   scatter one block per chunk, four waves: the block first sums every
//           expert's counts over all chunks and over the chunks before its
//           own, scans the totals into the experts' offsets, and so has each
//           expert's first output slot in its chunk (block 0 also writes the
//           offsets and the tile list); then each wave walks its quarter in
//           row order 64 rows at a time; lanes holding the same id find each
//           other with one ballot per id bit, so a row's slot is its chunk
//           base, plus the rows of its id in the chunk's earlier quarters,
//           plus the earlier rows of its id in its own quarter -- a stable
//           sort with no atomics.
// Beyond 2048 experts a separate one-block scan launch sits between the two
// and the scatter runs one wave per chunk (its LDS holds one count row).
#include <mutex>

#include "common.h"

namespace {

constexpr int kChunk = 1024;    // rows per histogram chunk
constexpr int kCountThreads = 256;
constexpr int kScanThreads = 1024;

__device__ __forceinline__ int clamp_id(int id, int E) { return id < 0 ? 0 : (id >= E ? E - 1 : id); }

// ids[i], read from an index clamped into [0, n) (n > 0) so that the read is
// unconditional: a thread's reads then issue back to back, where a branch
// around each one makes the compiler wait for each inside its branch.  The
// caller discards the value for i >= n.
__device__ __forceinline__ int load_id(const int32_t* __restrict__ ids, int64_t i, int64_t n) {
  return ids[i < n ? i : n - 1];
}

// counts: expert-major [E + 1][nchunks] (for the scan launch), or
// chunk-major [nchunks][E + 1] (for the scatter that scans; coalesced).
__global__ __launch_bounds__(kCountThreads) void route_count_kernel(const int32_t* __restrict__ ids, int64_t n,
                                                                    int E, int nchunks, bool chunk_major,
                                                                    int32_t* __restrict__ counts) {
  extern __shared__ int hist[];  // E + 1 (last slot: out-of-range ids)
  constexpr int kQ = kChunk / kCountThreads;
  const int64_t i0 = (int64_t)blockIdx.x * kChunk + threadIdx.x;
  int idv[kQ];  // launched with n > 0
#pragma unroll
  for (int q = 0; q < kQ; ++q) idv[q] = load_id(ids, i0 + q * kCountThreads, n);
  for (int e = threadIdx.x; e <= E; e += blockDim.x) hist[e] = 0;
  __syncthreads();
#pragma unroll
  for (int q = 0; q < kQ; ++q) {
    if (i0 + q * kCountThreads < n) {
      const int id = idv[q];
      if (id < 0 || id >= E) atomicAdd(&hist[E], 1);
      atomicAdd(&hist[clamp_id(id, E)], 1);
    }
  }
  __syncthreads();
  for (int e = threadIdx.x; e <= E; e += blockDim.x)
    counts[chunk_major ? (int64_t)blockIdx.x * (E + 1) + e : (int64_t)e * nchunks + blockIdx.x] = hist[e];
}

// Exclusive scan of one value per thread over a block of T threads; also
// returns the total.  Each wave scans its 64 values with shuffles, one wave
// scans the wave totals, and every thread adds its wave's base: three
// barriers.  lds holds at least T / 64 + 1 ints.
template <int T = kScanThreads>
__device__ int block_exclusive_scan(int v, int* lds, int* total) {
  static_assert(T % 64 == 0 && T <= 4096, "whole waves, at most 64");
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  constexpr int kWavesPerBlock = T / 64;
  int x = v;  // inclusive scan within the wave
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int y = __shfl_up(x, d, 64);
    if (lane >= d) x += y;
  }
  if (lane == 63) lds[w] = x;
  __syncthreads();
  if (w == 0) {
    const int t = lane < kWavesPerBlock ? lds[lane] : 0;
    int u = t;
#pragma unroll
    for (int d = 1; d < kWavesPerBlock; d <<= 1) {
      const int y = __shfl_up(u, d, 64);
      if (lane >= d) u += y;
    }
    if (lane < kWavesPerBlock) lds[lane] = u - t;  // exclusive base of wave `lane`
    if (lane == kWavesPerBlock - 1) lds[kWavesPerBlock] = u;
  }
  __syncthreads();
  *total = lds[kWavesPerBlock];
  const int res = lds[w] + x - v;
  __syncthreads();  // lds is free for the caller's next use
  return res;
}

// Tiles from offsets (offsets[0..E] visible to the block of T threads): one
// (row_start, expert) per tile_rows rows, expert-major; zero-fills
// [ntiles, max_tiles).
template <int T = kScanThreads>
__device__ void emit_tiles(const int32_t* offsets, int E, int tile_rows, int32_t* tile_row,
                           int32_t* tile_exp, int32_t* ntiles, int64_t max_tiles, int* lds) {
  const int tid = threadIdx.x;
  const int seg = (E + T - 1) / T;
  const int lo = min(tid * seg, E), hi = min(lo + seg, E);
  int local = 0;
  for (int e = lo; e < hi; ++e) local += (offsets[e + 1] - offsets[e] + tile_rows - 1) / tile_rows;
  int total;
  int64_t t = block_exclusive_scan<T>(local, lds, &total);
  for (int e = lo; e < hi; ++e) {
    const int s = offsets[e], q = offsets[e + 1];
    for (int r = s; r < q; r += tile_rows, ++t) {
      if (t < max_tiles) {
        tile_row[t] = r;
        tile_exp[t] = e;
      }
    }
  }
  const int64_t nt = min((int64_t)total, max_tiles);
  if (tid == 0) ntiles[0] = (int32_t)nt;
  for (int64_t j = nt + tid; j < max_tiles; j += T) {
    tile_row[j] = 0;
    tile_exp[j] = 0;
  }
}

// counts is the [E + 1][nchunks] table of route_count_kernel (row E: ids out
// of range).  One read pass: each thread keeps its contiguous segment of the
// table in registers (kSegMax values; a longer table is walked twice),
// writes back the exclusive prefix over rows 0..E-1 (each (expert, chunk)'s
// first output slot), reduces row E to the out-of-range count, and hands the
// expert offsets to the tile emission through LDS.
constexpr int kSegMax = 16;
constexpr int kScanMaxE = 8192;

__global__ __launch_bounds__(kScanThreads) void route_scan_kernel(int32_t* __restrict__ counts, int64_t n,
                                                                  int E, int nchunks, int tile_rows,
                                                                  int32_t* __restrict__ offsets,
                                                                  int32_t* __restrict__ tile_row,
                                                                  int32_t* __restrict__ tile_exp,
                                                                  int32_t* __restrict__ ntiles,
                                                                  int64_t max_tiles, int32_t* __restrict__ bad) {
  __shared__ int lds[kScanThreads];
  __shared__ int off[kScanMaxE + 1];
  const int tid = threadIdx.x;
  const int64_t Lmain = (int64_t)E * nchunks;
  const int64_t L = Lmain + nchunks;
  const int64_t seg = (L + kScanThreads - 1) / kScanThreads;
  const int64_t lo = min((int64_t)tid * seg, L), hi = min(lo + seg, L);
  int v[kSegMax];
  int local = 0, local_bad = 0;
  if (seg <= kSegMax) {
#pragma unroll
    for (int i = 0; i < kSegMax; ++i) v[i] = (lo + i < hi) ? counts[lo + i] : 0;
#pragma unroll
    for (int i = 0; i < kSegMax; ++i) {
      if (lo + i < Lmain) local += v[i];
      else local_bad += v[i];
    }
  } else {
    for (int64_t i = lo; i < hi; ++i) {
      if (i < Lmain) local += counts[i];
      else local_bad += counts[i];
    }
  }
  int nbad;
  block_exclusive_scan(local_bad, lds, &nbad);
  if (tid == 0) bad[0] = nbad;
  int total;
  int run = block_exclusive_scan(local, lds, &total);
  // an expert's offset is the prefix at its chunk-0 entry, index e * nchunks;
  // the thread's (expert, chunk) position advances with its index (one
  // division per thread, not one per entry)
  if (nchunks > 0) {
    int64_t e = lo / nchunks;
    int ch = (int)(lo - e * nchunks);
    if (seg <= kSegMax) {
#pragma unroll
      for (int i = 0; i < kSegMax; ++i) {
        const int64_t idx = lo + i;
        if (idx < hi && idx < Lmain) {
          counts[idx] = run;
          if (ch == 0) off[e] = run;
          run += v[i];
        }
        if (++ch == nchunks) {
          ch = 0;
          ++e;
        }
      }
    } else {
      for (int64_t idx = lo; idx < hi && idx < Lmain; ++idx) {
        const int c = counts[idx];
        counts[idx] = run;
        if (ch == 0) off[e] = run;
        run += c;
        if (++ch == nchunks) {
          ch = 0;
          ++e;
        }
      }
    }
  }
  if (nchunks == 0)
    for (int e = tid; e < E; e += kScanThreads) off[e] = 0;  // no rows: every segment is empty
  if (tid == 0) off[E] = (int)n;
  __syncthreads();
  for (int e = tid; e <= E; e += kScanThreads) offsets[e] = off[e];
  emit_tiles(off, E, tile_rows, tile_row, tile_exp, ntiles, max_tiles, lds);
}

// Stable scatter of one 1024-row chunk by W waves, wave w taking rows
// w * 1024/W .. in order.  Pass 1 matches equal ids within each 64-row step
// (one ballot per id bit), keeps the match masks and counts the wave's rows
// per id in its LDS row; a prefix over the waves, per id, turns the counts
// into each wave's first slot (the chunk's base from the scan first); pass 2
// ranks each row among the earlier rows of its id and writes it.
template <int W>
__global__ __launch_bounds__(64 * W) void route_scatter_kernel(const int32_t* __restrict__ ids, int64_t n, int E,
                                                               int nbits, int nchunks,
                                                               const int32_t* __restrict__ base,
                                                               int32_t* __restrict__ order,
                                                               int32_t* __restrict__ inv_order,
                                                               int32_t* __restrict__ sorted_ids) {
  extern __shared__ int run[];  // [W][E]
  constexpr int kSteps = kChunk / 64 / W;
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int c = blockIdx.x;
  int* my = run + w * E;
  const uint64_t lt = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  const int64_t r0 = (int64_t)c * kChunk + (int64_t)w * (kChunk / W);
  int idv[kSteps];  // the wave's ids, loaded up front (launched with n > 0)
#pragma unroll
  for (int step = 0; step < kSteps; ++step) idv[step] = load_id(ids, r0 + step * 64 + lane, n);
#pragma unroll
  for (int step = 0; step < kSteps; ++step)
    idv[step] = r0 + step * 64 + lane < n ? clamp_id(idv[step], E) : E;  // E: sentinel, never written
  for (int e = threadIdx.x; e < W * E; e += 64 * W) run[e] = 0;
  __syncthreads();
  uint64_t mv[kSteps];
#pragma unroll
  for (int step = 0; step < kSteps; ++step) {
    const bool valid = r0 + step * 64 + lane < n;
    const int id = idv[step];
    uint64_t m = __ballot(valid);
    if (!valid) m = ~m;
    for (int b = 0; b < nbits; ++b) {
      const bool bit = (id >> b) & 1;
      const uint64_t bb = __ballot(bit);
      m &= bit ? bb : ~bb;
    }
    mv[step] = m;
    if (valid && __popcll(m & lt) == 0) my[id] += __popcll(m);  // one leader per id and step
    __builtin_amdgcn_wave_barrier();
  }
  __syncthreads();
  for (int e = threadIdx.x; e < E; e += 64 * W) {
    int b = base[(int64_t)e * nchunks + c];
#pragma unroll
    for (int q = 0; q < W; ++q) {
      const int t = run[q * E + e];
      run[q * E + e] = b;
      b += t;
    }
  }
  __syncthreads();
#pragma unroll
  for (int step = 0; step < kSteps; ++step) {
    const int64_t i = r0 + step * 64 + lane;
    const bool valid = i < n;
    const int id = idv[step];
    const uint64_t m = mv[step];
    const int rank = __popcll(m & lt);
    if (valid) {
      const int dst = my[id] + rank;
      order[dst] = (int32_t)i;
      sorted_ids[dst] = id;
      inv_order[i] = dst;
    }
    __builtin_amdgcn_wave_barrier();  // every lane has read my[id] before the leader moves it
    if (valid && rank == 0) my[id] += __popcll(m);
    __builtin_amdgcn_wave_barrier();
  }
}

// route_scatter_kernel with the scan folded in (four waves per 1024-row
// chunk, E <= 2048).  counts is route_count_kernel's chunk-major
// [nchunks][E + 1] table.  Each block sums every expert's counts over all
// chunks (the expert's total) and over the chunks before its own (its prefix
// within the expert's segment), scans the totals in expert order into the
// offsets, and so holds its chunk's first slot per expert; block 0 also
// writes the offsets, the out-of-range count (row E) and the tile list.  The
// ranking and the writes are route_scatter_kernel's.
constexpr int kScanScatterWaves = 4;
constexpr int kScanScatterMaxE = 2048;

__global__ __launch_bounds__(64 * kScanScatterWaves) void route_scan_scatter_kernel(
    const int32_t* __restrict__ ids, int64_t n, int E, int nbits, int nchunks, const int32_t* __restrict__ counts,
    int tile_rows, int32_t* __restrict__ order, int32_t* __restrict__ inv_order, int32_t* __restrict__ sorted_ids,
    int32_t* __restrict__ offsets, int32_t* __restrict__ tile_row, int32_t* __restrict__ tile_exp,
    int32_t* __restrict__ ntiles, int64_t max_tiles, int32_t* __restrict__ bad) {
  constexpr int W = kScanScatterWaves;
  constexpr int T = 64 * W;
  constexpr int kSteps = kChunk / 64 / W;
  extern __shared__ int sm[];
  int* run = sm;             // [W][E]: per-wave counts, then first slots
  int* base = sm + W * E;    // [E]: the chunk's first slot per expert
  int* off = base + E;       // [E + 1]: the experts' offsets
  __shared__ int lds[T / 64 + 1];
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const int c = blockIdx.x;
  int* my = run + w * E;
  const uint64_t lt = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  const int64_t r0 = (int64_t)c * kChunk + (int64_t)w * (kChunk / W);
  int idv[kSteps];  // the wave's ids, loaded up front
  if (n > 0) {
#pragma unroll
    for (int step = 0; step < kSteps; ++step) idv[step] = load_id(ids, r0 + step * 64 + lane, n);
  }
#pragma unroll
  for (int step = 0; step < kSteps; ++step)
    idv[step] = r0 + step * 64 + lane < n ? clamp_id(idv[step], E) : E;  // E: sentinel, never written
  // block 0's last wave sums row E, the out-of-range ids, one chunk per lane
  // (the first 64 chunks' read unconditional, from a clamped index, so that
  // it overlaps the reads below rather than being waited for on its own)
  const bool sums_bad = c == 0 && w == W - 1 && nchunks > 0;  // wave-uniform
  int nb = 0, nb_rest = 0;
  if (sums_bad) {
    nb = counts[(int64_t)min(lane, nchunks - 1) * (E + 1) + E];
    for (int cc = lane + 64; cc < nchunks; cc += 64) nb_rest += counts[(int64_t)cc * (E + 1) + E];
  }
  // each expert's total over all chunks and its prefix over the chunks before
  // c, reading 16 chunks' counts at a time (all in flight together)
  constexpr int kBatch = 16;
  for (int e = tid; e < E; e += T) {
    int tot = 0, pre = 0;
    for (int c0 = 0; c0 < nchunks; c0 += kBatch) {
      int v[kBatch];
#pragma unroll
      for (int j = 0; j < kBatch; ++j) v[j] = c0 + j < nchunks ? counts[(int64_t)(c0 + j) * (E + 1) + e] : 0;
#pragma unroll
      for (int j = 0; j < kBatch; ++j) {
        tot += v[j];
        pre += c0 + j < c ? v[j] : 0;
      }
    }
    base[e] = pre;
    off[e] = tot;
  }
  if (sums_bad) {
    nb = (lane < nchunks ? nb : 0) + nb_rest;
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) nb += __shfl_xor(nb, d, 64);
    if (lane == 0) bad[0] = nb;
  } else if (c == 0 && w == W - 1 && lane == 0) {
    bad[0] = 0;  // no chunks
  }
  for (int e = tid; e < W * E; e += T) run[e] = 0;
  __syncthreads();
  {
    const int seg = (E + T - 1) / T;
    const int lo = min(tid * seg, E), hi = min(lo + seg, E);
    int local = 0;
    for (int e = lo; e < hi; ++e) local += off[e];
    int total;
    int r = block_exclusive_scan<T>(local, lds, &total);  // its barriers order the reads above before the writes
    for (int e = lo; e < hi; ++e) {
      const int t = off[e];
      off[e] = r;
      r += t;
    }
    if (tid == 0) off[E] = (int)n;
  }
  __syncthreads();
  for (int e = tid; e < E; e += T) base[e] += off[e];
  if (c == 0) {  // block-uniform
    for (int e = tid; e <= E; e += T) offsets[e] = off[e];
    emit_tiles<T>(off, E, tile_rows, tile_row, tile_exp, ntiles, max_tiles, lds);
  }
  uint64_t mv[kSteps];
#pragma unroll
  for (int step = 0; step < kSteps; ++step) {
    const bool valid = r0 + step * 64 + lane < n;
    const int id = idv[step];
    uint64_t m = __ballot(valid);
    if (!valid) m = ~m;
    for (int b = 0; b < nbits; ++b) {
      const bool bit = (id >> b) & 1;
      const uint64_t bb = __ballot(bit);
      m &= bit ? bb : ~bb;
    }
    mv[step] = m;
    if (valid && __popcll(m & lt) == 0) my[id] += __popcll(m);  // one leader per id and step
    __builtin_amdgcn_wave_barrier();
  }
  __syncthreads();
  for (int e = tid; e < E; e += T) {
    int b = base[e];
#pragma unroll
    for (int q = 0; q < W; ++q) {
      const int t = run[q * E + e];
      run[q * E + e] = b;
      b += t;
    }
  }
  __syncthreads();
#pragma unroll
  for (int step = 0; step < kSteps; ++step) {
    const int64_t i = r0 + step * 64 + lane;
    const bool valid = i < n;
    const int id = idv[step];
    const uint64_t m = mv[step];
    const int rank = __popcll(m & lt);
    if (valid) {
      const int dst = my[id] + rank;
      order[dst] = (int32_t)i;
      sorted_ids[dst] = id;
      inv_order[i] = dst;
    }
    __builtin_amdgcn_wave_barrier();  // every lane has read my[id] before the leader moves it
    if (valid && rank == 0) my[id] += __popcll(m);
    __builtin_amdgcn_wave_barrier();
  }
}

__global__ __launch_bounds__(kScanThreads) void tiles_from_sorted_kernel(const int32_t* __restrict__ sorted_ids,
                                                                         int64_t n, int E, int tile_rows,
                                                                         int32_t* __restrict__ offsets,
                                                                         int32_t* __restrict__ tile_row,
                                                                         int32_t* __restrict__ tile_exp,
                                                                         int32_t* __restrict__ ntiles,
                                                                         int64_t max_tiles) {
  __shared__ int lds[kScanThreads];
  for (int e = threadIdx.x; e <= E; e += kScanThreads) {
    int64_t lo = 0, hi = n;  // first row whose id >= e
    while (lo < hi) {
      const int64_t mid = (lo + hi) >> 1;
      if (sorted_ids[mid] < e) lo = mid + 1;
      else hi = mid;
    }
    offsets[e] = (int32_t)lo;
  }
  __syncthreads();
  emit_tiles(offsets, E, tile_rows, tile_row, tile_exp, ntiles, max_tiles, lds);
}

// The whole routing step in one block, for up to kFusedMaxN pairs and
// kFusedMaxE experts.  Wave w owns the contiguous row segment w of
// kFusedWaves and holds its ids in registers (at most kFusedSteps steps of 64
// rows, read once); its histogram row in LDS counts the segment, one block
// scan in (expert, wave) order turns the rows into each wave's first slot per
// expert, and the wave then walks its segment in order ranking equal ids with
// ballots, as route_scatter_kernel does per chunk -- stable, no global round
// trips between the phases.
constexpr int kFusedWaves = kScanThreads / 64;
constexpr int kFusedMaxE = 512;
constexpr int kFusedSteps = 4;
// measured in a graph of routing calls at 256 experts: 5.3 us at 80 pairs,
// 8.4 us at 4096 against 9.1 us for the count and scatter launches, where
// the block's serial walk has grown with n to about the launches' cost
constexpr int64_t kFusedMaxN = (int64_t)kFusedWaves * 64 * kFusedSteps;

__global__ __launch_bounds__(kScanThreads) void route_fused_kernel(
    const int32_t* __restrict__ ids, int64_t n, int E, int nbits, int tile_rows, int32_t* __restrict__ order,
    int32_t* __restrict__ inv_order, int32_t* __restrict__ sorted_ids, int32_t* __restrict__ offsets,
    int32_t* __restrict__ tile_row, int32_t* __restrict__ tile_exp, int32_t* __restrict__ ntiles,
    int64_t max_tiles, int32_t* __restrict__ bad) {
  extern __shared__ int sm[];
  int* hist = sm;                          // [kFusedWaves][E + 1]; slot E counts out-of-range ids
  int* off = sm + kFusedWaves * (E + 1);   // [E + 1]
  __shared__ int lds[kScanThreads];
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const int64_t seg = (n + kFusedWaves - 1) / kFusedWaves;
  const int64_t lo = min((int64_t)w * seg, n), hi = min(lo + seg, n);
  int* my = hist + w * (E + 1);
  int idv[kFusedSteps];  // the segment's ids (seg <= 64 * kFusedSteps)
  if (hi > lo) {  // wave-uniform
#pragma unroll
    for (int q = 0; q < kFusedSteps; ++q) idv[q] = load_id(ids, lo + 64 * q + lane, hi);
  }
  for (int i = tid; i < kFusedWaves * (E + 1); i += kScanThreads) hist[i] = 0;
  __syncthreads();
#pragma unroll
  for (int q = 0; q < kFusedSteps; ++q) {
    if (lo + 64 * q + lane < hi) {
      if (idv[q] < 0 || idv[q] >= E) atomicAdd(&my[E], 1);
      atomicAdd(&my[clamp_id(idv[q], E)], 1);
    }
  }
  __syncthreads();
  if (tid == 0) {
    int nb = 0;
    for (int q = 0; q < kFusedWaves; ++q) nb += hist[q * (E + 1) + E];
    bad[0] = nb;
  }
  // exclusive scan, in place, over f = e * kFusedWaves + w (expert-major): a
  // wave's rows of one expert come after every lower wave's rows of it
  const int L = E * kFusedWaves;
  const int per = (L + kScanThreads - 1) / kScanThreads;
  const int f0 = min(tid * per, L), f1 = min(f0 + per, L);
  int local = 0;
  for (int f = f0; f < f1; ++f) local += hist[(f % kFusedWaves) * (E + 1) + f / kFusedWaves];
  int total;
  int run = block_exclusive_scan(local, lds, &total);  // its barriers order every read above before the writes
  for (int f = f0; f < f1; ++f) {
    int* h = &hist[(f % kFusedWaves) * (E + 1) + f / kFusedWaves];
    const int c = *h;
    *h = run;
    run += c;
  }
  __syncthreads();
  for (int e = tid; e < E; e += kScanThreads) {
    off[e] = hist[e];  // wave 0's first slot = the expert's offset
    offsets[e] = hist[e];
  }
  if (tid == 0) {
    off[E] = (int)n;
    offsets[E] = (int32_t)n;
  }
  const uint64_t lt = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
#pragma unroll
  for (int q = 0; q < kFusedSteps; ++q) {
    if (lo + 64 * q >= hi) break;  // wave-uniform
    const int64_t i = lo + 64 * q + lane;
    const bool valid = i < hi;
    const int id = valid ? clamp_id(idv[q], E) : E;  // E: sentinel, never written
    uint64_t m = __ballot(valid);
    if (!valid) m = ~m;
    for (int bb = 0; bb < nbits; ++bb) {
      const bool bit = (id >> bb) & 1;
      const uint64_t x = __ballot(bit);
      m &= bit ? x : ~x;
    }
    const int rank = __popcll(m & lt);
    if (valid) {
      const int dst = my[id] + rank;
      order[dst] = (int32_t)i;
      sorted_ids[dst] = id;
      inv_order[i] = dst;
    }
    __builtin_amdgcn_wave_barrier();  // every lane has read my[id] before the leader moves it
    if (valid && rank == 0) my[id] += __popcll(m);
    __builtin_amdgcn_wave_barrier();
  }
  __syncthreads();
  emit_tiles(off, E, tile_rows, tile_row, tile_exp, ntiles, max_tiles, lds);
}

int64_t n_chunks(int64_t n) { return (n + kChunk - 1) / kChunk; }

// The routing launches, given a workspace of qmoe_route_workspace_size bytes
// (word 0 unused when `bad` points elsewhere, then (E + 1) * chunks counts).
int route_launch(const int32_t* ids, int64_t n_pairs, int32_t num_experts, int32_t tile_rows, int32_t* order,
                 int32_t* inv_order, int32_t* sorted_ids, int32_t* offsets, int32_t* tile_row, int32_t* tile_exp,
                 int32_t* ntiles, int64_t max_tiles, int32_t* ws, int32_t* bad, hipStream_t st);

}  // namespace

extern "C" size_t qmoe_route_workspace_size(int64_t n_pairs, int32_t num_experts) {
  if (n_pairs < 0 || num_experts <= 0) return 0;
  const int64_t words = 64 + (int64_t)(num_experts + 1) * n_chunks(n_pairs);
  return (size_t)(((words * 4) + 255) / 256 * 256);
}

extern "C" int qmoe_route(const int32_t* ids, int64_t n_pairs, int32_t num_experts, int32_t tile_rows,
                          int32_t* order, int32_t* inv_order, int32_t* sorted_ids, int32_t* offsets,
                          int32_t* tile_row, int32_t* tile_exp, int32_t* ntiles, int64_t max_tiles,
                          void* workspace, size_t workspace_bytes, void* stream) {
  if (n_pairs < 0 || num_experts <= 0 || tile_rows <= 0 || max_tiles < 0)
    return qmoe::fail(QMOE_ERR_INVALID, "bad sizes");
  if (num_experts > 8192) return qmoe::fail(QMOE_ERR_UNSUPPORTED, "num_experts=%d > 8192", num_experts);
  if (n_pairs > 0x7FFFFFFF) return qmoe::fail(QMOE_ERR_UNSUPPORTED, "too many pairs");
  if (!offsets || !tile_row || !tile_exp || !ntiles || (max_tiles == 0 && n_pairs > 0))
    return qmoe::fail(QMOE_ERR_INVALID, "null pointer");
  if (n_pairs > 0 && (!ids || !order || !inv_order || !sorted_ids)) return qmoe::fail(QMOE_ERR_INVALID, "null pointer");
  const size_t need = qmoe_route_workspace_size(n_pairs, num_experts);
  if (!workspace || workspace_bytes < need)
    return qmoe::fail(QMOE_ERR_WORKSPACE, "route needs %zu workspace bytes", need);
  int32_t* ws = static_cast<int32_t*>(workspace);
  return route_launch(ids, n_pairs, num_experts, tile_rows, order, inv_order, sorted_ids, offsets, tile_row,
                      tile_exp, ntiles, max_tiles, ws, ws, qmoe::as_stream(stream));
}

namespace {

int route_launch(const int32_t* ids, int64_t n_pairs, int32_t num_experts, int32_t tile_rows, int32_t* order,
                 int32_t* inv_order, int32_t* sorted_ids, int32_t* offsets, int32_t* tile_row, int32_t* tile_exp,
                 int32_t* ntiles, int64_t max_tiles, int32_t* ws, int32_t* bad, hipStream_t st) {
  const int64_t nch = n_chunks(n_pairs);
  int32_t* counts = ws + 64;
  if (n_pairs <= kFusedMaxN && num_experts <= kFusedMaxE) {
    int nbits = 1;
    while ((1 << nbits) <= num_experts) ++nbits;  // ids in [0, E] (E is the sentinel)
    const size_t shm = (size_t)(kFusedWaves + 1) * (num_experts + 1) * sizeof(int);
    route_fused_kernel<<<dim3(1), dim3(kScanThreads), shm, st>>>(ids, n_pairs, num_experts, nbits, tile_rows,
                                                                order, inv_order, sorted_ids, offsets, tile_row,
                                                                tile_exp, ntiles, max_tiles, bad);
    return qmoe::launch_status("route_fused_kernel");
  }
  int nbits = 1;
  while ((1 << nbits) <= num_experts) ++nbits;  // ids in [0, E] (E is the sentinel)
  const bool scan_in_scatter = num_experts <= kScanScatterMaxE;
  if (nch > 0) {
    route_count_kernel<<<dim3((unsigned)nch), dim3(kCountThreads), (num_experts + 1) * sizeof(int), st>>>(
        ids, n_pairs, num_experts, (int)nch, scan_in_scatter, counts);
    int rc = qmoe::launch_status("route_count_kernel");
    if (rc) return rc;
  }
  if (scan_in_scatter) {
    // (W + 2) * E + 1 ints of LDS; one block even without rows (it writes
    // the zero offsets and the empty tile list)
    const size_t shm = ((size_t)(kScanScatterWaves + 2) * num_experts + 1) * sizeof(int);
    route_scan_scatter_kernel<<<dim3((unsigned)(nch > 0 ? nch : 1)), dim3(64 * kScanScatterWaves), shm, st>>>(
        ids, n_pairs, num_experts, nbits, (int)nch, counts, tile_rows, order, inv_order, sorted_ids, offsets,
        tile_row, tile_exp, ntiles, max_tiles, bad);
    return qmoe::launch_status("route_scan_scatter_kernel");
  }
  route_scan_kernel<<<dim3(1), dim3(kScanThreads), 0, st>>>(counts, n_pairs, num_experts, (int)nch, tile_rows,
                                                            offsets, tile_row, tile_exp, ntiles, max_tiles, bad);
  int rc = qmoe::launch_status("route_scan_kernel");
  if (rc || nch == 0) return rc;
  route_scatter_kernel<1><<<dim3((unsigned)nch), dim3(64), num_experts * sizeof(int), st>>>(
      ids, n_pairs, num_experts, nbits, (int)nch, counts, order, inv_order, sorted_ids);
  return qmoe::launch_status("route_scatter_kernel");
}

}  // namespace

extern "C" int qmoe_build_tiles(const int32_t* sorted_ids, int64_t n_rows, int32_t num_experts,
                                int32_t tile_rows, int32_t* offsets, int32_t* tile_row, int32_t* tile_exp,
                                int32_t* ntiles, int64_t max_tiles, void* stream) {
  if (n_rows < 0 || num_experts <= 0 || tile_rows <= 0 || max_tiles < 0)
    return qmoe::fail(QMOE_ERR_INVALID, "bad sizes");
  if (n_rows > 0x7FFFFFFF) return qmoe::fail(QMOE_ERR_UNSUPPORTED, "too many rows");
  if (!offsets || !tile_row || !tile_exp || !ntiles || (n_rows > 0 && !sorted_ids))
    return qmoe::fail(QMOE_ERR_INVALID, "null pointer");
  tiles_from_sorted_kernel<<<dim3(1), dim3(kScanThreads), 0, qmoe::as_stream(stream)>>>(
      sorted_ids, n_rows, num_experts, tile_rows, offsets, tile_row, tile_exp, ntiles, max_tiles);
  return qmoe::launch_status("tiles_from_sorted_kernel");
}

// ------------------------------------------------------------------------
// qmoe_route_noalloc: qmoe_route with its workspace in a file-scope device
// array instead of caller memory, for callers that cannot allocate (code
// under graph capture, serving loops that forbid allocation).  Each GPU the
// library runs on holds its own copy of the array until the process ends;
// every call on that GPU shares it, so calls that overlap on one GPU race.
// Nothing in it has to start at zero: the count launch writes every
// (expert, chunk) count it later reads, and the out-of-range count is
// written to the caller's n_bad (or, when that is null, to word 0).
static __device__ __align__(256) int32_t scratch[QMOE_ROUTE_NOALLOC_SCRATCH_BYTES / sizeof(int32_t)];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
int32_t* g_scratch[kMaxDevices];  // device address of `scratch` per device, once looked up

// The device address of this device's `scratch`: looked up once per device,
// on the first call there, with that device current.  The array's host-side
// name is only a handle for the runtime, never a device address.
int scratch_for_device(int dev, int32_t** out) {
  if (dev < 0 || dev >= kMaxDevices) return qmoe::fail(QMOE_ERR_UNSUPPORTED, "device %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return qmoe::fail(QMOE_ERR_HIP, "hipGetSymbolAddress(scratch) on device %d: %s", dev, hipGetErrorString(e));
    g_scratch[dev] = static_cast<int32_t*>(p);
  }
  *out = g_scratch[dev];
  return QMOE_OK;
}

}  // namespace

extern "C" int qmoe_route_noalloc(const int32_t* ids, int64_t n_pairs, int32_t num_experts, int32_t tile_rows,
                                  int32_t* order, int32_t* inv_order, int32_t* sorted_ids, int32_t* offsets,
                                  int32_t* tile_row, int32_t* tile_exp, int32_t* ntiles, int64_t max_tiles,
                                  int32_t* n_bad, void* stream) {
  if (n_pairs < 0 || num_experts <= 0 || tile_rows <= 0 || max_tiles < 0)
    return qmoe::fail(QMOE_ERR_INVALID, "bad sizes");
  if (num_experts > 8192) return qmoe::fail(QMOE_ERR_UNSUPPORTED, "num_experts=%d > 8192", num_experts);
  if (n_pairs > 0x7FFFFFFF) return qmoe::fail(QMOE_ERR_UNSUPPORTED, "too many pairs");
  const size_t need = qmoe_route_workspace_size(n_pairs, num_experts);
  if (need > QMOE_ROUTE_NOALLOC_SCRATCH_BYTES)
    return qmoe::fail(QMOE_ERR_UNSUPPORTED,
                      "n_pairs=%lld with %d experts needs %zu scratch bytes; the static scratch holds %zu "
                      "(use qmoe_route with a workspace)",
                      (long long)n_pairs, num_experts, need, (size_t)QMOE_ROUTE_NOALLOC_SCRATCH_BYTES);
  if (!offsets || !tile_row || !tile_exp || !ntiles || (max_tiles == 0 && n_pairs > 0))
    return qmoe::fail(QMOE_ERR_INVALID, "null pointer");
  if (n_pairs > 0 && (!ids || !order || !inv_order || !sorted_ids)) return qmoe::fail(QMOE_ERR_INVALID, "null pointer");
  hipStream_t st = qmoe::as_stream(stream);
  int dev = -1, sdev = -1;
  if (hipGetDevice(&dev) != hipSuccess) return qmoe::fail(QMOE_ERR_HIP, "hipGetDevice failed");
  if (hipStreamGetDevice(st, &sdev) != hipSuccess) return qmoe::fail(QMOE_ERR_HIP, "hipStreamGetDevice failed");
  if (sdev != dev)
    return qmoe::fail(QMOE_ERR_INVALID, "stream is on device %d but device %d is current", sdev, dev);
  int32_t* ws = nullptr;
  const int rc = scratch_for_device(dev, &ws);
  if (rc) return rc;
  return route_launch(ids, n_pairs, num_experts, tile_rows, order, inv_order, sorted_ids, offsets, tile_row,
                      tile_exp, ntiles, max_tiles, ws, n_bad ? n_bad : ws, st);
}

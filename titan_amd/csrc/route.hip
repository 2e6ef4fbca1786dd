// Routing on the device: stable counting sort of expert ids, inverse
// permutation, per-expert segment offsets and the ragged tile list.
//
// Replaces _gather_sort (switch_layers.py:13-18: two mx.argsort calls and a
// gather) and the single-threadgroup tile walk of build_tiles
// (titan/kernels/moe_gather_ws.py:133-156).  Up to 8192 pairs and 512
// experts, one single-block launch does it all (route_fused_kernel); beyond,
// three launches:
//   count   one block per 1024-row chunk: per-chunk expert histogram in LDS
//   scan    one block: expert-major exclusive scan of the histograms, which
//           gives each (expert, chunk) its first output slot, the offsets,
//           and the tile list
//   scatter four waves per chunk (one for more than 2048 experts), each
//           walking its quarter in row order 64 rows at a time; lanes
//           holding the same id find each other with one ballot per id bit,
//           so a row's slot is its chunk base, plus the rows of its id in the
//           chunk's earlier quarters, plus the earlier rows of its id in its
//           own quarter -- a stable sort with no atomics.
#include <mutex>

#include "common.h"

namespace {

constexpr int kChunk = 1024;    // rows per histogram chunk
constexpr int kCountThreads = 256;
constexpr int kScanThreads = 1024;

__device__ __forceinline__ int clamp_id(int id, int E) { return id < 0 ? 0 : (id >= E ? E - 1 : id); }

__global__ __launch_bounds__(kCountThreads) void route_count_kernel(const int32_t* __restrict__ ids, int64_t n,
                                                                    int E, int nchunks,
                                                                    int32_t* __restrict__ counts) {
  extern __shared__ int hist[];  // E + 1 (last slot: out-of-range ids)
  for (int e = threadIdx.x; e <= E; e += blockDim.x) hist[e] = 0;
  __syncthreads();
#pragma unroll
  for (int q = 0; q < kChunk / kCountThreads; ++q) {
    const int64_t i = (int64_t)blockIdx.x * kChunk + q * kCountThreads + threadIdx.x;
    if (i < n) {
      const int id = ids[i];
      if (id < 0 || id >= E) atomicAdd(&hist[E], 1);
      atomicAdd(&hist[clamp_id(id, E)], 1);
    }
  }
  __syncthreads();
  for (int e = threadIdx.x; e <= E; e += blockDim.x) counts[(int64_t)e * nchunks + blockIdx.x] = hist[e];
}

// Exclusive scan of one value per thread over the block; also returns the
// total.  Each wave scans its 64 values with shuffles, one wave scans the
// 16 wave totals, and every thread adds its wave's base: three barriers.
__device__ int block_exclusive_scan(int v, int* lds, int* total) {
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  constexpr int kWavesPerBlock = kScanThreads / 64;
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

// Tiles from offsets (offsets[0..E] visible to the block): one (row_start,
// expert) per tile_rows rows, expert-major; zero-fills [ntiles, max_tiles).
__device__ void emit_tiles(const int32_t* offsets, int E, int tile_rows, int32_t* tile_row,
                           int32_t* tile_exp, int32_t* ntiles, int64_t max_tiles, int* lds) {
  const int tid = threadIdx.x;
  const int seg = (E + kScanThreads - 1) / kScanThreads;
  const int lo = min(tid * seg, E), hi = min(lo + seg, E);
  int local = 0;
  for (int e = lo; e < hi; ++e) local += (offsets[e + 1] - offsets[e] + tile_rows - 1) / tile_rows;
  int total;
  int64_t t = block_exclusive_scan(local, lds, &total);
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
  for (int64_t j = nt + tid; j < max_tiles; j += kScanThreads) {
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
  int idv[kSteps];  // the wave's ids, loaded up front (independent loads)
#pragma unroll
  for (int step = 0; step < kSteps; ++step) {
    const int64_t i = r0 + step * 64 + lane;
    idv[step] = i < n ? clamp_id(ids[i], E) : E;  // E: sentinel, never written
  }
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
// kFusedMaxE experts: three dependent launches cost ~17 us even for ten ids.
// Wave w owns the contiguous row segment w of kFusedWaves; its histogram row
// in LDS counts the segment, one block scan in (expert, wave) order turns the
// rows into each wave's first slot per expert, and the wave then walks its
// segment in order ranking equal ids with ballots, as route_scatter_kernel
// does per chunk -- stable, no global round trips between the phases.  Ids
// are loaded kBatch steps of 64 rows at a time so the loads overlap.
constexpr int kFusedWaves = kScanThreads / 64;
constexpr int kFusedMaxE = 512;
// measured: 8 us at 10 pairs against 17 us for the three launches, 59 us at
// 40960 pairs against 28 us (a block's serial walk grows with n)
constexpr int64_t kFusedMaxN = 8192;
constexpr int kBatch = 16;

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
  for (int i = tid; i < kFusedWaves * (E + 1); i += kScanThreads) hist[i] = 0;
  __syncthreads();
  for (int64_t b = lo; b < hi; b += 64 * kBatch) {
    int idv[kBatch];
#pragma unroll
    for (int q = 0; q < kBatch; ++q) {
      const int64_t i = b + 64 * q + lane;
      idv[q] = i < hi ? ids[i] : 0;
    }
#pragma unroll
    for (int q = 0; q < kBatch; ++q) {
      if (b + 64 * q + lane < hi) {
        if (idv[q] < 0 || idv[q] >= E) atomicAdd(&my[E], 1);
        atomicAdd(&my[clamp_id(idv[q], E)], 1);
      }
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
  for (int64_t b = lo; b < hi; b += 64 * kBatch) {
    int idv[kBatch];
#pragma unroll
    for (int q = 0; q < kBatch; ++q) {
      const int64_t i = b + 64 * q + lane;
      idv[q] = i < hi ? clamp_id(ids[i], E) : E;  // E: sentinel, never written
    }
#pragma unroll
    for (int q = 0; q < kBatch; ++q) {
      if (b + 64 * q >= hi) break;  // uniform
      const int64_t i = b + 64 * q + lane;
      const bool valid = i < hi;
      const int id = idv[q];
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
  if (nch > 0) {
    route_count_kernel<<<dim3((unsigned)nch), dim3(kCountThreads), (num_experts + 1) * sizeof(int), st>>>(
        ids, n_pairs, num_experts, (int)nch, counts);
    int rc = qmoe::launch_status("route_count_kernel");
    if (rc) return rc;
  }
  route_scan_kernel<<<dim3(1), dim3(kScanThreads), 0, st>>>(counts, n_pairs, num_experts, (int)nch, tile_rows,
                                                            offsets, tile_row, tile_exp, ntiles, max_tiles, bad);
  int rc = qmoe::launch_status("route_scan_kernel");
  if (rc || nch == 0) return rc;
  int nbits = 1;
  while ((1 << nbits) <= num_experts) ++nbits;  // ids in [0, E] (E is the sentinel)
  if (num_experts <= 2048)  // four waves per chunk: 4 * E ints of LDS
    route_scatter_kernel<4><<<dim3((unsigned)nch), dim3(256), 4 * num_experts * sizeof(int), st>>>(
        ids, n_pairs, num_experts, nbits, (int)nch, counts, order, inv_order, sorted_ids);
  else
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

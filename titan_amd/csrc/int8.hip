// int8-activation x int4-weight gate_up on int8 MFMA (gfx950).
//
// Activations: per-token symmetric int8, sx = max|x| / 127 (fp32, correctly
// rounded), xi = clamp(rint(x / sx), -127, 127).  Codes q in [0, 15] are
// valid signed int8 as they stand, so neither side needs a zero point (the
// reference's uint8 zero-point-128 scheme and its qsum table,
// titan/kernels/moe_gather_int8.py:15-33,189-248, have no counterpart here).
//
// Per 64-wide group g (= one affine group):
//   D_g[m, n] = sum_{k in g} xi[m, k] * q[n, k]      int32, exact, 2 MFMA k-steps
//   R_g[m]    = sum_{k in g} xi[m, k]                int32, exact
//   y[m, n]   = sx[m] * ( sum_g s[n,g] * D_g[m,n]  +  sum_g b[n,g] * R_g[m] )
// The first sum is rescaled in fp32 after every group; the second is a
// [rows x G] x [G x N] product run once at the end on bf16 MFMA with R split
// into two bf16 terms (|R| <= 8128: hi = bf16(R) and lo = R - hi are exact).
#include "gemm_common.h"

namespace {

// ---------------------------------------------------------------- quantizer

// One wave per row (K a multiple of 512); lane l owns the 8-element pieces
// 64t + l, so each 16-byte load instruction of the wave reads 1 KiB of the
// row contiguously (measured 10.4 -> 10.0 us at 4096 x 2048 and 21.7 -> 17.6
// us at 4096 x 4096 against 64 consecutive elements per lane).  Rows up to
// K = 4096 stay in registers between the max pass and the quantising pass;
// longer rows are read again.
constexpr int kQuantRegElems = 64;

// 8 bf16 of one 16-byte load -> 8 int8, rint(x / sc) clamped to [-127, 127]
// (sc == 0: zeros), packed low byte first.
__device__ __forceinline__ uint2 quant_pack(const uint4 q, float sc) {
  const uint32_t v[4] = {q.x, q.y, q.z, q.w};
  uint32_t packed[2] = {0u, 0u};
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const float xv = (j & 1) ? bf16hi(v[j >> 1]) : bf16lo(v[j >> 1]);
    float t = sc == 0.f ? 0.f : rintf(__fdiv_rn(xv, sc));
    t = fminf(fmaxf(t, -127.f), 127.f);
    packed[j >> 2] |= ((uint32_t)(int)t & 0xFFu) << (8 * (j & 3));
  }
  return make_uint2(packed[0], packed[1]);
}

__global__ __launch_bounds__(256) void quant_act_kernel(const uint16_t* __restrict__ x, int64_t R, int K,
                                                        int8_t* __restrict__ xi, float* __restrict__ sx) {
  const int64_t r = (int64_t)blockIdx.x * 4 + threadIdx.x / 64;
  const int lane = threadIdx.x % 64;
  if (r >= R) return;
  const int steps = K / 512;  // K % 512 == 0
  const uint16_t* xr = x + r * K + lane * 8;
  int8_t* out = xi + r * K + lane * 8;
  auto absmax8 = [](float m, const uint4 q) {
    const uint32_t v[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) m = fmaxf(m, fmaxf(fabsf(bf16lo(v[j])), fabsf(bf16hi(v[j]))));
    return m;
  };
  uint4 kept[kQuantRegElems / 8];
  float amax = 0.f;
  if (steps <= kQuantRegElems / 8) {  // wave-uniform: static register indices, all loads in flight together
#pragma unroll
    for (int t = 0; t < kQuantRegElems / 8; ++t)
      if (t < steps) kept[t] = *reinterpret_cast<const uint4*>(xr + 512 * t);
#pragma unroll
    for (int t = 0; t < kQuantRegElems / 8; ++t)
      if (t < steps) amax = absmax8(amax, kept[t]);
  } else {
    for (int t = 0; t < steps; ++t) amax = absmax8(amax, *reinterpret_cast<const uint4*>(xr + 512 * t));
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) amax = fmaxf(amax, __shfl_xor(amax, m, 64));
  const float sc = __fdiv_rn(amax, 127.0f);
  if (lane == 0) sx[r] = sc;
  if (steps <= kQuantRegElems / 8) {
#pragma unroll
    for (int t = 0; t < kQuantRegElems / 8; ++t)
      if (t < steps) *reinterpret_cast<uint2*>(out + 512 * t) = quant_pack(kept[t], sc);
  } else {
    for (int t = 0; t < steps; ++t)
      *reinterpret_cast<uint2*>(out + 512 * t) = quant_pack(*reinterpret_cast<const uint4*>(xr + 512 * t), sc);
  }
}

// ---------------------------------------------------------------- GEMM
//
// Work unit: one (128-row tile, 256-column block).  A block has sixteen waves,
// four per SIMD at no more than 128 VGPRs each: wave w owns the 32 columns of
// column group cw = w % 8 and the 16-row subtiles of parity rh = w / 8 (rh,
// rh + 2, ...), so both parities have rows on a short tile.  Persistent
// blocks, one per CU, take units heavy-first (gemm_common.h).  Per 64-wide K
// group g every operand byte reaches LDS through asynchronous copies into a
// ring of kStages stages:
//   A  the tile's int8 activation rows, 128 x 64 bytes, gathered through
//      x_rows, 16-byte unit u of row r stored at u ^ aswz(r); the parity-1
//      wave of column group cw copies rows 16cw .. +15;
//   B  column group cw's packed codes (tile layout: half a 2 KiB chunk; MLX
//      layout: 16 bytes per lane from the column's row), copied by its
//      parity-0 wave;
//   S  the scales of the 64-column block holding those columns (with the
//      biases in the tile layout's scale|bias words), copied by the same
//      wave; the bias term reads the biases once per tile, after the loop.
// After the barrier that publishes group g, a wave turns its code words into
// int8 with byte permutes (codes 0..15 are valid int8: no zero point), runs
// one v_mfma_i32_16x16x64_i8 per 16 x 16 subtile (D_g exact in int32) and
// folds acc += s * D_g in fp32; the parity-1 wave of column group cw also
// takes subtile cw's exact row sums R_g with v_dot4 and keeps them in LDS as
// int16 (|R_g| <= 64 * 127).  After the last group the bias term
// sum_g b[n,g] R_g[m] is a small bf16 MFMA product per subtile (R split into
// exact bf16 hi + lo), the rows are scaled by sx and the tile leaves through
// LDS as 512-byte row segments.
//
// K order inside a group is free as long as both operands agree: lane
// quarter qq of the 16 x 16 x 64 MFMA supplies group elements 16qq .. +15 of
// its row and of its column (tile_loop_i8).

using namespace qmoe_gemm;

constexpr int kBM = kTileRows;  // 128
constexpr int kWaves = 16;       // four per SIMD: the others' rescale fills one wave's waits
constexpr int kCols = 32;        // columns per wave
constexpr int kColGroups = 8;    // column groups per block; two waves (row parities) each
constexpr int kBN = kCols * kColGroups;
constexpr int kI8Threads = 64 * kWaves;
// Ring depth: the copies of group g + kStages - 1 go out during group g, so
// kStages - 2 groups of copies stay in flight past the one waited for.
#ifndef QMOE_I8_STAGES
#define QMOE_I8_STAGES 3
#endif
constexpr int kStages = QMOE_I8_STAGES;
static_assert(kStages >= 3, "the ring needs a stage being read, one landing and one in flight");
constexpr int kMaxG = 64;  // K <= 4096
constexpr int kI8BlocksPerCU = 1;
// Row sums R_g[row] live in LDS as int16 [group][kRStride]: consecutive rows
// are consecutive halves (conflict-free for the lanes of one group), and the
// pad shifts successive groups by one bank.
constexpr int kRStride = kTileRows + 2;

// Stage layout: A rows; B one 1 KiB code copy per column group (its 32
// columns); S the scale|bias words (tile layout) or the scale pairs of two
// consecutive groups (MLX layout) of the 64-column block holding the group's
// columns, one 256-byte copy each.
template <bool TILED>
struct ICfg {
  static constexpr int kAOff = 0;
  static constexpr int kABytes = kBM * 64;
  static constexpr int kBOff = kAOff + kABytes;
  static constexpr int kBBytes = kColGroups * 1024;
  static constexpr int kSOff = kBOff + kBBytes;
  static constexpr int kSBytes = kColGroups * 64 * 4;
  static constexpr int kStageBytes = kSOff + kSBytes;
  static constexpr int kRingBytes = kStages * kStageBytes;
  static constexpr int kRBytes = kRStride * kMaxG * 2;  // int16 row sums [group][row]
  static constexpr int kSxOff = kRingBytes + kRBytes;  // sx of the tile's rows
  // tile layout: the bias halves of the scale|bias words, saved as the groups
  // stream past, bf16 [column group][group][32 columns], for the bias term
  static constexpr int kBiasOff = kSxOff + kBM * 4;
  static constexpr int kBiasBytes = TILED ? kColGroups * kMaxG * 32 * 2 : 0;
  static constexpr int kLdsBytes = kBiasOff + kBiasBytes;
  static_assert(kI8BlocksPerCU * (kLdsBytes + 4 * kMaxOrder) <= 160 * 1024, "LDS per CU");
  static_assert(kRingBytes >= 64 * 512, "the epilogue stages 64 rows of 512 bytes in the ring");
  static_assert(kABytes == kColGroups * 1024, "one 1 KiB activation copy per parity-1 wave");
  static constexpr int kCopies0 = 2;  // a parity-0 wave's copies per group: B and S
  static constexpr int kCopies1 = 1;  // a parity-1 wave's: A
};

struct Int8Args {
  const int8_t* xi;
  const float* sx;
  const int32_t* x_rows;
  int64_t n_rows;
  int K;
  const uint32_t* w;   // MLX codes, or tile-layout codes
  const uint16_t* s;   // MLX scales (null for the tile layout)
  const uint16_t* b;   // MLX biases
  const uint32_t* sb;  // tile layout: scale|bias words
  int num_experts;
  int N;
  const int32_t* offsets;
  const int32_t* tile_row;
  const int32_t* tile_exp;
  const int32_t* ntiles;
  uint16_t* out;
};

template <bool TILED>
struct ICtx {
  const char* a_src;  // parity 1: the lane's activation 16-byte unit, group 0
  const char* b_src;  // parity 0: codes and scales of group 0
  const char* s_src;
  uint32_t lds;
  int G;
  int rh, cw, lane;  // row parity and column group: wave-uniform
  int tsub;          // the tile's 32-row subtiles
};

// 16 codes (two words, k order 0..15) -> 16 int8 in natural k order.
__device__ __forceinline__ i32x4_t codes_to_i8(uint32_t wa, uint32_t wb) {
  const uint32_t la = wa & 0x0F0F0F0Fu, ha = (wa >> 4) & 0x0F0F0F0Fu;
  const uint32_t lb = wb & 0x0F0F0F0Fu, hb = (wb >> 4) & 0x0F0F0F0Fu;
  i32x4_t r;
  r[0] = (int)__builtin_amdgcn_perm(ha, la, 0x05010400u);
  r[1] = (int)__builtin_amdgcn_perm(ha, la, 0x07030602u);
  r[2] = (int)__builtin_amdgcn_perm(hb, lb, 0x05010400u);
  r[3] = (int)__builtin_amdgcn_perm(hb, lb, 0x07030602u);
  return r;
}

// This wave's copies of group g into its ring stage.
template <bool TILED>
__device__ __forceinline__ void issue_group(const ICtx<TILED>& c, int g) {
  using C = ICfg<TILED>;
  const uint32_t st = c.lds + (uint32_t)(g % kStages) * C::kStageBytes;
  if (c.rh) {
    dma16(c.a_src + (size_t)g * 64, st + C::kAOff + (uint32_t)c.cw * 1024);
    return;
  }
  if constexpr (TILED) {
    dma16(c.b_src + (size_t)g * 2048, st + C::kBOff + (uint32_t)c.cw * 1024);
    dma4(c.s_src + (size_t)g * 256, st + C::kSOff + c.cw * 256);
  } else {
    dma16(c.b_src + (size_t)g * 32, st + C::kBOff + (uint32_t)c.cw * 1024);
    dma4(c.s_src + (size_t)(g >> 1) * 4, st + C::kSOff + c.cw * 256);
  }
}

// Wait until this wave's copies of the oldest group still in flight have
// landed (the kStages - 2 newer groups may stay outstanding).
template <bool TILED>
__device__ __forceinline__ void wait_oldest(const ICtx<TILED>& c) {
  if (c.rh) wait_vmem<(kStages - 2) * ICfg<TILED>::kCopies1>();
  else wait_vmem<(kStages - 2) * ICfg<TILED>::kCopies0>();
}

typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4_t;

// Accumulators of a wave: its 32 columns as two 16-column subtiles jj and its
// up to four 16-row subtiles j (tile subtile 2j + rh); D[m][n] of a 16 x 16
// MFMA tile sits in lane n (mod 16), register r at row 4 * (lane / 16) + r.
constexpr int kJJ = kCols / 16;
typedef f32x4_t Acc[kMaxSub][kJJ];

// Row swizzle of the 16-byte units of a 64-byte activation row in LDS: unit
// u of row r is stored at u ^ aswz(r).  A 16-byte read by a 16 x 16 x 64
// fragment has lane quarter qq read unit qq of rows r0 .. r0 + 15.  gfx950
// serves such a read 32 consecutive lanes (two quarters, 512 bytes) at a
// time, so rows r and r + 8, whose units share bank positions, must use
// different unit pairs: aswz(r + 8) = aswz(r) ^ 3.  Within rows 0..7 the
// units of equal row parity differ, which also keeps 8- and 16-lane passes
// conflict-free.  aswz(16 i + l) = aswz(l).
__device__ __forceinline__ int aswz(int row) { return ((row >> 1) & 3) ^ (3 * ((row >> 3) & 1)); }

// The weight-side operands of one group: int8 code fragments and the scales
// of the wave's two 16-column subtiles.
struct BState {
  i32x4_t bq[kJJ];
  float sc[kJJ];
  uint32_t bias[kJJ];  // tile layout: the columns' bias bits (bf16)
};

template <bool TILED>
__device__ __forceinline__ BState load_bstate(const ICtx<TILED>& c, const char* st, int g) {
  using C = ICfg<TILED>;
  const int l16 = c.lane & 15, qq = c.lane >> 4;
  BState b;
#pragma unroll
  for (int jj = 0; jj < kJJ; ++jj) {
    const int cc = 16 * jj + l16;  // column within the group's 32
    const uint2 wd = *reinterpret_cast<const uint2*>(st + C::kBOff + c.cw * 1024 + ((qq >> 1) * 32 + cc) * 16 +
                                                     (qq & 1) * 8);
    b.bq[jj] = codes_to_i8(wd.x, wd.y);
    const int sc_i = 32 * (c.cw & 1) + cc;  // the column within its 64-column block
    if constexpr (TILED) {
      const uint32_t* sw = reinterpret_cast<const uint32_t*>(st + C::kSOff + c.cw * 256);
      b.sc[jj] = __uint_as_float(sw[sc_i] << 16);
      b.bias[jj] = sw[sc_i] >> 16;
    } else {
      const uint32_t* sw = reinterpret_cast<const uint32_t*>(st + C::kSOff + c.cw * 256);
      b.sc[jj] = __uint_as_float((sw[sc_i] << ((g & 1) ? 0 : 16)) & 0xFFFF0000u);
      b.bias[jj] = 0u;  // the MLX layout's biases are read by the bias term itself
    }
  }
  return b;
}

// One group's MFMAs and rescales for the wave's MSUB (>= 1) subtiles, with
// the copies of group g + kStages - 1 issued after the first subtile's MFMAs.
template <bool TILED, int MSUB>
__device__ __forceinline__ void group_i8(const ICtx<TILED>& c, char* smem, const char* st, int g, int aoff, Acc& acc) {
  using C = ICfg<TILED>;
  const int G = c.G;
  const int l16 = c.lane & 15, qq = c.lane >> 4;
  const BState bs = load_bstate<TILED>(c, st, g);
  if constexpr (TILED) {
    // the parity-0 wave keeps its columns' biases of group g for the bias term
    if (!c.rh && qq == 0) {
      uint16_t* bl = reinterpret_cast<uint16_t*>(smem + C::kBiasOff) + (c.cw * kMaxG + g) * 32;
#pragma unroll
      for (int jj = 0; jj < kJJ; ++jj) bl[16 * jj + l16] = (uint16_t)bs.bias[jj];
    }
  }
  const char* abuf = st + C::kAOff + aoff;
  i32x4_t dc[kJJ], dn[kJJ];
  {
    const i32x4_t af = *reinterpret_cast<const i32x4_t*>(abuf);
#pragma unroll
    for (int jj = 0; jj < kJJ; ++jj) {
      const i32x4_t z = {};
      dc[jj] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af, bs.bq[jj], z, 0, 0, 0);
    }
  }
  issue_group<TILED>(c, min(g + kStages - 1, G - 1));
#pragma unroll
  for (int j = 0; j < MSUB; ++j) {
    if (j + 1 < MSUB) {
      const i32x4_t af = *reinterpret_cast<const i32x4_t*>(abuf + (j + 1) * 32 * 64);
#pragma unroll
      for (int jj = 0; jj < kJJ; ++jj) {
        const i32x4_t z = {};
        dn[jj] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af, bs.bq[jj], z, 0, 0, 0);
      }
    }
#pragma unroll
    for (int jj = 0; jj < kJJ; ++jj) {
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[j][jj][r] = __builtin_fmaf(bs.sc[jj], (float)dc[jj][r], acc[j][jj][r]);
      // keep the rescale here, between this subtile's and the next one's
      // MFMAs, rather than sunk to the end of the group
      asm volatile("" : "+v"(acc[j][jj]));
    }
#pragma unroll
    for (int jj = 0; jj < kJJ; ++jj) dc[jj] = dn[jj];
  }
}

// Main loop over the groups of one tile: the wave has MSUB 16-row subtiles
// holding valid rows (tile subtiles 2j + rh, j < MSUB; a parity-1 wave has
// one fewer when the tile's last 32 rows hold 16 or fewer, none on a tile of
// at most 16 rows, and still copies, waits and sums rows).  Per group and
// 16 x 16 subtile one v_mfma_i32_16x16x64_i8 covers the whole group; lane
// quarter qq supplies group elements 16qq .. +15 of its row (A: unit qq of the
// activation row) and of its column (B: code words 2(qq%2), +1 of the chunk
// lane (qq/2, column % 32)).  The MFMAs of subtile j + 1 are issued before
// subtile j is rescaled, so the matrix core and the vector unit overlap; the
// copies of group g + kStages - 1 go out after the first subtile's MFMAs.
template <bool TILED, int MSUB>
__device__ __forceinline__ void tile_loop_i8(const ICtx<TILED>& c, char* smem, Acc& acc) {
  using C = ICfg<TILED>;
  const int G = c.G;
  const int l16 = c.lane & 15, qq = c.lane >> 4;
  const int unit_off = l16 * 64 + ((qq ^ aswz(l16)) * 16);  // the lane's A unit within a subtile
  const int aoff = 16 * c.rh * 64 + unit_off;                // ... within the wave's first subtile
  int16_t* rsum = reinterpret_cast<int16_t*>(smem + C::kRingBytes);
#pragma unroll
  for (int p = 0; p < kStages - 1; ++p) issue_group<TILED>(c, min(p, G - 1));
  wait_oldest<TILED>(c);  // this wave's copies of group 0
  for (int g = 0; g < G; ++g) {
    // every wave's copies of group g have landed, and every wave is done with
    // the stage that group g + kStages - 1 overwrites
    __builtin_amdgcn_s_barrier();
    const char* st = smem + (g % kStages) * C::kStageBytes;
    if constexpr (MSUB == 0) issue_group<TILED>(c, min(g + kStages - 1, G - 1));
    else group_i8<TILED, MSUB>(c, smem, st, g, aoff, acc);
    // exact row sums of the group: the parity-1 wave of column group cw takes
    // tile subtile cw (16 int8 per lane, four lane quarters per row)
    if (c.rh && c.cw < 2 * c.tsub) {
      const i32x4_t af = *reinterpret_cast<const i32x4_t*>(st + C::kAOff + c.cw * 16 * 64 + unit_off);
      int part = 0;
#pragma unroll
      for (int t = 0; t < 4; ++t) part = __builtin_amdgcn_sdot4(af[t], 0x01010101, part, false);
      part += __shfl_xor(part, 16, 64);
      part += __shfl_xor(part, 32, 64);
      if (qq == 0) rsum[g * kRStride + 16 * c.cw + l16] = (int16_t)part;
    }
    wait_oldest<TILED>(c);  // this wave's copies of group g + 1
  }
  wait_vmem<0>();  // the trailing repeat copies
}

// Bias term: acc += R (rows x groups) . b^T (groups x columns), bf16 MFMA
// with R = hi + lo exact in bf16; then rows scaled by sx and stored.
template <bool TILED>
__device__ __forceinline__ void finish_tile(const Int8Args& a, char* smem, const ICtx<TILED>& c, Acc& acc, int e,
                                            int64_t row0, int valid, int msub, int nblk) {
  using C = ICfg<TILED>;
  const int G = c.G;
  const int l16 = c.lane & 15, qq = c.lane >> 4;
  const int16_t* rsum = reinterpret_cast<const int16_t*>(smem + C::kRingBytes);
  const float* sxl = reinterpret_cast<const float*>(smem + C::kRingBytes + C::kRBytes);
  const int col0 = nblk * kBN + c.cw * kCols;
  for (int g0 = 0; g0 < G; g0 += 32) {
    // lane quarter qq supplies groups g0 + 8qq .. +7
    i32x4_t bz[kJJ];
#pragma unroll
    for (int jj = 0; jj < kJJ; ++jj) {
      const int n = col0 + 16 * jj + l16;
      uint32_t v[8];
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        const int g = g0 + 8 * qq + t;
        uint32_t bits = 0;
        if (g < G) {
          if constexpr (TILED) {
            bits = reinterpret_cast<const uint16_t*>(smem + C::kBiasOff)[(c.cw * kMaxG + g) * 32 + (n - col0)];
          } else {
            bits = a.b[((int64_t)e * a.N + n) * G + g];
          }
        }
        v[t] = bits;
      }
      bz[jj] = i32x4_t{(int)(v[0] | (v[1] << 16)), (int)(v[2] | (v[3] << 16)), (int)(v[4] | (v[5] << 16)),
                       (int)(v[6] | (v[7] << 16))};
    }
#pragma unroll
    for (int j = 0; j < kMaxSub; ++j) {
      if (j >= msub) break;
      const int i = 2 * j + c.rh;  // tile subtile
      uint32_t hi[4], lo[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        float f[2];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const int g = g0 + 8 * qq + 2 * t + u;
          f[u] = g < G ? (float)rsum[g * kRStride + 16 * i + l16] : 0.f;
        }
        const uint32_t hb = cvt_pk_bf16(f[0], f[1]);  // |R| < 2^13: hi = bf16(R), lo = R - hi exact
        hi[t] = hb;
        lo[t] = cvt_pk_bf16(f[0] - bf16lo(hb), f[1] - bf16hi(hb));
      }
      const i32x4_t ah = {(int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
      const i32x4_t al = {(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3]};
#pragma unroll
      for (int jj = 0; jj < kJJ; ++jj) {
        acc[j][jj] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, ah),
                                                             __builtin_bit_cast(bf16x8_t, bz[jj]), acc[j][jj], 0, 0, 0);
        acc[j][jj] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, al),
                                                             __builtin_bit_cast(bf16x8_t, bz[jj]), acc[j][jj], 0, 0, 0);
      }
    }
  }
  // out = sx * acc through LDS, 64 rows (tile subtiles 4p .. 4p + 3) per
  // pass.  Lane (qq, 4a + k) holds column 4a + k of rows 4qq .. 4qq + 3 of a
  // 16 x 16 subtile; two quad-lane exchanges give it row 4qq + k of columns
  // 4a .. 4a + 3 as two bf16 pairs, one 8-byte granule.  Staging row m holds
  // the block's 256 columns (512 bytes), granule gi at gi ^ 4 (m & 7), so the
  // granule writes of 32 lanes (8 rows x 4 granules) and the 16-byte row
  // reads below (unit u at u ^ 2 (m & 7)) are conflict-free.
  char* ep = smem;
  const int tid = threadIdx.x;
  const int k = c.lane & 3, a4 = l16 >> 2;
  // stage-1 byte selectors: lane parity 0 keeps its low halves, 1 its high
  const uint32_t sel1 = (k & 1) ? 0x03020706u : 0x05040100u;
  const bool hiq = (k & 2) != 0;
  uint16_t* obase = a.out + row0 * (int64_t)a.N + nblk * kBN;
  for (int p = 0; 2 * p < msub; ++p) {
    __syncthreads();
#pragma unroll
    for (int j = 0; j < kMaxSub; ++j) {
      if ((j >> 1) != p) continue;  // tile subtile 2j + rh lies in rows 64p .. 64p + 63
      const int i = 2 * j + c.rh;
      const float4 sc4 = *reinterpret_cast<const float4*>(sxl + 16 * i + 4 * qq);  // rows 16i + 4qq .. +3
      const int m = 16 * i + 4 * qq + k - 64 * p;  // the lane's row within the pass after the exchange
#pragma unroll
      for (int jj = 0; jj < kJJ; ++jj) {
        // own column: rows (0, 1) and (2, 3) as bf16 pairs
        const uint32_t p0 = cvt_pk_bf16(sc4.x * acc[j][jj][0], sc4.y * acc[j][jj][1]);
        const uint32_t p1 = cvt_pk_bf16(sc4.z * acc[j][jj][2], sc4.w * acc[j][jj][3]);
        // with lane k ^ 1: rows 2t + (k & 1) of columns (k & 2, (k & 2) + 1)
        const uint32_t q0 = __builtin_amdgcn_update_dpp(0u, p0, 0xB1, 0xf, 0xf, false);  // quad_perm 1,0,3,2
        const uint32_t q1 = __builtin_amdgcn_update_dpp(0u, p1, 0xB1, 0xf, 0xf, false);
        const uint32_t a0 = __builtin_amdgcn_perm(q0, p0, sel1);
        const uint32_t a1 = __builtin_amdgcn_perm(q1, p1, sel1);
        // with lane k ^ 2: row k of column pairs 0 and 1
        const uint32_t keep = hiq ? a1 : a0;
        const uint32_t recv = __builtin_amdgcn_update_dpp(0u, hiq ? a0 : a1, 0x4E, 0xf, 0xf, false);  // 2,3,0,1
        const int gi = c.cw * 8 + 4 * jj + a4;  // granule of columns 4a .. 4a + 3 within the block's row
        *reinterpret_cast<uint2*>(ep + m * 512 + ((gi ^ (4 * (m & 7))) * 8)) =
            hiq ? make_uint2(recv, keep) : make_uint2(keep, recv);
      }
    }
    __syncthreads();
#pragma unroll
    for (int it = 0; it < 64 * 32 / kI8Threads; ++it) {
      const int m = it * (kI8Threads / 32) + tid / 32;
      const int u = tid % 32;
      const int row = 64 * p + m;
      const uint4 v = *reinterpret_cast<const uint4*>(ep + m * 512 + ((u ^ (2 * (m & 7))) * 16));
      if (row < valid) {  // non-temporal: written once, read (if at all) by a later launch
        const i32x4_t t = {(int)v.x, (int)v.y, (int)v.z, (int)v.w};
        __builtin_nontemporal_store(t, reinterpret_cast<i32x4_t*>(obase + (int64_t)row * a.N + u * 8));
      }
    }
  }
}

template <bool TILED>
__device__ __forceinline__ void run_unit_i8(const Int8Args& a, char* smem, int tile, int nblk) {
  using C = ICfg<TILED>;
  const TileRows tr = tile_rows_of(Tiles{a.offsets, a.tile_row, a.tile_exp, a.ntiles, a.n_rows, a.num_experts}, tile);
  if (tr.valid <= 0) return;
  const int e = tr.e, valid = tr.valid;
  const int64_t row0 = tr.row0;
  const int msub = (valid + 31) / 32;
  const int K = a.K;
  const int G = K / 64;
  const int tid = threadIdx.x;

  ICtx<TILED> c;
  c.G = G;
  const int wave = __builtin_amdgcn_readfirstlane(tid / 64);
  c.rh = wave / kColGroups;
  c.cw = wave % kColGroups;
  c.lane = tid % 64;
  c.lds = (uint32_t)(uintptr_t)smem;
  c.a_src = c.b_src = c.s_src = nullptr;
  float* sxl = reinterpret_cast<float*>(smem + C::kRingBytes + C::kRBytes);
  if (c.rh) {
    // The copy writes stage bytes cw * 1024 + lane * 16: row 16 cw + lane / 4,
    // stored unit lane % 4 holding logical unit (lane % 4) ^ aswz(row).  Rows
    // past the tile repeat its last row.
    const int row = 16 * c.cw + (c.lane >> 2);
    const int unit = (c.lane & 3) ^ aswz(row);
    int64_t src = row0 + min(row, valid - 1);
    if (a.x_rows) src = a.x_rows[src];
    c.a_src = reinterpret_cast<const char*>(a.xi + src * K + unit * 16);
  } else {
    // the group's 32 columns: half (cw & 1) of the 64-column block nblk * 4 + cw / 2
    const int c64 = nblk * (kBN / 64) + c.cw / 2;
    if constexpr (TILED) {
      const int64_t chunk0 = ((int64_t)e * (a.N / 64) + c64) * G;
      c.b_src = reinterpret_cast<const char*>(a.w) + (chunk0 * 2 + (c.cw & 1)) * 1024 + c.lane * 16;
      c.s_src = reinterpret_cast<const char*>(a.sb) + chunk0 * 256 + c.lane * 4;
    } else {
      const int64_t KW = K / 8;
      const int64_t col64 = (int64_t)e * a.N + c64 * 64;
      c.b_src = reinterpret_cast<const char*>(a.w + (col64 + 32 * (c.cw & 1) + c.lane % 32) * KW + (c.lane / 32) * 4);
      c.s_src = reinterpret_cast<const char*>(a.s + (col64 + c.lane) * G);
    }
  }
  if (tid < kBM) {
    int64_t src = row0 + min(tid, valid - 1);
    if (a.x_rows) src = a.x_rows[src];
    sxl[tid] = a.sx[src];
  }

  Acc acc;
#pragma unroll
  for (int i = 0; i < kMaxSub; ++i)
#pragma unroll
    for (int j = 0; j < kJJ; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[i][j][r] = 0.f;

  // the wave's 16-row subtiles that hold valid rows: rows 32j + 16rh .. +15
  c.tsub = msub;
  const int nsub = (valid - 16 * c.rh + 31) / 32;  // wave-uniform, 0 only for parity 1
  switch (nsub) {
    case 0: tile_loop_i8<TILED, 0>(c, smem, acc); break;
    case 1: tile_loop_i8<TILED, 1>(c, smem, acc); break;
    case 2: tile_loop_i8<TILED, 2>(c, smem, acc); break;
    case 3: tile_loop_i8<TILED, 3>(c, smem, acc); break;
    default: tile_loop_i8<TILED, 4>(c, smem, acc); break;
  }
  static_assert(kMaxSub == 4, "tile_loop_i8 is instantiated for 0..4 subtiles per parity");
  __syncthreads();  // row sums and sx visible to every wave; the ring is free
  finish_tile<TILED>(a, smem, c, acc, e, row0, valid, msub, nblk);
}

// The second bound is the minimum number of waves per SIMD.
template <bool TILED>
__global__ __launch_bounds__(kI8Threads, kI8BlocksPerCU * kWaves / 4) void gemm_int8_kernel(Int8Args a) {
  using C = ICfg<TILED>;
  __shared__ __attribute__((aligned(1024))) char smem[C::kLdsBytes];
  __shared__ int order[kMaxOrder];

  const Tiles tt{a.offsets, a.tile_row, a.tile_exp, a.ntiles, a.n_rows, a.num_experts};
  const int NB = a.N / kBN;
  const int ntiles = a.ntiles[0];
  const Snake sn((int64_t)ntiles * NB);
  if (sn.unit(0) < 0) return;
  const bool sorted = ntiles <= kMaxOrder;
  if (sorted) rank_tiles(tt, ntiles, order, reinterpret_cast<int*>(smem));
  for (int64_t k = 0;; ++k) {
    const int64_t u = sn.unit(k);
    if (u < 0) break;
    const int rank = (int)(u / NB);
    __syncthreads();  // every wave is done with the ring and the row sums
    run_unit_i8<TILED>(a, smem, sorted ? order[rank] : rank, (int)(u % NB));
  }
}

int launch_int8(const Int8Args& a, int64_t max_tiles, void* stream) {
  const dim3 grid((unsigned)grid_blocks(max_tiles * (a.N / kBN), kI8BlocksPerCU));
  hipStream_t st = qmoe::as_stream(stream);
  if (a.sb) gemm_int8_kernel<true><<<grid, dim3(kI8Threads), 0, st>>>(a);
  else gemm_int8_kernel<false><<<grid, dim3(kI8Threads), 0, st>>>(a);
  return qmoe::launch_status("gemm_int8_kernel");
}

int check_int8(const int8_t* xi, const float* sx, int64_t n_rows, int64_t K, int32_t num_experts, int64_t N,
               const int32_t* offsets, const int32_t* tile_row, const int32_t* tile_exp, const int32_t* ntiles,
               int64_t max_tiles, const uint16_t* out) {
  if (n_rows < 0 || K <= 0 || N <= 0 || num_experts <= 0 || max_tiles < 0)
    return qmoe::fail(QMOE_ERR_INVALID, "bad sizes");
  if (n_rows == 0 || max_tiles == 0) return QMOE_OK;
  if (!xi || !sx || !offsets || !tile_row || !tile_exp || !ntiles || !out)
    return qmoe::fail(QMOE_ERR_INVALID, "null pointer");
  if (K % 64 || K > 64 * kMaxG)
    return qmoe::fail(QMOE_ERR_UNSUPPORTED, "K=%lld: must be a multiple of 64, at most %d", (long long)K, 64 * kMaxG);
  if (N % kBN) return qmoe::fail(QMOE_ERR_UNSUPPORTED, "N=%lld: must be a multiple of %d", (long long)N, kBN);
  if (!qmoe::aligned16(xi) || !qmoe::aligned16(out)) return qmoe::fail(QMOE_ERR_UNSUPPORTED, "xi and out must be 16-byte aligned");
  if (N > 0x7FFFFFFF || n_rows > 0x7FFFFFFF) return qmoe::fail(QMOE_ERR_UNSUPPORTED, "sizes too large");
  return QMOE_OK;
}

}  // namespace

extern "C" int qmoe_quantize_act_int8(const uint16_t* x, int64_t R, int64_t K, int8_t* xi, float* sx,
                                      void* stream) {
  if (R < 0 || K <= 0) return qmoe::fail(QMOE_ERR_INVALID, "bad sizes");
  if (R == 0) return QMOE_OK;
  if (!x || !xi || !sx) return qmoe::fail(QMOE_ERR_INVALID, "null pointer");
  if (K % 512) return qmoe::fail(QMOE_ERR_UNSUPPORTED, "K=%lld: must be a multiple of 512", (long long)K);
  if (K > 0x7FFFFFFF) return qmoe::fail(QMOE_ERR_UNSUPPORTED, "K too large");
  if (!qmoe::aligned16(x) || !qmoe::aligned16(xi)) return qmoe::fail(QMOE_ERR_UNSUPPORTED, "x and xi must be 16-byte aligned");
  const int64_t blocks = (R + 3) / 4;
  if (blocks > 0x7FFFFFFF) return qmoe::fail(QMOE_ERR_UNSUPPORTED, "too many rows");
  quant_act_kernel<<<dim3((unsigned)blocks), dim3(256), 0, qmoe::as_stream(stream)>>>(x, R, (int)K, xi, sx);
  return qmoe::launch_status("quant_act_kernel");
}

extern "C" int qmoe_gather_qmm_int8_sorted(const int8_t* xi, const float* sx, const int32_t* x_rows, int64_t n_rows,
                                           int64_t K, const uint32_t* w, const uint16_t* scales,
                                           const uint16_t* biases, int32_t num_experts, int64_t N, int group_size,
                                           int bits, const int32_t* offsets, const int32_t* tile_row,
                                           const int32_t* tile_exp, const int32_t* ntiles, int64_t max_tiles,
                                           uint16_t* out, void* stream) {
  const int rc = check_int8(xi, sx, n_rows, K, num_experts, N, offsets, tile_row, tile_exp, ntiles, max_tiles, out);
  if (rc != QMOE_OK || n_rows == 0 || max_tiles == 0) return rc;
  if (!w || !scales || !biases) return qmoe::fail(QMOE_ERR_INVALID, "null pointer");
  if (bits != 4 || group_size != 64)
    return qmoe::fail(QMOE_ERR_UNSUPPORTED, "int8 GEMM takes 4-bit codes with group_size 64 (got %d, %d)", bits,
                      group_size);
  // scales and biases are copied in pairs of groups
  if (K % 128) return qmoe::fail(QMOE_ERR_UNSUPPORTED, "K=%lld: must be a multiple of 128", (long long)K);
  if (!qmoe::aligned16(w) || !qmoe::aligned16(scales) || !qmoe::aligned16(biases))
    return qmoe::fail(QMOE_ERR_UNSUPPORTED, "w, scales and biases must be 16-byte aligned");
  Int8Args a{xi, sx, x_rows, n_rows, (int)K, w, scales, biases, nullptr, num_experts, (int)N, offsets, tile_row,
             tile_exp, ntiles, out};
  return launch_int8(a, max_tiles, stream);
}

extern "C" int qmoe_gather_qmm_int8_sorted_tiles(const int8_t* xi, const float* sx, const int32_t* x_rows,
                                                 int64_t n_rows, int64_t K, const uint32_t* wp, const uint32_t* sb,
                                                 int32_t num_experts, int64_t N, const int32_t* offsets,
                                                 const int32_t* tile_row, const int32_t* tile_exp,
                                                 const int32_t* ntiles, int64_t max_tiles, uint16_t* out,
                                                 void* stream) {
  const int rc = check_int8(xi, sx, n_rows, K, num_experts, N, offsets, tile_row, tile_exp, ntiles, max_tiles, out);
  if (rc != QMOE_OK || n_rows == 0 || max_tiles == 0) return rc;
  if (!wp || !sb) return qmoe::fail(QMOE_ERR_INVALID, "null pointer");
  if (!qmoe::aligned16(wp) || !qmoe::aligned16(sb))
    return qmoe::fail(QMOE_ERR_UNSUPPORTED, "wp and sb must be 16-byte aligned");
  Int8Args a{xi, sx, x_rows, n_rows, (int)K, wp, nullptr, nullptr, sb, num_experts, (int)N, offsets, tile_row,
             tile_exp, ntiles, out};
  return launch_int8(a, max_tiles, stream);
}

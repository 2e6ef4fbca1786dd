// Prefill grouped GEMM over expert-sorted rows, bf16 MFMA on gfx950.
//
// Semantics: titan/kernels/moe_gather_ws.py:20-32 -- weights dequantised to
// bf16 as bf16_rne(fmaf(q, s, b)) (:343-344), bf16 x bf16 products, fp32
// accumulation.  Work unit: one (tile, column block).  A tile is up to
// kBM = 128 consecutive sorted rows of one expert (the tile list of the
// routing step); a column block is 64 * W output columns, one 64-column
// slice for each of the block's W waves (W = 8 when N is a multiple of 512,
// else 4).  Wide column blocks matter: the activation rows of a tile are
// fetched once per column block, and that re-fetch, not arithmetic, is the
// limit at 256 columns.
//
// Data movement: every operand byte reaches LDS through asynchronous copies
// (global_load_lds_dwordx4 / _dword, issued from inline assembly so that the
// copies stay in flight across iterations; the wait counts are explicit).  A
// ring of kStages stages each holds one 64-wide K group (one quantisation
// group):
//   A  the tile's activation rows, gathered through x_rows, 128 x 128 bytes,
//      16-byte units XOR-swizzled by row (swz) so MFMA operand reads are
//      bank-conflict free;
//   B  each wave's 64 columns of packed codes (16 bytes per lane and column
//      subtile: the lane's own half group);
//   S  the 64 columns' scales and biases.
// Per group a wave dequantises its own codes in registers into the MFMA B
// operand (columns are wave-private, so no dequant work is repeated) and runs
// four k-steps of v_mfma_f32_32x32x16_bf16 per 32 x 32 subtile.  Row subtiles
// past the tile's valid rows are compiled out (the loop is instantiated per
// subtile count), so a short tail tile costs only its own MFMAs.
//
// K order inside a group is free as long as A and B agree: lane half h
// supplies group elements 32h + 8kk .. +7 at k-step kk -- word kk of the
// lane's 16-byte code chunk and 16-byte unit 4h + kk of the activation row.
#include <type_traits>

#include "common.h"

namespace {

constexpr int kBM = 128;
constexpr int kABytes = kBM * 128;  // one group of the tile's activation rows: 16 KiB

// Layout and pipeline of one instantiation with W waves per block.  W = 8:
// 512 columns, a ring of 4 stages of 36 KiB, one block per CU.  W = 4: 256
// columns, 2 stages of 26 KiB, two blocks per CU.
template <int W>
struct Cfg {
  static constexpr int kWaves = W;
  static constexpr int kBN = 64 * W;
  static constexpr int kThreads = 64 * W;
  static constexpr int kStages = W == 8 ? 4 : 2;
  static constexpr int kBlocksPerCU = W == 8 ? 1 : 2;
  // stage layout (bytes)
  static constexpr int kAOff = 0;
  static constexpr int kBOff = kAOff + kABytes;
  static constexpr int kBBytes = W * 2 * 64 * 16;  // [wave][subtile][lane] x 16 B
  static constexpr int kSOff = kBOff + kBBytes;
  static constexpr int kSBytes = W * 2 * 64 * 4;  // [wave][scale|bias][lane] x 4 B
  static constexpr int kStageBytes = kSOff + kSBytes;
  static constexpr int kACopies = kABytes / (W * 1024);  // 16-byte-per-lane copies of A per wave
  static_assert(kStages * kStageBytes * kBlocksPerCU <= 160 * 1024, "LDS per CU");
  static_assert(kStages >= 2 && kStages <= 4, "wait_group covers up to two groups in flight");
};

struct GemmArgs {
  const uint16_t* x;
  const int32_t* x_rows;
  int64_t n_rows;
  int K;
  const uint32_t* w;
  const uint16_t* s;
  const uint16_t* b;
  const uint32_t* sb;  // tile layout: scale|bias words (w then holds the tile-layout codes)
  int num_experts;
  int N;
  const int32_t* offsets;
  const int32_t* tile_row;
  const int32_t* tile_exp;
  const int32_t* ntiles;
  uint16_t* out;
};

// Asynchronous 16- and 4-byte copies into LDS: lane i writes
// lds_base + i * size.  M0 carries the wave's LDS base and is restored.
__device__ __forceinline__ void dma16(const void* g, uint32_t lds_base) {
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %1\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %2, off\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "s"(lds_base), "v"(g)
      : "memory");
}
__device__ __forceinline__ void dma4(const void* g, uint32_t lds_base) {
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %1\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dword %2, off\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "s"(lds_base), "v"(g)
      : "memory");
}
template <int N>
__device__ __forceinline__ void wait_vmem() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

typedef __attribute__((__vector_size__(2 * sizeof(float)))) float f32x2_t;

__device__ __forceinline__ uint32_t cvt_pk_bf16(float a, float b) {
  f32x2_t v = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

// Byte b of v as a float: one v_cvt_f32_ubyte<b>.  Written as assembly
// because the compiler otherwise folds the preceding nibble mask into a
// bit-field extract and spends two instructions per code.
template <int B>
__device__ __forceinline__ float ubyte(uint32_t v) {
  float r;
  if constexpr (B == 0) asm("v_cvt_f32_ubyte0 %0, %1" : "=v"(r) : "v"(v));
  else if constexpr (B == 1) asm("v_cvt_f32_ubyte1 %0, %1" : "=v"(r) : "v"(v));
  else if constexpr (B == 2) asm("v_cvt_f32_ubyte2 %0, %1" : "=v"(r) : "v"(v));
  else asm("v_cvt_f32_ubyte3 %0, %1" : "=v"(r) : "v"(v));
  return r;
}

// 8 codes of one word -> 8 bf16 (k order 0..7), bf16_rne(fmaf(q, s, b)).
// lo holds codes 0,2,4,6 in its bytes, hi codes 1,3,5,7.
__device__ __forceinline__ i32x4_t dequant_word(uint32_t v, float s, float b) {
  const uint32_t lo = v & 0x0F0F0F0Fu;
  const uint32_t hi = (v >> 4) & 0x0F0F0F0Fu;
  i32x4_t r;
  r[0] = (int)cvt_pk_bf16(__builtin_fmaf(ubyte<0>(lo), s, b), __builtin_fmaf(ubyte<0>(hi), s, b));
  r[1] = (int)cvt_pk_bf16(__builtin_fmaf(ubyte<1>(lo), s, b), __builtin_fmaf(ubyte<1>(hi), s, b));
  r[2] = (int)cvt_pk_bf16(__builtin_fmaf(ubyte<2>(lo), s, b), __builtin_fmaf(ubyte<2>(hi), s, b));
  r[3] = (int)cvt_pk_bf16(__builtin_fmaf(ubyte<3>(lo), s, b), __builtin_fmaf(ubyte<3>(hi), s, b));
  return r;
}

// Row swizzle of the 16-byte units of an activation row in LDS: unit u of
// row r is stored at u ^ swz(r).  Conflict-free for b128 reads of one unit by
// consecutive rows whether the LDS serves 8 lanes per pass over 32 banks
// (swz distinct over rows r..r+7) or 16 lanes over 64 banks (swz distinct
// over the eight rows of each parity among r..r+15).
__device__ __forceinline__ int swz(int row) { return (row & 7) ^ ((row >> 3) & 1); }

// Copies per wave and group: A, two B, and the scales and biases -- two
// 4-byte copies (scale pair, bias pair) from the MLX layout, one (the
// column's scale|bias word) from the tile layout.
template <int W, bool TILED>
constexpr int kDmaPerGroup = Cfg<W>::kACopies + 2 + (TILED ? 1 : 2);

template <int W>
struct Ctx {
  // per-lane global sources at group 0 (advance per group)
  const char* a_src[Cfg<W>::kACopies];  // activation 16-byte units, one per A copy
  const char* b_src[2];  // codes of the lane's column in each subtile
  const char* s_src;     // MLX layout: scale pair (groups 2j, 2j+1) of column (wave*64 + lane);
                         // tile layout: scale|bias word of that column
  const char* z_src;     // MLX layout: bias pair
  uint32_t lds;          // LDS address of the ring
  uint32_t a_dst[Cfg<W>::kACopies];  // wave-uniform LDS offsets within a stage
  uint32_t b_dst[2];
  uint32_t s_dst, z_dst;
  int G;
  int wave, lane, l32, h;
};

template <int W, bool TILED>
__device__ __forceinline__ void issue_group(const Ctx<W>& c, int g) {
  using C = Cfg<W>;
  const uint32_t st = c.lds + (uint32_t)(g % C::kStages) * C::kStageBytes;
#pragma unroll
  for (int q = 0; q < C::kACopies; ++q) dma16(c.a_src[q] + (size_t)g * 128, st + c.a_dst[q]);
  if constexpr (TILED) {
    // one 2 KiB code chunk and one 256-byte scale|bias chunk per group
#pragma unroll
    for (int j = 0; j < 2; ++j) dma16(c.b_src[j] + (size_t)g * 2048, st + c.b_dst[j]);
    dma4(c.s_src + (size_t)g * 256, st + c.s_dst);
  } else {
#pragma unroll
    for (int j = 0; j < 2; ++j) dma16(c.b_src[j] + (size_t)g * 32, st + c.b_dst[j]);
    dma4(c.s_src + (size_t)(g >> 1) * 4, st + c.s_dst);
    dma4(c.z_src + (size_t)(g >> 1) * 4, st + c.z_dst);
  }
}

// Wait until this wave's copies of group g have landed: the copies of the
// groups issued after it (at most kStages - 2, each kDmaPerGroup copies)
// may stay in flight.
template <int D>
__device__ __forceinline__ void wait_group(int ahead) {
  if (ahead >= 2) wait_vmem<2 * D>();
  else if (ahead == 1) wait_vmem<D>();
  else wait_vmem<0>();
}

template <int W, bool TILED, int MSUB>
__device__ __forceinline__ void tile_loop(const Ctx<W>& c, const char* smem, f32x16_t (&acc)[4][2]) {
  using C = Cfg<W>;
  constexpr int kStages = C::kStages, kAOff = C::kAOff, kBOff = C::kBOff, kSOff = C::kSOff;
  const int G = c.G;
#pragma unroll
  for (int d = 0; d < kStages - 1; ++d)
    if (d < G) issue_group<W, TILED>(c, d);

  for (int g = 0; g < G; ++g) {
    wait_group<kDmaPerGroup<W, TILED>>(min(kStages - 2, G - 1 - g));
    __builtin_amdgcn_s_barrier();
    if (g + kStages - 1 < G) issue_group<W, TILED>(c, g + kStages - 1);

    const char* st = smem + (g % kStages) * C::kStageBytes;
    // this lane's codes, scales and biases for its two columns
    const uint4 raw0 = *reinterpret_cast<const uint4*>(st + kBOff + (c.wave * 2 + 0) * 1024 + c.lane * 16);
    const uint4 raw1 = *reinterpret_cast<const uint4*>(st + kBOff + (c.wave * 2 + 1) * 1024 + c.lane * 16);
    const uint32_t* sw = reinterpret_cast<const uint32_t*>(st + kSOff + c.wave * 512);
    float s0, s1, z0, z1;
    if constexpr (TILED) {
      const uint32_t v0 = sw[c.l32], v1 = sw[c.l32 + 32];
      s0 = __uint_as_float(v0 << 16);
      z0 = __uint_as_float(v0 & 0xFFFF0000u);
      s1 = __uint_as_float(v1 << 16);
      z1 = __uint_as_float(v1 & 0xFFFF0000u);
    } else {
      const int sh = (g & 1) ? 16 : 0;
      s0 = __uint_as_float((sw[c.l32] >> sh) << 16);
      s1 = __uint_as_float((sw[c.l32 + 32] >> sh) << 16);
      z0 = __uint_as_float((sw[64 + c.l32] >> sh) << 16);
      z1 = __uint_as_float((sw[64 + c.l32 + 32] >> sh) << 16);
    }
    const uint32_t w0[4] = {raw0.x, raw0.y, raw0.z, raw0.w};
    const uint32_t w1[4] = {raw1.x, raw1.y, raw1.z, raw1.w};
    const char* abuf = st + kAOff;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const i32x4_t b0 = dequant_word(w0[kk], s0, z0);
      const i32x4_t b1 = dequant_word(w1[kk], s1, z1);
      i32x4_t af[MSUB];
#pragma unroll
      for (int i = 0; i < MSUB; ++i) {
        const int row = 32 * i + c.l32;  // swz(row) == swz(l32): 32*i leaves bits 0..3 alone
        const int unit = (4 * c.h + kk) ^ swz(c.l32);
        af[i] = *reinterpret_cast<const i32x4_t*>(abuf + row * 128 + unit * 16);
      }
#pragma unroll
      for (int i = 0; i < MSUB; ++i) {
        acc[i][0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, af[i]),
                                                            __builtin_bit_cast(bf16x8_t, b0), acc[i][0], 0, 0, 0);
        acc[i][1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, af[i]),
                                                            __builtin_bit_cast(bf16x8_t, b1), acc[i][1], 0, 0, 0);
      }
    }
  }
}

template <int W, bool TILED>
__global__ __launch_bounds__(Cfg<W>::kThreads, Cfg<W>::kBlocksPerCU) void gemm_bf16_kernel(GemmArgs a) {
  using C = Cfg<W>;
  constexpr int kBN = C::kBN, kWaves = C::kWaves;
  __shared__ __attribute__((aligned(1024))) char smem[C::kStages * C::kStageBytes];

  const int NB = a.N / kBN;
  const int64_t n_active = (int64_t)a.ntiles[0] * NB;
  const int64_t hw = blockIdx.x;
  if (hw >= n_active) return;
  // XCD-aware order: hardware block ids are dealt round-robin to the 8 XCDs;
  // give each XCD a contiguous run of (tile, column block) units so the
  // tiles of one expert share that XCD's L2.
  const int64_t q8 = n_active / 8, r8 = n_active % 8, xcd = hw % 8;
  const int64_t logical = xcd * q8 + (xcd < r8 ? xcd : r8) + hw / 8;
  const int tile = (int)(logical / NB);
  const int nblk = (int)(logical % NB);

  const int e = min(max(a.tile_exp[tile], 0), a.num_experts - 1);
  const int64_t row0 = a.tile_row[tile];
  const int64_t rowend = min((int64_t)a.offsets[e + 1], a.n_rows);
  const int valid = (int)min((int64_t)kBM, rowend - row0);
  if (valid <= 0) return;
  const int msub = (valid + 31) / 32;

  const int K = a.K;
  const int G = K / 64;
  const int64_t KW = K / 8;
  const int tid = threadIdx.x;

  Ctx<W> c;
  c.G = G;
  c.wave = __builtin_amdgcn_readfirstlane(tid / 64);
  c.lane = tid % 64;
  c.l32 = c.lane % 32;
  c.h = c.lane / 32;
  c.lds = (uint32_t)(uintptr_t)smem;
  // A copies: wave w, copy q writes stage units (q*kWaves + w)*64 + lane, i.e.
  // row p/8 and stored unit p%8, which holds logical unit (p%8) ^ swz(row).
#pragma unroll
  for (int q = 0; q < C::kACopies; ++q) {
    const int p = (q * kWaves + c.wave) * 64 + c.lane;
    const int row = p >> 3;
    const int unit = (p & 7) ^ swz(row);
    int64_t src = row0 + min(row, valid - 1);
    if (a.x_rows) src = a.x_rows[src];
    c.a_src[q] = reinterpret_cast<const char*>(a.x + src * K + unit * 8);
    c.a_dst[q] = (uint32_t)(C::kAOff + (q * kWaves + c.wave) * 1024);
  }
  const int64_t col_base = (int64_t)e * a.N + nblk * kBN + c.wave * 64;
#pragma unroll
  for (int j = 0; j < 2; ++j) c.b_dst[j] = (uint32_t)(C::kBOff + (c.wave * 2 + j) * 1024);
  if constexpr (TILED) {
    // chunk (e, c, g) of the tile layout, c = the wave's 64-column block
    const int64_t chunk0 = ((int64_t)e * (a.N / 64) + nblk * kWaves + c.wave) * G;
#pragma unroll
    for (int j = 0; j < 2; ++j)
      c.b_src[j] = reinterpret_cast<const char*>(a.w) + (chunk0 * 2 + j) * 1024 + c.lane * 16;
    c.s_src = reinterpret_cast<const char*>(a.sb) + chunk0 * 256 + c.lane * 4;
    c.z_src = nullptr;
  } else {
#pragma unroll
    for (int j = 0; j < 2; ++j)
      c.b_src[j] = reinterpret_cast<const char*>(a.w + (col_base + j * 32 + c.l32) * KW + c.h * 4);
    c.s_src = reinterpret_cast<const char*>(a.s + (col_base + c.lane) * G);
    c.z_src = reinterpret_cast<const char*>(a.b + (col_base + c.lane) * G);
  }
  c.s_dst = (uint32_t)(C::kSOff + c.wave * 512);
  c.z_dst = c.s_dst + 256;

  f32x16_t acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  switch (msub) {
    case 1: tile_loop<W, TILED, 1>(c, smem, acc); break;
    case 2: tile_loop<W, TILED, 2>(c, smem, acc); break;
    case 3: tile_loop<W, TILED, 3>(c, smem, acc); break;
    default: tile_loop<W, TILED, 4>(c, smem, acc); break;
  }

  // epilogue: D[m][n] of a 32x32 subtile sits in lane n (mod 32), register
  // r at row 8*(r/4) + 4*(lane/32) + r%4.
  const int ncol = nblk * kBN + c.wave * 64 + c.l32;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if (i >= msub) continue;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int m = 32 * i + 8 * (r / 4) + 4 * c.h + (r % 4);
      if (m < valid) {
        uint16_t* orow = a.out + (row0 + m) * (int64_t)a.N + ncol;
        orow[0] = (uint16_t)f32_to_bf16(acc[i][0][r]);
        orow[32] = (uint16_t)f32_to_bf16(acc[i][1][r]);
      }
    }
  }
}

}  // namespace

extern "C" int qmoe_gemm_tile_rows(void) { return kBM; }

namespace {

int launch_gemm(const GemmArgs& a, int64_t max_tiles, bool tiled, void* stream) {
  const bool wide = a.N % Cfg<8>::kBN == 0;
  const int64_t blocks = max_tiles * (a.N / (wide ? Cfg<8>::kBN : Cfg<4>::kBN));
  if (blocks > 0x7FFFFFFF) return qmoe::fail(QMOE_ERR_UNSUPPORTED, "grid too large");
  const dim3 grid((unsigned)blocks);
  hipStream_t st = qmoe::as_stream(stream);
  if (wide && tiled) gemm_bf16_kernel<8, true><<<grid, dim3(Cfg<8>::kThreads), 0, st>>>(a);
  else if (wide) gemm_bf16_kernel<8, false><<<grid, dim3(Cfg<8>::kThreads), 0, st>>>(a);
  else if (tiled) gemm_bf16_kernel<4, true><<<grid, dim3(Cfg<4>::kThreads), 0, st>>>(a);
  else gemm_bf16_kernel<4, false><<<grid, dim3(Cfg<4>::kThreads), 0, st>>>(a);
  return qmoe::launch_status("gemm_bf16_kernel");
}

int check_common(const uint16_t* x, int64_t n_rows, int64_t K, int32_t num_experts, int64_t N,
                 const int32_t* offsets, const int32_t* tile_row, const int32_t* tile_exp, const int32_t* ntiles,
                 int64_t max_tiles, const uint16_t* out) {
  if (n_rows < 0 || K <= 0 || N <= 0 || num_experts <= 0 || max_tiles < 0)
    return qmoe::fail(QMOE_ERR_INVALID, "bad sizes");
  if (n_rows == 0 || max_tiles == 0) return QMOE_OK;
  if (!x || !offsets || !tile_row || !tile_exp || !ntiles || !out) return qmoe::fail(QMOE_ERR_INVALID, "null pointer");
  if (N % 256) return qmoe::fail(QMOE_ERR_UNSUPPORTED, "N=%lld: must be a multiple of 256", (long long)N);
  if (!qmoe::aligned16(x)) return qmoe::fail(QMOE_ERR_UNSUPPORTED, "x must be 16-byte aligned");
  if (K > 0x7FFFFFFF || N > 0x7FFFFFFF || n_rows > 0x7FFFFFFF)
    return qmoe::fail(QMOE_ERR_UNSUPPORTED, "sizes too large");
  return QMOE_OK;
}

}  // namespace

extern "C" int qmoe_gather_qmm_sorted(const uint16_t* x, const int32_t* x_rows, int64_t n_rows, int64_t K,
                                      const uint32_t* w, const uint16_t* scales, const uint16_t* biases,
                                      int32_t num_experts, int64_t N, int group_size, int bits,
                                      const int32_t* offsets, const int32_t* tile_row,
                                      const int32_t* tile_exp, const int32_t* ntiles, int64_t max_tiles,
                                      uint16_t* out, void* stream) {
  const int rc = check_common(x, n_rows, K, num_experts, N, offsets, tile_row, tile_exp, ntiles, max_tiles, out);
  if (rc != QMOE_OK || n_rows == 0 || max_tiles == 0) return rc;
  if (!w || !scales || !biases) return qmoe::fail(QMOE_ERR_INVALID, "null pointer");
  if (bits != 4 || group_size != 64)
    return qmoe::fail(QMOE_ERR_UNSUPPORTED, "sorted GEMM takes 4-bit codes with group_size 64 (got %d, %d)",
                      bits, group_size);
  // scales and biases are copied in pairs of groups: K / 64 must be even
  if (K % 128) return qmoe::fail(QMOE_ERR_UNSUPPORTED, "K=%lld: must be a multiple of 128", (long long)K);
  if (!qmoe::aligned16(w) || !qmoe::aligned16(scales) || !qmoe::aligned16(biases))
    return qmoe::fail(QMOE_ERR_UNSUPPORTED, "w, scales and biases must be 16-byte aligned");
  GemmArgs a{x, x_rows, n_rows, (int)K, w, scales, biases, nullptr, num_experts, (int)N, offsets, tile_row,
             tile_exp, ntiles, out};
  return launch_gemm(a, max_tiles, false, stream);
}

extern "C" int qmoe_gather_qmm_sorted_tiles(const uint16_t* x, const int32_t* x_rows, int64_t n_rows, int64_t K,
                                            const uint32_t* wp, const uint32_t* sb, int32_t num_experts,
                                            int64_t N, const int32_t* offsets, const int32_t* tile_row,
                                            const int32_t* tile_exp, const int32_t* ntiles, int64_t max_tiles,
                                            uint16_t* out, void* stream) {
  const int rc = check_common(x, n_rows, K, num_experts, N, offsets, tile_row, tile_exp, ntiles, max_tiles, out);
  if (rc != QMOE_OK || n_rows == 0 || max_tiles == 0) return rc;
  if (!wp || !sb) return qmoe::fail(QMOE_ERR_INVALID, "null pointer");
  if (K % 64) return qmoe::fail(QMOE_ERR_UNSUPPORTED, "K=%lld: must be a multiple of 64", (long long)K);
  if (!qmoe::aligned16(wp) || !qmoe::aligned16(sb))
    return qmoe::fail(QMOE_ERR_UNSUPPORTED, "wp and sb must be 16-byte aligned");
  GemmArgs a{x, x_rows, n_rows, (int)K, wp, nullptr, nullptr, sb, num_experts, (int)N, offsets, tile_row,
             tile_exp, ntiles, out};
  return launch_gemm(a, max_tiles, true, stream);
}

// Prefill grouped GEMM over expert-sorted rows, bf16 MFMA on gfx950.
//
// Semantics: titan/kernels/moe_gather_ws.py:20-32 -- weights dequantised to
// bf16 as bf16_rne(fmaf(q, s, b)) (:343-344), bf16 x bf16 products, fp32
// accumulation.  Work unit: one (tile, column block).  A tile is up to
// kBM = 128 consecutive sorted rows of one expert (the tile list of the
// routing step); a column block is kBN = 256 output columns, one 64-column
// slice for each of the block's four waves.  Every wave covers all the
// tile's rows, so each weight element is dequantised once per tile.
// Persistent blocks, two per CU, take the units heavy-first in a snake over
// XCD-contiguous slots (gemm_common.h).
//
// Register budget: two waves per SIMD (two blocks per CU), so a wave may hold
// 256 registers.  Its 128 x 64 output tile is 4 x 2 subtiles of 32 x 32 fp32
// (128 accumulator registers); operands and addresses use the rest.
//
// Per 64-wide K group (one quantisation group) a wave
//   - dequantises its 64 columns' codes in registers (two 16-byte code
//     chunks per lane: 64 codes), 17 VALU instructions per 8 codes:
//     the nibbles are masked into the low bits of 16-bit halves, where they
//     read as fp16 denormals q * 2^-24 (bits 0..3) or q * 2^-20 (bits 4..7);
//     v_fma_mix_f32 widens them exactly and computes
//     fma(q * 2^-24, s * 2^24, b) == fmaf(q, s, b) bit for bit (scaling by a
//     power of two is exact), then v_cvt_pk_bf16_f32 rounds to nearest even;
//   - runs 4 k-steps x 2 * MSUB (<= 8) v_mfma_f32_32x32x16_bf16, weights as the A operand
//     (rows = output columns) and activations as B (columns = token rows), so
//     each lane ends up owning four consecutive output columns per register
//     quad and the epilogue stores 8 bytes at a time.
//
// The k-steps are software-pipelined inside each wave: while the MFMAs of
// k-step s issue, one per slot, the wave reads the activation fragments of
// k-step s + 1 and dequantises its weight fragment between them, so the
// matrix core's busy cycles cover the wave's own vector work.
//
// Data movement: every operand byte reaches LDS through asynchronous copies
// (global_load_lds_dwordx4 / _dword from inline assembly, so the copies stay
// in flight across iterations with explicit wait counts; the weight side
// from wave-uniform SGPR bases) into a ring of stages.  A stage holds
//   A  the tile's activation rows for the group, gathered through x_rows,
//      32 x 128 bytes per row subtile, 16-byte units XOR-swizzled by row (swz)
//      so operand reads are bank-conflict free; only the subtiles the tile
//      has are copied;
//   B  each wave's 64 columns of packed codes (16 bytes per lane and subtile);
//   S  the 64 columns' scales and biases.
// Row subtiles past a tile's valid rows are compiled out (the loop is
// instantiated per subtile count 1..4), so a short tile costs only its own
// MFMAs and copies, and its smaller stages let the same LDS hold more of
// them: a one-subtile tile, whose weights stream from HBM for few rows,
// keeps four groups of copies in flight instead of two.
//
// K order inside a group is free as long as A and B agree: lane half h
// supplies group elements 32h + 8kk .. +7 at k-step kk -- word kk of the
// lane's 16-byte code chunk and 16-byte unit 4h + kk of the activation row.
#include <type_traits>

#include "gemm_common.h"

#ifdef QMOE_GEMM_STAMPS
// Measurement build only (libqmoe_stamps.so): lane 0 of each block records,
// for each of its first kGemmStampUnits units, s_memrealtime (100 MHz) before
// the unit and after the unit's epilogue stores are issued, the unit number
// and its tile's row count; and after its loop, how many units it ran.  A
// launch overwrites the records of its blocks.
constexpr int kGemmStampBlocks = 1024;
constexpr int kGemmStampUnits = 32;
__device__ uint64_t gemm_stamps[kGemmStampBlocks * kGemmStampUnits * 2];
__device__ int32_t gemm_stamp_units[kGemmStampBlocks * kGemmStampUnits * 2];
__device__ int32_t gemm_stamp_counts[kGemmStampBlocks];

extern "C" int qmoe_gemm_stamps_read(uint64_t* times, int32_t* units, int32_t* counts, int64_t nblocks) {
  if (!times || !units || !counts || nblocks < 0 || nblocks > kGemmStampBlocks)
    return qmoe::fail(QMOE_ERR_INVALID, "bad stamp request");
  const size_t per = (size_t)nblocks * kGemmStampUnits * 2;
  hipError_t e = hipMemcpyFromSymbol(times, HIP_SYMBOL(gemm_stamps), per * sizeof(uint64_t), 0, hipMemcpyDeviceToHost);
  if (e == hipSuccess)
    e = hipMemcpyFromSymbol(units, HIP_SYMBOL(gemm_stamp_units), per * sizeof(int32_t), 0, hipMemcpyDeviceToHost);
  if (e == hipSuccess)
    e = hipMemcpyFromSymbol(counts, HIP_SYMBOL(gemm_stamp_counts), (size_t)nblocks * sizeof(int32_t), 0,
                            hipMemcpyDeviceToHost);
  return e == hipSuccess ? QMOE_OK : qmoe::fail(QMOE_ERR_HIP, "hipMemcpyFromSymbol: %s", hipGetErrorString(e));
}
extern "C" int qmoe_gemm_stamp_units(void) { return kGemmStampUnits; }
#endif

namespace {

using namespace qmoe_gemm;

constexpr int kBM = kTileRows;
constexpr int kWaves = 4;
constexpr int kBN = 64 * kWaves;
static_assert(kThreads == 64 * kWaves, "four waves per block");

// Stage layout (bytes) for a tile of MSUB row subtiles: A holds MSUB x 32
// activation rows of 128 bytes, B the four waves' codes, S their scales and
// biases (TILED: one scale|bias word per column; MLX layout: a scale pair and
// a bias pair, two groups, per column).  The block's LDS is sized for three
// stages of a full tile; a shorter tile fits more stages into it, and keeps
// that many groups of copies in flight (5 at one subtile, 4 at two).
template <bool TILED, int MSUB = kMaxSub>
struct Cfg {
  static constexpr int kAOff = 0;
  static constexpr int kABytes = MSUB * 32 * 128;
  static constexpr int kBOff = kAOff + kABytes;
  static constexpr int kBBytes = kWaves * 2 * 64 * 16;  // [wave][subtile][lane] x 16 B
  static constexpr int kSOff = kBOff + kBBytes;
  static constexpr int kSBytes = kWaves * (TILED ? 1 : 2) * 64 * 4;
  static constexpr int kStageBytes = kSOff + kSBytes;
  static constexpr int kLdsBytes = 3 * (kMaxSub * 32 * 128 + kBBytes + kSBytes);
  static constexpr int kStages = kLdsBytes / kStageBytes > 5 ? 5 : kLdsBytes / kStageBytes;
  static_assert(kStages >= 3, "at least three stages");
  static_assert(kBlocksPerCU * (kLdsBytes + 4 * kMaxOrder) <= 160 * 1024, "LDS per CU");
  // copies per wave and group besides A: two code chunks, one (tiled) or two
  // (scale pair, bias pair) scale copies
  static constexpr int kOtherCopies = 2 + (TILED ? 1 : 2);
  static constexpr int kCopies = MSUB + kOtherCopies;  // per wave and group
  // at most 63 vector-memory operations outstanding per wave
  static_assert((kStages - 1) * kCopies <= 63, "vmcnt range");
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

// fma(h, s, b) in fp32 with h the fp16 in the low (HI = false) or high half
// of v, widened exactly (fp16 denormals included): one v_fma_mix_f32.
template <bool HI>
__device__ __forceinline__ float fma_mix(uint32_t v, float s, float b) {
  const _Float16 h = __builtin_bit_cast(_Float16, (uint16_t)(HI ? v >> 16 : v));
  return __builtin_fmaf((float)h, s, b);
}

// Row swizzle of the 16-byte units of an activation row in LDS: unit u of
// row r is stored at u ^ swz(r).  Conflict-free for b128 reads of one unit by
// consecutive rows whether the LDS serves 8 lanes per pass over 32 banks
// (swz distinct over rows r..r+7) or 16 lanes over 64 banks (swz distinct
// over the eight rows of each parity among r..r+15).
__device__ __forceinline__ int swz(int row) { return (row & 7) ^ ((row >> 3) & 1); }

template <bool TILED>
struct Ctx {
  // per-lane global sources at group 0 (advance per group)
  const char* a_src[kMaxSub];  // activation 16-byte unit of the lane's row in A copy q
  // weight side: wave-uniform bases at group 0 and per-lane byte offsets
  const char* b_base;  // codes of the wave's 64 columns
  const char* s_base;  // MLX layout: scale pairs; tile layout: scale|bias words
  const char* z_base;  // MLX layout: bias pairs
  uint32_t b_off[2];   // the lane's code bytes in each 32-column subtile
  uint32_t s_off;      // the lane's column's scales (and biases)
  uint32_t lds;        // LDS address of the ring
  int G;
  int wave, lane, l32, h;
};

// Copy d (0 <= d < MSUB + kOtherCopies) of group g into its ring stage:
// d < MSUB is activation copy q = d (rows 32q + 8*wave .. +7 of subtile q),
// then the two code chunks, then the scales and biases.
template <bool TILED, int MSUB>
__device__ __forceinline__ void issue_copy(const Ctx<TILED>& c, int g, int d) {
  using C = Cfg<TILED, MSUB>;
  const uint32_t st = c.lds + (uint32_t)(g % C::kStages) * C::kStageBytes;
  if (d < MSUB) {
    dma16(c.a_src[d] + (size_t)g * 128, st + C::kAOff + (uint32_t)(d * kWaves + c.wave) * 1024);
    return;
  }
  const int j = d - MSUB;
  const uint32_t bdst = st + C::kBOff + (uint32_t)c.wave * 2048;
  if constexpr (TILED) {
    // one 2 KiB code chunk and one 256-byte scale|bias chunk per group
    if (j < 2) dma16s(c.b_base + (size_t)g * 2048 + j * 1024, c.b_off[0], bdst + j * 1024);
    else dma4s(c.s_base + (size_t)g * 256, c.s_off, st + C::kSOff + c.wave * 256);
  } else {
    if (j < 2) dma16s(c.b_base + (size_t)g * 32, c.b_off[j], bdst + j * 1024);
    else if (j == 2) dma4s(c.s_base + (size_t)(g >> 1) * 4, c.s_off, st + C::kSOff + c.wave * 512);
    else dma4s(c.z_base + (size_t)(g >> 1) * 4, c.s_off, st + C::kSOff + c.wave * 512 + 256);
  }
}

template <bool TILED, int MSUB>
__device__ __forceinline__ void issue_group(const Ctx<TILED>& c, int g) {
#pragma unroll
  for (int d = 0; d < Cfg<TILED, MSUB>::kCopies; ++d) issue_copy<TILED, MSUB>(c, g, d);
}

// Operands of one k-step: the wave's two dequantised weight fragments and the
// MSUB activation fragments.
template <int MSUB>
struct Frag {
  i32x4_t b[2];
  i32x4_t a[MSUB];
};

// Per-group state of the weight side: the lane's 8 code words and the raw
// scale and bias words of its two columns (converted where the first dequant
// uses them, so the conversion does not wait on LDS ahead of the MFMAs).
struct WState {
  uint32_t w[2][4];
  float s24[2], s20[2], z[2];  // column j's scale times 2^24 and 2^20 (exact), its bias
};

// Scale and bias of column j from the words holding them as bf16 halves at
// bit offsets s_sh and z_sh.
__device__ __forceinline__ void set_scale(WState& ws, int j, uint32_t sraw, uint32_t zraw, int s_sh, int z_sh) {
  const float sc = __uint_as_float((sraw >> s_sh) << 16);
  ws.s24[j] = sc * 16777216.0f;
  ws.s20[j] = sc * 1048576.0f;
  ws.z[j] = __uint_as_float((zraw >> z_sh) << 16);
}

template <bool TILED, int MSUB>
__device__ __forceinline__ WState load_wstate(const Ctx<TILED>& c, const char* st, int g) {
  using C = Cfg<TILED, MSUB>;
  WState ws;
  const uint4 raw0 = *reinterpret_cast<const uint4*>(st + C::kBOff + c.wave * 2048 + c.lane * 16);
  const uint4 raw1 = *reinterpret_cast<const uint4*>(st + C::kBOff + c.wave * 2048 + 1024 + c.lane * 16);
  ws.w[0][0] = raw0.x; ws.w[0][1] = raw0.y; ws.w[0][2] = raw0.z; ws.w[0][3] = raw0.w;
  ws.w[1][0] = raw1.x; ws.w[1][1] = raw1.y; ws.w[1][2] = raw1.z; ws.w[1][3] = raw1.w;
  if constexpr (TILED) {
    // one word per column: scale in the low half, bias in the high half
    const uint32_t* sw = reinterpret_cast<const uint32_t*>(st + C::kSOff + c.wave * 256);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const uint32_t v = sw[c.l32 + 32 * j];
      set_scale(ws, j, v, v, 0, 16);
    }
  } else {
    // scale pair and bias pair of groups (2m, 2m+1): group g in half g & 1
    const uint32_t* sw = reinterpret_cast<const uint32_t*>(st + C::kSOff + c.wave * 512);
#pragma unroll
    for (int j = 0; j < 2; ++j) set_scale(ws, j, sw[c.l32 + 32 * j], sw[64 + c.l32 + 32 * j], (g & 1) * 16, (g & 1) * 16);
  }
  return ws;
}

template <int MSUB>
__device__ __forceinline__ void read_a(Frag<MSUB>& f, const char* abuf, int kk, int l32, int h) {
  const int unit = (4 * h + kk) ^ swz(l32);  // swz(32i + l32) == swz(l32)
#pragma unroll
  for (int i = 0; i < MSUB; ++i) f.a[i] = *reinterpret_cast<const i32x4_t*>(abuf + (32 * i + l32) * 128 + unit * 16);
}

// Dwords odd and odd + 2 of the dequantised fragment of code word j at
// k-step kk (pair pr = 2j + odd): bf16_rne(fmaf(code, s, b)) of the word's
// codes (2d, 2d + 1) for dword d, low half first (k order).  The word's codes
// sit at bits 4t..4t+3; masking keeps two of them in the low bits of the
// 16-bit halves, where they read as fp16 denormals: code 0 | 4 as
// q * 2^-24 (bits 0..3 of each half), code 1 | 5 as q * 2^-20 (bits 4..7);
// shifting the word by 8 first (odd) gives codes 2 | 6 and 3 | 7.  The low
// halves make dword odd, the high halves (codes 4..7) dword odd + 2, from
// the same two masked words.
__device__ __forceinline__ void dequant_pair(i32x4_t (&b)[2], const WState& ws, int kk, int pr) {
  const int j = pr >> 1, odd = pr & 1;
  const float s24 = ws.s24[j], s20 = ws.s20[j], z = ws.z[j];
  const uint32_t v = odd ? ws.w[j][kk] >> 8 : ws.w[j][kk];
  const uint32_t lo = v & 0x000F000Fu, hi = v & 0x00F000F0u;
  b[j][odd] = (int)cvt_pk_bf16(fma_mix<false>(lo, s24, z), fma_mix<false>(hi, s20, z));
  b[j][odd | 2] = (int)cvt_pk_bf16(fma_mix<true>(lo, s24, z), fma_mix<true>(hi, s20, z));
}

// One MFMA slot of a k-step: subtile pair (p, j) = (s / 2, s % 2).
template <int MSUB>
__device__ __forceinline__ void mfma_slot(const Frag<MSUB>& f, int s, f32x16_t (&acc)[kMaxSub][2]) {
  const int p = s >> 1, j = s & 1;
  acc[p][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, f.b[j]),
                                                      __builtin_bit_cast(bf16x8_t, f.a[p]), acc[p][j], 0, 0, 0);
}

// The MFMA slot after which dequant pair pr (0..3) of the next k-step is
// computed.  LATE: the pairs wait for operands read at the start of the step
// (the next group's code words), so the first two slots carry none.
template <int MSUB, bool LATE>
constexpr int pair_slot(int pr) {
  constexpr int S = 2 * MSUB;
  if constexpr (LATE) return S > 2 ? 2 + pr * (S - 2) / 4 : S - 1;
  return pr * S / 4;
}

// One software-pipelined k-step.  The MFMAs of the current operands (cur)
// issue one per slot; between them the wave computes the next k-step's
// operands (nxt: its activation fragments were read at the start of the
// step, its weight fragment is dequantised piece by piece from ws at k-step
// kkn) and issues its share of the ring copies of group cg.  A scheduling
// fence after every slot keeps the order, so each MFMA's matrix-core time
// covers the vector work that follows it instead of the wave alternating a
// dequant burst with an MFMA burst.  NEXT = false: the last k-step of the
// tile, nothing to prepare.
template <bool TILED, int MSUB, bool NEXT, bool LATE>
__device__ __forceinline__ void step_pipe(const Ctx<TILED>& c, const Frag<MSUB>& cur, Frag<MSUB>& nxt,
                                          const WState& ws, int kkn, int cg, int cstep,
                                          f32x16_t (&acc)[kMaxSub][2]) {
  constexpr int D = Cfg<TILED, MSUB>::kCopies;
  constexpr int S = 2 * MSUB;
#pragma unroll
  for (int s = 0; s < S; ++s) {
    mfma_slot<MSUB>(cur, s, acc);
    if constexpr (NEXT) {
#pragma unroll
      for (int pr = 0; pr < 4; ++pr)
        if (pair_slot<MSUB, LATE>(pr) == s) dequant_pair(nxt.b, ws, kkn, pr);
    }
    // the group's D copies spread over the 3 * S slots of k-steps 0..2
    if (cstep >= 0) {
#pragma unroll
      for (int d = 0; d < D; ++d)
        if (d * 3 * S / D == cstep * S + s) issue_copy<TILED, MSUB>(c, cg, d);
    }
    __builtin_amdgcn_sched_barrier(0);
  }
}

// One tile's main loop over the K groups, a ring of NS stages with the copies
// of groups g + 1 .. g + NS - 1 in flight while group g is computed (every
// group copies one: the last group again once the tile is exhausted, the same
// bytes into the stage that holds them, so the loop has no branches on it).
// The operands of k-step s are prepared during k-step s - 1.  The barrier
// that makes group g + 1 visible therefore sits at the start of group g's
// last k-step: past it every wave has read all of stage g % NS
// (lgkmcnt(0) before the barrier), so the copies into that stage, issued in
// group g + 1, cannot overtake a read.
template <bool TILED, int MSUB>
__device__ __forceinline__ void tile_loop(const Ctx<TILED>& c, const char* smem, f32x16_t (&acc)[kMaxSub][2]) {
  using C = Cfg<TILED, MSUB>;
  constexpr int D = C::kCopies;
  constexpr int NS = C::kStages;
  const int G = c.G;
#pragma unroll
  for (int i = 0; i < NS - 1; ++i) issue_group<TILED, MSUB>(c, min(i, G - 1));
  wait_vmem<(NS - 2) * D>();  // group 0 landed
  __builtin_amdgcn_s_barrier();
  Frag<MSUB> fa, fb;
  WState ws = load_wstate<TILED, MSUB>(c, smem, 0);
  read_a<MSUB>(fa, smem + C::kAOff, 0, c.l32, c.h);
#pragma unroll
  for (int pr = 0; pr < 4; ++pr) dequant_pair(fa.b, ws, 0, pr);
  // groups 0 .. G - 2: the last k-step prepares the next group's first
  for (int g = 0; g < G - 1; ++g) {
    const int cg = min(g + NS - 1, G - 1);
    const char* st = smem + (g % NS) * C::kStageBytes;
    read_a<MSUB>(fb, st + C::kAOff, 1, c.l32, c.h);
    step_pipe<TILED, MSUB, true, false>(c, fa, fb, ws, 1, cg, 0, acc);
    read_a<MSUB>(fa, st + C::kAOff, 2, c.l32, c.h);
    step_pipe<TILED, MSUB, true, false>(c, fb, fa, ws, 2, cg, 1, acc);
    read_a<MSUB>(fb, st + C::kAOff, 3, c.l32, c.h);
    step_pipe<TILED, MSUB, true, false>(c, fa, fb, ws, 3, cg, 2, acc);
    // group g + 1 landed for every wave (the copies of groups g + 2 ..
    // g + NS - 1 may be outstanding); this wave's reads of stage g % NS are
    // complete
    wait_vmem<(NS - 2) * D>();
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    const char* sn = smem + ((g + 1) % NS) * C::kStageBytes;
    ws = load_wstate<TILED, MSUB>(c, sn, g + 1);
    read_a<MSUB>(fa, sn + C::kAOff, 0, c.l32, c.h);
    step_pipe<TILED, MSUB, true, true>(c, fb, fa, ws, 0, cg, -1, acc);
  }
  {
    // the last group (its copies repeat it)
    const char* st = smem + ((G - 1) % NS) * C::kStageBytes;
    read_a<MSUB>(fb, st + C::kAOff, 1, c.l32, c.h);
    step_pipe<TILED, MSUB, true, false>(c, fa, fb, ws, 1, G - 1, 0, acc);
    read_a<MSUB>(fa, st + C::kAOff, 2, c.l32, c.h);
    step_pipe<TILED, MSUB, true, false>(c, fb, fa, ws, 2, G - 1, 1, acc);
    read_a<MSUB>(fb, st + C::kAOff, 3, c.l32, c.h);
    step_pipe<TILED, MSUB, true, false>(c, fa, fb, ws, 3, G - 1, 2, acc);
    step_pipe<TILED, MSUB, false, false>(c, fb, fa, ws, 0, G - 1, -1, acc);
  }
  wait_vmem<0>();  // the trailing repeat copies
}

template <bool TILED>
__device__ __forceinline__ void store_tile(const GemmArgs& a, char* smem, const Ctx<TILED>& c,
                                           const f32x16_t (&acc)[kMaxSub][2], int64_t row0, int valid, int msub,
                                           int nblk) {
  constexpr int kPassRows = 64;
  char* ep = smem;  // the ring is free once every wave has left the main loop
  // the thread index through an empty asm: the epilogue's lane offsets are
  // then computed here, not hoisted out of the unit loop and spilled across
  // the main loop (a spill reload waits for every store still in flight)
  int tid = threadIdx.x;
  asm volatile("" : "+v"(tid));
  const int l32 = tid % 32, h = (tid % 64) / 32;
  uint16_t* obase = a.out + uniform64(row0 * (int64_t)a.N + nblk * kBN);
  for (int p = 0; 2 * p < msub; ++p) {
    __syncthreads();  // the ring (first pass) or the previous pass's rows are no longer read
#pragma unroll
    for (int i = 0; i < kMaxSub; ++i) {
      if ((i >> 1) != p) continue;
      const int m = 32 * (i & 1) + l32;  // row within the pass; m & 31 == l32
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int gi = (c.wave * 64 + 32 * j + 8 * q + 4 * h) / 4;  // 8-byte granule within the row
          const uint2 v = make_uint2(cvt_pk_bf16(acc[i][j][4 * q], acc[i][j][4 * q + 1]),
                                     cvt_pk_bf16(acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]));
          *reinterpret_cast<uint2*>(ep + m * 512 + (gi ^ (2 * l32)) * 8) = v;
        }
    }
    __syncthreads();
    constexpr int kIt = kPassRows * 32 / kThreads;
    i32x4_t v[kIt];
    uint32_t ad[kIt];
#pragma unroll
    for (int it = 0; it < kIt; ++it) {
      const int m = it * (kThreads / 32) + tid / 32;
      ad[it] = (uint32_t)(uintptr_t)(ep + m * 512 + (((tid % 32) ^ (m & 31)) * 16));
    }
    lds_read16_all(v, ad);
#pragma unroll
    for (int it = 0; it < kIt; ++it) {
      const int m = it * (kThreads / 32) + tid / 32;
      const int row = kPassRows * p + m;
      // block-uniform base + 32-bit offset: SGPR-based stores, no 64-bit row
      // pointers; non-temporal, as each output byte is written once and read,
      // if at all, by a later launch (the 4096-token MoE block, whose down
      // GEMM writes 168 MB, measured 411.0 -> 406.2 us with the hint)
      if (row < valid) __builtin_nontemporal_store(v[it], reinterpret_cast<i32x4_t*>(obase + (uint32_t)(row * a.N + (tid % 32) * 8)));
    }
  }
}

// SwiGLU epilogue over gate/up-paired weights (qmoe_repack_tiles of the
// paired row order): subtile j = 0 of a wave holds gate rows and j = 1 the
// up rows of the same 32 intermediate indices, so every lane has both
// operands of its h elements: h = silu(gate) * up in fp32 from the
// accumulators (switch_layers.py:229-237, activations.py:9-11), with a
// hardware reciprocal for the sigmoid's division, rounded once to bf16.  The
// block's 128 h columns leave through LDS as 256-byte row segments, 16-byte
// unit u of staging row m at u ^ (m & 15).
template <bool TILED>
__device__ __forceinline__ void store_tile_swiglu(const GemmArgs& a, char* smem, const Ctx<TILED>& c,
                                                  const f32x16_t (&acc)[kMaxSub][2], int64_t row0, int valid,
                                                  int msub, int nblk) {
  constexpr int kPassRows = 64;
  constexpr int kHBlock = kBN / 2;  // h columns per block
  const int NH = a.N / 2;
  char* ep = smem;
  // the thread index through an empty asm: the epilogue's lane offsets are
  // then computed here, not hoisted out of the unit loop and spilled across
  // the main loop (a spill reload waits for every store still in flight)
  int tid = threadIdx.x;
  asm volatile("" : "+v"(tid));
  const int l32 = tid % 32, h = (tid % 64) / 32;
  uint16_t* obase = a.out + row0 * (int64_t)NH + nblk * kHBlock;
  for (int p = 0; 2 * p < msub; ++p) {
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kMaxSub; ++i) {
      if ((i >> 1) != p) continue;
      const int m = 32 * (i & 1) + l32;  // row within the pass
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        float hv[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const float g = acc[i][0][4 * q + t], u = acc[i][1][4 * q + t];
          // v_rcp_f32 (1 ulp in fp32, 2^-16 of a bf16 ulp) instead of an
          // IEEE division: the division's ~10 VALU per output cost ~10 us
          // of the 4096-token block
          hv[t] = g * __builtin_amdgcn_rcpf(1.0f + __expf(-g)) * u;
        }
        const int gi = (c.wave * 32 + 8 * q + 4 * h) / 4;  // 8-byte granule within the 256-byte row
        const uint2 v = make_uint2(cvt_pk_bf16(hv[0], hv[1]), cvt_pk_bf16(hv[2], hv[3]));
        *reinterpret_cast<uint2*>(ep + m * 256 + ((((gi >> 1) ^ (m & 15)) << 1) | (gi & 1)) * 8) = v;
      }
    }
    __syncthreads();
    constexpr int kIt = kPassRows * 16 / kThreads;
    i32x4_t v[kIt];
    uint32_t ad[kIt];
#pragma unroll
    for (int it = 0; it < kIt; ++it) {
      const int m = it * (kThreads / 16) + tid / 16;
      ad[it] = (uint32_t)(uintptr_t)(ep + m * 256 + (((tid % 16) ^ (m & 15)) * 16));
    }
    lds_read16_all(v, ad);
#pragma unroll
    for (int it = 0; it < kIt; ++it) {
      const int m = it * (kThreads / 16) + tid / 16;
      const int row = kPassRows * p + m;
      if (row < valid) __builtin_nontemporal_store(v[it], reinterpret_cast<i32x4_t*>(obase + (uint32_t)(row * NH + (tid % 16) * 8)));
    }
  }
}

template <bool TILED, bool SWIGLU>
__device__ __forceinline__ void run_unit(const GemmArgs& a, char* smem, int tile, int nblk) {
  const TileRows tr = tile_rows_of(Tiles{a.offsets, a.tile_row, a.tile_exp, a.ntiles, a.n_rows, a.num_experts}, tile);
  const int e = tr.e, valid = tr.valid;
  const int64_t row0 = tr.row0;
  if (valid <= 0) return;
  const int msub = (valid + 31) / 32;

  const int K = a.K;
  const int G = K / 64;
  const int64_t KW = K / 8;
  const int tid = threadIdx.x;

  Ctx<TILED> c;
  c.G = G;
  c.wave = __builtin_amdgcn_readfirstlane(tid / 64);
  c.lane = tid % 64;
  c.l32 = c.lane % 32;
  c.h = c.lane / 32;
  c.lds = (uint32_t)(uintptr_t)smem;
  // A copy q of wave w writes stage bytes (4q + w) * 1024 + lane * 16: row
  // 32q + 8w + lane/8, stored unit lane%8, which holds logical unit
  // (lane%8) ^ swz(row).  Rows past the tile repeat its last valid row.
#pragma unroll
  for (int q = 0; q < kMaxSub; ++q) {
    const int row = 32 * q + 8 * c.wave + (c.lane >> 3);
    const int unit = (c.lane & 7) ^ swz(row);
    int64_t src = row0 + min(row, valid - 1);
    if (a.x_rows) src = a.x_rows[src];
    c.a_src[q] = reinterpret_cast<const char*>(a.x + src * K + unit * 8);
  }
  if constexpr (TILED) {
    // chunk (e, c, g) of the tile layout, c = the wave's 64-column block
    const int64_t chunk0 = ((int64_t)e * (a.N / 64) + nblk * kWaves + c.wave) * G;
    c.b_base = reinterpret_cast<const char*>(a.w) + uniform64(chunk0 * 2048);
    c.b_off[0] = c.b_off[1] = (uint32_t)c.lane * 16;
    c.s_base = reinterpret_cast<const char*>(a.sb) + uniform64(chunk0 * 256);
    c.s_off = (uint32_t)c.lane * 4;
    c.z_base = nullptr;
  } else {
    const int64_t col_base = uniform64((int64_t)e * a.N + nblk * kBN + c.wave * 64);
    c.b_base = reinterpret_cast<const char*>(a.w + col_base * KW);
#pragma unroll
    for (int j = 0; j < 2; ++j) c.b_off[j] = (uint32_t)(((j * 32 + c.l32) * KW + c.h * 4) * 4);
    c.s_base = reinterpret_cast<const char*>(a.s + col_base * G);
    c.z_base = reinterpret_cast<const char*>(a.b + col_base * G);
    c.s_off = (uint32_t)(c.lane * G * 2);
  }

  f32x16_t acc[kMaxSub][2];
#pragma unroll
  for (int i = 0; i < kMaxSub; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  static_assert(kMaxSub == 4, "one tile_loop instance per subtile count 1..kMaxSub");
  switch (msub) {
    case 1: tile_loop<TILED, 1>(c, smem, acc); break;
    case 2: tile_loop<TILED, 2>(c, smem, acc); break;
    case 3: tile_loop<TILED, 3>(c, smem, acc); break;
    default: tile_loop<TILED, 4>(c, smem, acc); break;
  }

  // epilogue: subtile (i, j) holds D^T -- lane l32 is token row 32i + l32,
  // register r is output column 32j + 8(r/4) + 4h + r%4.  The tile goes out
  // through LDS, 64 rows at a time, so that each store instruction writes
  // whole 512-byte row segments (the block's 256 columns) instead of 32
  // scattered 16-byte pieces: every wave writes its 8-byte column quads into
  // a row-major staging area (16-byte unit u of row m at u ^ (m & 31), which
  // keeps both the quad writes and the 16-byte row reads spread over the
  // banks), then the block stores the rows.
  if constexpr (SWIGLU) store_tile_swiglu<TILED>(a, smem, c, acc, row0, valid, msub, nblk);
  else store_tile<TILED>(a, smem, c, acc, row0, valid, msub, nblk);
}

// Persistent grid (kBlocksPerCU blocks per CU), each block walking its
// slot's units of the ranked tile order.
template <bool TILED, bool SWIGLU>
__global__ __launch_bounds__(kThreads, kBlocksPerCU) void gemm_bf16_kernel(GemmArgs a) {
  using C = Cfg<TILED>;
  __shared__ __attribute__((aligned(1024))) char smem[C::kLdsBytes];
  __shared__ int order[kMaxOrder];

  const Tiles tt{a.offsets, a.tile_row, a.tile_exp, a.ntiles, a.n_rows, a.num_experts};
  const int NB = a.N / kBN;
  const int ntiles = a.ntiles[0];
  const Snake sn((int64_t)ntiles * NB);
  if (sn.unit(0) < 0) return;
  const bool sorted = ntiles <= kMaxOrder;
  if (sorted) rank_tiles(tt, ntiles, order, reinterpret_cast<int*>(smem));  // the ring is free until the first unit
  int64_t k = 0;
  for (;; ++k) {
    const int64_t u = sn.unit(k);
    if (u < 0) break;
    const int rank = (int)(u / NB);
    __syncthreads();  // every wave is done with the ring before it is refilled
    if constexpr (TILED) {
      // Two blocks share each CU, and the SIMDs issue from the older one's
      // waves first, so left alone the later block runs its units ~1.5x
      // slower and the grid's blocks end far apart.  Waves instead take the
      // higher issue priority on alternate units, the two halves of the grid
      // (one block of each per CU) in opposite phase: measured 202.5 -> 196.1
      // us on the 4096-token gate_up, 415.5 -> 407.9 us on the MoE block; the
      // MLX-layout form measured slower with it (246 -> 255 us) and keeps
      // the hardware's order.
      if (((uint32_t)k ^ (blockIdx.x >= gridDim.x / 2 ? 1u : 0u)) & 1u) __builtin_amdgcn_s_setprio(1);
      else __builtin_amdgcn_s_setprio(0);
    }
#ifdef QMOE_GEMM_STAMPS
    const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
#endif
    run_unit<TILED, SWIGLU>(a, smem, sorted ? order[rank] : rank, (int)(u % NB));
#ifdef QMOE_GEMM_STAMPS
    if (threadIdx.x == 0 && blockIdx.x < kGemmStampBlocks && k < kGemmStampUnits) {
      const uint64_t t1 = __builtin_amdgcn_s_memrealtime();
      const size_t o = ((size_t)blockIdx.x * kGemmStampUnits + k) * 2;
      gemm_stamps[o] = t0;
      gemm_stamps[o + 1] = t1;
      gemm_stamp_units[o] = (int32_t)u;
      gemm_stamp_units[o + 1] = tile_rows_of(tt, sorted ? order[rank] : rank).valid;
    }
#endif
  }
#ifdef QMOE_GEMM_STAMPS
  if (threadIdx.x == 0 && blockIdx.x < kGemmStampBlocks) gemm_stamp_counts[blockIdx.x] = (int32_t)k;
#endif
}

}  // namespace

extern "C" int qmoe_gemm_tile_rows(void) { return kBM; }

namespace {

int launch_gemm(const GemmArgs& a, int64_t max_tiles, bool tiled, void* stream, bool swiglu = false) {
  const dim3 grid((unsigned)grid_blocks(max_tiles * (a.N / kBN)));
  hipStream_t st = qmoe::as_stream(stream);
  if (swiglu) gemm_bf16_kernel<true, true><<<grid, dim3(kThreads), 0, st>>>(a);
  else if (tiled) gemm_bf16_kernel<true, false><<<grid, dim3(kThreads), 0, st>>>(a);
  else gemm_bf16_kernel<false, false><<<grid, dim3(kThreads), 0, st>>>(a);
  return qmoe::launch_status("gemm_bf16_kernel");
}

int check_common(const uint16_t* x, int64_t n_rows, int64_t K, int32_t num_experts, int64_t N,
                 const int32_t* offsets, const int32_t* tile_row, const int32_t* tile_exp, const int32_t* ntiles,
                 int64_t max_tiles, const uint16_t* out) {
  if (n_rows < 0 || K <= 0 || N <= 0 || num_experts <= 0 || max_tiles < 0)
    return qmoe::fail(QMOE_ERR_INVALID, "bad sizes");
  if (n_rows == 0 || max_tiles == 0) return QMOE_OK;
  if (!x || !offsets || !tile_row || !tile_exp || !ntiles || !out) return qmoe::fail(QMOE_ERR_INVALID, "null pointer");
  if (N % kBN) return qmoe::fail(QMOE_ERR_UNSUPPORTED, "N=%lld: must be a multiple of %d", (long long)N, kBN);
  if (!qmoe::aligned16(x)) return qmoe::fail(QMOE_ERR_UNSUPPORTED, "x must be 16-byte aligned");
  if (!qmoe::aligned16(out)) return qmoe::fail(QMOE_ERR_UNSUPPORTED, "out must be 16-byte aligned");
  // the epilogue addresses a tile's rows with 32-bit offsets row * N, row < kBM
  if (K > 0x7FFFFFFF || N > (1 << 24) || n_rows > 0x7FFFFFFF)
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

extern "C" int qmoe_gather_qmm_swiglu_sorted_tiles(const uint16_t* x, const int32_t* x_rows, int64_t n_rows,
                                                   int64_t K, const uint32_t* wp, const uint32_t* sb,
                                                   int32_t num_experts, int64_t N, const int32_t* offsets,
                                                   const int32_t* tile_row, const int32_t* tile_exp,
                                                   const int32_t* ntiles, int64_t max_tiles, uint16_t* h,
                                                   void* stream) {
  const int rc = check_common(x, n_rows, K, num_experts, N, offsets, tile_row, tile_exp, ntiles, max_tiles, h);
  if (rc != QMOE_OK || n_rows == 0 || max_tiles == 0) return rc;
  if (!wp || !sb) return qmoe::fail(QMOE_ERR_INVALID, "null pointer");
  if (K % 64) return qmoe::fail(QMOE_ERR_UNSUPPORTED, "K=%lld: must be a multiple of 64", (long long)K);
  if (!qmoe::aligned16(wp) || !qmoe::aligned16(sb))
    return qmoe::fail(QMOE_ERR_UNSUPPORTED, "wp and sb must be 16-byte aligned");
  GemmArgs a{x, x_rows, n_rows, (int)K, wp, nullptr, nullptr, sb, num_experts, (int)N, offsets, tile_row,
             tile_exp, ntiles, h};
  return launch_gemm(a, max_tiles, true, stream, true);
}

namespace qmoe_gemm {

int grid_blocks(int64_t units, int blocks_per_cu) {
  static int cus = 0;
  if (!cus) {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) == hipSuccess && hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess)
      cus = n;
    if (cus <= 0) cus = 256;
  }
  const int64_t full = ((int64_t)blocks_per_cu * cus + 7) / 8 * 8;
  const int64_t need = (units + 7) / 8 * 8;
  return (int)(need < full ? (need < 8 ? 8 : need) : full);
}

}  // namespace qmoe_gemm

// Prefill grouped GEMM over expert-sorted rows, bf16 MFMA on gfx950.
//
// Semantics: titan/kernels/moe_gather_ws.py:20-32 -- weights dequantised to
// bf16 as bf16_rne(fmaf(q, s, b)) (:343-344), bf16 x bf16 products, fp32
// accumulation.  Work unit: one (tile, column block).  A tile is up to
// kBM = 128 consecutive sorted rows of one expert (the tile list of the
// routing step); a column block is kBN = 256 output columns, one 64-column
// slice per wave.
//
// Data flow per 64-wide K group (one quantisation group):
//   A  the tile's activation rows (gathered through x_rows) are staged in LDS,
//      double-buffered, shared by the four waves;
//   B  each lane loads the 16 packed bytes of its own column and half-group,
//      dequantises them in registers straight into the MFMA B operand -- the
//      columns of a wave are its own, so B never touches LDS;
//   four k-steps of v_mfma_f32_32x32x16_bf16 per (32-row, 32-column) subtile.
// Row subtiles past the tile's valid rows are skipped, so a short tail tile
// costs only the MFMAs of its 32-row subtiles.
//
// K-order inside a group is free as long as A and B agree: lane half h
// (lanes 32h..32h+31) supplies group elements 32h + 8*kk .. +7 at k-step kk,
// which is word kk of the lane's 16-byte code load and bytes 64h + 16kk of the
// row's 128-byte group segment.
#include "common.h"

namespace {

constexpr int kBM = 128;
constexpr int kBN = 256;
constexpr int kThreads = 256;
constexpr int kLDA = 72;  // bf16 per LDS row: 64 + 8 pad keeps b128 reads conflict-free

struct GemmArgs {
  const uint16_t* x;
  const int32_t* x_rows;
  int64_t n_rows;
  int K;
  const uint32_t* w;
  const uint16_t* s;
  const uint16_t* b;
  int num_experts;
  int N;
  const int32_t* offsets;
  const int32_t* tile_row;
  const int32_t* tile_exp;
  const int32_t* ntiles;
  uint16_t* out;
};

// bf16 element i (0..7) of a 16-byte chunk
__device__ __forceinline__ float bf16_at(const uint4& c, int i) {
  const uint32_t w = (i & 4) ? ((i & 2) ? c.w : c.z) : ((i & 2) ? c.y : c.x);
  return (i & 1) ? bf16hi(w) : bf16lo(w);
}

typedef __attribute__((__vector_size__(2 * sizeof(float)))) float f32x2_t;

__device__ __forceinline__ uint32_t cvt_pk_bf16(float a, float b) {
  f32x2_t v = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

// 8 codes of one word -> 8 bf16 (k order 0..7), bf16_rne(fmaf(q, s, b)).
__device__ __forceinline__ i32x4_t dequant_word(uint32_t v, float s, float b) {
  const uint32_t lo = v & 0x0F0F0F0Fu;
  const uint32_t hi = (v >> 4) & 0x0F0F0F0Fu;
  i32x4_t r;
  r[0] = (int)cvt_pk_bf16(__builtin_fmaf((float)(lo & 0xFFu), s, b), __builtin_fmaf((float)(hi & 0xFFu), s, b));
  r[1] = (int)cvt_pk_bf16(__builtin_fmaf((float)((lo >> 8) & 0xFFu), s, b),
                          __builtin_fmaf((float)((hi >> 8) & 0xFFu), s, b));
  r[2] = (int)cvt_pk_bf16(__builtin_fmaf((float)((lo >> 16) & 0xFFu), s, b),
                          __builtin_fmaf((float)((hi >> 16) & 0xFFu), s, b));
  r[3] = (int)cvt_pk_bf16(__builtin_fmaf((float)(lo >> 24), s, b), __builtin_fmaf((float)(hi >> 24), s, b));
  return r;
}

struct BFrag {
  i32x4_t v[2][4];  // [column subtile][k-step]
};

__device__ __forceinline__ void dequant_b(const uint4 (&raw)[2], const float (&s)[2], const float (&b)[2],
                                          BFrag& f) {
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    f.v[j][0] = dequant_word(raw[j].x, s[j], b[j]);
    f.v[j][1] = dequant_word(raw[j].y, s[j], b[j]);
    f.v[j][2] = dequant_word(raw[j].z, s[j], b[j]);
    f.v[j][3] = dequant_word(raw[j].w, s[j], b[j]);
  }
}

__global__ __launch_bounds__(kThreads) void gemm_bf16_kernel(GemmArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t As[2][kBM * kLDA];

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
  const int wave = tid / 64;
  const int lane = tid % 64;
  const int l32 = lane % 32;
  const int h = lane / 32;

  // A staging: thread -> (row, half of the 128-byte group segment)
  const int arow = tid >> 1;
  const int ahalf = tid & 1;
  int64_t src = row0 + min(arow, valid - 1);
  if (a.x_rows) src = a.x_rows[src];
  const uint4* aptr = reinterpret_cast<const uint4*>(a.x + src * K + ahalf * 32);
  uint16_t* const adst0 = &As[0][arow * kLDA + ahalf * 32];
  uint16_t* const adst1 = &As[1][arow * kLDA + ahalf * 32];

  // B: this lane's two columns
  const int ncol = nblk * kBN + wave * 64 + l32;
  const int64_t c0 = (int64_t)e * a.N + ncol;
  const int64_t c1 = c0 + 32;
  const uint4* bp0 = reinterpret_cast<const uint4*>(a.w + c0 * KW) + h;
  const uint4* bp1 = reinterpret_cast<const uint4*>(a.w + c1 * KW) + h;
  const uint4* sp0 = reinterpret_cast<const uint4*>(a.s + c0 * G);
  const uint4* sp1 = reinterpret_cast<const uint4*>(a.s + c1 * G);
  const uint4* zp0 = reinterpret_cast<const uint4*>(a.b + c0 * G);
  const uint4* zp1 = reinterpret_cast<const uint4*>(a.b + c1 * G);

  f32x16_t acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  uint4 areg[4];
  uint4 braw[2];
  uint4 sch[2], bch[2];  // 8 groups of scales / biases per column
  BFrag fa, fb;

  // prologue: group 0
#pragma unroll
  for (int c = 0; c < 4; ++c) areg[c] = aptr[c];
  braw[0] = bp0[0];
  braw[1] = bp1[0];
  sch[0] = sp0[0];
  sch[1] = sp1[0];
  bch[0] = zp0[0];
  bch[1] = zp1[0];
#pragma unroll
  for (int c = 0; c < 4; ++c) reinterpret_cast<uint4*>(adst0)[c] = areg[c];
  {
    const float s2[2] = {bf16_at(sch[0], 0), bf16_at(sch[1], 0)};
    const float b2[2] = {bf16_at(bch[0], 0), bf16_at(bch[1], 0)};
    dequant_b(braw, s2, b2, fa);
  }

  auto step = [&](int g, const BFrag& cur, BFrag& nxt) {
    const bool more = g + 1 < G;
    if (more) {
      const int gn = g + 1;
#pragma unroll
      for (int c = 0; c < 4; ++c) areg[c] = aptr[gn * 8 + c];
      braw[0] = bp0[gn * 2];
      braw[1] = bp1[gn * 2];
      if ((gn & 7) == 0) {
        sch[0] = sp0[gn >> 3];
        sch[1] = sp1[gn >> 3];
        bch[0] = zp0[gn >> 3];
        bch[1] = zp1[gn >> 3];
      }
    }
    __syncthreads();
    const uint16_t* abuf = As[g & 1];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if (i < msub) {
          const i32x4_t af = *reinterpret_cast<const i32x4_t*>(abuf + (32 * i + l32) * kLDA + 32 * h + 8 * kk);
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, af),
                                                                __builtin_bit_cast(bf16x8_t, cur.v[j][kk]),
                                                                acc[i][j], 0, 0, 0);
          }
        }
      }
    }
    if (more) {
      uint16_t* d = (g & 1) ? adst0 : adst1;
#pragma unroll
      for (int c = 0; c < 4; ++c) reinterpret_cast<uint4*>(d)[c] = areg[c];
      const int gi = (g + 1) & 7;
      const float s2[2] = {bf16_at(sch[0], gi), bf16_at(sch[1], gi)};
      const float b2[2] = {bf16_at(bch[0], gi), bf16_at(bch[1], gi)};
      dequant_b(braw, s2, b2, nxt);
    }
  };

  for (int g = 0; g < G; g += 2) {
    step(g, fa, fb);
    step(g + 1, fb, fa);
  }

  // epilogue: D[m][n] of a 32x32 subtile sits in lane n (mod 32), register
  // r at row 8*(r/4) + 4*(lane/32) + r%4.
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if (i >= msub) continue;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int m = 32 * i + 8 * (r / 4) + 4 * h + (r % 4);
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

extern "C" int qmoe_gather_qmm_sorted(const uint16_t* x, const int32_t* x_rows, int64_t n_rows, int64_t K,
                                      const uint32_t* w, const uint16_t* scales, const uint16_t* biases,
                                      int32_t num_experts, int64_t N, int group_size, int bits,
                                      const int32_t* offsets, const int32_t* tile_row,
                                      const int32_t* tile_exp, const int32_t* ntiles, int64_t max_tiles,
                                      uint16_t* out, void* stream) {
  if (n_rows < 0 || K <= 0 || N <= 0 || num_experts <= 0 || max_tiles < 0)
    return qmoe::fail(QMOE_ERR_INVALID, "bad sizes");
  if (n_rows == 0 || max_tiles == 0) return QMOE_OK;
  if (!x || !w || !scales || !biases || !offsets || !tile_row || !tile_exp || !ntiles || !out)
    return qmoe::fail(QMOE_ERR_INVALID, "null pointer");
  if (bits != 4 || group_size != 64)
    return qmoe::fail(QMOE_ERR_UNSUPPORTED, "sorted GEMM takes 4-bit codes with group_size 64 (got %d, %d)",
                      bits, group_size);
  if (K % 1024) return qmoe::fail(QMOE_ERR_UNSUPPORTED, "K=%lld: must be a multiple of 1024", (long long)K);
  if (N % kBN) return qmoe::fail(QMOE_ERR_UNSUPPORTED, "N=%lld: must be a multiple of %d", (long long)N, kBN);
  if (!qmoe::aligned16(x) || !qmoe::aligned16(w) || !qmoe::aligned16(scales) || !qmoe::aligned16(biases))
    return qmoe::fail(QMOE_ERR_UNSUPPORTED, "x, w, scales and biases must be 16-byte aligned");
  if (K > 0x7FFFFFFF || N > 0x7FFFFFFF || n_rows > 0x7FFFFFFF)
    return qmoe::fail(QMOE_ERR_UNSUPPORTED, "sizes too large");
  const int64_t blocks = max_tiles * (N / kBN);
  if (blocks > 0x7FFFFFFF) return qmoe::fail(QMOE_ERR_UNSUPPORTED, "grid too large");
  GemmArgs a{x, x_rows, n_rows, (int)K, w, scales, biases, num_experts, (int)N, offsets, tile_row, tile_exp, ntiles,
             out};
  gemm_bf16_kernel<<<dim3((unsigned)blocks), dim3(kThreads), 0, qmoe::as_stream(stream)>>>(a);
  return qmoe::launch_status("gemm_bf16_kernel");
}

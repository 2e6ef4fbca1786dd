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
// into two bf16 terms (|R| <= 8128: hi = bf16(R) and lo = R - hi are exact),
// so it adds no per-group vector work.
#include "common.h"

namespace {

constexpr int kTileRows = 128;  // rows per routing tile (qmoe_gemm_tile_rows)
constexpr int kBM = 128;
constexpr int kBN = 256;
constexpr int kThreads = 256;
constexpr int kLDA = 80;   // bytes per LDS activation row: 64 + 16 pad
constexpr int kMaxG = 64;  // K <= 4096

// ---------------------------------------------------------------- quantizer

// One wave per row; each lane owns K/64 consecutive elements (a multiple of 8).
__global__ __launch_bounds__(256) void quant_act_kernel(const uint16_t* __restrict__ x, int64_t R, int K,
                                                        int8_t* __restrict__ xi, float* __restrict__ sx) {
  const int64_t r = (int64_t)blockIdx.x * 4 + threadIdx.x / 64;
  const int lane = threadIdx.x % 64;
  if (r >= R) return;
  const int per = K / 64;
  const uint16_t* xr = x + r * K + lane * per;
  float amax = 0.f;
  for (int i = 0; i < per; i += 8) {
    const uint4 q = *reinterpret_cast<const uint4*>(xr + i);
    const uint32_t v[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) amax = fmaxf(amax, fmaxf(fabsf(bf16lo(v[j])), fabsf(bf16hi(v[j]))));
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) amax = fmaxf(amax, __shfl_xor(amax, m, 64));
  const float sc = __fdiv_rn(amax, 127.0f);
  if (lane == 0) sx[r] = sc;
  int8_t* out = xi + r * K + lane * per;
  for (int i = 0; i < per; i += 8) {
    const uint4 q = *reinterpret_cast<const uint4*>(xr + i);
    const uint32_t v[4] = {q.x, q.y, q.z, q.w};
    uint32_t packed[2] = {0u, 0u};
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float xv = (j & 1) ? bf16hi(v[j >> 1]) : bf16lo(v[j >> 1]);
      float t = sc == 0.f ? 0.f : rintf(__fdiv_rn(xv, sc));
      t = fminf(fmaxf(t, -127.f), 127.f);
      packed[j >> 2] |= ((uint32_t)(int)t & 0xFFu) << (8 * (j & 3));
    }
    *reinterpret_cast<uint2*>(out + i) = make_uint2(packed[0], packed[1]);
  }
}

// ---------------------------------------------------------------- GEMM

struct Int8Args {
  const int8_t* xi;
  const float* sx;
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

__device__ __forceinline__ float bf16_at(const uint4& c, int i) {
  const uint32_t w = (i & 4) ? ((i & 2) ? c.w : c.z) : ((i & 2) ? c.y : c.x);
  return (i & 1) ? bf16hi(w) : bf16lo(w);
}

__device__ __forceinline__ int sum_i8x4(uint32_t v) {
  return (int)(int8_t)(v & 0xFF) + (int)(int8_t)((v >> 8) & 0xFF) + (int)(int8_t)((v >> 16) & 0xFF) +
         (int)(int8_t)(v >> 24);
}

__global__ __launch_bounds__(kThreads) void gemm_int8_kernel(Int8Args a) {
  __shared__ __attribute__((aligned(16))) int8_t As[2][kBM * kLDA];
  __shared__ __attribute__((aligned(16))) uint16_t Rhi[kBM][kMaxG + 8];
  __shared__ __attribute__((aligned(16))) uint16_t Rlo[kBM][kMaxG + 8];

  // A routing tile spans up to kTileRows rows; a block covers kBM of them.
  const int NB = a.N / kBN;
  constexpr int kHalves = kTileRows / kBM;
  const int64_t n_active = (int64_t)a.ntiles[0] * kHalves * NB;
  const int64_t hw = blockIdx.x;
  if (hw >= n_active) return;
  const int64_t q8 = n_active / 8, r8 = n_active % 8, xcd = hw % 8;
  const int64_t logical = xcd * q8 + (xcd < r8 ? xcd : r8) + hw / 8;
  const int tile = (int)(logical / (NB * kHalves));
  const int half = (int)(logical / NB % kHalves);
  const int nblk = (int)(logical % NB);

  const int e = min(max(a.tile_exp[tile], 0), a.num_experts - 1);
  const int64_t row0 = a.tile_row[tile] + (int64_t)half * kBM;
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

  // activation staging: thread -> (row, half of the 64-byte group segment)
  const int arow = tid >> 1;
  const int ahalf = tid & 1;
  int64_t src = row0 + min(arow, valid - 1);
  if (a.x_rows) src = a.x_rows[src];
  const uint4* aptr = reinterpret_cast<const uint4*>(a.xi + src * K + ahalf * 32);

  const int ncol = nblk * kBN + wave * 64 + l32;
  const int64_t c0 = (int64_t)e * a.N + ncol;
  const int64_t c1 = c0 + 32;
  const uint4* bp0 = reinterpret_cast<const uint4*>(a.w + c0 * KW) + h;
  const uint4* bp1 = reinterpret_cast<const uint4*>(a.w + c1 * KW) + h;
  const uint4* sp0 = reinterpret_cast<const uint4*>(a.s + c0 * G);
  const uint4* sp1 = reinterpret_cast<const uint4*>(a.s + c1 * G);

  f32x16_t acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  uint4 areg[2];
  uint4 braw[2];
  uint4 sch[2];

  auto stage_a = [&](int g, int buf) {
    // 32 int8 per thread: store, and the exact row sum of the group (two threads per row)
    int8_t* d = &As[buf][arow * kLDA + ahalf * 32];
    reinterpret_cast<uint4*>(d)[0] = areg[0];
    reinterpret_cast<uint4*>(d)[1] = areg[1];
    int part = sum_i8x4(areg[0].x) + sum_i8x4(areg[0].y) + sum_i8x4(areg[0].z) + sum_i8x4(areg[0].w) +
               sum_i8x4(areg[1].x) + sum_i8x4(areg[1].y) + sum_i8x4(areg[1].z) + sum_i8x4(areg[1].w);
    part += __shfl_xor(part, 1, 64);
    if (ahalf == 0) {
      const float rf = (float)part;
      const uint32_t hi = f32_to_bf16(rf);
      const float lo = rf - bf16_to_f32(hi);  // exact: |R| <= 8128
      Rhi[arow][g] = (uint16_t)hi;
      Rlo[arow][g] = (uint16_t)f32_to_bf16(lo);
    }
  };

  // prologue
  areg[0] = aptr[0];
  areg[1] = aptr[1];
  braw[0] = bp0[0];
  braw[1] = bp1[0];
  sch[0] = sp0[0];
  sch[1] = sp1[0];
  stage_a(0, 0);
  uint4 bcur[2] = {braw[0], braw[1]};
  float scur[2] = {bf16_at(sch[0], 0), bf16_at(sch[1], 0)};

  for (int g = 0; g < G; ++g) {
    const bool more = g + 1 < G;
    if (more) {
      const int gn = g + 1;
      areg[0] = aptr[gn * 4];
      areg[1] = aptr[gn * 4 + 1];
      braw[0] = bp0[gn * 2];
      braw[1] = bp1[gn * 2];
      if ((gn & 7) == 0) {
        sch[0] = sp0[gn >> 3];
        sch[1] = sp1[gn >> 3];
      }
    }
    __syncthreads();
    const int8_t* abuf = As[g & 1];
    i32x4_t bf[2][2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      bf[j][0] = codes_to_i8(bcur[j].x, bcur[j].y);
      bf[j][1] = codes_to_i8(bcur[j].z, bcur[j].w);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (i < msub) {
        const i32x4_t a0 = *reinterpret_cast<const i32x4_t*>(abuf + (32 * i + l32) * kLDA + 32 * h);
        const i32x4_t a1 = *reinterpret_cast<const i32x4_t*>(abuf + (32 * i + l32) * kLDA + 32 * h + 16);
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          i32x16_t d = {};
          d = __builtin_amdgcn_mfma_i32_32x32x32_i8(a0, bf[j][0], d, 0, 0, 0);
          d = __builtin_amdgcn_mfma_i32_32x32x32_i8(a1, bf[j][1], d, 0, 0, 0);
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[i][j][r] = __builtin_fmaf(scur[j], (float)d[r], acc[i][j][r]);
        }
      }
    }
    if (more) {
      stage_a(g + 1, (g + 1) & 1);
      bcur[0] = braw[0];
      bcur[1] = braw[1];
      const int gi = (g + 1) & 7;
      scur[0] = bf16_at(sch[0], gi);
      scur[1] = bf16_at(sch[1], gi);
    }
  }
  __syncthreads();

  // bias term: acc += R (rows x G) . b^T (G x cols), bf16 MFMA, R = hi + lo exactly
  const uint4* zp0 = reinterpret_cast<const uint4*>(a.b + c0 * G);
  const uint4* zp1 = reinterpret_cast<const uint4*>(a.b + c1 * G);
  for (int g0 = 0; g0 < G; g0 += 16) {
    // lane half h supplies g0 + 8h .. +7
    const int gc = (g0 >> 3) + h;
    const uint4 bz[2] = {zp0[gc], zp1[gc]};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (i < msub) {
        const i32x4_t rh = *reinterpret_cast<const i32x4_t*>(&Rhi[32 * i + l32][g0 + 8 * h]);
        const i32x4_t rl = *reinterpret_cast<const i32x4_t*>(&Rlo[32 * i + l32][g0 + 8 * h]);
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const bf16x8_t bb = __builtin_bit_cast(bf16x8_t, bz[j]);
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, rh), bb, acc[i][j], 0, 0, 0);
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, rl), bb, acc[i][j], 0, 0, 0);
        }
      }
    }
  }

#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if (i >= msub) continue;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int m = 32 * i + 8 * (r / 4) + 4 * h + (r % 4);
      if (m < valid) {
        int64_t xr = row0 + m;
        const float scale = a.sx[a.x_rows ? (int64_t)a.x_rows[xr] : xr];
        uint16_t* orow = a.out + (row0 + m) * (int64_t)a.N + ncol;
        orow[0] = (uint16_t)f32_to_bf16(scale * acc[i][0][r]);
        orow[32] = (uint16_t)f32_to_bf16(scale * acc[i][1][r]);
      }
    }
  }
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
  if (n_rows < 0 || K <= 0 || N <= 0 || num_experts <= 0 || max_tiles < 0)
    return qmoe::fail(QMOE_ERR_INVALID, "bad sizes");
  if (n_rows == 0 || max_tiles == 0) return QMOE_OK;
  if (!xi || !sx || !w || !scales || !biases || !offsets || !tile_row || !tile_exp || !ntiles || !out)
    return qmoe::fail(QMOE_ERR_INVALID, "null pointer");
  if (bits != 4 || group_size != 64)
    return qmoe::fail(QMOE_ERR_UNSUPPORTED, "int8 GEMM takes 4-bit codes with group_size 64 (got %d, %d)", bits,
                      group_size);
  if (K % 1024 || K > 64 * kMaxG)
    return qmoe::fail(QMOE_ERR_UNSUPPORTED, "K=%lld: must be a multiple of 1024, at most %d", (long long)K,
                      64 * kMaxG);
  if (N % kBN) return qmoe::fail(QMOE_ERR_UNSUPPORTED, "N=%lld: must be a multiple of %d", (long long)N, kBN);
  if (!qmoe::aligned16(xi) || !qmoe::aligned16(w) || !qmoe::aligned16(scales) || !qmoe::aligned16(biases))
    return qmoe::fail(QMOE_ERR_UNSUPPORTED, "xi, w, scales and biases must be 16-byte aligned");
  if (N > 0x7FFFFFFF || n_rows > 0x7FFFFFFF) return qmoe::fail(QMOE_ERR_UNSUPPORTED, "sizes too large");
  if (qmoe_gemm_tile_rows() != kTileRows) return qmoe::fail(QMOE_ERR_UNSUPPORTED, "tile rows mismatch");
  const int64_t blocks = max_tiles * (kTileRows / kBM) * (N / kBN);
  if (blocks > 0x7FFFFFFF) return qmoe::fail(QMOE_ERR_UNSUPPORTED, "grid too large");
  Int8Args a{xi, sx, x_rows, n_rows, (int)K, w, scales, biases, num_experts, (int)N, offsets, tile_row, tile_exp,
             ntiles, out};
  gemm_int8_kernel<<<dim3((unsigned)blocks), dim3(kThreads), 0, qmoe::as_stream(stream)>>>(a);
  return qmoe::launch_status("gemm_int8_kernel");
}

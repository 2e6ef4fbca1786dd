// Decode-shape quantized matrix-vector kernels for gfx950.
//
// One weight row is reduced by a group of LPR lanes (LPR = 16 for K = 2048):
// each lane owns NV chunks of 32 consecutive K elements, chunk v of lane l
// starting at k = v*32*LPR + l*32, so the LPR lanes of a group read 256
// contiguous bytes of packed codes per 16-byte load.  A wave holds 64/LPR
// groups and therefore streams 64/LPR rows at once.
//
// Inner product without materialising bf16 weights:
//   a code pair (q_a, q_b) becomes the bf16 pair (128 + q_a, 128 + q_b) by
//   OR-ing 0x4300 into each half (0x4300 is 128.0; 128 + q is exact in bf16),
//   v_dot2_f32_bf16 accumulates x*(128 + q) in fp32, and per 32-element chunk
//       sum_k x*(s*q + b) = s*(dot - 128*sum_x) + b*sum_x.
// This is the factored affine form of the reference decode kernels
// (engine/patches/decode-fusion/fused_kernels.py:57-79), with the codes fed
// to the dot unit two at a time.
#include <stdarg.h>

#include <stdlib.h>

#include "common.h"
#include "topk.h"

namespace {

constexpr uint32_t kMagic = 0x43004300u;  // bf16 128.0 in both halves

// Rows per row group of the 2048-chunk GEMV (see qmv64_kernel).  The fused
// gate_up form takes four gate/up pairs per wave (1280 waves at top-10 of
// I = 512); the plain form two groups of two rows (1024 waves at N = 4096).
#ifndef QMOE_QMV_RG_GU
#define QMOE_QMV_RG_GU 4
#endif
#ifndef QMOE_QMV_RG_DENSE
#define QMOE_QMV_RG_DENSE 2
#endif

// x pairs laid out to match the nibble pairs of one 32-bit code word:
// word j covers elements 8j..8j+7; pairs are (0,4), (1,5), (2,6), (3,7).
struct XChunk {
  uint32_t p[16];
  float sum;
};

__device__ __forceinline__ void load_x_chunk(const uint16_t* __restrict__ src, XChunk& c) {
  const uint4* q = reinterpret_cast<const uint4*>(src);
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    uint4 a = q[j];
    c.p[4 * j + 0] = (a.x & 0xFFFFu) | (a.z << 16);
    c.p[4 * j + 1] = (a.x >> 16) | (a.z & 0xFFFF0000u);
    c.p[4 * j + 2] = (a.y & 0xFFFFu) | (a.w << 16);
    c.p[4 * j + 3] = (a.y >> 16) | (a.w & 0xFFFF0000u);
    s += ((bf16lo(a.x) + bf16hi(a.x)) + (bf16lo(a.y) + bf16hi(a.y))) +
         ((bf16lo(a.z) + bf16hi(a.z)) + (bf16lo(a.w) + bf16hi(a.w)));
  }
  c.sum = s;
}

// (a & m) | c in one v_and_or_b32.  A gfx950 VOP3 instruction encodes no
// 32-bit literal and reads at most one SGPR, so the mask rides in an SGPR and
// the bf16 magic in a VGPR (`magic_vgpr()`); left to itself the compiler
// emits a v_and_b32 and a v_or_b32 with literals, 16 extra VALU ops per chunk.
__device__ __forceinline__ uint32_t and_or(uint32_t a, uint32_t m, uint32_t c) {
  uint32_t d;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(d) : "v"(a), "s"(m), "v"(c));
  return d;
}
// kMagic held in a VGPR for and_or; the empty asm keeps it out of constant folding.
__device__ __forceinline__ uint32_t magic_vgpr() {
  uint32_t v = kMagic;
  asm volatile("" : "+v"(v));
  return v;
}

// sum over the chunk of x*(128 + q): 4 and_or + 3 shifts + 4 v_dot2 per word
__device__ __forceinline__ float dot_chunk(const uint4& w, const XChunk& c, uint32_t mv) {
  const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
  const uint32_t m = 0x000F000Fu;
  float acc = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t v = ws[j];
    acc = dot2_bf16(and_or(v, m, mv), c.p[4 * j + 0], acc);
    acc = dot2_bf16(and_or(v >> 4, m, mv), c.p[4 * j + 1], acc);
    acc = dot2_bf16(and_or(v >> 8, m, mv), c.p[4 * j + 2], acc);
    acc = dot2_bf16(and_or(v >> 12, m, mv), c.p[4 * j + 3], acc);
  }
  return acc;
}

// n / d for a divisor fixed at launch and n < 2^31: q = (umulhi(n, m) + n) >> s
// with s = ceil(log2 d), m = ceil(2^(32+s) / d) - 2^32 (round-up reciprocal;
// exact because m*d - 2^(32+s) < d <= 2^s).  Replaces 64-bit divisions that
// the compiler expands into ~40 dependent scalar instructions at kernel entry.
struct FastDiv {
  uint32_t d, m, s;
};
inline FastDiv make_fastdiv(uint32_t d) {
  uint32_t s = 0;
  while ((1ull << s) < d) ++s;
  const uint64_t m = ((1ull << (32 + s)) + d - 1) / d - (1ull << 32);
  return {d, (uint32_t)m, s};
}
__device__ __forceinline__ uint32_t fast_div(uint32_t n, const FastDiv& f) {
  return (uint32_t)(((uint64_t)__umulhi(n, f.m) + n) >> f.s);
}

__device__ __forceinline__ float affine_chunk(float dq, float xsum, float s, float b) {
  return s * (dq - 128.0f * xsum) + b * xsum;
}

// 8-bit codes: a word holds elements 4j..4j+3, one byte each.  The nibbles of
// bytes (0, 2) and (1, 3) go through the same bf16 magic as the 4-bit codes,
// low and high nibble separately, so per word
//   sum x*(128 + lo) + 16 * sum x*(128 + hi) = sum x*q + 2176 * sum x.
// x pairs to match: p[2j] = (x[4j], x[4j+2]), p[2j+1] = (x[4j+1], x[4j+3]).
__device__ __forceinline__ void load_x_chunk8(const uint16_t* __restrict__ src, XChunk& c) {
  const uint4* q = reinterpret_cast<const uint4*>(src);
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint4 a = q[j];
    // words 2j (elements 8j..8j+3: a.x, a.y) and 2j+1 (8j+4..8j+7: a.z, a.w)
    c.p[4 * j + 0] = (a.x & 0xFFFFu) | (a.y << 16);
    c.p[4 * j + 1] = (a.x >> 16) | (a.y & 0xFFFF0000u);
    c.p[4 * j + 2] = (a.z & 0xFFFFu) | (a.w << 16);
    c.p[4 * j + 3] = (a.z >> 16) | (a.w & 0xFFFF0000u);
    s += ((bf16lo(a.x) + bf16hi(a.x)) + (bf16lo(a.y) + bf16hi(a.y))) +
         ((bf16lo(a.z) + bf16hi(a.z)) + (bf16lo(a.w) + bf16hi(a.w)));
  }
  c.sum = s;
}

// sum over the 32-element chunk (8 words in w0, w1) of x*(128 + lo) + 16*x*(128 + hi)
__device__ __forceinline__ float dot_chunk8(const uint4& w0, const uint4& w1, const XChunk& c, uint32_t mv) {
  const uint32_t ws[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
  const uint32_t m = 0x000F000Fu;
  float lo = 0.f, hi = 0.f;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const uint32_t v = ws[j];
    lo = dot2_bf16(and_or(v, m, mv), c.p[2 * j + 0], lo);
    hi = dot2_bf16(and_or(v >> 4, m, mv), c.p[2 * j + 0], hi);
    lo = dot2_bf16(and_or(v >> 8, m, mv), c.p[2 * j + 1], lo);
    hi = dot2_bf16(and_or(v >> 12, m, mv), c.p[2 * j + 1], hi);
  }
  return lo + 16.0f * hi;
}

__device__ __forceinline__ float affine_chunk8(float dq, float xsum, float s, float b) {
  return s * (dq - 2176.0f * xsum) + b * xsum;
}

// SwiGLU of one output in fp32 (switch_layers.py:229-237,
// activations.py:9-11): silu(gate) * up, the sigmoid through v_exp_f32 and
// v_rcp_f32 (a few fp32 ulps, far below the bf16 rounding that follows)
// rather than the library expf and an IEEE division, whose ~30 dependent
// instructions sit at the end of every decode wave's chain.  Every decode
// kernel uses this one expression, so their results stay bit-identical.
__device__ __forceinline__ float swiglu_f32(float gate, float up) {
  return gate * __builtin_amdgcn_rcpf(1.0f + __expf(-gate)) * up;
}

struct QmvArgs {
  const uint16_t* x;
  int64_t x_stride;      // elements between consecutive x rows
  const int32_t* x_rows; // may be null
  int64_t x_div;         // x row = pair / x_div when x_rows is null
  const int32_t* experts;  // may be null (dense: expert 0)
  int64_t n_pairs;
  int K;
  int group_size;
  const uint32_t* w;
  const uint16_t* s;
  const uint16_t* b;
  int num_experts;
  int n_out;  // outputs per pair (N, or I for the SwiGLU form)
  int n_w;    // weight rows per expert (N, or 2I)
  uint16_t* out;
  const uint32_t* sb;  // tile layout: scale|bias words (w then holds the tile-layout codes)
  FastDiv blk_div;     // qmv64: blocks per pair
  FastDiv x_divf;      // qmv64: x_div
  float* out_f32;      // plain row form only: fp32 results here instead of bf16 in out
  // tiled SwiGLU form: experts from each token's top-k of these [T, E] fp32
  // logits, written with their scores to topk_idx / topk_scores [T, k]
  const float* logits = nullptr;
  int32_t* topk_idx = nullptr;
  float* topk_scores = nullptr;
  int topk_norm = 1;
};

// The expert of pair pr = t * k + j of the tiled SwiGLU form: experts[pr], or
// with PER > 0 choice j of token t's top-k of its router logits, which is the
// last choice of its top-(j + 1) (the order is by value, then index).  The
// wave of the token's first column block and last slot, j = k - 1, also
// writes the token's k ids and scores: it runs the whole selection here, keeps
// it in ts, and computes and stores the scores in pair_topk_store, which the
// kernel calls once its weight loads are in flight.  Wave-uniform.
template <int PER>
struct PairTopk {
  bool writer = false;
  float v[PER > 0 ? PER : 1];
  int idx = 0;
  uint32_t key_j = 0;
};

template <int PER>
__device__ __forceinline__ int pair_expert(const QmvArgs& a, uint32_t pr, uint32_t t, bool first_block,
                                           PairTopk<PER>& ts) {
  if constexpr (PER == 0) {
    return a.experts[pr];
  } else {
    const int k = (int)a.x_div;
    const int j = __builtin_amdgcn_readfirstlane((int)(pr - t * (uint32_t)k));
    const float* lp = a.logits + (int64_t)t * a.num_experts;
    ts.writer = first_block && j == k - 1;
    if (!ts.writer) return qmoe_topk::wave_topk_last<PER>(lp, a.num_experts, j + 1);
    qmoe_topk::wave_topk_select<PER>(lp, a.num_experts, k, ts.v, ts.idx, ts.key_j);
    return __builtin_amdgcn_readlane(ts.idx, j);
  }
}

template <int PER>
__device__ __forceinline__ void pair_topk_store(const QmvArgs& a, uint32_t t, const PairTopk<PER>& ts) {
  if constexpr (PER > 0) {
    if (!ts.writer) return;
    const int k = (int)a.x_div;
    const float sc = qmoe_topk::wave_topk_scores<PER>(ts.v, k, a.topk_norm, ts.key_j);
    const int lane = threadIdx.x & 63;
    if (lane < k) {
      a.topk_idx[(int64_t)t * k + lane] = ts.idx;
      a.topk_scores[(int64_t)t * k + lane] = sc;
    }
  }
}

// MODE 0: out[r, n] = x_row . W[e][n]
// MODE 1: out[r, i] = silu(x_row . W[e][i]) * (x_row . W[e][n_out + i])
template <int NV, int LPR, int MODE, int BITS>
__global__ __launch_bounds__(64) void qmv_kernel(QmvArgs a) {
  constexpr int GPW = 64 / LPR;
  constexpr int WPC = BITS / 4;  // 16-byte code loads per 32-element chunk
  const int lane = threadIdx.x;
  const int grp = lane / LPR;
  const int l = lane % LPR;
  const int64_t nblk = (a.n_out + GPW - 1) / GPW;
  const int64_t r = blockIdx.x / nblk;
  if (r >= a.n_pairs) return;
  const int n = (int)(blockIdx.x % nblk) * GPW + grp;
  const bool valid = n < a.n_out;
  const int nn = valid ? n : 0;
  int e = a.experts ? a.experts[r] : 0;
  e = min(max(e, 0), a.num_experts - 1);
  const int64_t xr = a.x_rows ? (int64_t)a.x_rows[r] : r / a.x_div;
  const int K = a.K;
  const int G = K / a.group_size;
  const int64_t KW = (int64_t)K * BITS / 32;

  const int64_t rg = (int64_t)e * a.n_w + nn;
  // chunk v of lane l: elements v*32*LPR + 32l .., loads WPC*(v*LPR + l) ..
  const uint4* pg = reinterpret_cast<const uint4*>(a.w + rg * KW) + WPC * l;
  uint4 wg[NV][WPC];
#pragma unroll
  for (int v = 0; v < NV; ++v)
#pragma unroll
    for (int c = 0; c < WPC; ++c) wg[v][c] = pg[WPC * v * LPR + c];
  uint4 wu[MODE == 1 ? NV : 1][WPC];
  const int64_t ru = rg + a.n_out;
  if (MODE == 1) {
    const uint4* pu = reinterpret_cast<const uint4*>(a.w + ru * KW) + WPC * l;
#pragma unroll
    for (int v = 0; v < NV; ++v)
#pragma unroll
      for (int c = 0; c < WPC; ++c) wu[v][c] = pu[WPC * v * LPR + c];
  }
  float sg[NV], bg[NV], su[MODE == 1 ? NV : 1], bu[MODE == 1 ? NV : 1];
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    const int g = (v * 32 * LPR + l * 32) / a.group_size;
    sg[v] = bf16_to_f32(a.s[rg * G + g]);
    bg[v] = bf16_to_f32(a.b[rg * G + g]);
    if (MODE == 1) {
      su[v] = bf16_to_f32(a.s[ru * G + g]);
      bu[v] = bf16_to_f32(a.b[ru * G + g]);
    }
  }
  const uint16_t* xrow = a.x + xr * a.x_stride;
  XChunk xc[NV];
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    if (BITS == 8) load_x_chunk8(xrow + v * 32 * LPR + l * 32, xc[v]);
    else load_x_chunk(xrow + v * 32 * LPR + l * 32, xc[v]);
  }

  const uint32_t mv = magic_vgpr();
  float accg = 0.f, accu = 0.f;
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    if constexpr (BITS == 8) {
      accg += affine_chunk8(dot_chunk8(wg[v][0], wg[v][1], xc[v], mv), xc[v].sum, sg[v], bg[v]);
      if (MODE == 1) accu += affine_chunk8(dot_chunk8(wu[v][0], wu[v][1], xc[v], mv), xc[v].sum, su[v], bu[v]);
    } else {
      accg += affine_chunk(dot_chunk(wg[v][0], xc[v], mv), xc[v].sum, sg[v], bg[v]);
      if (MODE == 1) accu += affine_chunk(dot_chunk(wu[v][0], xc[v], mv), xc[v].sum, su[v], bu[v]);
    }
  }
  accg = group_sum<LPR>(accg);
  if (MODE == 1) accu = group_sum<LPR>(accu);
  if (l == 0 && valid) {
    float o = accg;
    if (MODE == 1) o = swiglu_f32(accg, accu);
    if (MODE == 0 && a.out_f32) a.out_f32[r * a.n_out + n] = o;
    else a.out[r * a.n_out + n] = (uint16_t)f32_to_bf16(o);
  }
}

// ---- whole-wave rows: the K = 2048 * NV fast path ------------------------
//
// A wave reduces eight weight rows at once; lane l owns chunks
// k = v*2048 + l*32 .. +31 of every row (NV chunks), so one 16-byte load per
// lane and chunk covers 1 KiB of a row.  The eight per-lane partials are
// reduced together: two lane-swap folds (v_permlane32_swap,
// v_permlane16_swap), a row_ror:8 fold and three DPP adds leave row q's sum
// in lanes 8q..8q+7 -- 19 operations for eight rows instead of a
// six-step shuffle tree per row.  Weight loads are non-temporal: every byte
// is used once.

__device__ __forceinline__ float as_f(uint32_t u) { return __uint_as_float(u); }
__device__ __forceinline__ uint32_t as_u(float f) { return __float_as_uint(f); }
// lanes < 32: a(l) + a(l+32); lanes >= 32: b(l-32) + b(l)
__device__ __forceinline__ float fold32(float a, float b) {
  auto r = __builtin_amdgcn_permlane32_swap(as_u(a), as_u(b), false, false);
  return as_f(r[0]) + as_f(r[1]);
}
// per 32-lane half: lanes [0,16): a(l) + a(l+16); [16,32): b(l-16) + b(l)
__device__ __forceinline__ float fold16(float a, float b) {
  auto r = __builtin_amdgcn_permlane16_swap(as_u(a), as_u(b), false, false);
  return as_f(r[0]) + as_f(r[1]);
}
// per 16-lane row: lanes [0,8): a(l) + a(l+8); [8,16): b(l-8) + b(l)
__device__ __forceinline__ float fold8(float a, float b, int lane) {
  const bool hi = lane & 8;
  const float send = hi ? a : b, keep = hi ? b : a;
  return keep + as_f(__builtin_amdgcn_update_dpp(0, as_u(send), 0x128, 0xf, 0xf, false));  // row_ror:8
}
__device__ __forceinline__ float sum8(float v) {
  v += as_f(__builtin_amdgcn_update_dpp(0, as_u(v), 0xB1, 0xf, 0xf, false));   // quad_perm 1,0,3,2
  v += as_f(__builtin_amdgcn_update_dpp(0, as_u(v), 0x4E, 0xf, 0xf, false));   // quad_perm 2,3,0,1
  v += as_f(__builtin_amdgcn_update_dpp(0, as_u(v), 0x141, 0xf, 0xf, false));  // row_half_mirror
  return v;
}
// eight per-lane partials -> 64-lane sums; lanes 8q..8q+7 hold sum q
__device__ __forceinline__ float reduce8(const float (&v)[8], int lane) {
  const float r0 = fold32(v[0], v[4]), r1 = fold32(v[1], v[5]), r2 = fold32(v[2], v[6]),
              r3 = fold32(v[3], v[7]);
  return sum8(fold8(fold16(r0, r2), fold16(r1, r3), lane));
}

__device__ __forceinline__ uint4 load_nt(const uint4* p) {
  const i32x4_t t = __builtin_nontemporal_load(reinterpret_cast<const i32x4_t*>(p));
  return make_uint4((uint32_t)t[0], (uint32_t)t[1], (uint32_t)t[2], (uint32_t)t[3]);
}

// A wave computes two row groups of RG consecutive rows (RG = 4 or 2):
// MODE 0 rows n0.. and n0 + RG.. (2*RG outputs); MODE 1 gate rows n0.. and up
// rows n_out + n0.. (RG SwiGLU outputs).  Row i of group g sits in partial
// slot 4g + i, so the transposed eight-slot reduction leaves row 4g + i in
// lanes 8(4g + i).. and each up row 32 lanes above its gate row.
// Scales and biases of the wave's rows -- four segments [array][group][RG rows][G]
// bf16 taken from the MLX arrays, RG*G/2 16-byte units -- are fetched with
// one load per lane and unit, staged once in LDS, and read back per lane for
// its own group.  The kernel's critical path is three dependent memory round
// trips (kernel arguments, the expert id, the weights), so the expert id is
// requested first, x next (it does not wait for the id), then the scales and
// biases and the codes row by row, in the order they are consumed.
#ifdef QMOE_QMV_STAMPS
// Measurement build only (libqmoe_stamps.so, never the product library):
// s_memrealtime stamps (100 MHz) of every block of qmv64_kernel, lane 0,
// kStampsPerBlock per block -- entry, kernel arguments ready, expert id ready,
// first weight row consumed, every weight row consumed and reduced, output
// store acknowledged.  A launch overwrites the stamps of its blocks.
constexpr int kStampsPerBlock = 6;
constexpr int kStampBlocks = 16384;
}  // namespace
__device__ uint64_t qmv_stamps[kStampBlocks * kStampsPerBlock];
namespace {
// A stamp is ordered after the value it names has arrived (an empty asm that
// reads the register makes the compiler wait for it there), so the stamped
// kernel keeps the product kernel's load order.
#define QMV_STAMP(var) const uint64_t var = __builtin_amdgcn_s_memrealtime()
#define QMV_AFTER_S(v) asm volatile("" ::"s"(v))
#define QMV_AFTER(v) asm volatile("" ::"v"(v))
#else
#define QMV_STAMP(var)
#define QMV_AFTER_S(v)
#define QMV_AFTER(v)
#endif

template <int NV, int TL, int MODE, int RG, int GS, bool GATHER, bool XROWS, int BITS>
__device__ __forceinline__ void qmv64_rows(const QmvArgs& a) {
  QMV_STAMP(ts_entry);
  // K = 2048 * NV + 512 * TL: NV whole chunks of 64 lanes x 32 elements and,
  // when TL > 0, a tail chunk held by lanes < 16 * TL (the others load
  // nothing and contribute zero: x = 0 there)
  constexpr int NC = NV + (TL > 0 ? 1 : 0);
  constexpr int KE = 2048 * NV + 512 * TL;
  // 8-bit codes (plain rows, no tail): a lane's 32 codes are two adjacent 16-byte units
  static_assert(BITS == 4 || (BITS == 8 && TL == 0 && MODE == 0), "8-bit: plain rows, K = 2048 * NV");
  constexpr int WPC = BITS / 4;
  static_assert(KE % (8 * GS) == 0, "16-byte scale units per row");
  constexpr int OUTS = MODE == 1 ? RG : 2 * RG;
  constexpr int G = KE / GS;            // groups per row
  constexpr int UPR = G / 8;            // 16-byte scale units per row
  constexpr int UNITS = 4 * RG * UPR;   // [array][row group][RG rows][UPR]
  constexpr int UPL = (UNITS + 63) / 64;
  __shared__ __attribute__((aligned(16))) uint16_t sbl[UNITS * 8];
  const int lane = threadIdx.x;
  const uint32_t bid = blockIdx.x;
  const uint32_t r = fast_div(bid, a.blk_div);
  const int n0 = (int)(bid - r * a.blk_div.d) * OUTS;
  QMV_AFTER_S(r);
  QMV_STAMP(ts_args);
  int e = GATHER ? a.experts[r] : 0;
  const uint32_t xr = XROWS ? (uint32_t)a.x_rows[r] : fast_div(r, a.x_divf);
  const uint16_t* xrow = a.x + (int64_t)xr * a.x_stride;
  const bool tail_lane = lane < 16 * TL;  // holds data in the tail chunk
  uint4 xa[NC][4];
#pragma unroll
  for (int v = 0; v < NC; ++v)
#pragma unroll
    for (int q = 0; q < 4; ++q)
      xa[v][q] = (v < NV || tail_lane) ? reinterpret_cast<const uint4*>(xrow + v * 2048 + lane * 32)[q]
                                       : make_uint4(0u, 0u, 0u, 0u);

  e = min(max(e, 0), a.num_experts - 1);
  QMV_AFTER_S(e);
  QMV_STAMP(ts_id);
  constexpr int64_t KW = KE * BITS / 32;
  const int64_t ebase = (int64_t)e * a.n_w;
  const int grp1 = MODE == 1 ? a.n_out + n0 : n0 + RG;
  // row of slot (group g, row i), clamped into the expert (slots past n_out are computed, not stored)
  auto row_of = [&](int g, int i) -> int64_t {
    const int n = (g == 0 ? n0 : grp1) + i;
    const int lim = MODE == 1 ? (g == 0 ? a.n_out - 1 : 2 * a.n_out - 1) : a.n_out - 1;
    return ebase + min(n, lim);
  };

  i32x4_t sbv[UPL];
#pragma unroll
  for (int j = 0; j < UPL; ++j) {
    const int u = lane + 64 * j;
    if (UNITS % 64 == 0 || u < UNITS) {
      const int seg = u / (RG * UPR), rem = u % (RG * UPR);
      const uint16_t* base = (seg >> 1) ? a.b : a.s;
      sbv[j] = *reinterpret_cast<const i32x4_t*>(base + row_of(seg & 1, rem / UPR) * G + (rem % UPR) * 8);
    }
  }
  uint4 wv[2][RG][NC][WPC];
#pragma unroll
  for (int g = 0; g < 2; ++g)
#pragma unroll
    for (int i = 0; i < RG; ++i) {
      const uint4* p = reinterpret_cast<const uint4*>(a.w + row_of(g, i) * KW) + WPC * lane;
#pragma unroll
      for (int v = 0; v < NC; ++v)
#pragma unroll
        for (int c = 0; c < WPC; ++c)
          wv[g][i][v][c] = (v < NV || tail_lane) ? load_nt(p + WPC * v * 64 + c) : make_uint4(0u, 0u, 0u, 0u);
    }
  XChunk xc[NC];
#pragma unroll
  for (int v = 0; v < NC; ++v) {
    float s = 0.f;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint4 t = xa[v][q];
      if constexpr (BITS == 8) {  // the pairing dot_chunk8 reads (load_x_chunk8)
        xc[v].p[4 * q + 0] = (t.x & 0xFFFFu) | (t.y << 16);
        xc[v].p[4 * q + 1] = (t.x >> 16) | (t.y & 0xFFFF0000u);
        xc[v].p[4 * q + 2] = (t.z & 0xFFFFu) | (t.w << 16);
        xc[v].p[4 * q + 3] = (t.z >> 16) | (t.w & 0xFFFF0000u);
      } else {
        xc[v].p[4 * q + 0] = (t.x & 0xFFFFu) | (t.z << 16);
        xc[v].p[4 * q + 1] = (t.x >> 16) | (t.z & 0xFFFF0000u);
        xc[v].p[4 * q + 2] = (t.y & 0xFFFFu) | (t.w << 16);
        xc[v].p[4 * q + 3] = (t.y >> 16) | (t.w & 0xFFFF0000u);
      }
      s += ((bf16lo(t.x) + bf16hi(t.x)) + (bf16lo(t.y) + bf16hi(t.y))) +
           ((bf16lo(t.z) + bf16hi(t.z)) + (bf16lo(t.w) + bf16hi(t.w)));
    }
    xc[v].sum = s;
  }
#pragma unroll
  for (int j = 0; j < UPL; ++j) {
    const int u = lane + 64 * j;
    if (UNITS % 64 == 0 || u < UNITS) *reinterpret_cast<i32x4_t*>(sbl + u * 8) = sbv[j];
  }
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the staged words are visible to the wave
  __builtin_amdgcn_wave_barrier();
  const uint32_t mv = magic_vgpr();
  float part[8];
#pragma unroll
  for (int q = 0; q < 8; ++q) part[q] = 0.f;
#ifdef QMOE_QMV_STAMPS
  uint64_t ts_first = 0;
#endif
#pragma unroll
  for (int g = 0; g < 2; ++g)
#pragma unroll
    for (int i = 0; i < RG; ++i) {
      float acc = 0.f;
#pragma unroll
      for (int v = 0; v < NC; ++v) {
        const int gi = min((v * 2048 + lane * 32) / GS, G - 1);  // tail lanes past K: any group (x = 0)
        const float sv = bf16_to_f32(sbl[((0 * 2 + g) * RG + i) * G + gi]);
        const float bv = bf16_to_f32(sbl[((1 * 2 + g) * RG + i) * G + gi]);
        if constexpr (BITS == 8)
          acc += affine_chunk8(dot_chunk8(wv[g][i][v][0], wv[g][i][v][WPC - 1], xc[v], mv), xc[v].sum, sv, bv);
        else
          acc += affine_chunk(dot_chunk(wv[g][i][v][0], xc[v], mv), xc[v].sum, sv, bv);
      }
      part[4 * g + i] = acc;
#ifdef QMOE_QMV_STAMPS
      if (g == 0 && i == 0) {
        QMV_AFTER(acc);
        QMV_STAMP(ts_first_);
        ts_first = ts_first_;
      }
#endif
    }
  const float t = reduce8(part, lane);  // lanes 8q..: slot q
  QMV_AFTER(t);
  QMV_STAMP(ts_reduced);
  const int q = lane >> 3;
  if (MODE == 1) {
    // gate slot q (< 4) in lanes 8q, its up slot 4 + q in lanes 8q + 32
    auto sw = __builtin_amdgcn_permlane32_swap(as_u(t), as_u(t), false, false);
    const float up = as_f(sw[1]);
    if (lane < 32 && (lane & 7) == 0 && q < RG && n0 + q < a.n_out)
      a.out[(int64_t)r * a.n_out + n0 + q] = (uint16_t)f32_to_bf16(swiglu_f32(t, up));
  } else {
    const int g = q >> 2, i = q & 3;
    const int n = (g == 0 ? n0 : grp1) + i;
    if ((lane & 7) == 0 && i < RG && n < a.n_out) {
      if (a.out_f32) a.out_f32[(int64_t)r * a.n_out + n] = t;
      else a.out[(int64_t)r * a.n_out + n] = (uint16_t)f32_to_bf16(t);
    }
  }
#ifdef QMOE_QMV_STAMPS
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  QMV_STAMP(ts_stored);
  if (lane == 0 && bid < kStampBlocks) {
    uint64_t* o = qmv_stamps + (size_t)bid * kStampsPerBlock;
    o[0] = ts_entry; o[1] = ts_args; o[2] = ts_id; o[3] = ts_first; o[4] = ts_reduced; o[5] = ts_stored;
  }
#endif
}

// 4-bit codes; the 8-bit plain-row form is its own kernel name, so the 4-bit
// kernels keep theirs in traces
template <int NV, int TL, int MODE, int RG, int GS, bool GATHER, bool XROWS>
__global__ __launch_bounds__(64) void qmv64_kernel(QmvArgs a) {
  qmv64_rows<NV, TL, MODE, RG, GS, GATHER, XROWS, 4>(a);
}
template <int NV, int RG, int GS, bool GATHER, bool XROWS>
__global__ __launch_bounds__(64) void qmv64_kernel8(QmvArgs a) {
  qmv64_rows<NV, 0, 0, RG, GS, GATHER, XROWS, 8>(a);
}

// Block id -> work item, XCD-contiguous: the hardware deals consecutive block
// ids round-robin to the 8 XCDs, so with nb % 8 == 0 item v = (b % 8) * nb/8
// + b / 8 puts consecutive items -- row groups that share 128-byte code lines
// or a 256-byte scale|bias chunk of the tile layout -- on one XCD, where the
// second reader finds the line in that XCD's L2.  A permutation of [0, nb).
__device__ __forceinline__ uint32_t xcd_item(uint32_t b, uint32_t nb) {
  return (nb & 7u) ? b : (b & 7u) * (nb >> 3) + (b >> 3);
}

// Two per-lane partials -> 64-lane sums by reduce8's tree (the same lane
// pairings at every level, so a slot summed here is bit-identical to the same
// slot summed there): lanes < 32 hold the sum of a, lanes >= 32 that of b.
__device__ __forceinline__ float reduce2(float a, float b, int lane) {
  float r = fold32(a, b);
  r = fold16(r, r);
  return sum8(fold8(r, r, lane));
}

// Fused gate_up + SwiGLU for one token (every pair reads x row 0), flat form:
// wave item b takes the kFlatRG consecutive slots f = b*kFlatRG .. of the
// n_pairs * n_out list (pair f / n_out, index f % n_out), so a wave may span
// two pairs, i.e. two experts (kFlatRG <= n_out).  Ten experts x 512 indices
// are then 1024 waves, one per SIMD of a 256-CU part, where the four-index
// waves of qmv64_kernel number 1280 and put two waves -- 16 rows of
// arithmetic -- on a quarter of the SIMDs, which finish last.  Per lane and row
// the arithmetic is qmv64_kernel's (same loads, same chunk sums), and the fifth
// slot's reduction follows reduce8's tree, so every output is bit-identical to
// that kernel's.  Slots past the list repeat its last entry and are not stored.
//
// The waves come W to a workgroup: wave w of block b is item
// xcd_item(b) * W + w, its lane is threadIdx.x % 64, its LDS staging its own
// slice, and a wave past the last item leaves at once (the kernel has no
// block-wide barrier).  Fewer, wider workgroups reach the GPU sooner: on
// workload 1's 1280-wave shape, the dependent chain arguments -> expert id ->
// first weight row -> store measured 2.86 us per launch in single-wave
// workgroups and 2.42 us in four-wave ones.
constexpr int kFlatRG = 5;
constexpr int kFlatWaves = 4;  // waves per workgroup

template <int NV, int GS, int W>
__global__ __launch_bounds__(64 * W) void qmv64_flat_kernel(QmvArgs a) {
  constexpr int KE = 2048 * NV;
  constexpr int G = KE / GS;            // groups per row
  constexpr int UPR = G / 8;            // 16-byte scale units per row
  constexpr int UNITS = 4 * kFlatRG * UPR;  // [slot][gate/up][scale/bias][UPR]
  constexpr int UPL = (UNITS + 63) / 64;
  constexpr int64_t KW = KE / 8;
  __shared__ __attribute__((aligned(16))) uint16_t sbl_w[W][UNITS * 8];
  QMV_STAMP(ts_entry);
  const int lane = threadIdx.x % 64;
  const int wave = W == 1 ? 0 : __builtin_amdgcn_readfirstlane((int)(threadIdx.x / 64));
  uint16_t* sbl = sbl_w[wave];
  // every kernel argument the wave reads, in one batch of scalar loads (left
  // alone, the compiler spreads them over three dependent round trips)
  const uint16_t* ax = a.x;
  const int32_t* aexp = a.experts;
  const uint32_t* aw = a.w;
  const uint16_t* as_ = a.s;
  const uint16_t* ab = a.b;
  uint16_t* aout = a.out;
  const int nexp = a.num_experts, n_out = a.n_out, n_w = a.n_w;
  const uint32_t npairs = (uint32_t)a.n_pairs, bd_m = a.blk_div.m, bd_s = a.blk_div.s;
  asm volatile("" ::"s"(ax), "s"(aexp), "s"(aw), "s"(as_), "s"(ab), "s"(aout), "s"(nexp), "s"(n_out), "s"(n_w),
               "s"(npairs), "s"(bd_m), "s"(bd_s));
  QMV_STAMP(ts_args);
  const FastDiv bd{(uint32_t)n_out, bd_m, bd_s};  // n_out
  const uint32_t total = npairs * (uint32_t)n_out;  // < 2^31 (host)
  // consecutive items on one XCD (xcd_item over the blocks, then the block's
  // waves): the scale and bias lines that two neighbouring waves split (five
  // rows of 64 bytes each) are then fetched into one L2, once
  // (the grid size from the batch above: gridDim.x would cost another dependent load)
  const uint32_t nitems = (total + kFlatRG - 1) / kFlatRG;
  const uint32_t item = xcd_item(blockIdx.x, (nitems + W - 1) / W) * (uint32_t)W + (uint32_t)wave;
  if (item >= nitems) return;
  const uint32_t f0 = item * (uint32_t)kFlatRG;
  const uint32_t flast = min(f0 + (uint32_t)(kFlatRG - 1), total - 1);
  const uint32_t ra = fast_div(f0, bd);
  const uint32_t rb = fast_div(flast, bd);
  uint4 xa[NV][4];
#pragma unroll
  for (int v = 0; v < NV; ++v)
#pragma unroll
    for (int q = 0; q < 4; ++q) xa[v][q] = reinterpret_cast<const uint4*>(ax + v * 2048 + lane * 32)[q];
  // the two expert ids as scalar loads while x is in flight (written as plain
  // loads after the batch above they would go through the vector path)
  int ea, eb;
  asm volatile(
      "s_load_dword %0, %2, 0x0\n\t"
      "s_load_dword %1, %3, 0x0\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&s"(ea), "=&s"(eb)
      : "s"(aexp + ra), "s"(aexp + rb)
      : "memory");
  QMV_AFTER_S(ea);
  QMV_AFTER_S(eb);
  QMV_STAMP(ts_id);
  ea = min(max(ea, 0), nexp - 1);
  eb = min(max(eb, 0), nexp - 1);
  // Slot s (0..kFlatRG-1) is list entry min(f0 + s, total - 1): in pair ra
  // below sp, in pair ra + 1 (= rb) from sp on.  Its gate (g = 0) or up (g = 1)
  // weight row, as a row index of the whole weight tensor (< 2^31: host), is
  // row_a + s or row_b + s (+ n_out for up); row_b may wrap below zero, and
  // adding s >= sp brings it back (exact modulo 2^32).
  const uint32_t fb = (ra + 1) * (uint32_t)n_out;  // list entry of the second pair's index 0
  const uint32_t sp = fb - f0;                     // >= 1
  const uint32_t smax = total - 1 - f0;
  const uint32_t row_a = (uint32_t)ea * (uint32_t)n_w + f0 - (fb - (uint32_t)n_out);
  const uint32_t row_b = (uint32_t)eb * (uint32_t)n_w + f0 - fb;
  auto slot_row = [&](uint32_t s, uint32_t g) -> uint32_t {
    const uint32_t se = min(s, smax);
    return (se < sp ? row_a : row_b) + se + (g ? (uint32_t)n_out : 0u);
  };

  i32x4_t sbv[UPL];
#pragma unroll
  for (int j = 0; j < UPL; ++j) {
    const int u = lane + 64 * j;
    if (UNITS % 64 == 0 || u < UNITS) {
      const uint32_t seg = (uint32_t)u / UPR, up = (uint32_t)u % UPR;  // seg = (s * 2 + g) * 2 + arr
      const uint16_t* base = (seg & 1) ? ab : as_;
      sbv[j] = *reinterpret_cast<const i32x4_t*>(base + (uint64_t)slot_row(seg >> 2, (seg >> 1) & 1) * G + up * 8);
    }
  }
  uint4 wv[2][kFlatRG][NV];
#pragma unroll
  for (int g = 0; g < 2; ++g)
#pragma unroll
    for (int s = 0; s < kFlatRG; ++s) {
      const uint4* p = reinterpret_cast<const uint4*>(aw + (uint64_t)slot_row((uint32_t)s, (uint32_t)g) * KW) + lane;
#pragma unroll
      for (int v = 0; v < NV; ++v) wv[g][s][v] = load_nt(p + v * 64);
    }
  XChunk xc[NV];
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    float sum = 0.f;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint4 t = xa[v][q];
      xc[v].p[4 * q + 0] = (t.x & 0xFFFFu) | (t.z << 16);
      xc[v].p[4 * q + 1] = (t.x >> 16) | (t.z & 0xFFFF0000u);
      xc[v].p[4 * q + 2] = (t.y & 0xFFFFu) | (t.w << 16);
      xc[v].p[4 * q + 3] = (t.y >> 16) | (t.w & 0xFFFF0000u);
      sum += ((bf16lo(t.x) + bf16hi(t.x)) + (bf16lo(t.y) + bf16hi(t.y))) +
             ((bf16lo(t.z) + bf16hi(t.z)) + (bf16lo(t.w) + bf16hi(t.w)));
    }
    xc[v].sum = sum;
  }
#pragma unroll
  for (int j = 0; j < UPL; ++j) {
    const int u = lane + 64 * j;
    if (UNITS % 64 == 0 || u < UNITS) *reinterpret_cast<i32x4_t*>(sbl + u * 8) = sbv[j];
  }
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the staged words are visible to the wave
  __builtin_amdgcn_wave_barrier();
  const uint32_t mv = magic_vgpr();
  // slots 0..3 as reduce8's eight partials (gate q, then up q at 4 + q), slot 4 apart
  float part[8], last[2];
#ifdef QMOE_QMV_STAMPS
  uint64_t ts_first = 0;
#endif
#pragma unroll
  for (int g = 0; g < 2; ++g)
#pragma unroll
    for (int s = 0; s < kFlatRG; ++s) {
      float acc = 0.f;
#pragma unroll
      for (int v = 0; v < NV; ++v) {
        const int gi = (v * 2048 + lane * 32) / GS;
        const float sv = bf16_to_f32(sbl[((s * 2 + g) * 2 + 0) * G + gi]);
        const float bv = bf16_to_f32(sbl[((s * 2 + g) * 2 + 1) * G + gi]);
        acc += affine_chunk(dot_chunk(wv[g][s][v], xc[v], mv), xc[v].sum, sv, bv);
      }
      if (s < 4) part[4 * g + s] = acc;
      else last[g] = acc;
#ifdef QMOE_QMV_STAMPS
      if (g == 0 && s == 0) {
        QMV_AFTER(acc);
        QMV_STAMP(ts_first_);
        ts_first = ts_first_;
      }
#endif
    }
  const float t = reduce8(part, lane);         // lanes 8q: gate q, lanes 8q + 32: up q (q < 4)
  const float t4 = reduce2(last[0], last[1], lane);  // lanes < 32: gate 4, lanes >= 32: up 4
  QMV_AFTER(t);
  QMV_AFTER(t4);
  QMV_STAMP(ts_reduced);
  auto sw = __builtin_amdgcn_permlane32_swap(as_u(t), as_u(t), false, false);
  auto sw4 = __builtin_amdgcn_permlane32_swap(as_u(t4), as_u(t4), false, false);
  // lane 8q stores slot q (q < 4), lane 1 slot 4
  const int q = lane >> 3;
  const bool st4 = lane == 1;
  const float gate = st4 ? t4 : t, up = as_f(st4 ? sw4[1] : sw[1]);
  const uint32_t f = f0 + (st4 ? 4u : (uint32_t)q);
  if (lane < 32 && ((lane & 7) == 0 || st4) && f < total)
    aout[f] = (uint16_t)f32_to_bf16(swiglu_f32(gate, up));
#ifdef QMOE_QMV_STAMPS
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  QMV_STAMP(ts_stored);
  if (lane == 0 && item < kStampBlocks) {
    uint64_t* o = qmv_stamps + (size_t)item * kStampsPerBlock;
    o[0] = ts_entry; o[1] = ts_args; o[2] = ts_id; o[3] = ts_first; o[4] = ts_reduced; o[5] = ts_stored;
  }
#endif
}

// qmv64 over tile-layout weights (group 64), plain row form: the code chunk of
// row n for group g, half h is 16 bytes at
// ((((e*NC + n/64)*G + g)*2 + (n%64)/32)*2 + h)*32 + n%32 (16-byte units), so
// the eight consecutive rows n0.. (n0 % 8 == 0) a wave reads at one (g, h)
// form one whole 128-byte line; their scale|bias words are 32 contiguous
// bytes of the group's 256-byte chunk, which eight consecutive items share.
// Loads are issued in the order they are consumed (x, scale|bias, then codes
// row by row) so the arithmetic starts as data lands.
template <int NV>
__global__ __launch_bounds__(64) void qmv64_tiled_kernel(QmvArgs a) {
  constexpr int OUTS = 8;
  const int lane = threadIdx.x;
  const uint32_t item = xcd_item(blockIdx.x, gridDim.x);
  const int64_t nblk = (a.n_out + OUTS - 1) / OUTS;
  const int64_t r = item / nblk;
  if (r >= a.n_pairs) return;
  const int n0 = (int)(item % nblk) * OUTS;
  int e = a.experts ? a.experts[r] : 0;
  e = min(max(e, 0), a.num_experts - 1);
  const int64_t xr = a.x_rows ? (int64_t)a.x_rows[r] : r / a.x_div;
  const int G = a.K / 64;
  const int NC = a.n_w / 64;
  const int h = lane & 1;

  const uint16_t* xrow = a.x + xr * a.x_stride;
  XChunk xc[NV];
#pragma unroll
  for (int v = 0; v < NV; ++v) load_x_chunk(xrow + v * 2048 + lane * 32, xc[v]);

  // rows n0 .. n0 + 7 (clamped into the expert; n_w % 64 == 0 keeps a clamped
  // row group inside one 32-row half)
  const int nq = min(n0, a.n_w - 8);
  uint4 sbv[2][NV];
#pragma unroll
  for (int u = 0; u < 2; ++u)
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      const int g = v * 32 + (lane >> 1);
      const int64_t chunk = ((int64_t)e * NC + nq / 64) * G + g;
      sbv[u][v] = *reinterpret_cast<const uint4*>(a.sb + chunk * 64 + (nq & 63) + 4 * u);
    }
  uint4 wv[8][NV];
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    const int n = nq + q;
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      const int g = v * 32 + (lane >> 1);
      const int64_t unit = ((((int64_t)e * NC + n / 64) * G + g) * 2 + ((n & 63) >> 5)) * 2 + h;
      wv[q][v] = load_nt(reinterpret_cast<const uint4*>(a.w) + unit * 32 + (n & 31));
    }
  }
  const uint32_t mv = magic_vgpr();
  float part[8];
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    part[q] = 0.f;
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      const uint4 sq = sbv[q >> 2][v];
      const uint32_t word = (q & 3) == 0 ? sq.x : (q & 3) == 1 ? sq.y : (q & 3) == 2 ? sq.z : sq.w;
      part[q] += affine_chunk(dot_chunk(wv[q][v], xc[v], mv), xc[v].sum, __uint_as_float(word << 16),
                              __uint_as_float(word & 0xFFFF0000u));
    }
  }
  const float t = reduce8(part, lane);  // lanes 8q..: row q
  const int q = lane >> 3;
  if ((lane & 7) == 0 && n0 + q < a.n_out) a.out[r * a.n_out + n0 + q] = (uint16_t)f32_to_bf16(t);
}

// Fused gate_up + SwiGLU over tile-layout weights in the gate/up-PAIRED row
// order of the SwiGLU grouped GEMM: the gate row of intermediate index i is
// paired row 64(i/32) + i%32 and its up row sits 32 rows below, so in the tile
// layout the two are halves j = 0 and 1 of one 64-row block, with the same row
// l = i%32 in the half.  A wave computes RG consecutive indices i0.. (RG | 32):
// per group g and half h its RG gate rows are RG*16 contiguous bytes of the
// chunk and its up rows another RG*16 (RG = 8: one whole 128-byte line each),
// and their scale|bias words RG*4 contiguous bytes each.  Items are dealt
// XCD-contiguously (xcd_item), so the row groups sharing a scale|bias chunk
// run on one XCD.  Per lane and row the arithmetic and the reduction tree are
// those of qmv64_kernel's fused form, so the result is bit-identical to it.
template <int NV, int RG, int PER = 0>
__global__ __launch_bounds__(64) void qmv64_paired_kernel(QmvArgs a) {
  static_assert(RG == 4 || RG == 8, "four or eight indices per wave");
  const int lane = threadIdx.x;
  const uint32_t item = xcd_item(blockIdx.x, gridDim.x);
  const uint32_t r = fast_div(item, a.blk_div);
  const int i0 = (int)(item - r * a.blk_div.d) * RG;
  const uint32_t xr = fast_div(r, a.x_divf);
  // the expert id is requested before x; a top-k selection goes after x's loads
  PairTopk<PER> ts;
  int e = 0;
  if constexpr (PER == 0) e = pair_expert<PER>(a, r, xr, false, ts);
  const uint16_t* xrow = a.x + (int64_t)xr * a.x_stride;
  uint4 xa[NV][4];
#pragma unroll
  for (int v = 0; v < NV; ++v)
#pragma unroll
    for (int q = 0; q < 4; ++q) xa[v][q] = reinterpret_cast<const uint4*>(xrow + v * 2048 + lane * 32)[q];
  if constexpr (PER > 0) e = pair_expert<PER>(a, r, xr, i0 == 0, ts);
  e = min(max(e, 0), a.num_experts - 1);
  const int G = 32 * NV;
  const int NC = a.n_w / 64;
  const int c = i0 >> 5, l0 = i0 & 31;
  const int h = lane & 1;
  const int64_t chunk0 = ((int64_t)e * NC + c) * G + (lane >> 1);  // chunk of the lane's group in column block c

  // scale|bias words: gate rows at l0.., up rows at 32 + l0.., RG/4 16-byte loads each
  uint4 sg[NV][RG / 4], su[NV][RG / 4];
#pragma unroll
  for (int v = 0; v < NV; ++v)
#pragma unroll
    for (int t = 0; t < RG / 4; ++t) {
      const uint32_t* base = a.sb + (chunk0 + v * 32) * 64 + l0 + 4 * t;
      sg[v][t] = *reinterpret_cast<const uint4*>(base);
      su[v][t] = *reinterpret_cast<const uint4*>(base + 32);
    }
  uint4 wg[RG][NV], wu[RG][NV];
#pragma unroll
  for (int q = 0; q < RG; ++q)
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      const uint4* units = reinterpret_cast<const uint4*>(a.w) + ((chunk0 + v * 32) * 4 + h) * 32 + l0 + q;
      wg[q][v] = load_nt(units);       // half j = 0: gate
      wu[q][v] = load_nt(units + 64);  // half j = 1: up, two 32-unit halves further
    }
  pair_topk_store<PER>(a, xr, ts);  // while the weights are in flight
  XChunk xc[NV];
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    float sum = 0.f;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint4 t = xa[v][q];
      xc[v].p[4 * q + 0] = (t.x & 0xFFFFu) | (t.z << 16);
      xc[v].p[4 * q + 1] = (t.x >> 16) | (t.z & 0xFFFF0000u);
      xc[v].p[4 * q + 2] = (t.y & 0xFFFFu) | (t.w << 16);
      xc[v].p[4 * q + 3] = (t.y >> 16) | (t.w & 0xFFFF0000u);
      sum += ((bf16lo(t.x) + bf16hi(t.x)) + (bf16lo(t.y) + bf16hi(t.y))) +
             ((bf16lo(t.z) + bf16hi(t.z)) + (bf16lo(t.w) + bf16hi(t.w)));
    }
    xc[v].sum = sum;
  }
  const uint32_t mv = magic_vgpr();
  auto word_of = [](const uint4& u, int k) { return k == 0 ? u.x : k == 1 ? u.y : k == 2 ? u.z : u.w; };
#pragma unroll
  for (int b = 0; b < RG / 4; ++b) {
    // slots 0..3: gate rows 4b.., 4..7: their up rows
    float part[8];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      float pg = 0.f, pu = 0.f;
#pragma unroll
      for (int v = 0; v < NV; ++v) {
        const uint32_t wgs = word_of(sg[v][b], q), wus = word_of(su[v][b], q);
        pg += affine_chunk(dot_chunk(wg[4 * b + q][v], xc[v], mv), xc[v].sum, __uint_as_float(wgs << 16),
                           __uint_as_float(wgs & 0xFFFF0000u));
        pu += affine_chunk(dot_chunk(wu[4 * b + q][v], xc[v], mv), xc[v].sum, __uint_as_float(wus << 16),
                           __uint_as_float(wus & 0xFFFF0000u));
      }
      part[q] = pg;
      part[4 + q] = pu;
    }
    const float t = reduce8(part, lane);  // lanes 8q..: slot q
    // gate slot q (< 4) in lanes 8q, its up slot 4 + q in lanes 8q + 32
    auto sw = __builtin_amdgcn_permlane32_swap(as_u(t), as_u(t), false, false);
    const float up = as_f(sw[1]);
    const int q = lane >> 3;
    if (lane < 32 && (lane & 7) == 0)
      a.out[(int64_t)r * a.n_out + i0 + 4 * b + q] = (uint16_t)f32_to_bf16(swiglu_f32(t, up));
  }
}

// Fused gate_up + SwiGLU over the gate/up-paired tile layout with line reads:
// a wave computes RG indices i0 .. (gate rows l0 .. l0 + RG - 1 of half j = 0
// of column block c = i0 / 32, up rows in half j = 1).  Lane 8r + s holds row
// slot r and group slot s; its load (p, h) reads the 16-byte unit
// (g = 8p + s, j, h, l0 + rr) of its row, so the lanes of one group slot read
// consecutive rows of one (g, j, h): RG = 8 gives each slot two whole 128-byte
// lines (rows of gate and of up, r = 0..7 each), RG = 4 one 64-byte half-line
// of gate rows (r < 4) and one of up rows (r >= 4), whose other halves the
// XCD-adjacent item reads.  x changes with the group, so the wave stages its x
// row in LDS once (per 32-element chunk: the 16 bf16 pairs matched to the
// nibble pairs, and the chunk's sum) and each lane reads the chunk of its
// (g, h) per step.  Per lane the affine chunk arithmetic is qmv64_kernel's;
// the row sums close over the eight group slots with three DPP steps.
template <int NV, int RG, int PER = 0>
__global__ __launch_bounds__(64) void qmv64_paired_lines_kernel(QmvArgs a) {
  static_assert(RG == 4 || RG == 8, "four or eight indices per wave");
  constexpr int NCH = 64 * NV;   // 32-element chunks of x
  constexpr int NP = 4 * NV;     // group steps per lane: g = 8p + s
  constexpr int NJ = RG / 4;     // row halves a lane reads: both (RG = 8) or its own (RG = 4)
  __shared__ uint4 xl[4][NCH];   // quarter q of chunk c at xl[q][c]: 16-byte reads of 8 chunks hit distinct banks
  __shared__ float xsum[NCH];
  const int lane = threadIdx.x;
  const int r = lane >> 3, sl = lane & 7;
  const int jr = RG == 8 ? 0 : r >> 2;        // RG = 4: the lane's half (gate or up)
  const int rr = RG == 8 ? r : (r & 3);       // row within the wave's RG rows
  const uint32_t item = xcd_item(blockIdx.x, gridDim.x);
  const uint32_t pr = fast_div(item, a.blk_div);
  const int i0 = (int)(item - pr * a.blk_div.d) * RG;
  const uint32_t xr = fast_div(pr, a.x_divf);
  // the expert id is requested before x; a top-k selection goes after x's loads
  PairTopk<PER> ts;
  int e = 0;
  if constexpr (PER == 0) e = pair_expert<PER>(a, pr, xr, false, ts);
  const uint16_t* xrow = a.x + (int64_t)xr * a.x_stride;
  uint4 xa[NV][4];
#pragma unroll
  for (int v = 0; v < NV; ++v)
#pragma unroll
    for (int q = 0; q < 4; ++q) xa[v][q] = reinterpret_cast<const uint4*>(xrow + v * 2048 + lane * 32)[q];
  if constexpr (PER > 0) e = pair_expert<PER>(a, pr, xr, i0 == 0, ts);
  e = min(max(e, 0), a.num_experts - 1);
  const int G = 32 * NV;
  const int NC = a.n_w / 64;
  const int c = i0 >> 5, l0 = i0 & 31;
  const int64_t cbase = ((int64_t)e * NC + c) * G;  // chunk of group 0 in column block c

  uint32_t sbw[NP][NJ];
  uint4 wv[NP][2][NJ];  // [step][h][row half]
#pragma unroll
  for (int pp = 0; pp < NP; ++pp) {
    const uint32_t* sbc = a.sb + (cbase + 8 * pp + sl) * 64 + l0 + rr;
#pragma unroll
    for (int jj = 0; jj < NJ; ++jj) sbw[pp][jj] = sbc[32 * (jr + jj)];
  }
#pragma unroll
  for (int pp = 0; pp < NP; ++pp)
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int jj = 0; jj < NJ; ++jj) {
        const int64_t chunk = cbase + 8 * pp + sl;
        wv[pp][h][jj] = load_nt(reinterpret_cast<const uint4*>(a.w) + ((chunk * 2 + jr + jj) * 2 + h) * 32 + l0 + rr);
      }
  pair_topk_store<PER>(a, xr, ts);  // while the weights are in flight
  // stage x: lane l writes chunk v*64 + l (elements v*2048 + 32l ..)
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    uint32_t pw[16];
    float sum = 0.f;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint4 t = xa[v][q];
      pw[4 * q + 0] = (t.x & 0xFFFFu) | (t.z << 16);
      pw[4 * q + 1] = (t.x >> 16) | (t.z & 0xFFFF0000u);
      pw[4 * q + 2] = (t.y & 0xFFFFu) | (t.w << 16);
      pw[4 * q + 3] = (t.y >> 16) | (t.w & 0xFFFF0000u);
      sum += ((bf16lo(t.x) + bf16hi(t.x)) + (bf16lo(t.y) + bf16hi(t.y))) +
             ((bf16lo(t.z) + bf16hi(t.z)) + (bf16lo(t.w) + bf16hi(t.w)));
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) xl[q][v * 64 + lane] = make_uint4(pw[4 * q], pw[4 * q + 1], pw[4 * q + 2], pw[4 * q + 3]);
    xsum[v * 64 + lane] = sum;
  }
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the staged x is visible to the wave
  __builtin_amdgcn_wave_barrier();
  const uint32_t mv = magic_vgpr();
  float acc[NJ];
#pragma unroll
  for (int jj = 0; jj < NJ; ++jj) acc[jj] = 0.f;
#pragma unroll
  for (int pp = 0; pp < NP; ++pp) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int ch = 2 * (8 * pp + sl) + h;  // chunk of (g, h)
      XChunk xc;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint4 t = xl[q][ch];
        xc.p[4 * q + 0] = t.x;
        xc.p[4 * q + 1] = t.y;
        xc.p[4 * q + 2] = t.z;
        xc.p[4 * q + 3] = t.w;
      }
      xc.sum = xsum[ch];
#pragma unroll
      for (int jj = 0; jj < NJ; ++jj)
        acc[jj] += affine_chunk(dot_chunk(wv[pp][h][jj], xc, mv), xc.sum, __uint_as_float(sbw[pp][jj] << 16),
                                __uint_as_float(sbw[pp][jj] & 0xFFFF0000u));
    }
  }
  float gate, up;
  if constexpr (RG == 8) {
    gate = sum8(acc[0]);
    up = sum8(acc[1]);
  } else {
    // lanes 8r, r < 4: gate row r; r >= 4: up row r - 4, 32 lanes above
    const float t = sum8(acc[0]);
    auto sw = __builtin_amdgcn_permlane32_swap(as_u(t), as_u(t), false, false);
    gate = t;
    up = as_f(sw[1]);
  }
  if (sl == 0 && r < RG)
    a.out[(int64_t)pr * a.n_out + i0 + r] = (uint16_t)f32_to_bf16(swiglu_f32(gate, up));
}

struct DownArgs {
  const uint16_t* h;  // [T, k, I]
  const int32_t* idx; // [T, k]
  const float* scores;
  int T, k, I, group_size;
  const uint32_t* w;  // [E, D, I/8]
  const uint16_t* s;
  const uint16_t* b;
  int num_experts, D;
  uint16_t* y;  // [T, D]
  const uint32_t* sb;  // tile layout: scale|bias words (w then holds the tile-layout codes)
};

// One block per group of 64/LPR output rows; wave t handles token t and walks
// its k experts, folding the router score into the lane partial so a single
// group reduction ends the row (fused_kernels.py:93-169 structure).  The
// waves of a block read the same rows of whichever experts their tokens share.
constexpr int kJB = 5;  // experts whose loads are issued together

template <int NV, int LPR>
__global__ __launch_bounds__(1024) void down_wsum_kernel(DownArgs a) {
  constexpr int GPW = 64 / LPR;
  const int t = threadIdx.x / 64;
  const int lane = threadIdx.x % 64;
  const int grp = lane / LPR;
  const int l = lane % LPR;
  const int d = blockIdx.x * GPW + grp;
  const bool valid = d < a.D;
  const int dd = valid ? d : 0;
  const int I = a.I;
  const int G = I / a.group_size;
  const int64_t KW = I / 8;
  const uint32_t mv = magic_vgpr();
  float acc = 0.f;
  for (int j0 = 0; j0 < a.k; j0 += kJB) {
    uint4 wv[kJB][NV];
    float sv[kJB][NV], bv[kJB][NV], sc[kJB];
    int64_t prow[kJB];
#pragma unroll
    for (int jj = 0; jj < kJB; ++jj) {
      const int j = min(j0 + jj, a.k - 1);
      const int p = t * a.k + j;
      int e = a.idx[p];
      e = min(max(e, 0), a.num_experts - 1);
      sc[jj] = (j0 + jj < a.k) ? a.scores[p] : 0.f;
      prow[jj] = p;
      const int64_t row = (int64_t)e * a.D + dd;
      const uint4* pw = reinterpret_cast<const uint4*>(a.w + row * KW) + l;
#pragma unroll
      for (int v = 0; v < NV; ++v) {
        wv[jj][v] = pw[v * LPR];
        const int g = (v * 32 * LPR + l * 32) / a.group_size;
        sv[jj][v] = bf16_to_f32(a.s[row * G + g]);
        bv[jj][v] = bf16_to_f32(a.b[row * G + g]);
      }
    }
#pragma unroll
    for (int jj = 0; jj < kJB; ++jj) {
      if (j0 + jj >= a.k) break;  // uniform across the block
      const uint16_t* hrow = a.h + prow[jj] * I;
      float part = 0.f;
#pragma unroll
      for (int v = 0; v < NV; ++v) {
        XChunk hc;
        load_x_chunk(hrow + v * 32 * LPR + l * 32, hc);
        part += affine_chunk(dot_chunk(wv[jj][v], hc, mv), hc.sum, sv[jj][v], bv[jj][v]);
      }
      acc += sc[jj] * part;
    }
  }
  acc = group_sum<LPR>(acc);
  if (l == 0 && valid) a.y[(int64_t)t * a.D + d] = (uint16_t)f32_to_bf16(acc);
}

// Fused down + weighted sum for I = 512, pair-parallel: one block per
// (token t, R output rows), one wave per expert slot j of the token (k waves).
// Lane (rg = lane/16, l = lane%16) owns 32-code chunk l of rows d0 + 4i + rg
// (i < R/4), so each 16-byte load instruction reads four consecutive 256-byte
// rows.  A wave streams only its own expert's R rows (R * 288 bytes), which
// puts k waves per row block in flight: at one token, 2560 waves where a wave
// per (token, row block) walking all k experts gives 256 and is latency-bound.
// The pair's h chunk is loaded before the expert id (it does not depend on
// it); the slots' score-weighted row values meet in LDS and are summed in
// slot order, so the result is deterministic (fused_kernels.py:93-169
// arithmetic: fp32 throughout, one bf16 rounding).  Tokens that share an
// expert read its rows from L2 or the Infinity Cache.
constexpr int kPairMaxK = 16;

template <int R>
__global__ __launch_bounds__(64 * kPairMaxK) void down_pair_kernel(DownArgs a) {
  constexpr int NI = R / 4;
  __shared__ float red[kPairMaxK][R];
  const int t = blockIdx.y;
  const int j = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int rg = lane >> 4, l = lane & 15;
  const int d0 = blockIdx.x * R;
  const int D = a.D;
  const int G = 512 / a.group_size;
  const int gi = (l * 32) / a.group_size;
  const int64_t p = (int64_t)t * a.k + j;
  // the pair's h chunk first: it does not wait for the expert id
  XChunk hc;
  load_x_chunk(a.h + p * 512 + l * 32, hc);
  int e = a.idx[p];
  e = min(max(e, 0), a.num_experts - 1);
  const float sc = a.scores[p];
  uint4 wq[NI];
  uint16_t sv[NI], bv[NI];
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int64_t row = (int64_t)e * D + min(d0 + 4 * i + rg, D - 1);
    wq[i] = load_nt(reinterpret_cast<const uint4*>(a.w + row * 64) + l);
    sv[i] = a.s[row * G + gi];
    bv[i] = a.b[row * G + gi];
  }
  const uint32_t mv = magic_vgpr();
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const float v = group_sum<16>(affine_chunk(dot_chunk(wq[i], hc, mv), hc.sum, bf16_to_f32(sv[i]),
                                               bf16_to_f32(bv[i])));
    if (l == 0) red[j][4 * i + rg] = sc * v;
  }
  __syncthreads();
  if (threadIdx.x < R) {
    float y = 0.f;
    for (int jj = 0; jj < a.k; ++jj) y += red[jj][threadIdx.x];
    const int d = d0 + threadIdx.x;
    if (d < D) a.y[(int64_t)t * D + d] = (uint16_t)f32_to_bf16(y);
  }
}

// down_pair_kernel over tile-layout down weights [E, D, I = 512] (group 64,
// G = 8): lane (rg, l) reads the 16-byte unit (g = l / 2, h = l % 2) of rows
// d0 + 4i + rg, which is the same 32 codes its MLX-layout counterpart reads,
// so the result is bit-identical to it.  One load instruction covers four
// consecutive rows (64 contiguous bytes per (g, h)); the R rows of a wave
// (d0 % R == 0, R | 32) fill whole 128-byte lines across its R/4 loads, which
// are ordinary (cached) loads so the later ones find the lines the first ones
// brought in.  The wave's scale|bias words (R per group, consecutive in the
// group's 256-byte chunk) arrive in one coalesced load and are moved to the
// lanes that need them across rows: with R = 16, lane row rg loads words
// 4rg..4rg+3 and two permlane32 and two permlane16 swaps transpose that 4 x 4
// block so VGPR i holds word 4i + rg; with R = 8, lane (rg, h) loads word
// rg + 4h and swaps it with its h neighbour.  (Four scattered 4-byte loads per
// wave instead, each touching eight chunks, cost 17-23% of the kernel at 8
// and 16 tokens.  Eight lanes per line with two h chunks per lane measured
// slower: every wave then reads twice the h row.)
template <int R>
__global__ __launch_bounds__(64 * kPairMaxK) void down_pair_tiled_kernel(DownArgs a) {
  constexpr int NI = R / 4;
  __shared__ float red[kPairMaxK][R];
  const int t = blockIdx.y;
  const int j = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int rg = lane >> 4, l = lane & 15;
  const int d0 = blockIdx.x * R;
  const int D = a.D;
  const int NCd = D / 64;
  const int g = l >> 1, h = l & 1;
  const int64_t p = (int64_t)t * a.k + j;
  XChunk hc;
  load_x_chunk(a.h + p * 512 + l * 32, hc);
  int e = a.idx[p];
  e = min(max(e, 0), a.num_experts - 1);
  const float sc = a.scores[p];
  static_assert(R == 8 || R == 16, "rows per wave");
  // D % 64 == 0 and d0 % R == 0: the wave's rows lie in one 64-row chunk
  const int64_t chunk = ((int64_t)e * NCd + (d0 >> 6)) * 8 + g;
  const uint32_t* sbg = a.sb + chunk * 64 + (d0 & 63);
  uint4 sq;
  uint32_t s1;
  if constexpr (NI == 4) sq = *reinterpret_cast<const uint4*>(sbg + 4 * rg);
  else s1 = sbg[rg + 4 * h];
  uint4 wq[NI];
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int row = d0 + 4 * i + rg;
    wq[i] = *(reinterpret_cast<const uint4*>(a.w) + ((chunk * 2 + ((row >> 5) & 1)) * 2 + h) * 32 + (row & 31));
  }
  uint32_t sbw[NI];  // the scale|bias word of row d0 + 4i + rg, group g
  if constexpr (NI == 4) {
    // lane row r holds M[r][c] = word 4r + c; after the swaps VGPR i holds M[i][r]
    const auto x02 = __builtin_amdgcn_permlane32_swap(sq.x, sq.z, false, false);  // rows 2,3 of c0/c1 <-> rows 0,1 of c2/c3
    const auto x13 = __builtin_amdgcn_permlane32_swap(sq.y, sq.w, false, false);
    const auto y01 = __builtin_amdgcn_permlane16_swap(x02[0], x13[0], false, false);  // odd rows <-> even rows
    const auto y23 = __builtin_amdgcn_permlane16_swap(x02[1], x13[1], false, false);
    sbw[0] = y01[0];
    sbw[1] = y01[1];
    sbw[2] = y23[0];
    sbw[3] = y23[1];
  } else {
    const uint32_t o = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)s1, 0xB1, 0xf, 0xf, false);  // lane ^ 1
    sbw[0] = h ? o : s1;
    sbw[1] = h ? s1 : o;
  }
  const uint32_t mv = magic_vgpr();
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const float v = group_sum<16>(affine_chunk(dot_chunk(wq[i], hc, mv), hc.sum, __uint_as_float(sbw[i] << 16),
                                               __uint_as_float(sbw[i] & 0xFFFF0000u)));
    if (l == 0) red[j][4 * i + rg] = sc * v;
  }
  __syncthreads();
  if (threadIdx.x < R) {
    float y = 0.f;
    for (int jj = 0; jj < a.k; ++jj) y += red[jj][threadIdx.x];
    const int d = d0 + threadIdx.x;
    if (d < D) a.y[(int64_t)t * D + d] = (uint16_t)f32_to_bf16(y);
  }
}

// Pick lanes-per-row and chunks-per-lane for a reduction length K.
bool pick_split(int64_t K, int* lpr, int* nv) {
  *lpr = 0;
  *nv = 0;
  if (K <= 0 || K % 32) return false;
  const int64_t chunks = K / 32;
  for (int L : {16, 8, 4}) {
    if (chunks % L == 0 && chunks / L >= 1 && chunks / L <= 8) {
      *lpr = L;
      *nv = (int)(chunks / L);
      return true;
    }
  }
  return false;
}

template <int MODE, int RG, int NV, int TL, int GS, int BITS = 4>
int launch_qmv64_k(const QmvArgs& a, dim3 grid, hipStream_t st) {
  if constexpr (BITS == 8) {
    static_assert(MODE == 0 && TL == 0, "8-bit codes: plain rows, K = 2048 * NV");
    if (!a.experts) qmv64_kernel8<NV, RG, GS, false, false><<<grid, dim3(64), 0, st>>>(a);
    else if (a.x_rows) qmv64_kernel8<NV, RG, GS, true, true><<<grid, dim3(64), 0, st>>>(a);
    else qmv64_kernel8<NV, RG, GS, true, false><<<grid, dim3(64), 0, st>>>(a);
    return qmoe::launch_status("qmv64_kernel8");
  }
  if (MODE == 1) {
    qmv64_kernel<NV, TL, MODE, RG, GS, true, false><<<grid, dim3(64), 0, st>>>(a);
  } else if (!a.experts) {
    qmv64_kernel<NV, TL, MODE, RG, GS, false, false><<<grid, dim3(64), 0, st>>>(a);
  } else if (a.x_rows) {
    qmv64_kernel<NV, TL, MODE, RG, GS, true, true><<<grid, dim3(64), 0, st>>>(a);
  } else {
    qmv64_kernel<NV, TL, MODE, RG, GS, true, false><<<grid, dim3(64), 0, st>>>(a);
  }
  return qmoe::launch_status("qmv64_kernel");
}

// K = 2048 * NV + 512 * TL; tails (TL > 0) are instantiated for group 64 only
template <int MODE, int RG, int NV, int TL, int BITS = 4>
int launch_qmv64_tl(const QmvArgs& a, dim3 grid, hipStream_t st) {
  if constexpr (TL == 0) {
    switch (a.group_size) {
      case 32: return launch_qmv64_k<MODE, RG, NV, 0, 32, BITS>(a, grid, st);
      case 64: return launch_qmv64_k<MODE, RG, NV, 0, 64, BITS>(a, grid, st);
      default: return launch_qmv64_k<MODE, RG, NV, 0, 128, BITS>(a, grid, st);
    }
  } else {
    return launch_qmv64_k<MODE, RG, NV, TL, 64>(a, grid, st);
  }
}

template <int MODE, int RG, int NV>
int launch_qmv64_nv(const QmvArgs& a, dim3 grid, hipStream_t st) {
  switch ((a.K % 2048) / 512) {
    case 0: return launch_qmv64_tl<MODE, RG, NV, 0>(a, grid, st);
    case 1: return launch_qmv64_tl<MODE, RG, NV, 1>(a, grid, st);
    case 2: return launch_qmv64_tl<MODE, RG, NV, 2>(a, grid, st);
    default: return launch_qmv64_tl<MODE, RG, NV, 3>(a, grid, st);
  }
}

// 8-bit codes: plain rows, K = 2048 * n
template <int RG>
int launch_qmv64_8(const QmvArgs& a, dim3 grid, hipStream_t st) {
  switch (a.K / 2048) {
    case 1: return launch_qmv64_tl<0, RG, 1, 0, 8>(a, grid, st);
    case 2: return launch_qmv64_tl<0, RG, 2, 0, 8>(a, grid, st);
    case 3: return launch_qmv64_tl<0, RG, 3, 0, 8>(a, grid, st);
    default: return launch_qmv64_tl<0, RG, 4, 0, 8>(a, grid, st);
  }
}

template <int MODE, int RG>
int launch_qmv64(const QmvArgs& a, dim3 grid, hipStream_t st) {
  switch (a.K / 2048) {
    case 1: return launch_qmv64_nv<MODE, RG, 1>(a, grid, st);
    case 2: return launch_qmv64_nv<MODE, RG, 2>(a, grid, st);
    case 3: return launch_qmv64_nv<MODE, RG, 3>(a, grid, st);
    default: return launch_qmv64_nv<MODE, RG, 4>(a, grid, st);
  }
}

// Shapes the 2048-chunk GEMV takes: K = 2048 * n + 512 * t (1 <= n <= 4,
// t < 4, and t == 0 unless group_size == 64) with 4-bit codes; K = 2048 * n
// with 8-bit codes (plain rows only).
bool qmv64_shape(int64_t K, int group_size, int bits) {
  if (K < 2048 || K % 512 || K / 2048 > 4) return false;
  if (bits == 8) return K % 2048 == 0;
  if (bits != 4) return false;
  return K % 2048 == 0 || group_size == 64;
}

// SIMDs of the current device (four per CU), looked up once.
int simd_count() {
  static int simds = 0;
  if (!simds) {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) == hipSuccess && hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess)
      simds = 4 * n;
    if (simds <= 0) simds = 1024;
  }
  return simds;
}

// One token's fused gate_up on qmv64_flat_kernel when that lowers the rows of
// arithmetic on the busiest SIMD: waves of RG indices compute 2 * RG rows, and
// ceil(waves / SIMDs) of them share a SIMD.  Returns -1 when the flat form does
// not apply or is no better.
// The one-token flat form where its shape rules hold and it puts fewer rows
// on the busiest SIMD than the four-index waves; QMOE_DECODE_FLAT=0 turns it
// off and QMOE_DECODE_FLAT=1 takes it wherever the shape allows (both results
// are bit-identical; tests pin the dispatch with it).  -1: not taken.
int launch_qmv_flat(const QmvArgs& a, hipStream_t st) {
  const char* env = getenv("QMOE_DECODE_FLAT");
  const int force = env && env[0] ? (env[0] == '1' ? 1 : 0) : -1;
  if (force == 0) return -1;
  if (a.x_rows || a.n_pairs != a.x_div || a.n_out < kFlatRG || a.K % 2048) return -1;
  const int64_t total = a.n_pairs * (int64_t)a.n_out;
  if (total <= 0 || total > 0x7FFFFFFF || (int64_t)a.num_experts * a.n_w > 0x7FFFFFFF) return -1;
  const int64_t S = simd_count();
  const int64_t waves4 = a.n_pairs * ((a.n_out + QMOE_QMV_RG_GU - 1) / QMOE_QMV_RG_GU);
  const int64_t waves5 = (total + kFlatRG - 1) / kFlatRG;
  if (force != 1 && (waves5 + S - 1) / S * (2 * kFlatRG) >= (waves4 + S - 1) / S * (2 * QMOE_QMV_RG_GU)) return -1;
  QmvArgs b = a;
  b.blk_div = make_fastdiv((uint32_t)a.n_out);
  dim3 grid((unsigned)((waves5 + kFlatWaves - 1) / kFlatWaves)), block(64 * kFlatWaves);
#define QMV_FLAT(NV_, GS_) \
  if (a.K == 2048 * NV_ && a.group_size == GS_) { \
    qmv64_flat_kernel<NV_, GS_, kFlatWaves><<<grid, block, 0, st>>>(b); \
    return qmoe::launch_status("qmv64_flat_kernel"); \
  }
#define QMV_FLAT_GS(NV_) QMV_FLAT(NV_, 32) QMV_FLAT(NV_, 64) QMV_FLAT(NV_, 128)
  QMV_FLAT_GS(1) QMV_FLAT_GS(2) QMV_FLAT_GS(3) QMV_FLAT_GS(4)
#undef QMV_FLAT_GS
#undef QMV_FLAT
  return -1;
}

template <int MODE>
int launch_qmv(const QmvArgs& a, int lpr, int nv, hipStream_t st, int bits = 4) {
  // qmv64 reads scales and biases 16 bytes at a time: G % 8 == 0 and aligned arrays
  const bool sb_ok = (a.K / a.group_size) % 8 == 0 && qmoe::aligned16(a.s) && qmoe::aligned16(a.b);
  if (qmv64_shape(a.K, a.group_size, bits) && (sb_ok || lpr == 0)) {
    if (!sb_ok) return qmoe::fail(QMOE_ERR_UNSUPPORTED, "scales and biases must be 16-byte aligned");
    if constexpr (MODE == 1) {
      if (bits == 4) {
        const int rc = launch_qmv_flat(a, st);
        if (rc >= 0) return rc;
      }
    }
    constexpr int RG = MODE == 1 ? QMOE_QMV_RG_GU : QMOE_QMV_RG_DENSE;
    constexpr int outs = MODE == 1 ? RG : 2 * RG;
    const int64_t nblk = (a.n_out + outs - 1) / outs;
    const int64_t blocks = a.n_pairs * nblk;
    if (blocks <= 0) return QMOE_OK;
    if (blocks > 0x7FFFFFFF) return qmoe::fail(QMOE_ERR_UNSUPPORTED, "grid too large");
    if (!a.x_rows && (a.x_div < 1 || a.x_div > 0x7FFFFFFF))
      return qmoe::fail(QMOE_ERR_INVALID, "x_div=%lld out of range", (long long)a.x_div);
    QmvArgs b = a;
    b.blk_div = make_fastdiv((uint32_t)nblk);
    b.x_divf = make_fastdiv(a.x_rows ? 1u : (uint32_t)a.x_div);
    dim3 grid((unsigned)blocks), block(64);
    if (bits == 8) {
      if constexpr (MODE == 0) return launch_qmv64_8<RG>(b, grid, st);
      return qmoe::fail(QMOE_ERR_UNSUPPORTED, "8-bit codes: plain rows only");
    }
    return launch_qmv64<MODE, RG>(b, grid, st);
  }
  const int gpw = 64 / lpr;
  const int64_t nblk = (a.n_out + gpw - 1) / gpw;
  const int64_t blocks = a.n_pairs * nblk;
  if (blocks <= 0) return QMOE_OK;
  if (blocks > 0x7FFFFFFF) return qmoe::fail(QMOE_ERR_UNSUPPORTED, "grid too large (%lld blocks)", (long long)blocks);
  dim3 grid((unsigned)blocks), block(64);
#define QMV_CASE(NV_, L_, B_) \
  if (nv == NV_ && lpr == L_) { qmv_kernel<NV_, L_, MODE, B_><<<grid, block, 0, st>>>(a); return qmoe::launch_status("qmv_kernel"); }
#define QMV_NV(L_, B_) QMV_CASE(1, L_, B_) QMV_CASE(2, L_, B_) QMV_CASE(3, L_, B_) QMV_CASE(4, L_, B_) \
  QMV_CASE(5, L_, B_) QMV_CASE(6, L_, B_) QMV_CASE(7, L_, B_) QMV_CASE(8, L_, B_)
  if constexpr (MODE == 0) {
    // 8-bit codes: the plain row form only (quantized_matmul, gather_qmv)
    if (bits == 8) {
      QMV_NV(16, 8) QMV_NV(8, 8) QMV_NV(4, 8)
      return qmoe::fail(QMOE_ERR_UNSUPPORTED, "no 8-bit qmv kernel for lpr=%d nv=%d", lpr, nv);
    }
  }
  QMV_NV(16, 4) QMV_NV(8, 4) QMV_NV(4, 4)
#undef QMV_NV
#undef QMV_CASE
  return qmoe::fail(QMOE_ERR_UNSUPPORTED, "no qmv kernel for lpr=%d nv=%d", lpr, nv);
}

int launch_qmv_tiled(const QmvArgs& a, hipStream_t st) {
  const int64_t blocks = a.n_pairs * ((a.n_out + 7) / 8);
  if (blocks <= 0) return QMOE_OK;
  if (blocks > 0x7FFFFFFF) return qmoe::fail(QMOE_ERR_UNSUPPORTED, "grid too large");
  dim3 grid((unsigned)blocks), block(64);
  switch (a.K / 2048) {
    case 1: qmv64_tiled_kernel<1><<<grid, block, 0, st>>>(a); break;
    case 2: qmv64_tiled_kernel<2><<<grid, block, 0, st>>>(a); break;
    case 3: qmv64_tiled_kernel<3><<<grid, block, 0, st>>>(a); break;
    default: qmv64_tiled_kernel<4><<<grid, block, 0, st>>>(a); break;
  }
  return qmoe::launch_status("qmv64_tiled_kernel");
}

template <int RG, int PER = 0>
int launch_qmv_paired_rg(QmvArgs a, hipStream_t st) {
  const int64_t nblk = a.n_out / RG;
  const int64_t blocks = a.n_pairs * nblk;
  if (blocks <= 0) return QMOE_OK;
  if (blocks > 0x7FFFFFFF) return qmoe::fail(QMOE_ERR_UNSUPPORTED, "grid too large");
  if (a.x_div < 1 || a.x_div > 0x7FFFFFFF) return qmoe::fail(QMOE_ERR_INVALID, "top_k out of range");
  a.blk_div = make_fastdiv((uint32_t)nblk);
  a.x_divf = make_fastdiv((uint32_t)a.x_div);
  dim3 grid((unsigned)blocks), block(64);
  switch (a.K / 2048) {
    case 1: qmv64_paired_kernel<1, RG, PER><<<grid, block, 0, st>>>(a); break;
    case 2: qmv64_paired_kernel<2, RG, PER><<<grid, block, 0, st>>>(a); break;
    default:
      if constexpr (RG == 4) {
        if (a.K / 2048 == 3) qmv64_paired_kernel<3, 4, PER><<<grid, block, 0, st>>>(a);
        else qmv64_paired_kernel<4, 4, PER><<<grid, block, 0, st>>>(a);
      } else {
        return qmoe::fail(QMOE_ERR_UNSUPPORTED, "K=%d: %d indices per wave take K <= 4096", a.K, RG);
      }
  }
  return qmoe::launch_status("qmv64_paired_kernel");
}

// K = 2048 n: RG indices per wave for n <= 2, four above (16 rows x n 16-byte
// code loads per lane would pass 256 registers)
// Indices per wave of the line-read paired kernel.
// (four measured faster than eight at the decode shapes: 5.7 against 6.1 us at
// one token x top-10 of 256 experts, hidden 2048; twice the waves in flight)
#ifndef QMOE_PAIRED_LINES_RG
#define QMOE_PAIRED_LINES_RG 4
#endif

template <int PER = 0>
int launch_qmv_paired(const QmvArgs& a, hipStream_t st) {
  if (a.K <= 4096) {
    // line reads with x staged in LDS (K = 2048 or 4096)
    constexpr int RG = QMOE_PAIRED_LINES_RG;
    QmvArgs b = a;
    const int64_t nblk = a.n_out / RG;
    const int64_t blocks = a.n_pairs * nblk;
    if (blocks <= 0) return QMOE_OK;
    if (blocks > 0x7FFFFFFF) return qmoe::fail(QMOE_ERR_UNSUPPORTED, "grid too large");
    if (a.x_div < 1 || a.x_div > 0x7FFFFFFF) return qmoe::fail(QMOE_ERR_INVALID, "top_k out of range");
    b.blk_div = make_fastdiv((uint32_t)nblk);
    b.x_divf = make_fastdiv((uint32_t)a.x_div);
    dim3 grid((unsigned)blocks), block(64);
    if (a.K == 2048) qmv64_paired_lines_kernel<1, RG, PER><<<grid, block, 0, st>>>(b);
    else qmv64_paired_lines_kernel<2, RG, PER><<<grid, block, 0, st>>>(b);
    return qmoe::launch_status("qmv64_paired_lines_kernel");
  }
  return launch_qmv_paired_rg<4, PER>(a, st);
}

int check_tiled(int64_t K, int64_t rows_per_expert, const void* x, const void* wp, const void* sb) {
  if (K % 2048 || K / 2048 > 4)
    return qmoe::fail(QMOE_ERR_UNSUPPORTED, "K=%lld: the tile-layout GEMV takes K = 2048 * n, n <= 4", (long long)K);
  if (rows_per_expert % 64)
    return qmoe::fail(QMOE_ERR_UNSUPPORTED, "%lld weight rows per expert: must be a multiple of 64",
                      (long long)rows_per_expert);
  if (rows_per_expert > 0x3FFFFFFF) return qmoe::fail(QMOE_ERR_UNSUPPORTED, "too many rows");
  if (!qmoe::aligned16(x) || !qmoe::aligned16(wp) || !qmoe::aligned16(sb))
    return qmoe::fail(QMOE_ERR_UNSUPPORTED, "x, wp and sb must be 16-byte aligned");
  return QMOE_OK;
}

// allow8: the entry point has 8-bit kernels (the plain row form): the qmv64
// fast path at K = 2048 * n, a lane split otherwise
int check_common(int64_t K, int group_size, int bits, int* lpr, int* nv, bool allow8 = false) {
  if (bits != 4 && !(allow8 && bits == 8))
    return qmoe::fail(QMOE_ERR_UNSUPPORTED, "bits=%d: this entry point has %s kernels", bits,
                      allow8 ? "4- and 8-bit" : "4-bit");
  if (group_size != 32 && group_size != 64 && group_size != 128)
    return qmoe::fail(QMOE_ERR_UNSUPPORTED, "group_size=%d: kernels take 32, 64 or 128", group_size);
  if (K % group_size) return qmoe::fail(QMOE_ERR_INVALID, "K=%lld not a multiple of group_size", (long long)K);
  // K = 2048*n + 512*t (qmv64_shape) always has the qmv64 kernel; other K need a lane split
  const bool qmv64_ok = qmv64_shape(K, group_size, bits);
  if (!pick_split(K, lpr, nv) && !qmv64_ok)
    return qmoe::fail(QMOE_ERR_UNSUPPORTED, "K=%lld: needs K = 32*L*n, L in {4,8,16}, n <= 8, or 2048*n, n <= 4",
                      (long long)K);
  return QMOE_OK;
}

}  // namespace

extern "C" int qmoe_gather_qmv(const uint16_t* x, const int32_t* x_rows, const int32_t* experts,
                               int64_t n_rows, int64_t K, const uint32_t* w,
                               const uint16_t* scales, const uint16_t* biases, int32_t num_experts,
                               int64_t N, int group_size, int bits, uint16_t* out, void* stream) {
  if (n_rows < 0 || N <= 0 || num_experts <= 0) return qmoe::fail(QMOE_ERR_INVALID, "bad sizes");
  if (n_rows == 0) return QMOE_OK;
  if (!x || !experts || !w || !scales || !biases || !out) return qmoe::fail(QMOE_ERR_INVALID, "null pointer");
  int lpr, nv;
  int rc = check_common(K, group_size, bits, &lpr, &nv, true);
  if (rc) return rc;
  if (!qmoe::aligned16(x) || !qmoe::aligned16(w)) return qmoe::fail(QMOE_ERR_UNSUPPORTED, "x and w must be 16-byte aligned");
  if (N > 0x7FFFFFFF) return qmoe::fail(QMOE_ERR_UNSUPPORTED, "N too large");
  QmvArgs a{x, K, x_rows, 1, experts, n_rows, (int)K, group_size, w, scales, biases, num_experts,
            (int)N, (int)N, out};
  return launch_qmv<0>(a, lpr, nv, qmoe::as_stream(stream), bits);
}

extern "C" int qmoe_quantized_matmul(const uint16_t* x, int64_t M, int64_t K, const uint32_t* w,
                                     const uint16_t* scales, const uint16_t* biases, int64_t N,
                                     int group_size, int bits, uint16_t* out, void* stream) {
  if (M < 0 || N <= 0) return qmoe::fail(QMOE_ERR_INVALID, "bad sizes");
  if (M == 0) return QMOE_OK;
  if (!x || !w || !scales || !biases || !out) return qmoe::fail(QMOE_ERR_INVALID, "null pointer");
  int lpr, nv;
  int rc = check_common(K, group_size, bits, &lpr, &nv, true);
  if (rc) return rc;
  if (!qmoe::aligned16(x) || !qmoe::aligned16(w)) return qmoe::fail(QMOE_ERR_UNSUPPORTED, "x and w must be 16-byte aligned");
  if (N > 0x7FFFFFFF) return qmoe::fail(QMOE_ERR_UNSUPPORTED, "N too large");
  QmvArgs a{x, K, nullptr, 1, nullptr, M, (int)K, group_size, w, scales, biases, 1, (int)N, (int)N, out};
  return launch_qmv<0>(a, lpr, nv, qmoe::as_stream(stream), bits);
}

extern "C" int qmoe_router_logits(const uint16_t* x, int64_t T, int64_t K, const uint32_t* w,
                                  const uint16_t* scales, const uint16_t* biases, int64_t E, int group_size,
                                  int bits, float* logits, void* stream) {
  if (T < 0 || E <= 0) return qmoe::fail(QMOE_ERR_INVALID, "bad sizes");
  if (T == 0) return QMOE_OK;
  if (!x || !w || !scales || !biases || !logits) return qmoe::fail(QMOE_ERR_INVALID, "null pointer");
  int lpr, nv;
  int rc = check_common(K, group_size, bits, &lpr, &nv, true);
  if (rc) return rc;
  if (!qmoe::aligned16(x) || !qmoe::aligned16(w)) return qmoe::fail(QMOE_ERR_UNSUPPORTED, "x and w must be 16-byte aligned");
  if (E > 0x7FFFFFFF) return qmoe::fail(QMOE_ERR_UNSUPPORTED, "E too large");
  QmvArgs a{x, K, nullptr, 1, nullptr, T, (int)K, group_size, w, scales, biases, 1, (int)E, (int)E, nullptr};
  a.out_f32 = logits;
  return launch_qmv<0>(a, lpr, nv, qmoe::as_stream(stream), bits);
}

extern "C" int qmoe_moe_gate_up_swiglu(const uint16_t* x, const int32_t* idx, int64_t T,
                                       int64_t top_k, int64_t K, const uint32_t* w,
                                       const uint16_t* scales, const uint16_t* biases,
                                       int32_t num_experts, int64_t I, int group_size, int bits,
                                       uint16_t* h, void* stream) {
  if (T < 0 || top_k <= 0 || I <= 0 || num_experts <= 0) return qmoe::fail(QMOE_ERR_INVALID, "bad sizes");
  if (T == 0) return QMOE_OK;
  if (!x || !idx || !w || !scales || !biases || !h) return qmoe::fail(QMOE_ERR_INVALID, "null pointer");
  int lpr, nv;
  int rc = check_common(K, group_size, bits, &lpr, &nv);
  if (rc) return rc;
  if (!qmoe::aligned16(x) || !qmoe::aligned16(w)) return qmoe::fail(QMOE_ERR_UNSUPPORTED, "x and w must be 16-byte aligned");
  if (I > 0x3FFFFFFF) return qmoe::fail(QMOE_ERR_UNSUPPORTED, "I too large");
  QmvArgs a{x, K, nullptr, top_k, idx, T * top_k, (int)K, group_size, w, scales, biases, num_experts,
            (int)I, (int)(2 * I), h};
  return launch_qmv<1>(a, lpr, nv, qmoe::as_stream(stream));
}

extern "C" int qmoe_moe_down_wsum(const uint16_t* h, const int32_t* idx, const float* scores,
                                  int64_t T, int64_t top_k, int64_t I, const uint32_t* w,
                                  const uint16_t* scales, const uint16_t* biases,
                                  int32_t num_experts, int64_t D, int group_size, int bits,
                                  uint16_t* y, void* stream) {
  if (T < 0 || top_k <= 0 || D <= 0 || num_experts <= 0) return qmoe::fail(QMOE_ERR_INVALID, "bad sizes");
  if (T == 0) return QMOE_OK;
  if (!h || !idx || !scores || !w || !scales || !biases || !y) return qmoe::fail(QMOE_ERR_INVALID, "null pointer");
  if (T > 16) return qmoe::fail(QMOE_ERR_UNSUPPORTED, "T=%lld: the fused down kernel takes at most 16 tokens", (long long)T);
  if (top_k > 64) return qmoe::fail(QMOE_ERR_UNSUPPORTED, "top_k=%lld too large", (long long)top_k);
  int lpr, nv;
  int rc = check_common(I, group_size, bits, &lpr, &nv);
  if (rc) return rc;
  if (lpr == 0) return qmoe::fail(QMOE_ERR_UNSUPPORTED, "I=%lld: no lane split for the fused down kernel", (long long)I);
  if (!qmoe::aligned16(h) || !qmoe::aligned16(w)) return qmoe::fail(QMOE_ERR_UNSUPPORTED, "h and w must be 16-byte aligned");
  if (D > 0x3FFFFFFF) return qmoe::fail(QMOE_ERR_UNSUPPORTED, "D too large");
  DownArgs a{h, idx, scores, (int)T, (int)top_k, (int)I, group_size, w, scales, biases,
             num_experts, (int)D, y};
  hipStream_t st = qmoe::as_stream(stream);
  if (I == 512 && top_k <= kPairMaxK) {
    // rows per wave: 8 for one token (more waves in flight), 16 from two on
    // (measured: 3.6 vs 4.5 us at T = 1, 11.6 vs 14.9 us at T = 8)
    const int R = T == 1 ? 8 : 16;
    dim3 grid2((unsigned)((D + R - 1) / R), (unsigned)T), block2((unsigned)(64 * top_k));
    if (R == 8) down_pair_kernel<8><<<grid2, block2, 0, st>>>(a);
    else down_pair_kernel<16><<<grid2, block2, 0, st>>>(a);
    return qmoe::launch_status("down_pair_kernel");
  }
  const int gpw = 64 / lpr;
  dim3 grid((unsigned)((D + gpw - 1) / gpw)), block((unsigned)(64 * T));
#define DW_CASE(NV_, L_) \
  if (nv == NV_ && lpr == L_) { down_wsum_kernel<NV_, L_><<<grid, block, 0, st>>>(a); return qmoe::launch_status("down_wsum_kernel"); }
#define DW_NV(L_) DW_CASE(1, L_) DW_CASE(2, L_) DW_CASE(3, L_) DW_CASE(4, L_) \
  DW_CASE(5, L_) DW_CASE(6, L_) DW_CASE(7, L_) DW_CASE(8, L_)
  DW_NV(16) DW_NV(8) DW_NV(4)
#undef DW_NV
#undef DW_CASE
  return qmoe::fail(QMOE_ERR_UNSUPPORTED, "no down kernel for lpr=%d nv=%d", lpr, nv);
}

extern "C" int qmoe_gather_qmv_tiles(const uint16_t* x, const int32_t* x_rows, const int32_t* experts,
                                     int64_t n_rows, int64_t K, const uint32_t* wp, const uint32_t* sb,
                                     int32_t num_experts, int64_t N, uint16_t* out, void* stream) {
  if (n_rows < 0 || K <= 0 || N <= 0 || num_experts <= 0) return qmoe::fail(QMOE_ERR_INVALID, "bad sizes");
  if (n_rows == 0) return QMOE_OK;
  if (!x || !wp || !sb || !out) return qmoe::fail(QMOE_ERR_INVALID, "null pointer");
  const int rc = check_tiled(K, N, x, wp, sb);
  if (rc) return rc;
  QmvArgs a{x, K, x_rows, 1, experts, n_rows, (int)K, 64, wp, nullptr, nullptr, num_experts, (int)N, (int)N,
            out, sb};
  return launch_qmv_tiled(a, qmoe::as_stream(stream));
}

extern "C" int qmoe_moe_gate_up_swiglu_tiles(const uint16_t* x, const int32_t* idx, int64_t T, int64_t top_k,
                                             int64_t K, const uint32_t* wp, const uint32_t* sb,
                                             int32_t num_experts, int64_t I, uint16_t* h, void* stream) {
  if (T < 0 || top_k <= 0 || I <= 0 || num_experts <= 0) return qmoe::fail(QMOE_ERR_INVALID, "bad sizes");
  if (T == 0) return QMOE_OK;
  if (!x || !idx || !wp || !sb || !h) return qmoe::fail(QMOE_ERR_INVALID, "null pointer");
  if (I % 32) return qmoe::fail(QMOE_ERR_UNSUPPORTED, "I=%lld: the paired layout needs I %% 32 == 0", (long long)I);
  const int rc = check_tiled(K, 2 * I, x, wp, sb);
  if (rc) return rc;
  QmvArgs a{x, K, nullptr, top_k, idx, T * top_k, (int)K, 64, wp, nullptr, nullptr, num_experts, (int)I,
            (int)(2 * I), h, sb};
  return launch_qmv_paired(a, qmoe::as_stream(stream));
}

extern "C" int qmoe_moe_down_wsum_tiles(const uint16_t* h, const int32_t* idx, const float* scores, int64_t T,
                                        int64_t top_k, int64_t I, const uint32_t* wp, const uint32_t* sb,
                                        int32_t num_experts, int64_t D, uint16_t* y, void* stream) {
  if (T < 0 || top_k <= 0 || D <= 0 || num_experts <= 0) return qmoe::fail(QMOE_ERR_INVALID, "bad sizes");
  if (T == 0) return QMOE_OK;
  if (!h || !idx || !scores || !wp || !sb || !y) return qmoe::fail(QMOE_ERR_INVALID, "null pointer");
  if (I != 512) return qmoe::fail(QMOE_ERR_UNSUPPORTED, "I=%lld: the tiled down kernel takes I = 512", (long long)I);
  if (T > 16) return qmoe::fail(QMOE_ERR_UNSUPPORTED, "T=%lld: the fused down kernel takes at most 16 tokens", (long long)T);
  if (top_k > kPairMaxK) return qmoe::fail(QMOE_ERR_UNSUPPORTED, "top_k=%lld > %d", (long long)top_k, kPairMaxK);
  if (D % 64) return qmoe::fail(QMOE_ERR_UNSUPPORTED, "D=%lld: must be a multiple of 64", (long long)D);
  if (D > 0x3FFFFFFF) return qmoe::fail(QMOE_ERR_UNSUPPORTED, "D too large");
  if (!qmoe::aligned16(h) || !qmoe::aligned16(wp) || !qmoe::aligned16(sb))
    return qmoe::fail(QMOE_ERR_UNSUPPORTED, "h, wp and sb must be 16-byte aligned");
  DownArgs a{h, idx, scores, (int)T, (int)top_k, (int)I, 64, wp, nullptr, nullptr, num_experts, (int)D, y, sb};
  hipStream_t st = qmoe::as_stream(stream);
  // rows per wave as for the MLX-layout kernel: 8 for one token, 16 from two on
  const int R = T == 1 ? 8 : 16;
  dim3 grid((unsigned)(D / R), (unsigned)T), block((unsigned)(64 * top_k));
  if (R == 8) down_pair_tiled_kernel<8><<<grid, block, 0, st>>>(a);
  else down_pair_tiled_kernel<16><<<grid, block, 0, st>>>(a);
  return qmoe::launch_status("down_pair_tiled_kernel");
}

namespace {
// Routing from logits: k <= 64 choices of at most 1024 experts (the router
// top-k's envelope), four or sixteen logits per lane.
int check_topk(const float* logits, int64_t top_k, int32_t num_experts, int* per) {
  if (!logits) return qmoe::fail(QMOE_ERR_INVALID, "null pointer");
  if (top_k > num_experts)
    return qmoe::fail(QMOE_ERR_INVALID, "top_k=%lld > num_experts=%d", (long long)top_k, num_experts);
  if (top_k > qmoe_topk::kMaxK || num_experts > 64 * qmoe_topk::kMaxPer)
    return qmoe::fail(QMOE_ERR_UNSUPPORTED, "top_k=%lld, E=%d: the in-kernel top-k takes k <= %d, E <= %d",
                      (long long)top_k, num_experts, qmoe_topk::kMaxK, 64 * qmoe_topk::kMaxPer);
  *per = num_experts <= 256 ? 4 : 16;
  return QMOE_OK;
}
}  // namespace

extern "C" int qmoe_moe_gate_up_swiglu_tiles_topk(const uint16_t* x, const float* logits, int norm, int64_t T,
                                                  int64_t top_k, int64_t K, const uint32_t* wp, const uint32_t* sb,
                                                  int32_t num_experts, int64_t I, uint16_t* h, int32_t* idx,
                                                  float* scores, void* stream) {
  if (T < 0 || top_k <= 0 || I <= 0 || num_experts <= 0) return qmoe::fail(QMOE_ERR_INVALID, "bad sizes");
  if (T == 0) return QMOE_OK;
  if (!x || !wp || !sb || !h || !idx || !scores) return qmoe::fail(QMOE_ERR_INVALID, "null pointer");
  int per = 0;
  int rc = check_topk(logits, top_k, num_experts, &per);
  if (rc) return rc;
  if (I % 32) return qmoe::fail(QMOE_ERR_UNSUPPORTED, "I=%lld: the paired layout needs I %% 32 == 0", (long long)I);
  rc = check_tiled(K, 2 * I, x, wp, sb);
  if (rc) return rc;
  QmvArgs a{x, K, nullptr, top_k, nullptr, T * top_k, (int)K, 64, wp, nullptr, nullptr, num_experts, (int)I,
            (int)(2 * I), h, sb};
  a.logits = logits;
  a.topk_idx = idx;
  a.topk_scores = scores;
  a.topk_norm = norm ? 1 : 0;
  hipStream_t st = qmoe::as_stream(stream);
  return per == 4 ? launch_qmv_paired<4>(a, st) : launch_qmv_paired<16>(a, st);
}

#ifdef QMOE_QMV_STAMPS
// Measurement build only: copies the first n stamps of qmv64_kernel's blocks
// to host memory (after the stream has finished).
extern "C" int qmoe_qmv_stamps_read(uint64_t* host, int64_t n) {
  if (!host || n < 0 || n > (int64_t)kStampBlocks * kStampsPerBlock)
    return qmoe::fail(QMOE_ERR_INVALID, "bad stamp count");
  const hipError_t e = hipMemcpyFromSymbol(host, HIP_SYMBOL(qmv_stamps), (size_t)n * sizeof(uint64_t), 0,
                                           hipMemcpyDeviceToHost);
  return e == hipSuccess ? QMOE_OK : qmoe::fail(QMOE_ERR_HIP, "hipMemcpyFromSymbol: %s", hipGetErrorString(e));
}
#endif

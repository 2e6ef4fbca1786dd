// Shared helpers for the gfx950 kernels of libqmoe.so.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "qmoe.h"

namespace qmoe {

// Thread-local error message; returns `code` so call sites can `return fail(...)`.
int fail(int code, const char* fmt, ...);
// Maps a pending HIP launch error to QMOE_ERR_HIP.
int launch_status(const char* what);

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
inline bool aligned4(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 3u) == 0; }
inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

}  // namespace qmoe

typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2_t;
typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4_t;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16_t;
typedef __attribute__((__vector_size__(4 * sizeof(int)))) int i32x4_t;
typedef __attribute__((__vector_size__(16 * sizeof(int)))) int i32x16_t;

__device__ __forceinline__ float bf16_to_f32(uint32_t h16) { return __uint_as_float(h16 << 16); }
__device__ __forceinline__ float bf16lo(uint32_t pair) { return __uint_as_float(pair << 16); }
__device__ __forceinline__ float bf16hi(uint32_t pair) { return __uint_as_float(pair & 0xFFFF0000u); }

// Round to nearest even (finite inputs; NaN stays NaN).
__device__ __forceinline__ uint32_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x007FFFFFu)) return (u >> 16) | 0x40u;
  return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}
__device__ __forceinline__ float round_bf16(float f) { return bf16_to_f32(f32_to_bf16(f)); }
// Two floats -> packed bf16 pair (low half = a), both RNE.
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  return f32_to_bf16(a) | (f32_to_bf16(b) << 16);
}

// D += dot of two bf16 pairs, fp32 accumulate (v_dot2_f32_bf16).
__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                         __builtin_bit_cast(bf16x2_t, b), c, false);
}

// v plus lane (l ^ 1), (l ^ 2), mirror-in-8 and rotate-by-8 partners: DPP
// moves within a 16-lane row, no LDS crossbar (ds_bpermute, which
// __shfl_xor lowers to, costs a memory round trip per step).
__device__ __forceinline__ float dpp_add(float v, int ctrl) {
  switch (ctrl) {  // the control word must be a constant
    case 0xB1: return v + __uint_as_float(__builtin_amdgcn_update_dpp(0u, __float_as_uint(v), 0xB1, 0xf, 0xf, false));
    case 0x4E: return v + __uint_as_float(__builtin_amdgcn_update_dpp(0u, __float_as_uint(v), 0x4E, 0xf, 0xf, false));
    case 0x141: return v + __uint_as_float(__builtin_amdgcn_update_dpp(0u, __float_as_uint(v), 0x141, 0xf, 0xf, false));
    default: return v + __uint_as_float(__builtin_amdgcn_update_dpp(0u, __float_as_uint(v), 0x128, 0xf, 0xf, false));
  }
}

// Sum over aligned groups of W lanes (W a power of two <= 64), result in
// every lane.  W <= 16 stays inside a DPP row: quad_perm 1,0,3,2 and
// 2,3,0,1 sum each quad, row_half_mirror pairs the quads of an 8-lane half,
// row_ror:8 pairs the halves of the row.
template <int W>
__device__ __forceinline__ float group_sum(float v) {
  if constexpr (W <= 16) {
    if constexpr (W >= 2) v = dpp_add(v, 0xB1);   // quad_perm 1,0,3,2
    if constexpr (W >= 4) v = dpp_add(v, 0x4E);   // quad_perm 2,3,0,1
    if constexpr (W >= 8) v = dpp_add(v, 0x141);  // row_half_mirror
    if constexpr (W >= 16) v = dpp_add(v, 0x128); // row_ror:8
    return v;
  } else {
#pragma unroll
    for (int m = W / 2; m >= 1; m >>= 1) v += __shfl_xor(v, m, W);
    return v;
  }
}

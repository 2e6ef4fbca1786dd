// Error reporting, ABI version, and the layout kernels (unpack, dequantize).
#include <stdarg.h>
#include <stdio.h>

#include "common.h"

namespace qmoe {

static thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int launch_status(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(QMOE_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
  return QMOE_OK;
}

}  // namespace qmoe

extern "C" int qmoe_abi_version(void) { return QMOE_ABI_VERSION; }
extern "C" const char* qmoe_last_error(void) { return qmoe::g_err; }

namespace {

// One thread per packed word; writes 32/bits codes, low bits first.
__global__ void unpack_kernel(const uint32_t* __restrict__ w, int64_t n_words, int bits,
                              uint8_t* __restrict__ codes) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n_words) return;
  const uint32_t v = w[i];
  const int per = 32 / bits;
  const uint32_t mask = (1u << bits) - 1u;
  for (int t = 0; t < per; ++t) codes[i * per + t] = (uint8_t)((v >> (bits * t)) & mask);
}

// One thread per packed word: bf16_rne(fmaf(q, s, b)) for each of its codes
// (titan/kernels/moe_gather_ws.py:343-344).
__global__ void dequant_kernel(const uint32_t* __restrict__ w, const uint16_t* __restrict__ s,
                               const uint16_t* __restrict__ b, int64_t rows, int64_t K,
                               int group_size, int bits, uint16_t* __restrict__ out) {
  const int per = 32 / bits;
  const int64_t words_per_row = K / per;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= rows * words_per_row) return;
  const int64_t r = i / words_per_row;
  const int64_t k0 = (i % words_per_row) * per;
  const int64_t G = K / group_size;
  const uint32_t v = w[i];
  const uint32_t mask = (1u << bits) - 1u;
  for (int t = 0; t < per; ++t) {
    const int64_t k = k0 + t;
    const float sc = bf16_to_f32(s[r * G + k / group_size]);
    const float bi = bf16_to_f32(b[r * G + k / group_size]);
    const float q = (float)((v >> (bits * t)) & mask);
    out[r * K + k] = (uint16_t)f32_to_bf16(__builtin_fmaf(q, sc, bi));
  }
}

}  // namespace

extern "C" int qmoe_unpack(const uint32_t* w, int64_t n_words, int bits, uint8_t* codes,
                           void* stream) {
  if (bits != 4 && bits != 8) return qmoe::fail(QMOE_ERR_UNSUPPORTED, "bits=%d", bits);
  if (n_words < 0) return qmoe::fail(QMOE_ERR_INVALID, "n_words < 0");
  if (n_words == 0) return QMOE_OK;
  if (!w || !codes) return qmoe::fail(QMOE_ERR_INVALID, "null pointer");
  const int64_t blocks = (n_words + 255) / 256;
  if (blocks > 0x7FFFFFFF) return qmoe::fail(QMOE_ERR_UNSUPPORTED, "too many words");
  unpack_kernel<<<dim3((unsigned)blocks), dim3(256), 0, qmoe::as_stream(stream)>>>(w, n_words, bits, codes);
  return qmoe::launch_status("unpack_kernel");
}

extern "C" int qmoe_dequantize(const uint32_t* w, const uint16_t* scales, const uint16_t* biases,
                               int64_t rows, int64_t K, int group_size, int bits, uint16_t* out,
                               void* stream) {
  if (bits != 4 && bits != 8) return qmoe::fail(QMOE_ERR_UNSUPPORTED, "bits=%d", bits);
  if (rows < 0 || K <= 0 || group_size <= 0 || K % group_size || K % (32 / bits))
    return qmoe::fail(QMOE_ERR_INVALID, "bad sizes rows=%lld K=%lld group_size=%d", (long long)rows,
                      (long long)K, group_size);
  if (rows == 0) return QMOE_OK;
  if (!w || !scales || !biases || !out) return qmoe::fail(QMOE_ERR_INVALID, "null pointer");
  const int64_t words = rows * (K / (32 / bits));
  const int64_t blocks = (words + 255) / 256;
  if (blocks > 0x7FFFFFFF) return qmoe::fail(QMOE_ERR_UNSUPPORTED, "too many words");
  dequant_kernel<<<dim3((unsigned)blocks), dim3(256), 0, qmoe::as_stream(stream)>>>(
      w, scales, biases, rows, K, group_size, bits, out);
  return qmoe::launch_status("dequant_kernel");
}

// ------------------------------------------------------------ tile repack

namespace {

// One thread per 16-byte unit of wp, in wp order (coalesced stores): unit
// u = ((((e*NC + c)*G + g)*2 + j)*2 + h)*32 + l holds words 8g + 4h .. +3 of
// row 64c + 32j + l of expert e.
__global__ void repack_codes_kernel(const uint4* __restrict__ w, uint4* __restrict__ wp, int64_t units, int64_t N,
                                    int NC, int G) {
  const int64_t u = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (u >= units) return;
  const int l = (int)(u & 31), h = (int)((u >> 5) & 1), j = (int)((u >> 6) & 1);
  const int64_t q = u >> 7;
  const int g = (int)(q % G);
  const int64_t ec = q / G;
  const int c = (int)(ec % NC);
  const int64_t e = ec / NC;
  const int64_t row = e * N + (int64_t)c * 64 + j * 32 + l;
  wp[u] = w[row * (2 * (int64_t)G) + g * 2 + h];
}

// One thread per scale|bias word, in sb order: v = ((e*NC + c)*G + g)*64 + i.
__global__ void repack_sb_kernel(const uint16_t* __restrict__ s, const uint16_t* __restrict__ b,
                                 uint32_t* __restrict__ sb, int64_t words, int64_t N, int NC, int G) {
  const int64_t v = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (v >= words) return;
  const int i = (int)(v & 63);
  const int64_t q = v >> 6;
  const int g = (int)(q % G);
  const int64_t ec = q / G;
  const int c = (int)(ec % NC);
  const int64_t e = ec / NC;
  const int64_t idx = (e * N + (int64_t)c * 64 + i) * G + g;
  sb[v] = (uint32_t)s[idx] | ((uint32_t)b[idx] << 16);
}

}  // namespace

extern "C" int qmoe_repack_tiles(const uint32_t* w, const uint16_t* scales, const uint16_t* biases,
                                 int32_t num_experts, int64_t N, int64_t K, int group_size, int bits, uint32_t* wp,
                                 uint32_t* sb, void* stream) {
  if (num_experts < 0 || N < 0 || K < 0) return qmoe::fail(QMOE_ERR_INVALID, "bad sizes");
  if ((int64_t)num_experts * N * K == 0) return QMOE_OK;
  if (!w || !scales || !biases || !wp || !sb) return qmoe::fail(QMOE_ERR_INVALID, "null pointer");
  if (bits != 4 || group_size != 64)
    return qmoe::fail(QMOE_ERR_UNSUPPORTED, "the tile layout takes 4-bit codes with group_size 64 (got %d, %d)", bits,
                      group_size);
  if (N % 64 || K % 64) return qmoe::fail(QMOE_ERR_UNSUPPORTED, "N=%lld, K=%lld: both must be multiples of 64",
                                          (long long)N, (long long)K);
  if (!qmoe::aligned16(w) || !qmoe::aligned16(wp)) return qmoe::fail(QMOE_ERR_UNSUPPORTED, "w and wp must be 16-byte aligned");
  const int64_t G = K / 64, NC = N / 64;
  if (G > 0x7FFFFFFF || NC > 0x7FFFFFFF) return qmoe::fail(QMOE_ERR_UNSUPPORTED, "sizes too large");
  const int64_t units = (int64_t)num_experts * N * G * 2;  // 16-byte units: 32 bytes per (row, group)
  const int64_t words = (int64_t)num_experts * N * G;
  hipStream_t st = qmoe::as_stream(stream);
  const int64_t bu = (units + 255) / 256, bw = (words + 255) / 256;
  if (bu > 0x7FFFFFFF || bw > 0x7FFFFFFF) return qmoe::fail(QMOE_ERR_UNSUPPORTED, "too many words");
  repack_codes_kernel<<<dim3((unsigned)bu), dim3(256), 0, st>>>(reinterpret_cast<const uint4*>(w),
                                                                 reinterpret_cast<uint4*>(wp), units, N, (int)NC,
                                                                 (int)G);
  int rc = qmoe::launch_status("repack_codes_kernel");
  if (rc != QMOE_OK) return rc;
  repack_sb_kernel<<<dim3((unsigned)bw), dim3(256), 0, st>>>(scales, biases, sb, words, N, (int)NC, (int)G);
  return qmoe::launch_status("repack_sb_kernel");
}

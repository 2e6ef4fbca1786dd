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

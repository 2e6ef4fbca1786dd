/*
 * CPU oracle for the quantized MoE gather_qmm path.  TEST INFRASTRUCTURE ONLY:
 * loaded by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg,
 * never by the product.  Built with -ffp-contract=off so that every product
 * and sum below is one IEEE operation, exactly as written.
 *
 * Which checks pin each function is listed in the test files that load it
 * (tests/test_oracle_*.py).
 */
#include "qmoe_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------ bf16 */

uint16_t orc_bf16_rne(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x007FFFFFu)) {
    return (uint16_t)((u >> 16) | 0x0040u); /* quiet NaN */
  }
  uint32_t bias = 0x7FFFu + ((u >> 16) & 1u);
  return (uint16_t)((u + bias) >> 16);
}

float orc_bf16_to_f32(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

uint16_t orc_bf16_rne_f64(double d) {
  if (isnan(d)) return 0x7FC0u;
  uint16_t sign = signbit(d) ? 0x8000u : 0u;
  double a = fabs(d);
  if (a == 0.0) return sign;
  if (isinf(a)) return (uint16_t)(sign | 0x7F80u);
  int e;
  double m = frexp(a, &e); /* a = m * 2^e, m in [0.5, 1) */
  double q, r;
  if (e - 1 >= -126) {
    q = rint(ldexp(m, 8)); /* 8 significant bits, half to even */
    r = ldexp(q, e - 8);
  } else {
    q = rint(ldexp(a, 133)); /* subnormal grid 2^-133 */
    r = ldexp(q, -133);
  }
  if (r > 3.3895313892515355e38) return (uint16_t)(sign | 0x7F80u);
  float f = (float)r; /* exact */
  uint32_t u;
  memcpy(&u, &f, 4);
  return (uint16_t)(sign | (u >> 16));
}

/* ---------------------------------------------------------- pack / unpack */

/* MLX affine packing: tests/kernels/test_moe_gather_int8.py:110-113. */
void orc_unpack(const uint32_t* w, int64_t n_words, int bits, uint8_t* codes) {
  const int per = 32 / bits;
  const uint32_t mask = (1u << bits) - 1u;
  for (int64_t i = 0; i < n_words; ++i) {
    uint32_t v = w[i];
    for (int t = 0; t < per; ++t) codes[i * per + t] = (uint8_t)((v >> (bits * t)) & mask);
  }
}

void orc_pack(const uint8_t* codes, int64_t n_codes, int bits, uint32_t* w) {
  const int per = 32 / bits;
  const uint32_t mask = (1u << bits) - 1u;
  for (int64_t i = 0; i < n_codes / per; ++i) {
    uint32_t v = 0;
    for (int t = 0; t < per; ++t) v |= ((uint32_t)codes[i * per + t] & mask) << (bits * t);
    w[i] = v;
  }
}

static inline uint32_t code_at(const uint32_t* row, int64_t k, int bits) {
  const int per = 32 / bits;
  return (row[k / per] >> (bits * (int)(k % per))) & ((1u << bits) - 1u);
}

/* -------------------------------------------------------------- dequant */

/* moe_gather_ws.py:343-344: bfloat(fma(float(q), s, b)). */
void orc_dequantize_bf16(const uint32_t* w, const uint16_t* s, const uint16_t* b,
                         int64_t rows, int64_t K, int group_size, int bits,
                         uint16_t* out) {
  const int64_t G = K / group_size;
  const int64_t words = K * bits / 32;
  for (int64_t n = 0; n < rows; ++n) {
    const uint32_t* row = w + n * words;
    for (int64_t k = 0; k < K; ++k) {
      float sc = orc_bf16_to_f32(s[n * G + k / group_size]);
      float bi = orc_bf16_to_f32(b[n * G + k / group_size]);
      float q = (float)code_at(row, k, bits);
      out[n * K + k] = orc_bf16_rne(fmaf(q, sc, bi));
    }
  }
}

/* Exact affine (mode 0) or bf16-materialised (mode 1) weights of one row. */
static void deq_row_f64(const uint32_t* row, const uint16_t* s, const uint16_t* b,
                        int64_t K, int group_size, int bits, int deq_mode,
                        double* out) {
  for (int64_t k = 0; k < K; ++k) {
    float sc = orc_bf16_to_f32(s[k / group_size]);
    float bi = orc_bf16_to_f32(b[k / group_size]);
    uint32_t q = code_at(row, k, bits);
    if (deq_mode == 1) {
      out[k] = (double)orc_bf16_to_f32(orc_bf16_rne(fmaf((float)q, sc, bi)));
    } else {
      out[k] = (double)sc * (double)q + (double)bi;
    }
  }
}

/* ------------------------------------------------------ gather_qmm rows */

static int cmp_pair(const void* a, const void* b) {
  const int64_t* x = (const int64_t*)a;
  const int64_t* y = (const int64_t*)b;
  if (x[0] != y[0]) return x[0] < y[0] ? -1 : 1;
  return x[1] < y[1] ? -1 : (x[1] > y[1]);
}

/* Rows grouped by expert so each expert's weights are dequantised once;
 * semantics are per row (mx.gather_qmm with transpose=True:
 * switch_layers.py:87-98, moe_gather_ws.py:403-414). */
void orc_gather_qmm_rows(const uint16_t* x, int64_t K, const int32_t* x_rows,
                         const int32_t* experts, int64_t n_rows,
                         const uint32_t* w, const uint16_t* s, const uint16_t* b,
                         int64_t N, int group_size, int bits, int deq_mode,
                         double* out_f64, uint16_t* out_bf16, int n_threads) {
  if (n_rows <= 0) return;
  const int64_t G = K / group_size;
  const int64_t words = K * bits / 32;
  int64_t* pairs = (int64_t*)malloc(sizeof(int64_t) * 2 * n_rows);
  for (int64_t r = 0; r < n_rows; ++r) {
    pairs[2 * r] = experts[r];
    pairs[2 * r + 1] = r;
  }
  qsort(pairs, (size_t)n_rows, sizeof(int64_t) * 2, cmp_pair);
  /* x rows used, as double (exact from bf16) */
  double* xr = (double*)malloc(sizeof(double) * n_rows * K);
  for (int64_t i = 0; i < n_rows; ++i) {
    int64_t r = pairs[2 * i + 1];
    int64_t src = x_rows ? x_rows[r] : r;
    for (int64_t k = 0; k < K; ++k) xr[i * K + k] = (double)orc_bf16_to_f32(x[src * K + k]);
  }
  int nt = n_threads > 0 ? n_threads : orc_max_threads();
  int64_t i0 = 0;
  while (i0 < n_rows) {
    int64_t e = pairs[2 * i0];
    int64_t i1 = i0;
    while (i1 < n_rows && pairs[2 * i1] == e) ++i1;
    const uint32_t* we = w + e * N * words;
    const uint16_t* se = s + e * N * G;
    const uint16_t* be = b + e * N * G;
#pragma omp parallel num_threads(nt)
    {
      double* wrow = (double*)malloc(sizeof(double) * K);
#pragma omp for schedule(static)
      for (int64_t n = 0; n < N; ++n) {
        deq_row_f64(we + n * words, se + n * G, be + n * G, K, group_size, bits,
                    deq_mode, wrow);
        for (int64_t i = i0; i < i1; ++i) {
          const double* xv = xr + i * K;
          double acc = 0.0;
          for (int64_t k = 0; k < K; ++k) acc += xv[k] * wrow[k];
          int64_t r = pairs[2 * i + 1];
          if (out_f64) out_f64[r * N + n] = acc;
          if (out_bf16) out_bf16[r * N + n] = orc_bf16_rne_f64(acc);
        }
      }
      free(wrow);
    }
    i0 = i1;
  }
  free(xr);
  free(pairs);
}

/* ---------------------------------------------------------------- routing */

/* switch_layers.py:13-18 with a stable sort; counting sort over E buckets. */
int orc_route_sort(const int32_t* ids, int64_t n, int32_t E, int32_t* order,
                   int32_t* inv_order, int32_t* sorted_ids) {
  int64_t* cnt = (int64_t*)calloc((size_t)E + 1, sizeof(int64_t));
  for (int64_t i = 0; i < n; ++i) {
    if (ids[i] < 0 || ids[i] >= E) {
      free(cnt);
      return -1;
    }
    cnt[ids[i] + 1]++;
  }
  for (int32_t e = 0; e < E; ++e) cnt[e + 1] += cnt[e];
  for (int64_t i = 0; i < n; ++i) {
    int64_t dst = cnt[ids[i]]++;
    order[dst] = (int32_t)i;
  }
  for (int64_t i = 0; i < n; ++i) {
    inv_order[order[i]] = (int32_t)i;
    sorted_ids[i] = ids[order[i]];
  }
  free(cnt);
  return 0;
}

/* moe_gather_ws.py:133-156 (lower_bound offsets, tiles per TMT rows). */
int64_t orc_build_tiles(const int32_t* sorted_ids, int64_t n, int32_t E,
                        int32_t tile_rows, int32_t* offsets, int32_t* tile_row,
                        int32_t* tile_exp, int64_t max_tiles) {
  for (int32_t e = 0; e <= E; ++e) {
    int64_t lo = 0, hi = n;
    while (lo < hi) {
      int64_t mid = (lo + hi) >> 1;
      if (sorted_ids[mid] < e) lo = mid + 1;
      else hi = mid;
    }
    offsets[e] = (int32_t)lo;
  }
  int64_t t = 0;
  for (int32_t e = 0; e < E; ++e) {
    for (int64_t r = offsets[e]; r < offsets[e + 1]; r += tile_rows) {
      if (t < max_tiles) {
        tile_row[t] = (int32_t)r;
        tile_exp[t] = e;
      }
      ++t;
    }
  }
  int64_t nt = t < max_tiles ? t : max_tiles;
  for (int64_t j = nt; j < max_tiles; ++j) {
    tile_row[j] = 0;
    tile_exp[j] = 0;
  }
  return nt;
}

/* ---------------------------------------------------------------- swiglu */

/* activations.py:9-11: silu(gate) * up, gate rows first (switch_layers.py:229-237). */
void orc_swiglu(const double* gu, int64_t rows, int64_t I, double* h_f64,
                uint16_t* h_bf16) {
  for (int64_t r = 0; r < rows; ++r) {
    for (int64_t i = 0; i < I; ++i) {
      double g = gu[r * 2 * I + i];
      double u = gu[r * 2 * I + I + i];
      double h = g / (1.0 + exp(-g)) * u;
      if (h_f64) h_f64[r * I + i] = h;
      if (h_bf16) h_bf16[r * I + i] = orc_bf16_rne_f64(h);
    }
  }
}

/* ---------------------------------------------------------- weighted sum */

static inline float rb(float v) { return orc_bf16_to_f32(orc_bf16_rne(v)); }

/* moe_weighted_sum.py:44-98 arithmetic: slot j mod 8, sequential combine. */
void orc_weighted_sum(const uint16_t* xs, const int32_t* inv, const float* scores,
                      int64_t rows, int64_t k, int64_t dim, int mode,
                      uint16_t* out) {
  const int round_prod = mode >= 1;
  const int bf_acc = mode == 2;
  for (int64_t r = 0; r < rows; ++r) {
    for (int64_t d = 0; d < dim; ++d) {
      float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
      for (int64_t j = 0; j < k; ++j) {
        int64_t p = r * k + j;
        int64_t src = inv ? inv[p] : p;
        float sc = mode >= 1 ? rb(scores[p]) : scores[p];
        float prod = sc * orc_bf16_to_f32(xs[src * dim + d]);
        if (round_prod) prod = rb(prod);
        float t = acc[j % 8] + prod;
        acc[j % 8] = bf_acc ? rb(t) : t;
      }
      float a = acc[0];
      for (int j = 1; j < 8; ++j) {
        a = a + acc[j];
        if (bf_acc) a = rb(a);
      }
      out[r * dim + d] = orc_bf16_rne(a);
    }
  }
}

/* -------------------------------------------------- decode down + wsum */

/* decode-fusion/test_exact.py:31-50 golden, down half. */
void orc_down_wsum(const uint16_t* h, const int32_t* idx, const float* scores,
                   int64_t T, int64_t k, int64_t I, const uint32_t* w,
                   const uint16_t* s, const uint16_t* b, int64_t D,
                   int group_size, int bits, double* y_f64, uint16_t* y_bf16,
                   int n_threads) {
  const int64_t G = I / group_size;
  const int64_t words = I * bits / 32;
  int nt = n_threads > 0 ? n_threads : orc_max_threads();
#pragma omp parallel num_threads(nt)
  {
    double* wrow = (double*)malloc(sizeof(double) * I);
#pragma omp for schedule(static)
    for (int64_t d = 0; d < D; ++d) {
      for (int64_t t = 0; t < T; ++t) {
        double y = 0.0;
        for (int64_t j = 0; j < k; ++j) {
          int64_t e = idx[t * k + j];
          deq_row_f64(w + (e * D + d) * words, s + (e * D + d) * G,
                      b + (e * D + d) * G, I, group_size, bits, 0, wrow);
          const uint16_t* hv = h + (t * k + j) * I;
          double acc = 0.0;
          for (int64_t i = 0; i < I; ++i) acc += (double)orc_bf16_to_f32(hv[i]) * wrow[i];
          y += (double)scores[t * k + j] * acc;
        }
        if (y_f64) y_f64[t * D + d] = y;
        if (y_bf16) y_bf16[t * D + d] = orc_bf16_rne_f64(y);
      }
    }
    free(wrow);
  }
}

/* ------------------------------------------------------------------ int8 */

void orc_quant_act_int8(const uint16_t* x, int64_t R, int64_t K, int8_t* xi,
                        float* sx) {
  for (int64_t r = 0; r < R; ++r) {
    float amax = 0.0f;
    for (int64_t k = 0; k < K; ++k) {
      float v = fabsf(orc_bf16_to_f32(x[r * K + k]));
      if (v > amax) amax = v;
    }
    float sc = amax / 127.0f;
    sx[r] = sc;
    for (int64_t k = 0; k < K; ++k) {
      if (sc == 0.0f) {
        xi[r * K + k] = 0;
        continue;
      }
      float q = rintf(orc_bf16_to_f32(x[r * K + k]) / sc);
      if (q > 127.0f) q = 127.0f;
      if (q < -127.0f) q = -127.0f;
      xi[r * K + k] = (int8_t)q;
    }
  }
}

void orc_gather_qmm_int8_rows(const int8_t* xi, const float* sx, int64_t K,
                              const int32_t* x_rows, const int32_t* experts,
                              int64_t n_rows, const uint32_t* w,
                              const uint16_t* s, const uint16_t* b, int64_t N,
                              int group_size, int bits, double* out_f64,
                              uint16_t* out_bf16, int n_threads) {
  if (n_rows <= 0) return;
  const int64_t G = K / group_size;
  const int64_t words = K * bits / 32;
  int64_t* pairs = (int64_t*)malloc(sizeof(int64_t) * 2 * n_rows);
  for (int64_t r = 0; r < n_rows; ++r) {
    pairs[2 * r] = experts[r];
    pairs[2 * r + 1] = r;
  }
  qsort(pairs, (size_t)n_rows, sizeof(int64_t) * 2, cmp_pair);
  int nt = n_threads > 0 ? n_threads : orc_max_threads();
  int64_t i0 = 0;
  while (i0 < n_rows) {
    int64_t e = pairs[2 * i0];
    int64_t i1 = i0;
    while (i1 < n_rows && pairs[2 * i1] == e) ++i1;
#pragma omp parallel num_threads(nt)
    {
      double* wrow = (double*)malloc(sizeof(double) * K);
#pragma omp for schedule(static)
      for (int64_t n = 0; n < N; ++n) {
        deq_row_f64(w + (e * N + n) * words, s + (e * N + n) * G,
                    b + (e * N + n) * G, K, group_size, bits, 0, wrow);
        for (int64_t i = i0; i < i1; ++i) {
          int64_t r = pairs[2 * i + 1];
          int64_t src = x_rows ? x_rows[r] : r;
          const int8_t* xv = xi + src * K;
          double acc = 0.0;
          for (int64_t k = 0; k < K; ++k) acc += (double)xv[k] * wrow[k];
          double y = (double)sx[src] * acc;
          if (out_f64) out_f64[r * N + n] = y;
          if (out_bf16) out_bf16[r * N + n] = orc_bf16_rne_f64(y);
        }
      }
      free(wrow);
    }
    i0 = i1;
  }
  free(pairs);
}

int orc_max_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

/* -------------------------------------------------------------- router */

/* fused_kernels.py:288-330: k rounds of (max value, lowest index holding it). */
void orc_router_topk(const float* logits, int64_t T, int64_t E, int64_t k, int norm,
                     int32_t* idx, double* scores) {
  for (int64_t t = 0; t < T; ++t) {
    const float* l = logits + t * E;
    unsigned char* taken = (unsigned char*)calloc((size_t)E, 1);
    double lmax = -INFINITY;
    for (int64_t e = 0; e < E; ++e) if ((double)l[e] > lmax) lmax = l[e];
    double all = 0.0;
    for (int64_t e = 0; e < E; ++e) all += exp((double)l[e] - lmax);
    for (int64_t j = 0; j < k; ++j) {
      int64_t best = -1;
      for (int64_t e = 0; e < E; ++e)
        if (!taken[e] && (best < 0 || l[e] > l[best])) best = e;
      taken[best] = 1;
      idx[t * k + j] = (int32_t)best;
    }
    if (norm) {
      const double l0 = l[idx[t * k]];
      double sum = 0.0;
      for (int64_t j = 0; j < k; ++j) sum += exp((double)l[idx[t * k + j]] - l0);
      for (int64_t j = 0; j < k; ++j) scores[t * k + j] = exp((double)l[idx[t * k + j]] - l0) / sum;
    } else {
      for (int64_t j = 0; j < k; ++j) scores[t * k + j] = exp((double)l[idx[t * k + j]] - lmax) / all;
    }
    free(taken);
  }
}

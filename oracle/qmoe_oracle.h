/*
 * CPU oracle for the quantized MoE gather_qmm path.  TEST INFRASTRUCTURE ONLY.
 *
 * This is a plain-C restatement of the arithmetic of MLX-affine quantized
 * matmuls as the reference calls them.  It is test infrastructure: only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg load it, and the
 * product (titan_amd/) never links, imports or calls it.
 *
 * Conventions
 *   bf16 values travel as uint16_t bit patterns.
 *   Packed weights are uint32 words, MLX affine layout: element k of a row sits
 *   in word (k*bits)/32 at bit offset bits*(k mod (32/bits)); the low bits hold
 *   the earliest k (reference: tests/kernels/test_moe_gather_int8.py:110-113,
 *   engine/patches/decode-fusion/test_exact.py:19-28).
 *   Scales and biases are bf16 [rows, K/group_size]; w = s*q + b.
 *
 * Every function cites the reference file:line whose semantics it restates.
 */
#ifndef QMOE_ORACLE_H
#define QMOE_ORACLE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* bf16 <-> fp32.  Round to nearest even, NaN kept quiet. */
uint16_t orc_bf16_rne(float f);
float orc_bf16_to_f32(uint16_t h);
uint16_t orc_bf16_rne_f64(double d);  /* one rounding, exact double -> bf16 */

/* a1: unpack / pack of MLX affine codes (bits 4 or 8). */
void orc_unpack(const uint32_t* w, int64_t n_words, int bits, uint8_t* codes);
void orc_pack(const uint8_t* codes, int64_t n_codes, int bits, uint32_t* w);

/* a2: materialised dequant, bf16(fmaf(q, s, b)) per element
 * (titan/kernels/moe_gather_ws.py:343-344).  rows x K elements. */
void orc_dequantize_bf16(const uint32_t* w, const uint16_t* s, const uint16_t* b,
                         int64_t rows, int64_t K, int group_size, int bits,
                         uint16_t* out);

/* a5 / a16: gather_qmm in row form.  Output row r is
 *   out[r, n] = sum_k x[x_rows[r], k] * W[experts[r]][n, k]
 * with W[e] = dequant of w + e*N*K*bits/32 (scales/biases likewise).
 * deq_mode 0: exact affine s*q+b (double), the factored form of
 *             engine/patches/decode-fusion/fused_kernels.py:57-79;
 * deq_mode 1: bf16-materialised weights (moe_gather_ws.py:343-344).
 * Accumulation in double.  x_rows may be NULL (identity).  out_f64 and/or
 * out_bf16 (RNE of the double sum) may be NULL.  n_threads <= 0: all. */
void orc_gather_qmm_rows(const uint16_t* x, int64_t K, const int32_t* x_rows,
                         const int32_t* experts, int64_t n_rows,
                         const uint32_t* w, const uint16_t* s, const uint16_t* b,
                         int64_t N, int group_size, int bits, int deq_mode,
                         double* out_f64, uint16_t* out_bf16, int n_threads);

/* a3: stable argsort of expert ids (switch_layers.py:13-18) by counting sort.
 * order[i] = pair index of sorted row i, inv_order = argsort(order),
 * sorted_ids[i] = ids[order[i]].  Ids must lie in [0, E). Returns 0, or -1 on
 * an out-of-range id. */
int orc_route_sort(const int32_t* ids, int64_t n, int32_t E, int32_t* order,
                   int32_t* inv_order, int32_t* sorted_ids);

/* a4: segment offsets and the ragged (row_start, expert) tile list
 * (titan/kernels/moe_gather_ws.py:133-156, 176-178).  offsets has E+1
 * entries (offsets[e] = lower_bound(e)); tiles are emitted expert by expert,
 * one per tile_rows rows; entries past the count (up to max_tiles) are zero.
 * Returns the number of tiles (capped at max_tiles). */
int64_t orc_build_tiles(const int32_t* sorted_ids, int64_t n, int32_t E,
                        int32_t tile_rows, int32_t* offsets, int32_t* tile_row,
                        int32_t* tile_exp, int64_t max_tiles);

/* a8: h = silu(gate) * up from gate_up rows laid out [gate(I) | up(I)]
 * (switch_layers.py:229-237, activations.py:9-11), in double, then RNE. */
void orc_swiglu(const double* gu, int64_t rows, int64_t I, double* h_f64,
                uint16_t* h_bf16);

/* a13: moe_weighted_sum (titan/kernels/moe_weighted_sum.py:44-98).
 * out[r, d] = sum_j sc[r, j] * xs[src(r, j), d], src = inv[r*k + j] or
 * r*k + j when inv is NULL.  mode 0 fast (fp32 scores and products),
 * 1 ops (bf16 scores, bf16-rounded products, fp32 partials),
 * 2 clone (bf16 scores, bf16 products, bf16 partials); eight partial slots
 * by j mod 8, combined in slot order.  No fused multiply-add anywhere. */
void orc_weighted_sum(const uint16_t* xs, const int32_t* inv, const float* scores,
                      int64_t rows, int64_t k, int64_t dim, int mode,
                      uint16_t* out);

/* Fused decode down projection + weighted sum golden
 * (engine/patches/decode-fusion/test_exact.py:31-50):
 * y[t, :] = sum_j score[t, j] * (W[idx[t, j]] @ h[t, j, :]), exact affine
 * weights, double throughout.  h is bf16 [T, k, I]. */
void orc_down_wsum(const uint16_t* h, const int32_t* idx, const float* scores,
                   int64_t T, int64_t k, int64_t I, const uint32_t* w,
                   const uint16_t* s, const uint16_t* b, int64_t D,
                   int group_size, int bits, double* y_f64, uint16_t* y_bf16,
                   int n_threads);

/* a10 (config form): per-token symmetric int8 quantisation.
 * sx = absmax/127 (fp32, correctly rounded division), xi = clamp(rint(x/sx),
 * -127, 127) with rint half-to-even; a row of zeros gives sx = 0, xi = 0. */
void orc_quant_act_int8(const uint16_t* x, int64_t R, int64_t K, int8_t* xi,
                        float* sx);

/* a12 (config form): int8-activation x int4-weight gather, fake-quant golden
 * y[r, n] = sx[x_rows[r]] * sum_k xi[x_rows[r], k] * (s*q + b), in double. */
void orc_gather_qmm_int8_rows(const int8_t* xi, const float* sx, int64_t K,
                              const int32_t* x_rows, const int32_t* experts,
                              int64_t n_rows, const uint32_t* w,
                              const uint16_t* s, const uint16_t* b, int64_t N,
                              int group_size, int bits, double* out_f64,
                              uint16_t* out_bf16, int n_threads);

/* a14: fused router top-k (engine/patches/decode-fusion/fused_kernels.py:363-371
 * router_topk, kernel source :288-330).  Per token the k largest logits in
 * descending order, ties to the lower expert index; scores in double:
 * norm != 0: exp(l_j - l_0) / sum_{j<k} exp(l_j - l_0) (the softmax over
 * all experts renormalised over the chosen k, language.py:65-71);
 * norm == 0: exp(l_j - max) / sum_all exp(l - max). */
void orc_router_topk(const float* logits, int64_t T, int64_t E, int64_t k, int norm,
                     int32_t* idx, double* scores);

/* Number of OpenMP threads the oracle would use (for the CPU baseline). */
int orc_max_threads(void);

#ifdef __cplusplus
}
#endif
#endif

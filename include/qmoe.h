/*
 * qmoe.h -- C ABI of libqmoe.so, the MI355X (gfx950) quantized mixture-of-experts
 * matmul path: MLX-affine group-quantized weights, gather_qmm for the fused
 * gate_up and down expert projections, the int8-activation x int4-weight
 * gate_up variant, and the fused SwiGLU / top-k weighted-sum epilogues.
 *
 * Conventions (every entry point):
 *  - Plain device pointers and sizes; no framework types.  bf16 tensors are
 *    uint16_t bit patterns; packed weights are uint32_t words in MLX affine
 *    layout: element k of a row sits in word k*bits/32 at bit offset
 *    bits*(k mod 32/bits), low bits first.  Scales and biases are bf16
 *    [rows, K/group_size]; the weight is w = scale*q + bias.
 *  - All tensors are contiguous, row-major.  Expert tensors are
 *    [num_experts, N, K*bits/32] (weights) and [num_experts, N, K/group_size]
 *    (scales, biases).
 *  - The caller owns and allocates every output and workspace.  The library
 *    never allocates or frees caller memory and keeps no state between calls
 *    beyond a thread-local error message.
 *  - Every launch is enqueued on `stream` (a hipStream_t; NULL is the null
 *    stream).  No entry point synchronises the host.
 *  - Return value: QMOE_OK, or an error code with a message readable through
 *    qmoe_last_error().  QMOE_ERR_UNSUPPORTED means "this shape, dtype, bit
 *    width or group size has no kernel": callers fall back to their stock
 *    path, as the reference's patches do (engine/patches/moe-int8/patch.py:78-122).
 *
 * Each declaration names the reference interface it replaces (paths relative
 * to the reference repository root).
 */
#ifndef QMOE_H
#define QMOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define QMOE_ABI_VERSION 4

enum {
  QMOE_OK = 0,
  QMOE_ERR_INVALID = 1,     /* bad argument (null pointer, inconsistent sizes) */
  QMOE_ERR_UNSUPPORTED = 2, /* no kernel for this configuration: fall back */
  QMOE_ERR_HIP = 3,         /* a HIP runtime call failed */
  QMOE_ERR_WORKSPACE = 4    /* workspace missing or too small */
};

/* Weighted-sum rounding modes: titan/kernels/moe_weighted_sum.py:44-49. */
enum { QMOE_WSUM_FAST = 0, QMOE_WSUM_OPS = 1, QMOE_WSUM_CLONE = 2 };

int qmoe_abi_version(void);
/* Thread-local message of the last failing call on this thread. */
const char* qmoe_last_error(void);

/* ---------------------------------------------------------------- layout --
 * MLX affine unpack (layout contract evidenced by
 * tests/kernels/test_moe_gather_int8.py:104-115) and materialised dequant
 * out = bf16_rne(fmaf(q, s, b)) (titan/kernels/moe_gather_ws.py:343-344),
 * the device counterparts of mx.dequantize. */
int qmoe_unpack(const uint32_t* w, int64_t n_words, int bits, uint8_t* codes,
                void* stream);
int qmoe_dequantize(const uint32_t* w, const uint16_t* scales,
                    const uint16_t* biases, int64_t rows, int64_t K,
                    int group_size, int bits, uint16_t* out, void* stream);

/* --------------------------------------------------------------- routing --
 * Replaces _gather_sort (titan/adapters/mlx/vendor/mlx_lm/models/
 * switch_layers.py:13-18) together with build_tiles
 * (titan/kernels/moe_gather_ws.py:181-202), on the device, no host sync:
 *   order      [n] pair index of sorted row i (stable argsort of ids)
 *   inv_order  [n] argsort(order)
 *   sorted_ids [n] ids[order]
 *   offsets    [E+1] first sorted row of each expert (lower_bound)
 *   tile_row / tile_exp [max_tiles] one (row_start, expert) per tile_rows
 *              rows of each expert, expert-major; entries past the count are 0
 *   ntiles     [1] number of tiles, capped at max_tiles
 * max_tiles >= ceil(n/tile_rows) + E always suffices (moe_gather_ws.py:176-178).
 * Ids outside [0, E) are clamped into range and counted in workspace word 0
 * (readable after the stream completes), so every index written stays valid.
 * Workspace: qmoe_route_workspace_size(n, E) bytes. */
size_t qmoe_route_workspace_size(int64_t n_pairs, int32_t num_experts);
int qmoe_route(const int32_t* ids, int64_t n_pairs, int32_t num_experts,
               int32_t tile_rows, int32_t* order, int32_t* inv_order,
               int32_t* sorted_ids, int32_t* offsets, int32_t* tile_row,
               int32_t* tile_exp, int32_t* ntiles, int64_t max_tiles,
               void* workspace, size_t workspace_bytes, void* stream);

/* qmoe_route without a caller workspace.  No counterpart in the reference:
 * this is for callers that cannot allocate device memory (code under HIP
 * graph capture, serving loops or harnesses that forbid hipMalloc).  The
 * routing workspace is a file-scope device array of
 * QMOE_ROUTE_NOALLOC_SCRATCH_BYTES inside the library, one per GPU, held
 * until the process ends; the entry point calls no allocator.  Calls whose
 * qmoe_route_workspace_size(n_pairs, num_experts) exceeds it return
 * QMOE_ERR_UNSUPPORTED (at 256 experts: up to 1,043,456 pairs).  Every call
 * on one GPU shares that GPU's array, so calls that overlap on one GPU (two
 * streams, two host threads) race; serialise them.  The stream must belong
 * to the current device.  Outputs as for qmoe_route; the count of ids
 * outside [0, E) goes to n_bad[0] when n_bad is not NULL. */
#define QMOE_ROUTE_NOALLOC_SCRATCH_BYTES (1u << 20)
int qmoe_route_noalloc(const int32_t* ids, int64_t n_pairs, int32_t num_experts,
                       int32_t tile_rows, int32_t* order, int32_t* inv_order,
                       int32_t* sorted_ids, int32_t* offsets, int32_t* tile_row,
                       int32_t* tile_exp, int32_t* ntiles, int64_t max_tiles,
                       int32_t* n_bad, void* stream);

/* build_tiles over ids that are already sorted ascending
 * (titan/kernels/moe_gather_ws.py:133-156,181-202). */
int qmoe_build_tiles(const int32_t* sorted_ids, int64_t n_rows,
                     int32_t num_experts, int32_t tile_rows, int32_t* offsets,
                     int32_t* tile_row, int32_t* tile_exp, int32_t* ntiles,
                     int64_t max_tiles, void* stream);

/* ------------------------------------------------------------ gather_qmm --
 * Row form of mx.gather_qmm(x, w, scales, biases, lhs_indices, rhs_indices,
 * transpose=True, group_size, bits) (called at switch_layers.py:87-98;
 * positional contract engine/patches/moe-int8/patch.py:81-90):
 *   out[r, n] = sum_k x[x_rows[r], k] * W[experts[r]][n, k]
 * x_rows == NULL means x_rows[r] = r (x already gathered).  A caller maps the
 * broadcast (lhs_indices, rhs_indices) batch onto rows; rows need not be sorted.
 * Matrix-vector kernel: every row streams its expert's weights, so this is the
 * decode / small-batch path.  fp32 accumulation of the factored affine form
 * s*sum(x*q) + b*sum(x) (engine/patches/decode-fusion/fused_kernels.py:57-79),
 * bf16 output.  bits 4 or 8 (8-bit codes need K = 2048*n with n <= 4, or
 * K = 32*L*n with L in {4, 8, 16} and n <= 8), group_size 32, 64 or 128
 * (engine/patches/smallm/kernel.py:38, 319-327). */
int qmoe_gather_qmv(const uint16_t* x, const int32_t* x_rows,
                    const int32_t* experts, int64_t n_rows, int64_t K,
                    const uint32_t* w, const uint16_t* scales,
                    const uint16_t* biases, int32_t num_experts, int64_t N,
                    int group_size, int bits, uint16_t* out, void* stream);

/* mx.quantized_matmul(x, w, scales, biases, transpose=True, group_size, bits)
 * for x [M, K] (titan/adapters/mlx/compiled.py:209-218; small-M drop-in
 * engine/patches/smallm/kernel.py:333-391): out [M, N].  Same bit widths and
 * group sizes as qmoe_gather_qmv. */
int qmoe_quantized_matmul(const uint16_t* x, int64_t M, int64_t K,
                          const uint32_t* w, const uint16_t* scales,
                          const uint16_t* biases, int64_t N, int group_size,
                          int bits, uint16_t* out, void* stream);

/* Sorted grouped GEMM: the prefill form of gather_qmm with
 * sorted_indices=True, replacing titan/kernels/moe_gather_ws.py:417-445
 * (and its MLX reference :403-414).  Rows [0, n_rows) are grouped by expert
 * as described by (offsets, tile_row, tile_exp, ntiles) from qmoe_route or
 * qmoe_build_tiles built with tile_rows == qmoe_gemm_tile_rows().
 *   out[r, n] = sum_k x[x_rows[r], k] * W[e(r)][n, k]   (x_rows NULL: identity)
 * Weights are dequantised to bf16 as bf16_rne(fmaf(q, s, b)) and multiplied on
 * bf16 MFMA with fp32 accumulation (moe_gather_ws.py:20-32 semantics). */
int qmoe_gemm_tile_rows(void);
int qmoe_gather_qmm_sorted(const uint16_t* x, const int32_t* x_rows,
                           int64_t n_rows, int64_t K, const uint32_t* w,
                           const uint16_t* scales, const uint16_t* biases,
                           int32_t num_experts, int64_t N, int group_size,
                           int bits, const int32_t* offsets,
                           const int32_t* tile_row, const int32_t* tile_exp,
                           const int32_t* ntiles, int64_t max_tiles,
                           uint16_t* out, void* stream);

/* ------------------------------------------------------ fused decode MoE --
 * Gather gate_up GEMV + SwiGLU in one launch, replacing
 * engine/patches/decode-fusion/fused_kernels.py:31-88,194-210 (gate_up_silu)
 * and the split + swiglu of switch_layers.py:229-237:
 *   g = x[t] . W[idx[t,j]][i, :],  u = x[t] . W[idx[t,j]][I + i, :]
 *   h[t, j, i] = bf16(silu(g) * u)         (fp32 throughout, gate rows first)
 * x [T, K] bf16, idx [T, top_k] int32, w [E, 2I, K*bits/32]. */
int qmoe_moe_gate_up_swiglu(const uint16_t* x, const int32_t* idx, int64_t T,
                            int64_t top_k, int64_t K, const uint32_t* w,
                            const uint16_t* scales, const uint16_t* biases,
                            int32_t num_experts, int64_t I, int group_size,
                            int bits, uint16_t* h, void* stream);

/* Gather down GEMV + router-weighted top-k sum in one launch, replacing
 * engine/patches/decode-fusion/fused_kernels.py:93-169,213-231 (down_wsum)
 * and the weighted-sum tail of qwen3_5_moe/language.py:78-83:
 *   y[t, :] = bf16( sum_j scores[t, j] * (W[idx[t,j]] @ h[t, j, :]) )
 * Each distinct expert's weights are read once and shared by every (t, j)
 * routed to it.  h [T, top_k, I] bf16, scores [T, top_k] fp32,
 * w [E, D, I*bits/32], y [T, D] bf16.  T*top_k <= 1024. */
int qmoe_moe_down_wsum(const uint16_t* h, const int32_t* idx,
                       const float* scores, int64_t T, int64_t top_k,
                       int64_t I, const uint32_t* w, const uint16_t* scales,
                       const uint16_t* biases, int32_t num_experts, int64_t D,
                       int group_size, int bits, uint16_t* y, void* stream);

/* ----------------------------------------------------------- weighted sum --
 * moe_weighted_sum (titan/kernels/moe_weighted_sum.py:142-195):
 *   out[r, d] = sum_j sc[r, j] * xs[src, d],  src = inv_order[r*k + j]
 * (inv_order NULL: src = r*k + j, the token-major layout).  mode is one of
 * QMOE_WSUM_*: fast keeps fp32 scores and products; ops rounds scores and
 * products to bf16; clone also keeps the eight partial sums in bf16.  Eight
 * partial slots (j mod 8) combined in order; no fused multiply-add.
 * xs [rows*k, dim] bf16, scores [rows, k] fp32, out [rows, dim] bf16. */
int qmoe_weighted_sum(const uint16_t* xs, const int32_t* inv_order,
                      const float* scores, int64_t rows, int64_t top_k,
                      int64_t dim, int mode, uint16_t* out, void* stream);

/* ----------------------------------------------------------- tile layout --
 * Load-time repack of 4-bit, group-64 expert weights into the layout the
 * grouped GEMMs copy contiguously: per (expert, 64-column block, group) one
 * 2 KiB chunk of codes and one 256-byte chunk of scale/bias pairs.  Replaces,
 * in role, the reference's per-tensor prepared tables
 * (titan/kernels/moe_gather_int8.py:189-248 build_tables): built once per
 * weight tensor, owned by the caller; the MLX-layout tensors stay accepted by
 * every other entry point.  With G = K/64 and c the 64-column block:
 *   wp[e][c][g][j][h][l][t] = w[e][64c + 32j + l][8g + 4h + t]
 *        (j < 2, h < 2, l < 32, t < 4; as many words as w)
 *   sb[e][c][g][i]          = s[e][64c + i][g] | b[e][64c + i][g] << 16
 *        (i < 64; as many bytes as scales and biases together)
 * Requires bits == 4, group_size == 64, N % 64 == 0, K % 64 == 0. */
int qmoe_repack_tiles(const uint32_t* w, const uint16_t* scales,
                      const uint16_t* biases, int32_t num_experts, int64_t N,
                      int64_t K, int group_size, int bits, uint32_t* wp,
                      uint32_t* sb, void* stream);

/* qmoe_gather_qmm_sorted over tile-layout weights (wp, sb from
 * qmoe_repack_tiles); same rows, tiles, arithmetic and summation order, so
 * the result is bit-identical to the MLX-layout call. */
int qmoe_gather_qmm_sorted_tiles(const uint16_t* x, const int32_t* x_rows,
                                 int64_t n_rows, int64_t K, const uint32_t* wp,
                                 const uint32_t* sb, int32_t num_experts,
                                 int64_t N, const int32_t* offsets,
                                 const int32_t* tile_row,
                                 const int32_t* tile_exp,
                                 const int32_t* ntiles, int64_t max_tiles,
                                 uint16_t* out, void* stream);

/* Decode gather-GEMV (qmoe_gather_qmv) over tile-layout weights; same results
 * as the MLX-layout call (the same factored arithmetic and reduction order).
 * Requires K = 2048*n (n <= 4) and 64 | N. */
int qmoe_gather_qmv_tiles(const uint16_t* x, const int32_t* x_rows,
                          const int32_t* experts, int64_t n_rows, int64_t K,
                          const uint32_t* wp, const uint32_t* sb,
                          int32_t num_experts, int64_t N, uint16_t* out,
                          void* stream);

/* The fused decode gate_up + SwiGLU (qmoe_moe_gate_up_swiglu) over tile-layout
 * weights in the gate/up-PAIRED row order of
 * qmoe_gather_qmm_swiglu_sorted_tiles (one resident copy serves both the
 * decode and the prefill gate_up): the MLX-layout call's arithmetic per
 * 32-code chunk, summed in another order.  Requires K = 2048*n (n <= 4) and
 * 32 | I. */
int qmoe_moe_gate_up_swiglu_tiles(const uint16_t* x, const int32_t* idx,
                                  int64_t T, int64_t top_k, int64_t K,
                                  const uint32_t* wp, const uint32_t* sb,
                                  int32_t num_experts, int64_t I, uint16_t* h,
                                  void* stream);

/* The fused decode down + weighted sum (qmoe_moe_down_wsum, replacing
 * engine/patches/decode-fusion/fused_kernels.py:93-169,213-231) over
 * tile-layout down weights [E, D, I]; bit-identical to the MLX-layout call.
 * Requires I = 512, 64 | D, T <= 16, top_k <= 16. */
int qmoe_moe_down_wsum_tiles(const uint16_t* h, const int32_t* idx,
                             const float* scores, int64_t T, int64_t top_k,
                             int64_t I, const uint32_t* wp, const uint32_t* sb,
                             int32_t num_experts, int64_t D, uint16_t* y,
                             void* stream);

/* qmoe_moe_gate_up_swiglu_tiles with the router's top-k folded in (replacing
 * engine/patches/decode-fusion/fused_kernels.py:363-371 router_topk ahead of
 * gate_up_silu, decode-fusion/kernel.py:111-138): each wave picks its pair's
 * expert from the token's fp32 router logits [T, num_experts] by
 * qmoe_router_topk's own selection, and the token's ids and scores (norm as
 * in qmoe_router_topk) are written to idx and scores [T, top_k] for
 * qmoe_moe_down_wsum_tiles, so h, idx and scores equal qmoe_router_topk
 * followed by qmoe_moe_gate_up_swiglu_tiles, bit for bit, with one launch
 * fewer.  Requires top_k <= 64 and num_experts <= 1024 besides the call's own
 * envelope. */
int qmoe_moe_gate_up_swiglu_tiles_topk(const uint16_t* x, const float* logits,
                                       int norm, int64_t T, int64_t top_k,
                                       int64_t K, const uint32_t* wp,
                                       const uint32_t* sb, int32_t num_experts,
                                       int64_t I, uint16_t* h, int32_t* idx,
                                       float* scores, void* stream);

/* ------------------------------------------------------------------ int8 --
 * int8-activation x int4-weight gate_up (replaces
 * titan/kernels/moe_gather_int8.py:132-182 quantize_activations and
 * :393-425 metal, with per-token symmetric activations):
 *   sx[r] = max_k |x[r,k]| / 127 (fp32),  xi = clamp(rint(x / sx), -127, 127)
 * A row of zeros gives sx = 0 and xi = 0. */
int qmoe_quantize_act_int8(const uint16_t* x, int64_t R, int64_t K,
                           int8_t* xi, float* sx, void* stream);

/* out[r, n] = sx[x_rows[r]] * sum_g ( s[n,g] * D_g + b[n,g] * R_g ),
 * D_g = sum_{k in g} xi*q and R_g = sum_{k in g} xi exact in int32, on int8
 * MFMA; rows grouped by expert as for qmoe_gather_qmm_sorted with tile_rows
 * == qmoe_gemm_tile_rows(). */
int qmoe_gather_qmm_int8_sorted(const int8_t* xi, const float* sx,
                                const int32_t* x_rows, int64_t n_rows,
                                int64_t K, const uint32_t* w,
                                const uint16_t* scales, const uint16_t* biases,
                                int32_t num_experts, int64_t N, int group_size,
                                int bits, const int32_t* offsets,
                                const int32_t* tile_row,
                                const int32_t* tile_exp, const int32_t* ntiles,
                                int64_t max_tiles, uint16_t* out,
                                void* stream);

/* qmoe_gather_qmm_int8_sorted over tile-layout weights (wp, sb from
 * qmoe_repack_tiles); same rows, tiles and arithmetic.  Replaces the same
 * reference op (titan/kernels/moe_gather_int8.py:393-425) with the prepared
 * tables (:189-248) in the role of the tile layout. */
int qmoe_gather_qmm_int8_sorted_tiles(const int8_t* xi, const float* sx,
                                      const int32_t* x_rows, int64_t n_rows,
                                      int64_t K, const uint32_t* wp,
                                      const uint32_t* sb, int32_t num_experts,
                                      int64_t N, const int32_t* offsets,
                                      const int32_t* tile_row,
                                      const int32_t* tile_exp,
                                      const int32_t* ntiles, int64_t max_tiles,
                                      uint16_t* out, void* stream);

/* gate_up grouped GEMM with the SwiGLU epilogue fused: weights [E, N = 2I, K]
 * in the tile layout of the gate/up-PAIRED row order (row 64c + j of the
 * paired order is gate row 32c + j for j < 32 and up row I + 32c + j - 32
 * otherwise; ops.repack_tiles(..., swiglu_pairs=True)), output
 * h [n_rows, I] bf16 = silu(gate) * up from the fp32 accumulators, rounded
 * once.  Replaces SwitchGLU's gate_up gather, split and activation
 * (switch_layers.py:213-237) for the sorted prefill form; N % 256 == 0. */
int qmoe_gather_qmm_swiglu_sorted_tiles(const uint16_t* x, const int32_t* x_rows,
                                        int64_t n_rows, int64_t K,
                                        const uint32_t* wp, const uint32_t* sb,
                                        int32_t num_experts, int64_t N,
                                        const int32_t* offsets,
                                        const int32_t* tile_row,
                                        const int32_t* tile_exp,
                                        const int32_t* ntiles, int64_t max_tiles,
                                        uint16_t* h, void* stream);

/* ---------------------------------------------------------------- router --
 * Top-k experts per token from fp32 router logits [T, E] (replaces the
 * reference's fused router_topk, engine/patches/decode-fusion/
 * fused_kernels.py:363-371, and the stock softmax / argpartition / take /
 * renormalise of qwen3_5_moe/language.py:65-71): idx[t, j] the j-th largest
 * logit's expert (descending, ties to the lower index), scores[t, j] fp32:
 * norm != 0: exp(l_j - l_0) / sum_{j<k} exp(l_j - l_0); norm == 0: the full
 * softmax probability.  k <= 64, E <= 1024; logits are expected finite (a
 * NaN ranks below every number, after which ties go to the lower index). */
int qmoe_router_topk(const float* logits, int64_t T, int64_t E, int64_t k,
                     int norm, int32_t* idx, float* scores, void* stream);

/* Router logits in fp32 from an affine-quantized router weight [E, K*bits/32]
 * (replaces the fused router's quantized matvec,
 * engine/patches/decode-fusion/fused_kernels.py:232-260, 353-363):
 * logits[t, e] = s*sum(x*q) + b*sum(x) per group, fp32 accumulation, no
 * dequantised weight.  The GEMV kernels of qmoe_quantized_matmul with an fp32
 * store; same bit widths and group sizes. */
int qmoe_router_logits(const uint16_t* x, int64_t T, int64_t K,
                       const uint32_t* w, const uint16_t* scales,
                       const uint16_t* biases, int64_t E, int group_size,
                       int bits, float* logits, void* stream);

/* Router logits in fp32 from a dense bf16 router weight [E, K] (the
 * unquantised nn.Linear gate, qwen3_5_moe/language.py:52, 61):
 * logits[t, e] = sum_k x[t, k] * W[e, k], fp32 accumulation.  K % 8 == 0.
 * Any T: one wave per (token, expert) at decode widths, a tiled bf16 MFMA
 * GEMM from 48 tokens on (when E >= 32 and K % 128 == 0). */
int qmoe_router_logits_dense(const uint16_t* x, int64_t T, int64_t K,
                             const uint16_t* w, int64_t E, float* logits,
                             void* stream);

#ifdef __cplusplus
}
#endif
#endif /* QMOE_H */

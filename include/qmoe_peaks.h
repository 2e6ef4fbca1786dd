/*
 * qmoe_peaks.h -- measured-ceiling probes for MI355X (libqmoe_peaks.so).
 *
 * Not part of the MoE path: bench.py times these to report its roofline
 * fractions against what this part sustains as well as against the vendor
 * figures (the reference's method: measure the device's own peaks with a
 * read kernel and a matrix-unit loop, engine/patches/prefill-int4/peak_table.py:1-30).
 * Same conventions as qmoe.h: device pointers, caller-owned buffers, launches
 * on `stream`, no host synchronisation, 0 on success.
 */
#ifndef QMOE_PEAKS_H
#define QMOE_PEAKS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Reads `bytes` (a multiple of 16, 16-byte aligned) once with 16-byte
 * non-temporal loads from every CU; folds what it read into sink[block]
 * (sink holds qmoe_peak_stream_blocks() words) so nothing is optimised away. */
int qmoe_peak_stream_blocks(void);
int qmoe_peak_stream_read(const void* buf, size_t bytes, uint32_t* sink, void* stream);

/* Dense matrix-unit loops over register operands seeded per lane:
 * qmoe_peak_mfma_waves() waves each issue `iters` x 4 independent
 * v_mfma_f32_32x32x16_bf16 (32768 flops each) or v_mfma_i32_32x32x32_i8
 * (65536 ops each).  sink holds one word per wave. */
int qmoe_peak_mfma_waves(void);
int qmoe_peak_mfma_bf16(int iters, uint32_t* sink, void* stream);
int qmoe_peak_mfma_i8(int iters, uint32_t* sink, void* stream);

/* The per-call floor of a decode step that is one launch of waves, in
 * workgroups of waves_per_block (1, 2 or 4) waves.  qmoe_peak_launch: `waves`
 * waves that do nothing.  qmoe_peak_chain: slots * (rows_per_expert /
 * rows_per_block) waves; wave (slot, rb) reads ids[slot] (clamped to
 * [0, num_experts)), then the first 64 16-byte units of row
 * rb * rows_per_block of that expert's rows in w (num_experts x
 * rows_per_expert rows of row_bytes bytes, 16-byte aligned; row_bytes a
 * multiple of 16 and at least 1024), and writes one word to sink[wave].
 * Returns 1 on arguments that break these rules (including a wave count that
 * waves_per_block does not divide). */
int qmoe_peak_launch(int waves, int waves_per_block, void* stream);
int qmoe_peak_chain(const int32_t* ids, int slots, int num_experts, const void* w, int rows_per_expert,
                    int row_bytes, int rows_per_block, int waves_per_block, uint32_t* sink, void* stream);

/* qmoe_peak_burst: qmoe_peak_chain's waves, each reading, after its id, all
 * of its rows_per_block rows of row_bytes bytes (contiguous: 4, 8 or 16 KiB per
 * wave, one 16-byte load per lane and KiB) and the rows' scale and bias
 * bytes, srow_bytes per row in s and in b (num_experts x rows_per_expert rows
 * each, 16-byte aligned; rows_per_block * srow_bytes a multiple of 16 and at
 * most 1024), in workgroups of 1, 2, 4 or 10 waves: the memory work of a
 * decode GEMV that learns its experts before reading their weights, without
 * its arithmetic.  Returns 1 on arguments that break these rules. */
int qmoe_peak_burst(const int32_t* ids, int slots, int num_experts, const void* w, const void* s, const void* b,
                    int rows_per_expert, int row_bytes, int srow_bytes, int rows_per_block, int waves_per_block,
                    uint32_t* sink, void* stream);

/* One single-wave launch that writes the GPU's constant 100 MHz clock
 * (s_memrealtime, 10 ns ticks) to stamps[slot] (slot >= 0, within the
 * caller's buffer).  Returns 1 on a null buffer or a negative slot. */
int qmoe_peak_stamp(uint64_t* stamps, int slot, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* QMOE_PEAKS_H */

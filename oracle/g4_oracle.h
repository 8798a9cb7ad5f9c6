/*
 * CPU restatement of the reference's wNa8o8 projection path and PLE gather.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the product library links, loads or calls this code.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it, and only as the
 * checker (or the timed CPU baseline), never as the thing measured or shipped.
 *
 * Every function cites the reference file:line it restates (paths relative to the reference repo
 * Ar5en1c/gemma4-webgpu-engine). The reference is TypeScript + WGSL; its own oracles are JS
 * functions co-located with each kernel. These are written in C from their published behaviour.
 *
 * Parity pins (what checks each function, in tests/test_oracle_*.py):
 *   or_round_ties_even     np.rint over every half integer in [-300,300] and 1e6 random f32
 *   or_srq_code            the in-tree known answer srqCodes(-11.435039520263672, 0.6181102395057678)
 *                          = -18 (quant.ts:324-329), numpy f32 divide + rint on 1e6 values
 *   or_unpack_* / or_pack  brute force over all 256 byte values; pack(unpack) = identity
 *   or_qgemv / or_qgemm    numpy f64 dequantized matmul on exact-grid fixtures (the reference's own
 *                          fixture recipe, qgemv.ts:1365-1388), integer matmul on random codes
 *   or_qmatmul8            same, plus the serial f32 order brute-forced in Python on tiny K
 *   or_embed_gather        numpy gather + f64 dequant; float16 conversion via numpy astype
 *   or_f32_to_f16_bits     numpy astype(float16) over 2^20 random and all edge values
 *   or_plan_table_split    the three known answers quoted in tableSplit.ts:13-77 and embedGather.ts
 *   or_qgemv_split_scaled  per-band sums checked against numpy slices; fold vs numpy cumulative f32
 *   or_qgemv8_ref_lanes    equals fround(exact) whenever every lane partial < 2^24 (checked), and
 *                          brute-forced against a pure-Python replay of the 32-lane butterfly
 *   or_ple_gate_split      the buffer read as numpy [N/4][splits][4] equals or_qgemv_split's
 *                          [N][splits] partials; the bands sum to the unsplit exact accumulator
 *   or_ple_fold_gate       fold(gate split) equals the unsplit qgemv-8bit f32 output (or_qgemv with
 *                          outScale gate_out) bit for bit at every split count; a pure-Python
 *                          replay on tiny K; ties and clamps at the gate snap
 *   or_qgemv_tile8u        calibrated: equals or_qgemv (the classic oracle) bit for bit on random
 *                          codes (the same exact integer); f32 on exact-grid fixtures equals
 *                          or_qgemv bit for bit (every order is exact there); f32 on random data
 *                          within 2^-18 relative of or_qgemv's f64 sum and equal to a pure-Python
 *                          replay of the lane order and the butterfly on tiny K; a dropped zero
 *                          point or a transposed lane mapping fails the grid check
 */
#ifndef G4_ORACLE_H
#define G4_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* quant.ts:350-357 roundTiesToEven, in f32. */
float or_round_ties_even(float x);

/* quant.ts:309-334 srqCodes for one value at 8 bits: clamp(RNE(f32(v / s)), -128, 127) as an
 * integer-valued f32 (negative zero kept, NaN propagates). s == 0 returns 0. */
float or_srq_code_f32(float v, float s);

/* The same code as an int8. The reference's WGSL casts clamp(round(v/s)) to i32, and WGSL clamp is
 * min(max(e, lo), hi) with NaN-ignoring max, so NaN lands on -128 (qgemv.ts:620-626). */
int8_t or_srq_code(float v, float s);

/* quant.ts:278-288 applySrq over n values (in place allowed). */
void or_apply_srq(const float *v, int64_t n, float s, float *out);

/* quant.ts:309-334 srqCodes over n values, as int8 (NaN -> -128 as above). */
void or_srq_codes(const float *v, int64_t n, float s, int8_t *out);

/* quant.ts:87-96 unpackInt4, :121-129 unpackInt8, :139-152 packCodes (bits 4 or 8). */
void or_unpack_int4(const uint8_t *packed, int64_t width, int8_t *out);
void or_unpack_int8(const uint8_t *packed, int64_t width, int8_t *out);
void or_pack_codes(int bits, const int8_t *codes, int64_t width, uint8_t *out);

/* f16Cast.ts:120-155 f32ToF16Bits (round to nearest even, overflow to inf, NaN quiet). */
uint16_t or_f32_to_f16_bits(float v);
/* f16Cast.ts f16BitsToF32 (exact). */
float or_f16_bits_to_f32(uint16_t h);

/*
 * qgemv.ts:1131-1176 qgemvOracle for bits 4 or 8 over num_rows rows of row-major packed weights.
 *   calibrated (in_scale != 0): xq = srqCodes(x, in_scale); acc = sum(wcode * xq) exact;
 *     y = f32(f32(in_scale * scale[r]) * f32(acc))
 *   uncalibrated: sum(wcode * x) in f64 (the JS double), then y = f32(scale[r] * f32(sum))
 *   then applySrq(y, out_scale).
 * out_f32 (reference dst), acc (exact i32 sum, calibrated only) and codes (int8 q, out_scale != 0)
 * are each optional (NULL). Returns 0, or -1 on a bad argument.
 */
int or_qgemv(int bits, const uint8_t *packed, const float *scales, const float *x,
             int64_t num_rows, int64_t k, float in_scale, float out_scale,
             float *out_f32, int32_t *acc, int8_t *codes);

/* qgemm.ts:532-552 qgemmOracle and qgemvWide.ts:452-468: the GEMV per token column. x is [m][k]
 * row major, outputs are [m][num_rows] (dst[col * N + row]). Parallel over columns (OpenMP). */
int or_qgemm(int bits, const uint8_t *packed, const float *scales, const float *x,
             int64_t num_rows, int64_t k, int64_t m_cols, float in_scale, float out_scale,
             float *out_f32, int32_t *acc, int8_t *codes);

/* pleMatmul.ts:176-229 qmatmul8Oracle: I8 weights; calibrated identical to or_qgemm(8); the
 * uncalibrated path mirrors the shader's serial vec4 order in f32. */
int or_qmatmul8(const uint8_t *packed, const float *scales, const float *x,
                int64_t num_rows, int64_t k, int64_t m_cols, float in_scale, float out_scale,
                float *out_f32);

/*
 * qgemv.ts:521-548 + :1267-1290: the split-K build of the classic 4/8-bit loop, one word per lane.
 * Iteration slots are kIters = kWords / 32 whole iterations plus the guarded tail; the band of split
 * s is slots [s*per, s*per+per) with per = ceil(slots / splits). exact = 0 writes the scaled partial
 * f32(f32(xs*scale)*f32(sum)) (qgemv-4bit-split); exact = 1 writes f32(sum) (exactSplit.ts:16).
 * partials is [num_rows][splits].
 */
int or_qgemv_split(int bits, const uint8_t *packed, const float *scales, const float *x,
                   int64_t num_rows, int64_t k, int splits, int exact, float in_scale,
                   float *partials);

/* attnPrologue.ts:287-296 foldPartialsOracle / qgemv.ts:1027-1072 qgemv-merge: ascending f32 sum
 * of the partials of each row, then applySrq(out_scale). */
void or_qgemv_merge(const float *partials, int64_t num_rows, int splits, float out_scale,
                    float *out);

/* exactSplit.ts:45-57 qgemv-exact-merge: t = ascending f32 sum; v = f32(f32(in*scale[r]) * t);
 * snapped when out_scale != 0. */
void or_qgemv_exact_merge(const float *partials, const float *scales, int64_t num_rows,
                          int splits, float in_scale, float out_scale, float *out);

/* pleSplit.ts:17-23 ple-gate-split: the exact 8-bit split partials of or_qgemv_split (exact = 1,
 * qgemv.ts:521-548 with exactPartials) laid out for the fold's vec4 read,
 * partials[(row / 4) * 4 * splits + split * 4 + row % 4]. num_rows % 4 == 0. Returns 0 or -1. */
int or_ple_gate_split(const uint8_t *packed, const float *scales, const float *x,
                      int64_t num_rows, int64_t k, int splits, float in_scale, float *partials);

/* pleSplit.ts:33-41 foldGate over k gate elements: total = the splits' partials summed in split
 * order from 0 (the layout above, read as vec4 [k / 4][splits]); v = f32(f32(gate_in *
 * gate_scales[i]) * total); applySrq(v, gate_out). out[k]. */
void or_ple_fold_gate(const float *partials, int64_t k, int splits, const float *gate_scales,
                      float gate_in, float gate_out, float *out);

/* The reference qgemv-8bit reduction structure (qgemv.ts:497-519, 680; subgroupReduce.ts:49-59):
 * 32 lanes, lane l sums words l + 32 i exactly in i32, f32(acc) per lane, then the f32 xor
 * butterfly 1,2,4,8,16. Returns that f32 sum for one row of codes, so a test can say when the
 * reference's per-lane handoff rounds (partials above 2^24) and where it agrees with fround(exact). */
float or_qgemv_ref_lane_sum(int bits, const uint8_t *row_packed, const int8_t *xq, int64_t k);

/* qgemv.ts:870-1015, the tile8u loop of qgemv-4bit, over the ROW layout (the tile layout is a
 * permutation of the same codes): calibrated, the exact integer sum per lane, f32 per lane, then
 * the sgSum32 butterfly; uncalibrated, the loop's own f32 order per lane (k = 128 i + 4 l + j),
 * then the butterfly. x is f32 (the gelu prologue's values already formed). out_f32 / codes as
 * or_qgemv. Returns 0, or non-zero when K is not a multiple of 128. */
int or_qgemv_tile8u(const uint8_t *packed, const float *scales, const float *x, int64_t num_rows,
                    int64_t k, float in_scale, float out_scale, float *out_f32, int8_t *codes);

/*
 * embedGather.ts:319-344 embedGatherOracle (4-bit row layout) with the sliced guard of
 * embedGather.ts:188-196: slots whose id is outside [slice_start, slice_start + slice_count) are
 * left untouched (only when sliced != 0). Codes are the slice's rows (local row = id - start);
 * scales are addressed by the absolute row. out = f32((code - 8) * f32(16 * scale)).
 * scale_kind: 0 = f32 scales, 1 = fp16 scales (widened exactly). out_kind: 0 = f32, 1 = fp16
 * (f32ToF16Bits of the f32 value), 2 = int8 code - 8.
 */
int or_embed_gather(const uint8_t *codes, const void *scales, int scale_kind, const int32_t *ids,
                    int64_t slots, int64_t cols, int64_t group_size, int64_t groups_per_row,
                    int sliced, int64_t slice_start, int64_t slice_count, void *out, int out_kind);

/* tableSplit.ts:125-215 planTableSplit. Fills up to max_slices slices (start, count pairs) and
 * returns the slice count (0 when infeasible: one row does not fit). rows_per_slice and
 * limit_bytes are written when non NULL. */
int64_t or_plan_table_split(int64_t rows, int64_t row_bytes, int64_t max_binding,
                            int64_t max_buffer, int64_t max_slice_bytes, int64_t *limit_bytes,
                            int64_t *rows_per_slice, int64_t *starts, int64_t *counts,
                            int64_t max_slices);

/* Number of OpenMP threads the parallel oracles use. */
int or_num_threads(void);

#ifdef __cplusplus
}
#endif

#endif

/*
 * CPU restatement of the reference's wNa8o8 projection path and PLE gather.
 * TEST INFRASTRUCTURE ONLY: see g4_oracle.h for what may use it and what pins each function.
 *
 * Build: gcc -O2 -fopenmp -ffp-contract=off -fno-fast-math (oracle/Makefile). Every float
 * operation below is a single correctly rounded binary32 (or, where the reference's JS oracle
 * works in doubles, binary64) operation in the order written; FMA contraction is off.
 */
#include "g4_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

int or_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* quant.ts:350-357. Exactly on a half: step to the even neighbour; otherwise Math.round, which for
 * a non-tie is the nearest integer with the sign of a zero result kept (-0.3 -> -0). */
float or_round_ties_even(float x) {
    if (!isfinite(x)) return x;
    float t = truncf(x);
    float f = x - t; /* exact: t and x share sign and exponent range */
    if (f != 0.5f && f != -0.5f) {
        /* Math.round(x) = floor(x + 0.5) in f64, exact for an f32 x; -0 kept for x in [-0.5, 0). */
        float r = (float)floor((double)x + 0.5);
        if (r == 0.0f && signbit(x)) r = -0.0f;
        return r;
    }
    if (fmodf(t, 2.0f) == 0.0f) return t;
    return t + (f > 0 ? 1.0f : -1.0f);
}

/* quant.ts:309-334 at 8 bits: the f32 quotient, ties to even, clamp with NaN passing through. */
float or_srq_code_f32(float v, float s) {
    if (!isfinite(s) || s == 0.0f) return 0.0f;
    float q = v / s; /* IEEE binary32 divide == Math.fround(f64 quotient) for f32 operands */
    float r = or_round_ties_even(q);
    if (r < -128.0f) return -128.0f;
    if (r > 127.0f) return 127.0f;
    return r;
}

int8_t or_srq_code(float v, float s) {
    float r = or_srq_code_f32(v, s);
    if (isnan(r)) return -128;
    return (int8_t)(int)r;
}

void or_apply_srq(const float *v, int64_t n, float s, float *out) {
    if (!isfinite(s) || s == 0.0f) {
        if (out != v) memmove(out, v, (size_t)n * sizeof(float));
        return;
    }
    for (int64_t i = 0; i < n; i++) {
        float c = or_srq_code_f32(v[i], s);
        out[i] = c * s;
    }
}

void or_srq_codes(const float *v, int64_t n, float s, int8_t *out) {
    for (int64_t i = 0; i < n; i++) out[i] = or_srq_code(v[i], s);
}

/* quant.ts:87-96: low nibble first, minus the zero point 8. */
void or_unpack_int4(const uint8_t *packed, int64_t width, int8_t *out) {
    for (int64_t i = 0; i < width; i++) {
        uint8_t b = packed[i >> 1];
        int nib = (i & 1) ? ((b >> 4) & 0x0f) : (b & 0x0f);
        out[i] = (int8_t)(nib - 8);
    }
}

/* quant.ts:121-129: the signed byte is the code. */
void or_unpack_int8(const uint8_t *packed, int64_t width, int8_t *out) {
    for (int64_t i = 0; i < width; i++) out[i] = (int8_t)packed[i];
}

/* quant.ts:139-152. */
void or_pack_codes(int bits, const int8_t *codes, int64_t width, uint8_t *out) {
    if (bits == 8) {
        for (int64_t i = 0; i < width; i++) out[i] = (uint8_t)codes[i];
        return;
    }
    int64_t nbytes = (width + 1) / 2;
    memset(out, 0, (size_t)nbytes);
    for (int64_t i = 0; i < width; i++) {
        int code = (int)codes[i] + 8;
        out[i >> 1] |= (uint8_t)((code & 0x0f) << ((i & 1) * 4));
    }
}

/* f16Cast.ts:120-155. */
uint16_t or_f32_to_f16_bits(float value) {
    uint32_t x;
    memcpy(&x, &value, 4);
    uint32_t sign = (x >> 31) << 15;
    uint32_t exp = (x >> 23) & 0xff;
    uint32_t mant = x & 0x7fffff;
    if (exp == 0xff) return (uint16_t)(sign | 0x7c00 | (mant != 0 ? 0x200 : 0));
    int32_t e = (int32_t)exp - 112;
    if (e >= 0x1f) return (uint16_t)(sign | 0x7c00);
    if (e > 0) {
        uint32_t bits = sign | ((uint32_t)e << 10) | (mant >> 13);
        uint32_t rem = mant & 0x1fff;
        if (rem > 0x1000 || (rem == 0x1000 && ((mant >> 13) & 1) == 1)) bits += 1;
        return (uint16_t)(bits & 0xffff);
    }
    if (e < -10) return (uint16_t)sign;
    uint32_t m = mant | 0x800000;
    uint32_t shift = (uint32_t)(14 - e);
    uint32_t half = m >> shift;
    uint32_t rem = m & ((1u << shift) - 1);
    uint32_t halfway = 1u << (shift - 1);
    if (rem > halfway || (rem == halfway && (half & 1) == 1)) half += 1;
    return (uint16_t)((sign | half) & 0xffff);
}

float or_f16_bits_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000) << 16;
    uint32_t exp = (h >> 10) & 0x1f;
    uint32_t mant = h & 0x3ff;
    uint32_t bits;
    if (exp == 0) {
        if (mant == 0) {
            bits = sign;
        } else {
            /* subnormal: value = mant * 2^-24, exact in f32 */
            float f = (float)mant * 5.9604644775390625e-08f;
            memcpy(&bits, &f, 4);
            bits |= sign;
        }
    } else if (exp == 0x1f) {
        bits = sign | 0x7f800000 | (mant << 13);
    } else {
        bits = sign | ((exp + 112) << 23) | (mant << 13);
    }
    float out;
    memcpy(&out, &bits, 4);
    return out;
}

static int row_bytes_for(int bits, int64_t k) { return bits == 4 ? (int)((k + 1) / 2) : (int)k; }

static void unpack_row(int bits, const uint8_t *row, int64_t k, int8_t *codes) {
    if (bits == 4) or_unpack_int4(row, k, codes);
    else or_unpack_int8(row, k, codes);
}

/* One column of qgemvOracle (qgemv.ts:1131-1176) over the rows [r0, r1). */
static void qgemv_column(int bits, const uint8_t *packed, const float *scales, const float *x,
                         int64_t num_rows, int64_t k, float in_scale, float out_scale,
                         const int8_t *xq, float *out_f32, int32_t *acc, int8_t *codes,
                         int8_t *scratch) {
    int calibrated = isfinite(in_scale) && in_scale != 0.0f;
    int64_t rb = row_bytes_for(bits, k);
    for (int64_t r = 0; r < num_rows; r++) {
        unpack_row(bits, packed + r * rb, k, scratch);
        float scale = isfinite(scales[r]) ? scales[r] : 0.0f;
        float y;
        if (calibrated) {
            int64_t sum = 0;
            for (int64_t i = 0; i < k; i++) sum += (int64_t)scratch[i] * (int64_t)xq[i];
            if (acc) acc[r] = (int32_t)sum;
            float xs_s = in_scale * scale;
            y = xs_s * (float)sum;
        } else {
            double sum = 0.0; /* the JS double of qgemvOracle */
            for (int64_t i = 0; i < k; i++) sum += (double)scratch[i] * (double)x[i];
            if (acc) acc[r] = 0;
            float xs_s = 1.0f * scale;
            y = xs_s * (float)sum;
        }
        float snapped = y;
        if (isfinite(out_scale) && out_scale != 0.0f) {
            float c = or_srq_code_f32(y, out_scale);
            snapped = c * out_scale;
            if (codes) codes[r] = isnan(c) ? (int8_t)-128 : (int8_t)(int)c;
        } else if (codes) {
            codes[r] = 0;
        }
        if (out_f32) out_f32[r] = snapped;
    }
}

int or_qgemv(int bits, const uint8_t *packed, const float *scales, const float *x,
             int64_t num_rows, int64_t k, float in_scale, float out_scale,
             float *out_f32, int32_t *acc, int8_t *codes) {
    return or_qgemm(bits, packed, scales, x, num_rows, k, 1, in_scale, out_scale, out_f32, acc,
                    codes);
}

int or_qgemm(int bits, const uint8_t *packed, const float *scales, const float *x,
             int64_t num_rows, int64_t k, int64_t m_cols, float in_scale, float out_scale,
             float *out_f32, int32_t *acc, int8_t *codes) {
    if ((bits != 4 && bits != 8) || k <= 0 || num_rows <= 0 || m_cols <= 0) return -1;
    int calibrated = isfinite(in_scale) && in_scale != 0.0f;
    int64_t rb = row_bytes_for(bits, k);
    /* Parallel over (column, row block): every output is independent. */
    int64_t row_block = 64;
    int64_t blocks = (num_rows + row_block - 1) / row_block;
    int64_t total = blocks * m_cols;
    int fail = 0;
#pragma omp parallel
    {
        int8_t *scratch = (int8_t *)malloc((size_t)k);
        int8_t *xq = (int8_t *)malloc((size_t)k);
        int64_t last_col = -1;
        if (!scratch || !xq) fail = 1;
#pragma omp for schedule(dynamic, 1)
        for (int64_t t = 0; t < total; t++) {
            if (!scratch || !xq) continue;
            int64_t col = t / blocks;
            int64_t b = t % blocks;
            int64_t r0 = b * row_block;
            int64_t r1 = r0 + row_block < num_rows ? r0 + row_block : num_rows;
            const float *xc = x + col * k;
            if (calibrated && col != last_col) {
                or_srq_codes(xc, k, in_scale, xq);
                last_col = col;
            }
            int64_t o = col * num_rows + r0;
            qgemv_column(bits, packed + r0 * rb, scales + r0, xc, r1 - r0, k, in_scale, out_scale,
                         xq, out_f32 ? out_f32 + o : NULL, acc ? acc + o : NULL,
                         codes ? codes + o : NULL, scratch);
        }
        free(scratch);
        free(xq);
    }
    return fail ? -1 : 0;
}

/* pleMatmul.ts:176-229. */
int or_qmatmul8(const uint8_t *packed, const float *scales, const float *x,
                int64_t num_rows, int64_t k, int64_t m_cols, float in_scale, float out_scale,
                float *out_f32) {
    if (k <= 0 || (k % 4) != 0 || num_rows <= 0 || m_cols <= 0) return -1;
    int calibrated = isfinite(in_scale) && in_scale != 0.0f;
    if (calibrated)
        return or_qgemm(8, packed, scales, x, num_rows, k, m_cols, in_scale, out_scale, out_f32,
                        NULL, NULL);
    int64_t kw = k / 4;
#pragma omp parallel for schedule(static)
    for (int64_t t = 0; t < num_rows * m_cols; t++) {
        int64_t col = t / num_rows, r = t % num_rows;
        const int8_t *codes = (const int8_t *)(packed + r * k);
        const float *xc = x + col * k;
        float sum = 0.0f;
        for (int64_t w = 0; w < kw; w++) {
            float d = 0.0f;
            for (int j = 0; j < 4; j++) {
                float p = (float)codes[w * 4 + j] * xc[w * 4 + j];
                d = d + p;
            }
            sum = sum + d;
        }
        float scale = isfinite(scales[r]) ? scales[r] : 0.0f;
        float y = (1.0f * scale) * sum;
        float v = y;
        if (isfinite(out_scale) && out_scale != 0.0f) v = or_srq_code_f32(y, out_scale) * out_scale;
        out_f32[col * num_rows + r] = v;
    }
    return 0;
}

/* qgemv.ts:521-548 band arithmetic for the classic loop at one word per lane. */
int or_qgemv_split(int bits, const uint8_t *packed, const float *scales, const float *x,
                   int64_t num_rows, int64_t k, int splits, int exact, float in_scale,
                   float *partials) {
    if ((bits != 4 && bits != 8) || splits < 1 || k <= 0 || num_rows <= 0) return -1;
    int64_t codes_per_word = bits == 4 ? 8 : 4;
    if (k % codes_per_word) return -1;
    int64_t k_words = k / codes_per_word;
    int64_t k_iters = k_words / 32;
    int64_t slots = k_iters + (exact ? ((k_words % 32) != 0 ? 1 : 0) : 1);
    int64_t per = (slots + splits - 1) / splits;
    int calibrated = isfinite(in_scale) && in_scale != 0.0f;
    int64_t rb = row_bytes_for(bits, k);
    int8_t *xq = (int8_t *)malloc((size_t)k);
    if (!xq) return -1;
    if (calibrated) or_srq_codes(x, k, in_scale, xq);
    int fail = 0;
#pragma omp parallel
    {
        int8_t *codes = (int8_t *)malloc((size_t)k);
        if (!codes) fail = 1;
#pragma omp for schedule(static)
        for (int64_t r = 0; r < num_rows; r++) {
            if (!codes) continue;
            unpack_row(bits, packed + r * rb, k, codes);
            float scale = isfinite(scales[r]) ? scales[r] : 0.0f;
            for (int s = 0; s < splits; s++) {
                int64_t lo = s * per < slots ? s * per : slots;
                int64_t hi = lo + per < slots ? lo + per : slots;
                /* iterations [lo, min(hi, kIters)) are whole; the tail belongs to hi > kIters */
                int64_t w_lo = lo * 32;
                int64_t w_hi = (hi < k_iters ? hi : k_iters) * 32;
                if (hi > k_iters) w_hi = k_words;
                if (w_lo > w_hi) w_lo = w_hi;
                int64_t c_lo = w_lo * codes_per_word, c_hi = w_hi * codes_per_word;
                float part;
                if (calibrated) {
                    int64_t sum = 0;
                    for (int64_t i = c_lo; i < c_hi; i++) sum += (int64_t)codes[i] * xq[i];
                    part = exact ? (float)sum : (in_scale * scale) * (float)sum;
                } else {
                    double sum = 0.0;
                    for (int64_t i = c_lo; i < c_hi; i++) sum += (double)codes[i] * (double)x[i];
                    part = exact ? (float)sum : (1.0f * scale) * (float)sum;
                }
                partials[r * splits + s] = part;
            }
        }
        free(codes);
    }
    free(xq);
    return fail ? -1 : 0;
}

void or_qgemv_merge(const float *partials, int64_t num_rows, int splits, float out_scale,
                    float *out) {
    for (int64_t r = 0; r < num_rows; r++) {
        float t = 0.0f;
        for (int s = 0; s < splits; s++) t = t + partials[r * splits + s];
        out[r] = t;
    }
    or_apply_srq(out, num_rows, out_scale, out);
}

void or_qgemv_exact_merge(const float *partials, const float *scales, int64_t num_rows,
                          int splits, float in_scale, float out_scale, float *out) {
    for (int64_t r = 0; r < num_rows; r++) {
        float t = 0.0f;
        for (int s = 0; s < splits; s++) t = t + partials[r * splits + s];
        float v = (in_scale * scales[r]) * t;
        or_apply_srq(&v, 1, out_scale, &v);
        out[r] = v;
    }
}

int or_ple_gate_split(const uint8_t *packed, const float *scales, const float *x,
                      int64_t num_rows, int64_t k, int splits, float in_scale, float *partials) {
    if (num_rows <= 0 || num_rows % 4 || splits < 1) return -1;
    float *rm = (float *)malloc((size_t)num_rows * (size_t)splits * sizeof(float));
    if (!rm) return -1;
    int rc = or_qgemv_split(8, packed, scales, x, num_rows, k, splits, 1, in_scale, rm);
    if (rc == 0)
        for (int64_t r = 0; r < num_rows; r++)
            for (int s = 0; s < splits; s++)
                partials[(r / 4) * 4 * splits + s * 4 + r % 4] = rm[r * splits + s];
    free(rm);
    return rc;
}

void or_ple_fold_gate(const float *partials, int64_t k, int splits, const float *gate_scales,
                      float gate_in, float gate_out, float *out) {
    for (int64_t i = 0; i < k; i++) {
        float total = 0.0f;
        for (int s = 0; s < splits; s++) total = total + partials[(i / 4) * 4 * splits + s * 4 + i % 4];
        float v = (gate_in * gate_scales[i]) * total;
        or_apply_srq(&v, 1, gate_out, &v);
        out[i] = v;
    }
}

float or_qgemv_ref_lane_sum(int bits, const uint8_t *row_packed, const int8_t *xq, int64_t k) {
    int64_t cpw = bits == 4 ? 8 : 4;
    int64_t k_words = k / cpw;
    float lane[32];
    for (int l = 0; l < 32; l++) {
        int64_t acc = 0; /* i32 in the shader; exact while it fits, which it does for K <= 131072 */
        for (int64_t w = l; w < k_words; w += 32) {
            for (int64_t j = 0; j < cpw; j++) {
                int64_t i = w * cpw + j;
                int code;
                if (bits == 4) {
                    uint8_t b = row_packed[i >> 1];
                    code = ((i & 1) ? (b >> 4) : b) & 0x0f;
                    code -= 8;
                } else {
                    code = (int8_t)row_packed[i];
                }
                acc += (int64_t)code * xq[i];
            }
        }
        lane[l] = (float)(int32_t)acc;
    }
    for (int m = 1; m < 32; m <<= 1) {
        float nxt[32];
        for (int l = 0; l < 32; l++) nxt[l] = lane[l] + lane[l ^ m];
        memcpy(lane, nxt, sizeof(lane));
    }
    return lane[0];
}

int or_embed_gather(const uint8_t *codes, const void *scales, int scale_kind, const int32_t *ids,
                    int64_t slots, int64_t cols, int64_t group_size, int64_t groups_per_row,
                    int sliced, int64_t slice_start, int64_t slice_count, void *out, int out_kind) {
    if (cols <= 0 || (cols % 8) != 0 || group_size <= 0 || cols % group_size != 0) return -1;
    if (groups_per_row != cols / group_size) return -1;
    int64_t row_bytes = cols / 2;
    const float out_scale = 16.0f; /* PLE_EMBED_SCALE, quant.ts:46; an exact f32 literal */
#pragma omp parallel for schedule(static)
    for (int64_t slot = 0; slot < slots; slot++) {
        int64_t row = (int64_t)(uint32_t)ids[slot];
        int64_t local = row;
        if (sliced) {
            if (row < slice_start || row - slice_start >= slice_count) continue;
            local = row - slice_start;
        }
        const uint8_t *src = codes + local * row_bytes;
        for (int64_t col = 0; col < cols; col++) {
            int64_t si = row * groups_per_row + col / group_size;
            float s = scale_kind == 1 ? or_f16_bits_to_f32(((const uint16_t *)scales)[si])
                                      : ((const float *)scales)[si];
            float scale = out_scale * s;
            uint8_t b = src[col >> 1];
            int code = ((col & 1) ? (b >> 4) : b) & 0x0f;
            float v = (float)(code - 8) * scale;
            int64_t o = slot * cols + col;
            if (out_kind == 0) ((float *)out)[o] = v;
            else if (out_kind == 1) ((uint16_t *)out)[o] = or_f32_to_f16_bits(v);
            else ((int8_t *)out)[o] = (int8_t)(code - 8);
        }
    }
    return 0;
}

/* tableSplit.ts:125-215. */
int64_t or_plan_table_split(int64_t rows_in, int64_t row_bytes_in, int64_t max_binding,
                            int64_t max_buffer, int64_t max_slice_bytes, int64_t *limit_out,
                            int64_t *rows_per_slice_out, int64_t *starts, int64_t *counts,
                            int64_t max_slices) {
    int64_t rows = rows_in > 0 ? rows_in : 0;
    int64_t row_bytes = row_bytes_in > 1 ? row_bytes_in : 1;
    int64_t total = rows * row_bytes;
    int64_t limit = max_binding < max_buffer ? max_binding : max_buffer;
    if (limit < 0) limit = 0;
    if (limit_out) *limit_out = limit;
    int fits_whole = total > 0 && total <= limit;
    int64_t cap = max_slice_bytes > 0 ? max_slice_bytes : 256LL * 1024 * 1024;
    int64_t slice_cap = limit < cap ? limit : cap;
    if (slice_cap < 1) slice_cap = 1;
    int64_t rows_per_slice = (fits_whole ? limit : slice_cap) / row_bytes;
    if (rows_per_slice < 1) {
        if (rows_per_slice_out) *rows_per_slice_out = 0;
        return 0;
    }
    int64_t aligned = rows_per_slice >= 16 ? rows_per_slice - (rows_per_slice % 16) : rows_per_slice;
    int64_t per = rows < aligned ? rows : aligned;
    if (rows_per_slice_out) *rows_per_slice_out = per;
    int64_t n = 0;
    if (per > 0) {
        for (int64_t start = 0; start < rows; start += per) {
            if (n < max_slices) {
                starts[n] = start;
                counts[n] = per < rows - start ? per : rows - start;
            }
            n++;
        }
    }
    if (n == 0) {
        if (max_slices > 0) {
            starts[0] = 0;
            counts[0] = 0;
        }
        n = 1;
    }
    return n;
}

/* qgemv.ts:870-1015 qgemv4TileWgsl (the tile8u loop) on a row-layout 4-bit matrix: lane l of the
 * 32-lane group takes k = 128 i + 4 l + j (i over K / 128, j = 0..3).
 *  calibrated: exact sum(u x) and sum(x) in integers (the packed-pair arithmetic of :940-948 is
 *    exact), f32(sum(u x) - 8 sum(x)) per lane;
 *  f32: acc_r = acc_r + f32(u) * x_j, one rounding each (no contraction), sxf = sxf + x_j, in
 *    the loop's order, then acc_r - f32(8 * sxf);
 *  then sgSum32 (subgroupReduce.ts:49-59): x = x + x[l ^ m] for m = 1, 2, 4, 8, 16, lane 0's value;
 *  then f32(f32(xs * scale) * sum) (xs = in_scale, or 1 uncalibrated) and srqOut on out_scale. */
int or_qgemv_tile8u(const uint8_t *packed, const float *scales, const float *x, int64_t num_rows,
                    int64_t k, float in_scale, float out_scale, float *out_f32, int8_t *codes) {
    if (k <= 0 || k % 128 != 0) return 1;
    int calibrated = isfinite(in_scale) && in_scale != 0.0f;
    int64_t rb = k / 2, iters = k / 128;
    int8_t *xq = (int8_t *)malloc((size_t)k);
    if (!xq) return 2;
    if (calibrated)
        for (int64_t i = 0; i < k; i++) xq[i] = or_srq_code(x[i], in_scale);
#pragma omp parallel for schedule(static)
    for (int64_t row = 0; row < num_rows; row++) {
        const uint8_t *w = packed + row * rb;
        float lane[32];
        for (int l = 0; l < 32; l++) {
            if (calibrated) {
                int64_t sux = 0, sx = 0;
                for (int64_t i = 0; i < iters; i++)
                    for (int j = 0; j < 4; j++) {
                        int64_t kk = 128 * i + 4 * l + j;
                        int u = (w[kk >> 1] >> (4 * (kk & 1))) & 15;
                        sux += (int64_t)u * xq[kk];
                        sx += xq[kk];
                    }
                lane[l] = (float)(int32_t)(sux - 8 * sx);
            } else {
                float acc = 0.0f, sxf = 0.0f;
                for (int64_t i = 0; i < iters; i++)
                    for (int j = 0; j < 4; j++) {
                        int64_t kk = 128 * i + 4 * l + j;
                        int u = (w[kk >> 1] >> (4 * (kk & 1))) & 15;
                        sxf = sxf + x[kk];
                        acc = acc + (float)u * x[kk];
                    }
                float sx8f = 8.0f * sxf;
                lane[l] = acc - sx8f;
            }
        }
        for (int m = 1; m < 32; m <<= 1) {
            float nxt[32];
            for (int l = 0; l < 32; l++) nxt[l] = lane[l] + lane[l ^ m];
            memcpy(lane, nxt, sizeof(lane));
        }
        float scale = isfinite(scales[row]) ? scales[row] : 0.0f;
        float xs_s = (calibrated ? in_scale : 1.0f) * scale;
        float y = xs_s * lane[0];
        float snapped = y;
        if (isfinite(out_scale) && out_scale != 0.0f) {
            float c = or_srq_code_f32(y, out_scale);
            snapped = c * out_scale;
            if (codes) codes[row] = isnan(c) ? (int8_t)-128 : (int8_t)(int)c;
        } else if (codes) {
            codes[row] = 0;
        }
        if (out_f32) out_f32[row] = snapped;
    }
    free(xq);
    return 0;
}

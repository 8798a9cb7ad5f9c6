/*
 * CPU restatement of the decode-step glue (TEST INFRASTRUCTURE ONLY; see g4_decode_oracle.h).
 * Compiled with -ffp-contract=off: every multiply and add below rounds on its own, as the device
 * code does with __fmul_rn / __fadd_rn.
 */
#include "g4_decode_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "g4_oracle.h"

float g4d_expf(float x) {
    if (x != x) return x;
    if (x > 88.7f) return INFINITY;
    if (x < -87.0f) return 0.0f;
    const float log2e = 0x1.715476p+0f;   /* f32(log2 e) */
    const float ln2_hi = 0x1.62e4p-1f;    /* 0.693145751953125: 15 significant bits */
    const float ln2_lo = 0x1.7f7d1cp-20f; /* f32(ln 2 - ln2_hi) */
    const float n = rintf(x * log2e);
    float r = x - n * ln2_hi;
    r = r - n * ln2_lo;
    /* Taylor series to r^6 on |r| <= 0.35: truncation below 2^-24 relative */
    float p = 0x1.6c16c2p-10f;        /* f32(1/720) */
    p = p * r + 0x1.111112p-7f;       /* f32(1/120) */
    p = p * r + 0x1.555556p-5f;       /* f32(1/24) */
    p = p * r + 0x1.555556p-3f;       /* f32(1/6) */
    p = p * r + 0.5f;
    p = p * r + 1.0f;
    p = p * r + 1.0f;
    return ldexpf(p, (int)n);
}

/* exp(y) - 1 for |y| <= 0.35 (no range reduction needed): the Taylor chain of g4d_expf stopped
 * before its final "+ 1", times y, so no cancellation against 1 occurs. */
static float expm1_small(float y) {
    float p = 0x1.6c16c2p-10f;
    p = p * y + 0x1.111112p-7f;
    p = p * y + 0x1.555556p-5f;
    p = p * y + 0x1.555556p-3f;
    p = p * y + 0.5f;
    p = p * y + 1.0f;
    return p * y;
}

float g4d_tanhf(float x) {
    const float ax = fabsf(x);
    if (ax < 0x1p-12f) return x; /* tanh x = x (1 - x^2/3 + ...): below half an ulp */
    float r;
    if (ax < 0.171875f) {
        /* tanh a = -em / (2 + em) with em = expm1(-2a): exact form, no 1 - t cancellation */
        const float em = expm1_small(-2.0f * ax);
        r = -em / (2.0f + em);
    } else {
        const float t = g4d_expf(-2.0f * ax);
        r = (1.0f - t) / (1.0f + t);
    }
    return copysignf(r, x);
}

float g4d_gelu_tanh(float x) {
    const float cube = (x * x) * x;
    float inner = 0x1.988454p-1f * (x + 0x1.6e4e26p-5f * cube); /* f32(sqrt(2/pi)), f32(0.044715) */
    inner = fminf(fmaxf(inner, -10.0f), 10.0f);
    return (0.5f * x) * (1.0f + g4d_tanhf(inner));
}

/* The fixed reduction: lane l accumulates elements l, l + T, ... ascending, then a pairwise tree
 * (stride T/2 down to 1, lane l adds lane l + stride). */
static float tree_sum(float *part) {
    for (int stride = G4D_THREADS / 2; stride >= 1; stride >>= 1)
        for (int l = 0; l < stride; ++l) part[l] = part[l] + part[l + stride];
    return part[0];
}

float g4d_sumsq(const float *x, int64_t n) {
    float part[G4D_THREADS];
    for (int l = 0; l < G4D_THREADS; ++l) {
        float acc = 0.0f;
        for (int64_t i = l; i < n; i += G4D_THREADS) acc = acc + x[i] * x[i];
        part[l] = acc;
    }
    return tree_sum(part);
}

float g4d_sum(const float *x, int64_t n) {
    float part[G4D_THREADS];
    for (int l = 0; l < G4D_THREADS; ++l) {
        float acc = 0.0f;
        for (int64_t i = l; i < n; i += G4D_THREADS) acc = acc + x[i];
        part[l] = acc;
    }
    return tree_sum(part);
}

static float inv_rms(const float *x, int64_t width, float eps) {
    const float mean = g4d_sumsq(x, width) / (float)width;
    return 1.0f / sqrtf(mean + eps);
}

void g4d_rms_norm(const float *x, const float *gain, int64_t rows, int64_t width, float eps,
                  float *out) {
    for (int64_t r = 0; r < rows; ++r) {
        const float *row = x + r * width;
        float *dst = out + r * width;
        const float inv = inv_rms(row, width, eps);
        for (int64_t i = 0; i < width; ++i) {
            const float v = row[i] * inv;
            dst[i] = gain ? v * gain[i] : v;
        }
    }
}

void g4d_norm_residual(const float *src, const float *gain, const float *resid, int64_t rows,
                       int64_t width, float eps, float *out) {
    for (int64_t r = 0; r < rows; ++r) {
        const float *row = src + r * width;
        const float inv = inv_rms(row, width, eps);
        for (int64_t i = 0; i < width; ++i)
            out[r * width + i] = resid[r * width + i] + (row[i] * inv) * gain[i];
    }
}

void g4d_norm_residual_norm(const float *src, const float *gain, const float *resid,
                            const float *gain2, float alpha, int64_t rows, int64_t width,
                            float eps, float in_scale, float *hidden, int8_t *codes) {
    float *normed = (float *)malloc(sizeof(float) * (size_t)width);
    for (int64_t r = 0; r < rows; ++r) {
        const float *row = src + r * width;
        float *h = hidden + r * width;
        const float inv = inv_rms(row, width, eps);
        for (int64_t i = 0; i < width; ++i) {
            float v = resid[r * width + i] + (row[i] * inv) * gain[i];
            if (alpha != 1.0f) v = v * alpha;
            h[i] = v;
        }
        g4d_rms_norm(h, gain2, 1, width, eps, normed);
        for (int64_t i = 0; i < width; ++i) codes[r * width + i] = or_srq_code(normed[i], in_scale);
    }
    free(normed);
}

void g4d_rms_norm_codes(const float *x, const float *gain, int64_t rows, int64_t width, float eps,
                        float in_scale, int8_t *codes) {
    float *normed = (float *)malloc(sizeof(float) * (size_t)width);
    for (int64_t r = 0; r < rows; ++r) {
        g4d_rms_norm(x + r * width, gain, 1, width, eps, normed);
        for (int64_t i = 0; i < width; ++i) codes[r * width + i] = or_srq_code(normed[i], in_scale);
    }
    free(normed);
}

void g4d_rope_row(const float *x, const float *cos_row, const float *sin_row, int64_t head_dim,
                  float *out) {
    const int64_t p = head_dim / 2;
    for (int64_t i = 0; i < p; ++i) {
        const float lo = x[i], hi = x[i + p];
        const float c = cos_row[i], s = sin_row[i];
        out[i] = lo * c - hi * s;
        out[i + p] = hi * c + lo * s;
    }
}

void g4d_q_norm_rope(const int8_t *q_codes, float q_scale, const float *gain, const float *cos_row,
                     const float *sin_row, int64_t heads, int64_t head_dim, float eps, float *out) {
    float *tmp = (float *)calloc((size_t)head_dim * 2, sizeof(float));
    float *normed = tmp + head_dim;
    for (int64_t h = 0; h < heads; ++h) {
        for (int64_t i = 0; i < head_dim; ++i) tmp[i] = (float)q_codes[h * head_dim + i] * q_scale;
        g4d_rms_norm(tmp, gain, 1, head_dim, eps, normed);
        g4d_rope_row(normed, cos_row, sin_row, head_dim, out + h * head_dim);
    }
    free(tmp);
}

void g4d_kv_norm_rope(const int8_t *k_codes, float k_scale, const int8_t *v_codes, float v_scale,
                      const float *gain, const float *cos_row, const float *sin_row,
                      int64_t head_dim, float eps, float *k_row, float *v_row) {
    float *tmp = (float *)calloc((size_t)head_dim * 2, sizeof(float));
    float *normed = tmp + head_dim;
    for (int64_t i = 0; i < head_dim; ++i) tmp[i] = (float)k_codes[i] * k_scale;
    g4d_rms_norm(tmp, gain, 1, head_dim, eps, normed);
    g4d_rope_row(normed, cos_row, sin_row, head_dim, k_row);
    for (int64_t i = 0; i < head_dim; ++i) tmp[i] = (float)v_codes[i] * v_scale;
    g4d_rms_norm(tmp, NULL, 1, head_dim, eps, v_row);
    free(tmp);
}

float g4d_score(const float *q, const float *k, int64_t head_dim) {
    const int64_t seg = head_dim / 8;
    float s[8];
    for (int g = 0; g < 8; ++g) {
        float acc = 0.0f;
        for (int64_t i = g * seg; i < (g + 1) * seg; ++i) acc = fmaf(q[i], k[i], acc);
        s[g] = acc;
    }
    return ((s[0] + s[1]) + (s[2] + s[3])) + ((s[4] + s[5]) + (s[6] + s[7]));
}

void g4d_attention_decode(const float *q, const float *k, const float *v, int64_t heads,
                          int64_t head_dim, int64_t p, int64_t window, float *out) {
    const int64_t lo = window > 0 ? (p - window + 1 > 0 ? p - window + 1 : 0) : 0;
    const int64_t span = p - lo + 1;
    const int64_t chunks = (span + G4D_ATTN_CHUNK - 1) / G4D_ATTN_CHUNK;
    float *m = (float *)malloc(sizeof(float) * (size_t)chunks);
    float *l = (float *)malloc(sizeof(float) * (size_t)chunks);
    float *o = (float *)malloc(sizeof(float) * (size_t)(chunks * head_dim));
    float e[G4D_ATTN_CHUNK];
    for (int64_t h = 0; h < heads; ++h) {
        const float *qh = q + h * head_dim;
        for (int64_t c = 0; c < chunks; ++c) {
            const int64_t start = lo + c * G4D_ATTN_CHUNK;
            const int64_t end = start + G4D_ATTN_CHUNK < p + 1 ? start + G4D_ATTN_CHUNK : p + 1;
            const int64_t cnt = end - start;
            float mx = -INFINITY;
            for (int64_t j = 0; j < cnt; ++j) {
                const float d = g4d_score(qh, k + (start + j) * head_dim, head_dim);
                e[j] = d;
                if (d > mx) mx = d;
            }
            for (int64_t j = 0; j < cnt; ++j) e[j] = g4d_expf(e[j] - mx);
            m[c] = mx;
            l[c] = g4d_sum(e, cnt);
            for (int64_t i = 0; i < head_dim; ++i) {
                float a = 0.0f;
                for (int64_t j = 0; j < cnt; ++j) a = fmaf(e[j], v[(start + j) * head_dim + i], a);
                o[c * head_dim + i] = a;
            }
        }
        float M = -INFINITY;
        for (int64_t c = 0; c < chunks; ++c) M = m[c] > M ? m[c] : M;
        float L = 0.0f;
        for (int64_t c = 0; c < chunks; ++c) L = L + l[c] * g4d_expf(m[c] - M);
        for (int64_t i = 0; i < head_dim; ++i) {
            float O = 0.0f;
            for (int64_t c = 0; c < chunks; ++c) O = O + o[c * head_dim + i] * g4d_expf(m[c] - M);
            out[h * head_dim + i] = O / L;
        }
    }
    free(m);
    free(l);
    free(o);
}

void g4d_gelu_mul_codes(const int8_t *g_codes, float g_scale, const int8_t *u_codes, float u_scale,
                        const float *up_f32, int64_t n, float in_scale, int8_t *codes) {
    for (int64_t i = 0; i < n; ++i) {
        const float g = (float)g_codes[i] * g_scale;
        const float u = up_f32 ? up_f32[i] : (float)u_codes[i] * u_scale;
        codes[i] = or_srq_code(g4d_gelu_tanh(g) * u, in_scale);
    }
}

void g4d_gelu_mul_f32_codes(const float *g, const float *u, int64_t n, float in_scale,
                            int8_t *codes) {
    for (int64_t i = 0; i < n; ++i) codes[i] = or_srq_code(g4d_gelu_tanh(g[i]) * u[i], in_scale);
}

void g4d_embed_row(const uint8_t *row_codes, float row_scale, int64_t cols, float embed_scale,
                   float *out) {
    const float s = row_scale * embed_scale;
    for (int64_t i = 0; i < cols; ++i) {
        const int code = (int)((row_codes[i >> 1] >> (4 * (i & 1))) & 0xF) - 8;
        out[i] = (float)code * s;
    }
}

void g4d_ple_combine(const int8_t *proj_codes, float proj_scale, float alpha, const float *gain,
                     const float *identity, int64_t groups, int64_t group, float eps, float *out) {
    float *tmp = (float *)malloc(sizeof(float) * (size_t)group * 2);
    float *normed = tmp + group;
    const float s12 = 0x1.6a09e6p-1f; /* f32(2^-0.5) */
    for (int64_t g = 0; g < groups; ++g) {
        for (int64_t i = 0; i < group; ++i) tmp[i] = ((float)proj_codes[g * group + i] * proj_scale) * alpha;
        g4d_rms_norm(tmp, gain, 1, group, eps, normed);
        for (int64_t i = 0; i < group; ++i)
            out[g * group + i] = (normed[i] + identity[g * group + i]) * s12;
    }
    free(tmp);
}

void g4d_softcap(const float *x, int64_t n, float cap, float *out) {
    for (int64_t i = 0; i < n; ++i) out[i] = cap == 0.0f ? x[i] : g4d_tanhf(x[i] / cap) * cap;
}

int64_t g4d_argmax(const float *x, int64_t n) {
    int64_t best = -1;
    float bv = -INFINITY;
    for (int64_t i = 0; i < n; ++i)
        if (x[i] > bv) {
            bv = x[i];
            best = i;
        }
    return best;
}

/*
 * CPU restatement of the decode-step glue around the wNa8o8 projections: the RMS norms and their
 * residual joins, q/k norm + RoPE + KV store, split attention decode and its merge, gelu * up, the
 * per-layer-input combine, the token embedding, the logit softcap and the two-stage argmax.
 *
 * TEST INFRASTRUCTURE ONLY, like g4_oracle.h: only tests/ and bench.py's cpu_baseline leg use it,
 * as the checker, never as the thing measured or shipped.
 *
 * The reference (Ar5en1c/gemma4-webgpu-engine) states these kernels' CPU oracles in f64 and holds
 * its WGSL shaders to them within argued tolerances (rmsNorm.ts:191-207, attention.ts:847-857,
 * geluMul.ts:200-208, logitSoftcap.ts:95-103). This restatement is the f32 computation the HIP
 * kernels perform, written out so the GPU can be held to it bit for bit:
 *   - every reduction has a fixed order (G4D_THREADS lane-strided partial sums, then a pairwise
 *     tree; attention splits of G4D_ATTN_CHUNK positions, merged in ascending split order);
 *   - 1/sqrt is the IEEE square root then the IEEE divide (WGSL's inverseSqrt allows 2 ULP);
 *   - exp and tanh are g4d_expf / g4d_tanhf below: Cody-Waite range reduction and a degree-6
 *     Taylor polynomial, every operation separately rounded (no FMA), identical on the device;
 *   - the attention score and P·V sums take one fused multiply-add per element (C fmaf, a single
 *     IEEE rounding, as the device's v_fma_f32); every other product and sum is rounded apart;
 *   - products and sums follow the WGSL expression order of each reference shader.
 * tests/test_oracle_decode.py pins each function against the reference's own f64 formulation
 * within the reference's stated tolerance, and the math functions against libm.
 */
#ifndef G4_DECODE_ORACLE_H
#define G4_DECODE_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define G4D_THREADS 256     /* lanes of every reduction */
#define G4D_ATTN_CHUNK 32   /* positions per attention split */

/* exp(x) in f32 (returns 0 below -87, +inf above 88.7). */
float g4d_expf(float x);
/* tanh(x) in f32: x itself for |x| < 2^-12; -em / (2 + em) with em = expm1(-2|x|) (the exp
 * polynomial without its final + 1, no range reduction) for |x| < 0.171875; otherwise
 * (1 - t) / (1 + t) with t = g4d_expf(-2|x|); the sign of x applied last. */
float g4d_tanhf(float x);
/* geluMul.ts:101-116 geluTanh in the shader's order: cube = (x*x)*x,
 * inner = clamp(0.7978845608028654 * (x + 0.044715 * cube), -10, 10), (0.5*x) * (1 + tanh(inner)). */
float g4d_gelu_tanh(float x);

/* The fixed-order f32 sum of squares of n values (lane l sums l, l+256, ... ascending; tree). */
float g4d_sumsq(const float *x, int64_t n);
/* The fixed-order f32 sum of n values (same lane/tree order). */
float g4d_sum(const float *x, int64_t n);

/* rmsNorm.ts:131-180: inv = 1 / sqrt(sumsq / width + eps); out = (x * inv) * gain (gain NULL:
 * weightless). rows x width row major; out may alias x. */
void g4d_rms_norm(const float *x, const float *gain, int64_t rows, int64_t width, float eps,
                  float *out);

/* mlpEpilogue.ts:196-230 norm-residual: out = resid + (src * inv) * gain, inv from src. */
void g4d_norm_residual(const float *src, const float *gain, const float *resid, int64_t rows,
                       int64_t width, float eps, float *out);

/* blockJoin.ts:160-175 norm-residual-norm: hidden = f32(resid + (src*inv)*gain) * alpha (alpha 1:
 * no multiply), normed = rms_norm(hidden, gain2). Writes hidden and the int8 codes of normed on
 * in_scale (the next projection's input snap). */
void g4d_norm_residual_norm(const float *src, const float *gain, const float *resid,
                            const float *gain2, float alpha, int64_t rows, int64_t width,
                            float eps, float in_scale, float *hidden, int8_t *codes);

/* rmsNorm.ts input_layernorm with the next projection's snap fused: codes = srq(rms_norm(x)). */
void g4d_rms_norm_codes(const float *x, const float *gain, int64_t rows, int64_t width, float eps,
                        float in_scale, int8_t *codes);

/* rope.ts:275-303 ropeOracle, split half form, on one row of head_dim with table row (cos, sin)
 * of head_dim/2: out[i] = lo*c - hi*s, out[i+p] = hi*c + lo*s. */
void g4d_rope_row(const float *x, const float *cos_row, const float *sin_row, int64_t head_dim,
                  float *out);

/* attnPrologue.ts:268-280 q-norm-rope: q = codes * q_scale (f32), per head rms_norm(gain) then
 * rope at the position's table row. heads rows of head_dim. */
void g4d_q_norm_rope(const int8_t *q_codes, float q_scale, const float *gain, const float *cos_row,
                     const float *sin_row, int64_t heads, int64_t head_dim, float eps, float *out);

/* attnPrologue.ts:316-329 kv-norm-rope-store for one position: k = rope(rms_norm(k_codes*k_scale,
 * gain)); v = rms_norm(v_codes*v_scale) weightless; written to k_row / v_row. */
void g4d_kv_norm_rope(const int8_t *k_codes, float k_scale, const int8_t *v_codes, float v_scale,
                      const float *gain, const float *cos_row, const float *sin_row,
                      int64_t head_dim, float eps, float *k_row, float *v_row);

/*
 * attention.ts:858-918 attention decode of one query position p for `heads` heads sharing one KV
 * head, scale 1.0 (plan.ts:518-519), window w (0: unwindowed; else positions p-w+1 .. p).
 * Split form: positions lo .. p in chunks of G4D_ATTN_CHUNK; per chunk m = max score,
 * e = g4d_expf(s - m), l = fixed-order sum of e, o[d] = sum over positions ascending of e * v[d]
 * (each step one fmaf);
 * merge in ascending chunk order with w_c = g4d_expf(m_c - M): L = sum l_c * w_c,
 * O[d] = sum o_c[d] * w_c, out = O / L. A score is eight sequential f32 dot products over the
 * eighths of d, combined by a pairwise tree ((s0 + s1) + (s2 + s3)) + ((s4 + s5) + (s6 + s7))
 * (g4d_score).
 * q: [heads][head_dim]; k, v: [positions][head_dim]; out: [heads][head_dim].
 */
/* The attention score q . k over head_dim (a multiple of 8): sequential fmaf sums over each
 * eighth, then the pairwise tree ((s0 + s1) + (s2 + s3)) + ((s4 + s5) + (s6 + s7)). */
float g4d_score(const float *q, const float *k, int64_t head_dim);

void g4d_attention_decode(const float *q, const float *k, const float *v, int64_t heads,
                          int64_t head_dim, int64_t p, int64_t window, float *out);

/* geluMul.ts:219-233 gelu-mul with the consumer's snap: codes = srq(gelu(g*sg) * (u*su), in_scale)
 * where g, u are int8 codes; up_f32 (when non NULL) replaces u*su (the per-layer-input form). */
void g4d_gelu_mul_codes(const int8_t *g_codes, float g_scale, const int8_t *u_codes, float u_scale,
                        const float *up_f32, int64_t n, float in_scale, int8_t *codes);

/* The same with f32 operands (the reference's gate and up buffers): codes = srq(gelu(g) * u). */
void g4d_gelu_mul_f32_codes(const float *g, const float *u, int64_t n, float in_scale,
                            int8_t *codes);

/* embedGather.ts:93-113 token embedding with the embed scale folded once:
 * x = (code - 8) * f32(scale[row] * f32(sqrt(1536))) for an int4 row of `cols` codes. */
void g4d_embed_row(const uint8_t *row_codes, float row_scale, int64_t cols, float embed_scale,
                   float *out);

/* plan.ts:670-690 / execute.ts:522-556 per-layer input: proj = (codes * proj_scale) * alpha;
 * normed = rms_norm(proj rows of group, gain); out = (normed + identity) * f32(2^-0.5). */
void g4d_ple_combine(const int8_t *proj_codes, float proj_scale, float alpha, const float *gain,
                     const float *identity, int64_t groups, int64_t group, float eps, float *out);

/* logitSoftcap.ts:104-124 softcap: out = g4d_tanhf(x / cap) * cap (cap 0: copy). */
void g4d_softcap(const float *x, int64_t n, float cap, float *out);

/* argmax.ts:267-300: the first strict maximum (lowest index among maxima; NaN never wins). */
int64_t g4d_argmax(const float *x, int64_t n);

#ifdef __cplusplus
}
#endif

#endif

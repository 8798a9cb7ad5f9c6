/*
 * g4decode.h - the decode-step glue kernels around the wNa8o8 projections, and a native runner for
 * one whole decode step of the E2B-shape model (35 layers, hidden 1536, FFN 6144, 8 query heads
 * and one KV head of 256, tied int4 head over 262144 rows).
 *
 * Each glue entry replaces one registry kernel's bind of Ar5en1c/gemma4-webgpu-engine (the WGSL
 * kernel plus the `Kernel.bind` of src/kernels/<name>.ts); the runner replaces the dispatch walk
 * of src/plan.ts:780-792 (planDecodeStep) executed by src/execute.ts. Conventions as g4w8a8.h:
 * device pointers, G4_OK or a G4_ERR_* status with g4_last_error(), `stream` NULL = the default
 * stream, launches only (no host synchronisation), so every call can be graph-captured.
 *
 * The arithmetic is fixed (256-lane strided partial sums then a pairwise tree for every reduction,
 * IEEE sqrt then divide for 1/sqrt, one exp/tanh restatement, attention in splits of 32 positions
 * merged in ascending order with segment-wise score dot products), so the results are
 * bit-reproducible and a CPU restatement states them exactly. Every kernel that feeds a projection emits that projection's int8 input
 * snap (quant.ts:309-334 srqCodes) directly.
 */
#ifndef G4DECODE_H
#define G4DECODE_H

#include "g4w8a8.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ---- glue kernels ---------------------------------------------------------------------------- */

/*
 * rms-norm (src/kernels/rmsNorm.ts:131-180), norm-residual (src/kernels/mlpEpilogue.ts:196-230)
 * and norm-residual-norm (src/kernels/blockJoin.ts:160-175) in one entry, one row per block:
 *   y = (src * inv) * gain          inv = 1 / sqrt(sum(src^2) / width + eps); gain NULL: weightless
 *   resid given:  y = resid + y, then y * alpha when alpha != 1 (the layer scalar)
 *   hidden (optional) receives y; codes (optional) receive the snap on in_scale of
 *   (y * inv2) * gain2 when gain2 is given (the next norm), else of y itself.
 * src is f32 (src_kind G4_KIND_F32) or int8 codes times src_scale (G4_KIND_I8, a projection's
 * output). width <= 2048. hidden may alias resid.
 */
int g4_rms_join(const void *src, int src_kind, float src_scale, const float *gain,
                const float *resid, float alpha, const float *gain2, int rows, int width,
                float eps, float in_scale, float *hidden, int8_t *codes, void *stream);

/*
 * q-norm-rope and kv-norm-rope-store (src/kernels/attnPrologue.ts:268-329): per query head
 * q = rope(rms_norm(q_codes * q_scale, q_gain)) into q_out [rows][heads][256]; with k_codes given
 * (a KV producer layer) also k = rope(rms_norm(k_codes * k_scale, k_gain)) and the weightless
 * v = rms_norm(v_codes * v_scale) stored at position `pos` of the caches. RoPE is the split-half
 * form (src/kernels/rope.ts:240-258) with cos_tab / sin_tab [positions][128] host-built tables.
 * pos_dev (optional): a device int32 holding the position, read when the kernel runs (graph
 * replay); then `pos` is the largest position it may hold (the word is clamped to [0, pos]).
 * Row r of a cache starts at cache + r * cache_row_stride.
 * head_dim must be 256.
 */
int g4_attn_prologue(const int8_t *q_codes, float q_scale, const int8_t *k_codes, float k_scale,
                     const int8_t *v_codes, float v_scale, const float *q_gain,
                     const float *k_gain, const float *cos_tab, const float *sin_tab, int rows,
                     int heads, int head_dim, float eps, float *q_out, float *k_cache,
                     float *v_cache, int64_t cache_row_stride, int pos, const int32_t *pos_dev,
                     void *stream);

/*
 * attention-decode-split + attention-decode-merge (src/kernels/attention.ts:858-918; the split
 * form of plan.ts:562-570): one query position per row, `heads` query heads sharing the single KV
 * head, scale 1.0 (plan.ts:518-519), window > 0 = the last `window` positions inclusive, 0 =
 * unwindowed; heads <= 8. Output: the o_proj input codes on in_scale (codes) and/or the f32 rows
 * (out_f32),
 * [rows][heads][256]. With pos_dev, `pos` is the largest position the device word may hold (it
 * sizes the split grid and the workspace; the word is clamped to [0, pos]).
 * workspace: g4_attention_workspace_bytes(...) bytes.
 */
int g4_attention_decode(const float *q, const float *k_cache, const float *v_cache,
                        int64_t cache_row_stride, int rows, int heads, int head_dim, int pos,
                        const int32_t *pos_dev, int window, float *workspace,
                        size_t workspace_bytes, float in_scale, int8_t *codes, float *out_f32,
                        void *stream);
size_t g4_attention_workspace_bytes(int rows, int heads, int pos, int window);

/*
 * gelu-mul (src/kernels/geluMul.ts:101-116, 171-232) with the consumer's snap:
 * codes = srq(gelu_tanh(g_codes * g_scale) * u, in_scale), u = u_codes * u_scale, or (up_f32
 * given: the per-layer-input form, plan.ts:634-639) u = up_f32[row * up_stride + i].
 */
int g4_gelu_mul(const int8_t *g_codes, float g_scale, const int8_t *u_codes, float u_scale,
                const float *up_f32, int64_t up_stride, int rows, int n, float in_scale,
                int8_t *codes, void *stream);

/*
 * gelu-mul on the reference's f32 buffers (src/kernels/geluMul.ts:101-116, bind :250-278): dst[i] =
 * gelu_tanh(gate[i]) * up[i], then clamp(RNE(v / srq_scale), -128, 127) * srq_scale when srq_scale
 * != 0 (the consuming linear's input scale; 0 = uncalibrated, no rounding). count must be a
 * positive multiple of 4 (:253-255); the buffers 16-byte aligned.
 */
int g4_gelu_mul_f32(const float *gate, const float *up, float *dst, int64_t count,
                    float srq_scale, void *stream);

/*
 * The token embedding of a tied int4 table (embed-gather, src/kernels/embedGather.ts:93-113 and
 * :176-261 with the embed scale folded into the row scale once): x[r] = (code - 8) *
 * f32(row_scales[id] * embed_scale) over `cols` codes of row ids[r] (two per byte, low nibble
 * first); codes (optional) = the snap of x on in_scale (the per-layer model projection's input).
 * The table has `vocab` rows; an id outside [0, vocab) gives a zero row (and zero codes).
 */
int g4_embed_tokens(const void *table, const float *row_scales, const int32_t *ids, int rows,
                    int64_t vocab, int cols, float embed_scale, float in_scale, float *x,
                    int8_t *codes, void *stream);

/*
 * The per-layer inputs (plan.ts:670-700, execute.ts:522-556): per group of 256,
 * out = (rms_norm((proj_codes * proj_scale) * alpha, gain) + identity) * f32(2^-0.5), where alpha
 * is the projection scale hidden^-0.5 and identity the PLE gather's f32 rows. [rows][groups][256].
 */
int g4_ple_combine(const int8_t *proj_codes, float proj_scale, float alpha, const float *gain,
                   const float *identity, int rows, int groups, int group, float eps, float *out,
                   void *stream);

/*
 * logit-softcap + argmax-partial + argmax-final (src/kernels/logitSoftcap.ts:104-124,
 * src/kernels/argmax.ts:267-300): y = tanh(x / cap) * cap (cap 0: y = x), optionally stored in
 * `capped`; tokens[r] = the first strict maximum of row r (lowest index among equals; NaN never
 * wins; -1 when nothing exceeds -inf). workspace: g4_argmax_workspace_bytes(rows, vocab).
 */
int g4_softcap_argmax(const float *logits, int rows, int64_t vocab, float cap, float *capped,
                      void *workspace, size_t workspace_bytes, int32_t *tokens, void *stream);
size_t g4_argmax_workspace_bytes(int rows, int64_t vocab);

/* Seeded fills for synthetic tensors without a host round trip (no reference counterpart: the
 * reference's fixtures are host arrays). h(i) = splitmix64(seed + i);
 * f32: lo + ((h >> 40) * 2^-24) * f32(hi - lo), every step one f32 rounding; u8: h >> 56. */
int g4_fill_hash_f32(float *out, int64_t n, uint64_t seed, float lo, float hi, void *stream);
int g4_fill_hash_u8(void *out, int64_t n, uint64_t seed, void *stream);

/* ---- the decode step --------------------------------------------------------------------------- */

/* The model and run shape (plan.ts:62-82 GEMMA4_E2B, with the synthetic config's uniform FFN and
 * head_dim). Layer l is global when (l % global_period) == global_period - 1; layers below
 * kv_producers own KV caches, later ones read the last producer of their own kind (kv.ts:76-93). */
typedef struct g4_decode_shape {
    int layers;          /* 35 */
    int kv_producers;    /* 15 */
    int hidden;          /* 1536 */
    int ffn;             /* 6144 */
    int q_heads;         /* 8 */
    int head_dim;        /* 256 (the only value this build serves) */
    int ple_dim;         /* 256 */
    int global_period;   /* 5: layers 4, 9, 14, ... are global */
    int sliding_window;  /* 512 */
    int kv_capacity;     /* positions per cache, e.g. 4096 */
    int batch;           /* sequences decoded per step (1 .. 64) */
    int64_t vocab;       /* 262144 */
    float eps;           /* 1e-6 */
    float final_softcap; /* 30 */
    float in_scale;      /* the static input snap every calibrated linear uses */
    float out_scale;     /* the static output snap every calibrated linear uses */
    /* Batch 1 only, a test switch: the launch folds the runner leaves out even where they fit.
     * Bit 0: o_proj stays a GEMV plan (not inside the attention merge); bit 1: gate / up /
     * gelu-mul / down stay plans (no FFN block); bit 2: per_layer_input_gate and
     * per_layer_projection stay plans (no per-layer-input block). 0 (a zeroed shape) folds every
     * one that fits. Results are identical either way. */
    int fold_off;
} g4_decode_shape;

/* One layer's weights (device pointers). Projections: int4 packed [N][K/2] (q, k, v, o, gate, up,
 * down) or int8 [N][K] (ple_gate [ple_dim][hidden], ple_proj [hidden][ple_dim]), one f32 scale per
 * output row. k, v, k_norm are read only on producer layers. */
typedef struct g4_decode_layer {
    const void *q, *k, *v, *o, *gate, *up, *down, *ple_gate, *ple_proj;
    const float *q_s, *k_s, *v_s, *o_s, *gate_s, *up_s, *down_s, *ple_gate_s, *ple_proj_s;
    const float *input_norm;     /* [hidden] input_layernorm */
    const float *post_attn_norm; /* [hidden] post_attention_layernorm */
    const float *pre_ffn_norm;   /* [hidden] pre_feedforward_layernorm */
    const float *post_ffn_norm;  /* [hidden] post_feedforward_layernorm */
    const float *post_ple_norm;  /* [hidden] post_per_layer_input_norm */
    const float *q_norm;         /* [head_dim] */
    const float *k_norm;         /* [head_dim] */
    float layer_scalar;
} g4_decode_layer;

typedef struct g4_decode_weights {
    const void *embed;            /* tied int4 [vocab][hidden/2]: the embedding and the head */
    const float *embed_s;         /* [vocab] */
    const void *ple_table;        /* int4 [vocab][layers * ple_dim / 2] */
    const float *ple_table_s;     /* f32 [vocab][layers], one per 256-wide layer group */
    const void *ple_model_proj;   /* int4 [layers * ple_dim][hidden/2] */
    const float *ple_model_proj_s;
    const float *ple_proj_norm;   /* [ple_dim] per_layer_projection_norm */
    const float *final_norm;      /* [hidden] */
    const float *rope_local_cos, *rope_local_sin;   /* [kv_capacity][head_dim/2] */
    const float *rope_global_cos, *rope_global_sin; /* [kv_capacity][head_dim/2] */
    const g4_decode_layer *layer; /* host array of `layers` entries (copied by create) */
    /* Optional split storage of ple_table (buffers.ts sliceName(PLE_CODES, i); plan.ts:709-725 one
     * gather step per slice, run here as one fused launch): with ple_num_slices >= 1, slice i is a
     * device buffer of vocabulary rows [ple_slice_start[i], ple_slice_start[i] + ple_slice_rows[i])
     * and ple_table may be NULL. The slices must partition [0, vocab) in order (at most 16). The
     * scales stay whole (ple_table_s), addressed by the absolute row. Host arrays, copied by
     * create. ple_num_slices 0: the single ple_table. */
    int ple_num_slices;
    const void *const *ple_slice_codes;
    const int64_t *ple_slice_start;
    const int64_t *ple_slice_rows;
} g4_decode_weights;

typedef struct g4_decode g4_decode;

/* Validates the shape and weights, allocates the KV caches ([batch][2][kv_capacity][head_dim] f32
 * per producer, K then V) and every work buffer, and builds the per-layer GEMV plans. At batch 1
 * it also keeps a copy of every layer's down_proj in the FFN block's layout (hidden * ffn / 2
 * bytes per layer), taken after the device has finished the work queued before the call: the
 * weights are read at creation and must not change while the runner lives. */
int g4_decode_create(const g4_decode_shape *shape, const g4_decode_weights *weights,
                     g4_decode **out);
int g4_decode_destroy(g4_decode *d);

/* The K and V cache base of producer layer `layer` (row r at base + r * *row_stride floats). */
int g4_decode_kv(g4_decode *d, int layer, float **k, float **v, int64_t *row_stride);

/* The device int32 the step reads its position from (set it with a copy before each step). */
int g4_decode_position(g4_decode *d, int32_t **pos);

/* Sets that word in stream order (a one-thread kernel: no host copy, graph-capturable), so the
 * steps of several tokens can be enqueued back to back, each reading the tokens the previous one
 * wrote, with the host waiting only on what it reads back (the reference's lookahead keeps steps
 * in flight the same way, plan.ts:942-973). */
int g4_decode_set_position(g4_decode *d, int pos, void *stream);

/*
 * One decode step for every row: token ids [batch] (device int32) at the position held by the
 * device word, through embedding, the per-layer inputs, 35 layers (each writing its KV at that
 * position when a producer) and the head, to next_tokens [batch] (device int32). Launch only:
 * capture it in a graph and replay it with a new position word each token.
 */
int g4_decode_step(g4_decode *d, const int32_t *tokens, int32_t *next_tokens, void *stream);

/* A named work buffer of the last step (device pointer and bytes), for tests and tooling:
 * "hidden" f32 [batch][hidden] (after the last layer's join), "logits" f32 [batch][vocab] (capped),
 * "per_layer" f32 [batch][layers][ple_dim], "head_codes" int8 [batch][hidden] (the final-norm
 * snap the head reads), "codes" int8 [batch][hidden] (the next projection input snap). */
int g4_decode_buffer(g4_decode *d, const char *name, void **ptr, size_t *bytes);

/* Stop the step after layer `last_layer` (-1: run everything, the default): the join of that layer
 * then writes "hidden" with the next layer's input snap, and no head runs. For layer-by-layer
 * parity tests only. */
int g4_decode_set_stop(g4_decode *d, int last_layer);

#ifdef __cplusplus
}
#endif

#endif /* G4DECODE_H */

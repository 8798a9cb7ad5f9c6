// Shared internals of libg4w8a8: status plumbing (host) and the SRQ / epilogue arithmetic (device).
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>

#include <cstdarg>
#include <cstdint>
#include <string>

#include "../../include/g4w8a8.h"

namespace g4 {

// Native 128-bit vectors for register arrays: HIP's uint4 is a union-wrapped struct that the
// optimizer keeps in memory when it sits in an array (then promoted to LDS or scratch).
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef int v4i __attribute__((ext_vector_type(4)));

// ---- host: status and last error ----------------------------------------------------------------

int set_error(int status, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();
int hip_status(hipError_t err, const char *what);

#define G4_HIP(call)                                              \
    do {                                                          \
        hipError_t g4_err_ = (call);                              \
        if (g4_err_ != hipSuccess) return ::g4::hip_status(g4_err_, #call); \
    } while (0)

// The launch error of the last kernel, checked right after every launch.
#define G4_LAUNCHED(what)                                         \
    do {                                                          \
        hipError_t g4_err_ = hipGetLastError();                   \
        if (g4_err_ != hipSuccess) return ::g4::hip_status(g4_err_, what); \
    } while (0)

inline hipStream_t as_stream(void *s) { return reinterpret_cast<hipStream_t>(s); }

// Number of compute units of the current device (cached per device).
int device_cu_count();

// The gelu activation prologue of one GEMV job (qgemv.ts:359-400): the job's x is the gate, and
// the GEMV reads gelu_tanh(gate[i]) * up[i] in place of x[i]. `up` already carries the offset;
// null means no prologue. gate codes (x_kind int8) are times g_scale, up codes times u_scale.
// With fold_parts set (ple-fold-projection, pleSplit.ts:24-41) the gate is not read from x: gate
// element i is the fold of the split partials fold_parts[(i / 4) * 4 * fold_splits + s * 4 + i % 4]
// (ascending s from 0), times f32(fold_in * fold_scales[i]), snapped on fold_out when non-zero.
struct GeluAct {
    const void *up = nullptr;
    float g_scale = 0.0f;
    float u_scale = 0.0f;
    int up_kind = G4_KIND_F32;
    const float *fold_parts = nullptr;
    const float *fold_scales = nullptr;
    int fold_splits = 0;
    float fold_in = 0.0f;
    float fold_out = 0.0f;
};

// The gelu-mul pass folded into the gate's GEMV epilogue (the decode runner's form, no reference
// counterpart): the job's rows are the gate, its output codes go back on out_scale, and dst
// receives srq(gelu(gate) * up, act_scale) with up the same row of a paired 4-bit up projection
// (w_up, s_up) or up_vec[row] (f32). act_scale 0: no epilogue.
struct GeluEpilogue {
    const void *w_up = nullptr;
    const float *s_up = nullptr;
    const float *up_vec = nullptr;
    float act_scale = 0.0f;
};

// A GEMV plan whose projections may carry a gelu epilogue (qgemv_stream.hip).
int gemv_plan_create_epilogue(const g4_gemv_desc *descs, const GeluEpilogue *epis, int count,
                              g4_gemv_plan **out);

// One row's RMS join, the arguments of g4_rms_join for rows = 1 (g4_rowops.h rms_join_row).
struct JoinTail {
    const void *src = nullptr;
    int src_kind = G4_KIND_F32;
    float src_scale = 1.0f;
    const float *gain = nullptr;
    const float *resid = nullptr;
    float alpha = 1.0f;
    const float *gain2 = nullptr;
    int width = 0;
    float eps = 0.0f;
    float in_scale = 0.0f;
    float *hidden = nullptr;
    int8_t *codes = nullptr;
    // src_kind G4_KIND_I32 (join_acc): src holds acc_splits int32 partial accumulators of the
    // producing linear, split s at src + s * acc_split_stride, each laid out [row][width]; their
    // sum is the linear's exact accumulator, and element i is the linear's int8 output code
    // snap(f32(acc_in_scale * acc_scales[i]) * f32(sum)) on src_scale, times src_scale
    const float *acc_scales = nullptr;
    float acc_in_scale = 0.0f;
    int acc_splits = 0;
    int64_t acc_split_stride = 0;
};

constexpr int kSplitAccMax = 4;

// The small-M MFMA kernel over K split in `splits` equal ranges (k a multiple of splits * 128,
// 3 <= m <= 32, int8 codes in): part[s][m][n] = the int32 accumulator of range s (zero point
// included), for a consumer that sums them (join_acc).
int linear_split_acc(int bits, const uint8_t *wq, const float *scales, const int8_t *x, int k,
                     int n, int m, int splits, int32_t *part, hipStream_t stream);

// The RMS join of `rows` rows over a JoinTail whose src holds split accumulators (src_kind int32).
int join_acc(const JoinTail &J, int rows, hipStream_t stream);

// Makes the RMS join `j` the prologue of a plan (the decode runner's launch fold, no reference
// counterpart): every projection of the plan reads j.codes (at one bit width), and takes them
// from the join, which every block computes in place of its snap; block 0 also stores j.hidden and
// j.codes. j.hidden must not alias j.resid (blocks still read the residual while block 0 writes).
int gemv_plan_set_prologue_join(g4_gemv_plan *p, const JoinTail &j);

// One output of a grouped linear: weights, row scales, destination and row count.
struct LinearOut {
    const void *wq;
    const float *scales;
    void *dst;
    int n;
};

// Several linears over the same activations x (m rows of k) and scales (qgemm.hip): one launch of
// the small-M kernel when every output takes it (m 3..32) and there are at most 4, else one
// library call each. Validated as g4_linear validates each.
int linear_grouped(int bits, const void *x, int x_kind, int k, int m, float in_scale,
                   float out_scale, int out_kind, const LinearOut *outs, int count, void *stream);

// The gate linear of m int8-coded rows with the gelu-mul pass in its epilogue (qgemm.hip): act =
// srq(gelu(gate code * out_scale) * u, act_scale), u the same row of a paired 4-bit up projection
// (w_up, s_up; its code times out_scale) or up_vec[row * up_stride + i] (f32). Runs when the shape
// takes the small-M kernel (m 3..32); otherwise enqueues nothing and sets *launched = false.
int linear_gelu(int bits, const void *x, int k, int m, float in_scale, float out_scale,
                const void *w_gate, const float *s_gate, const void *w_up, const float *s_up,
                const float *up_vec, int64_t up_stride, int n, float act_scale, int8_t *act,
                void *stream, bool *launched);

// The attention prologue (q-norm + RoPE; on a producer layer k-norm + RoPE, the weightless
// v-norm and the KV store at the position) run inside the split attention kernel, the decode
// runner's form of g4_attn_prologue + g4_attention_decode with no q buffer between them
// (decode.hip). Every block rebuilds the query heads; the block whose chunk holds the position
// builds and stores the new K and V rows.
struct AttnPrologue {
    const int8_t *q_codes;
    float q_scale;
    const int8_t *k_codes;  // null on a consumer layer (no KV store)
    float k_scale;
    const int8_t *v_codes;
    float v_scale;
    const float *q_gain;
    const float *k_gain;
    const float *cos_tab;  // [positions][128]
    const float *sin_tab;
    float eps;
    int32_t *zero = nullptr;  // zero_n int32 the split kernel clears (the folded o_proj's accumulator)
    int zero_n = 0;
};

// o_proj folded into the attention merge (one decode row): w is its 4-bit [n][k] weights with
// k = heads * 256; part (n int32, zero when the merge starts: AttnPrologue::zero) receives o_proj's
// exact accumulator, each head's K range added atomically (a JoinTail with src_kind
// G4_KIND_I32 and one split reads it).
struct MergeLinear {
    const void *w = nullptr;
    int n = 0;
    int k = 0;
    int32_t *part = nullptr;
};

// The decode runner's per-layer-input block at one row (decode.hip ple_block_kernel): the join
// (codes for the gate), the 8-bit gate [p][H] with its gelu x per-layer-row epilogue, and the 8-bit
// projection [H][p] contracted into acc (H int32, zero on entry: its exact accumulator).
struct PleFold {
    JoinTail join;
    const int8_t *w_gate = nullptr;
    const float *s_gate = nullptr;
    const float *up_vec = nullptr;  // the layer's per-layer row (p f32)
    const int8_t *w_proj = nullptr;
    int p = 0;                      // the gate's rows, the projection's K
    float in_scale = 0.0f;          // every input snap (the gate's x, the projection's codes)
    float out_scale = 0.0f;         // the gate's output snap
    int32_t *acc = nullptr;
};
bool ple_fold_fits(const PleFold &F);
int ple_block(const PleFold &F, void *stream);

// The decode runner's FFN block at one row (decode.hip ffn_block_kernel): the join (codes for gate
// and up), the 4-bit gate and up [f][H] with the gelu-mul epilogue, and the 4-bit down contracted
// into acc (H int32, zero on entry: its exact accumulator). Block b takes gate / up rows
// b * kFfnRows .. + kFfnRows, so it reads down's K range of that width in every row; w_down holds
// down [H][f] repacked by ffn_repack_down so that this range is one contiguous run per block:
// [f / kFfnRows][H][kFfnRows / 2] bytes.
constexpr int kFfnRows = 32;
struct FfnFold {
    JoinTail join;
    const uint8_t *w_gate = nullptr;
    const uint8_t *w_up = nullptr;
    const float *s_gate = nullptr;
    const float *s_up = nullptr;
    const uint8_t *w_down = nullptr;  // repacked
    int f = 0;                // gate / up rows, down's K
    float in_scale = 0.0f;    // gate / up input snap
    float out_scale = 0.0f;   // gate / up output snap
    float act_scale = 0.0f;   // the gelu-mul codes' snap (down's input)
    // acc_copies accumulators [H] at acc + c * H (block b adds into copy b % acc_copies): the
    // atomics of one address serialize, so spreading the blocks over copies takes their cost off
    // the kernel's tail; the reader sums the copies (a JoinTail with acc_splits = acc_copies)
    int32_t *acc = nullptr;
    int acc_copies = 1;
};
constexpr int kFfnAccCopies = 4;
static_assert(kFfnAccCopies <= kSplitAccMax, "the join sums at most kSplitAccMax copies");
bool ffn_fold_fits(const FfnFold &F);
int ffn_block(const FfnFold &F, void *stream);
// down [h][f] (4-bit, row-major) -> out [f / kFfnRows][h][kFfnRows / 2]; f % kFfnRows == 0.
int ffn_repack_down(const uint8_t *w, uint8_t *out, int h, int f, hipStream_t stream);

// Whether the merge can fold `lin` in (rows 1, n a multiple of the merge's row block, k = heads * 256).
bool merge_linear_fits(const MergeLinear &lin, int rows, int heads);

// g4_attention_decode with the prologue fused (head_dim 256, int8 codes out on in_scale). With
// `lin`, the merge also runs o_proj's per-head partial accumulators (codes stay the merge's).
int attention_decode_fused(const AttnPrologue &pro, float *k_cache, float *v_cache,
                           int64_t cache_row_stride, int rows, int heads, int pos,
                           const int32_t *pos_dev, int window, float *workspace,
                           size_t workspace_bytes, float in_scale, int8_t *codes, void *stream,
                           const MergeLinear *lin = nullptr);

// Makes a plan snap each block's first activation vector inside its first tile, after that tile's
// weight loads are out (the decode runner's small plans: the snap's latency overlaps the weights').
int gemv_plan_set_first_tile_snap(g4_gemv_plan *p);

// The internal form of a public g4_gelu_act (NULL or a NULL up: no prologue).
GeluAct gelu_act_of(const g4_gelu_act *a);

// Validates one GEMV descriptor (and its prologue, when act.up is set) against what the GEMV
// kernels assume (qgemv.hip).
int check_job_desc(const g4_gemv_desc &d, const GeluAct &act, const char *who);

// Launches calibrated M = 1 GEMVs on the streaming kernel when every one has a compiled shape
// class (qgemv_stream.hip); otherwise enqueues nothing and sets *launched = false. acts: one per
// descriptor, or null for none.
int stream_try_launch(const g4_gemv_desc *descs, const GeluAct *acts, int count, hipStream_t stream,
                      bool *launched);

// The streaming shape class of a row of K codes at `bits`, or -1 (qgemv_stream.hip).
int stream_class_for(int bits, int k);

// Releases the GEMM workspace of a stream about to be destroyed (qgemm.hip, g4_workspace.h).
int workspace_forget_stream(void *stream);

// g4_qgemm with the caller's buffer for the snapped activation codes in place of the stream's
// workspace (codes_bytes bytes; refused when the call's path needs more). Allocates nothing. The
// call is validated and routed first; `source` gives the buffer's address and is called only when
// the routed path needs one.
typedef int (*CodesSource)(int8_t **codes);
int qgemm_given_codes(int bits, const void *wq, const float *scales, const void *x, int x_kind,
                      void *dst, int out_kind, int k, int num_rows, int m_cols, float in_scale,
                      float out_scale, void *stream, CodesSource source, size_t codes_bytes,
                      const char *who);

// ---- device: the static range quantization arithmetic (src/quant.ts:248-357) -----------------

// srqCodes at 8 bits: clamp(RNE(f32(v / s)), -128, 127). __fdiv_rn is the IEEE binary32 divide;
// rintf is round-half-to-even (v_rndne_f32). fmaxf drops a NaN, so NaN lands on -128 exactly as
// WGSL's clamp = min(max(e, lo), hi) does on the reference (qgemv.ts:620-626).
__device__ __forceinline__ float srq_code_f(float v, float s) {
    float r = rintf(__fdiv_rn(v, s));
    return fminf(fmaxf(r, -128.0f), 127.0f);
}

__device__ __forceinline__ int srq_code_i(float v, float s) { return (int)srq_code_f(v, s); }

// The same code without a divide on the common path. With r = fl(1/s), t = fl(v * r) is within
// |v/s| * 1.5 * 2^-23 of the correctly rounded quotient fl(v / s), so both round to the same
// integer unless t lies within that distance of a half integer; there (about 1e-5 of the inputs)
// the IEEE divide decides. Beyond |v/s| = 256 both clamp. `r_ok` is false when 1/s overflows, and
// then every element takes the divide.
__device__ __forceinline__ float srq_code_fast(float v, float s, float r, bool r_ok) {
    const float t = __fmul_rn(v, r);
    float n = rintf(t);
    const float d = fabsf(t - n);
    const float thr = fmaxf(fabsf(t), 1.0f) * 0x1p-20f;
    if (!r_ok || d >= 0.5f - thr) n = rintf(__fdiv_rn(v, s));
    return fminf(fmaxf(n, -128.0f), 127.0f);
}

// fl(1/s) and whether it is finite (a subnormal or zero scale leaves only the divide).
__device__ __forceinline__ float srq_recip(float s, bool &ok) {
    const float r = __fdiv_rn(1.0f, s);
    ok = isfinite(r) && r != 0.0f;
    return r;
}

// ---- device: deterministic exp, tanh and gelu (geluMul.ts:101-116) --------------------------------
// Every step is one IEEE f32 rounding (no FMA), so a CPU restatement (oracle/g4_decode_oracle.c)
// reproduces them bit for bit. exp: Cody-Waite reduction by ln 2 (15-bit high part), a degree-6
// Taylor polynomial on |r| <= ln2 / 2, ldexp; within 3 ulp of exp. tanh: x below 2^-12, the exact
// form -em / (2 + em) with em = expm1(-2|x|) below 0.171875, else (1 - t) / (1 + t) with
// t = exp(-2|x|); within 8 ulp of tanh. gelu: the tanh form in the shader's operation order.

__device__ __forceinline__ float d_expf(float x) {
    if (x != x) return x;
    if (x > 88.7f) return __int_as_float(0x7f800000);
    if (x < -87.0f) return 0.0f;
    const float n = rintf(__fmul_rn(x, 0x1.715476p+0f));             // round(x * log2 e)
    float r = __fsub_rn(x, __fmul_rn(n, 0x1.62e4p-1f));              // x - n * ln2_hi (15-bit)
    r = __fsub_rn(r, __fmul_rn(n, 0x1.7f7d1cp-20f));                 // - n * ln2_lo
    float p = 0x1.6c16c2p-10f;                                       // 1/720
    p = __fadd_rn(__fmul_rn(p, r), 0x1.111112p-7f);                  // 1/120
    p = __fadd_rn(__fmul_rn(p, r), 0x1.555556p-5f);                  // 1/24
    p = __fadd_rn(__fmul_rn(p, r), 0x1.555556p-3f);                  // 1/6
    p = __fadd_rn(__fmul_rn(p, r), 0.5f);
    p = __fadd_rn(__fmul_rn(p, r), 1.0f);
    p = __fadd_rn(__fmul_rn(p, r), 1.0f);
    return ldexpf(p, (int)n);
}

// exp(y) - 1 for |y| <= 0.35: d_expf's Taylor chain stopped before its final + 1, times y.
__device__ __forceinline__ float d_expm1_small(float y) {
    float p = 0x1.6c16c2p-10f;
    p = __fadd_rn(__fmul_rn(p, y), 0x1.111112p-7f);
    p = __fadd_rn(__fmul_rn(p, y), 0x1.555556p-5f);
    p = __fadd_rn(__fmul_rn(p, y), 0x1.555556p-3f);
    p = __fadd_rn(__fmul_rn(p, y), 0.5f);
    p = __fadd_rn(__fmul_rn(p, y), 1.0f);
    return __fmul_rn(p, y);
}

// Below 0.171875 the form -em / (2 + em), em = expm1(-2|x|), avoids the cancellation of 1 - t.
__device__ __forceinline__ float d_tanhf(float x) {
    const float ax = fabsf(x);
    if (ax < 0x1p-12f) return x;
    float r;
    if (ax < 0.171875f) {
        const float em = d_expm1_small(-2.0f * ax);
        r = __fdiv_rn(-em, __fadd_rn(2.0f, em));
    } else {
        const float t = d_expf(-2.0f * ax);
        r = __fdiv_rn(__fsub_rn(1.0f, t), __fadd_rn(1.0f, t));
    }
    return copysignf(r, x);
}

// geluMul.ts:101-116 in the shader's order.
__device__ __forceinline__ float d_gelu(float x) {
    const float cube = __fmul_rn(__fmul_rn(x, x), x);
    float inner = __fmul_rn(0x1.988454p-1f, __fadd_rn(x, __fmul_rn(0x1.6e4e26p-5f, cube)));
    inner = fminf(fmaxf(inner, -10.0f), 10.0f);
    return __fmul_rn(__fmul_rn(0.5f, x), __fadd_rn(1.0f, d_tanhf(inner)));
}


// Eight activation values e .. e + 7 of an f32 vector, or of int8 codes times `scale`.
__device__ __forceinline__ void act_vals8(const void *p, int kind, float scale, int64_t e,
                                          float v[8]) {
    if (kind == G4_KIND_I8) {
        const uint2 w = *reinterpret_cast<const uint2 *>(reinterpret_cast<const int8_t *>(p) + e);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            v[i] = __fmul_rn((float)(int8_t)((w.x >> (8 * i)) & 0xff), scale);
            v[4 + i] = __fmul_rn((float)(int8_t)((w.y >> (8 * i)) & 0xff), scale);
        }
    } else {
        const float4 *q = reinterpret_cast<const float4 *>(reinterpret_cast<const float *>(p) + e);
        const float4 a = q[0], b = q[1];
        v[0] = a.x, v[1] = a.y, v[2] = a.z, v[3] = a.w;
        v[4] = b.x, v[5] = b.y, v[6] = b.z, v[7] = b.w;
    }
}

// The gelu prologue's codes for activations e .. e + 7: srq(gelu_tanh(gate) * up) on s, the
// gelu-mul kernel's expression and snap (geluMul.ts:101-116), so the fused GEMV reads exactly the
// codes the separate pass would have written.
__device__ __forceinline__ void gelu_codes8(const void *gate, int g_kind, float gs, const void *up,
                                            int u_kind, float us, int64_t e, float s, float r,
                                            bool r_ok, int c[8]) {
    float g[8], u[8];
    act_vals8(gate, g_kind, gs, e, g);
    act_vals8(up, u_kind, us, e, u);
#pragma unroll
    for (int i = 0; i < 8; ++i) c[i] = (int)srq_code_fast(__fmul_rn(d_gelu(g[i]), u[i]), s, r, r_ok);
}

// foldGate (pleSplit.ts:33-41) for the four gate elements of vec4 index i: the split partials
// summed in split order from 0, the gate linear's epilogue f32(f32(in * scale) * total), then its
// output snap (srqOut with the IEEE divide) when out != 0.
__device__ __forceinline__ float4 fold_gate4(const GeluAct &a, int64_t i) {
    const float4 *parts = reinterpret_cast<const float4 *>(a.fold_parts) + i * a.fold_splits;
    float4 t = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    for (int s = 0; s < a.fold_splits; ++s) {
        const float4 p = parts[s];
        t.x = __fadd_rn(t.x, p.x);
        t.y = __fadd_rn(t.y, p.y);
        t.z = __fadd_rn(t.z, p.z);
        t.w = __fadd_rn(t.w, p.w);
    }
    const float4 sc = reinterpret_cast<const float4 *>(a.fold_scales)[i];
    float v[4] = {__fmul_rn(__fmul_rn(a.fold_in, sc.x), t.x), __fmul_rn(__fmul_rn(a.fold_in, sc.y), t.y),
                  __fmul_rn(__fmul_rn(a.fold_in, sc.z), t.z), __fmul_rn(__fmul_rn(a.fold_in, sc.w), t.w)};
    if (a.fold_out != 0.0f) {
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = __fmul_rn(srq_code_f(v[j], a.fold_out), a.fold_out);
    }
    return make_float4(v[0], v[1], v[2], v[3]);
}

// The ple-fold-projection prologue's codes for activations e .. e + 7 (e a multiple of 8):
// srq(gelu_tanh(foldGate) * up) on s.
__device__ __forceinline__ void fold_gelu_codes8(const GeluAct &a, int64_t e, float s, float r,
                                                 bool r_ok, int c[8]) {
    const float4 g0 = fold_gate4(a, e >> 2), g1 = fold_gate4(a, (e >> 2) + 1);
    const float g[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
    float u[8];
    act_vals8(a.up, a.up_kind, a.u_scale, e, u);
#pragma unroll
    for (int i = 0; i < 8; ++i) c[i] = (int)srq_code_fast(__fmul_rn(d_gelu(g[i]), u[i]), s, r, r_ok);
}

// One prologue activation as f32 (the uncalibrated path reads it unsnapped, qgemv.ts:359-400):
// gelu_tanh(gate[i]) * up[i], the gate from x (f32 or codes times g_scale) or from the fold.
__device__ __forceinline__ float gelu_act_value(const GeluAct &a, const void *gate, int g_kind,
                                                int64_t i) {
    float g;
    if (a.fold_parts) {
        const float4 g4v = fold_gate4(a, i >> 2);
        const int j = (int)(i & 3);
        g = j == 0 ? g4v.x : j == 1 ? g4v.y : j == 2 ? g4v.z : g4v.w;
    } else {
        g = g_kind == G4_KIND_I8 ? __fmul_rn((float)reinterpret_cast<const int8_t *>(gate)[i], a.g_scale)
                                 : reinterpret_cast<const float *>(gate)[i];
    }
    const float u = a.up_kind == G4_KIND_I8
                        ? __fmul_rn((float)reinterpret_cast<const int8_t *>(a.up)[i], a.u_scale)
                        : reinterpret_cast<const float *>(a.up)[i];
    return __fmul_rn(d_gelu(g), u);
}

// The closing expression of every quantized linear (qgemv.ts:1168-1172, :680-686), in its order:
// one f32 multiply folds the input scale into the row scale, one more multiplies the reduced sum.
__device__ __forceinline__ float linear_epilogue(float in_scale, float row_scale, float sum) {
    return __fmul_rn(__fmul_rn(in_scale, row_scale), sum);
}

// Stores one output element of a linear in the requested kind. `y` is the pre-snap f32 value and
// `acc` the exact integer sum (calibrated path only; 0 on the f32 path).
__device__ __forceinline__ void store_linear_out(void *dst, int64_t idx, int out_kind, float y,
                                                 int acc, float out_scale) {
    if (out_kind == G4_KIND_I8) {
        reinterpret_cast<int8_t *>(dst)[idx] = (int8_t)srq_code_i(y, out_scale);
    } else if (out_kind == G4_KIND_I32) {
        reinterpret_cast<int32_t *>(dst)[idx] = acc;
    } else {
        float v = y;
        if (out_scale != 0.0f) v = __fmul_rn(srq_code_f(y, out_scale), out_scale);
        reinterpret_cast<float *>(dst)[idx] = v;
    }
}

// Reads activation element i of kind f32 / f16 as f32 (f16 widening is exact).
__device__ __forceinline__ float load_act(const void *x, int kind, int64_t i) {
    if (kind == G4_KIND_F16) return __half2float(reinterpret_cast<const __half *>(x)[i]);
    return reinterpret_cast<const float *>(x)[i];
}

// ---- device: block barrier for LDS-only communication ------------------------------------------

// A workgroup barrier for kernels whose waves communicate only through LDS. __syncthreads() is a
// release/acquire fence plus s_barrier, and the fence drains every outstanding global load of the
// wave (vmcnt), which would empty a prefetch pipeline at each stage. Here only this wave's LDS
// traffic is waited for (lgkmcnt(0)); the "memory" clobber keeps the compiler from moving memory
// operations across the barrier.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// ---- device: cross-lane sums --------------------------------------------------------------------

// Sum over each aligned group of 16 lanes (one DPP row), result in every lane of the group.
// quad_perm(1,0,3,2), quad_perm(2,3,0,1), row_half_mirror, row_mirror.
__device__ __forceinline__ int row16_sum_i32(int v) {
    v += __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false);
    v += __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false);
    v += __builtin_amdgcn_update_dpp(0, v, 0x141, 0xF, 0xF, false);
    v += __builtin_amdgcn_update_dpp(0, v, 0x140, 0xF, 0xF, false);
    return v;
}

__device__ __forceinline__ float dpp_f32_b1(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0xB1, 0xF, 0xF, false));
}
__device__ __forceinline__ float dpp_f32_4e(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x4E, 0xF, 0xF, false));
}
__device__ __forceinline__ float dpp_f32_half_mirror(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x141, 0xF, 0xF, false));
}
__device__ __forceinline__ float dpp_f32_mirror(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x140, 0xF, 0xF, false));
}

// The same 16-lane tree in f32: ((l0+l1)+(l2+l3)) + ((l4+l5)+(l6+l7)) + ... pairwise, every lane
// ends with the identical value because each step adds a commutative pair.
__device__ __forceinline__ float row16_sum_f32(float v) {
    v = __fadd_rn(v, dpp_f32_b1(v));
    v = __fadd_rn(v, dpp_f32_4e(v));
    v = __fadd_rn(v, dpp_f32_half_mirror(v));
    v = __fadd_rn(v, dpp_f32_mirror(v));
    return v;
}

}  // namespace g4

// The native decode-step runner: one E2B-shape decode step for `batch` sequences as a fixed list of
// launches on one stream (the dispatch walk of plan.ts:780-792 planDecodeStep, executed as
// execute.ts does, without the per-dispatch bind work: every buffer and GEMV plan is built once in
// g4_decode_create). The step reads its position from a device word, so a captured graph of one
// step replays every later token unchanged.
//
// Per layer (plan.ts:487-665, with the synthetic config's uniform FFN and head_dim):
//   [layer 0: input_layernorm, from the embedding phase]
//   q (+ k, v on a producer) GEMV        -> int8 codes on out_scale
//   attention decode over the layer's cache (own, or the last producer of its kind) -> o input
//   snap, with q-norm-rope (+ kv-norm-rope-store) run inside its split kernel
//   o GEMV; norm-residual-norm (post_attention_layernorm, residual, pre_feedforward_layernorm)
//   gate and up GEMV with the gelu-mul pass in their epilogue (batch 1: one paired launch), or the
//   two GEMVs then the gelu-mul pass; down GEMV
//   norm-residual (post_feedforward_layernorm, residual), snapped for per_layer_input_gate
//   per_layer_input_gate (int8 GEMV) with gelu(gate) times the layer's per-layer-input row in its
//   epilogue (or the gelu-mul pass after it); per_layer_projection (int8 GEMV)
//   norm-residual-norm (post_per_layer_input_norm, residual, layer_scalar, then the next layer's
//   input_layernorm, or the final norm on the last layer)
// The residual stream alternates between two rows: a join reads one and writes the other. At
// batch 1 every join but the final norm runs inside the launch that reads its codes (the FFN block,
// the per-layer-input block, the next layer's q/k/v plan), computed by each of its blocks in place
// of an activation snap, so it costs no launch of its own; block 0 writes the new residual row,
// which the other blocks never read. o_proj, down_proj and per_layer_projection add exact int32
// partials into accumulators inside the attention merge, the FFN block and the per-layer-input
// block, and the join after each reads the accumulator through the linear's epilogue and snap.
// Embedding phase (plan.ts:720-729): tied int4 embed gather (x sqrt(hidden) folded), PLE gather,
// per_layer_model_projection (int4 GEMV, then hidden^-0.5), per_layer_projection_norm, + identity,
// x 2^-0.5. Head (plan.ts:768-777): tied int4 GEMV to f32 logits, softcap, two-stage argmax.
#include <cmath>
#include <cstring>
#include <new>
#include <string>
#include <vector>

#include "g4_internal.h"
#include "../../include/g4decode.h"

namespace {

using namespace g4;

// Writes one int32 from a kernel argument: the position word, set in stream order (and inside a
// graph capture) without a host copy.
__global__ void set_word_kernel(int32_t *word, int32_t value) { *word = value; }

struct Plan {
    g4_gemv_plan *p = nullptr;
    bool gelu = false;  // the gelu-mul pass is folded into this plan's epilogue
};

struct DeviceAlloc {
    std::vector<void *> ptrs;
    int get(void **out, size_t bytes) {
        void *p = nullptr;
        if (hipMalloc(&p, bytes < 256 ? 256 : bytes) != hipSuccess)
            return set_error(G4_ERR_HIP, "decode: hipMalloc of %zu bytes failed", bytes);
        ptrs.push_back(p);
        *out = p;
        return G4_OK;
    }
    ~DeviceAlloc() {
        for (void *p : ptrs) (void)hipFree(p);
    }
};

}  // namespace

struct g4_decode {
    g4_decode_shape s{};
    g4_decode_weights w{};
    std::vector<g4_decode_layer> layers;
    std::vector<const void *> ple_split_codes;  // the split PLE table's slices (empty: one table)
    std::vector<int64_t> ple_split_start, ple_split_rows;
    DeviceAlloc mem;
    int32_t *pos = nullptr;
    float *identity = nullptr, *per_layer = nullptr;
    float *hbuf[2] = {nullptr, nullptr};  // the residual stream's two rows (a join reads one, writes the other)
    float *attn_ws = nullptr, *logits = nullptr;
    size_t attn_ws_bytes = 0, argmax_ws_bytes = 0;
    void *argmax_ws = nullptr;
    int8_t *embed_codes = nullptr, *ple_codes = nullptr, *xcodes = nullptr, *qc = nullptr,
           *kc = nullptr, *vc = nullptr, *attn_codes = nullptr, *oc = nullptr, *gc = nullptr,
           *uc = nullptr, *act = nullptr, *dc = nullptr, *pgc = nullptr, *pac = nullptr,
           *ppc = nullptr, *head_codes = nullptr;
    // batch 3..32: down_proj runs as kAccSplits K ranges of int32 accumulators, summed by the
    // post-FFN join (null when down is one launch)
    int32_t *acc = nullptr;
    // batch 1: o_proj runs inside the attention merge, each query head's K range added atomically
    // into this int32 accumulator [hidden] (cleared by the split kernel); the post-attention join
    // applies o_proj's epilogue to it (null when o_proj is a plan)
    int32_t *oacc = nullptr;
    // batch 1: per_layer_input_gate and per_layer_projection in one launch (ple_block), the
    // projection's accumulator in oacc + hidden (cleared with it); the tail join reads it
    bool fold_ple = false;
    bool fold_o = false;  // o_proj inside the attention merge (its accumulator at oacc)
    // batch 1: gate, up, the gelu-mul pass and down_proj in one launch (ffn_block), down's
    // accumulator in oacc + 2 * hidden (cleared with it); the post-FFN join reads it
    bool fold_ffn = false;
    std::vector<uint8_t *> down_packed;  // per layer: down_proj in the FFN block's layout
    std::vector<float *> kv;  // per producer: [batch][2][capacity][head_dim]
    int stop = -1;
    // M = 1 GEMV plans per layer: qkv (or q), o, gate+up, down, ple gate, ple projection.
    std::vector<Plan> plans;
    Plan ple_model_plan, head_plan;
    // the step's RMS joins in order: the layer-0 input norm, then three per layer; each either the
    // prologue of the plan that reads its codes (carried) or a g4_rms_join launch
    std::vector<JoinTail> joins;
    std::vector<char> carried;
    ~g4_decode() {
        for (Plan &p : plans)
            if (p.p) g4_qgemv_plan_destroy(p.p);
        if (ple_model_plan.p) g4_qgemv_plan_destroy(ple_model_plan.p);
        if (head_plan.p) g4_qgemv_plan_destroy(head_plan.p);
    }
};

namespace {

enum { P_QKV = 0, P_O, P_GATEUP, P_DOWN, P_PLE_GATE, P_PLE_PROJ, P_PER_LAYER };

bool is_global(const g4_decode_shape &s, int l) { return l % s.global_period == s.global_period - 1; }

// kv.ts:76-93: producers read their own cache; consumers the last producer of their own kind.
int kv_source(const g4_decode_shape &s, int l) {
    if (l < s.kv_producers) return l;
    int last = -1;
    for (int p = 0; p < s.kv_producers; ++p)
        if (is_global(s, p) == is_global(s, l)) last = p;
    return last;
}

g4_gemv_desc desc(const void *w, const float *sc, const void *x, void *dst, int bits, int k, int n,
                  int out_kind, float in_scale, float out_scale) {
    g4_gemv_desc d{};
    d.wq = w;
    d.scales = sc;
    d.x = x;
    d.dst = dst;
    d.bits = bits;
    d.x_kind = G4_KIND_I8;
    d.out_kind = out_kind;
    d.k = k;
    d.num_rows = n;
    d.in_scale = in_scale;
    d.out_scale = out_scale;
    return d;
}

// One linear of `batch` int8-coded rows: the prebuilt M = 1 plan when there is one (batch 1 and a
// streaming shape class), else the library's routing (GEMV columns, small-M MFMA up to 32 rows).
int run_linear_rows(const g4_decode &d, const Plan &plan, const g4_gemv_desc &one, void *stream) {
    if (d.s.batch == 1 && plan.p) return g4_qgemv_plan_launch(plan.p, stream);
    return g4_linear(one.bits, one.wq, one.scales, one.x, G4_KIND_I8, one.dst, one.out_kind, one.k,
                     one.num_rows, d.s.batch, one.in_scale, one.out_scale, stream);
}

#define G4_TRY(call)             \
    do {                         \
        int rc_ = (call);        \
        if (rc_ != G4_OK) return rc_; \
    } while (0)

int check_shape(const g4_decode_shape &s) {
    if (s.layers <= 0 || s.layers > 64 || s.kv_producers <= 0 || s.kv_producers > s.layers)
        return set_error(G4_ERR_INVALID, "decode: layers %d / kv_producers %d", s.layers,
                         s.kv_producers);
    if (s.head_dim != 256 || s.ple_dim != 256)
        return set_error(G4_ERR_UNSUPPORTED, "decode: head_dim and ple_dim must be 256");
    if (s.hidden <= 0 || s.hidden % 256 || s.hidden > 2048)
        return set_error(G4_ERR_UNSUPPORTED, "decode: hidden %d (a multiple of 256, at most 2048)",
                         s.hidden);
    if (s.ffn <= 0 || s.ffn % 256 || s.ffn > 16384)
        return set_error(G4_ERR_UNSUPPORTED, "decode: ffn %d (a multiple of 256, at most 16384)", s.ffn);
    if (s.q_heads <= 0 || (s.q_heads * s.head_dim) % 256 || s.q_heads * s.head_dim > 16384)
        return set_error(G4_ERR_UNSUPPORTED, "decode: q_heads %d", s.q_heads);
    if (s.global_period <= 0 || s.sliding_window <= 0)
        return set_error(G4_ERR_INVALID, "decode: global_period and sliding_window must be positive");
    if (s.kv_capacity <= 0 || s.kv_capacity > (1 << 20))
        return set_error(G4_ERR_INVALID, "decode: kv_capacity %d", s.kv_capacity);
    if (s.batch <= 0 || s.batch > 64) return set_error(G4_ERR_INVALID, "decode: batch %d (1..64)", s.batch);
    if (s.vocab <= 0 || s.vocab > (int64_t)1 << 30)
        return set_error(G4_ERR_INVALID, "decode: vocab %lld", (long long)s.vocab);
    if (s.in_scale <= 0.0f || s.out_scale <= 0.0f)
        return set_error(G4_ERR_INVALID, "decode: the static scales must be calibrated (non-zero)");
    if (s.fold_off < 0 || s.fold_off > 7) return set_error(G4_ERR_INVALID, "decode: fold_off %d (bits 0..2)", s.fold_off);
    for (int l = 0; l < s.layers; ++l)
        if (kv_source(s, l) < 0)
            return set_error(G4_ERR_INVALID, "decode: layer %d has no producer of its kind", l);
    return G4_OK;
}

int check_weights(const g4_decode_shape &s, const g4_decode_weights &w) {
    if (w.ple_num_slices < 0 || w.ple_num_slices > 16)
        return set_error(G4_ERR_INVALID, "decode: %d PLE slices (0..16)", w.ple_num_slices);
    if (w.ple_num_slices > 0) {
        if (!w.ple_slice_codes || !w.ple_slice_start || !w.ple_slice_rows)
            return set_error(G4_ERR_INVALID, "decode: PLE slices need codes, starts and row counts");
        int64_t expect = 0;
        for (int i = 0; i < w.ple_num_slices; ++i) {
            if (!w.ple_slice_codes[i] || w.ple_slice_start[i] != expect || w.ple_slice_rows[i] <= 0)
                return set_error(G4_ERR_INVALID,
                                 "decode: PLE slice %d must start at row %lld with rows and a buffer",
                                 i, (long long)expect);
            expect += w.ple_slice_rows[i];
        }
        if (expect != s.vocab)
            return set_error(G4_ERR_INVALID, "decode: the PLE slices cover %lld rows, not the vocabulary's %lld",
                             (long long)expect, (long long)s.vocab);
    }
    if (!w.embed || !w.embed_s || (!w.ple_table && w.ple_num_slices == 0) || !w.ple_table_s || !w.ple_model_proj ||
        !w.ple_model_proj_s || !w.ple_proj_norm || !w.final_norm || !w.rope_local_cos ||
        !w.rope_local_sin || !w.rope_global_cos || !w.rope_global_sin || !w.layer)
        return set_error(G4_ERR_INVALID, "decode: a model-level weight is missing");
    for (int l = 0; l < s.layers; ++l) {
        const g4_decode_layer &L = w.layer[l];
        const bool prod = l < s.kv_producers;
        if (!L.q || !L.o || !L.gate || !L.up || !L.down || !L.ple_gate || !L.ple_proj || !L.q_s ||
            !L.o_s || !L.gate_s || !L.up_s || !L.down_s || !L.ple_gate_s || !L.ple_proj_s ||
            !L.input_norm || !L.post_attn_norm || !L.pre_ffn_norm || !L.post_ffn_norm ||
            !L.post_ple_norm || !L.q_norm)
            return set_error(G4_ERR_INVALID, "decode: layer %d misses a weight", l);
        if (prod && (!L.k || !L.v || !L.k_s || !L.v_s || !L.k_norm))
            return set_error(G4_ERR_INVALID, "decode: producer layer %d misses k, v or k_norm", l);
    }
    return G4_OK;
}

// A grouped M = 1 plan, or none when a shape has no streaming class (the runner then launches
// each projection through g4_linear).
int try_plan(const g4_gemv_desc *descs, int count, Plan &out) {
    const int rc = g4_qgemv_plan_create(descs, count, &out.p);
    if (rc == G4_ERR_UNSUPPORTED) {
        out.p = nullptr;
        clear_error();
        return G4_OK;
    }
    return rc;
}

// A plan with the gelu-mul pass in the gate's epilogue; none when a shape has no streaming class
// (the runner then launches the unfused chain).
int try_gelu_plan(const g4_gemv_desc &gate, const GeluEpilogue &epi, Plan &out) {
    const int rc = gemv_plan_create_epilogue(&gate, &epi, 1, &out.p);
    if (rc == G4_ERR_UNSUPPORTED) {
        out.p = nullptr;
        clear_error();
        return G4_OK;
    }
    out.gelu = rc == G4_OK;
    return rc;
}

// The joins of a step: index 0 the layer-0 input norm (no residual), then for layer l the three at
// 1 + 3 l + {0, 1, 2}: post-attention (+ pre-feedforward norm), post-feedforward, and the
// per-layer-input tail (+ layer scalar, the next input norm or the final norm). Join k > 0 reads
// the residual row hbuf[(k - 1) & 1] and writes hbuf[k & 1].
int join_index(int layer, int which) { return 1 + 3 * layer + which; }

float *join_resid(g4_decode &d, int k) { return d.hbuf[(k - 1) & 1]; }
float *join_out(g4_decode &d, int k) { return d.hbuf[k & 1]; }

JoinTail make_join(g4_decode &d, int k, const void *src, int src_kind, float src_scale,
                   const float *gain, float alpha, const float *gain2, int8_t *codes) {
    const g4_decode_shape &s = d.s;
    JoinTail j;
    j.src = src;
    j.src_kind = src_kind;
    j.src_scale = src_scale;
    j.gain = gain;
    j.resid = k > 0 ? join_resid(d, k) : nullptr;
    j.alpha = alpha;
    j.gain2 = gain2;
    j.width = s.hidden;
    j.eps = s.eps;
    j.in_scale = s.in_scale;
    j.hidden = k > 0 ? join_out(d, k) : nullptr;
    j.codes = codes;
    return j;
}

// down_proj over two K ranges, each range's blocks a grid of their own: at batch 32 the E2B
// shape's 96 column blocks each walked K = 6144 as two LDS chunks one after the other (18 us);
// split, 192 blocks take one chunk each and the join adds the two exact int32 partials (step
// 4.25 -> 4.08 ms). o_proj (K = 2048, one chunk) split the same way measured no faster at batch
// 32 and slower at batch 3. Four K ranges (384 blocks, so 4 waves each in place of 16, and half
// the codes copied per block) measured slower: 2.95 against 2.87 ms per batch-32 step.
// The batch-1 folds' int32 accumulators, [kAccRows][hidden]: o_proj, per_layer_projection, then
// down_proj's kFfnAccCopies copies.
constexpr int kAccRows = 2 + kFfnAccCopies;

constexpr int kAccSplits = 2;
static_assert(kAccSplits <= kSplitAccMax, "the join sums at most kSplitAccMax partials");

bool acc_split(const g4_decode_shape &s) {
    return s.batch >= 3 && s.batch <= 32 && s.ffn % (kAccSplits * 128) == 0 &&
           kAccSplits * ((s.hidden + 15) / 16) <= device_cu_count();
}

// Join j reads the split accumulators of the linear (scales, in_scale) in place of its codes.
void join_from_acc(const g4_decode &d, JoinTail &j, const float *scales) {
    j.src = d.acc;
    j.src_kind = G4_KIND_I32;
    j.acc_scales = scales;
    j.acc_in_scale = d.s.in_scale;
    j.acc_splits = kAccSplits;
    j.acc_split_stride = (int64_t)d.s.batch * d.s.hidden;
}

void build_joins(g4_decode &d) {
    const g4_decode_shape &s = d.s;
    const float out = s.out_scale;
    d.joins.clear();
    d.joins.push_back(make_join(d, 0, d.hbuf[0], G4_KIND_F32, 1.0f, d.layers[0].input_norm, 1.0f,
                                nullptr, d.xcodes));
    for (int l = 0; l < s.layers; ++l) {
        const g4_decode_layer &L = d.layers[l];
        const bool last = l + 1 == s.layers;
        d.joins.push_back(make_join(d, join_index(l, 0), d.oc, G4_KIND_I8, out, L.post_attn_norm,
                                    1.0f, L.pre_ffn_norm, d.xcodes));
        d.joins.push_back(make_join(d, join_index(l, 1), d.dc, G4_KIND_I8, out, L.post_ffn_norm,
                                    1.0f, nullptr, d.xcodes));
        if (d.acc) join_from_acc(d, d.joins.back(), L.down_s);
        d.joins.push_back(make_join(d, join_index(l, 2), d.ppc, G4_KIND_I8, out, L.post_ple_norm,
                                    L.layer_scalar, last ? d.w.final_norm : d.layers[l + 1].input_norm,
                                    last ? d.head_codes : d.xcodes));
    }
    d.carried.assign(d.joins.size(), 0);
}

// Makes join k the prologue of `plan` when the plan exists.
int carry_join(g4_decode &d, int k, const Plan &plan) {
    if (!plan.p) return G4_OK;
    G4_TRY(gemv_plan_set_prologue_join(plan.p, d.joins[k]));
    d.carried[k] = 1;
    return G4_OK;
}

// Join k for the step's `batch` rows as a launch of its own (int32 accumulator sources included).
int launch_join(g4_decode &d, int k, void *st) {
    const JoinTail &j = d.joins[k];
    if (j.src_kind == G4_KIND_I32) return join_acc(j, d.s.batch, as_stream(st));
    return g4_rms_join(j.src, j.src_kind, j.src_scale, j.gain, j.resid, j.alpha, j.gain2, d.s.batch,
                       j.width, j.eps, j.in_scale, j.hidden, j.codes, st);
}

// Join k for the step's `batch` rows, unless a plan carries it.
int run_join(g4_decode &d, int k, void *st) { return d.carried[k] ? G4_OK : launch_join(d, k, st); }

// The per-layer-input block of layer l at batch 1 (ple_block), accumulating into acc.
PleFold ple_fold(const g4_decode &d, int l, void *acc) {
    const g4_decode_layer &L = d.layers[l];
    PleFold F;
    F.join = d.joins[join_index(l, 1)];
    F.w_gate = static_cast<const int8_t *>(L.ple_gate);
    F.s_gate = L.ple_gate_s;
    F.up_vec = d.per_layer + (size_t)l * d.s.ple_dim;
    F.w_proj = static_cast<const int8_t *>(L.ple_proj);
    F.p = d.s.ple_dim;
    F.in_scale = d.s.in_scale;
    F.out_scale = d.s.out_scale;
    F.acc = static_cast<int32_t *>(acc);
    return F;
}

// The FFN block of layer l at batch 1 (ffn_block), accumulating down_proj into acc.
FfnFold ffn_fold(const g4_decode &d, int l, int32_t *acc) {
    const g4_decode_layer &L = d.layers[l];
    FfnFold F;
    F.join = d.joins[join_index(l, 0)];
    F.w_gate = static_cast<const uint8_t *>(L.gate);
    F.w_up = static_cast<const uint8_t *>(L.up);
    F.s_gate = L.gate_s;
    F.s_up = L.up_s;
    F.w_down = d.down_packed.empty() ? static_cast<const uint8_t *>(L.down) : d.down_packed[l];
    F.f = d.s.ffn;
    F.in_scale = d.s.in_scale;
    F.out_scale = d.s.out_scale;
    F.act_scale = d.s.in_scale;
    F.acc = acc;
    // the per-layer-input block's join sums accumulator copies; a plan prologue reads one
    F.acc_copies = d.fold_ple ? kFfnAccCopies : 1;
    return F;
}

int build(g4_decode &d) {
    const g4_decode_shape &s = d.s;
    const int B = s.batch, H = s.hidden, F = s.ffn, QW = s.q_heads * s.head_dim;
    const int PL = s.layers * s.ple_dim;
    DeviceAlloc &m = d.mem;
    auto f32 = [&](float **p, size_t n) { return m.get((void **)p, n * sizeof(float)); };
    auto i8 = [&](int8_t **p, size_t n) { return m.get((void **)p, n); };
    G4_TRY(m.get((void **)&d.pos, sizeof(int32_t)));
    G4_HIP(hipMemset(d.pos, 0, sizeof(int32_t)));
    G4_TRY(f32(&d.identity, (size_t)B * PL));
    G4_TRY(f32(&d.per_layer, (size_t)B * PL));
    G4_TRY(f32(&d.hbuf[0], (size_t)B * H));
    G4_TRY(f32(&d.hbuf[1], (size_t)B * H));
    G4_TRY(f32(&d.logits, (size_t)B * s.vocab));
    d.attn_ws_bytes = g4_attention_workspace_bytes(B, s.q_heads, s.kv_capacity - 1, 0);
    G4_TRY(m.get((void **)&d.attn_ws, d.attn_ws_bytes));
    d.argmax_ws_bytes = g4_argmax_workspace_bytes(B, s.vocab);
    G4_TRY(m.get(&d.argmax_ws, d.argmax_ws_bytes));
    G4_TRY(i8(&d.embed_codes, (size_t)B * H));
    G4_TRY(i8(&d.ple_codes, (size_t)B * PL));
    G4_TRY(i8(&d.xcodes, (size_t)B * H));
    G4_TRY(i8(&d.qc, (size_t)B * QW));
    G4_TRY(i8(&d.kc, (size_t)B * s.head_dim));
    G4_TRY(i8(&d.vc, (size_t)B * s.head_dim));
    G4_TRY(i8(&d.attn_codes, (size_t)B * QW));
    G4_TRY(i8(&d.oc, (size_t)B * H));
    G4_TRY(i8(&d.gc, (size_t)B * F));
    G4_TRY(i8(&d.uc, (size_t)B * F));
    G4_TRY(i8(&d.act, (size_t)B * F));
    G4_TRY(i8(&d.dc, (size_t)B * H));
    G4_TRY(i8(&d.pgc, (size_t)B * s.ple_dim));
    G4_TRY(i8(&d.pac, (size_t)B * s.ple_dim));
    G4_TRY(i8(&d.ppc, (size_t)B * H));
    G4_TRY(i8(&d.head_codes, (size_t)B * H));
    if (acc_split(s))
        G4_TRY(m.get((void **)&d.acc, (size_t)kAccSplits * B * H * sizeof(int32_t)));
    const size_t cache = (size_t)B * 2 * s.kv_capacity * s.head_dim;
    d.kv.assign(s.kv_producers, nullptr);
    for (int p = 0; p < s.kv_producers; ++p) {
        G4_TRY(f32(&d.kv[p], cache));
        G4_HIP(hipMemset(d.kv[p], 0, cache * sizeof(float)));
    }
    build_joins(d);
    if (B != 1) return G4_OK;
    const float in = s.in_scale, out = s.out_scale;
    // o_proj folded into the attention merge when every layer's weights fit its form: each head's
    // merge block contracts its 256 codes with that head's K range of o_proj and adds the exact
    // partial into one int32 accumulator; the post-attention join applies o_proj's epilogue and
    // snap to it, so it reads o_proj's own codes (one launch fewer per layer)
    bool &fold_o = d.fold_o;
    fold_o = !(s.fold_off & 1);
    for (int l = 0; l < s.layers; ++l) {
        MergeLinear lin;
        lin.w = d.layers[l].o;
        lin.n = H;
        lin.k = QW;
        lin.part = reinterpret_cast<int32_t *>(d.hbuf[0]);  // any non-null pointer: shape check only
        fold_o = fold_o && merge_linear_fits(lin, B, s.q_heads);
    }
    // per_layer_input_gate and per_layer_projection in one launch when every layer fits it: the
    // post-FFN join, the gate rows with their gelu x per-layer-row epilogue and the projection's
    // K range of those rows, added atomically into one int32 accumulator that the tail join reads
    d.fold_ple = !(s.fold_off & 4);
    for (int l = 0; l < s.layers; ++l) d.fold_ple = d.fold_ple && ple_fold_fits(ple_fold(d, l, d.hbuf[0]));
    // gate / up / gelu-mul / down in one launch when every layer fits it: each block's gate and up
    // rows, their gelu-mul codes, and down's K range of those codes added atomically into one
    // int32 accumulator that the post-FFN join reads
    d.fold_ffn = !(s.fold_off & 2);
    for (int l = 0; l < s.layers; ++l)
        d.fold_ffn = d.fold_ffn && ffn_fold_fits(ffn_fold(d, l, reinterpret_cast<int32_t *>(d.hbuf[0])));
    if (fold_o || d.fold_ple || d.fold_ffn)
        G4_TRY(m.get((void **)&d.oacc, (size_t)kAccRows * H * sizeof(int32_t)));
    if (d.fold_ffn) {
        // each layer's down_proj in the block's layout (a copy taken here: the runner reads it in
        // place of the caller's down weights from now on), after every upload the caller queued
        G4_HIP(hipDeviceSynchronize());
        d.down_packed.assign(s.layers, nullptr);
        for (int l = 0; l < s.layers; ++l) {
            G4_TRY(m.get((void **)&d.down_packed[l], (size_t)H * F / 2));
            G4_TRY(ffn_repack_down(static_cast<const uint8_t *>(d.layers[l].down), d.down_packed[l], H, F, nullptr));
        }
        G4_HIP(hipDeviceSynchronize());
        for (int l = 0; l < s.layers; ++l) {
            JoinTail &j = d.joins[join_index(l, 1)];
            j.src = d.oacc + 2 * H;
            j.src_kind = G4_KIND_I32;
            j.acc_scales = d.layers[l].down_s;
            j.acc_in_scale = in;
            j.acc_splits = ffn_fold(d, l, d.oacc + 2 * H).acc_copies;
            j.acc_split_stride = H;
            d.carried[join_index(l, 0)] = 1;  // ffn_block runs it
        }
    }
    if (d.fold_ple) {
        for (int l = 0; l < s.layers; ++l) {
            JoinTail &j = d.joins[join_index(l, 2)];
            j.src = d.oacc + H;
            j.src_kind = G4_KIND_I32;
            j.acc_scales = d.layers[l].ple_proj_s;
            j.acc_in_scale = in;
            j.acc_splits = 1;
            j.acc_split_stride = H;
            d.carried[join_index(l, 1)] = 1;  // ple_block runs it
        }
    }
    if (fold_o) {
        for (int l = 0; l < s.layers; ++l) {
            JoinTail &j = d.joins[join_index(l, 0)];
            j.src = d.oacc;
            j.src_kind = G4_KIND_I32;
            j.acc_scales = d.layers[l].o_s;
            j.acc_in_scale = in;
            j.acc_splits = 1;
            j.acc_split_stride = H;
        }
    }
    // M = 1: one grouped-GEMV plan per launch group.
    d.plans.assign((size_t)s.layers * P_PER_LAYER, Plan{});
    for (int l = 0; l < s.layers; ++l) {
        const g4_decode_layer &L = d.layers[l];
        Plan *P = &d.plans[(size_t)l * P_PER_LAYER];
        std::vector<g4_gemv_desc> g{desc(L.q, L.q_s, d.xcodes, d.qc, 4, H, QW, G4_KIND_I8, in, out)};
        if (l < s.kv_producers) {
            g.push_back(desc(L.k, L.k_s, d.xcodes, d.kc, 4, H, s.head_dim, G4_KIND_I8, in, out));
            g.push_back(desc(L.v, L.v_s, d.xcodes, d.vc, 4, H, s.head_dim, G4_KIND_I8, in, out));
        }
        G4_TRY(try_plan(g.data(), (int)g.size(), P[P_QKV]));
        if (!d.fold_o) {
            g4_gemv_desc o = desc(L.o, L.o_s, d.attn_codes, d.oc, 4, QW, H, G4_KIND_I8, in, out);
            G4_TRY(try_plan(&o, 1, P[P_O]));
        }
        if (!d.fold_ffn) {
            // gate and up rows stream through one paired tile whose epilogue is the gelu-mul pass:
            // act = srq(gelu(gate code * out) * (up code * out), in), the codes down_proj reads
            GeluEpilogue gue;
            gue.w_up = L.up;
            gue.s_up = L.up_s;
            gue.act_scale = in;
            G4_TRY(try_gelu_plan(desc(L.gate, L.gate_s, d.xcodes, d.act, 4, H, F, G4_KIND_I8, in, out),
                                 gue, P[P_GATEUP]));
            if (!P[P_GATEUP].p) {
                g4_gemv_desc gu[2] = {desc(L.gate, L.gate_s, d.xcodes, d.gc, 4, H, F, G4_KIND_I8, in, out),
                                      desc(L.up, L.up_s, d.xcodes, d.uc, 4, H, F, G4_KIND_I8, in, out)};
                G4_TRY(try_plan(gu, 2, P[P_GATEUP]));
            }
            g4_gemv_desc dn = desc(L.down, L.down_s, d.act, d.dc, 4, F, H, G4_KIND_I8, in, out);
            G4_TRY(try_plan(&dn, 1, P[P_DOWN]));
        }
        if (d.fold_ple) continue;  // the per-layer-input block is one ple_block launch
        // per_layer_input_gate's epilogue multiplies gelu(gate) by the layer's per-layer-input row
        GeluEpilogue pge;
        pge.up_vec = d.per_layer + (size_t)l * s.ple_dim;
        pge.act_scale = in;
        G4_TRY(try_gelu_plan(desc(L.ple_gate, L.ple_gate_s, d.xcodes, d.pac, 8, H, s.ple_dim,
                                  G4_KIND_I8, in, out),
                             pge, P[P_PLE_GATE]));
        if (!P[P_PLE_GATE].p) {
            g4_gemv_desc pg = desc(L.ple_gate, L.ple_gate_s, d.xcodes, d.pgc, 8, H, s.ple_dim,
                                   G4_KIND_I8, in, out);
            G4_TRY(try_plan(&pg, 1, P[P_PLE_GATE]));
        }
        g4_gemv_desc pp = desc(L.ple_proj, L.ple_proj_s, d.pac, d.ppc, 8, s.ple_dim, H, G4_KIND_I8,
                               in, out);
        G4_TRY(try_plan(&pp, 1, P[P_PLE_PROJ]));
    }
    g4_gemv_desc pm = desc(d.w.ple_model_proj, d.w.ple_model_proj_s, d.embed_codes, d.ple_codes, 4,
                           H, PL, G4_KIND_I8, in, out);
    G4_TRY(try_plan(&pm, 1, d.ple_model_plan));
    g4_gemv_desc hd = desc(d.w.embed, d.w.embed_s, d.head_codes, d.logits, 4, H, (int)s.vocab,
                           G4_KIND_F32, in, 0.0f);
    G4_TRY(try_plan(&hd, 1, d.head_plan));
    // the plans without a join snap inside their first tile
    for (int l = 0; l < s.layers; ++l) {
        const Plan *P = &d.plans[(size_t)l * P_PER_LAYER];
        for (int i : {P_O, P_DOWN, P_PLE_PROJ})
            if (P[i].p) G4_TRY(gemv_plan_set_first_tile_snap(P[i].p));
    }
    // each join rides in the plan that reads its codes
    G4_TRY(carry_join(d, 0, d.plans[P_QKV]));
    for (int l = 0; l < s.layers; ++l) {
        const Plan *P = &d.plans[(size_t)l * P_PER_LAYER];
        const bool last = l + 1 == s.layers;
        G4_TRY(carry_join(d, join_index(l, 0), P[P_GATEUP]));
        if (!d.fold_ple) G4_TRY(carry_join(d, join_index(l, 1), P[P_PLE_GATE]));
        // the final norm runs as a join launch of its own: carried, it would put the 201 MB head
        // plan on the join instantiation of the stream kernel (half its occupancy), which costs
        // more than the launch (1.422 against 1.415 ms per step)
        if (!last) G4_TRY(carry_join(d, join_index(l, 2), d.plans[(size_t)(l + 1) * P_PER_LAYER + P_QKV]));
    }
    return G4_OK;
}

int run_layer(g4_decode &d, int l, void *st) {
    const g4_decode_shape &s = d.s;
    const g4_decode_layer &L = d.layers[l];
    const int B = s.batch, H = s.hidden, F = s.ffn, QW = s.q_heads * s.head_dim;
    const float in = s.in_scale, out = s.out_scale;
    const bool prod = l < s.kv_producers, glob = is_global(s, l);
    const Plan *P = d.plans.empty() ? nullptr : &d.plans[(size_t)l * P_PER_LAYER];
    static const Plan none;
    auto plan = [&](int i) -> const Plan & { return P ? P[i] : none; };

    // attention block
    if (plan(P_QKV).p) {
        G4_TRY(g4_qgemv_plan_launch(plan(P_QKV).p, st));
    } else {  // q (+ k, v) over the same codes: one grouped launch
        const LinearOut qkv[3] = {{L.q, L.q_s, d.qc, QW},
                                  {L.k, L.k_s, d.kc, s.head_dim},
                                  {L.v, L.v_s, d.vc, s.head_dim}};
        G4_TRY(linear_grouped(4, d.xcodes, G4_KIND_I8, H, B, in, out, G4_KIND_I8, qkv, prod ? 3 : 1, st));
    }
    const int src = kv_source(s, l);
    float *kb = d.kv[src];
    float *vb = kb + (size_t)s.kv_capacity * s.head_dim;
    const int64_t row_stride = (int64_t)2 * s.kv_capacity * s.head_dim;
    const float *cos_tab = glob ? d.w.rope_global_cos : d.w.rope_local_cos;
    const float *sin_tab = glob ? d.w.rope_global_sin : d.w.rope_local_sin;
    AttnPrologue pro{};
    pro.q_codes = d.qc;
    pro.q_scale = out;
    pro.k_codes = prod ? d.kc : nullptr;
    pro.k_scale = out;
    pro.v_codes = prod ? d.vc : nullptr;
    pro.v_scale = out;
    pro.q_gain = L.q_norm;
    pro.k_gain = prod ? L.k_norm : nullptr;
    pro.cos_tab = cos_tab;
    pro.sin_tab = sin_tab;
    pro.eps = s.eps;
    pro.zero = d.oacc;
    pro.zero_n = d.oacc ? kAccRows * H : 0;
    MergeLinear lin;
    lin.w = L.o;
    lin.n = H;
    lin.k = QW;
    lin.part = d.oacc;
    G4_TRY(attention_decode_fused(pro, kb, vb, row_stride, B, s.q_heads, s.kv_capacity - 1, d.pos,
                                  glob ? 0 : s.sliding_window, d.attn_ws, d.attn_ws_bytes, in,
                                  d.attn_codes, st, d.fold_o ? &lin : nullptr));
    if (!d.fold_o)
        G4_TRY(run_linear_rows(d, plan(P_O), desc(L.o, L.o_s, d.attn_codes, d.oc, 4, QW, H, G4_KIND_I8, in, out), st));
    G4_TRY(run_join(d, join_index(l, 0), st));
    // MLP block: gate, up and the gelu-mul pass (one paired launch when folded), then down; at
    // batch 1 all of it is one ffn_block launch
    if (d.fold_ffn) {
        G4_TRY(ffn_block(ffn_fold(d, l, d.oacc + 2 * H), st));
    } else if (plan(P_GATEUP).gelu) {
        G4_TRY(g4_qgemv_plan_launch(plan(P_GATEUP).p, st));
    } else {
        // batch > 1: the small-M kernel with paired gate/up rows and the gelu-mul epilogue
        bool fused = false;
        if (!plan(P_GATEUP).p)
            G4_TRY(linear_gelu(4, d.xcodes, H, B, in, out, L.gate, L.gate_s, L.up, L.up_s, nullptr,
                               0, F, in, d.act, st, &fused));
        if (!fused) {
            if (plan(P_GATEUP).p) {
                G4_TRY(g4_qgemv_plan_launch(plan(P_GATEUP).p, st));
            } else {  // gate and up over the same codes: one grouped launch
                const LinearOut gu[2] = {{L.gate, L.gate_s, d.gc, F}, {L.up, L.up_s, d.uc, F}};
                G4_TRY(linear_grouped(4, d.xcodes, G4_KIND_I8, H, B, in, out, G4_KIND_I8, gu, 2, st));
            }
            G4_TRY(g4_gelu_mul(d.gc, out, d.uc, out, nullptr, 0, B, F, in, d.act, st));
        }
    }
    if (d.acc)
        G4_TRY(linear_split_acc(4, static_cast<const uint8_t *>(L.down), L.down_s, d.act, F, H, B,
                                kAccSplits, d.acc, as_stream(st)));
    else if (!d.fold_ffn)
        G4_TRY(run_linear_rows(d, plan(P_DOWN), desc(L.down, L.down_s, d.act, d.dc, 4, F, H, G4_KIND_I8, in, out), st));
    G4_TRY(run_join(d, join_index(l, 1), st));
    // per-layer-input block: the gate (with gelu times the layer's row folded when planned), then
    // per_layer_projection
    if (d.fold_ple) {
        G4_TRY(ple_block(ple_fold(d, l, d.oacc + H), st));
    } else if (plan(P_PLE_GATE).gelu) {
        G4_TRY(g4_qgemv_plan_launch(plan(P_PLE_GATE).p, st));
    } else {
        bool fused = false;
        if (!plan(P_PLE_GATE).p)
            G4_TRY(linear_gelu(8, d.xcodes, H, B, in, out, L.ple_gate, L.ple_gate_s, nullptr, nullptr,
                               d.per_layer + (size_t)l * s.ple_dim, (int64_t)s.layers * s.ple_dim,
                               s.ple_dim, in, d.pac, st, &fused));
        if (!fused) {
            G4_TRY(run_linear_rows(d, plan(P_PLE_GATE), desc(L.ple_gate, L.ple_gate_s, d.xcodes, d.pgc, 8, H, s.ple_dim, G4_KIND_I8, in, out), st));
            G4_TRY(g4_gelu_mul(d.pgc, out, nullptr, 0.0f, d.per_layer + (size_t)l * s.ple_dim,
                               (int64_t)s.layers * s.ple_dim, B, s.ple_dim, in, d.pac, st));
        }
    }
    if (!d.fold_ple)
        G4_TRY(run_linear_rows(d, plan(P_PLE_PROJ), desc(L.ple_proj, L.ple_proj_s, d.pac, d.ppc, 8, s.ple_dim, H, G4_KIND_I8, in, out), st));
    // the tail join: residual, layer scalar, then the next input norm (or the final norm)
    // the tail join: residual, layer scalar, then the next input norm (or the final norm); a step
    // that stops here launches it even when the next layer's plan would carry it
    const int k = join_index(l, 2);
    if (!d.carried[k] || (l == d.stop && l + 1 < s.layers)) G4_TRY(launch_join(d, k, st));
    return G4_OK;
}

// The index of the step's last join (its row is the final residual): the tail join of the last
// layer run.
int last_join(const g4_decode &d) {
    const int last = d.stop >= 0 ? d.stop : d.s.layers - 1;
    return join_index(last, 2);
}

}  // namespace

extern "C" {

int g4_decode_create(const g4_decode_shape *shape, const g4_decode_weights *weights,
                     g4_decode **out) {
    if (!shape || !weights || !out) return set_error(G4_ERR_INVALID, "decode: null argument");
    *out = nullptr;
    G4_TRY(check_shape(*shape));
    G4_TRY(check_weights(*shape, *weights));
    g4_decode *d = new (std::nothrow) g4_decode();
    if (!d) return set_error(G4_ERR_INVALID, "decode: out of host memory");
    d->s = *shape;
    d->w = *weights;
    d->layers.assign(weights->layer, weights->layer + shape->layers);
    d->w.layer = d->layers.data();
    if (weights->ple_num_slices > 0) {
        const int n = weights->ple_num_slices;
        d->ple_split_codes.assign(weights->ple_slice_codes, weights->ple_slice_codes + n);
        d->ple_split_start.assign(weights->ple_slice_start, weights->ple_slice_start + n);
        d->ple_split_rows.assign(weights->ple_slice_rows, weights->ple_slice_rows + n);
    }
    d->w.ple_slice_codes = nullptr;  // the copies above are the runner's
    d->w.ple_slice_start = d->w.ple_slice_rows = nullptr;
    int rc = build(*d);
    if (rc != G4_OK) {
        delete d;
        return rc;
    }
    *out = d;
    return G4_OK;
}

int g4_decode_destroy(g4_decode *d) {
    if (d) {
        (void)hipDeviceSynchronize();
        delete d;
    }
    return G4_OK;
}

int g4_decode_kv(g4_decode *d, int layer, float **k, float **v, int64_t *row_stride) {
    if (!d || layer < 0 || layer >= d->s.kv_producers)
        return set_error(G4_ERR_INVALID, "decode: layer %d owns no KV cache", layer);
    if (k) *k = d->kv[layer];
    if (v) *v = d->kv[layer] + (size_t)d->s.kv_capacity * d->s.head_dim;
    if (row_stride) *row_stride = (int64_t)2 * d->s.kv_capacity * d->s.head_dim;
    return G4_OK;
}

int g4_decode_position(g4_decode *d, int32_t **pos) {
    if (!d || !pos) return set_error(G4_ERR_INVALID, "decode: null argument");
    *pos = d->pos;
    return G4_OK;
}

int g4_decode_set_position(g4_decode *d, int pos, void *stream) {
    if (!d) return set_error(G4_ERR_INVALID, "decode: null argument");
    if (pos < 0 || pos >= d->s.kv_capacity)
        return set_error(G4_ERR_INVALID, "decode: position %d outside the KV capacity %d", pos,
                         d->s.kv_capacity);
    hipLaunchKernelGGL(set_word_kernel, dim3(1), dim3(1), 0, as_stream(stream), d->pos, pos);
    G4_LAUNCHED("set_word_kernel");
    return G4_OK;
}

int g4_decode_set_stop(g4_decode *d, int last_layer) {
    if (!d || last_layer < -1 || last_layer >= d->s.layers)
        return set_error(G4_ERR_INVALID, "decode: stop layer %d", last_layer);
    d->stop = last_layer;
    return G4_OK;
}

int g4_decode_buffer(g4_decode *d, const char *name, void **ptr, size_t *bytes) {
    if (!d || !name || !ptr) return set_error(G4_ERR_INVALID, "decode: null argument");
    const g4_decode_shape &s = d->s;
    const size_t B = (size_t)s.batch;
    struct Named {
        const char *n;
        void *p;
        size_t b;
    } all[] = {
        {"hidden", d->hbuf[last_join(*d) & 1], B * s.hidden * 4},
        {"logits", d->logits, B * (size_t)s.vocab * 4},
        {"per_layer", d->per_layer, B * s.layers * s.ple_dim * 4},
        {"head_codes", d->head_codes, B * s.hidden},
        {"codes", d->xcodes, B * s.hidden},
    };
    for (const Named &n : all)
        if (std::strcmp(n.n, name) == 0) {
            *ptr = n.p;
            if (bytes) *bytes = n.b;
            return G4_OK;
        }
    return set_error(G4_ERR_INVALID, "decode: no buffer named '%s'", name);
}

int g4_decode_step(g4_decode *d, const int32_t *tokens, int32_t *next_tokens, void *stream) {
    if (!d || !tokens || !next_tokens) return set_error(G4_ERR_INVALID, "decode: null argument");
    const g4_decode_shape &s = d->s;
    const int B = s.batch, H = s.hidden, PL = s.layers * s.ple_dim;
    const float in = s.in_scale, out = s.out_scale;
    // embedding phase: the residual stream starts at the scaled embedding
    const float embed_scale = (float)std::sqrt((double)H);
    G4_TRY(g4_embed_tokens(d->w.embed, d->w.embed_s, tokens, B, s.vocab, H, embed_scale, in,
                           d->hbuf[0], d->embed_codes, stream));
    // the unsliced gather over all `vocab` rows, or every slice of a split table in one launch;
    // either way an id outside the vocabulary gives a zero row
    if (d->ple_split_codes.empty())
        G4_TRY(g4_ple_gather(d->w.ple_table, d->w.ple_table_s, 0, tokens, d->identity, G4_KIND_F32,
                             B, PL, s.ple_dim, s.layers, 0, 0, s.vocab, stream));
    else
        G4_TRY(g4_ple_gather_split(d->ple_split_codes.data(), d->ple_split_start.data(),
                                   d->ple_split_rows.data(), (int)d->ple_split_codes.size(), d->w.ple_table_s, G4_KIND_F32, tokens,
                                   d->identity, G4_KIND_F32, B, PL, s.ple_dim, s.layers, stream));
    G4_TRY(run_linear_rows(*d, d->ple_model_plan,
                           desc(d->w.ple_model_proj, d->w.ple_model_proj_s, d->embed_codes,
                                d->ple_codes, 4, H, PL, G4_KIND_I8, in, out),
                           stream));
    const float alpha = (float)std::pow((double)H, -0.5);
    G4_TRY(g4_ple_combine(d->ple_codes, out, alpha, d->w.ple_proj_norm, d->identity, B, s.layers,
                          s.ple_dim, s.eps, d->per_layer, stream));
    G4_TRY(run_join(*d, 0, stream));
    const int last = d->stop >= 0 ? d->stop : s.layers - 1;
    for (int l = 0; l <= last; ++l) G4_TRY(run_layer(*d, l, stream));
    if (last != s.layers - 1) return G4_OK;
    // head: tied int4 GEMV to f32 logits, softcap in place, argmax
    G4_TRY(run_linear_rows(*d, d->head_plan,
                           desc(d->w.embed, d->w.embed_s, d->head_codes, d->logits, 4, H,
                                (int)s.vocab, G4_KIND_F32, in, 0.0f),
                           stream));
    G4_TRY(g4_softcap_argmax(d->logits, B, s.vocab, s.final_softcap, d->logits, d->argmax_ws,
                             d->argmax_ws_bytes, next_tokens, stream));
    return G4_OK;
}

}  // extern "C"

// The decode-step glue around the quantized projections (the E2B-shape step of BASELINE config 4):
// RMS norm and its residual joins, q/k norm + RoPE + KV store, split attention decode and merge,
// gelu * up, the token embedding, the per-layer-input combine, logit softcap and argmax.
//
// Reference kernels (Ar5en1c/gemma4-webgpu-engine): rmsNorm.ts:131-180 (rms-norm),
// mlpEpilogue.ts:196-230 (norm-residual), blockJoin.ts:160-175 (norm-residual-norm),
// attnPrologue.ts:268-329 (q-norm-rope, kv-norm-rope-store), rope.ts:240-258 (split half form),
// attention.ts:858-918 (attention decode, scale 1.0, sliding window), geluMul.ts:101-116 (gelu),
// embedGather.ts:93-113 (embed scale folded once), plan.ts:670-690 (per-layer inputs),
// logitSoftcap.ts:104-124 and argmax.ts:267-300 (first strict maximum).
//
// The arithmetic is fixed so the CPU oracle (oracle/g4_decode_oracle.c) can state it exactly:
//  - every reduction is 256 lane-strided partial sums (lane l takes elements l, l+256, ...
//    ascending) followed by a pairwise tree (stride 128 down to 1, lane l adds lane l + stride);
//  - 1/sqrt is the IEEE square root then the IEEE divide;
//  - exp and tanh are d_expf / d_tanhf: Cody-Waite reduction, a degree-6 Taylor polynomial and
//    ldexp (tanh of small arguments through the same polynomial as expm1), every step separately
//    rounded;
//  - attention runs in chunks of 32 positions, merged in ascending chunk order; a score is eight
//    sequential 32-dim dot products combined by a pairwise tree.
// The projections between these kernels are the library's GEMV/GEMM entry points, which take and
// give int8 codes: every kernel here that feeds a projection emits its input snap directly.
#include "g4_rowops.h"
#include "../../include/g4decode.h"
#include <algorithm>
#include <cmath>

namespace g4 {

constexpr int kDecThreads = 256;
constexpr int kAttnChunk = 32;
constexpr int kAttnMaxHeads = 8;
// Word 3 of a gfx9 buffer resource for untyped dword loads (DATA_FORMAT 32, no swizzle).
constexpr int kBufferRsrcWord3 = 0x00020000;

// d_expf, d_tanhf and d_gelu (the deterministic exp / tanh / gelu) live in g4_internal.h, shared
// with the GEMV gelu prologues; block_tree_sum, inv_rms and the RMS join row in g4_rowops.h, shared
// with the GEMV whose last block runs a join.
static_assert(kDecThreads == kRowThreads, "the glue kernels run the shared 256-lane row operations");

// ---- rms-norm / norm-residual / norm-residual-norm --------------------------------------------------

// One block per row (rms_join_row). ACC: the source is split accumulators (acc_sum, acc_value).
// G2 false: a join without a second gain (the one after down_proj), whose launcher picks this form
// when J.gain2 is null, so the absent operand is neither loaded nor tested.
template <bool ACC, int PER, bool G2 = true>
__global__ __launch_bounds__(kDecThreads) void join_kernel(JoinTail J) {
    __shared__ float lds[2 * kDecThreads];
    rms_join_row<ACC ? kSplitAccMax : 0, PER, G2>(J, blockIdx.x, lds);
}

int join_acc(const JoinTail &J, int rows, hipStream_t stream) {
    if (J.src_kind != G4_KIND_I32 || !J.src || !J.acc_scales || J.acc_splits < 1 ||
        J.acc_splits > kSplitAccMax || rows <= 0 || J.width <= 0 ||
        J.width > kJoinMaxPer * kDecThreads || J.src_scale == 0.0f || !J.codes ||
        J.in_scale == 0.0f)
        return set_error(G4_ERR_INVALID, "join over split accumulators: bad arguments");
    const bool narrow = join_narrow(J.width);
    if (narrow && J.gain2)
        hipLaunchKernelGGL((join_kernel<true, kJoinPerNarrow>), dim3(rows), dim3(kDecThreads), 0, stream, J);
    else if (narrow)
        hipLaunchKernelGGL((join_kernel<true, kJoinPerNarrow, false>), dim3(rows), dim3(kDecThreads), 0, stream, J);
    else if (J.gain2)
        hipLaunchKernelGGL((join_kernel<true, kJoinMaxPer>), dim3(rows), dim3(kDecThreads), 0, stream, J);
    else
        hipLaunchKernelGGL((join_kernel<true, kJoinMaxPer, false>), dim3(rows), dim3(kDecThreads), 0, stream, J);
    G4_LAUNCHED("join_kernel");
    return G4_OK;
}

// ---- q-norm-rope and kv-norm-rope-store ----------------------------------------------------------

// The position a step works on: the device word when the step is replayed from a captured graph,
// clamped to [0, pos_host] (then the largest position the caches and the split grid were sized
// for, so no value of the word reaches outside them), else the host value.
__device__ __forceinline__ int step_pos(int pos_host, const int32_t *pos_dev) {
    return pos_dev ? min(max(*pos_dev, 0), pos_host) : pos_host;
}

// Grid (heads [+ 2 on a producer layer], rows); 256 threads = one head_dim 256 row. Blocks below
// `heads` norm + rotate a query head into q_out [row][heads][256]; block `heads` norms + rotates
// k into the K cache at the position, block heads + 1 norms v (weightless) into the V cache there.
// cos_tab / sin_tab: [positions][128] tables, read at the position's row.
__global__ __launch_bounds__(kDecThreads) void attn_prologue_kernel(
    const int8_t *q_codes, float q_scale, const int8_t *k_codes, float k_scale,
    const int8_t *v_codes, float v_scale, const float *q_gain, const float *k_gain,
    const float *cos_tab, const float *sin_tab, int heads, float eps, float *q_out, float *k_cache,
    float *v_cache, int64_t cache_row_stride, int pos_host, const int32_t *pos_dev) {
    __shared__ float lds[kDecThreads];
    __shared__ float xs[kDecThreads];
    const int t = threadIdx.x;
    const int h = blockIdx.x;
    const int64_t row = blockIdx.y;
    const int pos = step_pos(pos_host, pos_dev);
    const float *cos_row = cos_tab + (int64_t)pos * (kDecThreads / 2);
    const float *sin_row = sin_tab + (int64_t)pos * (kDecThreads / 2);
    const int8_t *src;
    float scale;
    const float *gain;
    float *dst;
    bool rotate = true;
    if (h < heads) {
        src = q_codes + (row * heads + h) * kDecThreads;
        scale = q_scale;
        gain = q_gain;
        dst = q_out + (row * heads + h) * kDecThreads;
    } else if (h == heads) {
        src = k_codes + row * kDecThreads;
        scale = k_scale;
        gain = k_gain;
        dst = k_cache + row * cache_row_stride + (int64_t)pos * kDecThreads;
    } else {
        src = v_codes + row * kDecThreads;
        scale = v_scale;
        gain = nullptr;
        dst = v_cache + row * cache_row_stride + (int64_t)pos * kDecThreads;
        rotate = false;
    }
    constexpr int P = kDecThreads / 2;
    const int i = t < P ? t : t - P;
    const float x = __fmul_rn((float)src[t], scale);
    const float gt = gain ? gain[t] : 1.0f;
    const float c = cos_row[i], s = sin_row[i];  // loaded before the barriers, like the rest
    const float inv = inv_rms(block_tree_sum(__fmul_rn(x, x), lds), kDecThreads, eps);
    float y = __fmul_rn(x, inv);
    if (gain) y = __fmul_rn(y, gt);
    if (!rotate) {
        dst[t] = y;
        return;
    }
    xs[t] = y;
    __syncthreads();
    const float lo = xs[i], hi = xs[i + P];
    dst[t] = t < P ? __fsub_rn(__fmul_rn(lo, c), __fmul_rn(hi, s))
                   : __fadd_rn(__fmul_rn(hi, c), __fmul_rn(lo, s));
}

// ---- attention decode: split partials, then the ordered merge -------------------------------------

// attn_prologue_kernel's arithmetic for one 256-wide head vector on one wave: lane l holds
// elements l, l + 64, l + 128 and l + 192, so the block tree's levels 128 and 64 are in-lane adds
// in the same order (x[l]^2 + x[l+128]^2, then + (x[l+64]^2 + x[l+192]^2)) and the rest is the same
// shuffle tree; the RoPE pairs (i, i + 128) are in-lane too. The operands are loaded first and kept
// raw, so a caller can put them ahead of a longer stream of loads without waiting. Every operand is
// loaded unconditionally (callers pass valid stand-ins for what they will not use): a load under a
// branch makes the compiler wait for it at the branch's end, which put a memory round trip per
// head ahead of the chunk's K and V loads. Each load instruction costs the wave the same address
// work whatever its width, so the codes come as one 4-byte load per lane and the gain and the
// position's cos / sin row once per wave for all of its vectors.
struct RopeRow {
    float c[2], sn[2];
};

__device__ __forceinline__ RopeRow wave_rope_row(const float *cos_row, const float *sin_row) {
    const int l = threadIdx.x & 63;
    RopeRow r;
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        r.c[k] = cos_row[l + 64 * k];
        r.sn[k] = sin_row[l + 64 * k];
    }
    return r;
}

__device__ __forceinline__ void wave_gain_load(const float *gain, float (&gt)[4]) {
    const int l = threadIdx.x & 63;
#pragma unroll
    for (int k = 0; k < 4; ++k) gt[k] = gain[l + 64 * k];
}

// A 256-code vector (4-byte aligned) as codes 4 l .. 4 l + 3 in lane l; wave_codes_spread hands
// lane l its codes l + 64 k (from lane l / 4 + 16 k, byte l % 4) by cross-lane reads.
__device__ __forceinline__ uint32_t wave_codes_word(const int8_t *src) {
    return reinterpret_cast<const uint32_t *>(src)[threadIdx.x & 63];
}

__device__ __forceinline__ void wave_codes_spread(uint32_t word, int (&code)[4]) {
    const int l = threadIdx.x & 63;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const uint32_t v = (uint32_t)__builtin_amdgcn_ds_bpermute(((l >> 2) + 16 * k) << 2, (int)word);
        code[k] = (int)(int8_t)(v >> (8 * (l & 3)));
    }
}

// Writes the four results of the lane to out[l + 64 k].
__device__ __forceinline__ void wave_norm_rope(const int (&code)[4], const float (&gt)[4],
                                               const RopeRow &rope, float scale, bool gain,
                                               bool rotate, float eps, float *out) {
    const int l = threadIdx.x & 63;
    float x[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) x[k] = __fmul_rn((float)code[k], scale);
    float part = __fadd_rn(__fadd_rn(__fmul_rn(x[0], x[0]), __fmul_rn(x[2], x[2])),
                           __fadd_rn(__fmul_rn(x[1], x[1]), __fmul_rn(x[3], x[3])));
    const float inv = inv_rms(wave_tree_sum(part), kDecThreads, eps);
    float y[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        y[k] = __fmul_rn(x[k], inv);
        if (gain) y[k] = __fmul_rn(y[k], gt[k]);
    }
    if (!rotate) {
#pragma unroll
        for (int k = 0; k < 4; ++k) out[l + 64 * k] = y[k];
        return;
    }
#pragma unroll
    for (int k = 0; k < 2; ++k) {  // pair (l + 64 k, l + 64 k + 128)
        const float lo = y[k], hi = y[k + 2];
        out[l + 64 * k] = __fsub_rn(__fmul_rn(lo, rope.c[k]), __fmul_rn(hi, rope.sn[k]));
        out[l + 64 * k + 128] = __fadd_rn(__fmul_rn(hi, rope.c[k]), __fmul_rn(lo, rope.sn[k]));
    }
}

// Grid (max chunks, rows), HALVES x 256 threads (t = the thread's index in its half of 256).
// Chunk c covers positions lo + 32 c .. min(+32, pos + 1), for every query head of the row at once
// (heads <= 8 share the one KV head), so each K and V row of the chunk is fetched once per block.
// HALVES 2 (a grid no wider than the CU count: batch 1): half 0 takes heads 0..3, half 1 heads
// 4..7, two waves per SIMD with half the dependent chains each; HALVES 1 (wide grids, where the
// chip is full anyway): every thread takes all heads. Scores: thread t takes eighth t & 7 (32 dims, sequential) of position t >> 3 against its
// half's heads, and the position's eight lanes combine by the pairwise tree
// ((s0 + s1) + (s2 + s3)) + ((s4 + s5) + (s6 + s7)) (an xor butterfly: IEEE addition commutes, so
// every lane ends with the tree's value). Per head (one 32-lane group of half 0 each): m = max,
// e = exp(s - m), l = the 32-lane pairwise tree of e. Then thread t accumulates, for its half's
// heads, sum over positions (ascending) of e * v[t]. Writes (m, l) and o[256] per (row, head,
// chunk). PRO: q (and on a producer, the position's K and V rows) come from the prologue run here:
// wave w rebuilds query heads w, w + waves, ...; in the block whose chunk holds the position, waves
// 0 and 1 also build the new K and V rows, which the block stores and uses in place of the stale
// rows it loaded.
// Float4 slot of the chunk's K group (row r, float4 column c4) in the split kernel's LDS copy.
// Within each 8-slot segment (one lane's 32 dims), slot m moves to (m + seg/2 + 4*(r&1)) mod 8:
// the 16 lanes of one ds_read_b128 phase (two rows x eight segments, same m) then hit 16
// distinct 4-bank groups, and 16 consecutive columns of one row (a write phase) stay distinct.
__device__ __forceinline__ int k_slot(int r, int c4) {
    const int seg = c4 >> 3;
    return r * (kDecThreads / 4) + seg * 8 + (((c4 & 7) + (seg >> 1) + 4 * (r & 1)) & 7);
}

template <bool PRO, int HALVES, bool KST>
__global__ __launch_bounds__(HALVES * kDecThreads) void attn_split_kernel(
    const float *q, const float *k_cache, const float *v_cache, int64_t cache_row_stride, int heads,
    int pos_host, const int32_t *pos_dev, int window, float *part_ml, float *part_o, int max_chunks,
    AttnPrologue pro) {
    __shared__ __align__(16) float qs[kAttnMaxHeads * kDecThreads];
    __shared__ __align__(16) float es[kAttnMaxHeads * kAttnChunk];
    __shared__ __align__(16) float kvnew[PRO ? 2 * kDecThreads : 1];
    __shared__ __align__(16) float4 ks[KST ? kAttnChunk * kDecThreads / 4 : 1];
    constexpr int THREADS = HALVES * kDecThreads, WAVES = THREADS / 64;
    constexpr int HH = kAttnMaxHeads / HALVES;        // heads per thread in scores and PV
    constexpr int QPW = (kAttnMaxHeads + WAVES - 1) / WAVES;  // query heads per wave (prologue)
    const int tid = threadIdx.x;
    const int half = tid >> 8, t = tid & (kDecThreads - 1), w = tid >> 6;
    const int c = blockIdx.x;
    const int64_t row = blockIdx.y;
    const int pos = step_pos(pos_host, pos_dev);
    const int lo = window > 0 ? max(0, pos - window + 1) : 0;
    const int chunks = (pos - lo + 1 + kAttnChunk - 1) / kAttnChunk;
    if (c >= chunks) return;  // whole block
    // the accumulator the merge adds o_proj's per-head partials into starts at zero
    if (PRO && pro.zero && c == 0 && row == 0)
        for (int i = tid; i < pro.zero_n; i += THREADS) pro.zero[i] = 0;
    const int start = lo + c * kAttnChunk;
    const int cnt = min(kAttnChunk, pos + 1 - start);
    float *kb = const_cast<float *>(k_cache) + row * cache_row_stride;
    float *vb = const_cast<float *>(v_cache) + row * cache_row_stride;
    // the producer's new K and V rows belong to the chunk that holds the position (its last)
    const bool store_kv = PRO && pro.k_codes && c == chunks - 1;
    // the prologue's few operands go out first, then the chunk's K segment and V rows, so the
    // prologue's arithmetic waits for its own loads only and overlaps the chunk's
    uint32_t qw[QPW], kvw = 0;
    float qg[4], kg[4];
    RopeRow rope;
    if (PRO) {
        // heads past the last and the K / V rows of waves that do not build them read valid
        // stand-ins (the last head, this row's first query head, the q gain) whose values go unused
        const float *cos_row = pro.cos_tab + (int64_t)pos * (kDecThreads / 2);
        const float *sin_row = pro.sin_tab + (int64_t)pos * (kDecThreads / 2);
#pragma unroll
        for (int i = 0; i < QPW; ++i) {
            const int h = min(w + WAVES * i, heads - 1);
            qw[i] = wave_codes_word(pro.q_codes + (row * heads + h) * kDecThreads);
        }
        const bool kv_wave = store_kv && w < 2;  // wave 0: the K row, wave 1: the V row
        const int8_t *kv_src = !kv_wave ? pro.q_codes + row * heads * kDecThreads
                               : w == 0 ? pro.k_codes + row * kDecThreads
                                        : pro.v_codes + row * kDecThreads;
        kvw = wave_codes_word(kv_src);
        wave_gain_load(pro.q_gain, qg);
        wave_gain_load(kv_wave && w == 0 ? pro.k_gain : pro.q_gain, kg);
        rope = wave_rope_row(cos_row, sin_row);
    }
    __builtin_amdgcn_sched_barrier(0);  // the prologue's loads first, then K, then V
    const int j = t >> 3, sg = t & 7;
    float4 kq[8];
    // KST: the chunk's K rows come in as whole-row float4 runs (one load instruction covers
    // consecutive 16-byte columns) and reach the lanes' 32-dim segments through LDS; otherwise
    // each lane reads its own segment (eight loads, each spread over 64 lines)
    constexpr int KPT = KST ? kAttnChunk * kDecThreads / 4 / THREADS : 1;
    float4 kl[KPT];
    // The chunk's rows start .. start + cnt - 1 of K and V as buffer resources: a load is the
    // lane's byte offset (one VGPR for every load) plus a scalar row offset, where 64-bit vector
    // addresses per load would hold two VGPRs each until it issues. Every offset stays inside the
    // cnt rows (rows clamped to cnt - 1).
    constexpr int kRowBytes = kDecThreads * 4;
    const __amdgpu_buffer_rsrc_t kres = __builtin_amdgcn_make_buffer_rsrc(
        kb + (int64_t)start * kDecThreads, (short)0, cnt * kRowBytes, kBufferRsrcWord3);
    const __amdgpu_buffer_rsrc_t vres = __builtin_amdgcn_make_buffer_rsrc(
        vb + (int64_t)start * kDecThreads, (short)0, cnt * kRowBytes, kBufferRsrcWord3);
    // KST, load i: thread f = tid + i * THREADS takes row f / 64 (wave-uniform), float4 column
    // f % 64, of K and of V
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63;
    if (KST) {
#pragma unroll
        for (int i = 0; i < KPT; ++i) {
            const int r = min(wv + WAVES * i, cnt - 1);
            kl[i] = __builtin_bit_cast(
                float4, __builtin_amdgcn_raw_buffer_load_b128(kres, lane * 16, r * kRowBytes, 0));
        }
    } else {
        const float4 *kr = reinterpret_cast<const float4 *>(
            kb + (int64_t)(start + min(j, cnt - 1)) * kDecThreads + sg * 32);
#pragma unroll
        for (int i4 = 0; i4 < 8; ++i4) kq[i4] = kr[i4];
    }
    __builtin_amdgcn_sched_barrier(0);  // K ahead of V: the wait for K leaves V in flight
    // KST: V as whole-row float4 runs too, staged through the K copy's LDS once the scores are
    // done; otherwise lane t loads dim t of every position
    float4 vl[KST ? KPT : 1];
    float vv[KST ? 1 : kAttnChunk];
    if (KST) {
#pragma unroll
        for (int i = 0; i < KPT; ++i) {
            const int r = min(wv + WAVES * i, cnt - 1);
            vl[i] = __builtin_bit_cast(
                float4, __builtin_amdgcn_raw_buffer_load_b128(vres, lane * 16, r * kRowBytes, 0));
        }
    } else {
#pragma unroll
        for (int u = 0; u < kAttnChunk; ++u)
            vv[u] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                                  vres, t * 4, min(u, cnt - 1) * kRowBytes, 0));
    }
    __builtin_amdgcn_sched_barrier(0);  // every load issued before the prologue's arithmetic
    if (PRO) {
#pragma unroll
        for (int i = 0; i < QPW; ++i) {
            const int h = w + WAVES * i;
            if (h < heads) {
                int code[4];
                wave_codes_spread(qw[i], code);
                wave_norm_rope(code, qg, rope, pro.q_scale, true, true, pro.eps, qs + h * kDecThreads);
            }
        }
        if (store_kv && w < 2) {
            int code[4];
            wave_codes_spread(kvw, code);
            if (w == 0) wave_norm_rope(code, kg, rope, pro.k_scale, true, true, pro.eps, kvnew);
            else wave_norm_rope(code, kg, rope, pro.v_scale, false, false, pro.eps, kvnew + kDecThreads);
        }
    } else {
        for (int i = tid; i < heads * kDecThreads; i += THREADS)
            qs[i] = q[row * heads * kDecThreads + i];
    }
    if (KST) {
#pragma unroll
        for (int i = 0; i < KPT; ++i) {
            const int f = tid + i * THREADS;
            ks[k_slot(f / (kDecThreads / 4), f % (kDecThreads / 4))] = kl[i];
        }
    }
    __syncthreads();
    if (KST) {
#pragma unroll
        for (int i4 = 0; i4 < 8; ++i4) kq[i4] = ks[k_slot(j, sg * 8 + i4)];
    }
    if (store_kv) {
        // the position's row: the cache gets it, and this block's operands take it in place of the
        // stale row they loaded
        const int jp = pos - start;
        if (half == 0) {
            kb[(int64_t)pos * kDecThreads + t] = kvnew[t];
            vb[(int64_t)pos * kDecThreads + t] = kvnew[kDecThreads + t];
        }
        if (j == jp) {
#pragma unroll
            for (int i4 = 0; i4 < 8; ++i4)
                kq[i4] = *reinterpret_cast<const float4 *>(kvnew + sg * 32 + 4 * i4);
        }
        if (!KST) {  // KST: the V row is replaced where the rows go to LDS
#pragma unroll
            for (int u = 0; u < kAttnChunk; ++u)
                if (u == jp) vv[u] = kvnew[kDecThreads + t];
        }
    }

    // scores of this half's heads: eight sequential 32-dim dot products (segment sg) per score, one
    // fused multiply-add (a single rounding) per element, as the CPU restatement's fmaf;
    // then the pairwise tree over the segments by DPP within each aligned 8-lane group:
    // quad_perm(1,0,3,2) and (2,3,0,1) give every lane of a quad ((s0+s1)+(s2+s3)), then
    // row_half_mirror brings the other quad's sum (a commutative last add). With every head
    // present the guard-free form lets the eight chains interleave.
    float sc[HH];
    auto score = [&](int h) {
        const float *qh = qs + h * kDecThreads + sg * 32;
        float a = 0.0f;
#pragma unroll
        for (int i4 = 0; i4 < 8; ++i4) {
            const float4 qv = *reinterpret_cast<const float4 *>(qh + 4 * i4);
            const float4 kv = kq[i4];
            a = __fmaf_rn(qv.x, kv.x, a);
            a = __fmaf_rn(qv.y, kv.y, a);
            a = __fmaf_rn(qv.z, kv.z, a);
            a = __fmaf_rn(qv.w, kv.w, a);
        }
        return a;
    };
    if (heads == kAttnMaxHeads) {
#pragma unroll
        for (int hh = 0; hh < HH; ++hh) sc[hh] = score(half * HH + hh);
    } else {
#pragma unroll
        for (int hh = 0; hh < HH; ++hh) sc[hh] = half * HH + hh < heads ? score(half * HH + hh) : 0.0f;
    }
#pragma unroll
    for (int hh = 0; hh < HH; ++hh) {
        float a = __fadd_rn(sc[hh], dpp_f32_b1(sc[hh]));
        a = __fadd_rn(a, dpp_f32_4e(a));
        sc[hh] = __fadd_rn(a, dpp_f32_half_mirror(a));
    }
    if (sg == 0) {
#pragma unroll
        for (int hh = 0; hh < HH; ++hh) {
            const int h = half * HH + hh;
            if (h < heads) es[h * kAttnChunk + j] = j < cnt ? sc[hh] : -__int_as_float(0x7f800000);
        }
    }
    __syncthreads();
    if (KST) {
        // the chunk's V rows into the K copy's LDS (every thread read its K operands before the
        // barrier above), row-major: position u's 256 dims at u * 256 floats; a producer's last
        // chunk takes the position's new row from kvnew
        int jp = -1;
        if constexpr (PRO) jp = store_kv ? pos - start : -1;
#pragma unroll
        for (int i = 0; i < KPT; ++i) {
            const int r = wv + WAVES * i;
            float4 v = vl[i];
            if constexpr (PRO)
                if (r == jp) v = *reinterpret_cast<const float4 *>(kvnew + kDecThreads + 4 * lane);
            ks[r * (kDecThreads / 4) + lane] = v;
        }
    }

    // per head, uniform within its 32-lane group of half 0: max, exp, the pairwise sum
    const int hh = t >> 5, p = t & 31;
    if (half == 0 && hh < heads) {
        const float x = es[hh * kAttnChunk + p];
        float m = x;
        {  // the group's maximum, in every lane of the group
            const float mg = half_wave_max(m);
            const float m0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mg), 0));
            const float m1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mg), 32));
            m = (t & 32) ? m1 : m0;
        }
        const float e = p < cnt ? d_expf(__fsub_rn(x, m)) : 0.0f;
        float l = e;
        l = half_wave_tree_sum(l);  // lane p = 0 of each 32-lane group holds its head's sum
        es[hh * kAttnChunk + p] = e;
        if (p == 0) {
            const int64_t slot = (row * heads + hh) * max_chunks + c;
            part_ml[slot * 2] = m;
            part_ml[slot * 2 + 1] = l;
        }
    }
    __syncthreads();

    // o[h][d] = sum over positions (ascending) of e[h][j] * v[j][d] (one fused multiply-add each),
    // for this half's heads; a whole chunk with every head present takes the guard-free form, whose
    // chains interleave (each V value read once for all of them)
    const float *vsf = reinterpret_cast<const float *>(ks);
    auto vval = [&](int u) { return KST ? vsf[u * kDecThreads + t] : vv[u]; };
    if (heads == kAttnMaxHeads && cnt == kAttnChunk) {
        float o[HH];
#pragma unroll
        for (int g = 0; g < HH; ++g) o[g] = 0.0f;
#pragma unroll
        for (int u4 = 0; u4 < kAttnChunk; u4 += 4) {  // four weights per LDS read
            float v[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) v[i] = vval(u4 + i);
#pragma unroll
            for (int g = 0; g < HH; ++g) {
                const float4 e4 = *reinterpret_cast<const float4 *>(es + (half * HH + g) * kAttnChunk + u4);
                o[g] = __fmaf_rn(e4.x, v[0], o[g]);
                o[g] = __fmaf_rn(e4.y, v[1], o[g]);
                o[g] = __fmaf_rn(e4.z, v[2], o[g]);
                o[g] = __fmaf_rn(e4.w, v[3], o[g]);
            }
        }
#pragma unroll
        for (int g = 0; g < HH; ++g)
            part_o[((row * heads + half * HH + g) * max_chunks + c) * kDecThreads + t] = o[g];
    } else {
#pragma unroll
        for (int g = 0; g < HH; ++g) {
            const int h = half * HH + g;
            if (h >= heads) continue;
            float o = 0.0f;
#pragma unroll
            for (int u4 = 0; u4 < kAttnChunk; u4 += 4) {
                const float4 e4 = *reinterpret_cast<const float4 *>(es + h * kAttnChunk + u4);
                const float e[4] = {e4.x, e4.y, e4.z, e4.w};
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    if (u4 + i < cnt) o = __fmaf_rn(e[i], vval(u4 + i), o);
            }
            part_o[((row * heads + h) * max_chunks + c) * kDecThreads + t] = o;
        }
    }
}

// The split launch: two halves of four heads while the grid fits the CUs once; the chunk's K
// staged through LDS while the grid stays resident at that kernel's occupancy (its 44 KB of LDS
// allows three blocks per CU), else each lane loads its own K segment (11 KB, eight blocks per
// CU), which measured faster for grids of several rounds (E2B global layers at batch 32: 78.9
// against 85.3 us; with V staged through LDS as well, the whole batch-32 step 2.872 against
// 2.887 ms).
template <bool PRO>
static void launch_split(int chunks, int rows, hipStream_t st, const float *q, const float *k_cache,
                         const float *v_cache, int64_t cache_row_stride, int heads, int pos,
                         const int32_t *pos_dev, int window, float *part_ml, float *part_o,
                         const AttnPrologue &pro) {
    const int64_t blocks = (int64_t)chunks * rows, cus = device_cu_count();
    const dim3 grid(chunks, rows);
    if (blocks <= cus)
        hipLaunchKernelGGL((attn_split_kernel<PRO, 2, true>), grid, dim3(2 * kDecThreads), 0, st,
                           q, k_cache, v_cache, cache_row_stride, heads, pos, pos_dev, window,
                           part_ml, part_o, chunks, pro);
    else if (blocks <= 3 * cus)
        hipLaunchKernelGGL((attn_split_kernel<PRO, 1, true>), grid, dim3(kDecThreads), 0, st, q,
                           k_cache, v_cache, cache_row_stride, heads, pos, pos_dev, window, part_ml,
                           part_o, chunks, pro);
    else
        hipLaunchKernelGGL((attn_split_kernel<PRO, 1, false>), grid, dim3(kDecThreads), 0, st, q,
                           k_cache, v_cache, cache_row_stride, heads, pos, pos_dev, window, part_ml,
                           part_o, chunks, pro);
}

// Thread d merges dim d of head h, row `row`, over the chunks in ascending order: M = max m_c,
// w_c = exp(m_c - M) (once per chunk, staged in LDS), L = sum l_c w_c, O = sum o_c w_c,
// returns O / L. Every load that does not depend on M goes out first (the chunk's (m, l) pairs
// and the first kB partials of the thread's dim); M is a shuffle max in each wave and a max over
// the four waves (max is exact in any order). red: 4 floats, ws / ls: kDecThreads floats of LDS.
// Up to NB chunks (NB <= 256): every partial of the thread's dimension requested at once (indices
// clamped, so all valid), then the same ascending sum as the batched form below, so the same bits.
// The batched form waits one memory round trip per batch of 16 chunks (a 4096-position layer has
// 128): 1.290 -> 1.277 ms per batch-1 step. Staging the partials through LDS with 16-byte loads
// instead (a quarter of the load instructions, 146 KB of LDS per block) measured 1.69 ms.
template <int NB>
__device__ __forceinline__ float merge_head_dim_all(const float *part_ml, const float *part_o, int64_t slot0,
                                                    int chunks, float *red, float *ws, float *ls) {
    const int t = threadIdx.x;
    float oa[NB];
#pragma unroll
    for (int u = 0; u < NB; ++u) oa[u] = part_o[(slot0 + min(u, chunks - 1)) * kDecThreads + t];
    const float mt = t < chunks ? part_ml[(slot0 + t) * 2] : -__int_as_float(0x7f800000);
    const float lt = t < chunks ? part_ml[(slot0 + t) * 2 + 1] : 0.0f;
    const float m = wave_max(mt);  // lane 0 holds the wave's maximum
    if ((t & 63) == 0) red[t >> 6] = m;
    __syncthreads();
    const float M = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    if (t < chunks) {
        ws[t] = d_expf(__fsub_rn(mt, M));
        ls[t] = lt;
    }
    __syncthreads();
    float L = 0.0f, O = 0.0f;
#pragma unroll
    for (int u = 0; u < NB; ++u) {
        if (u < chunks) {
            L = __fadd_rn(L, __fmul_rn(ls[u], ws[u]));
            O = __fadd_rn(O, __fmul_rn(oa[u], ws[u]));
        }
    }
    __syncthreads();
    return __fdiv_rn(O, L);
}

__device__ __forceinline__ float merge_head_dim(const float *part_ml, const float *part_o, int heads,
                                                int h, int64_t row, int pos, int window,
                                                int max_chunks, float *red, float *ws, float *ls) {
    constexpr int kB = 16;  // partials loaded together (indices clamped, so all valid)
    const int t = threadIdx.x;
    const int lo = window > 0 ? max(0, pos - window + 1) : 0;
    const int chunks = (pos - lo + 1 + kAttnChunk - 1) / kAttnChunk;
    const int64_t slot0 = (row * heads + h) * max_chunks;
    if (chunks <= 16) return merge_head_dim_all<16>(part_ml, part_o, slot0, chunks, red, ws, ls);
    if (chunks <= 32) return merge_head_dim_all<32>(part_ml, part_o, slot0, chunks, red, ws, ls);
    if (chunks <= 64) return merge_head_dim_all<64>(part_ml, part_o, slot0, chunks, red, ws, ls);
    if (chunks <= 128) return merge_head_dim_all<128>(part_ml, part_o, slot0, chunks, red, ws, ls);
    float oo[kB];
#pragma unroll
    for (int u = 0; u < kB; ++u) oo[u] = part_o[(slot0 + min(u, chunks - 1)) * kDecThreads + t];
    float m = -__int_as_float(0x7f800000), lt = 0.0f;
    for (int c = t; c < chunks; c += kDecThreads) m = fmaxf(m, part_ml[(slot0 + c) * 2]);
    if (t < chunks) lt = part_ml[(slot0 + t) * 2 + 1];
    m = wave_max(m);  // lane 0 holds the wave's maximum
    if ((t & 63) == 0) red[t >> 6] = m;
    __syncthreads();
    const float M = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    // The partials of chunk batch u0 + kB are requested while batch u0 is summed (two register
    // buffers), and a whole batch is summed without per-chunk guards; the order stays ascending.
    float L = 0.0f, O = 0.0f;
    float ob[kB];
    auto load = [&](float (&dst)[kB], int c0, int u0, int n) {
#pragma unroll
        for (int u = 0; u < kB; ++u) dst[u] = part_o[(slot0 + c0 + min(u0 + u, n - 1)) * kDecThreads + t];
    };
    auto accumulate = [&](const float (&src)[kB], int u0, int n) {
        if (u0 + kB <= n) {
#pragma unroll
            for (int u = 0; u < kB; ++u) {
                L = __fadd_rn(L, __fmul_rn(ls[u0 + u], ws[u0 + u]));
                O = __fadd_rn(O, __fmul_rn(src[u], ws[u0 + u]));
            }
        } else {
#pragma unroll
            for (int u = 0; u < kB; ++u) {
                if (u0 + u < n) {
                    L = __fadd_rn(L, __fmul_rn(ls[u0 + u], ws[u0 + u]));
                    O = __fadd_rn(O, __fmul_rn(src[u], ws[u0 + u]));
                }
            }
        }
    };
    for (int c0 = 0; c0 < chunks; c0 += kDecThreads) {
        const int n = min(kDecThreads, chunks - c0);
        if (t < n) {
            ws[t] = d_expf(__fsub_rn(part_ml[(slot0 + c0 + t) * 2], M));
            ls[t] = c0 == 0 ? lt : part_ml[(slot0 + c0 + t) * 2 + 1];
        }
        __syncthreads();
        if (c0 > 0) load(oo, c0, 0, n);
        for (int u0 = 0; u0 < n; u0 += 2 * kB) {
            if (u0 + kB < n) load(ob, c0, u0 + kB, n);
            accumulate(oo, u0, n);
            if (u0 + kB < n) {
                if (u0 + 2 * kB < n) load(oo, c0, u0 + 2 * kB, n);
                accumulate(ob, u0 + kB, n);
            }
        }
        __syncthreads();
    }
    return __fdiv_rn(O, L);
}

// Grid (heads, rows): the merged attention row of head h, then the o_proj input snap.
__global__ __launch_bounds__(kDecThreads) void attn_merge_kernel(
    const float *part_ml, const float *part_o, int heads, int pos_host, const int32_t *pos_dev,
    int window, int max_chunks, float in_scale, int8_t *codes, float *out_f32) {
    __shared__ float red[kDecThreads / 64];
    __shared__ float ws[kDecThreads];
    __shared__ float ls[kDecThreads];
    const int t = threadIdx.x, h = blockIdx.x;
    const int64_t row = blockIdx.y;
    const float y = merge_head_dim(part_ml, part_o, heads, h, row, step_pos(pos_host, pos_dev), window,
                                   max_chunks, red, ws, ls);
    const int64_t o = (row * heads + h) * kDecThreads + t;
    if (out_f32) out_f32[o] = y;
    if (codes) codes[o] = snap_code(y, in_scale);
}

// The merge with o_proj folded in (one decode row): grid (heads, n / kMergeRows). Block (h, g)
// merges head h (the merge kernel's arithmetic, so the same codes), snaps it on o_proj's inScale
// into LDS, and contracts those 256 codes with the 128-byte slices of o_proj's 4-bit rows
// g * kMergeRows .. + kMergeRows that head h's columns occupy: the exact int32 accumulator of
// o_proj row n over K range 256 h .. 256 h + 255 (zero point included), added atomically into
// acc[n] (zeroed by the split kernel before). Integer addition is exact in any order, so acc[n]
// is o_proj's accumulator and a consumer that applies o_proj's epilogue to it (acc_value) reads
// o_proj's codes bit for bit. The weight slices are requested before the merge, so their memory
// latency overlaps it. Eight lanes share a row: lane t reads the row's 16-byte chunk t % 8, then
// a three-step xor sum.
// sum(u * x) over one 16-byte word group of 32 packed 4-bit codes u (unsigned nibbles, low first)
// and their 32 activation codes x in the snap layout: the low and high nibbles each dot one half.
__device__ __forceinline__ int chunk_dot4(const u32x4 &w, const uint8_t *x) {
    const u32x4 xa = *reinterpret_cast<const u32x4 *>(x);
    const u32x4 xb = *reinterpret_cast<const u32x4 *>(x + 16);
    const uint32_t wv[4] = {w.x, w.y, w.z, w.w};
    const uint32_t xv[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
    int acc = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        acc = __builtin_amdgcn_sdot4((int)(wv[i] & 0x0F0F0F0Fu), (int)xv[2 * i], acc, false);
        acc = __builtin_amdgcn_sdot4((int)((wv[i] >> 4) & 0x0F0F0F0Fu), (int)xv[2 * i + 1], acc, false);
    }
    return acc;
}

constexpr int kMergeRows = 64;
__global__ __launch_bounds__(kDecThreads) void attn_merge_o_kernel(
    const float *part_ml, const float *part_o, int heads, int pos_host, const int32_t *pos_dev,
    int window, int max_chunks, float in_scale, int8_t *codes, const uint8_t *w, int n_out,
    int k_total, int32_t *part) {
    constexpr int kPasses = kMergeRows / (kDecThreads / 8);
    __shared__ float red[kDecThreads / 64];
    __shared__ float ws[kDecThreads];
    __shared__ float ls[kDecThreads];
    __shared__ __align__(16) uint8_t xs[kDecThreads];
    __shared__ int csum[kDecThreads / 64];
    const int t = threadIdx.x, h = blockIdx.x;
    const int row0 = blockIdx.y * kMergeRows;
    const int64_t row_bytes = k_total >> 1;
    u32x4 wv[kPasses];
#pragma unroll
    for (int p = 0; p < kPasses; ++p) {
        const int r = min(row0 + p * (kDecThreads / 8) + (t >> 3), n_out - 1);
        wv[p] = __builtin_nontemporal_load(
            reinterpret_cast<const u32x4 *>(w + r * row_bytes + h * (kDecThreads / 2) + (t & 7) * 16));
    }
    const float y = merge_head_dim(part_ml, part_o, heads, h, 0, step_pos(pos_host, pos_dev), window,
                                   max_chunks, red, ws, ls);
    const int c = srq_code_i(y, in_scale);
    if (blockIdx.y == 0 && codes) codes[h * kDecThreads + t] = (int8_t)c;
    // codes in the 4-bit snap layout: each 8-code group as [x0 x2 x4 x6 | x1 x3 x5 x7]
    const int j = t & 7;
    xs[(t & ~7) + (j & 1 ? 4 : 0) + (j >> 1)] = (uint8_t)c;
    const int s = wave_sum_i32_first(c);  // lane 0: the wave's code sum
    if ((t & 63) == 0) csum[t >> 6] = s;
    __syncthreads();
    const int xsum = csum[0] + csum[1] + csum[2] + csum[3];
#pragma unroll
    for (int p = 0; p < kPasses; ++p) {
        int acc = chunk_dot4(wv[p], xs + (t & 7) * 32);
        acc += __shfl_xor(acc, 1);
        acc += __shfl_xor(acc, 2);
        acc += __shfl_xor(acc, 4);
        const int r = row0 + p * (kDecThreads / 8) + (t >> 3);
        if ((t & 7) == 0 && r < n_out) atomicAdd(part + r, acc - 8 * xsum);
    }
}

// ---- the per-layer-input block at one decode row: join, gate, gelu x row, projection ------------

// per_layer_input_gate and per_layer_projection in one launch (the decode runner at batch 1):
// block b runs the post-FFN join that produces the gate's input codes (every block, the join
// kernel's arithmetic; block 0 also stores the join's residual row), the gate rows
// b * kPleRows .. + kPleRows (8-bit, exact int32 dot, the GEMV epilogue, then the gelu epilogue
// with the layer's per-layer row: the codes the gate plan would store), and contracts those
// kPleRows codes with the matching 16 columns of the 8-bit projection: the projection's exact
// int32 accumulator over that K range, added atomically into acc[n] (zeroed by the split kernel
// before). The weight loads of both go out right behind the join's operand loads, so their memory
// latency overlaps the join's arithmetic.
constexpr int kPleRows = 4;
// The projection's kPleRows int8 weights of a row (and the block's kPleRows codes) as one word.
template <int ROWS> struct PleWord;
template <> struct PleWord<4> { typedef uint32_t type; };
template <> struct PleWord<8> { typedef unsigned int type __attribute__((ext_vector_type(2))); };
__device__ __forceinline__ int ple_dot(uint32_t w, uint32_t a) { return __builtin_amdgcn_sdot4((int)w, (int)a, 0, false); }
__device__ __forceinline__ int ple_dot(PleWord<8>::type w, PleWord<8>::type a) {
    return __builtin_amdgcn_sdot4((int)w.y, (int)a.y, __builtin_amdgcn_sdot4((int)w.x, (int)a.x, 0, false), false);
}

// PER: join elements per thread (hidden <= PER * 256).
template <int ROWS, int PER>
__global__ __launch_bounds__(kDecThreads) void ple_block_kernel(PleFold F) {
    extern __shared__ __align__(16) uint8_t dyn[];
    constexpr int kGateLanes = kDecThreads / ROWS;  // lanes per gate row (32 or 64)
    static_assert(kGateLanes == 32 || kGateLanes == 64, "a gate row is half a wave or a wave");
    typedef typename PleWord<ROWS>::type PW;
    const int t = threadIdx.x;
    const int r0 = blockIdx.x * ROWS;
    const int H = F.join.width;
    uint8_t *xs = dyn;                                               // H codes, natural order
    float *red = reinterpret_cast<float *>(dyn + ((H + 15) & ~15));  // 512 floats
    __shared__ __align__(16) int8_t act[16];
    // gate row r0 + t / kGateLanes: this lane's 16-byte chunks c = t % kGateLanes, c + kGateLanes, ...
    constexpr int kGateChunks = kJoinMaxPer * kDecThreads / 16 / kGateLanes;  // chunks per lane, max
    const int gchunks = H / 16;                                                  // chunks per row
    const int grow = r0 + t / kGateLanes, glane = t % kGateLanes;
    u32x4 gw[kGateChunks];
    float gscale, up;
    // projection rows n = t + 256 i: the ROWS bytes of columns r0 .. r0 + ROWS - 1
    PW pw[PER];
    // the weights, requested behind the join's own operands
    auto load_weights = [&]() {
#pragma unroll
        for (int u = 0; u < kGateChunks; ++u)
            gw[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(
                F.w_gate + (int64_t)grow * H + min(glane + u * kGateLanes, gchunks - 1) * 16));
        gscale = F.s_gate[grow];
        up = F.up_vec[grow];
#pragma unroll
        for (int i = 0; i < PER; ++i)
            pw[i] = __builtin_nontemporal_load(reinterpret_cast<const PW *>(
                F.w_proj + (int64_t)min(t + i * kDecThreads, H - 1) * F.p + r0));
        __builtin_amdgcn_sched_barrier(0);
    };
    JoinTail J = F.join;  // J.codes stays set: the join emits codes only when it has a destination
    if (blockIdx.x != 0) J.hidden = nullptr;
    auto emit = [&](int i, int8_t c) { xs[i] = (uint8_t)c; };  // the codes stay in this block's LDS
    // an int32 source: down's accumulator, possibly in several copies (the FFN block's)
    // the general join form: the no-second-gain form (no load, no test of that operand) measured
    // 1.253 -> 1.306 ms per batch-1 step here, with the same arithmetic
    if (J.src_kind == G4_KIND_I32) rms_join_row_emit<kSplitAccMax, PER>(J, 0, red, emit, load_weights);
    else rms_join_row_emit<0, PER>(J, 0, red, emit, load_weights);
    __syncthreads();
    int acc = 0;
#pragma unroll
    for (int u = 0; u < kGateChunks; ++u) {
        const int c = glane + u * kGateLanes;
        if (c < gchunks) {
            const u32x4 xa = *reinterpret_cast<const u32x4 *>(xs + c * 16);
            acc = __builtin_amdgcn_sdot4((int)gw[u].x, (int)xa.x, acc, false);
            acc = __builtin_amdgcn_sdot4((int)gw[u].y, (int)xa.y, acc, false);
            acc = __builtin_amdgcn_sdot4((int)gw[u].z, (int)xa.z, acc, false);
            acc = __builtin_amdgcn_sdot4((int)gw[u].w, (int)xa.w, acc, false);
        }
    }
    acc = row16_sum_i32(acc);
    acc += __shfl_xor(acc, 16);
    if (kGateLanes == 64) acc += __shfl_xor(acc, 32);
    if (glane == 0) {
        // the gate plan's epilogue: GEMV output code on out_scale, gelu, times the row, snap
        const float y = linear_epilogue(F.in_scale, gscale, (float)acc);
        const float g = __fmul_rn(srq_code_f(y, F.out_scale), F.out_scale);
        act[t / kGateLanes] = (int8_t)srq_code_i(__fmul_rn(d_gelu(g), up), F.in_scale);
    }
    __syncthreads();
    const PW a = *reinterpret_cast<const PW *>(act);
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        const int n = t + i * kDecThreads;
        if (n >= H) break;
        atomicAdd(F.acc + n, ple_dot(pw[i], a));
    }
}

bool ple_fold_fits(const PleFold &F) {
    const int H = F.join.width;
    return F.join.codes && F.w_gate && F.s_gate && F.up_vec && F.w_proj && F.acc && H > 0 && H % 16 == 0 &&
           H <= kJoinMaxPer * kDecThreads && F.p > 0 && F.p % kPleRows == 0 &&
           (reinterpret_cast<uintptr_t>(F.w_gate) & 15) == 0 && (reinterpret_cast<uintptr_t>(F.w_proj) & 15) == 0 &&
           F.in_scale != 0.0f && F.out_scale != 0.0f;
}

int ple_block(const PleFold &F, void *stream) {
    if (!ple_fold_fits(F)) return set_error(G4_ERR_INVALID, "per-layer-input block: shape or operands do not fit");
    const size_t lds = ((F.join.width + 15) & ~15) + 2 * kRowThreads * sizeof(float);
    if (F.join.width <= 6 * kDecThreads)
        hipLaunchKernelGGL((ple_block_kernel<kPleRows, 6>), dim3(F.p / kPleRows), dim3(kDecThreads), lds,
                           as_stream(stream), F);
    else
        hipLaunchKernelGGL((ple_block_kernel<kPleRows, kJoinMaxPer>), dim3(F.p / kPleRows), dim3(kDecThreads),
                           lds, as_stream(stream), F);
    G4_LAUNCHED("ple_block_kernel");
    return G4_OK;
}

// ---- the FFN block at one decode row: join, gate and up, gelu-mul, down's K range ---------------

// gate_proj, up_proj, the gelu-mul pass and down_proj in one launch (the decode runner at batch 1):
// block b runs the post-attention join that produces the gate / up input codes (every block, the
// join kernel's arithmetic; block 0 also stores the join's residual row), the gate and up rows
// b * R .. + R (4-bit, exact int32 dots, each linear's epilogue and output snap, then the gelu-mul
// pass: the codes down_proj would read), and contracts those R codes with the matching R columns
// of every down_proj row: down's exact int32 accumulator over that K range, added atomically into
// acc[n] (zeroed by the split kernel before). The weight loads go out right behind the join's
// operand loads, so the join waits for its own operands only and the weights stream in under its
// arithmetic. H = 512 * CPL: a gate / up row is 16 lanes x CPL 16-byte chunks (2R rows, 16 per
// pass), and each thread takes 2 * CPL down rows (R / 2 bytes each, consecutive threads consecutive
// rows of the block's repacked run).

template <int R, int CPL>
__global__ __launch_bounds__(kDecThreads) void ffn_block_kernel(FfnFold F) {
    extern __shared__ __align__(16) uint8_t dyn[];
    constexpr int kPasses = 2 * R / 16;   // gate rows, then up rows, 16 a pass
    constexpr int kDownRows = 2 * CPL;    // down rows per thread: H / 256
    constexpr int kDownChunks = R / 32;   // 16-byte chunks of a down row in this K range
    static_assert(R % 32 == 0 && R <= 64, "a block's K range of down is whole 16-byte chunks, one wave's lanes");
    const int t = threadIdx.x, lr = t & 15;
    const int H = F.join.width;
    const int r0 = blockIdx.x * R;
    uint8_t *xs = dyn;                                               // H codes, snap layout
    float *red = reinterpret_cast<float *>(dyn + ((H + 15) & ~15));  // 512 floats
    __shared__ int accs[2 * R];
    __shared__ __align__(16) uint8_t act[R];
    __shared__ int sums[2];
    const int64_t row_bytes = H / 2;
    u32x4 gw[kPasses][CPL];
    u32x4 dw[kDownRows][kDownChunks];
    float sg, su;
    // the weights and scales, requested behind the join's own operands
    auto load_weights = [&]() {
#pragma unroll
        for (int p = 0; p < kPasses; ++p) {
            const bool gate = p < R / 16;
            const int row = r0 + (gate ? p : p - R / 16) * 16 + (t >> 4);
            const uint8_t *w = (gate ? F.w_gate : F.w_up) + (int64_t)row * row_bytes + lr * 16;
#pragma unroll
            for (int u = 0; u < CPL; ++u)
                gw[p][u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(w + u * 256));
        }
        const uint8_t *wd = F.w_down + (int64_t)blockIdx.x * H * (R / 2);
#pragma unroll
        for (int i = 0; i < kDownRows; ++i)
#pragma unroll
            for (int c = 0; c < kDownChunks; ++c)
                dw[i][c] = __builtin_nontemporal_load(
                    reinterpret_cast<const u32x4 *>(wd + (int64_t)(t + i * kDecThreads) * (R / 2) + c * 16));
        sg = F.s_gate[r0 + (t & (R - 1))];
        su = F.s_up[r0 + (t & (R - 1))];
        __builtin_amdgcn_sched_barrier(0);  // all of them before the join's arithmetic
    };
    if (t == 0) sums[0] = 0;
    JoinTail J = F.join;  // J.codes stays set: the join emits codes only when it has a destination
    if (blockIdx.x != 0) J.hidden = nullptr;
    int local = 0;
    auto emit = [&](int i, int8_t c) {  // the codes stay in this block's LDS, in the snap layout
        const int j = i & 7;
        xs[(i & ~7) + (j & 1 ? 4 : 0) + (j >> 1)] = (uint8_t)c;
        local += c;
    };
    if (J.src_kind == G4_KIND_I32) rms_join_row_emit<1, 2 * CPL>(J, 0, red, emit, load_weights);
    else rms_join_row_emit<0, 2 * CPL>(J, 0, red, emit, load_weights);
    local = row16_sum_i32(local);
    if (lr == 0 && local != 0) atomicAdd(&sums[0], local);
    __syncthreads();
    const int sx = sums[0];
#pragma unroll
    for (int p = 0; p < kPasses; ++p) {
        int acc = 0;
#pragma unroll
        for (int u = 0; u < CPL; ++u) acc += chunk_dot4(gw[p][u], xs + (lr + 16 * u) * 32);
        acc = row16_sum_i32(acc);
        if (lr == 0) accs[p * 16 + (t >> 4)] = acc - 8 * sx;
    }
    __syncthreads();
    if (t < 64) {
        // the paired tile's gelu epilogue: gate and up each through their linear's epilogue and
        // output snap, then srq(gelu(gate) * up) on act_scale
        int a = 0;
        if (t < R) {
            const float yg = linear_epilogue(F.in_scale, sg, (float)accs[t]);
            const float yu = linear_epilogue(F.in_scale, su, (float)accs[R + t]);
            const float g = __fmul_rn(srq_code_f(yg, F.out_scale), F.out_scale);
            const float u = __fmul_rn(srq_code_f(yu, F.out_scale), F.out_scale);
            a = srq_code_i(__fmul_rn(d_gelu(g), u), F.act_scale);
            const int j = t & 7;
            act[(t & ~7) + (j & 1 ? 4 : 0) + (j >> 1)] = (uint8_t)a;
        }
        a = wave_sum_i32_first(a);  // lane 0: the block's code sum
        if (t == 0) sums[1] = a;
    }
    __syncthreads();
    const int sa = sums[1];
    int32_t *dacc = F.acc + (int64_t)(blockIdx.x % F.acc_copies) * H;
#pragma unroll
    for (int i = 0; i < kDownRows; ++i) {
        int acc = 0;
#pragma unroll
        for (int c = 0; c < kDownChunks; ++c) acc += chunk_dot4(dw[i][c], act + c * 32);
        atomicAdd(dacc + t + i * kDecThreads, acc - 8 * sa);
    }
}

bool ffn_fold_fits(const FfnFold &F) {
    const int H = F.join.width;
    auto a16 = [](const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
    return F.join.codes && F.w_gate && F.w_up && F.s_gate && F.s_up && F.w_down && F.acc &&
           F.acc_copies >= 1 && F.acc_copies <= kSplitAccMax && H > 0 &&
           H % 512 == 0 && H <= kJoinMaxPer * kDecThreads && F.f > 0 && F.f % kFfnRows == 0 &&
           F.f % 32 == 0 && a16(F.w_gate) && a16(F.w_up) && a16(F.w_down) && F.in_scale != 0.0f &&
           F.out_scale != 0.0f && F.act_scale != 0.0f;
}

// One 16-byte piece per thread: piece i of the output is (K range kr, row n, piece c of the run).
__global__ __launch_bounds__(256) void ffn_repack_kernel(const uint8_t *w, uint8_t *out, int h, int f) {
    constexpr int kPieces = kFfnRows / 32;
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (int64_t)(f / kFfnRows) * h * kPieces) return;
    const int c = (int)(i % kPieces);
    const int64_t n = (i / kPieces) % h, kr = i / ((int64_t)kPieces * h);
    *reinterpret_cast<u32x4 *>(out + i * 16) =
        *reinterpret_cast<const u32x4 *>(w + n * (f / 2) + kr * (kFfnRows / 2) + c * 16);
}

int ffn_repack_down(const uint8_t *w, uint8_t *out, int h, int f, hipStream_t stream) {
    if (!w || !out || h <= 0 || f <= 0 || f % kFfnRows != 0 || (reinterpret_cast<uintptr_t>(w) & 15) ||
        (reinterpret_cast<uintptr_t>(out) & 15))
        return set_error(G4_ERR_INVALID, "FFN block: down_proj repack operands do not fit");
    const int64_t pieces = (int64_t)(f / kFfnRows) * h * (kFfnRows / 32);
    hipLaunchKernelGGL(ffn_repack_kernel, dim3((unsigned)((pieces + 255) / 256)), dim3(256), 0, stream, w, out, h, f);
    G4_LAUNCHED("ffn_repack_kernel");
    return G4_OK;
}

int ffn_block(const FfnFold &F, void *stream) {
    if (!ffn_fold_fits(F)) return set_error(G4_ERR_INVALID, "FFN block: shape or operands do not fit");
    const size_t lds = ((F.join.width + 15) & ~15) + 2 * kRowThreads * sizeof(float);
    const dim3 grid(F.f / kFfnRows), block(kDecThreads);
    hipStream_t s = as_stream(stream);
    switch (F.join.width / 512) {
    case 1: hipLaunchKernelGGL((ffn_block_kernel<kFfnRows, 1>), grid, block, lds, s, F); break;
    case 2: hipLaunchKernelGGL((ffn_block_kernel<kFfnRows, 2>), grid, block, lds, s, F); break;
    case 3: hipLaunchKernelGGL((ffn_block_kernel<kFfnRows, 3>), grid, block, lds, s, F); break;
    default: hipLaunchKernelGGL((ffn_block_kernel<kFfnRows, 4>), grid, block, lds, s, F); break;
    }
    G4_LAUNCHED("ffn_block_kernel");
    return G4_OK;
}

// ---- gelu * up with the consumer's snap ------------------------------------------------------------

// rows x n: codes = srq(gelu(g * gs) * u, in_scale) with u = up codes * us, or (up_f32 given) the
// f32 value at up_f32[row * up_stride + i] (the per-layer-input form).
__global__ void gelu_mul_kernel(const int8_t *g, float gs, const int8_t *u, float us,
                                const float *up_f32, int64_t up_stride, int n, float in_scale,
                                int8_t *codes) {
    const int64_t row = blockIdx.y;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) {
        const float gv = __fmul_rn((float)g[row * n + i], gs);
        const float uv = up_f32 ? up_f32[row * up_stride + i] : __fmul_rn((float)u[row * n + i], us);
        codes[row * n + i] = snap_code(__fmul_rn(d_gelu(gv), uv), in_scale);
    }
}

// gelu-mul on the reference's f32 buffers (geluMul.ts:101-116 and its main, 4 elements per vec4
// lane): dst = gelu_tanh(gate) * up, then q * s with q = srq(v, s) when s != 0.
__global__ void gelu_mul_f32_kernel(const float4 *g, const float4 *u, float4 *dst, int64_t n4,
                                    float srq_scale) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4;
         i += (int64_t)gridDim.x * blockDim.x) {
        const float4 a = g[i], b = u[i];
        float v[4] = {__fmul_rn(d_gelu(a.x), b.x), __fmul_rn(d_gelu(a.y), b.y),
                      __fmul_rn(d_gelu(a.z), b.z), __fmul_rn(d_gelu(a.w), b.w)};
        if (srq_scale != 0.0f) {
#pragma unroll
            for (int j = 0; j < 4; ++j) v[j] = __fmul_rn(srq_code_f(v[j], srq_scale), srq_scale);
        }
        dst[i] = make_float4(v[0], v[1], v[2], v[3]);
    }
}

// ---- the token embedding (tied int4 table) -----------------------------------------------------------

// One block per row: x = (code - 8) * f32(scale[id] * embed_scale); also the codes of x snapped on
// in_scale (the input of the per-layer model projection). An id outside [0, vocab) (argmax's -1
// over an all-NaN row, or a caller's bad token) reads nothing and gives a zero row.
__global__ __launch_bounds__(kDecThreads) void embed_kernel(
    const uint8_t *table, const float *row_scales, const int32_t *ids, int64_t vocab, int cols,
    float embed_scale, float in_scale, float *x, int8_t *codes) {
    const int64_t row = blockIdx.x;
    const int64_t id = ids[row];
    if (id < 0 || id >= vocab) {
        for (int i = threadIdx.x; i < cols; i += kDecThreads) {
            x[row * cols + i] = 0.0f;
            if (codes) codes[row * cols + i] = 0;
        }
        return;
    }
    const float s = __fmul_rn(row_scales[id], embed_scale);
    const uint8_t *src = table + id * (int64_t)(cols / 2);
    for (int i = threadIdx.x; i < cols; i += kDecThreads) {
        const int code = (int)((src[i >> 1] >> (4 * (i & 1))) & 0xF) - 8;
        const float v = __fmul_rn((float)code, s);
        x[row * cols + i] = v;
        if (codes) codes[row * cols + i] = snap_code(v, in_scale);
    }
}

// ---- per-layer inputs: projection norm, add the gathered identity, scale by 2^-0.5 -----------------

// Grid (groups, rows), 256 threads = one group of 256.
__global__ __launch_bounds__(kDecThreads) void ple_combine_kernel(
    const int8_t *proj_codes, float proj_scale, float alpha, const float *gain,
    const float *identity, int groups, float eps, float *out) {
    __shared__ float lds[kDecThreads];
    const int t = threadIdx.x;
    const int64_t o = ((int64_t)blockIdx.y * groups + blockIdx.x) * kDecThreads + t;
    const float x = __fmul_rn(__fmul_rn((float)proj_codes[o], proj_scale), alpha);
    const float gt = gain[t], id = identity[o];  // loaded before the barriers
    const float inv = inv_rms(block_tree_sum(__fmul_rn(x, x), lds), kDecThreads, eps);
    const float y = __fmul_rn(__fmul_rn(x, inv), gt);
    out[o] = __fmul_rn(__fadd_rn(y, id), 0x1.6a09e6p-1f);
}

// ---- logit softcap and the two-stage argmax ------------------------------------------------------

// logits per partial block: 1024 spreads a 262144-row head over 256 blocks, every CU, for the
// softcap's divide and tanh (4096 gave 64 blocks). With the logits requested up front, the step
// went 1.246 -> 1.239 ms at batch 1 and 2.836 -> 2.823 ms at batch 32. The winner is the largest
// value, ties to the lower index, whatever the span.
constexpr int kArgmaxSpan = 1024;

// argmax.ts:267-300's strict rule: a value wins only above the best so far, starting from -inf,
// so -inf and NaN never win and an empty winner stays (-inf, -1). Equal values above -inf (two
// partial winners) resolve to the lower index.
__device__ __forceinline__ void better(float &bv, int &bi, float v, int i) {
    if (v > bv || (v == bv && v > -__int_as_float(0x7f800000) && (unsigned)i < (unsigned)bi)) {
        bv = v;
        bi = i;
    }
}

// Grid (ceil(vocab / kArgmaxSpan), rows). capped = tanh(x / cap) * cap (cap 0: x), optionally stored;
// each block leaves its first strict maximum (value, index).
__global__ __launch_bounds__(kDecThreads) void softcap_argmax_partial_kernel(
    const float *logits, int64_t vocab, float cap, float *capped, float *part_v, int *part_i) {
    __shared__ float sv[kDecThreads];
    __shared__ int si[kDecThreads];
    const int t = threadIdx.x;
    const int64_t row = blockIdx.y;
    const int64_t b0 = (int64_t)blockIdx.x * kArgmaxSpan;
    float bv = -__int_as_float(0x7f800000);
    int bi = -1;
    // every logit of the thread requested first (indices clamped into the row), then the same
    // ascending sequence of softcaps and comparisons: a load per iteration waited a memory round
    // trip each (14 us per batch-1 step for 1 MB)
    constexpr int PT = kArgmaxSpan / kDecThreads;
    static_assert(PT * kDecThreads == kArgmaxSpan, "a block's span is whole passes of its threads");
    const int64_t end = min(b0 + kArgmaxSpan, vocab);
    float xs[PT];
#pragma unroll
    for (int k = 0; k < PT; ++k) xs[k] = logits[row * vocab + min(b0 + t + k * kDecThreads, vocab - 1)];
#pragma unroll
    for (int k = 0; k < PT; ++k) {
        const int64_t i = b0 + t + k * kDecThreads;
        if (i >= end) break;
        const float x = xs[k];
        const float y = cap != 0.0f ? __fmul_rn(d_tanhf(__fdiv_rn(x, cap)), cap) : x;
        if (capped) capped[row * vocab + i] = y;
        better(bv, bi, y, (int)i);
    }
    sv[t] = bv;
    si[t] = bi;
    __syncthreads();
    for (int stride = kDecThreads / 2; stride >= 1; stride >>= 1) {
        if (t < stride) {
            float v = sv[t];
            int i = si[t];
            better(v, i, sv[t + stride], si[t + stride]);
            sv[t] = v;
            si[t] = i;
        }
        __syncthreads();
    }
    if (t == 0) {
        part_v[row * gridDim.x + blockIdx.x] = sv[0];
        part_i[row * gridDim.x + blockIdx.x] = si[0];
    }
}

// One block per row over its `parts` partials: the winning index goes to tokens[row].
__global__ __launch_bounds__(64) void argmax_final_kernel(const float *part_v, const int *part_i,
                                                          int parts, int32_t *tokens) {
    __shared__ float sv[64];
    __shared__ int si[64];
    const int t = threadIdx.x;
    const int64_t row = blockIdx.x;
    float bv = -__int_as_float(0x7f800000);
    int bi = -1;
    for (int p = t; p < parts; p += 64) better(bv, bi, part_v[row * parts + p], part_i[row * parts + p]);
    sv[t] = bv;
    si[t] = bi;
    __syncthreads();
    for (int stride = 32; stride >= 1; stride >>= 1) {
        if (t < stride) {
            float v = sv[t];
            int i = si[t];
            better(v, i, sv[t + stride], si[t + stride]);
            sv[t] = v;
            si[t] = i;
        }
        __syncthreads();
    }
    if (t == 0) tokens[row] = si[0];
}

// ---- seeded fills (synthetic KV histories without a host round trip) ------------------------------

__device__ __forceinline__ uint64_t splitmix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

// out[i] = lo + u * span with u = (splitmix64(seed + i) >> 40) * 2^-24, in [0, 1); each step one
// f32 rounding. The same stream in numpy reproduces it bit for bit.
__global__ void fill_hash_f32_kernel(float *out, int64_t n, uint64_t seed, float lo, float span) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x) {
        const float u = (float)(splitmix64(seed + (uint64_t)i) >> 40) * 0x1p-24f;
        out[i] = __fadd_rn(lo, __fmul_rn(u, span));
    }
}

// out[i] = the top byte of splitmix64(seed + i): uniform int4 pairs or int8 codes.
__global__ void fill_hash_u8_kernel(uint8_t *out, int64_t n, uint64_t seed) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x)
        out[i] = (uint8_t)(splitmix64(seed + (uint64_t)i) >> 56);
}

}  // namespace g4


using namespace g4;

static int grid_1d(int64_t n, int threads) {
    int64_t b = (n + threads - 1) / threads;
    return (int)(b < 1 ? 1 : (b > 65536 ? 65536 : b));
}

static int attn_chunks(int pos, int window) {
    const int lo = window > 0 ? (pos - window + 1 > 0 ? pos - window + 1 : 0) : 0;
    return (pos - lo + 1 + kAttnChunk - 1) / kAttnChunk;
}

namespace g4 {

int attention_decode_fused(const AttnPrologue &pro, float *k_cache, float *v_cache,
                           int64_t cache_row_stride, int rows, int heads, int pos,
                           const int32_t *pos_dev, int window, float *workspace,
                           size_t workspace_bytes, float in_scale, int8_t *codes, void *stream,
                           const MergeLinear *lin) {
    if (!pro.q_codes || !pro.q_gain || !pro.cos_tab || !pro.sin_tab || !k_cache || !v_cache ||
        !workspace || !codes || rows <= 0 || heads <= 0 || heads > kAttnMaxHeads || pos < 0 ||
        window < 0 || in_scale == 0.0f)
        return set_error(G4_ERR_INVALID, "attention (fused prologue): bad arguments");
    if (pro.k_codes && (!pro.v_codes || !pro.k_gain))
        return set_error(G4_ERR_INVALID, "attention (fused prologue): k without v or k gain");
    // the prologue reads each 256-code vector as one 4-byte word per lane
    if (((uintptr_t)pro.q_codes | (uintptr_t)pro.k_codes | (uintptr_t)pro.v_codes) & 3)
        return set_error(G4_ERR_INVALID, "attention (fused prologue): code rows not 4-byte aligned");
    const int chunks = attn_chunks(pos, window);
    if (workspace_bytes < g4_attention_workspace_bytes(rows, heads, pos, window))
        return set_error(G4_ERR_INVALID, "attention (fused prologue): workspace too small");
    float *part_ml = workspace;
    float *part_o = workspace + (size_t)rows * heads * chunks * 2;
    launch_split<true>(chunks, rows, as_stream(stream), nullptr, k_cache, v_cache,
                                cache_row_stride, heads, pos, pos_dev, window, part_ml, part_o, pro);
    G4_LAUNCHED("attn_split_kernel");
    if (lin) {
        if (!merge_linear_fits(*lin, rows, heads))
            return set_error(G4_ERR_INVALID, "attention (fused prologue): the folded o_proj does not fit");
        hipLaunchKernelGGL(attn_merge_o_kernel, dim3(heads, lin->n / kMergeRows), dim3(kDecThreads), 0,
                           as_stream(stream), part_ml, part_o, heads, pos, pos_dev, window, chunks,
                           in_scale, codes, reinterpret_cast<const uint8_t *>(lin->w), lin->n, lin->k, lin->part);
        G4_LAUNCHED("attn_merge_o_kernel");
        return G4_OK;
    }
    hipLaunchKernelGGL(attn_merge_kernel, dim3(heads, rows), dim3(kDecThreads), 0,
                       as_stream(stream), part_ml, part_o, heads, pos, pos_dev, window, chunks,
                       in_scale, codes, nullptr);
    G4_LAUNCHED("attn_merge_kernel");
    return G4_OK;
}

bool merge_linear_fits(const MergeLinear &lin, int rows, int heads) {
    return lin.w && lin.part && rows == 1 && heads >= 1 && heads <= kAttnMaxHeads && lin.n > 0 &&
           lin.n % kMergeRows == 0 && lin.k == heads * kDecThreads &&
           (reinterpret_cast<uintptr_t>(lin.w) & 15) == 0;
}

}  // namespace g4

extern "C" {

int g4_rms_join(const void *src, int src_kind, float src_scale, const float *gain,
                const float *resid, float alpha, const float *gain2, int rows, int width,
                float eps, float in_scale, float *hidden, int8_t *codes, void *stream) {
    if (!src || rows <= 0 || width <= 0)
        return set_error(G4_ERR_INVALID, "rms-norm needs params.rows and params.width and input src");
    if (width > kJoinMaxPer * kDecThreads)
        return set_error(G4_ERR_UNSUPPORTED, "rms-norm: width %d exceeds %d", width,
                         kJoinMaxPer * kDecThreads);
    if (src_kind != G4_KIND_F32 && src_kind != G4_KIND_I8)
        return set_error(G4_ERR_INVALID, "rms-norm: src_kind must be f32 or int8 codes");
    if (!hidden && !codes) return set_error(G4_ERR_INVALID, "rms-norm: no output");
    if (codes && in_scale == 0.0f)
        return set_error(G4_ERR_INVALID, "rms-norm: int8 codes need the consumer's inScale");
    if (gain2 && !codes) return set_error(G4_ERR_INVALID, "norm-residual-norm: gain2 without codes");
    JoinTail J;
    J.src = src;
    J.src_kind = src_kind;
    J.src_scale = src_scale;
    J.gain = gain;
    J.resid = resid;
    J.alpha = alpha;
    J.gain2 = gain2;
    J.width = width;
    J.eps = eps;
    J.in_scale = in_scale;
    J.hidden = hidden;
    J.codes = codes;
    if (join_narrow(J.width))
        hipLaunchKernelGGL((join_kernel<false, kJoinPerNarrow>), dim3(rows), dim3(kDecThreads), 0,
                           as_stream(stream), J);
    else
        hipLaunchKernelGGL((join_kernel<false, kJoinMaxPer>), dim3(rows), dim3(kDecThreads), 0,
                           as_stream(stream), J);
    G4_LAUNCHED("join_kernel");
    return G4_OK;
}

int g4_attn_prologue(const int8_t *q_codes, float q_scale, const int8_t *k_codes, float k_scale,
                     const int8_t *v_codes, float v_scale, const float *q_gain,
                     const float *k_gain, const float *cos_tab, const float *sin_tab, int rows,
                     int heads, int head_dim, float eps, float *q_out, float *k_cache,
                     float *v_cache, int64_t cache_row_stride, int pos, const int32_t *pos_dev,
                     void *stream) {
    if (head_dim != kDecThreads)
        return set_error(G4_ERR_UNSUPPORTED, "q-norm-rope: head_dim %d (this build serves 256)",
                         head_dim);
    if (!q_codes || !q_gain || !cos_tab || !sin_tab || !q_out || rows <= 0 || heads <= 0)
        return set_error(G4_ERR_INVALID, "q-norm-rope needs inputs q, gain, cosTab, sinTab");
    if (pos < 0) return set_error(G4_ERR_INVALID, "q-norm-rope: position %d", pos);
    const bool producer = k_codes != nullptr;
    if (producer && (!v_codes || !k_gain || !k_cache || !v_cache))
        return set_error(G4_ERR_INVALID, "kv-norm-rope-store needs k, v, k gain and both caches");
    hipLaunchKernelGGL(attn_prologue_kernel, dim3(heads + (producer ? 2 : 0), rows),
                       dim3(kDecThreads), 0, as_stream(stream), q_codes, q_scale, k_codes, k_scale,
                       v_codes, v_scale, q_gain, k_gain, cos_tab, sin_tab, heads, eps, q_out,
                       k_cache, v_cache, cache_row_stride, pos, pos_dev);
    G4_LAUNCHED("attn_prologue_kernel");
    return G4_OK;
}

size_t g4_attention_workspace_bytes(int rows, int heads, int pos, int window) {
    if (rows <= 0 || heads <= 0 || pos < 0 || window < 0) return 0;
    return (size_t)rows * heads * attn_chunks(pos, window) * (2 + kDecThreads) * sizeof(float);
}

int g4_attention_decode(const float *q, const float *k_cache, const float *v_cache,
                        int64_t cache_row_stride, int rows, int heads, int head_dim, int pos,
                        const int32_t *pos_dev, int window, float *workspace,
                        size_t workspace_bytes, float in_scale, int8_t *codes, float *out_f32,
                        void *stream) {
    if (head_dim != kDecThreads)
        return set_error(G4_ERR_UNSUPPORTED, "attention-decode: head_dim %d (this build serves 256)",
                         head_dim);
    if (!q || !k_cache || !v_cache || !workspace || rows <= 0 || heads <= 0 || pos < 0 ||
        window < 0)
        return set_error(G4_ERR_INVALID, "attention-decode needs q, k, v, a workspace and pos >= 0");
    if (heads > kAttnMaxHeads)
        return set_error(G4_ERR_UNSUPPORTED, "attention-decode: %d query heads per KV head (at most %d)",
                         heads, kAttnMaxHeads);
    if (!codes && !out_f32) return set_error(G4_ERR_INVALID, "attention-decode: no output");
    if (codes && in_scale == 0.0f)
        return set_error(G4_ERR_INVALID, "attention-decode: int8 codes need the o_proj inScale");
    const int chunks = attn_chunks(pos, window);
    const size_t need = g4_attention_workspace_bytes(rows, heads, pos, window);
    if (workspace_bytes < need)
        return set_error(G4_ERR_INVALID, "attention-decode: workspace %zu B < %zu B",
                         workspace_bytes, need);
    float *part_ml = workspace;
    float *part_o = workspace + (size_t)rows * heads * chunks * 2;
    launch_split<false>(chunks, rows, as_stream(stream), q, k_cache, v_cache,
                                cache_row_stride, heads, pos, pos_dev, window, part_ml, part_o, AttnPrologue{});
    G4_LAUNCHED("attn_split_kernel");
    hipLaunchKernelGGL(attn_merge_kernel, dim3(heads, rows), dim3(kDecThreads), 0,
                       as_stream(stream), part_ml, part_o, heads, pos, pos_dev, window, chunks,
                       in_scale, codes, out_f32);
    G4_LAUNCHED("attn_merge_kernel");
    return G4_OK;
}

int g4_gelu_mul(const int8_t *g_codes, float g_scale, const int8_t *u_codes, float u_scale,
                const float *up_f32, int64_t up_stride, int rows, int n, float in_scale,
                int8_t *codes, void *stream) {
    if (!g_codes || !codes || (!u_codes && !up_f32) || rows <= 0 || n <= 0)
        return set_error(G4_ERR_INVALID, "gelu-mul needs inputs gate and up and an output");
    if (in_scale == 0.0f)
        return set_error(G4_ERR_INVALID, "gelu-mul: codes need the consumer's inScale");
    if (up_f32 && up_stride < n) return set_error(G4_ERR_INVALID, "gelu-mul: up stride < n");
    const int bx = grid_1d(n, kDecThreads);
    hipLaunchKernelGGL(gelu_mul_kernel, dim3(bx, rows), dim3(kDecThreads), 0, as_stream(stream),
                       g_codes, g_scale, u_codes, u_scale, up_f32, up_stride, n, in_scale, codes);
    G4_LAUNCHED("gelu_mul_kernel");
    return G4_OK;
}

int g4_gelu_mul_f32(const float *gate, const float *up, float *dst, int64_t count,
                    float srq_scale, void *stream) {
    if (count <= 0 || count % 4 != 0)
        return set_error(G4_ERR_INVALID, "gelu-mul needs params.count a positive multiple of 4, got %lld",
                         (long long)count);
    if (!gate || !up) return set_error(G4_ERR_INVALID, "gelu-mul needs inputs named gate and up");
    if (!dst) return set_error(G4_ERR_INVALID, "gelu-mul needs an output");
    if (((reinterpret_cast<uintptr_t>(gate) | reinterpret_cast<uintptr_t>(up) |
          reinterpret_cast<uintptr_t>(dst)) & 15) != 0)
        return set_error(G4_ERR_INVALID, "gelu-mul: gate, up and dst must be 16-byte aligned");
    if (!std::isfinite(srq_scale)) return set_error(G4_ERR_INVALID, "gelu-mul: srqScale must be finite");
    const int64_t n4 = count / 4;
    const int blocks = (int)std::min<int64_t>((n4 + kDecThreads - 1) / kDecThreads, 8 * 1024);
    hipLaunchKernelGGL(gelu_mul_f32_kernel, dim3(blocks), dim3(kDecThreads), 0, as_stream(stream),
                       reinterpret_cast<const float4 *>(gate), reinterpret_cast<const float4 *>(up),
                       reinterpret_cast<float4 *>(dst), n4, srq_scale);
    G4_LAUNCHED("gelu_mul_f32_kernel");
    return G4_OK;
}

int g4_embed_tokens(const void *table, const float *row_scales, const int32_t *ids, int rows,
                    int64_t vocab, int cols, float embed_scale, float in_scale, float *x,
                    int8_t *codes, void *stream) {
    if (!table || !row_scales || !ids || !x || rows <= 0 || vocab <= 0 || cols <= 0 || (cols & 1))
        return set_error(G4_ERR_INVALID, "embed-gather needs codes, scales, ids, the row count "
                                         "and an even width");
    if (codes && in_scale == 0.0f)
        return set_error(G4_ERR_INVALID, "embed-gather: codes need inScale");
    hipLaunchKernelGGL(embed_kernel, dim3(rows), dim3(kDecThreads), 0, as_stream(stream),
                       reinterpret_cast<const uint8_t *>(table), row_scales, ids, vocab, cols,
                       embed_scale, in_scale, x, codes);
    G4_LAUNCHED("embed_kernel");
    return G4_OK;
}

int g4_ple_combine(const int8_t *proj_codes, float proj_scale, float alpha, const float *gain,
                   const float *identity, int rows, int groups, int group, float eps, float *out,
                   void *stream) {
    if (group != kDecThreads)
        return set_error(G4_ERR_UNSUPPORTED, "per-layer inputs: group %d (serves 256)", group);
    if (!proj_codes || !gain || !identity || !out || rows <= 0 || groups <= 0)
        return set_error(G4_ERR_INVALID,
                         "per-layer inputs need the projection, gain and identity rows");
    hipLaunchKernelGGL(ple_combine_kernel, dim3(groups, rows), dim3(kDecThreads), 0,
                       as_stream(stream), proj_codes, proj_scale, alpha, gain, identity, groups,
                       eps, out);
    G4_LAUNCHED("ple_combine_kernel");
    return G4_OK;
}

size_t g4_argmax_workspace_bytes(int rows, int64_t vocab) {
    if (rows <= 0 || vocab <= 0) return 0;
    return (size_t)rows * (size_t)((vocab + kArgmaxSpan - 1) / kArgmaxSpan) * 8;
}

int g4_softcap_argmax(const float *logits, int rows, int64_t vocab, float cap, float *capped,
                      void *workspace, size_t workspace_bytes, int32_t *tokens, void *stream) {
    if (!logits || !tokens || !workspace || rows <= 0 || vocab <= 0 || vocab > INT32_MAX)
        return set_error(G4_ERR_INVALID, "argmax needs logits, a workspace and tokens");
    if (workspace_bytes < g4_argmax_workspace_bytes(rows, vocab))
        return set_error(G4_ERR_INVALID, "argmax: workspace %zu B < %zu B", workspace_bytes,
                         g4_argmax_workspace_bytes(rows, vocab));
    const int parts = (int)((vocab + kArgmaxSpan - 1) / kArgmaxSpan);
    float *pv = reinterpret_cast<float *>(workspace);
    int *pi = reinterpret_cast<int *>(pv + (size_t)rows * parts);
    hipLaunchKernelGGL(softcap_argmax_partial_kernel, dim3(parts, rows), dim3(kDecThreads), 0,
                       as_stream(stream), logits, vocab, cap, capped, pv, pi);
    G4_LAUNCHED("softcap_argmax_partial_kernel");
    hipLaunchKernelGGL(argmax_final_kernel, dim3(rows), dim3(64), 0, as_stream(stream), pv, pi,
                       parts, tokens);
    G4_LAUNCHED("argmax_final_kernel");
    return G4_OK;
}

int g4_fill_hash_f32(float *out, int64_t n, uint64_t seed, float lo, float hi, void *stream) {
    if (!out || n < 0) return set_error(G4_ERR_INVALID, "fill: bad arguments");
    if (n == 0) return G4_OK;
    hipLaunchKernelGGL(fill_hash_f32_kernel, dim3(grid_1d(n, 256)), dim3(256), 0,
                       as_stream(stream), out, n, seed, lo, hi - lo);
    G4_LAUNCHED("fill_hash_f32_kernel");
    return G4_OK;
}

int g4_fill_hash_u8(void *out, int64_t n, uint64_t seed, void *stream) {
    if (!out || n < 0) return set_error(G4_ERR_INVALID, "fill: bad arguments");
    if (n == 0) return G4_OK;
    hipLaunchKernelGGL(fill_hash_u8_kernel, dim3(grid_1d(n, 256)), dim3(256), 0,
                       as_stream(stream), reinterpret_cast<uint8_t *>(out), n, seed);
    G4_LAUNCHED("fill_hash_u8_kernel");
    return G4_OK;
}

}  // extern "C"

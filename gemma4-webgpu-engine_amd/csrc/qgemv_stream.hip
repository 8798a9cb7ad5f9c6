// The streaming decode GEMV (M = 1, calibrated path) for gfx950: qgemv-4bit / qgemv-8bit, the
// projection batches and the grouped layer GEMV (src/kernels/qgemv.ts, projectionBatch.ts) when
// the row length falls in one of the compiled shape classes.
//
// Shape class (BITS, LPR, CPL): a row is LPR * CPL 16-byte chunks. LPR lanes serve one row
// (16, 32 or 64), each lane streams CPL chunks of it (chunk lr + u * LPR), so one wave covers
// 64 / LPR rows with every weight load unguarded (the row index is clamped, the store is not).
// A tile is the 4 waves of a block over 4 * 64 / LPR consecutive rows of one job.
//
// Schedule. Jobs (one projection each) are laid end to end as tiles; block b takes the contiguous
// tile range [b * T / G, (b + 1) * T / G), so all blocks stream the same number of tiles. A block
// snaps the activation vector of its current job once into LDS (int8 codes, the same IEEE divide
// and ties-to-even as the reference's srqIn), then for every tile: 16-byte non-temporal weight
// loads and the row scale, the v_dot4_i32_i8 dot against the LDS codes, the fixed DPP / shuffle
// reduction over the row's lanes (exact int32), and the reference's epilogue on one lane.
//
// Why this shape: at 8 TB/s a layer's 17.8 MB is 2.2 us, so the kernel has to keep the HBM queue
// full rather than save ALU. Every load goes through the global address space (a flat load would
// also count against the LDS wait counter and serialize the weight stream behind the LDS reads),
// the body needs 45 VGPRs so 8 waves per SIMD fit, and the grid holds 8 blocks per CU.
//
// Job descriptors travel in the kernel arguments (up to kMaxKargJobs, the per-call entry points)
// or in a device table built once by g4_qgemv_plan_create (any count, the decode-step form: the
// reference caches its per-token bind the same way, runtime.ts:702-767).
#include "g4_rowops.h"

#include <algorithm>
#include <vector>

namespace g4 {

constexpr int kStreamThreads = 256;
constexpr int kMaxKargJobs = 16;
constexpr int kStreamMaxK = 16384;
// Blocks per CU in a streaming grid: every block resident at once at 4 waves per SIMD (the
// two-deep tile loop holds two tiles' weights, 123 VGPRs).
constexpr int kBlocksPerCu = 4;
static_assert(kStreamThreads == kRowThreads, "a prologue join runs on the GEMV's block");

#define G4_GLOBAL __attribute__((address_space(1)))

// One projection of a streaming launch (112 bytes). With the gelu prologue (up set) x is the gate
// and the block snaps gelu_tanh(gate) * up instead of x. With a gelu epilogue (epi != 0) the job's
// rows are the gate and dst receives srq(gelu(gate code * out_scale) * u, act_scale), where u is
// the same row of a paired up projection (epi 1: aux / aux_scales are its weights and scales) or
// aux[row] of an f32 vector (epi 2): the gelu-mul pass folded into the producer.
struct StreamJob {
    const uint8_t *w;
    const float *scales;
    const void *x;
    void *dst;
    const void *up;
    const void *aux;
    const float *aux_scales;
    int k;
    int rows;
    int tile_begin;
    int tiles;
    float in_scale;
    float out_scale;
    float g_scale;
    float u_scale;
    float act_scale;
    int8_t bits;
    int8_t x_kind;
    int8_t out_kind;
    int8_t cls;
    int8_t up_kind;
    int8_t epi;
    int8_t pre;  // x is the codes of the plan's prologue join, computed by every block (no snap)
    int8_t pad[13];
};
static_assert(sizeof(StreamJob) == 112, "StreamJob is one 112-byte record");

struct StreamArgs {
    const StreamJob *table;  // device table (plan launches); null for kernel-argument jobs
    const int *block_job;    // plan launches: the job of each block's first tile
    const int *block_tile;   // plan launches: block b takes tiles [block_tile[b], block_tile[b + 1])
    int njobs;
    int total_tiles;
    const JoinTail *pre;     // plan launches: the RMS join whose codes the `pre` jobs read; or null
    StreamJob job[kMaxKargJobs];
};

// The compiled classes. Index = StreamJob::cls.
struct ClassShape {
    int bits, lpr, cpl;
};
constexpr ClassShape kClasses[] = {
    {4, 16, 1}, {4, 16, 2}, {4, 16, 3}, {4, 16, 4}, {4, 32, 3}, {4, 32, 4}, {4, 64, 3}, {4, 64, 4},
    {8, 16, 1}, {8, 16, 2}, {8, 16, 3}, {8, 16, 4}, {8, 32, 3}, {8, 32, 4}, {8, 64, 3}, {8, 64, 4},
    {8, 64, 6},
};
constexpr int kNumClasses = sizeof(kClasses) / sizeof(kClasses[0]);

// The class of a row of K codes at `bits`, or -1 when no compiled class fits.
int stream_class_for(int bits, int k) {
    if (k <= 0 || k > kStreamMaxK) return -1;
    const int row_bytes = bits == 4 ? k / 2 : k;
    if (row_bytes % 16) return -1;
    const int chunks = row_bytes / 16;
    for (int lpr : {16, 32, 64}) {
        if (chunks % lpr) continue;
        const int cpl = chunks / lpr;
        for (int c = 0; c < kNumClasses; ++c)
            if (kClasses[c].bits == bits && kClasses[c].lpr == lpr && kClasses[c].cpl == cpl) return c;
    }
    return -1;
}

static int rows_per_tile(int cls) { return 4 * (64 / kClasses[cls].lpr); }

typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// Loads and stores through the global address space (C casts: reinterpret_cast cannot change
// the address space).
template <typename T>
__device__ __forceinline__ T gload(const void *p) {
    return *(const G4_GLOBAL T *)p;
}
template <typename T>
__device__ __forceinline__ void gstore(void *p, T v) {
    *(G4_GLOBAL T *)p = v;
}

__device__ __forceinline__ u32x4 load_w16(const uint8_t *p) {
    return __builtin_nontemporal_load((const G4_GLOBAL u32x4 *)p);
}

__device__ __forceinline__ uint32_t pack_bytes(int a, int b, int c, int d) {
    return (uint32_t)(a & 0xff) | ((uint32_t)(b & 0xff) << 8) | ((uint32_t)(c & 0xff) << 16) |
           ((uint32_t)(d & 0xff) << 24);
}

// Activation groups (8 values) per thread whose loads go out together in the snap (f32 groups
// are twice as wide, so half as many fit the register budget).
template <int KIND>
constexpr int snap_batch() { return KIND == G4_KIND_F32 ? 2 : 4; }

template <int KIND>
struct RawGroup {
    u32x4 a, b;  // f32: 32 bytes; f16: a only; int8: a.xy
};

template <int KIND>
__device__ __forceinline__ RawGroup<KIND> load_group(const void *x, int g) {
    RawGroup<KIND> r;
    if (KIND == G4_KIND_F32) {
        const float *p = reinterpret_cast<const float *>(x) + g * 8;
        r.a = gload<u32x4>(p);
        r.b = gload<u32x4>(p + 4);
    } else if (KIND == G4_KIND_F16) {
        r.a = gload<u32x4>(reinterpret_cast<const __half *>(x) + g * 8);
    } else {
        const u32x2 v = gload<u32x2>(reinterpret_cast<const int8_t *>(x) + g * 8);
        r.a = u32x4{v.x, v.y, 0u, 0u};
    }
    return r;
}

template <int KIND>
__device__ __forceinline__ void group_codes(const RawGroup<KIND> &r, float s, float rcp, bool r_ok,
                                            int c[8]) {
    if (KIND == G4_KIND_F32) {
        const uint32_t v[8] = {r.a.x, r.a.y, r.a.z, r.a.w, r.b.x, r.b.y, r.b.z, r.b.w};
#pragma unroll
        for (int i = 0; i < 8; ++i) c[i] = (int)srq_code_fast(__uint_as_float(v[i]), s, rcp, r_ok);
    } else if (KIND == G4_KIND_F16) {
        const uint32_t w[4] = {r.a.x, r.a.y, r.a.z, r.a.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            c[2 * i] = (int)srq_code_fast(
                __half2float(__ushort_as_half((unsigned short)(w[i] & 0xffff))), s, rcp, r_ok);
            c[2 * i + 1] = (int)srq_code_fast(
                __half2float(__ushort_as_half((unsigned short)(w[i] >> 16))), s, rcp, r_ok);
        }
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            c[i] = (int)(int8_t)((r.a.x >> (8 * i)) & 0xff);
            c[4 + i] = (int)(int8_t)((r.a.y >> (8 * i)) & 0xff);
        }
    }
}

// The snap body for one activation kind: each thread issues the loads of a batch of groups
// (indices clamped, so every load is valid) before converting any, so a long vector costs one
// memory latency per batch rather than one per group.
template <int KIND>
__device__ __forceinline__ int snap_kind(const StreamJob &J, uint8_t *xs, int tid) {
    bool r_ok;
    const float s = J.in_scale;
    const float rcp = srq_recip(s, r_ok);
    const int groups = J.k >> 3;
    int local = 0;
    constexpr int B = snap_batch<KIND>();
    for (int g0 = tid; g0 < groups; g0 += B * kStreamThreads) {
        RawGroup<KIND> raw[B];
#pragma unroll
        for (int i = 0; i < B; ++i)
            raw[i] = load_group<KIND>(J.x, min(g0 + i * kStreamThreads, groups - 1));
#pragma unroll
        for (int i = 0; i < B; ++i) {
            const int g = g0 + i * kStreamThreads;
            if (g < groups) {
                int c[8];
                group_codes<KIND>(raw[i], s, rcp, r_ok, c);
                uint2 packed;
                if (J.bits == 4) {
                    packed.x = pack_bytes(c[0], c[2], c[4], c[6]);
                    packed.y = pack_bytes(c[1], c[3], c[5], c[7]);
                } else {
                    packed.x = pack_bytes(c[0], c[1], c[2], c[3]);
                    packed.y = pack_bytes(c[4], c[5], c[6], c[7]);
                }
                *reinterpret_cast<uint2 *>(xs + g * 8) = packed;
                local += c[0] + c[1] + c[2] + c[3] + c[4] + c[5] + c[6] + c[7];
            }
        }
    }
    return local;
}

// The gelu prologue's snap: codes of gelu_tanh(gate) * up for the job's K activations.
__device__ __forceinline__ int snap_gelu(const StreamJob &J, uint8_t *xs, int tid) {
    bool r_ok;
    const float s = J.in_scale;
    const float rcp = srq_recip(s, r_ok);
    const int groups = J.k >> 3;
    int local = 0;
    for (int g = tid; g < groups; g += kStreamThreads) {
        int c[8];
        gelu_codes8(J.x, J.x_kind, J.g_scale, J.up, J.up_kind, J.u_scale, (int64_t)g * 8, s, rcp,
                    r_ok, c);
        uint2 packed;
        if (J.bits == 4) {
            packed.x = pack_bytes(c[0], c[2], c[4], c[6]);
            packed.y = pack_bytes(c[1], c[3], c[5], c[7]);
        } else {
            packed.x = pack_bytes(c[0], c[1], c[2], c[3]);
            packed.y = pack_bytes(c[4], c[5], c[6], c[7]);
        }
        *reinterpret_cast<uint2 *>(xs + g * 8) = packed;
        local += c[0] + c[1] + c[2] + c[3] + c[4] + c[5] + c[6] + c[7];
    }
    return local;
}

// The block's sum of its threads' code sums (after the snap's LDS stores).
__device__ __forceinline__ int block_code_sum(int local, int *s_sum, int tid) {
    if (tid == 0) *s_sum = 0;
    lds_barrier();
    local = row16_sum_i32(local);
    if ((tid & 15) == 0 && local != 0) atomicAdd(s_sum, local);
    lds_barrier();
    return *s_sum;
}

// The prologue join's snap: every block runs the RMS join that produces the job's activation row
// (the same arithmetic as the join kernel, so the same codes) and stores its codes in the snap
// layout; block 0 also stores the join's outputs (the new residual row and the codes) for the
// kernels after this one. Replaces a join launch between the producer GEMV and this one.
template <typename Loads = NoLoads>
__device__ __forceinline__ int snap_join(const JoinTail *pre, int four, uint8_t *xs,
                                         Loads after_loads = Loads()) {
    JoinTail T = *pre;
    // the reduction tree sits in the dynamic LDS after the codes (the launch sizes it so); a
    // static array would shift every code address of the tile loop by its size
    float *red = reinterpret_cast<float *>(xs + ((T.width + 15) & ~15));
    int8_t *codes = blockIdx.x == 0 ? T.codes : nullptr;
    if (blockIdx.x != 0) T.hidden = nullptr;
    int local = 0;
    auto emit = [&](int i, int8_t c) {
        const int j = i & 7;
        xs[four ? (i & ~7) + (j & 1 ? 4 : 0) + (j >> 1) : i] = (uint8_t)c;
        if (codes) gstore<int8_t>(codes + i, c);
        local += c;
    };
    // an int32 accumulator source (the decode runner's o_proj folded into the attention merge)
    // runs the producing linear's epilogue and snap first
    // rows up to 1536 wide take 6 elements per thread (no loads past the row)
    if (join_narrow(T.width)) {
        if (T.src_kind == G4_KIND_I32) rms_join_row_emit<1, kJoinPerNarrow>(T, 0, red, emit, after_loads);
        else rms_join_row_emit<0, kJoinPerNarrow>(T, 0, red, emit, after_loads);
    } else {
        if (T.src_kind == G4_KIND_I32) rms_join_row_emit<1>(T, 0, red, emit, after_loads);
        else rms_join_row_emit<0>(T, 0, red, emit, after_loads);
    }
    return local;
}

// Snaps the K activations of job J into int8 codes in LDS (4-bit jobs: each 8-code group stored
// as [x0 x2 x4 x6 | x1 x3 x5 x7] so a weight word's low and high nibbles each dot one half) and
// returns sum(xq) over the whole vector, which takes the 4-bit zero point off once per row.
__device__ __forceinline__ int snap_activations(const StreamJob &J, uint8_t *xs, int *s_sum, int tid) {
    int local;
    if (J.up)
        local = snap_gelu(J, xs, tid);
    else if (J.x_kind == G4_KIND_F16)
        local = snap_kind<G4_KIND_F16>(J, xs, tid);
    else if (J.x_kind == G4_KIND_F32)
        local = snap_kind<G4_KIND_F32>(J, xs, tid);
    else
        local = snap_kind<G4_KIND_I8>(J, xs, tid);
    return block_code_sum(local, s_sum, tid);
}

// The codes of a prologue join in the snap layout, and their sum. after_loads: as for
// rms_join_row_emit (the caller's tile loads, queued behind the join's operands).
template <typename Loads = NoLoads>
__device__ __forceinline__ int snap_join_codes(const JoinTail *pre, bool four, uint8_t *xs,
                                               int *s_sum, int tid, Loads after_loads = Loads()) {
    return block_code_sum(snap_join(pre, four, xs, after_loads), s_sum, tid);
}

// One output element of job J at row `row` (the reference's epilogue, qgemv.ts:680-686).
__device__ __forceinline__ void stream_store(const StreamJob &J, int row, int s, float scale) {
    const float y = linear_epilogue(J.in_scale, scale, (float)s);
    if (J.out_kind == G4_KIND_I8) {
        gstore<int8_t>(reinterpret_cast<int8_t *>(J.dst) + row, (int8_t)srq_code_i(y, J.out_scale));
    } else if (J.out_kind == G4_KIND_I32) {
        gstore<int32_t>(reinterpret_cast<int32_t *>(J.dst) + row, s);
    } else {
        float v = y;
        if (J.out_scale != 0.0f) v = __fmul_rn(srq_code_f(y, J.out_scale), J.out_scale);
        gstore<float>(reinterpret_cast<float *>(J.dst) + row, v);
    }
}

// The dot of one 16-byte weight chunk against its LDS codes.
template <int BITS>
__device__ __forceinline__ int chunk_dot(const u32x4 &w, const uint8_t *xs, int ch, int acc) {
    const uint32_t wv[4] = {w.x, w.y, w.z, w.w};
    if (BITS == 4) {
        const u32x4 xa = *reinterpret_cast<const u32x4 *>(xs + ch * 32);
        const u32x4 xb = *reinterpret_cast<const u32x4 *>(xs + ch * 32 + 16);
        const uint32_t xv[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            acc = __builtin_amdgcn_sdot4((int)(wv[i] & 0x0F0F0F0Fu), (int)xv[2 * i], acc, false);
            acc = __builtin_amdgcn_sdot4((int)((wv[i] >> 4) & 0x0F0F0F0Fu), (int)xv[2 * i + 1], acc,
                                         false);
        }
    } else {
        const u32x4 xa = *reinterpret_cast<const u32x4 *>(xs + ch * 16);
        acc = __builtin_amdgcn_sdot4((int)wv[0], (int)xa.x, acc, false);
        acc = __builtin_amdgcn_sdot4((int)wv[1], (int)xa.y, acc, false);
        acc = __builtin_amdgcn_sdot4((int)wv[2], (int)xa.z, acc, false);
        acc = __builtin_amdgcn_sdot4((int)wv[3], (int)xa.w, acc, false);
    }
    return acc;
}

template <int LPR>
__device__ __forceinline__ int row_reduce(int acc) {
    acc = row16_sum_i32(acc);
    if (LPR >= 32) acc += __shfl_xor(acc, 16);
    if (LPR >= 64) acc += __shfl_xor(acc, 32);
    return acc;
}

// The gelu epilogue of a gate row (epi != 0): the gate's int8 code back on out_scale, the up value
// (a paired row's code on out_scale, or the f32 vector entry), and the snap of gelu(g) * u on
// act_scale: the gelu-mul pass (geluMul.ts:101-116) on exactly the values it would have read.
__device__ __forceinline__ void stream_store_gelu(const StreamJob &J, int row, float y_gate,
                                                  float u) {
    const float g = __fmul_rn(srq_code_f(y_gate, J.out_scale), J.out_scale);
    gstore<int8_t>(reinterpret_cast<int8_t *>(J.dst) + row,
                   (int8_t)srq_code_i(__fmul_rn(d_gelu(g), u), J.act_scale));
}

// One tile of one job for class <BITS, LPR, CPL>: this lane's CPL 16-byte chunks of its row
// (row index clamped, so every load is valid) and the row scale, the dot against the LDS codes,
// the fixed reduction over the row's LPR lanes (exact int32), and the row's output from one lane.
// PAIR: the same rows of the paired up projection stream beside the gate's, for the gelu epilogue.
// PRE (a block's first tile): the block fills the LDS codes inside the tile (sx is their sum): 1,
// the plan's prologue join, whose operand loads go out first and the tile's weight loads right
// behind them (the join waits for its own operands only); 2, the job's own snap, after the weight
// loads. Either way the codes' memory latency overlaps the weight stream's. Returns sx.
template <int BITS, int LPR, int CPL, bool PAIR, int PRE = 0>
__device__ __forceinline__ int stream_tile(const StreamJob &J, int t, uint8_t *xs, int sx, int wave,
                                           int lane, const JoinTail *pre = nullptr,
                                           int *s_sum = nullptr) {
    constexpr int RPW = 64 / LPR;
    constexpr int ROW_BYTES = LPR * CPL * 16;
    const int lr = lane & (LPR - 1);
    const int row = (t - J.tile_begin) * (4 * RPW) + wave * RPW + lane / LPR;
    const int rc = min(row, J.rows - 1);
    const uint8_t *base = J.w + (int64_t)rc * ROW_BYTES + lr * 16;
    u32x4 w[CPL];
    u32x4 w2[PAIR ? CPL : 1];
    float scale, scale2 = 0.0f;
    auto load_tile = [&]() {
#pragma unroll
        for (int u = 0; u < CPL; ++u) w[u] = load_w16(base + u * LPR * 16);
        if (PAIR) {
            const uint8_t *base2 = reinterpret_cast<const uint8_t *>(J.aux) + (int64_t)rc * ROW_BYTES + lr * 16;
#pragma unroll
            for (int u = 0; u < CPL; ++u) w2[u] = load_w16(base2 + u * LPR * 16);
        }
        scale = gload<float>(J.scales + rc);
        if (PAIR) scale2 = gload<float>(J.aux_scales + rc);
    };
    if (PRE == 1) {
        // the join's operands go out first, the tile's weights right behind them
        sx = snap_join_codes(pre, BITS == 4, xs, s_sum, threadIdx.x, [&]() {
            load_tile();
            __builtin_amdgcn_sched_barrier(0);
        });
    } else {
        load_tile();
        if (PRE == 2) sx = snap_activations(J, xs, s_sum, threadIdx.x);
    }
    int acc = 0, acc2 = 0;
#pragma unroll
    for (int u = 0; u < CPL; ++u) acc = chunk_dot<BITS>(w[u], xs, lr + u * LPR, acc);
    if (PAIR) {
#pragma unroll
        for (int u = 0; u < CPL; ++u) acc2 = chunk_dot<BITS>(w2[u], xs, lr + u * LPR, acc2);
    }
    acc = row_reduce<LPR>(acc);
    if (PAIR) acc2 = row_reduce<LPR>(acc2);
    if (lr != 0 || row >= J.rows) return sx;
    const int a = BITS == 4 ? acc - 8 * sx : acc;
    if (J.epi == 0) {
        stream_store(J, row, a, scale);
    } else if (PAIR) {
        const int a2 = BITS == 4 ? acc2 - 8 * sx : acc2;
        const float yu = linear_epilogue(J.in_scale, scale2, (float)a2);
        stream_store_gelu(J, row, linear_epilogue(J.in_scale, scale, (float)a),
                          __fmul_rn(srq_code_f(yu, J.out_scale), J.out_scale));
    } else {
        stream_store_gelu(J, row, linear_epilogue(J.in_scale, scale, (float)a),
                          gload<float>(reinterpret_cast<const float *>(J.aux) + row));
    }
    return sx;
}

// Tiles [ta, tb) of one job (epi 0), two deep: tile t+1's weight loads go out before tile t's dot,
// reduction and store, so a wave never waits a full memory latency between tiles (the one-tile loop
// of stream_tile left each wave with nothing in flight while it finished a tile). The rows, the dot,
// the reduction and the store are stream_tile's, so the results are the same bits.
template <int BITS, int LPR, int CPL>
__device__ __forceinline__ void stream_job_tiles(const StreamJob &J, int ta, int tb, const uint8_t *xs,
                                                 int sx, int wave, int lane) {
    constexpr int RPW = 64 / LPR;
    constexpr int ROW_BYTES = LPR * CPL * 16;
    const int lr = lane & (LPR - 1);
    const int rbase = wave * RPW + lane / LPR - J.tile_begin * (4 * RPW);
    auto load = [&](int t, u32x4 (&w)[CPL], float &sc) {
        const int rc = min(t * (4 * RPW) + rbase, J.rows - 1);
        const uint8_t *base = J.w + (int64_t)rc * ROW_BYTES + lr * 16;
#pragma unroll
        for (int u = 0; u < CPL; ++u) w[u] = load_w16(base + u * LPR * 16);
        sc = gload<float>(J.scales + rc);
    };
    auto finish = [&](int t, const u32x4 (&w)[CPL], float sc) {
        int acc = 0;
#pragma unroll
        for (int u = 0; u < CPL; ++u) acc = chunk_dot<BITS>(w[u], xs, lr + u * LPR, acc);
        acc = row_reduce<LPR>(acc);
        const int row = t * (4 * RPW) + rbase;
        if (lr == 0 && row < J.rows) stream_store(J, row, BITS == 4 ? acc - 8 * sx : acc, sc);
    };
    u32x4 wa[CPL], wb[CPL];
    float sa, sb;
    load(ta, wa, sa);
    int t = ta;
    for (; t + 1 < tb; t += 2) {
        load(t + 1, wb, sb);
        finish(t, wa, sa);
        if (t + 2 < tb) load(t + 2, wa, sa);
        finish(t + 1, wb, sb);
    }
    if (t < tb) finish(t, wa, sa);
}

// stream_job_tiles for the job's class.
__device__ __forceinline__ void stream_dispatch_job(const StreamJob &J, int ta, int tb, const uint8_t *xs,
                                                    int sx, int wave, int lane) {
    switch (J.cls) {
#define G4_CASE(i)                                                                                 \
    case i:                                                                                        \
        stream_job_tiles<kClasses[i].bits, kClasses[i].lpr, kClasses[i].cpl>(J, ta, tb, xs, sx, wave, lane); \
        break;
        G4_CASE(0) G4_CASE(1) G4_CASE(2) G4_CASE(3) G4_CASE(4) G4_CASE(5) G4_CASE(6) G4_CASE(7)
        G4_CASE(8) G4_CASE(9) G4_CASE(10) G4_CASE(11) G4_CASE(12) G4_CASE(13) G4_CASE(14)
        G4_CASE(15) G4_CASE(16)
#undef G4_CASE
        default:
            break;
    }
}

// A block's first tile with its codes filled inside it (stream_tile PRE); returns the code sum.
template <bool PAIR, int PRE>
__device__ __forceinline__ int stream_dispatch_first(const StreamJob &J, int t, uint8_t *xs, int wave,
                                                     int lane, const JoinTail *pre, int *s_sum) {
    if (PAIR && J.epi == 1) {
        switch (J.cls) {
#define G4_CASE(i)                                                                               \
    case i:                                                                                      \
        return stream_tile<kClasses[i].bits, kClasses[i].lpr, kClasses[i].cpl, true, PRE>(       \
            J, t, xs, 0, wave, lane, pre, s_sum);
            G4_CASE(0) G4_CASE(1) G4_CASE(2) G4_CASE(3) G4_CASE(4) G4_CASE(5) G4_CASE(6) G4_CASE(7)
#undef G4_CASE
            default:
                break;
        }
    } else {
        switch (J.cls) {
#define G4_CASE(i)                                                                               \
    case i:                                                                                      \
        return stream_tile<kClasses[i].bits, kClasses[i].lpr, kClasses[i].cpl, false, PRE>(      \
            J, t, xs, 0, wave, lane, pre, s_sum);
            G4_CASE(0) G4_CASE(1) G4_CASE(2) G4_CASE(3) G4_CASE(4) G4_CASE(5) G4_CASE(6) G4_CASE(7)
            G4_CASE(8) G4_CASE(9) G4_CASE(10) G4_CASE(11) G4_CASE(12) G4_CASE(13) G4_CASE(14)
            G4_CASE(15) G4_CASE(16)
#undef G4_CASE
            default:
                break;
        }
    }
    // no class: codes only
    if (PRE == 1) return snap_join_codes(pre, J.bits == 4, xs, s_sum, threadIdx.x);
    return snap_activations(J, xs, s_sum, threadIdx.x);
}

template <bool PAIR>
__device__ __forceinline__ void stream_dispatch(const StreamJob &J, int t, uint8_t *xs,
                                                int sx, int wave, int lane) {
    if (PAIR && J.epi == 1) {
        // paired gate/up rows: the 4-bit classes only (the host refuses others)
        switch (J.cls) {
#define G4_CASE(i)                                                                               \
    case i:                                                                                      \
        stream_tile<kClasses[i].bits, kClasses[i].lpr, kClasses[i].cpl, true>(J, t, xs, sx, wave, \
                                                                              lane);             \
        break;
            G4_CASE(0) G4_CASE(1) G4_CASE(2) G4_CASE(3) G4_CASE(4) G4_CASE(5) G4_CASE(6) G4_CASE(7)
#undef G4_CASE
            default:
                break;
        }
        return;
    }
    switch (J.cls) {
#define G4_CASE(i)                                                                                \
    case i:                                                                                       \
        stream_tile<kClasses[i].bits, kClasses[i].lpr, kClasses[i].cpl, false>(J, t, xs, sx, wave, \
                                                                               lane);             \
        break;
        G4_CASE(0) G4_CASE(1) G4_CASE(2) G4_CASE(3) G4_CASE(4) G4_CASE(5) G4_CASE(6) G4_CASE(7)
        G4_CASE(8) G4_CASE(9) G4_CASE(10) G4_CASE(11) G4_CASE(12) G4_CASE(13) G4_CASE(14)
        G4_CASE(15) G4_CASE(16)
#undef G4_CASE
        default:
            break;
    }
}
static_assert(kNumClasses == 17, "stream_dispatch lists every class");
static_assert(kClasses[7].bits == 4 && kClasses[8].bits == 8, "classes 0-7 are the 4-bit ones");

// MODE 1 (plan launches whose jobs all read a prologue join's codes): the block's codes come from
// the join, run inside its first tile after that tile's weight loads are out, and stay for every
// job. MODE 2: the first job's snap runs inside the first tile the same way; later jobs snap as
// usual. MODE 0: every snap before its tiles.
template <bool TABLE, bool PAIR, int MODE>
__device__ __forceinline__ void stream_body(const StreamArgs &A, uint8_t *xs, int *s_sum) {
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const unsigned G = gridDim.x, b = blockIdx.x;
    const int t0 = TABLE ? A.block_tile[b] : (int)(((uint64_t)b * (unsigned)A.total_tiles) / G);
    const int t1 = TABLE ? A.block_tile[b + 1] : (int)(((uint64_t)(b + 1) * (unsigned)A.total_tiles) / G);
    if (t0 >= t1) return;
    int j;
    if (TABLE) {
        j = A.block_job[b];
    } else {
        j = 0;
#pragma unroll
        for (int i = 1; i < kMaxKargJobs; ++i)
            if (i < A.njobs && t0 >= A.job[i].tile_begin) j = i;
    }
    int sx;
    StreamJob J = TABLE ? A.table[j] : A.job[j];
    if (MODE == 0 && !PAIR) {
        // each job's run of this block's tiles two deep; a gelu-epilogue job tile by tile
        sx = snap_activations(J, xs, s_sum, tid);
        int t = t0;
        while (true) {
            const int te = min(t1, J.tile_begin + J.tiles);
            if (J.epi == 0) {
                stream_dispatch_job(J, t, te, xs, sx, wave, lane);
            } else {
                for (int tt = t; tt < te; ++tt) stream_dispatch<PAIR>(J, tt, xs, sx, wave, lane);
            }
            t = te;
            if (t >= t1) break;
            ++j;
            J = TABLE ? A.table[j] : A.job[j];
            __syncthreads();
            sx = snap_activations(J, xs, s_sum, tid);
        }
        return;
    }
    if (MODE != 0)
        sx = stream_dispatch_first<PAIR, MODE>(J, t0, xs, wave, lane, A.pre, s_sum);  // tile t0 done
    else
        sx = snap_activations(J, xs, s_sum, tid);
    for (int t = MODE != 0 ? t0 + 1 : t0; t < t1; ++t) {
        if (t >= J.tile_begin + J.tiles) {
            ++j;
            J = TABLE ? A.table[j] : A.job[j];
            if (MODE != 1) {
                __syncthreads();  // every wave is done with the previous job's codes
                sx = snap_activations(J, xs, s_sum, tid);
            }
        }
        stream_dispatch<PAIR>(J, t, xs, sx, wave, lane);
    }
}

// 4 waves per SIMD: MODE 0 streams its tiles two deep, and a plan that fills its codes inside the
// first tile (MODE 1 or 2) holds that tile's weights across the join or snap; either needs more
// than the 64 registers of 8 waves per SIMD. On config 1's 245-projection plan the two-deep loop at
// 4 waves measured 81.0% of 8 TB/s against 78.5% for the one-tile loop at 8 (same box, back to
// back); 8 blocks per CU at 4 waves (two rounds) gave 80.1%.
template <bool TABLE, int MODE>
__global__ __launch_bounds__(kStreamThreads) __attribute__((amdgpu_waves_per_eu(4, 8)))
void qgemv_stream_kernel(StreamArgs A) {
    extern __shared__ __align__(16) uint8_t xs[];
    __shared__ int s_sum;
    stream_body<TABLE, false, MODE>(A, xs, &s_sum);
}

// The same with paired gate/up jobs: twice the weight registers, so half the waves per SIMD.
template <bool TABLE, int MODE>
__global__ __launch_bounds__(kStreamThreads) __attribute__((amdgpu_waves_per_eu(4, 8)))
void qgemv_stream_pair_kernel(StreamArgs A) {
    extern __shared__ __align__(16) uint8_t xs[];
    __shared__ int s_sum;
    stream_body<TABLE, true, MODE>(A, xs, &s_sum);
}

// Fills a StreamJob from a validated descriptor and prologue; returns false when no class fits.
bool stream_job_from(const g4_gemv_desc &d, const GeluAct &act, StreamJob &J) {
    const int cls = stream_class_for(d.bits, d.k);
    if (cls < 0 || d.in_scale == 0.0f) return false;
    J = StreamJob{};
    J.w = reinterpret_cast<const uint8_t *>(d.wq);
    J.scales = d.scales;
    J.x = d.x;
    J.dst = d.dst;
    J.k = d.k;
    J.rows = d.num_rows;
    J.in_scale = d.in_scale;
    J.out_scale = d.out_scale;
    J.bits = (int8_t)d.bits;
    J.x_kind = (int8_t)d.x_kind;
    J.out_kind = (int8_t)d.out_kind;
    J.cls = (int8_t)cls;
    J.up = act.up;
    J.up_kind = (int8_t)act.up_kind;
    J.g_scale = act.g_scale;
    J.u_scale = act.u_scale;
    return true;
}

// Lays the jobs out as tiles; returns the total tile count and the widest K.
static int layout_tiles(StreamJob *jobs, int count, int &max_k) {
    int t = 0;
    max_k = 0;
    for (int i = 0; i < count; ++i) {
        const int rpt = rows_per_tile(jobs[i].cls);
        jobs[i].tile_begin = t;
        jobs[i].tiles = (jobs[i].rows + rpt - 1) / rpt;
        t += jobs[i].tiles;
        max_k = std::max(max_k, jobs[i].k);
    }
    return t;
}

static int grid_for(int tiles) {
    return std::max(1, std::min(tiles, kBlocksPerCu * device_cu_count()));
}

// Launches up to kMaxKargJobs streaming jobs with the descriptors in the kernel arguments.
int launch_stream_karg(StreamJob *jobs, int count, hipStream_t stream) {
    if (count < 1 || count > kMaxKargJobs)
        return set_error(G4_ERR_INVALID, "streaming GEMV: %d jobs (1..%d per call)", count, kMaxKargJobs);
    StreamArgs A{};
    int max_k = 0;
    A.total_tiles = layout_tiles(jobs, count, max_k);
    A.njobs = count;
    for (int i = 0; i < count; ++i) A.job[i] = jobs[i];
    const int grid = grid_for(A.total_tiles);
    hipLaunchKernelGGL((qgemv_stream_kernel<false, 0>), dim3(grid), dim3(kStreamThreads),
                       (size_t)((max_k + 15) & ~15), stream, A);
    G4_LAUNCHED("qgemv_stream_kernel");
    return G4_OK;
}

// Launches the jobs on the streaming kernel when every one of them is calibrated and has a shape
// class; otherwise enqueues nothing and reports *launched = false.
int stream_try_launch(const g4_gemv_desc *descs, const GeluAct *acts, int count, hipStream_t stream,
                      bool *launched) {
    *launched = false;
    if (count < 1 || count > kMaxKargJobs) return G4_OK;
    StreamJob jobs[kMaxKargJobs];
    for (int i = 0; i < count; ++i)
        if (!stream_job_from(descs[i], acts ? acts[i] : GeluAct{}, jobs[i])) return G4_OK;
    int rc = launch_stream_karg(jobs, count, stream);
    if (rc == G4_OK) *launched = true;
    return rc;
}

}  // namespace g4

using namespace g4;

// A reusable launch over any number of projections: the job table and block map live on the
// device, built once.
struct g4_gemv_plan {
    StreamJob *table = nullptr;
    int *block_job = nullptr;
    int njobs = 0;
    int total_tiles = 0;
    int grid = 0;
    int max_k = 0;
    int device = 0;
    bool paired = false;  // launches qgemv_stream_pair_kernel
    JoinTail *pre = nullptr;  // device copy of the prologue join, or null
    bool first_tile_snap = false;  // MODE 2: the snap inside each block's first tile
};

namespace g4 {

// Uploads a validated job list as a plan.
static int plan_from_jobs(std::vector<StreamJob> &jobs, g4_gemv_plan **out) {
    const int count = (int)jobs.size();
    int max_k = 0;
    const int tiles = layout_tiles(jobs.data(), count, max_k);
    const int grid = grid_for(tiles);
    // Blocks take equal shares of the weight bytes, not of the tiles: a tile of o_proj (K 2048)
    // holds 16 KB where the others hold 12 KB, and with every block resident at once the launch
    // lasts as long as its heaviest block. block_job[0, grid): the job of each block's first
    // tile; block_job[grid, 2 grid]: the tile ranges.
    std::vector<uint64_t> cum(tiles + 1, 0);
    for (int j = 0; j < count; ++j) {
        const uint64_t tb = (uint64_t)rows_per_tile(jobs[j].cls) * (jobs[j].bits == 4 ? jobs[j].k / 2 : jobs[j].k) *
                            (jobs[j].epi == 1 ? 2 : 1);
        for (int t = jobs[j].tile_begin; t < jobs[j].tile_begin + jobs[j].tiles; ++t) cum[t + 1] = cum[t] + tb;
    }
    std::vector<int> block_job(2 * (size_t)grid + 1);
    int *block_tile = block_job.data() + grid;
    for (int b = 0, t = 0; b < grid; ++b) {
        const uint64_t target = cum[tiles] * (uint64_t)b / (uint64_t)grid;
        while (t < tiles && cum[t] < target) ++t;
        block_tile[b] = t;
    }
    block_tile[grid] = tiles;
    for (int b = 0, j = 0; b < grid; ++b) {
        const int tb = std::min(block_tile[b], tiles - 1);
        while (j + 1 < count && jobs[j + 1].tile_begin <= tb) ++j;
        block_job[b] = j;
    }
    g4_gemv_plan *p = new g4_gemv_plan();
    p->njobs = count;
    p->total_tiles = tiles;
    p->grid = grid;
    p->max_k = max_k;
    for (const StreamJob &J : jobs) p->paired |= J.epi == 1;
    hipError_t err = hipGetDevice(&p->device);
    if (err == hipSuccess) err = hipMalloc(&p->table, sizeof(StreamJob) * count);
    if (err == hipSuccess) err = hipMalloc(&p->block_job, sizeof(int) * block_job.size());
    if (err == hipSuccess)
        err = hipMemcpy(p->table, jobs.data(), sizeof(StreamJob) * count, hipMemcpyHostToDevice);
    if (err == hipSuccess)
        err = hipMemcpy(p->block_job, block_job.data(), sizeof(int) * block_job.size(), hipMemcpyHostToDevice);
    if (err != hipSuccess) {
        (void)hipFree(p->table);
        (void)hipFree(p->block_job);
        delete p;
        return hip_status(err, "GEMV plan");
    }
    *out = p;
    return G4_OK;
}

int gemv_plan_create_epilogue(const g4_gemv_desc *descs, const GeluEpilogue *epis, int count,
                              g4_gemv_plan **out) {
    if (!out || !descs || count < 1) return set_error(G4_ERR_INVALID, "GEMV plan: no projections");
    *out = nullptr;
    std::vector<StreamJob> jobs(count);
    for (int i = 0; i < count; ++i) {
        int rc = check_job_desc(descs[i], GeluAct{}, "GEMV plan");
        if (rc) return rc;
        if (!stream_job_from(descs[i], GeluAct{}, jobs[i]))
            return set_error(G4_ERR_UNSUPPORTED, "GEMV plan: projection %d has no streaming class", i);
        const GeluEpilogue *e = epis ? &epis[i] : nullptr;
        if (!e || e->act_scale == 0.0f) continue;
        if (descs[i].out_kind != G4_KIND_I8 || descs[i].out_scale == 0.0f)
            return set_error(G4_ERR_INVALID, "GEMV plan: a gelu epilogue needs int8 gate codes");
        StreamJob &J = jobs[i];
        J.act_scale = e->act_scale;
        if (e->w_up) {
            if (descs[i].bits != 4)
                return set_error(G4_ERR_UNSUPPORTED, "GEMV plan: paired gate/up rows are 4-bit only");
            if (!e->s_up || (reinterpret_cast<uintptr_t>(e->w_up) & 15))
                return set_error(G4_ERR_INVALID,
                                 "GEMV plan: paired up weights need scales and 16-byte alignment");
            J.epi = 1;
            J.aux = e->w_up;
            J.aux_scales = e->s_up;
        } else {
            if (!e->up_vec)
                return set_error(G4_ERR_INVALID, "GEMV plan: a gelu epilogue needs an up operand");
            J.epi = 2;
            J.aux = e->up_vec;
        }
    }
    return plan_from_jobs(jobs, out);
}

int gemv_plan_set_first_tile_snap(g4_gemv_plan *p) {
    if (!p) return set_error(G4_ERR_INVALID, "GEMV plan: plan is NULL");
    p->first_tile_snap = true;
    return G4_OK;
}

int gemv_plan_set_prologue_join(g4_gemv_plan *p, const JoinTail &j) {
    if (!p) return set_error(G4_ERR_INVALID, "GEMV plan join: plan is NULL");
    if (!j.src || j.width <= 0 || j.width > kJoinMaxPer * kRowThreads || (j.width & 7))
        return set_error(G4_ERR_INVALID, "GEMV plan join: width %d (a multiple of 8, at most %d)",
                         j.width, kJoinMaxPer * kRowThreads);
    if (j.src_kind != G4_KIND_F32 && j.src_kind != G4_KIND_I8 && j.src_kind != G4_KIND_I32)
        return set_error(G4_ERR_INVALID, "GEMV plan join: src_kind must be f32, int8 codes or int32 partials");
    if (j.src_kind == G4_KIND_I32 && (!j.acc_scales || j.acc_splits != 1))
        return set_error(G4_ERR_INVALID, "GEMV plan join: an int32 accumulator source needs its scales and one split");
    if (!j.codes || j.in_scale == 0.0f)
        return set_error(G4_ERR_INVALID, "GEMV plan join: needs its codes and the consumer's inScale");
    if (j.resid && j.hidden == j.resid)
        return set_error(G4_ERR_INVALID,
                         "GEMV plan join: every block reads the residual, so the new row needs "
                         "its own buffer");
    // the projections read the join's codes from the join
    std::vector<StreamJob> jobs(p->njobs);
    G4_HIP(hipMemcpy(jobs.data(), p->table, sizeof(StreamJob) * p->njobs, hipMemcpyDeviceToHost));
    // (every job, with one bit width: a block snaps once, at its first tile)
    for (StreamJob &J : jobs) {
        if (J.x != j.codes || J.x_kind != G4_KIND_I8 || J.up || J.k != j.width ||
            J.in_scale != j.in_scale || J.bits != jobs[0].bits)
            return set_error(G4_ERR_INVALID,
                             "GEMV plan join: every projection of the plan must read the join's %d "
                             "int8 codes on its inScale, at one bit width, without a gelu prologue",
                             j.width);
        J.pre = 1;
    }
    G4_HIP(hipMemcpy(p->table, jobs.data(), sizeof(StreamJob) * p->njobs, hipMemcpyHostToDevice));
    if (!p->pre) G4_HIP(hipMalloc(&p->pre, sizeof(JoinTail)));
    G4_HIP(hipMemcpy(p->pre, &j, sizeof(JoinTail), hipMemcpyHostToDevice));
    return G4_OK;
}

}  // namespace g4

extern "C" {

int g4_qgemv_plan_create(const g4_gemv_desc *descs, int count, g4_gemv_plan **out) {
    return g4_qgemv_plan_create_gelu(descs, nullptr, count, out);
}

int g4_qgemv_plan_create_gelu(const g4_gemv_desc *descs, const g4_gelu_act *acts, int count,
                              g4_gemv_plan **out) {
    if (!out) return set_error(G4_ERR_INVALID, "g4_qgemv_plan_create: plan is NULL");
    *out = nullptr;
    if (!descs || count < 1)
        return set_error(G4_ERR_INVALID, "g4_qgemv_plan_create: needs at least one descriptor");
    std::vector<StreamJob> jobs(count);
    for (int i = 0; i < count; ++i) {
        if (acts && acts[i].up && acts[i].up_offset < 0)
            return set_error(G4_ERR_INVALID, "GEMV plan: projection %d has a negative upOffset", i);
        const GeluAct act = gelu_act_of(acts ? &acts[i] : nullptr);
        int rc = check_job_desc(descs[i], act, "GEMV plan");
        if (rc) return rc;
        if (!stream_job_from(descs[i], act, jobs[i]))
            return set_error(G4_ERR_UNSUPPORTED,
                             "GEMV plan: projection %d (bits %d, K %d, inScale %g) has no streaming "
                             "shape class; run it through g4_qgemv",
                             i, descs[i].bits, descs[i].k, (double)descs[i].in_scale);
    }
    return plan_from_jobs(jobs, out);
}

int g4_qgemv_plan_launch(const g4_gemv_plan *p, void *stream) {
    if (!p) return set_error(G4_ERR_INVALID, "g4_qgemv_plan_launch: plan is NULL");
    StreamArgs A{};
    A.table = p->table;
    A.block_job = p->block_job;
    A.block_tile = p->block_job + p->grid;
    A.njobs = p->njobs;
    A.total_tiles = p->total_tiles;
    A.pre = p->pre;
    // with a prologue join, the join's two reduction buffers follow the codes
    const size_t lds = (size_t)((p->max_k + 15) & ~15) + (p->pre ? 2 * kRowThreads * sizeof(float) : 0);
    const dim3 grid(p->grid), block(kStreamThreads);
    const hipStream_t st = as_stream(stream);
    const int mode = p->pre ? 1 : p->first_tile_snap ? 2 : 0;
    if (p->paired && mode == 1)
        hipLaunchKernelGGL((qgemv_stream_pair_kernel<true, 1>), grid, block, lds, st, A);
    else if (p->paired && mode == 2)
        hipLaunchKernelGGL((qgemv_stream_pair_kernel<true, 2>), grid, block, lds, st, A);
    else if (p->paired)
        hipLaunchKernelGGL((qgemv_stream_pair_kernel<true, 0>), grid, block, lds, st, A);
    else if (mode == 1)
        hipLaunchKernelGGL((qgemv_stream_kernel<true, 1>), grid, block, lds, st, A);
    else if (mode == 2)
        hipLaunchKernelGGL((qgemv_stream_kernel<true, 2>), grid, block, lds, st, A);
    else
        hipLaunchKernelGGL((qgemv_stream_kernel<true, 0>), grid, block, lds, st, A);
    G4_LAUNCHED("qgemv_stream_kernel");
    return G4_OK;
}

int g4_qgemv_plan_info(const g4_gemv_plan *p, int *tiles, int *grid) {
    if (!p) return set_error(G4_ERR_INVALID, "g4_qgemv_plan_info: plan is NULL");
    if (tiles) *tiles = p->total_tiles;
    if (grid) *grid = p->grid;
    return G4_OK;
}

int g4_qgemv_plan_destroy(g4_gemv_plan *p) {
    if (!p) return G4_OK;
    (void)hipFree(p->table);
    (void)hipFree(p->block_job);
    (void)hipFree(p->pre);
    delete p;
    return G4_OK;
}

}  // extern "C"

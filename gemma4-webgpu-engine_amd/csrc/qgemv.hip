// The decode GEMV family on gfx950: qgemv-4bit / qgemv-8bit (M = 1), the wide -m2 forms (M = 2),
// the projection batches (qkv / gate-up), the grouped layer GEMV, and the split-K build with its
// two folds (src/kernels/qgemv.ts, qgemvWide.ts, projectionBatch.ts, exactSplit.ts).
//
// Layout of one launch. A block is 256 threads = 4 wave64s. Each wave serves 4 output rows at a
// time, one per 16-lane DPP row, so a block covers 16 rows per pass and `passes` passes. A lane
// streams 16-byte chunks of its row (chunk lane16 + 16 t), so the 16 lanes of a row read 256
// contiguous bytes per load instruction and the 4 rows of a wave read 4 such runs.
//
// The calibrated (integer) path. The block snaps its activation columns once into LDS as int8
// codes (IEEE f32 divide, ties to even, clamp), and accumulates sum(u * xq) with v_dot4_i32_i8,
// where u = nibble in [0, 15] (4-bit) or the signed byte (8-bit). The 4-bit zero point comes off
// once per row as -8 * sum(xq), which is exact integer arithmetic: sum((u - 8) * x) =
// sum(u * x) - 8 sum(x). To dot a word's low nibbles [k0 k2 k4 k6] and high nibbles [k1 k3 k5 k7]
// without shuffling the weights, the LDS code layout interleaves each 8-code group as
// [x0 x2 x4 x6 | x1 x3 x5 x7]. The int32 row sum is exact (|sum| <= K * 8 * 128 < 2^31), so the
// order of the reduction does not matter, and the epilogue is the reference's expression.
//
// The uncalibrated (inScale == 0) path keeps the f32 code dot: per lane in k order, then the fixed
// 16-lane DPP tree (row16_sum_f32).
#include "g4_internal.h"

#include <algorithm>
#include <vector>

namespace g4 {

constexpr int kGemvThreads = 256;
constexpr int kRowsPerPass = 16;
constexpr int kMaxGemvK = 16384;
constexpr int kChunkBatch = 4;
constexpr int kMaxPasses = 8;

struct GemvJob {
    const uint8_t *w;
    const float *scales;
    const void *x;
    void *dst;
    int bits;
    int x_kind;
    int out_kind;
    int k;
    int rows;
    float in_scale;
    float out_scale;
    int wg_begin;
    int passes;
    int kwaves;  // waves splitting K inside a block: 1, 2 or 4
    GeluAct act; // the gelu prologue (act.up set): x is the gate
};

struct GemvLaunch {
    GemvJob job[G4_MAX_GROUP];
    int count;
    int splits;       // 1: plain GEMV. > 1: split-K partials (one job, one column)
    int split_exact;  // split only: 1 writes raw integer partials, 0 the scaled ones
    int split_layout; // split only: 0 [rows][splits]; 1 the PLE gate's row-interleaved layout
};

// Index of (row, split) in the partials: [rows][splits], or ple-gate-split's interleave
// dst[(row / 4) * 4 * splits + split * 4 + row % 4] (pleSplit.ts:17-23), which the fold reads as
// one vec4 per (4 rows, split).
__device__ __forceinline__ int64_t split_index(const GemvLaunch &L, int row, int split) {
    if (L.split_layout)
        return (int64_t)(row >> 2) * 4 * L.splits + split * 4 + (row & 3);
    return (int64_t)row * L.splits + split;
}

__device__ __forceinline__ uint32_t pack4(int a, int b, int c, int d) {
    return (uint32_t)(a & 0xff) | ((uint32_t)(b & 0xff) << 8) | ((uint32_t)(c & 0xff) << 16) |
           ((uint32_t)(d & 0xff) << 24);
}

// Band of the split-K cut in codes, mirroring qgemv.ts:521-548 at one word per lane: kIters whole
// 32-word iterations plus the guarded tail slot (always counted unless the partials are exact).
__device__ __forceinline__ void split_band(int k, int bits, int splits, int split, int exact,
                                           int &c_lo, int &c_hi) {
    if (splits <= 1) {
        c_lo = 0;
        c_hi = k;
        return;
    }
    int cpw = bits == 4 ? 8 : 4;
    int k_words = k / cpw;
    int k_iters = k_words / 32;
    int slots = k_iters + (exact ? ((k_words % 32) != 0 ? 1 : 0) : 1);
    int per = (slots + splits - 1) / splits;
    int lo = min(split * per, slots);
    int hi = min(lo + per, slots);
    int w_lo = lo * 32;
    int w_hi = min(hi, k_iters) * 32;
    if (hi > k_iters) w_hi = k_words;
    if (w_lo > w_hi) w_lo = w_hi;
    c_lo = w_lo * cpw;
    c_hi = w_hi * cpw;
}

__device__ __forceinline__ int find_job(const GemvLaunch &L, int b) {
    int j = 0;
#pragma unroll
    for (int i = 1; i < G4_MAX_GROUP; ++i)
        if (i < L.count && b >= L.job[i].wg_begin) j = i;
    return j;
}

// Snap 8 activations starting at element e (f32, f16 or ready int8 codes) into codes c[0..7].
__device__ __forceinline__ void load_codes8(const void *x, int kind, int64_t e, float s, float r,
                                            bool r_ok, int c[8]) {
    if (kind == G4_KIND_I8) {
        uint2 v = *reinterpret_cast<const uint2 *>(reinterpret_cast<const int8_t *>(x) + e);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            c[i] = (int)(int8_t)((v.x >> (8 * i)) & 0xff);
            c[4 + i] = (int)(int8_t)((v.y >> (8 * i)) & 0xff);
        }
    } else if (kind == G4_KIND_F16) {
        uint4 v = *reinterpret_cast<const uint4 *>(reinterpret_cast<const __half *>(x) + e);
        uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            __half lo = __ushort_as_half((unsigned short)(w[i] & 0xffff));
            __half hi = __ushort_as_half((unsigned short)(w[i] >> 16));
            c[2 * i] = (int)srq_code_fast(__half2float(lo), s, r, r_ok);
            c[2 * i + 1] = (int)srq_code_fast(__half2float(hi), s, r, r_ok);
        }
    } else {
        const float4 *p = reinterpret_cast<const float4 *>(reinterpret_cast<const float *>(x) + e);
        float4 a = p[0], b = p[1];
        c[0] = (int)srq_code_fast(a.x, s, r, r_ok);
        c[1] = (int)srq_code_fast(a.y, s, r, r_ok);
        c[2] = (int)srq_code_fast(a.z, s, r, r_ok);
        c[3] = (int)srq_code_fast(a.w, s, r, r_ok);
        c[4] = (int)srq_code_fast(b.x, s, r, r_ok);
        c[5] = (int)srq_code_fast(b.y, s, r, r_ok);
        c[6] = (int)srq_code_fast(b.z, s, r, r_ok);
        c[7] = (int)srq_code_fast(b.w, s, r, r_ok);
    }
}

// A 16-byte streaming load: weights are read once, so keep them from displacing cached data.
__device__ __forceinline__ u32x4 load16_stream(const uint8_t *p) {
    return __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
}

// Loads the 16-byte chunks [t0, t0 + kChunkBatch) of this lane (chunk index t * 16 + lane16 of the
// wave's chunk range), zero past the range.
__device__ __forceinline__ void load_batch(u32x4 (&dst)[kChunkBatch], const uint8_t *wrow, int t0,
                                           int T, int nchw, int lane16) {
#pragma unroll
    for (int u = 0; u < kChunkBatch; ++u) {
        const int t = t0 + u;
        const int ch = t * 16 + lane16;
        dst[u] = (t < T && ch < nchw) ? load16_stream(wrow + (int64_t)ch * 16) : u32x4{0, 0, 0, 0};
    }
}

// Accumulates one batch of chunks against the LDS codes (xl = this wave's first chunk's codes).
template <int COLS>
__device__ __forceinline__ void dot_batch(int (&acc)[COLS], const u32x4 (&w)[kChunkBatch],
                                          const uint8_t *xl0, int lds_stride, int bits, int t0,
                                          int T, int nchw, int lane16) {
#pragma unroll
    for (int u = 0; u < kChunkBatch; ++u) {
        const int t = t0 + u;
        const int ch = t * 16 + lane16;
        if (t < T && ch < nchw) {
            const uint32_t wv[4] = {w[u].x, w[u].y, w[u].z, w[u].w};
#pragma unroll
            for (int c = 0; c < COLS; ++c) {
                const uint8_t *xl = xl0 + c * lds_stride;
                int a = acc[c];
                if (bits == 4) {
                    const u32x4 xa = *reinterpret_cast<const u32x4 *>(xl + ch * 32);
                    const u32x4 xb = *reinterpret_cast<const u32x4 *>(xl + ch * 32 + 16);
                    const uint32_t xv[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const uint32_t lo = wv[i] & 0x0F0F0F0Fu;
                        const uint32_t hi = (wv[i] >> 4) & 0x0F0F0F0Fu;
                        a = __builtin_amdgcn_sdot4((int)lo, (int)xv[2 * i], a, false);
                        a = __builtin_amdgcn_sdot4((int)hi, (int)xv[2 * i + 1], a, false);
                    }
                } else {
                    const u32x4 xa = *reinterpret_cast<const u32x4 *>(xl + ch * 16);
                    a = __builtin_amdgcn_sdot4((int)wv[0], (int)xa.x, a, false);
                    a = __builtin_amdgcn_sdot4((int)wv[1], (int)xa.y, a, false);
                    a = __builtin_amdgcn_sdot4((int)wv[2], (int)xa.z, a, false);
                    a = __builtin_amdgcn_sdot4((int)wv[3], (int)xa.w, a, false);
                }
                acc[c] = a;
            }
        }
    }
}

// Block layout: wave w serves the 4-row group w / kwaves of each pass over the K part w % kwaves,
// so a block covers 16 / kwaves rows per pass. Long rows (K >= 3072) split K over the waves so
// every block streams about the same bytes; the parts fold through LDS integer atomics (exact).
// The first weight batch is requested before the activation snap, so the weight latency overlaps
// it.
template <int COLS>
__global__ __launch_bounds__(kGemvThreads) void qgemv_int_kernel(GemvLaunch L) {
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ int s_sum[COLS];
    __shared__ int s_acc[kMaxPasses * kRowsPerPass * COLS];

    const int j = find_job(L, blockIdx.x);
    const GemvJob &J = L.job[j];
    const int tid = threadIdx.x;
    const int bits = J.bits;
    const int k = J.k;
    const int split = blockIdx.y;
    int c_lo, c_hi;
    split_band(k, bits, L.splits, split, L.split_exact, c_lo, c_hi);
    const int kl = c_hi - c_lo;              // codes in this block's band
    const int lds_stride = (kl + 15) & ~15;  // bytes of codes per column in LDS

    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int lane16 = lane & 15;
    const int kwaves = J.kwaves;
    const int rows_per_pass = kRowsPerPass / kwaves;
    const int rgroup = wave / kwaves;
    const int kpart = wave - rgroup * kwaves;
    const int row_bytes = bits == 4 ? (k >> 1) : k;
    const int cpc = bits == 4 ? 32 : 16;  // codes per 16-byte chunk
    const int nch = kl / cpc;             // chunks of the band
    const int w_lo = (nch * kpart) / kwaves;
    const int nchw = (nch * (kpart + 1)) / kwaves - w_lo;  // chunks of this wave's part
    const int T = (nchw + 15) >> 4;
    const int block_row0 = (blockIdx.x - J.wg_begin) * (J.passes * rows_per_pass);
    const int64_t band_off = (int64_t)(c_lo / cpc + w_lo) * 16;

    auto row_of = [&](int p) { return block_row0 + p * rows_per_pass + rgroup * 4 + (lane >> 4); };
    auto wrow_of = [&](int p) {
        return J.w + (int64_t)min(row_of(p), J.rows - 1) * row_bytes + band_off;
    };

    // Request pass 0's first weight batch before touching the activations.
    u32x4 cur[kChunkBatch];
    load_batch(cur, wrow_of(0), 0, T, nchw, lane16);

    for (int i = tid; i < kMaxPasses * kRowsPerPass * COLS; i += kGemvThreads) s_acc[i] = 0;
    if (tid < COLS) s_sum[tid] = 0;
    __syncthreads();

    // ---- snap the activation band into LDS (once per block) ----
    {
        bool r_ok;
        const float r = srq_recip(J.in_scale, r_ok);
        const int groups = kl >> 3;
        int local = 0;
        for (int g = tid; g < groups * COLS; g += kGemvThreads) {
            const int col = COLS == 1 ? 0 : g / groups;
            const int gi = COLS == 1 ? g : g - col * groups;
            int c[8];
            const int64_t e = (int64_t)col * k + c_lo + gi * 8;
            if (J.act.fold_parts)
                fold_gelu_codes8(J.act, e, J.in_scale, r, r_ok, c);
            else if (J.act.up)
                gelu_codes8(J.x, J.x_kind, J.act.g_scale, J.act.up, J.act.up_kind, J.act.u_scale, e,
                            J.in_scale, r, r_ok, c);
            else
                load_codes8(J.x, J.x_kind, e, J.in_scale, r, r_ok, c);
            uint2 packed;
            if (bits == 4) {
                packed.x = pack4(c[0], c[2], c[4], c[6]);
                packed.y = pack4(c[1], c[3], c[5], c[7]);
            } else {
                packed.x = pack4(c[0], c[1], c[2], c[3]);
                packed.y = pack4(c[4], c[5], c[6], c[7]);
            }
            *reinterpret_cast<uint2 *>(smem + col * lds_stride + gi * 8) = packed;
            const int sum8 = c[0] + c[1] + c[2] + c[3] + c[4] + c[5] + c[6] + c[7];
            if (COLS == 1)
                local += sum8;
            else
                atomicAdd(&s_sum[col], sum8);
        }
        if (COLS == 1) {
            local = row16_sum_i32(local);
            if ((tid & 15) == 0 && local != 0) atomicAdd(&s_sum[0], local);
        }
    }
    lds_barrier();

    int sx[COLS];
#pragma unroll
    for (int c = 0; c < COLS; ++c) sx[c] = s_sum[c];
    const uint8_t *xl0 = smem + (int64_t)w_lo * (bits == 4 ? 32 : 16);

    for (int p = 0; p < J.passes; ++p) {
        const bool active = block_row0 + p * rows_per_pass + rgroup * 4 < J.rows;  // wave-uniform
        const int row = row_of(p);
        int acc[COLS];
#pragma unroll
        for (int c = 0; c < COLS; ++c) acc[c] = 0;
        if (active) {
            const uint8_t *wrow = wrow_of(p);
            for (int t0 = 0; t0 < T; t0 += kChunkBatch) {
                u32x4 nxt[kChunkBatch];
                load_batch(nxt, wrow, t0 + kChunkBatch, T, nchw, lane16);
                dot_batch<COLS>(acc, cur, xl0, lds_stride, bits, t0, T, nchw, lane16);
#pragma unroll
                for (int u = 0; u < kChunkBatch; ++u) cur[u] = nxt[u];
            }
        }
        if (p + 1 < J.passes) load_batch(cur, wrow_of(p + 1), 0, T, nchw, lane16);
#pragma unroll
        for (int c = 0; c < COLS; ++c) acc[c] = row16_sum_i32(acc[c]);
        if (!active || lane16 != 0 || row >= J.rows) continue;
        if (kwaves > 1) {
            const int slot = p * kRowsPerPass + rgroup * 4 + (lane >> 4);
#pragma unroll
            for (int c = 0; c < COLS; ++c) atomicAdd(&s_acc[slot * COLS + c], acc[c]);
            continue;
        }
        const float scale = J.scales[row];
#pragma unroll
        for (int c = 0; c < COLS; ++c) {
            const int s = bits == 4 ? acc[c] - 8 * sx[c] : acc[c];
            if (L.splits > 1) {
                const float part = L.split_exact ? (float)s : linear_epilogue(J.in_scale, scale, (float)s);
                reinterpret_cast<float *>(J.dst)[split_index(L, row, split)] = part;
            } else {
                const float y = linear_epilogue(J.in_scale, scale, (float)s);
                store_linear_out(J.dst, (int64_t)c * J.rows + row, J.out_kind, y, s, J.out_scale);
            }
        }
    }
    if (kwaves > 1) {
        __syncthreads();
        const int n_out = J.passes * rows_per_pass;
        for (int i = tid; i < n_out * COLS; i += kGemvThreads) {
            const int local_row = i / COLS;
            const int c = i - local_row * COLS;
            const int p = local_row / rows_per_pass;
            const int r_in = local_row - p * rows_per_pass;
            const int row = block_row0 + local_row;
            if (row >= J.rows) continue;
            const int acc = s_acc[(p * kRowsPerPass + r_in) * COLS + c];
            const int s = bits == 4 ? acc - 8 * sx[c] : acc;
            const float scale = J.scales[row];
            if (L.splits > 1) {
                const float part = L.split_exact ? (float)s : linear_epilogue(J.in_scale, scale, (float)s);
                reinterpret_cast<float *>(J.dst)[split_index(L, row, split)] = part;
            } else {
                const float y = linear_epilogue(J.in_scale, scale, (float)s);
                store_linear_out(J.dst, (int64_t)c * J.rows + row, J.out_kind, y, s, J.out_scale);
            }
        }
    }
}

// The uncalibrated f32 code dot (inScale == 0, qgemv.ts:666-675): x stays f32 in LDS, each lane
// sums code * x over its chunks in k order (separate rounded multiply and add), then the 16-lane
// tree. One column per blockIdx.z. Parity against the reference's order is unpinned beyond the
// exact-grid fixtures (the reference's own f32 order is adapter dependent).
__global__ __launch_bounds__(kGemvThreads) void qgemv_f32_kernel(GemvLaunch L) {
    extern __shared__ __align__(16) uint8_t smem[];
    float *xs = reinterpret_cast<float *>(smem);
    const int j = find_job(L, blockIdx.x);
    const GemvJob &J = L.job[j];
    const int tid = threadIdx.x;
    const int k = J.k;
    const int col = blockIdx.z;
    for (int i = tid; i < k; i += kGemvThreads) {
        const int64_t e = (int64_t)col * k + i;
        xs[i] = J.act.up ? gelu_act_value(J.act, J.x, J.x_kind, e) : load_act(J.x, J.x_kind, e);
    }
    __syncthreads();
    const int lane = tid & 63, wave = tid >> 6, lane16 = lane & 15;
    const int bits = J.bits;
    const int row_bytes = bits == 4 ? (k >> 1) : k;
    const int cpc = bits == 4 ? 32 : 16;
    const int nch = k / cpc;
    const int row_block = (blockIdx.x - J.wg_begin) * (J.passes * kRowsPerPass);
    for (int p = 0; p < J.passes; ++p) {
        const int wave_row0 = row_block + p * kRowsPerPass + wave * 4;
        if (wave_row0 >= J.rows) break;
        const int row = wave_row0 + (lane >> 4);
        const int rrow = min(row, J.rows - 1);
        const uint8_t *wrow = J.w + (int64_t)rrow * row_bytes;
        float acc = 0.0f;
        for (int ch = lane16; ch < nch; ch += 16) {
            const uint4 v = *reinterpret_cast<const uint4 *>(wrow + (int64_t)ch * 16);
            const uint32_t wv[4] = {v.x, v.y, v.z, v.w};
            const float *xc = xs + ch * cpc;
            if (bits == 4) {
#pragma unroll
                for (int i = 0; i < 32; ++i) {
                    const int code = (int)((wv[i >> 3] >> (4 * (i & 7))) & 0xf) - 8;
                    acc = __fadd_rn(acc, __fmul_rn((float)code, xc[i]));
                }
            } else {
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const int code = (int)(int8_t)((wv[i >> 2] >> (8 * (i & 3))) & 0xff);
                    acc = __fadd_rn(acc, __fmul_rn((float)code, xc[i]));
                }
            }
        }
        const float sum = row16_sum_f32(acc);
        if (lane16 == 0 && row < J.rows) {
            const float y = linear_epilogue(1.0f, J.scales[row], sum);
            store_linear_out(J.dst, (int64_t)col * J.rows + row, J.out_kind, y, 0, J.out_scale);
        }
    }
}

// qgemv-merge (qgemv.ts:1027-1072) and qgemv-exact-merge (exactSplit.ts:45-57).
__global__ void qgemv_merge_kernel(const float *part, const float *scales, void *dst, int out_kind,
                                   int rows, int splits, int exact, float in_scale,
                                   float out_scale) {
    const int row = blockIdx.x * blockDim.x + threadIdx.x;
    if (row >= rows) return;
    float t = 0.0f;
    for (int s = 0; s < splits; ++s) t = __fadd_rn(t, part[(int64_t)row * splits + s]);
    const float y = exact ? linear_epilogue(in_scale, scales[row], t) : t;
    store_linear_out(dst, row, out_kind, y, 0, out_scale);
}

// ---- host side ----------------------------------------------------------------------------------

static bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// Validates one job against what the kernels assume (shape, alignment, kinds). `who` names the
// registry kernel in the message.
int check_job(const GemvJob &J, int cols, const char *who) {
    if (!J.w || !J.scales || !J.x || !J.dst)
        return set_error(G4_ERR_INVALID, "%s needs inputs named wq, scales and x, and an output", who);
    if (J.bits != 4 && J.bits != 8)
        return set_error(G4_ERR_INVALID, "%s: bits must be 4 or 8, got %d", who, J.bits);
    if (J.k <= 0 || J.rows <= 0)
        return set_error(G4_ERR_INVALID, "%s needs params.k and params.numRows", who);
    const int cpc = J.bits == 4 ? 32 : 16;
    if (J.k % cpc != 0)
        return set_error(G4_ERR_INVALID, "%s: K %d does not fill whole 16-byte chunks", who, J.k);
    if (J.k > kMaxGemvK)
        return set_error(G4_ERR_INVALID, "%s: K %d exceeds %d (the exact int32/f32 bound)", who, J.k,
                         kMaxGemvK);
    if (J.x_kind != G4_KIND_F32 && J.x_kind != G4_KIND_F16 && J.x_kind != G4_KIND_I8)
        return set_error(G4_ERR_INVALID, "%s: x_kind %d is not f32, f16 or int8", who, J.x_kind);
    if (J.out_kind != G4_KIND_F32 && J.out_kind != G4_KIND_I8 && J.out_kind != G4_KIND_I32)
        return set_error(G4_ERR_INVALID, "%s: out_kind %d is not f32, int8 or int32", who,
                         J.out_kind);
    if (J.out_kind == G4_KIND_I8 && J.out_scale == 0.0f)
        return set_error(G4_ERR_INVALID,
                         "%s: int8 output codes need a calibrated outScale (0.0 means no output snap)",
                         who);
    if (J.in_scale == 0.0f && (J.x_kind == G4_KIND_I8 || J.out_kind == G4_KIND_I32))
        return set_error(G4_ERR_INVALID,
                         "%s: inScale 0.0 is the uncalibrated f32 path, which has no int8 input codes "
                         "and no integer accumulator", who);
    if (!std::isfinite(J.in_scale) || !std::isfinite(J.out_scale))
        return set_error(G4_ERR_INVALID, "%s: scales must be finite", who);
    if (!aligned16(J.w) || !aligned16(J.x))
        return set_error(G4_ERR_INVALID, "%s: wq and x must be 16-byte aligned", who);
    if (cols < 1 || cols > 2) return set_error(G4_ERR_INVALID, "%s: cols %d not in 1..2", who, cols);
    if (J.act.up) {
        // qgemv.ts:359-400 (and the wide form, qgemvWide.ts:193-283): the prologue binds gate and
        // up in place of x; on an uncalibrated site the f32 code dot reads the product unsnapped
        if (J.act.fold_parts) {
            // pleSplit.ts:24-41: the gate is the fold of the split partials, one token
            if (cols != 1) return set_error(G4_ERR_INVALID, "PLE split needs one token");
            if (J.act.fold_splits != 2 && J.act.fold_splits != 4 && J.act.fold_splits != 8)
                return set_error(G4_ERR_INVALID, "PLE splits must be 1, 2, 4 or 8");
            if (!J.act.fold_scales)
                return set_error(G4_ERR_INVALID, "%s needs inputs named gate, up and gateScales", who);
            if (!aligned16(J.act.fold_parts) || !aligned16(J.act.fold_scales))
                return set_error(G4_ERR_INVALID, "%s: gate partials and gateScales must be 16-byte aligned", who);
            if (!std::isfinite(J.act.fold_in) || !std::isfinite(J.act.fold_out))
                return set_error(G4_ERR_INVALID, "%s: gateInScale and gateOutScale must be finite", who);
        }
        if (J.x_kind != G4_KIND_F32 && J.x_kind != G4_KIND_I8)
            return set_error(G4_ERR_INVALID, "%s: gate must be f32 or int8 codes", who);
        if (J.act.up_kind != G4_KIND_F32 && J.act.up_kind != G4_KIND_I8)
            return set_error(G4_ERR_INVALID, "%s: up must be f32 or int8 codes", who);
        const uintptr_t need_up = J.act.up_kind == G4_KIND_F32 ? 15 : 7;
        if (reinterpret_cast<uintptr_t>(J.act.up) & need_up)
            return set_error(G4_ERR_INVALID, "%s: up (after upOffset) must be %d-byte aligned", who,
                             (int)need_up + 1);
        if ((J.x_kind == G4_KIND_I8 && !std::isfinite(J.act.g_scale)) ||
            (J.act.up_kind == G4_KIND_I8 && !std::isfinite(J.act.u_scale)))
            return set_error(G4_ERR_INVALID, "%s: gate and up scales must be finite", who);
    }
    return G4_OK;
}

GeluAct gelu_act_of(const g4_gelu_act *a) {
    GeluAct g;
    if (!a || !a->up) return g;
    const size_t elem = a->up_kind == G4_KIND_I8 ? 1 : 4;
    g.up = reinterpret_cast<const uint8_t *>(a->up) + (size_t)a->up_offset * elem;
    g.up_kind = a->up_kind;
    g.g_scale = a->gate_scale;
    g.u_scale = a->up_scale;
    return g;
}

static g4_gemv_desc desc_of(const GemvJob &J) {
    g4_gemv_desc d{};
    d.wq = J.w;
    d.scales = J.scales;
    d.x = J.x;
    d.dst = J.dst;
    d.bits = J.bits;
    d.x_kind = J.x_kind;
    d.out_kind = J.out_kind;
    d.k = J.k;
    d.num_rows = J.rows;
    d.in_scale = J.in_scale;
    d.out_scale = J.out_scale;
    return d;
}

static GemvJob job_of(const g4_gemv_desc &d) {
    GemvJob J{};
    J.w = reinterpret_cast<const uint8_t *>(d.wq);
    J.scales = d.scales;
    J.x = d.x;
    J.dst = d.dst;
    J.bits = d.bits;
    J.x_kind = d.x_kind;
    J.out_kind = d.out_kind;
    J.k = d.k;
    J.rows = d.num_rows;
    J.in_scale = d.in_scale;
    J.out_scale = d.out_scale;
    return J;
}

int check_job_desc(const g4_gemv_desc &d, const GeluAct &act, const char *who) {
    GemvJob J = job_of(d);
    J.act = act;
    return check_job(J, 1, who);
}

// Single-column launches of calibrated jobs go to the streaming kernel when their shapes allow.
static int try_stream(const GemvLaunch &L, int cols, hipStream_t stream, bool *launched) {
    *launched = false;
    if (cols != 1 || L.splits > 1) return G4_OK;
    g4_gemv_desc d[G4_MAX_GROUP];
    GeluAct a[G4_MAX_GROUP];
    for (int i = 0; i < L.count; ++i) {
        if (L.job[i].act.fold_parts) return G4_OK;  // the fold prologue runs on qgemv_int_kernel
        d[i] = desc_of(L.job[i]);
        a[i] = L.job[i].act;
    }
    return stream_try_launch(d, a, L.count, stream, launched);
}

// Waves splitting K in a block: long rows split so every block streams about the same bytes.
static int kwaves_for(int k) { return k >= 6144 ? 4 : k >= 3072 ? 2 : 1; }

static int rows_per_block(const GemvJob &J) { return J.passes * (kRowsPerPass / J.kwaves); }

// Picks passes per block so the launch offers a few blocks per CU without starving small jobs.
static void plan_blocks(GemvLaunch &L, int max_passes, bool split_k_waves) {
    int64_t total_groups = 0;
    for (int i = 0; i < L.count; ++i) {
        L.job[i].kwaves = split_k_waves ? kwaves_for(L.job[i].k) : 1;
        total_groups += (L.job[i].rows + kRowsPerPass / L.job[i].kwaves - 1) /
                        (kRowsPerPass / L.job[i].kwaves);
    }
    const int64_t target_blocks = 8LL * device_cu_count();
    int passes = 1;
    while (passes < max_passes && total_groups / passes > target_blocks) passes *= 2;
    int wg = 0;
    for (int i = 0; i < L.count; ++i) {
        L.job[i].passes = passes;
        L.job[i].wg_begin = wg;
        wg += (L.job[i].rows + rows_per_block(L.job[i]) - 1) / rows_per_block(L.job[i]);
    }
}

static int total_blocks(const GemvLaunch &L) {
    const GemvJob &last = L.job[L.count - 1];
    return last.wg_begin + (last.rows + rows_per_block(last) - 1) / rows_per_block(last);
}

// Launches the integer or f32 GEMV over L.count jobs with `cols` token columns (1 or 2).
int launch_gemv(GemvLaunch &L, int cols, hipStream_t stream) {
    if (L.count < 1 || L.count > G4_MAX_GROUP)
        return set_error(G4_ERR_INVALID, "grouped GEMV: count %d not in 1..%d", L.count, G4_MAX_GROUP);
    const bool calibrated = L.job[0].in_scale != 0.0f;
    for (int i = 1; i < L.count; ++i)
        if ((L.job[i].in_scale != 0.0f) != calibrated)
            return set_error(G4_ERR_UNSUPPORTED,
                             "grouped GEMV: calibrated and uncalibrated projections in one launch");
    if (L.splits > 1 && (L.count != 1 || cols != 1 || !calibrated))
        return set_error(G4_ERR_UNSUPPORTED, "split-K needs one calibrated single-column job");
    if (calibrated) {
        bool launched = false;
        int rc = try_stream(L, cols, stream, &launched);
        if (rc || launched) return rc;
    }
    plan_blocks(L, L.splits > 1 ? 1 : kMaxPasses, calibrated);
    const int blocks = total_blocks(L);
    int max_k = 0;
    for (int i = 0; i < L.count; ++i) max_k = std::max(max_k, L.job[i].k);
    if (calibrated) {
        const size_t lds = (size_t)cols * ((max_k + 15) & ~15);
        dim3 grid(blocks, std::max(1, L.splits), 1);
        if (cols == 1)
            hipLaunchKernelGGL(qgemv_int_kernel<1>, grid, dim3(kGemvThreads), lds, stream, L);
        else
            hipLaunchKernelGGL(qgemv_int_kernel<2>, grid, dim3(kGemvThreads), lds, stream, L);
        G4_LAUNCHED("qgemv_int_kernel");
    } else {
        const size_t lds = (size_t)max_k * sizeof(float);
        dim3 grid(blocks, 1, cols);
        hipLaunchKernelGGL(qgemv_f32_kernel, grid, dim3(kGemvThreads), lds, stream, L);
        G4_LAUNCHED("qgemv_f32_kernel");
    }
    return G4_OK;
}

// One GEMV job over m_cols columns, issued as launches of at most 2 columns (the wide kernel).
int gemv_columns(int bits, const void *wq, const float *scales, const void *x, int x_kind,
                 void *dst, int out_kind, int k, int num_rows, int m_cols, float in_scale,
                 float out_scale, hipStream_t stream, const char *who) {
    const size_t x_elem = x_kind == G4_KIND_F32 ? 4 : x_kind == G4_KIND_F16 ? 2 : 1;
    const size_t d_elem = out_kind == G4_KIND_I8 ? 1 : 4;
    for (int c0 = 0; c0 < m_cols; c0 += 2) {
        const int cols = std::min(2, m_cols - c0);
        GemvLaunch L{};
        L.count = 1;
        L.splits = 1;
        GemvJob &J = L.job[0];
        J.w = reinterpret_cast<const uint8_t *>(wq);
        J.scales = scales;
        J.x = reinterpret_cast<const uint8_t *>(x) + (size_t)c0 * k * x_elem;
        J.dst = reinterpret_cast<uint8_t *>(dst) + (size_t)c0 * num_rows * d_elem;
        J.bits = bits;
        J.x_kind = x_kind;
        J.out_kind = out_kind;
        J.k = k;
        J.rows = num_rows;
        J.in_scale = in_scale;
        J.out_scale = out_scale;
        int rc = check_job(J, cols, who);
        if (rc) return rc;
        rc = launch_gemv(L, cols, stream);
        if (rc) return rc;
    }
    return G4_OK;
}

}  // namespace g4

using namespace g4;

extern "C" {

// qgemv-4bit / qgemv-8bit / -m2 (qgemv.ts:1299-1363, qgemvWide.ts:515-574).
int g4_qgemv(int bits, const void *wq, const float *scales, const void *x, int x_kind, void *dst,
             int out_kind, int k, int num_rows, int cols, float in_scale, float out_scale,
             void *stream) {
    char who[32];
    snprintf(who, sizeof who, "qgemv-%dbit%s", bits, cols > 1 ? "-m2" : "");
    if (k <= 0 || num_rows <= 0) return set_error(G4_ERR_INVALID, "qgemv needs params.k and params.numRows");
    if (bits != 4 && bits != 8) return set_error(G4_ERR_INVALID, "qgemv: bits must be 4 or 8, got %d", bits);
    const int span = bits == 4 ? 256 : 128;  // K_SPAN_PER_ITER, qgemv.ts:1258
    if (k % span != 0)
        return set_error(G4_ERR_INVALID,
                         "qgemv-%dbit needs K a multiple of %d, got %d. Every text tensor satisfies "
                         "this; a caller that does not is packing the wrong tensor.",
                         bits, span, k);
    if (cols <= 0 || cols > 2)
        return set_error(G4_ERR_INVALID, "%s needs params.cols in 1..2, got %d", who, cols);
    return gemv_columns(bits, wq, scales, x, x_kind, dst, out_kind, k, num_rows, cols, in_scale,
                        out_scale, as_stream(stream), who);
}

// qkv-batch-4bit / gate-up-batch-4bit (projectionBatch.ts:85-128).
int g4_projection_batch(int bits, int count, const void *const *w, const float *const *scales,
                        const void *x, int x_kind, void *const *out, int out_kind, const int *rows,
                        const float *in_scales, const float *out_scales, int k, void *stream) {
    if (count != 2 && count != 3)
        return set_error(G4_ERR_INVALID, "projection batch count must be 2 (gate/up) or 3 (q/k/v), got %d", count);
    if (k <= 0 || k % 128 != 0)
        return set_error(G4_ERR_INVALID, "batched projection K must be a positive multiple of 128");
    if (!w || !scales || !out || !rows || !in_scales || !out_scales || !x)
        return set_error(G4_ERR_INVALID, "batched projection is missing an input buffer");
    for (int i = 0; i < count; ++i)
        if (rows[i] <= 0) return set_error(G4_ERR_INVALID, "batched projection rows must be positive integers");
    if (count == 2 && rows[0] != rows[1])
        return set_error(G4_ERR_INVALID, "gate/up batch requires equal row counts");
    GemvLaunch L{};
    L.count = count;
    L.splits = 1;
    const char *who = count == 3 ? "qkv-batch-4bit" : "gate-up-batch-4bit";
    for (int i = 0; i < count; ++i) {
        GemvJob &J = L.job[i];
        J.w = reinterpret_cast<const uint8_t *>(w[i]);
        J.scales = scales[i];
        J.x = x;
        J.dst = out[i];
        J.bits = bits;
        J.x_kind = x_kind;
        J.out_kind = out_kind;
        J.k = k;
        J.rows = rows[i];
        J.in_scale = in_scales[i];
        J.out_scale = out_scales[i];
        int rc = check_job(J, 1, who);
        if (rc) return rc;
    }
    // A mix of calibrated and uncalibrated projections (the reference's cases mix them) runs as
    // one launch per side.
    bool mixed = false;
    for (int i = 1; i < count; ++i) mixed |= (L.job[i].in_scale != 0.0f) != (L.job[0].in_scale != 0.0f);
    if (!mixed) return launch_gemv(L, 1, as_stream(stream));
    for (int side = 0; side < 2; ++side) {
        GemvLaunch S{};
        S.splits = 1;
        for (int i = 0; i < count; ++i)
            if ((L.job[i].in_scale != 0.0f) == (side == 0)) S.job[S.count++] = L.job[i];
        if (S.count) {
            int rc = launch_gemv(S, 1, as_stream(stream));
            if (rc) return rc;
        }
    }
    return G4_OK;
}

int g4_qgemv_grouped(const g4_gemv_desc *descs, int count, void *stream) {
    if (!descs || count < 1 || count > G4_MAX_GROUP)
        return set_error(G4_ERR_INVALID, "grouped GEMV: count %d not in 1..%d", count, G4_MAX_GROUP);
    GemvLaunch L{};
    L.count = count;
    L.splits = 1;
    for (int i = 0; i < count; ++i) {
        const g4_gemv_desc &d = descs[i];
        GemvJob &J = L.job[i];
        J.w = reinterpret_cast<const uint8_t *>(d.wq);
        J.scales = d.scales;
        J.x = d.x;
        J.dst = d.dst;
        J.bits = d.bits;
        J.x_kind = d.x_kind;
        J.out_kind = d.out_kind;
        J.k = d.k;
        J.rows = d.num_rows;
        J.in_scale = d.in_scale;
        J.out_scale = d.out_scale;
        int rc = check_job(J, 1, "grouped GEMV");
        if (rc) return rc;
        if (d.in_scale == 0.0f)
            return set_error(G4_ERR_UNSUPPORTED, "grouped GEMV runs calibrated projections only");
    }
    return launch_gemv(L, 1, as_stream(stream));
}

// qgemv-4bit-split / qgemv-8bit-split / exact split (qgemv.ts:521-548, exactSplit.ts:19-31).
int g4_qgemv_split(int bits, const void *wq, const float *scales, const void *x, int x_kind,
                   float *partials, int k, int num_rows, int k_splits, int exact, float in_scale,
                   void *stream) {
    if (k_splits != 1 && k_splits != 2 && k_splits != 4 && k_splits != 8)
        return set_error(G4_ERR_INVALID, "gemv geometry: kSplits must be 1, 2, 4 or 8, got %d", k_splits);
    if (exact && (!(in_scale > 0.0f) || k > 16384))
        return set_error(G4_ERR_INVALID, "exact split needs calibrated int8 input and K <= 16384");
    if (in_scale == 0.0f)
        return set_error(G4_ERR_UNSUPPORTED, "the split-K build runs the calibrated path only");
    const int span = bits == 4 ? 256 : 128;
    if (k <= 0 || num_rows <= 0) return set_error(G4_ERR_INVALID, "qgemv needs params.k and params.numRows");
    if (k % span != 0)
        return set_error(G4_ERR_INVALID, "qgemv-%dbit needs K a multiple of %d, got %d", bits, span, k);
    GemvLaunch L{};
    L.count = 1;
    L.splits = k_splits;
    L.split_exact = exact ? 1 : 0;
    GemvJob &J = L.job[0];
    J.w = reinterpret_cast<const uint8_t *>(wq);
    J.scales = scales;
    J.x = x;
    J.dst = partials;
    J.bits = bits;
    J.x_kind = x_kind;
    J.out_kind = G4_KIND_F32;
    J.k = k;
    J.rows = num_rows;
    J.in_scale = in_scale;
    J.out_scale = 0.0f;
    int rc = check_job(J, 1, bits == 4 ? "qgemv-4bit-split" : "qgemv-8bit-split");
    if (rc) return rc;
    return launch_gemv(L, 1, as_stream(stream));
}

// qgemv-4bit-gelu / qgemv-8bit-gelu, their -m2 forms, the gelu exact split and the PLE fold
// projection (qgemv.ts:359-400, 1668-1696; qgemvWide.ts:660-709; exactSplit.ts:19-31;
// pleSplit.ts:24-84): the GEMV or split build with the prologue reading gate and up. `fold` (may be
// null) makes the gate the fold of ple-gate-split's partials; `gate` is then those partials.
static int gelu_gemv(int bits, const void *wq, const float *scales, const void *gate,
                     int gate_kind, const g4_gelu_act *act, const GeluAct *fold, void *dst,
                     int out_kind, int k, int num_rows, int cols, int k_splits, int exact,
                     float in_scale, float out_scale, void *stream, const char *who) {
    const bool split = k_splits > 0;
    if (!act || !act->up) return set_error(G4_ERR_INVALID, "%s needs inputs named gate and up", who);
    if (bits != 4 && bits != 8) return set_error(G4_ERR_INVALID, "%s: bits must be 4 or 8", who);
    if (k <= 0 || num_rows <= 0) return set_error(G4_ERR_INVALID, "%s needs params.k and params.numRows", who);
    if (cols <= 0 || cols > 2)
        return set_error(G4_ERR_INVALID, "%s needs params.cols in 1..2, got %d", who, cols);
    const int span = bits == 4 ? 256 : 128;
    if (k % span != 0)
        return set_error(G4_ERR_INVALID, "%s needs K a multiple of %d, got %d", who, span, k);
    if (act->up_offset < 0) return set_error(G4_ERR_INVALID, "%s: upOffset must be >= 0", who);
    if (split && k_splits != 1 && k_splits != 2 && k_splits != 4 && k_splits != 8)
        return set_error(G4_ERR_INVALID, "gemv geometry: kSplits must be 1, 2, 4 or 8, got %d", k_splits);
    if (split && exact && (!(in_scale > 0.0f) || k > 16384))
        return set_error(G4_ERR_INVALID, "exact split needs calibrated int8 input and K <= 16384");
    if (split && in_scale == 0.0f)
        return set_error(G4_ERR_UNSUPPORTED, "the split-K build runs the calibrated path only");
    GemvLaunch L{};
    L.count = 1;
    L.splits = split ? k_splits : 1;
    L.split_exact = split && exact ? 1 : 0;
    GemvJob &J = L.job[0];
    J.w = reinterpret_cast<const uint8_t *>(wq);
    J.scales = scales;
    J.x = gate;
    J.dst = dst;
    J.bits = bits;
    J.x_kind = gate_kind;
    J.out_kind = split ? G4_KIND_F32 : out_kind;
    J.k = k;
    J.rows = num_rows;
    J.in_scale = in_scale;
    J.out_scale = split ? 0.0f : out_scale;
    J.act = gelu_act_of(act);
    if (fold) {
        J.act.fold_parts = fold->fold_parts;
        J.act.fold_scales = fold->fold_scales;
        J.act.fold_splits = fold->fold_splits;
        J.act.fold_in = fold->fold_in;
        J.act.fold_out = fold->fold_out;
    }
    int rc = check_job(J, cols, who);
    if (rc) return rc;
    return launch_gemv(L, cols, as_stream(stream));
}

int g4_qgemv_gelu(int bits, const void *wq, const float *scales, const void *gate, int gate_kind,
                  const g4_gelu_act *act, void *dst, int out_kind, int k, int num_rows,
                  float in_scale, float out_scale, void *stream) {
    char who[32];
    snprintf(who, sizeof who, "qgemv-%dbit-gelu", bits);
    return gelu_gemv(bits, wq, scales, gate, gate_kind, act, nullptr, dst, out_kind, k, num_rows,
                     1, 0, 0, in_scale, out_scale, stream, who);
}

// qgemv-4bit-gelu-m2 / qgemv-8bit-gelu-m2 (qgemvWide.ts:660-669, 698-709; bindGemvWide :515-574).
int g4_qgemv_gelu_m2(int bits, const void *wq, const float *scales, const void *gate, int gate_kind,
                     const g4_gelu_act *act, void *dst, int out_kind, int k, int num_rows, int cols,
                     float in_scale, float out_scale, void *stream) {
    char who[32];
    snprintf(who, sizeof who, "qgemv-%dbit-gelu-m2", bits);
    return gelu_gemv(bits, wq, scales, gate, gate_kind, act, nullptr, dst, out_kind, k, num_rows,
                     cols, 0, 0, in_scale, out_scale, stream, who);
}

int g4_qgemv_gelu_split(int bits, const void *wq, const float *scales, const void *gate,
                        int gate_kind, const g4_gelu_act *act, float *partials, int k,
                        int num_rows, int k_splits, int exact, float in_scale, void *stream) {
    if (k_splits < 1)
        return set_error(G4_ERR_INVALID, "gemv geometry: kSplits must be 1, 2, 4 or 8, got %d", k_splits);
    char who[40];
    snprintf(who, sizeof who, "qgemv-%dbit-gelu%s", bits, exact ? "-exact-split" : "-split");
    return gelu_gemv(bits, wq, scales, gate, gate_kind, act, nullptr, partials, G4_KIND_F32, k,
                     num_rows, 1, k_splits, exact, in_scale, 0.0f, stream, who);
}

// pleSplit.ts:10-16: the split count the two PLE kernels run (pleGateSplits(), 1 runs as 2).
static int ple_active_splits(int k_splits) { return k_splits == 1 ? 2 : k_splits; }

// ple-gate-split (pleSplit.ts:17-23, bind :50-63).
int g4_ple_gate_split(const void *wq, const float *scales, const void *x, int x_kind,
                      float *partials, int k, int num_rows, int k_splits, float in_scale,
                      void *stream) {
    if (k_splits != 1 && k_splits != 2 && k_splits != 4 && k_splits != 8)
        return set_error(G4_ERR_INVALID, "PLE splits must be 1, 2, 4 or 8");
    if (num_rows % 4 != 0)
        return set_error(G4_ERR_INVALID, "PLE split row count must be divisible by four");
    if (!(in_scale > 0.0f)) return set_error(G4_ERR_INVALID, "PLE split needs calibrated input");
    if (k <= 0 || num_rows <= 0)
        return set_error(G4_ERR_INVALID, "ple-gate-split needs params.k and params.numRows");
    if (k % 128 != 0)
        return set_error(G4_ERR_INVALID, "qgemv-8bit needs K a multiple of 128, got %d", k);
    if (k > kMaxGemvK)
        return set_error(G4_ERR_INVALID, "exact split needs calibrated int8 input and K <= 16384");
    GemvLaunch L{};
    L.count = 1;
    L.splits = ple_active_splits(k_splits);
    L.split_exact = 1;
    L.split_layout = 1;
    GemvJob &J = L.job[0];
    J.w = reinterpret_cast<const uint8_t *>(wq);
    J.scales = scales;
    J.x = x;
    J.dst = partials;
    J.bits = 8;
    J.x_kind = x_kind;
    J.out_kind = G4_KIND_F32;
    J.k = k;
    J.rows = num_rows;
    J.in_scale = in_scale;
    J.out_scale = 0.0f;
    int rc = check_job(J, 1, "ple-gate-split");
    if (rc) return rc;
    return launch_gemv(L, 1, as_stream(stream));
}

// ple-fold-projection (pleSplit.ts:24-41, bind :64-84).
int g4_ple_fold_projection(const void *wq, const float *scales, const float *gate_parts,
                           const float *gate_scales, int k_splits, float gate_in_scale,
                           float gate_out_scale, const g4_gelu_act *act, void *dst, int out_kind,
                           int k, int num_rows, float in_scale, float out_scale, void *stream) {
    if (k_splits != 1 && k_splits != 2 && k_splits != 4 && k_splits != 8)
        return set_error(G4_ERR_INVALID, "PLE splits must be 1, 2, 4 or 8");
    if (!gate_parts || !gate_scales)
        return set_error(G4_ERR_INVALID, "ple-fold-projection needs inputs named gate, up and gateScales");
    GeluAct fold;
    fold.fold_parts = gate_parts;
    fold.fold_scales = gate_scales;
    fold.fold_splits = ple_active_splits(k_splits);
    fold.fold_in = gate_in_scale;
    fold.fold_out = gate_out_scale;
    return gelu_gemv(8, wq, scales, gate_parts, G4_KIND_F32, act, &fold, dst, out_kind, k,
                     num_rows, 1, 0, 0, in_scale, out_scale, stream, "ple-fold-projection");
}

static int merge_common(const float *partials, const float *scales, void *dst, int out_kind,
                        int num_rows, int k_splits, int exact, float in_scale, float out_scale,
                        void *stream, const char *who) {
    if (num_rows <= 0) return set_error(G4_ERR_INVALID, "%s needs a positive params.numRows", who);
    if (k_splits < 2)
        return set_error(G4_ERR_INVALID, "%s only exists on a split dispatch, got kSplits %d", who, k_splits);
    if (!partials || !dst || (exact && !scales))
        return set_error(G4_ERR_INVALID, "%s needs an input named part", who);
    if (out_kind != G4_KIND_F32 && out_kind != G4_KIND_I8)
        return set_error(G4_ERR_INVALID, "%s: out_kind must be f32 or int8", who);
    if (out_kind == G4_KIND_I8 && out_scale == 0.0f)
        return set_error(G4_ERR_INVALID, "%s: int8 output codes need a calibrated outScale", who);
    hipLaunchKernelGGL(qgemv_merge_kernel, dim3((num_rows + 63) / 64), dim3(64), 0,
                       as_stream(stream), partials, scales, dst, out_kind, num_rows, k_splits,
                       exact, in_scale, out_scale);
    G4_LAUNCHED("qgemv_merge_kernel");
    return G4_OK;
}

int g4_qgemv_merge(const float *partials, void *dst, int out_kind, int num_rows, int k_splits,
                   float out_scale, void *stream) {
    return merge_common(partials, nullptr, dst, out_kind, num_rows, k_splits, 0, 0.0f, out_scale,
                        stream, "qgemv-merge");
}

int g4_qgemv_exact_merge(const float *partials, const float *scales, void *dst, int out_kind,
                         int num_rows, int k_splits, float in_scale, float out_scale,
                         void *stream) {
    return merge_common(partials, scales, dst, out_kind, num_rows, k_splits, 1, in_scale,
                        out_scale, stream, "qgemv-exact-merge");
}

}  // extern "C"

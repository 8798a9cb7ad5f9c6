// The M-column quantized linears on gfx950 int8 MFMA: qgemm-4bit (src/kernels/qgemm.ts) and
// qmatmul-8bit (src/kernels/pleMatmul.ts), plus the shape routing of src/execute.ts:372-430.
//
// Pipeline of one call (calibrated path):
//  1. The activation snap (the SRQ input prologue): M <= 32 fuses it into the small kernel (codes
//     in LDS, each 8-code group interleaved [x0 x2 x4 x6 x1 x3 x5 x7] for 4-bit weights so a weight
//     word's even and odd nibble lanes line up with the codes). The tile kernel takes an int8
//     caller's natural-order codes as given (and permutes the 4-bit B to match); f16 / f32 input is
//     snapped once per row by quantize_rows_kernel into a per-stream workspace, interleaved.
//  2. An MFMA kernel contracts codes x weights with v_mfma_i32_16x16x64_i8 in exact int32. The
//     int32 sums are exact, so the k order the MFMA uses internally is irrelevant; only the A and
//     B operands have to agree on it, and they do by construction.
//  3. The epilogue is the reference's f32(f32(inScale * scale[n]) * f32(acc)) and output snap.
//
// Kernels by M (chosen per shape, see pick_kernel):
//   M <= 2         the GEMV family (qgemv.hip): bit-identical, cheaper than any tile at this M.
//   3 <= M <= 32   qgemm_small_kernel: one launch with the snap fused (codes in LDS), 16 weight
//                  rows per block, the block's waves split K (4, or 16 when the grid is no wider
//                  than the CU count), an LDS fold of the partials; several projections of the
//                  same x can share one grid (linear_grouped).
//   M > 32, or over 32768+ rows
//                  qgemm_tile_kernel: 64 x 96 output tiles, activation codes and weights streamed
//                  global -> LDS by direct loads through a 3-4 stage ring, XCD-aware tile order.
#include "g4_internal.h"
#include "g4_workspace.h"

#include <algorithm>
#include <string>
#include <type_traits>

namespace g4 {

int gemv_columns(int bits, const void *wq, const float *scales, const void *x, int x_kind,
                 void *dst, int out_kind, int k, int num_rows, int m_cols, float in_scale,
                 float out_scale, hipStream_t stream, const char *who);


constexpr int kQuantThreads = 256;
constexpr int kTileBK = 128;

__device__ __forceinline__ uint32_t pack4b(int a, int b, int c, int d) {
    return (uint32_t)(a & 0xff) | ((uint32_t)(b & 0xff) << 8) | ((uint32_t)(c & 0xff) << 16) |
           ((uint32_t)(d & 0xff) << 24);
}

constexpr int kQuantGroups = 4;  // 8-code groups per thread per pass, all loaded before any snap

// The activation snap of the tile kernels: n8 groups of 8 activations (f16 or f32; x 16-byte
// aligned, each group one or two 16-byte loads) into codes, interleaved per 8-code group when
// PERM. A flat grid over the groups: each thread issues the loads of kQuantGroups groups, then
// snaps and stores them (one 8-byte store per group), so a pass costs one memory latency.
template <bool PERM, bool F16>
__global__ __launch_bounds__(kQuantThreads) void quantize_rows_kernel(const void *x, int64_t n8,
                                                                      float scale, int8_t *codes) {
    bool r_ok;
    const float r = srq_recip(scale, r_ok);
    const int64_t stride = (int64_t)gridDim.x * kQuantThreads * kQuantGroups;
    for (int64_t g0 = (int64_t)blockIdx.x * kQuantThreads * kQuantGroups + threadIdx.x; g0 < n8;
         g0 += stride) {
        u32x4 raw[kQuantGroups][F16 ? 1 : 2];
#pragma unroll
        for (int u = 0; u < kQuantGroups; ++u) {
            const int64_t g = min(g0 + (int64_t)u * kQuantThreads, n8 - 1);  // clamped: valid
            const u32x4 *p = reinterpret_cast<const u32x4 *>(x) + g * (F16 ? 1 : 2);
            raw[u][0] = p[0];
            if (!F16) raw[u][F16 ? 0 : 1] = p[1];
        }
#pragma unroll
        for (int u = 0; u < kQuantGroups; ++u) {
            const int64_t g = g0 + (int64_t)u * kQuantThreads;
            if (g >= n8) break;
            float v[8];
            if (F16) {
                const uint32_t h[4] = {raw[u][0].x, raw[u][0].y, raw[u][0].z, raw[u][0].w};
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    v[2 * i] = __half2float(__ushort_as_half((unsigned short)(h[i] & 0xffff)));
                    v[2 * i + 1] = __half2float(__ushort_as_half((unsigned short)(h[i] >> 16)));
                }
            } else {
                const uint32_t w[8] = {raw[u][0].x, raw[u][0].y, raw[u][0].z, raw[u][0].w,
                                       raw[u][F16 ? 0 : 1].x, raw[u][F16 ? 0 : 1].y,
                                       raw[u][F16 ? 0 : 1].z, raw[u][F16 ? 0 : 1].w};
#pragma unroll
                for (int i = 0; i < 8; ++i) v[i] = __uint_as_float(w[i]);
            }
            int c[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) c[i] = (int)srq_code_fast(v[i], scale, r, r_ok);
            uint2 out;
            if (PERM) {
                out.x = pack4b(c[0], c[2], c[4], c[6]);
                out.y = pack4b(c[1], c[3], c[5], c[7]);
            } else {
                out.x = pack4b(c[0], c[1], c[2], c[3]);
                out.y = pack4b(c[4], c[5], c[6], c[7]);
            }
            reinterpret_cast<uint2 *>(codes)[g] = out;
        }
    }
}

// srqCodes as a kernel (quant.ts:309-334), natural order.
__global__ void srq_quantize_kernel(const void *x, int x_kind, int8_t *codes, int64_t n, float s) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    bool r_ok;
    const float r = srq_recip(s, r_ok);
    for (int64_t e = i; e < n; e += stride)
        codes[e] = (int8_t)srq_code_fast(load_act(x, x_kind, e), s, r, r_ok);
}

// qmatmul-8bit on its uncalibrated path (inScale 0; pleMatmul.ts:139-147, oracle :212-222): one
// thread per (row, token column), a serial loop over the row's 4-code words. Each word's four
// products are summed in order starting from 0, then added to the accumulator, every step one f32
// rounding; the closing multiply is f32(f32(1 * scale) * acc). The order is the reference's
// definition, so nothing here may be reassociated: no FMA, no split of K across lanes. Each thread
// reads 16 codes (one 16-byte load) per iteration; K % 16 == 0 is checked by the caller.
template <bool F16>
__global__ __launch_bounds__(256) void qmatmul8_serial_kernel(
    const int8_t *wq, const float *scales, const void *x, void *dst, int out_kind, int k, int n,
    float out_scale) {
    const int row = blockIdx.x * 256 + threadIdx.x;
    const int col = blockIdx.y;
    if (row >= n) return;
    const uint4 *w = reinterpret_cast<const uint4 *>(wq + (int64_t)row * k);
    float acc = 0.0f;
    for (int i = 0; i < k / 16; ++i) {
        const uint4 ww = w[i];
        const uint32_t words[4] = {ww.x, ww.y, ww.z, ww.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int64_t e = (int64_t)col * k + 16 * i + 4 * j;
            float xs[4];
            if (F16) {  // f16 activations widen exactly to the reference's f32
                const __half2 *h = reinterpret_cast<const __half2 *>(reinterpret_cast<const __half *>(x) + e);
                const float2 a = __half22float2(h[0]), b = __half22float2(h[1]);
                xs[0] = a.x, xs[1] = a.y, xs[2] = b.x, xs[3] = b.y;
            } else {
                const float4 xv = *reinterpret_cast<const float4 *>(reinterpret_cast<const float *>(x) + e);
                xs[0] = xv.x, xs[1] = xv.y, xs[2] = xv.z, xs[3] = xv.w;
            }
            float d = 0.0f;
#pragma unroll
            for (int e = 0; e < 4; ++e)
                d = __fadd_rn(d, __fmul_rn((float)(int8_t)((words[j] >> (8 * e)) & 0xff), xs[e]));
            acc = __fadd_rn(acc, d);
        }
    }
    const float sr = scales[row];
    const float scale = isfinite(sr) ? sr : 0.0f;
    const float y = __fmul_rn(__fmul_rn(1.0f, scale), acc);
    store_linear_out(dst, (int64_t)col * n + row, out_kind, y, 0, out_scale);
}

// The B operand of one 16x16x64 step from 8 bytes (16 codes) of weights at `p`.
template <int BITS>
__device__ __forceinline__ v4i b_operand(uint32_t w0, uint32_t w1, uint32_t w2, uint32_t w3,
                                         int step) {
    v4i b;
    if (BITS == 4) {
        const uint32_t a = step == 0 ? w0 : w2;
        const uint32_t c = step == 0 ? w1 : w3;
        b.x = (int)(a & 0x0F0F0F0Fu);
        b.y = (int)((a >> 4) & 0x0F0F0F0Fu);
        b.z = (int)(c & 0x0F0F0F0Fu);
        b.w = (int)((c >> 4) & 0x0F0F0F0Fu);
    } else {
        (void)w2;
        (void)w3;
        b.x = (int)w0;
        b.y = (int)w1;
        b.z = (int)w2;
        b.w = (int)w3;
    }
    return b;
}

__device__ __forceinline__ void store_tile_out(void *dst, int m, int n, int N, int out_kind,
                                               int acc, float in_scale, float scale,
                                               float out_scale) {
    const float y = linear_epilogue(in_scale, scale, (float)acc);
    store_linear_out(dst, (int64_t)m * N + n, out_kind, y, acc, out_scale);
}

// ---- small M: M <= MT token rows, 16 weight rows per block, K split over the block's waves ------
// The activation snap is fused: the block snaps its MT token rows into LDS as int8 codes (the
// 4-bit interleave per 8-code group) one K chunk at a time, so a draft-verify or small prefill
// call is one launch. The 4-bit zero point needs sum(xq) per token row: one more MFMA per step
// against an all-ones B operand gives it exactly, folded with the partials like the products.
// Lane (j = lane % 16, g = lane / 16) owns weight row n0 + j; per 128-code stage it loads 16 bytes
// of that row (8-bit: 32), and MFMA half-step s takes codes g*32 + s*16 .. +16 of the stage from
// both operands. The LDS rows are padded by 16 bytes so the 16 token rows of one A read fall on
// distinct banks.
//
// WAVES: 4 for wide outputs (many blocks); 16 when the output has too few 16-row blocks to fill
// the chip (N = 1536 gives 96), so each block walks its K four times faster: a chunk of 128-code
// steps has one step per wave, and the fold of the 16 partial tiles goes through LDS. The sums are
// int32 and exact, so the split changes no result.
//
// Grouped launches: up to kSmallMaxJobs projections of the same x, K and scales (q, k, v; gate and
// up) share one grid; block b belongs to the first job whose block_end exceeds it.
//
// EPI (one job, its rows the gate): the gelu-mul pass in the epilogue, as the batch-1 plans fold
// it: the gate's output code back on out_scale, times the up value (EPI 1: the same row of the
// paired up projection w_up / s_up, streamed beside the gate's and snapped on out_scale; EPI 2:
// aux[m * aux_stride + n], f32), and dst receives srq(gelu(g) * u, act_scale).
constexpr int kSmallMaxJobs = 4;
struct SmallJobs {
    const uint8_t *w[kSmallMaxJobs];
    const float *scales[kSmallMaxJobs];
    void *dst[kSmallMaxJobs];
    int n[kSmallMaxJobs];
    int block_end[kSmallMaxJobs];  // cumulative 16-row blocks
    int count;
    const uint8_t *w_up;
    const float *s_up;
    const float *aux;
    int64_t aux_stride;
    float act_scale;
};

// Codes of a row per LDS chunk: 3072 (16-wave blocks) or 1536 (4-wave) at MT = 32, so the E2B
// shape's K = 1536 projections take one chunk (the gate / up pair at batch 32: two 1024-code
// chunks measured a 4.09 ms step, one chunk 4.01 ms).
template <int MT, int WAVES> constexpr int small_kc() { return (WAVES >= 16 ? 98304 : 49152) / MT; }

// One batch of a lane's weight loads for K steps kb0, kb0 + WAVES, ... (clamped: every load valid).
template <int BITS, int NP, int BATCH, int WAVES>
__device__ __forceinline__ void load_small_weights(u32x4 (&bw)[NP][BATCH][BITS == 4 ? 1 : 2],
                                                   const uint8_t *wrow, const uint8_t *wrow2, int kb0,
                                                   int ksteps, int kbase, int g) {
#pragma unroll
    for (int p = 0; p < NP; ++p) {
        const uint8_t *wr = p == 0 ? wrow : wrow2;
#pragma unroll
        for (int u = 0; u < BATCH; ++u) {
            const int kb = min(kb0 + WAVES * u, ksteps - 1);
            if (BITS == 4) {
                bw[p][u][0] = *reinterpret_cast<const u32x4 *>(wr + (kbase + kb) * 64 + g * 16);
            } else {
                bw[p][u][0] = *reinterpret_cast<const u32x4 *>(wr + (kbase + kb) * 128 + g * 32);
                bw[p][u][BITS == 4 ? 0 : 1] = *reinterpret_cast<const u32x4 *>(wr + (kbase + kb) * 128 + g * 32 + 16);
            }
        }
    }
}

template <int BITS, int MT, int WAVES, int EPI>
__global__ __launch_bounds__(WAVES * 64) void qgemm_small_kernel(
    const void *__restrict__ x, int x_kind, SmallJobs jobs, int M, int K, float in_scale,
    float out_scale, int out_kind, int ksplit) {
    constexpr int THREADS = WAVES * 64;
    constexpr int TM = MT / 16;
    constexpr int KC = small_kc<MT, WAVES>();  // codes of a row per LDS chunk
    constexpr int XSTR = KC + 16;              // LDS bytes per token row
    constexpr int BATCH = WAVES >= 16 ? 1 : 4;
    constexpr int NP = EPI == 1 ? 2 : 1;             // product sets: the gate's (and the up's)
    constexpr int NACC = BITS == 4 ? (NP + 1) * TM : NP * TM;  // products, then the row sums
    // the codes during the K loop, and every wave's partial tiles for the fold: in a region of
    // their own when both fit (two blocks of 4 waves per CU, or one of 16), so the fold needs no
    // barrier for the last reads of the codes; else over the codes' bytes
    constexpr int XS_BYTES = MT * XSTR, RED_BYTES = WAVES * NACC * 64 * 16;
    constexpr bool SEP_RED = XS_BYTES + RED_BYTES <= (WAVES >= 16 ? 160 * 1024 : 80 * 1024);
    __shared__ __align__(16) int8_t smem[SEP_RED ? XS_BYTES + RED_BYTES
                                                 : (XS_BYTES > RED_BYTES ? XS_BYTES : RED_BYTES)];
    int8_t *xs = smem;
    v4i(*red)[NACC][64] = reinterpret_cast<v4i(*)[NACC][64]>(smem + (SEP_RED ? XS_BYTES : 0));
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int j = lane & 15;
    const int g = lane >> 4;
    // the block's job (uniform selects, no indexed kernel-argument array)
    const uint8_t *W = jobs.w[0];
    const float *scales = jobs.scales[0];
    void *dst = jobs.dst[0];
    int N = jobs.n[0], begin = 0;
#pragma unroll
    for (int i = 1; i < kSmallMaxJobs; ++i) {
        if (i < jobs.count && (int)blockIdx.x >= jobs.block_end[i - 1]) {
            W = jobs.w[i];
            scales = jobs.scales[i];
            dst = jobs.dst[i];
            N = jobs.n[i];
            begin = jobs.block_end[i - 1];
        }
    }
    const int n0 = ((int)blockIdx.x - begin) * 16;
    const int m0 = blockIdx.y * MT;
    const int n = min(n0 + j, N - 1);
    const int row_bytes = BITS == 4 ? (K >> 1) : K;
    const uint8_t *wrow = W + (int64_t)n * row_bytes;
    const uint8_t *wrow2 = EPI == 1 ? jobs.w_up + (int64_t)n * row_bytes : wrow;
    bool r_ok;
    const float rcp = srq_recip(in_scale, r_ok);
    // the epilogue's per-output operands (row scales; the paired up rows' scales; the f32 up
    // vector), requested now so the epilogue does not wait a memory round trip for them
    constexpr int EQ = (TM * 256 + THREADS - 1) / THREADS;  // outputs per thread
    float e_scale[EQ], e_scale2[EQ], e_aux[EQ];
#pragma unroll
    for (int e = 0; e < EQ; ++e) {
        const int q = min(tid + e * THREADS, TM * 256 - 1);
        const int t = q >> 8, ln = (q >> 2) & 63, r = q & 3;
        const int nn = min(n0 + (ln & 15), N - 1);
        const int m = min(m0 + t * 16 + 4 * (ln >> 4) + r, M - 1);
        e_scale[e] = scales[nn];
        e_scale2[e] = EPI == 1 ? jobs.s_up[nn] : 0.0f;
        e_aux[e] = EPI == 2 ? jobs.aux[(int64_t)m * jobs.aux_stride + nn] : 0.0f;
    }
    v4i acc[NACC];
#pragma unroll
    for (int t = 0; t < NACC; ++t) acc[t] = v4i{0, 0, 0, 0};
    const v4i ones = v4i{0x01010101, 0x01010101, 0x01010101, 0x01010101};

    // ksplit > 0: block z takes codes [z ksplit, (z + 1) ksplit) of K and stores its int32 partial
    // accumulator (out_kind int32) to dst[z][M][N]; the splits' sum is the exact accumulator
    const int kbeg = ksplit > 0 ? (int)blockIdx.z * ksplit : 0;
    const int kend = ksplit > 0 ? min(K, kbeg + ksplit) : K;
    for (int kc0 = kbeg; kc0 < kend; kc0 += KC) {
        const int kcn = min(KC, kend - kc0);
        const int gpr = kcn >> 3;  // 8-code groups per row in this chunk
        const int ksteps = kcn / kTileBK;
        const int kbase = kc0 / kTileBK;
        // The chunk's first batch of weights is requested before the codes are copied, so the two
        // memory latencies overlap (the weights do not depend on the codes). Requesting the codes
        // first measured slower: every block reads the same few KB of codes, and at the head of
        // the queue those requests pile onto the same L2 lines.
        u32x4 bw_first[NP][BATCH][BITS == 4 ? 1 : 2];
        load_small_weights<BITS, NP, BATCH, WAVES>(bw_first, wrow, wrow2, wave, ksteps, kbase, g);
        lds_barrier();  // the previous chunk's codes are no longer read
        // the snap: each thread issues the loads of SB groups (indices clamped, so every load is
        // valid) before converting any, so a chunk costs one memory latency per SB groups. Only
        // the block's real token rows are snapped: a padding row's LDS codes reach only the
        // products of its own output row, which is never stored.
        constexpr int SB = 4;
        const int total = min(MT, M - m0) * gpr;
        if (x_kind == G4_KIND_I8) {
            // codes as given: 16-byte loads (two groups), all of a thread's loads in flight at
            // once, then a byte permute per 8-code group for 4-bit weights
            constexpr int U16 = (MT * KC / 16 + THREADS - 1) / THREADS;
            const int upr = kcn >> 4, total16 = min(MT, M - m0) * upr;
            u32x4 raw[U16];
            int rr[U16], uu[U16];
#pragma unroll
            for (int u = 0; u < U16; ++u) {
                const int q = min(tid + u * THREADS, total16 - 1);
                rr[u] = q / upr;
                uu[u] = q - rr[u] * upr;
                raw[u] = *reinterpret_cast<const u32x4 *>(reinterpret_cast<const int8_t *>(x) +
                                                          (int64_t)(m0 + rr[u]) * K + kc0 + uu[u] * 16);
            }
#pragma unroll
            for (int u = 0; u < U16; ++u) {
                if (tid + u * THREADS >= total16) break;
                u32x4 o = raw[u];
                if (BITS == 4) {  // [x0 x2 x4 x6 | x1 x3 x5 x7] per 8-code group
                    o = u32x4{__builtin_amdgcn_perm(raw[u].y, raw[u].x, 0x06040200u),
                              __builtin_amdgcn_perm(raw[u].y, raw[u].x, 0x07050301u),
                              __builtin_amdgcn_perm(raw[u].w, raw[u].z, 0x06040200u),
                              __builtin_amdgcn_perm(raw[u].w, raw[u].z, 0x07050301u)};
                }
                *reinterpret_cast<u32x4 *>(&xs[rr[u] * XSTR + uu[u] * 16]) = o;
            }
        }
        for (int q0 = tid; x_kind != G4_KIND_I8 && q0 < total; q0 += SB * THREADS) {
            u32x4 raw_a[SB], raw_b[SB];
            int rr[SB], gg[SB];  // row and group of each load, kept for the stores (one divide)
#pragma unroll
            for (int u = 0; u < SB; ++u) {
                const int q = min(q0 + u * THREADS, total - 1);
                const int r = q / gpr, gi = q - r * gpr;
                rr[u] = r;
                gg[u] = gi;
                const int64_t e = (int64_t)(m0 + r) * K + kc0 + gi * 8;
                if (x_kind == G4_KIND_I8) {
                    const uint2 v = *reinterpret_cast<const uint2 *>(reinterpret_cast<const int8_t *>(x) + e);
                    raw_a[u] = u32x4{v.x, v.y, 0u, 0u};
                    raw_b[u] = u32x4{0u, 0u, 0u, 0u};
                } else if (x_kind == G4_KIND_F16) {
                    raw_a[u] = *reinterpret_cast<const u32x4 *>(reinterpret_cast<const __half *>(x) + e);
                    raw_b[u] = u32x4{0u, 0u, 0u, 0u};
                } else {
                    const u32x4 *p4 = reinterpret_cast<const u32x4 *>(reinterpret_cast<const float *>(x) + e);
                    raw_a[u] = p4[0];
                    raw_b[u] = p4[1];
                }
            }
#pragma unroll
            for (int u = 0; u < SB; ++u) {
                if (q0 + u * THREADS >= total) break;
                const int r = rr[u], gi = gg[u];
                int c[8];
                {
                    if (x_kind == G4_KIND_I8) {
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            c[i] = (int)(int8_t)((raw_a[u].x >> (8 * i)) & 0xff);
                            c[4 + i] = (int)(int8_t)((raw_a[u].y >> (8 * i)) & 0xff);
                        }
                    } else if (x_kind == G4_KIND_F16) {
                        const uint32_t h[4] = {raw_a[u].x, raw_a[u].y, raw_a[u].z, raw_a[u].w};
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            c[2 * i] = (int)srq_code_fast(
                                __half2float(__ushort_as_half((unsigned short)(h[i] & 0xffff))), in_scale, rcp, r_ok);
                            c[2 * i + 1] = (int)srq_code_fast(
                                __half2float(__ushort_as_half((unsigned short)(h[i] >> 16))), in_scale, rcp, r_ok);
                        }
                    } else {
                        const uint32_t v[8] = {raw_a[u].x, raw_a[u].y, raw_a[u].z, raw_a[u].w,
                                               raw_b[u].x, raw_b[u].y, raw_b[u].z, raw_b[u].w};
#pragma unroll
                        for (int i = 0; i < 8; ++i) c[i] = (int)srq_code_fast(__uint_as_float(v[i]), in_scale, rcp, r_ok);
                    }
                }
                uint2 packed;
                if (BITS == 4) {
                    packed.x = pack4b(c[0], c[2], c[4], c[6]);
                    packed.y = pack4b(c[1], c[3], c[5], c[7]);
                } else {
                    packed.x = pack4b(c[0], c[1], c[2], c[3]);
                    packed.y = pack4b(c[4], c[5], c[6], c[7]);
                }
                *reinterpret_cast<uint2 *>(&xs[r * XSTR + gi * 8]) = packed;
            }
        }
        lds_barrier();
        for (int kb0 = wave; kb0 < ksteps; kb0 += WAVES * BATCH) {
            u32x4 bw[NP][BATCH][BITS == 4 ? 1 : 2];
            if (kb0 == wave) {
#pragma unroll
                for (int p = 0; p < NP; ++p)
#pragma unroll
                    for (int u = 0; u < BATCH; ++u)
#pragma unroll
                        for (int h = 0; h < (BITS == 4 ? 1 : 2); ++h) bw[p][u][h] = bw_first[p][u][h];
            } else {
                load_small_weights<BITS, NP, BATCH, WAVES>(bw, wrow, wrow2, kb0, ksteps, kbase, g);
            }
            // every A operand of the batch read from LDS before the first MFMA, so the reads'
            // latencies overlap (step indices clamped: a step past the end is read, not used)
            v4i av[BATCH][2][TM];
#pragma unroll
            for (int u = 0; u < BATCH; ++u) {
                const int kb = min(kb0 + WAVES * u, ksteps - 1);
#pragma unroll
                for (int s = 0; s < 2; ++s)
#pragma unroll
                    for (int t = 0; t < TM; ++t)
                        av[u][s][t] = *reinterpret_cast<const v4i *>(
                            &xs[(t * 16 + j) * XSTR + kb * kTileBK + g * 32 + s * 16]);
            }
#pragma unroll
            for (int u = 0; u < BATCH; ++u) {
                const int kb = kb0 + WAVES * u;
                if (kb < ksteps) {
#pragma unroll
                    for (int s = 0; s < 2; ++s) {
                        v4i b[NP];
#pragma unroll
                        for (int p = 0; p < NP; ++p) {
                            if (BITS == 4)
                                b[p] = b_operand<4>(bw[p][u][0].x, bw[p][u][0].y, bw[p][u][0].z,
                                                    bw[p][u][0].w, s);
                            else
                                b[p] = __builtin_bit_cast(v4i, bw[p][u][BITS == 4 ? 0 : s]);
                        }
#pragma unroll
                        for (int t = 0; t < TM; ++t) {
                            const v4i a = av[u][s][t];
#pragma unroll
                            for (int p = 0; p < NP; ++p)
                                acc[p * TM + t] =
                                    __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b[p], acc[p * TM + t], 0, 0, 0);
                            if (BITS == 4)  // each code counted once: both halves
                                acc[NP * TM + t] =
                                    __builtin_amdgcn_mfma_i32_16x16x64_i8(a, ones, acc[NP * TM + t], 0, 0, 0);
                        }
                    }
                }
            }
        }
        // A batch's clamped loads past the last step are never read; without this wait the
        // compiler counts them as pending into the next chunk and waits for every load in flight
        // (the epilogue's early operand loads included) before the next chunk's first request.
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    }
    // Fold: every wave leaves its partial tiles in LDS (over the codes, once all waves are done
    // with them, when the two share bytes); then the block's threads take the outputs, each
    // summing the waves' partials of one (row, column) in wave order, so the epilogue (a gelu for
    // EPI) is spread over all waves.
    if (!SEP_RED) __syncthreads();
#pragma unroll
    for (int t = 0; t < NACC; ++t) red[wave][t][lane] = acc[t];
    __syncthreads();
    bool o_ok;
    const float orcp = srq_recip(out_scale, o_ok);
#pragma unroll
    for (int e = 0; e < EQ; ++e) {
        const int q = tid + e * THREADS;
        if (q >= TM * 256) break;
        // D layout: lane l, register r -> row 4 (l / 16) + r of A, column l % 16 of B.
        const int t = q >> 8, ln = (q >> 2) & 63, r = q & 3;
        const int lr = t * 16 + 4 * (ln >> 4) + r;
        const int m = m0 + lr, nn = n0 + (ln & 15);
        if (m >= M || nn >= N) continue;
        int v = 0, v2 = 0, rsum = 0;
#pragma unroll
        for (int w = 0; w < WAVES; ++w) {
            v += reinterpret_cast<const int *>(&red[w][t][ln])[r];
            if (EPI == 1) v2 += reinterpret_cast<const int *>(&red[w][TM + t][ln])[r];
            if (BITS == 4) rsum += reinterpret_cast<const int *>(&red[w][NP * TM + t][ln])[r];
        }
        if (BITS == 4) {  // the ones product: sum(xq) of row lr
            v -= 8 * rsum;
            v2 -= 8 * rsum;
        }
        const float yv = __fmul_rn(__fmul_rn(in_scale, e_scale[e]), (float)v);
        const int64_t o = (int64_t)m * N + nn;
        if (EPI != 0) {  // gelu(gate) * up, snapped for the consumer
            const float gq = __fmul_rn(srq_code_fast(yv, out_scale, orcp, o_ok), out_scale);
            float uq;
            if (EPI == 1) {
                const float yu = __fmul_rn(__fmul_rn(in_scale, e_scale2[e]), (float)v2);
                uq = __fmul_rn(srq_code_fast(yu, out_scale, orcp, o_ok), out_scale);
            } else {
                uq = e_aux[e];
            }
            reinterpret_cast<int8_t *>(dst)[o] =
                (int8_t)srq_code_i(__fmul_rn(d_gelu(gq), uq), jobs.act_scale);
        } else if (out_kind == G4_KIND_I8) {
            reinterpret_cast<int8_t *>(dst)[o] = (int8_t)srq_code_fast(yv, out_scale, orcp, o_ok);
        } else if (out_kind == G4_KIND_I32) {
            reinterpret_cast<int32_t *>(dst)[o + (int64_t)blockIdx.z * M * N] = v;
        } else {
            float f = yv;
            if (out_scale != 0.0f) f = __fmul_rn(srq_code_fast(yv, out_scale, orcp, o_ok), out_scale);
            reinterpret_cast<float *>(dst)[o] = f;
        }
    }
}

// ---- tile: 64 x 96 outputs per block, both operands streamed through an LDS ring ---------------
// Each K stage is 128 codes. Stage st of the tile is
//   A: 64 rows x 128 bytes of activation codes (8 KB),
//   B: 96 columns x 64 bytes of packed int4 weights (6 KB), or 96 x 128 bytes of int8 weights.
// Both go global -> LDS by direct loads (global_load_lds_dwordx4: no VGPRs, no ds_write), NS stages
// deep. Four waves in a 2 x 2 layout own 32 x 48 outputs each (2 x 3 MFMA tiles of 16 x 16).
// Per stage a wave waits for its own loads of stage st+1, joins the block barrier, reads the
// operands of stage st+1 into registers (so their LDS latency hides under the MFMAs), refills the
// buffer stage st-1 used with stage st+NS-1, and runs stage st's 12 v_mfma_i32_16x16x64_i8.
// Every wave issues the same number of loads per stage (the weight remainder re-loads a chunk
// another wave also loads, to the same LDS bytes): with a per-wave count the compiler splits the
// loop into branches and then drains the LDS reads before each stage's first MFMA.
//
// Operand layouts (the k assignment inside an MFMA is free as long as A and B agree, because the
// int32 sums are exact):
//   lane (j = lane % 16, g = lane / 16), half-step s takes codes 32 g + 16 s .. +16 of the stage.
//   A is the per-8 interleaved code row [x0 x2 x4 x6 x1 x3 x5 x7] (4-bit) or natural (8-bit, and
//   4-bit NAT, where nib_natural16 puts B in natural order instead).
//   4-bit B: a lane's 16 bytes of column j are codes 32 g .. 32 g + 31; with w' = w ^ 0x88888888,
//   (w' << 4) & 0xF0F0F0F0 holds 16 * (even codes) and w' & 0xF0F0F0F0 16 * (odd codes) as signed
//   bytes, so the accumulator is 16 * sum(code * x), exact (|sum| <= 2^31 / 16 for K <= 16384),
//   and no zero-point sums are needed.
// LDS rows are XOR-swizzled so that any 16 consecutive lanes of a b128 read (and any 8) hit
// distinct banks: A row r (128 B) keeps chunk c at position c ^ ((r & 7) ^ ((r >> 3) & 1)); 4-bit B
// column c (64 B) keeps chunk g at g ^ (((c >> 1) ^ (c >> 3)) & 3).
constexpr int kTileBM = 64;
constexpr int kTileBN = 96;
constexpr int kTileEpiStride = kTileBN + 4;  // int32 words per staged output row (bank spread)

// 16 bytes per lane from global memory into LDS at lds + 16 * lane. Issued through asm: when the
// compiler sees an LDS DMA it waits for every outstanding load (vmcnt(0)) before the next LDS
// read, which would empty the ring at every stage; here the waits are explicit (tile_wait). M0
// carries the wave-uniform LDS address; nothing else in these kernels uses M0.
__device__ __forceinline__ void lds_dma16(const void *src, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off"
                 :: "s"(__builtin_amdgcn_readfirstlane(lds)), "v"(src) : "memory", "m0");
}

// At most N of this wave's vector-memory operations still in flight (its loads of the awaited
// stage have landed), its LDS reads drained, then the block barrier: afterwards every wave's data
// for that stage is in LDS and every wave has finished reading the buffer the next refill
// overwrites. The LDS drain is the builtin so the compiler's own wait bookkeeping sees it.
template <int N> __device__ __forceinline__ void tile_wait() {
    static_assert(N >= 0 && N < 64, "vmcnt holds 6 bits");
    asm volatile("s_waitcnt vmcnt(%0)" :: "n"(N) : "memory");
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0), vmcnt and expcnt unconstrained
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// tile_wait for `later` stages of DPS loads each still allowed in flight (a runtime count mapped
// onto the immediate vmcnt; a count beyond the counter's range waits for everything).
template <int DPS, int L = 0> __device__ __forceinline__ void tile_wait_stages(int later) {
    if constexpr (L * DPS >= 64 || L > 15) {
        tile_wait<0>();
    } else {
        if (later == L) tile_wait<L * DPS>();
        else tile_wait_stages<DPS, L + 1>(later);
    }
}

__device__ __forceinline__ uint32_t nib_even16(uint32_t w) { return ((w ^ 0x88888888u) << 4) & 0xF0F0F0F0u; }
__device__ __forceinline__ uint32_t nib_odd16(uint32_t w) { return (w ^ 0x88888888u) & 0xF0F0F0F0u; }
// Eight packed codes c0..c7 (one weight word) as 16 x code signed bytes in natural order: the even
// and odd nibble bytes [c0 c2 c4 c6] and [c1 c3 c5 c7] interleaved by two byte permutes into
// [c0 c1 c2 c3] and [c4 c5 c6 c7], so the activation codes need no interleave.
__device__ __forceinline__ void nib_natural16(uint32_t w, int &lo, int &hi) {
    const uint32_t e = nib_even16(w), o = nib_odd16(w);
    lo = (int)__builtin_amdgcn_perm(o, e, 0x05010400u);  // bytes e0 o0 e1 o1
    hi = (int)__builtin_amdgcn_perm(o, e, 0x07030602u);  // bytes e2 o2 e3 o3
}

// NAT (4-bit): A holds natural-order codes and B is permuted to match in registers; otherwise A is
// the per-8 interleaved row the nibble lanes read directly (no permutes).
// BM: 64 tile rows (each wave 32 x 48), or 32 (each wave 16 x 48) for grids that would leave CUs
// idle at 64: a block keeps about as many bytes in flight as the CU allows, so the launch's
// bandwidth grows with the number of CUs it occupies.
template <int BITS, int NS, bool NAT, int BM = kTileBM>
__global__ __launch_bounds__(256) void qgemm_tile_kernel(
    const int8_t *__restrict__ A, const uint8_t *__restrict__ W, const float *__restrict__ scales,
    void *dst, int M, int N, int K, float in_scale, float out_scale, int out_kind, int tiles_m,
    int tiles_n) {
    static_assert(BM == 64 || BM == 32, "tile rows");
    constexpr int BN = kTileBN, TM = BM / 32, TN = 3, WR = BM / 2;  // WR: rows of a wave's tile
    constexpr int BROW = BITS == 4 ? 64 : 128;  // weight bytes of one column per stage
    constexpr int A_BYTES = BM * 128, B_BYTES = BN * BROW, SB = A_BYTES + B_BYTES;
    constexpr int A_PW = A_BYTES / 1024 / 4;                   // loads per wave per stage
    constexpr int B_INS = B_BYTES / 1024, B_PW = (B_INS + 3) / 4;
    constexpr int DPS = A_PW + B_PW;
    constexpr int ESTR = kTileEpiStride;
    static_assert(NS >= 3 && NS * SB <= 160 * 1024, "ring depth");
    static_assert(NS * SB >= BM * ESTR * 4 + BN * 4, "the epilogue staging fits the ring");
    __shared__ __align__(1024) uint8_t smem[NS * SB];

    // Blocks go to the 8 XCDs round robin; one XCD gets every M tile of a run of N tiles, so its L2
    // fetches those weight columns once.
    const int b = blockIdx.x;
    const int xcd = b & 7, idx = b >> 3;
    const int tm = idx % tiles_m;
    const int tn = (idx / tiles_m) * 8 + xcd;
    if (tn >= tiles_n) return;  // whole block, before any barrier
    const int m0 = tm * BM, n0 = tn * BN;
    const int tid = threadIdx.x, lane = tid & 63;
    // the epilogue's column scale, requested now so the epilogue does not wait a memory round trip
    const float col_scale = tid < BN ? scales[min(n0 + tid, N - 1)] : 0.0f;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int j = lane & 15, g = lane >> 4;
    const int wm = wave >> 1, wn = wave & 1;
    const int row_bytes = BITS == 4 ? K >> 1 : K;
    const uint32_t sbase = (uint32_t)(uintptr_t)smem;

    // Direct-load sources. A load q covers tile rows 8 q .. 8 q + 7; lane i fills row 8 q + i / 8,
    // position i % 8, with the chunk the swizzle puts there. Rows and columns past the matrix are
    // clamped to the last one (their products land in outputs that are not stored).
    const int8_t *asrc[A_PW];
    uint32_t adst[A_PW];
#pragma unroll
    for (int i = 0; i < A_PW; ++i) {
        const int q = wave + 4 * i;
        const int r = 8 * q + (lane >> 3);
        const int c = (lane & 7) ^ (((lane >> 3) & 7) ^ (q & 1));
        asrc[i] = A + (int64_t)min(m0 + r, M - 1) * K + 16 * c;
        adst[i] = q * 1024;
    }
    const uint8_t *bsrc[B_PW];
    uint32_t bdst[B_PW];
#pragma unroll
    for (int i = 0; i < B_PW; ++i) {
        const int q = min(wave + 4 * i, B_INS - 1);
        int col, c;
        if (BITS == 4) {  // load q: columns 16 q .. +15, 4 chunks each
            const int cl = lane >> 2;
            col = 16 * q + cl;
            c = (lane & 3) ^ (((cl >> 1) ^ (cl >> 3)) & 3);
        } else {  // load q: columns 8 q .. +7, 8 chunks each (the A swizzle)
            col = 8 * q + (lane >> 3);
            c = (lane & 7) ^ (((lane >> 3) & 7) ^ (q & 1));
        }
        bsrc[i] = W + (int64_t)min(n0 + col, N - 1) * row_bytes + 16 * c;
        bdst[i] = A_BYTES + q * 1024;
    }
    auto issue = [&](int st, int buf) {
        const uint32_t base = sbase + buf * SB;
#pragma unroll
        for (int i = 0; i < A_PW; ++i) lds_dma16(asrc[i] + st * 128, base + adst[i]);
#pragma unroll
        for (int i = 0; i < B_PW; ++i) lds_dma16(bsrc[i] + st * BROW, base + bdst[i]);
    };
    // LDS byte offsets of this lane's operands inside a stage buffer.
    const int sig = (j & 7) ^ ((j >> 3) & 1);
    uint32_t aoff[2], boff[2];
#pragma unroll
    for (int s = 0; s < 2; ++s) {
        aoff[s] = (wm * WR / 8 + (j >> 3)) * 1024 + (j & 7) * 128 + 16 * ((2 * g + s) ^ sig);
        boff[s] = A_BYTES + (wn * 48 / 8 + (j >> 3)) * 1024 + (j & 7) * 128 + 16 * ((2 * g + s) ^ sig);
    }
    const uint32_t boff4 = A_BYTES + (wn * 48 + j) * 64 + 16 * (g ^ (((j >> 1) ^ (j >> 3)) & 3));

    v4i acc[TM][TN];
#pragma unroll
    for (int t = 0; t < TM; ++t)
#pragma unroll
        for (int u = 0; u < TN; ++u) acc[t][u] = v4i{0, 0, 0, 0};
    constexpr int BR = BITS == 4 ? 1 : 2;  // b128 weight reads per column tile per stage
    v4i ra[2][TM][2];
    u32x4 rb[2][TN][BR];
    auto read_ops = [&](int buf, v4i (&a)[TM][2], u32x4 (&bw)[TN][BR]) {
        const uint8_t *sa = smem + buf * SB;
#pragma unroll
        for (int t = 0; t < TM; ++t)
#pragma unroll
            for (int s = 0; s < 2; ++s) a[t][s] = *reinterpret_cast<const v4i *>(sa + aoff[s] + t * 2048);
#pragma unroll
        for (int u = 0; u < TN; ++u) {
            if (BITS == 4) {
                bw[u][0] = *reinterpret_cast<const u32x4 *>(sa + boff4 + u * 1024);
            } else {
#pragma unroll
                for (int s = 0; s < BR; ++s) bw[u][s] = *reinterpret_cast<const u32x4 *>(sa + boff[s] + u * 2048);
            }
        }
    };
    auto compute = [&](const v4i (&a)[TM][2], const u32x4 (&bw)[TN][BR]) {
        v4i bo[2][TN];
#pragma unroll
        for (int u = 0; u < TN; ++u) {
            if (BITS == 4) {
                const u32x4 w = bw[u][0];
                if (NAT) {
                    int a0, a1, b0, b1, c0, c1, d0, d1;
                    nib_natural16(w.x, a0, a1);
                    nib_natural16(w.y, b0, b1);
                    nib_natural16(w.z, c0, c1);
                    nib_natural16(w.w, d0, d1);
                    bo[0][u] = v4i{a0, a1, b0, b1};
                    bo[1][u] = v4i{c0, c1, d0, d1};
                } else {
                    bo[0][u] = v4i{(int)nib_even16(w.x), (int)nib_odd16(w.x), (int)nib_even16(w.y), (int)nib_odd16(w.y)};
                    bo[1][u] = v4i{(int)nib_even16(w.z), (int)nib_odd16(w.z), (int)nib_even16(w.w), (int)nib_odd16(w.w)};
                }
            } else {
                bo[0][u] = __builtin_bit_cast(v4i, bw[u][0]);
                bo[1][u] = __builtin_bit_cast(v4i, bw[u][BR - 1]);
            }
        }
        // all six accumulators of one half-step before the next: consecutive MFMAs are independent
#pragma unroll
        for (int s = 0; s < 2; ++s)
#pragma unroll
            for (int u = 0; u < TN; ++u)
#pragma unroll
                for (int t = 0; t < TM; ++t)
                    acc[t][u] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[t][s], bo[s][u], acc[t][u], 0, 0, 0);
    };

    // nk >= NS - 1 (the host picks NS). Stages 0 .. NS-2 in flight, then stage 0's operands.
    const int nk = K >> 7;
#pragma unroll
    for (int st = 0; st < NS - 1; ++st) issue(st, st);
    tile_wait_stages<DPS>(NS - 2);
    read_ops(0, ra[0], rb[0]);
    // Stage st: stage st+1 landed; read its operands, refill the buffer of stage st-1 with stage
    // st+NS-1, then stage st's MFMAs. Pairs of stages keep the register double buffer static.
    int s0 = 0;
    for (; s0 + NS + 1 <= nk; s0 += 2) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int st = s0 + h;
            tile_wait_stages<DPS>(NS - 3);  // stages issued after st+1: st+2 .. st+NS-2
            read_ops((st + 1) % NS, ra[h ^ 1], rb[h ^ 1]);
            issue(st + NS - 1, (st + NS - 1) % NS);
            __builtin_amdgcn_sched_barrier(0);  // operand reads and loads go out before the MFMAs
            compute(ra[h], rb[h]);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    // The remaining stages (nothing or fewer loads left to issue), also in register pairs.
    for (; s0 < nk; s0 += 2) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int st = s0 + h;
            if (st >= nk) break;
            if (st + 1 < nk) {
                const int last = min(nk - 1, st + NS - 2);  // the last stage issued so far
                tile_wait_stages<DPS>(last - (st + 1));
                read_ops((st + 1) % NS, ra[h ^ 1], rb[h ^ 1]);
                if (st + NS - 1 < nk) issue(st + NS - 1, (st + NS - 1) % NS);
            }
            __builtin_amdgcn_sched_barrier(0);
            compute(ra[h], rb[h]);
            __builtin_amdgcn_sched_barrier(0);
        }
    }

    // Epilogue. The int32 sums go to LDS (rows of ESTR words), then each thread takes runs of 8
    // columns of one row: one column-scale multiply, the snap, and one store per run.
    tile_wait<0>();  // every wave is done with the ring
    int32_t *sacc = reinterpret_cast<int32_t *>(smem);
    float *sscale = reinterpret_cast<float *>(smem + BM * ESTR * 4);
    if (tid < BN) sscale[tid] = __fmul_rn(in_scale, col_scale);
#pragma unroll
    for (int t = 0; t < TM; ++t)
#pragma unroll
        for (int u = 0; u < TN; ++u)
#pragma unroll
            for (int r = 0; r < 4; ++r)  // D layout: lane l, register r -> row 4 (l / 16) + r, column l % 16
                sacc[(wm * WR + t * 16 + 4 * g + r) * ESTR + wn * 48 + u * 16 + j] =
                    BITS == 4 ? acc[t][u][r] >> 4 : acc[t][u][r];
    __syncthreads();
    bool r_ok;
    const float rcp = srq_recip(out_scale, r_ok);
    constexpr int RC = BN / 8;
    for (int q = tid; q < BM * RC; q += 256) {
        const int lr = q / RC, c = q - lr * RC;
        const int m = m0 + lr, n = n0 + c * 8;
        if (m >= M || n >= N) continue;
        const v4i x0 = *reinterpret_cast<const v4i *>(sacc + lr * ESTR + c * 8);
        const v4i x1 = *reinterpret_cast<const v4i *>(sacc + lr * ESTR + c * 8 + 4);
        const int v[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
        const int live = min(8, N - n);
        const int64_t o = (int64_t)m * N + n;
        if (out_kind == G4_KIND_I32) {
            int32_t *d = reinterpret_cast<int32_t *>(dst) + o;
            if (live == 8 && (o & 3) == 0) {
                reinterpret_cast<v4i *>(d)[0] = x0;
                reinterpret_cast<v4i *>(d)[1] = x1;
            } else {
                for (int e = 0; e < live; ++e) d[e] = v[e];
            }
            continue;
        }
        float y[8], code[8];
        bool near = !r_ok;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            y[e] = __fmul_rn(sscale[c * 8 + e], (float)v[e]);  // the reference's epilogue order
            const float t = __fmul_rn(y[e], rcp);
            code[e] = rintf(t);
            // |fl(y * fl(1/s)) - fl(y / s)| < 2^-13 while |y / s| <= 256 (beyond, both clamp), so a
            // quotient farther than that from a half integer rounds to the same code either way.
            near |= fabsf(t - code[e]) >= 0.5f - 0x1p-13f;
        }
        if (near) {
#pragma unroll
            for (int e = 0; e < 8; ++e) code[e] = rintf(__fdiv_rn(y[e], out_scale));
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) code[e] = fminf(fmaxf(code[e], -128.0f), 127.0f);
        if (out_kind == G4_KIND_I8) {
            uint32_t p0 = 0, p1 = 0;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                p0 |= ((uint32_t)(int)code[e] & 0xffu) << (8 * e);
                p1 |= ((uint32_t)(int)code[e + 4] & 0xffu) << (8 * e);
            }
            int8_t *d = reinterpret_cast<int8_t *>(dst) + o;
            if (live == 8 && (o & 7) == 0) {
                *reinterpret_cast<uint2 *>(d) = make_uint2(p0, p1);
            } else {
                for (int e = 0; e < live; ++e) d[e] = (int8_t)(int)code[e];
            }
        } else {  // f32: q * outScale, or y itself when outScale is 0 (no output snap)
            float f[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) f[e] = out_scale != 0.0f ? __fmul_rn(code[e], out_scale) : y[e];
            float *d = reinterpret_cast<float *>(dst) + o;
            if (live == 8 && (o & 3) == 0) {
                reinterpret_cast<float4 *>(d)[0] = make_float4(f[0], f[1], f[2], f[3]);
                reinterpret_cast<float4 *>(d)[1] = make_float4(f[4], f[5], f[6], f[7]);
            } else {
                for (int e = 0; e < live; ++e) d[e] = f[e];
            }
        }
    }
}

// ---- the wide tile: 4-bit weights, 64 x 192 outputs per block of 8 waves -----------------------
//
// For grids that fill the device (M >= 256 and at least one block per CU). Against the 64 x 96
// tile above it halves the unpack work and the LDS operand reads per MFMA:
//   - each wave owns 64 x 48 outputs (4 x 3 MFMA tiles) over one K half of every 128-code stage:
//     wave = 4 kh + wn, kh the K half (codes 64 kh + 16 g .. +15 of the stage for lane group g),
//     wn the 48-column quarter. One unpacked weight operand feeds four MFMAs, where the 2 x 2
//     layout of the narrow tile fed two. Lane groups g and g + 1 read the two 8-byte halves of
//     one 16-byte weight chunk, so a 32-lane pass of the 8-byte reads covers 16 columns x 16 bytes
//     at distinct swizzled chunk positions: no bank conflicts;
//   - waves 0-3 load the stage's activation rows (2 direct loads each), waves 4-7 its weight
//     columns (3 each); both stream global -> LDS through a 4-stage ring (80 KB, two blocks per CU
//     at large M);
//   - the stage barrier does not drain the LDS reads: the reads of stage st+1 are issued between
//     stage st's MFMAs and only the ring slot of stage st-1 (read a full stage earlier) is
//     refilled after the barrier;
//   - the MFMA takes the weights as its A operand, so the accumulator is the transposed tile: lane
//     (j, g) holds output row j, columns 4 g .. 4 g + 3 of each 16 x 16 tile, so the epilogue
//     packs 4 consecutive int8 outputs per lane into one word; a whole tile's words are gathered
//     in LDS and written as 16-byte runs of 192-byte tile rows (9.6 -> 9.0 us at M = 512,
//     28.9 -> 26.0 us at M = 2048, against one 4-byte store per group);
//   - the two K halves meet through LDS (each wave keeps two of its four row tiles), then every
//     wave snaps 2 x 3 groups of 4 outputs. A group falls back to the IEEE divide only when some
//     lane's quotient lies within 2^-13 of a half integer (one branch per group, not per output).
// The LDS layouts, swizzles and the stage's A and B loads are the narrow tile's (a stage buffer is
// 64 activation rows then 192 weight columns).
constexpr int kWideBM = 64;
constexpr int kWideBN = 192;
constexpr int kWideNS = 4;
constexpr int kWideA = kWideBM * 128;              // activation bytes per stage
constexpr int kWideSB = kWideA + kWideBN * 64;     // stage buffer: activations + packed weights
// The epilogue's int8 code tile, in the ring after the K-half exchange (48 KB) and the scales.
constexpr int kWideCodeTile = 50 * 1024;
constexpr int kWideCodeRow = kWideBN + 16;
static_assert(8 * 6 * 1024 + kWideBN * 4 <= kWideCodeTile && kWideCodeTile + kWideBM * kWideCodeRow <= kWideNS * kWideSB,
              "the epilogue code tile fits the ring after the exchange and the scales");

template <int N, bool LGKM> __device__ __forceinline__ void wide_wait() {
    static_assert(N >= 0 && N < 64, "vmcnt holds 6 bits");
    asm volatile("s_waitcnt vmcnt(%0)" :: "n"(N) : "memory");
    if (LGKM) __builtin_amdgcn_s_waitcnt(0xC07F);
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}
template <int DPS, bool LGKM> __device__ __forceinline__ void wide_wait_stages(int later) {
    switch (later) {
        case 0: wide_wait<0, LGKM>(); break;
        case 1: wide_wait<1 * DPS, LGKM>(); break;
        case 2: wide_wait<2 * DPS, LGKM>(); break;
        default: wide_wait<0, LGKM>(); break;
    }
}

struct WideOps {
    v4i a[4];
    uint2 b[3];
};

// The K loop of one wave. NL direct loads per stage (src[i] advancing STEP bytes a stage into ring
// offset dst[i]); nk >= kWideNS - 1 stages.
// NK > 0: the stage count is a compile-time constant and the loop is unrolled whole. Then the
// compiler's wait for a stage's operands counts only the reads issued after them (lgkmcnt(7)), so
// stage st+1's reads stay in flight under stage st's MFMAs; across a loop back-edge it waits for
// every outstanding LDS read instead, which is why the runtime form issues the reads between the
// MFMAs.
template <int NL, int STEP, bool NAT, int NK>
__device__ __forceinline__ void wide_k_loop(const uint8_t *const (&src)[NL], const uint32_t (&dst)[NL],
                                            uint32_t sbase, const uint8_t *smem, uint32_t aoff,
                                            uint32_t boff, int nk_rt, v4i (&acc)[4][3]) {
    constexpr int NS = kWideNS;
    auto issue = [&](int st, int buf) {
#pragma unroll
        for (int i = 0; i < NL; ++i) lds_dma16(src[i] + st * STEP, sbase + buf * kWideSB + dst[i]);
    };
    auto read_ops = [&](int buf, WideOps &o) {
        const uint8_t *p = smem + buf * kWideSB;
#pragma unroll
        for (int t = 0; t < 4; ++t) o.a[t] = *reinterpret_cast<const v4i *>(p + aoff + t * 2048);
#pragma unroll
        for (int u = 0; u < 3; ++u) o.b[u] = *reinterpret_cast<const uint2 *>(p + boff + u * 1024);
    };
    auto mfma_cols = [&](const WideOps &o, int ulo, int uhi) {
#pragma unroll
        for (int u = 0; u < 3; ++u) {
            if (u < ulo || u >= uhi) continue;
            v4i bo;
            if (NAT) {
                int l0, h0, l1, h1;
                nib_natural16(o.b[u].x, l0, h0);
                nib_natural16(o.b[u].y, l1, h1);
                bo = v4i{l0, h0, l1, h1};
            } else {
                bo = v4i{(int)nib_even16(o.b[u].x), (int)nib_odd16(o.b[u].x), (int)nib_even16(o.b[u].y),
                         (int)nib_odd16(o.b[u].y)};
            }
#pragma unroll
            for (int t = 0; t < 4; ++t)
                acc[t][u] = __builtin_amdgcn_mfma_i32_16x16x64_i8(bo, o.a[t], acc[t][u], 0, 0, 0);
        }
    };
    WideOps r[2];
#pragma unroll
    for (int st = 0; st < NS - 1; ++st) issue(st, st);
    wide_wait_stages<NL, true>(NS - 2);
    read_ops(0, r[0]);
    if constexpr (NK > 0) {
        // stage st: the barrier after stage st+1 landed, its operand reads, the refill of the slot
        // of stage st-1 with stage st+NS-1, stage st's MFMAs
#pragma unroll
        for (int st = 0; st < NK; ++st) {
            if (st + 1 < NK) {
                const int last = min(NK - 1, st + NS - 2);
                wide_wait_stages<NL, false>(last - (st + 1));
                read_ops((st + 1) % NS, r[(st + 1) & 1]);
                if (st + NS - 1 < NK) issue(st + NS - 1, (st + NS - 1) % NS);
            }
            __builtin_amdgcn_sched_barrier(0);
            mfma_cols(r[st & 1], 0, 3);
            __builtin_amdgcn_sched_barrier(0);
        }
        wide_wait<0, true>();
        return;
    }
    const int nk = nk_rt;
    int s0 = 0;
    // Stage st: the barrier after stage st+1 landed; refill the slot of stage st-1 (its operands
    // were read during stage st-2 and consumed by stage st-1) with stage st+NS-1; two column tiles
    // of MFMAs; the operand reads of stage st+1; the last column tile.
    for (; s0 + NS + 1 <= nk; s0 += 2) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int st = s0 + h;
            wide_wait_stages<NL, false>(NS - 3);
            issue(st + NS - 1, (st + NS - 1) % NS);
            __builtin_amdgcn_sched_barrier(0);
            mfma_cols(r[h], 0, 2);
            __builtin_amdgcn_sched_barrier(0);
            read_ops((st + 1) % NS, r[h ^ 1]);
            __builtin_amdgcn_sched_barrier(0);
            mfma_cols(r[h], 2, 3);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    for (; s0 < nk; s0 += 2) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int st = s0 + h;
            if (st >= nk) break;
            if (st + 1 < nk) {
                const int last = min(nk - 1, st + NS - 2);  // the last stage issued so far
                wide_wait_stages<NL, false>(last - (st + 1));
                read_ops((st + 1) % NS, r[h ^ 1]);
                if (st + NS - 1 < nk) issue(st + NS - 1, (st + NS - 1) % NS);
            }
            __builtin_amdgcn_sched_barrier(0);
            mfma_cols(r[h], 0, 3);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    wide_wait<0, true>();  // the ring is free for the epilogue
}

template <bool NAT>
__global__ __launch_bounds__(512, 4) void qgemm_wide_kernel(
    const int8_t *__restrict__ A, const uint8_t *__restrict__ W, const float *__restrict__ scales,
    void *dst, int M, int N, int K, float in_scale, float out_scale, int out_kind, int tiles_m,
    int tiles_n) {
    __shared__ __align__(1024) uint8_t smem[kWideNS * kWideSB];
    static_assert(kWideNS * kWideSB >= 8 * 6 * 1024 + kWideBN * 4, "the K-half exchange and the scales fit the ring");
    // XCD-aware order: XCD x takes the N tiles x, x + 8, ... and its consecutive blocks walk those N
    // tiles fastest, so the blocks resident on one XCD share a run of activation rows (at M = 2048,
    // two blocks per CU: 16 row tiles x 4 column tiles, 2.1 MB, inside the XCD's 4 MB L2).
    const int b = blockIdx.x;
    const int xcd = b & 7, idx = b >> 3;
    const int tnx = (tiles_n + 7) >> 3;
    const int tm = idx / tnx;
    const int tn = (idx % tnx) * 8 + xcd;
    if (tn >= tiles_n) return;  // whole block, before any barrier
    const int m0 = tm * kWideBM, n0 = tn * kWideBN;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int kh = wave >> 2, wn = wave & 3;
    const int j = lane & 15, g = lane >> 4;
    const uint32_t sbase = (uint32_t)(uintptr_t)smem;
    const int row_bytes = K >> 1;
    // this lane's operand offsets in a stage buffer (the narrow tile's swizzles)
    const int sig = (j & 7) ^ ((j >> 3) & 1);
    const uint32_t aoff = (j >> 3) * 1024 + (j & 7) * 128 + 16 * ((4 * kh + g) ^ sig);
    const uint32_t boff = kWideA + (wn * 48 + j) * 64 + 16 * ((2 * kh + (g >> 1)) ^ (((j >> 1) ^ (j >> 3)) & 3)) +
                          8 * (g & 1);
    // the tile's column scales (one per thread), loaded now so their latency hides under the K loop
    const float col_scale = tid < kWideBN ? scales[min(n0 + tid, N - 1)] : 0.0f;
    v4i acc[4][3];
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int u = 0; u < 3; ++u) acc[t][u] = v4i{0, 0, 0, 0};
    const int nk = K / kTileBK;
    if (kh == 0) {  // activation rows 8 q .. 8 q + 7, q = wn and wn + 4
        const uint8_t *src[2];
        uint32_t dsto[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int q = wn + 4 * i;
            const int r = 8 * q + (lane >> 3);
            const int c = (lane & 7) ^ (((lane >> 3) & 7) ^ (q & 1));
            src[i] = reinterpret_cast<const uint8_t *>(A + (int64_t)min(m0 + r, M - 1) * K + 16 * c);
            dsto[i] = q * 1024;
        }
        if (nk == 12) wide_k_loop<2, 128, NAT, 12>(src, dsto, sbase, smem, aoff, boff, nk, acc);
        else if (nk == 16) wide_k_loop<2, 128, NAT, 16>(src, dsto, sbase, smem, aoff, boff, nk, acc);
        else wide_k_loop<2, 128, NAT, 0>(src, dsto, sbase, smem, aoff, boff, nk, acc);
    } else {  // weight columns 16 q .. 16 q + 15, q = wn, wn + 4, wn + 8
        const uint8_t *src[3];
        uint32_t dsto[3];
#pragma unroll
        for (int i = 0; i < 3; ++i) {
            const int q = wn + 4 * i;
            const int cl = lane >> 2;
            const int c = (lane & 3) ^ (((cl >> 1) ^ (cl >> 3)) & 3);
            src[i] = W + (int64_t)min(n0 + 16 * q + cl, N - 1) * row_bytes + 16 * c;
            dsto[i] = kWideA + q * 1024;
        }
        if (nk == 12) wide_k_loop<3, 64, NAT, 12>(src, dsto, sbase, smem, aoff, boff, nk, acc);
        else if (nk == 16) wide_k_loop<3, 64, NAT, 16>(src, dsto, sbase, smem, aoff, boff, nk, acc);
        else wide_k_loop<3, 64, NAT, 0>(src, dsto, sbase, smem, aoff, boff, nk, acc);
    }

    // The K halves meet: wave (wn, kh) keeps row tiles 2 kh, 2 kh + 1 and hands the other two to
    // wave (wn, 1 - kh). Register indices stay compile-time constants.
    v4i *P = reinterpret_cast<v4i *>(smem);
    float *S = reinterpret_cast<float *>(smem + 8 * 6 * 1024);  // inScale x the column scales, after P
    v4i sum[2][3];
    auto meet = [&](auto khc) {
        constexpr int KH = decltype(khc)::value;
#pragma unroll
        for (int tt = 0; tt < 2; ++tt)
#pragma unroll
            for (int u = 0; u < 3; ++u) P[(wave * 6 + tt * 3 + u) * 64 + lane] = acc[2 * (1 - KH) + tt][u];
        if (tid < kWideBN) S[tid] = __fmul_rn(in_scale, col_scale);  // f32(inScale * scale[n])
        __syncthreads();
#pragma unroll
        for (int tt = 0; tt < 2; ++tt)
#pragma unroll
            for (int u = 0; u < 3; ++u)
                sum[tt][u] = acc[2 * KH + tt][u] + P[((wave ^ 4) * 6 + tt * 3 + u) * 64 + lane];
    };
    if (kh == 0) meet(std::integral_constant<int, 0>{});
    else meet(std::integral_constant<int, 1>{});

    bool r_ok;
    const float rcp = srq_recip(out_scale, r_ok);
    // A whole tile of int8 outputs (the usual case): the same snap with no row, column or
    // alignment checks per group of 4. Each group's 4 codes go to a 64 x 192 code tile in LDS
    // (rows 208 bytes apart, so the 64 lanes of a group store hit distinct banks); then each
    // thread stores 16-byte runs of whole tile rows (192 contiguous bytes per row), in place of
    // 4-byte stores scattered over 16 rows per instruction. N % 16 == 0 and a 16-byte aligned dst
    // keep every run aligned.
    if (out_kind == G4_KIND_I8 && out_scale != 0.0f && m0 + kWideBM <= M && n0 + kWideBN <= N && (N & 15) == 0 &&
        ((uintptr_t)dst & 15) == 0) {
        uint8_t *T = smem + kWideCodeTile;
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
            uint8_t *trow = T + ((2 * kh + tt) * 16 + j) * kWideCodeRow + wn * 48 + 4 * g;
#pragma unroll
            for (int u = 0; u < 3; ++u) {
                const float4 s4 = *reinterpret_cast<const float4 *>(S + wn * 48 + u * 16 + 4 * g);
                const float sc[4] = {s4.x, s4.y, s4.z, s4.w};
                const int v[4] = {sum[tt][u].x >> 4, sum[tt][u].y >> 4, sum[tt][u].z >> 4, sum[tt][u].w >> 4};
                float y[4], code[4];
                float worst = r_ok ? 0.0f : 1.0f;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    y[e] = __fmul_rn(sc[e], (float)v[e]);  // the reference's order
                    const float t = __fmul_rn(y[e], rcp);
                    code[e] = rintf(t);
                    worst = fmaxf(worst, fabsf(t - code[e]));
                }
                if (worst >= 0.5f - 0x1p-13f) {  // the quotient bound of the generic path below
#pragma unroll
                    for (int e = 0; e < 4; ++e) code[e] = rintf(__fdiv_rn(y[e], out_scale));
                }
                uint32_t bb[4];
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    bb[e] = __float_as_uint(__fadd_rn(fminf(fmaxf(code[e], -128.0f), 127.0f), 12582912.0f));
                const uint32_t lo = __builtin_amdgcn_perm(bb[1], bb[0], 0x0C0C0400u);
                const uint32_t hi = __builtin_amdgcn_perm(bb[3], bb[2], 0x0C0C0400u);
                *reinterpret_cast<uint32_t *>(trow + u * 16) = __builtin_amdgcn_perm(hi, lo, 0x05040100u);
            }
        }
        __syncthreads();
        for (int c = tid; c < kWideBM * (kWideBN / 16); c += 512) {
            const int r = c / (kWideBN / 16), cc = c - r * (kWideBN / 16);
            const u32x4 v = *reinterpret_cast<const u32x4 *>(T + r * kWideCodeRow + cc * 16);
            __builtin_nontemporal_store(
                v, reinterpret_cast<u32x4 *>(reinterpret_cast<int8_t *>(dst) + (int64_t)(m0 + r) * N + n0 + cc * 16));
        }
        return;
    }
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
        const int m = m0 + (2 * kh + tt) * 16 + j;
#pragma unroll
        for (int u = 0; u < 3; ++u) {
            const int n = n0 + wn * 48 + u * 16 + 4 * g;
            const int live = min(4, N - n);
            const bool row_ok = m < M && live > 0;
            const int64_t o = (int64_t)m * N + n;
            const int v[4] = {sum[tt][u].x >> 4, sum[tt][u].y >> 4, sum[tt][u].z >> 4, sum[tt][u].w >> 4};
            if (out_kind == G4_KIND_I32) {
                if (!row_ok) continue;
                int32_t *d = reinterpret_cast<int32_t *>(dst) + o;
                if (live == 4 && (o & 3) == 0) *reinterpret_cast<v4i *>(d) = v4i{v[0], v[1], v[2], v[3]};
                else for (int e = 0; e < live; ++e) d[e] = v[e];
                continue;
            }
            const float4 s4 = *reinterpret_cast<const float4 *>(S + wn * 48 + u * 16 + 4 * g);
            const float sc[4] = {s4.x, s4.y, s4.z, s4.w};
            float y[4], code[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) y[e] = __fmul_rn(sc[e], (float)v[e]);  // the reference's order
            if (out_scale == 0.0f) {  // f32 output without an output snap (int8 needs a scale)
                if (!row_ok) continue;
                float *d = reinterpret_cast<float *>(dst) + o;
                if (live == 4 && (o & 3) == 0) *reinterpret_cast<float4 *>(d) = make_float4(y[0], y[1], y[2], y[3]);
                else for (int e = 0; e < live; ++e) d[e] = y[e];
                continue;
            }
            float worst = r_ok ? 0.0f : 1.0f;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float t = __fmul_rn(y[e], rcp);
                code[e] = rintf(t);
                worst = fmaxf(worst, fabsf(t - code[e]));
            }
            // |fl(y * fl(1/s)) - fl(y / s)| < 2^-13 while |y / s| <= 256 (beyond, both clamp): a
            // quotient farther than that from a half integer rounds the same either way.
            if (worst >= 0.5f - 0x1p-13f) {
#pragma unroll
                for (int e = 0; e < 4; ++e) code[e] = rintf(__fdiv_rn(y[e], out_scale));
            }
            if (!row_ok) continue;
            if (out_kind == G4_KIND_I8) {
                // code + 1.5 * 2^23 is exact and its low byte is the code's two's complement byte
                uint32_t b[4];
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    b[e] = __float_as_uint(__fadd_rn(fminf(fmaxf(code[e], -128.0f), 127.0f), 12582912.0f));
                int8_t *d = reinterpret_cast<int8_t *>(dst) + o;
                if (live == 4 && (o & 3) == 0) {
                    const uint32_t lo = __builtin_amdgcn_perm(b[1], b[0], 0x0C0C0400u);  // b0.0 b1.0
                    const uint32_t hi = __builtin_amdgcn_perm(b[3], b[2], 0x0C0C0400u);  // b2.0 b3.0
                    *reinterpret_cast<uint32_t *>(d) = __builtin_amdgcn_perm(hi, lo, 0x05040100u);
                } else {
                    for (int e = 0; e < live; ++e) d[e] = (int8_t)(b[e] & 0xffu);
                }
            } else {  // f32: q * outScale
                float f[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) f[e] = __fmul_rn(fminf(fmaxf(code[e], -128.0f), 127.0f), out_scale);
                float *d = reinterpret_cast<float *>(dst) + o;
                if (live == 4 && (o & 3) == 0) *reinterpret_cast<float4 *>(d) = make_float4(f[0], f[1], f[2], f[3]);
                else for (int e = 0; e < live; ++e) d[e] = f[e];
            }
        }
    }
}

// ---- per-stream workspace for the snapped activation codes ------------------------------------

namespace {

int ws_alloc(void **p, size_t bytes) { return hipMalloc(p, bytes) != hipSuccess; }
int ws_release(void *p) { return hipFree(p) != hipSuccess; }
int ws_drain(void *s) { return hipStreamSynchronize(as_stream(s)) != hipSuccess; }
int ws_capturing(void *s, bool *yes) {
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(as_stream(s), &st) != hipSuccess) return 1;
    *yes = st != hipStreamCaptureStatusNone;
    return 0;
}

WorkspaceCache &ws_cache() {
    static WorkspaceCache cache(WorkspaceOps{ws_alloc, ws_release, ws_drain, ws_capturing});
    return cache;
}

}  // namespace

// A device buffer of at least `bytes` owned by (device, stream), under the rules of
// g4_workspace.h: never grown inside a capture, never freed while a captured graph may hold it.
static int workspace(void *stream, size_t bytes, void **out) {
    int dev = 0;
    G4_HIP(hipGetDevice(&dev));
    std::string err;
    switch (ws_cache().get(dev, stream, bytes, out, &err)) {
        case WorkspaceCache::kOk: return G4_OK;
        case WorkspaceCache::kRefused: return set_error(G4_ERR_INVALID, "qgemm: %s", err.c_str());
        default: return set_error(G4_ERR_HIP, "qgemm: %s", err.c_str());
    }
}

int workspace_forget_stream(void *stream) {
    int dev = 0;
    G4_HIP(hipGetDevice(&dev));
    if (ws_cache().forget_stream(dev, stream) != WorkspaceCache::kOk)
        return set_error(G4_ERR_HIP, "stream destroy: draining the stream's workspace failed");
    return G4_OK;
}

enum KernelChoice { K_GEMV = 0, K_SKINNY16, K_SKINNY32, K_TILE128, K_GEMV_F32, K_GEMV_COLS,
                    K_SERIAL8, K_WIDE };

// gemm_mode: the caller named qgemm-4bit / qmatmul-8bit (execute.ts matmulKernel in gemm mode).
// Uncalibrated qmatmul-8bit then keeps the reference's serial per-output order at any M; the
// routed g4_linear is gemm mode only above two tokens (a decode step's 8-bit linear is qgemv-8bit,
// execute.ts:372-375).
static KernelChoice pick_kernel(int bits, int m, int n, int k, float in_scale, bool gemm_mode) {
    if (in_scale == 0.0f) return bits == 8 && gemm_mode ? K_SERIAL8 : K_GEMV_F32;
    if (m <= 2) return K_GEMV;
    if (k % kTileBK != 0) return K_GEMV_COLS;
    // the small kernel snaps all of x in each 16-row block: past 32768 rows (the tied head) the
    // re-reads outweigh the weights, and the 64-row tile (mostly padding rows) streams faster
    if (n >= 32768 && k >= 2 * kTileBK) return K_TILE128;
    if (m <= 16) return K_SKINNY16;
    if (k < 2 * kTileBK) return K_SKINNY32;  // the tile ring needs two K stages
    if (m <= 32) return K_SKINNY32;
    // the wide tile once its grid fills the device: 4-bit weights, M >= 256, three K stages
    const int64_t wide_blocks = (int64_t)((m + kWideBM - 1) / kWideBM) * ((n + kWideBN - 1) / kWideBN);
    if (bits == 4 && m >= 256 && k >= kWideNS * kTileBK - kTileBK && wide_blocks >= device_cu_count())
        return K_WIDE;
    return K_TILE128;
}

static const char *choice_name(KernelChoice c, int bits) {
    switch (c) {
        case K_GEMV: return bits == 4 ? "qgemv-4bit" : "qgemv-8bit";
        case K_SKINNY16: return bits == 4 ? "qgemm-4bit-mfma-small16" : "qmatmul-8bit-mfma-small16";
        case K_SKINNY32: return bits == 4 ? "qgemm-4bit-mfma-small32" : "qmatmul-8bit-mfma-small32";
        case K_TILE128: return bits == 4 ? "qgemm-4bit-mfma-tile" : "qmatmul-8bit-mfma-tile";
        case K_WIDE: return "qgemm-4bit-mfma-wide";
        case K_GEMV_F32: return bits == 4 ? "qgemv-4bit-f32" : "qgemv-8bit-f32";
        case K_SERIAL8: return "qmatmul-8bit-serial";
        default: return bits == 4 ? "qgemv-4bit-columns" : "qgemv-8bit-columns";
    }
}

// The small-M kernel over `jobs` (16-row blocks laid end to end): 16 waves per block when the
// grid has no more blocks than the device has CUs (each block then walks its K four times
// faster), else 4.
template <int BITS, int MT, int EPI>
static void launch_small_t(const void *x, int x_kind, const SmallJobs &jobs, int m, int k,
                           float in_scale, float out_scale, int out_kind, hipStream_t stream,
                           int splits = 1) {
    const int ksplit = splits > 1 ? k / splits : 0;
    const dim3 grid(jobs.block_end[jobs.count - 1], (m + MT - 1) / MT, splits);
    if ((int64_t)grid.x * grid.y * grid.z <= device_cu_count())
        hipLaunchKernelGGL((qgemm_small_kernel<BITS, MT, 16, EPI>), grid, dim3(1024), 0, stream, x,
                           x_kind, jobs, m, k, in_scale, out_scale, out_kind, ksplit);
    else
        hipLaunchKernelGGL((qgemm_small_kernel<BITS, MT, 4, EPI>), grid, dim3(256), 0, stream, x,
                           x_kind, jobs, m, k, in_scale, out_scale, out_kind, ksplit);
}

// epi: 0 plain (any job count), 1 the paired gate/up gelu epilogue (4-bit), 2 the f32-vector one.
static int launch_small(int bits, int mt, int epi, const void *x, int x_kind, const SmallJobs &jobs,
                        int m, int k, float in_scale, float out_scale, int out_kind,
                        hipStream_t stream) {
#define G4_SMALL(B, T, E) launch_small_t<B, T, E>(x, x_kind, jobs, m, k, in_scale, out_scale, out_kind, stream)
    if (epi == 1 && mt == 16) G4_SMALL(4, 16, 1);
    else if (epi == 1) G4_SMALL(4, 32, 1);
    else if (epi == 2 && bits == 4 && mt == 16) G4_SMALL(4, 16, 2);
    else if (epi == 2 && bits == 4) G4_SMALL(4, 32, 2);
    else if (epi == 2 && mt == 16) G4_SMALL(8, 16, 2);
    else if (epi == 2) G4_SMALL(8, 32, 2);
    else if (bits == 4 && mt == 16) G4_SMALL(4, 16, 0);
    else if (bits == 4) G4_SMALL(4, 32, 0);
    else if (mt == 16) G4_SMALL(8, 16, 0);
    else G4_SMALL(8, 32, 0);
#undef G4_SMALL
    G4_LAUNCHED("qgemm_small_kernel");
    return G4_OK;
}

int linear_split_acc(int bits, const uint8_t *wq, const float *scales, const int8_t *x, int k,
                     int n, int m, int splits, int32_t *part, hipStream_t stream) {
    if (!wq || !scales || !x || !part || m < 3 || m > 32 || n <= 0 || splits < 2 ||
        splits > kSplitAccMax || k % (splits * kTileBK))
        return set_error(G4_ERR_INVALID, "split accumulators: bad arguments (m %d, k %d, splits %d)",
                         m, k, splits);
    SmallJobs jobs{};
    jobs.w[0] = wq;
    jobs.scales[0] = scales;
    jobs.dst[0] = part;
    jobs.n[0] = n;
    jobs.block_end[0] = (n + 15) / 16;
    jobs.count = 1;
    if (bits == 4 && m <= 16)
        launch_small_t<4, 16, 0>(x, G4_KIND_I8, jobs, m, k, 1.0f, 0.0f, G4_KIND_I32, stream, splits);
    else if (bits == 4)
        launch_small_t<4, 32, 0>(x, G4_KIND_I8, jobs, m, k, 1.0f, 0.0f, G4_KIND_I32, stream, splits);
    else if (m <= 16)
        launch_small_t<8, 16, 0>(x, G4_KIND_I8, jobs, m, k, 1.0f, 0.0f, G4_KIND_I32, stream, splits);
    else
        launch_small_t<8, 32, 0>(x, G4_KIND_I8, jobs, m, k, 1.0f, 0.0f, G4_KIND_I32, stream, splits);
    G4_LAUNCHED("qgemm_small_kernel");
    return G4_OK;
}

template <int BITS>
static int launch_tile(const int8_t *codes, bool natural, const uint8_t *w, const float *scales,
                       void *dst, int m, int n, int k, float in_scale, float out_scale,
                       int out_kind, hipStream_t stream) {
    const int tiles_n = (n + kTileBN - 1) / kTileBN;
    // 32-row tiles when 64-row ones would not give every CU a block (config 2 at M = 128: 256
    // blocks in place of 128), and for M <= 32 (the tied head at a decode batch), where half of a
    // 64-row tile would be padding rows: batch-32 step 2.823 -> 2.816 ms
    const bool half = m <= kTileBM / 2 ||
                      ((int64_t)((m + kTileBM - 1) / kTileBM) * tiles_n < device_cu_count() && m > 32);
    const int bm = half ? kTileBM / 2 : kTileBM;
    const int tiles_m = (m + bm - 1) / bm;
    const int blocks = tiles_m * ((tiles_n + 7) / 8) * 8;  // XCD-aware order: whole groups of 8
    const int nk = k / kTileBK;  // >= 2 (k % 128 == 0 and k >= 256 here)
    // 8-bit weights are natural-order bytes already: their A is natural either way
    const bool nat = BITS == 4 && natural;
#define G4_TILE(NS_, NAT_, BM_)                                                                   \
    hipLaunchKernelGGL((qgemm_tile_kernel<BITS, NS_, NAT_, BM_>), dim3(blocks), dim3(256), 0,      \
                       stream, codes, w, scales, dst, m, n, k, in_scale, out_scale, out_kind,     \
                       tiles_m, tiles_n)
    if (half) {
        if (nk >= 3 && nat) G4_TILE(4, true, 32);
        else if (nk >= 3) G4_TILE(4, false, 32);
        else if (nat) G4_TILE(3, true, 32);
        else G4_TILE(3, false, 32);
    } else {
        if (nk >= 3 && nat) G4_TILE(4, true, 64);
        else if (nk >= 3) G4_TILE(4, false, 64);
        else if (nat) G4_TILE(3, true, 64);
        else G4_TILE(3, false, 64);
    }
#undef G4_TILE
    G4_LAUNCHED("qgemm_tile_kernel");
    return G4_OK;
}

static int check_linear(int bits, const void *wq, const float *scales, const void *x, int x_kind,
                        void *dst, int out_kind, int k, int n, int m, float in_scale,
                        float out_scale, const char *who) {
    if (!wq || !scales || !x || !dst)
        return set_error(G4_ERR_INVALID, "%s needs inputs named wq, scales and x", who);
    if (k <= 0 || n <= 0 || m <= 0)
        return set_error(G4_ERR_INVALID, "%s needs params.k, params.numRows and params.mCols", who);
    if (bits != 4 && bits != 8) return set_error(G4_ERR_INVALID, "%s: bits must be 4 or 8", who);
    if (x_kind != G4_KIND_F32 && x_kind != G4_KIND_F16 && x_kind != G4_KIND_I8)
        return set_error(G4_ERR_INVALID, "%s: x_kind %d is not f32, f16 or int8", who, x_kind);
    if (out_kind != G4_KIND_F32 && out_kind != G4_KIND_I8 && out_kind != G4_KIND_I32)
        return set_error(G4_ERR_INVALID, "%s: out_kind %d is not f32, int8 or int32", who, out_kind);
    if (out_kind == G4_KIND_I8 && out_scale == 0.0f)
        return set_error(G4_ERR_INVALID, "%s: int8 output codes need a calibrated outScale", who);
    if (in_scale == 0.0f && (x_kind == G4_KIND_I8 || out_kind == G4_KIND_I32))
        return set_error(G4_ERR_INVALID,
                         "%s: inScale 0.0 is the uncalibrated f32 path (no int8 codes, no int32 "
                         "accumulator)", who);
    if ((reinterpret_cast<uintptr_t>(wq) & 15) || (reinterpret_cast<uintptr_t>(x) & 15))
        return set_error(G4_ERR_INVALID, "%s: wq and x must be 16-byte aligned", who);
    if ((int64_t)m * (int64_t)n > (int64_t)INT32_MAX)
        return set_error(G4_ERR_INVALID, "%s: M * N exceeds the 32-bit index range", who);
    return G4_OK;
}

// The small-M kernel snaps f16 / f32 activations itself, in every one of its blocks: past about
// 4 Mi snaps in total (M * K per block times the blocks along N), one snap pass over the M * K
// activations into a buffer of codes, then the kernel on int8 codes, costs less (config 2: M = 8,
// K = 1536 over 384 blocks is 4.7 Mi).
static bool small_presnap(int m, int n, int k) {
    return (int64_t)m * k * ((n + 15) / 16) >= ((int64_t)1 << 22);
}

// Whether a call snaps f16 / f32 activations into a buffer of M * K codes first (the tile kernels,
// and the small-M kernel past small_presnap): the only paths of this file that need memory beyond
// their operands.
static bool needs_codes_buffer(int bits, int m, int n, int k, float in_scale, int x_kind,
                               bool gemm_mode) {
    const KernelChoice c = pick_kernel(bits, m, n, k, in_scale, gemm_mode);
    if (x_kind == G4_KIND_I8) return false;
    if (c == K_TILE128 || c == K_WIDE) return true;
    return (c == K_SKINNY16 || c == K_SKINNY32) && small_presnap(m, n, k);
}

// The snap pass: M * K f16 / f32 activations (16-byte aligned, K % 128 == 0) into int8 codes in
// `given` or the stream's workspace, interleaved per 8-code group when perm (the tile kernels'
// 4-bit layout) or in natural order.
static int snap_pass(const void *x, int x_kind, int m, int k, float in_scale, bool perm,
                     hipStream_t stream, int8_t *given, const int8_t **codes) {
    void *ws = given;
    if (!ws) {
        int rc = workspace(stream, (size_t)m * k, &ws);
        if (rc) return rc;
    }
    const int64_t n8 = (int64_t)m * k / 8;
    const int64_t per_block = (int64_t)kQuantThreads * kQuantGroups;
    const int qblocks = (int)std::min<int64_t>((n8 + per_block - 1) / per_block, 8 * 1024);
    int8_t *wsc = reinterpret_cast<int8_t *>(ws);
    if (x_kind == G4_KIND_F16) {
        if (perm)
            hipLaunchKernelGGL((quantize_rows_kernel<true, true>), dim3(qblocks), dim3(kQuantThreads), 0,
                               stream, x, n8, in_scale, wsc);
        else
            hipLaunchKernelGGL((quantize_rows_kernel<false, true>), dim3(qblocks), dim3(kQuantThreads), 0,
                               stream, x, n8, in_scale, wsc);
    } else {
        if (perm)
            hipLaunchKernelGGL((quantize_rows_kernel<true, false>), dim3(qblocks), dim3(kQuantThreads), 0,
                               stream, x, n8, in_scale, wsc);
        else
            hipLaunchKernelGGL((quantize_rows_kernel<false, false>), dim3(qblocks), dim3(kQuantThreads), 0,
                               stream, x, n8, in_scale, wsc);
    }
    G4_LAUNCHED("quantize_rows_kernel");
    *codes = wsc;
    return G4_OK;
}

// given_codes: a caller's buffer for the snapped codes (at least M * K bytes, checked by the
// caller), or null for the stream's workspace.
static int run_linear(int bits, const void *wq, const float *scales, const void *x, int x_kind,
                      void *dst, int out_kind, int k, int n, int m, float in_scale,
                      float out_scale, hipStream_t stream, const char *who, bool gemm_mode = true,
                      int8_t *given_codes = nullptr) {
    const KernelChoice c = pick_kernel(bits, m, n, k, in_scale, gemm_mode);
    if (c == K_SERIAL8) {
        const dim3 grid((n + 255) / 256, m);
        if (x_kind == G4_KIND_F16)
            hipLaunchKernelGGL(qmatmul8_serial_kernel<true>, grid, dim3(256), 0, stream,
                               reinterpret_cast<const int8_t *>(wq), scales, x, dst, out_kind, k, n,
                               out_scale);
        else
            hipLaunchKernelGGL(qmatmul8_serial_kernel<false>, grid, dim3(256), 0, stream,
                               reinterpret_cast<const int8_t *>(wq), scales, x, dst, out_kind, k, n,
                               out_scale);
        G4_LAUNCHED("qmatmul8_serial_kernel");
        return G4_OK;
    }
    if (c == K_GEMV || c == K_GEMV_F32 || c == K_GEMV_COLS)
        return gemv_columns(bits, wq, scales, x, x_kind, dst, out_kind, k, n, m, in_scale,
                            out_scale, stream, who);
    if (k > 16384)
        return set_error(G4_ERR_INVALID, "%s: K %d exceeds 16384 (the exact int32/f32 bound)", who, k);
    if (c == K_SKINNY16 || c == K_SKINNY32) {
        // One launch, the activation snap fused into the small-M kernel; or, past small_presnap,
        // the snap pass first (natural order: the kernel's int8 path interleaves for 4-bit).
        if (x_kind != G4_KIND_I8 && small_presnap(m, n, k)) {
            const int8_t *codes = nullptr;
            int rc = snap_pass(x, x_kind, m, k, in_scale, false, stream, given_codes, &codes);
            if (rc) return rc;
            x = codes;
            x_kind = G4_KIND_I8;
        }
        SmallJobs jobs{};
        jobs.w[0] = reinterpret_cast<const uint8_t *>(wq);
        jobs.scales[0] = scales;
        jobs.dst[0] = dst;
        jobs.n[0] = n;
        jobs.block_end[0] = (n + 15) / 16;
        jobs.count = 1;
        return launch_small(bits, c == K_SKINNY16 ? 16 : 32, 0, x, x_kind, jobs, m, k, in_scale,
                            out_scale, out_kind, stream);
    }
    // An int8 caller's natural-order codes go to the tile kernel as given (one launch; the 4-bit
    // B operand is permuted to match). f16 / f32 input is snapped once into a per-stream
    // workspace, interleaved for 4-bit weights so the tile kernel needs no permutes.
    const int8_t *codes = reinterpret_cast<const int8_t *>(x);
    const bool natural = x_kind == G4_KIND_I8;
    if (!natural) {
        int rc = snap_pass(x, x_kind, m, k, in_scale, bits == 4, stream, given_codes, &codes);
        if (rc) return rc;
    }
    const uint8_t *w = reinterpret_cast<const uint8_t *>(wq);
    if (c == K_WIDE) {
        const int tiles_m = (m + kWideBM - 1) / kWideBM;
        const int tiles_n = (n + kWideBN - 1) / kWideBN;
        const int blocks = tiles_m * ((tiles_n + 7) / 8) * 8;
        if (natural)
            hipLaunchKernelGGL(qgemm_wide_kernel<true>, dim3(blocks), dim3(512), 0, stream, codes, w,
                               scales, dst, m, n, k, in_scale, out_scale, out_kind, tiles_m, tiles_n);
        else
            hipLaunchKernelGGL(qgemm_wide_kernel<false>, dim3(blocks), dim3(512), 0, stream, codes, w,
                               scales, dst, m, n, k, in_scale, out_scale, out_kind, tiles_m, tiles_n);
        G4_LAUNCHED("qgemm_wide_kernel");
        return G4_OK;
    }
    if (bits == 4)
        return launch_tile<4>(codes, natural, w, scales, dst, m, n, k, in_scale, out_scale, out_kind,
                              stream);
    return launch_tile<8>(codes, natural, w, scales, dst, m, n, k, in_scale, out_scale, out_kind,
                          stream);
}

int linear_grouped(int bits, const void *x, int x_kind, int k, int m, float in_scale,
                   float out_scale, int out_kind, const LinearOut *outs, int count, void *stream) {
    if (!outs || count < 1) return set_error(G4_ERR_INVALID, "grouped linear: no outputs");
    const char *who = bits == 4 ? "qgemm-4bit" : "qmatmul-8bit";
    bool small = count <= kSmallMaxJobs && k <= 16384;
    for (int i = 0; i < count; ++i) {
        const LinearOut &o = outs[i];
        int rc = check_linear(bits, o.wq, o.scales, x, x_kind, o.dst, out_kind, k, o.n, m, in_scale,
                              out_scale, who);
        if (rc) return rc;
        const KernelChoice c = pick_kernel(bits, m, o.n, k, in_scale, false);
        small &= c == K_SKINNY16 || c == K_SKINNY32;
    }
    if (!small) {  // one call each, through the library's routing
        for (int i = 0; i < count; ++i) {
            int rc = run_linear(bits, outs[i].wq, outs[i].scales, x, x_kind, outs[i].dst, out_kind,
                                k, outs[i].n, m, in_scale, out_scale, as_stream(stream), who);
            if (rc) return rc;
        }
        return G4_OK;
    }
    SmallJobs jobs{};
    int blocks = 0;
    for (int i = 0; i < count; ++i) {
        jobs.w[i] = reinterpret_cast<const uint8_t *>(outs[i].wq);
        jobs.scales[i] = outs[i].scales;
        jobs.dst[i] = outs[i].dst;
        jobs.n[i] = outs[i].n;
        blocks += (outs[i].n + 15) / 16;
        jobs.block_end[i] = blocks;
    }
    jobs.count = count;
    return launch_small(bits, m <= 16 ? 16 : 32, 0, x, x_kind, jobs, m, k, in_scale, out_scale,
                        out_kind, as_stream(stream));
}

int linear_gelu(int bits, const void *x, int k, int m, float in_scale, float out_scale,
                const void *w_gate, const float *s_gate, const void *w_up, const float *s_up,
                const float *up_vec, int64_t up_stride, int n, float act_scale, int8_t *act,
                void *stream, bool *launched) {
    *launched = false;
    const char *who = "gelu linear";
    int rc = check_linear(bits, w_gate, s_gate, x, G4_KIND_I8, act, G4_KIND_I8, k, n, m, in_scale,
                          out_scale, who);
    if (rc) return rc;
    const KernelChoice c = pick_kernel(bits, m, n, k, in_scale, false);
    if ((c != K_SKINNY16 && c != K_SKINNY32) || k > 16384 || act_scale == 0.0f) return G4_OK;
    if (w_up ? (bits != 4 || !s_up || (reinterpret_cast<uintptr_t>(w_up) & 15)) : (!up_vec || up_stride < n))
        return set_error(G4_ERR_INVALID, "gelu linear: the up operand (4-bit paired rows with scales, "
                                         "or an f32 vector with stride >= n)");
    SmallJobs jobs{};
    jobs.w[0] = reinterpret_cast<const uint8_t *>(w_gate);
    jobs.scales[0] = s_gate;
    jobs.dst[0] = act;
    jobs.n[0] = n;
    jobs.block_end[0] = (n + 15) / 16;
    jobs.count = 1;
    jobs.w_up = reinterpret_cast<const uint8_t *>(w_up);
    jobs.s_up = s_up;
    jobs.aux = up_vec;
    jobs.aux_stride = up_stride;
    jobs.act_scale = act_scale;
    rc = launch_small(bits, c == K_SKINNY16 ? 16 : 32, w_up ? 1 : 2, x, G4_KIND_I8, jobs, m, k,
                      in_scale, out_scale, G4_KIND_I8, as_stream(stream));
    if (rc == G4_OK) *launched = true;
    return rc;
}

// The bind-time refusals of qgemm-4bit (qgemm.ts:589-639) and qmatmul-8bit (pleMatmul.ts:257-303).
static int check_qgemm(int bits, const void *wq, const float *scales, const void *x, int x_kind,
                       void *dst, int out_kind, int k, int num_rows, int m_cols, float in_scale,
                       float out_scale) {
    const char *who = bits == 4 ? "qgemm-4bit" : "qmatmul-8bit";
    if (bits == 4) {
        if (k <= 0 || num_rows <= 0 || m_cols <= 0)
            return set_error(G4_ERR_INVALID, "qgemm needs params.k, params.numRows and params.mCols");
        if (k % 256 != 0)
            return set_error(G4_ERR_INVALID, "qgemm-4bit needs K a multiple of 256, got %d", k);
    } else if (bits == 8) {
        if (k <= 0 || num_rows <= 0 || m_cols <= 0)
            return set_error(G4_ERR_INVALID,
                             "qmatmul-8bit needs params.k and params.numRows, with params.mCols "
                             "absent for a decode step");
        if (k % 4 != 0)
            return set_error(G4_ERR_INVALID,
                             "qmatmul-8bit needs K a multiple of 4, got %d. Both real tensors are 1536 "
                             "and 256, so a caller that does not is packing the wrong tensor.", k);
        if (k % 16 != 0)
            return set_error(G4_ERR_UNSUPPORTED,
                             "qmatmul-8bit: K %d is a multiple of 4 but not of 16, which this path "
                             "does not implement", k);
    } else {
        return set_error(G4_ERR_INVALID, "qgemm: bits must be 4 or 8, got %d", bits);
    }
    return check_linear(bits, wq, scales, x, x_kind, dst, out_kind, k, num_rows, m_cols, in_scale,
                        out_scale, who);
}

// g4_qgemm with the snapped-codes buffer supplied by the caller (codes_bytes bytes at `codes`):
// nothing is allocated. A call whose path needs more codes than that is refused.
int qgemm_given_codes(int bits, const void *wq, const float *scales, const void *x, int x_kind,
                      void *dst, int out_kind, int k, int num_rows, int m_cols, float in_scale,
                      float out_scale, void *stream, CodesSource source, size_t codes_bytes,
                      const char *who) {
    int rc = check_qgemm(bits, wq, scales, x, x_kind, dst, out_kind, k, num_rows, m_cols, in_scale,
                         out_scale);
    if (rc) return rc;
    int8_t *codes = nullptr;
    if (needs_codes_buffer(bits, m_cols, num_rows, k, in_scale, x_kind, true)) {
        const size_t need = (size_t)m_cols * (size_t)k;
        if (need > codes_bytes)
            return set_error(G4_ERR_INVALID,
                             "%s: M * K = %zu activation codes exceed the %zu-byte scratch buffer "
                             "(pass int8 codes already snapped, or a smaller M)",
                             who, need, codes_bytes);
        rc = source(&codes);
        if (rc) return rc;
    }
    return run_linear(bits, wq, scales, x, x_kind, dst, out_kind, k, num_rows, m_cols, in_scale,
                      out_scale, as_stream(stream), bits == 4 ? "qgemm-4bit" : "qmatmul-8bit", true,
                      codes);
}

}  // namespace g4

using namespace g4;

extern "C" {

// qgemm-4bit (qgemm.ts:589-639) and qmatmul-8bit (pleMatmul.ts:257-303).
int g4_qgemm(int bits, const void *wq, const float *scales, const void *x, int x_kind, void *dst,
             int out_kind, int k, int num_rows, int m_cols, float in_scale, float out_scale,
             void *stream) {
    int rc = check_qgemm(bits, wq, scales, x, x_kind, dst, out_kind, k, num_rows, m_cols, in_scale,
                         out_scale);
    if (rc) return rc;
    return run_linear(bits, wq, scales, x, x_kind, dst, out_kind, k, num_rows, m_cols, in_scale,
                      out_scale, as_stream(stream), bits == 4 ? "qgemm-4bit" : "qmatmul-8bit", true);
}

// execute.ts:372-430: a step over more than two tokens is gemm mode (qgemm-4bit / qmatmul-8bit),
// one or two tokens the decode GEMV family (qgemv-4/8bit, -m2).
int g4_linear(int bits, const void *wq, const float *scales, const void *x, int x_kind, void *dst,
              int out_kind, int k, int num_rows, int m_cols, float in_scale, float out_scale,
              void *stream) {
    int rc = check_qgemm(bits, wq, scales, x, x_kind, dst, out_kind, k, num_rows, m_cols, in_scale,
                         out_scale);
    if (rc) return rc;
    return run_linear(bits, wq, scales, x, x_kind, dst, out_kind, k, num_rows, m_cols, in_scale,
                      out_scale, as_stream(stream), bits == 4 ? "qgemm-4bit" : "qmatmul-8bit",
                      m_cols > 2);
}

int g4_kernel_for_shape(int bits, int m_cols, int num_rows, int k, char *buf, size_t buf_len) {
    if (!buf || buf_len == 0) return set_error(G4_ERR_INVALID, "g4_kernel_for_shape: no buffer");
    const KernelChoice c = pick_kernel(bits, m_cols, num_rows, k, 1.0f, true);
    const char *name = choice_name(c, bits);
    if (c == K_GEMV && m_cols == 1 && stream_class_for(bits, k) >= 0)
        name = bits == 4 ? "qgemv-4bit-stream" : "qgemv-8bit-stream";
    snprintf(buf, buf_len, "%s", name);
    return G4_OK;
}

int g4_srq_quantize(const void *x, int x_kind, int8_t *codes, int64_t n, float scale,
                    void *stream) {
    if (!x || !codes || n < 0) return set_error(G4_ERR_INVALID, "srq quantize: bad arguments");
    if (x_kind != G4_KIND_F32 && x_kind != G4_KIND_F16)
        return set_error(G4_ERR_INVALID, "srq quantize: x_kind must be f32 or f16");
    if (scale == 0.0f)
        return set_error(G4_ERR_INVALID, "srq quantize: a scale of 0.0 means uncalibrated; there are no codes");
    if (n == 0) return G4_OK;
    int64_t blocks = (n + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL(srq_quantize_kernel, dim3((unsigned)blocks), dim3(256), 0, as_stream(stream),
                       x, x_kind, codes, n, scale);
    G4_LAUNCHED("srq_quantize_kernel");
    return G4_OK;
}

}  // extern "C"

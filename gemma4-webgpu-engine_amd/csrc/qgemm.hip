// The M-column quantized linears on gfx950 int8 MFMA: qgemm-4bit (src/kernels/qgemm.ts) and
// qmatmul-8bit (src/kernels/pleMatmul.ts), plus the shape routing of src/execute.ts:372-430.
//
// Pipeline of one call (calibrated path):
//  1. quantize_rows_kernel snaps x [M][K] once into int8 codes (the SRQ input prologue), written
//     to a per-stream workspace with each 8-code group interleaved [x0 x2 x4 x6 x1 x3 x5 x7] for
//     4-bit weights (so a weight word's low and high nibble lanes line up with the codes without
//     a shuffle), and sum(xq) per row for the 4-bit zero point.
//  2. An MFMA kernel contracts codes x weights with v_mfma_i32_16x16x64_i8. The 4-bit weights are
//     unpacked to unsigned nibbles (w & 0x0F0F0F0F, (w >> 4) & 0x0F0F0F0F) and the zero point comes
//     off once per output as -8 * sum(xq[m]). The int32 accumulators are exact, so the k order the
//     MFMA uses internally is irrelevant; only the A and B operands have to agree on it, and they
//     do because both are filled with the same (lane group, byte) -> k assignment.
//  3. The epilogue is the reference's f32(f32(inScale * scale[n]) * f32(acc)) and output snap.
//
// Kernels by M (chosen per shape, see pick_kernel):
//   M <= 2         the GEMV family (qgemv.hip): bit-identical, cheaper than any tile at this M.
//   3 <= M <= 32   qgemm_small_kernel: one launch with the snap fused (codes in LDS), 16 weight
//                  rows per block, the 4 waves split K, an LDS fold of the 4 partials.
//   M > 32         qgemm_mfma_kernel: 64 x 96 output tiles, activation codes straight to registers,
//                  weights expanded to int8 in double-buffered LDS, XCD-aware tile order.
#include "g4_internal.h"

#include <algorithm>
#include <map>
#include <mutex>
#include <utility>

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

// One block per token row: snap K activations into codes (interleaved when PERM), zero the pad to
// kp, and write sum(codes) for the row.
template <bool PERM>
__global__ __launch_bounds__(kQuantThreads) void quantize_rows_kernel(
    const void *x, int x_kind, int k, int kp, float scale, int8_t *codes, int *row_sums) {
    __shared__ int s_sum;
    const int m = blockIdx.x;
    const int tid = threadIdx.x;
    if (tid == 0) s_sum = 0;
    __syncthreads();
    int local = 0;
    const int groups = kp >> 3;
    const int live = k >> 3;
    bool r_ok;
    const float r = srq_recip(scale, r_ok);
    for (int g = tid; g < groups; g += kQuantThreads) {
        int c[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        if (g < live) {
            const int64_t e = (int64_t)m * k + (int64_t)g * 8;
            if (x_kind == G4_KIND_I8) {
                const uint2 v = *reinterpret_cast<const uint2 *>(reinterpret_cast<const int8_t *>(x) + e);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    c[i] = (int)(int8_t)((v.x >> (8 * i)) & 0xff);
                    c[4 + i] = (int)(int8_t)((v.y >> (8 * i)) & 0xff);
                }
            } else {
#pragma unroll
                for (int i = 0; i < 8; ++i)
                    c[i] = (int)srq_code_fast(load_act(x, x_kind, e + i), scale, r, r_ok);
            }
        }
        uint2 out;
        if (PERM) {
            out.x = pack4b(c[0], c[2], c[4], c[6]);
            out.y = pack4b(c[1], c[3], c[5], c[7]);
        } else {
            out.x = pack4b(c[0], c[1], c[2], c[3]);
            out.y = pack4b(c[4], c[5], c[6], c[7]);
        }
        *reinterpret_cast<uint2 *>(codes + (int64_t)m * kp + (int64_t)g * 8) = out;
        local += c[0] + c[1] + c[2] + c[3] + c[4] + c[5] + c[6] + c[7];
    }
    local = row16_sum_i32(local);
    if ((tid & 15) == 0 && local != 0) atomicAdd(&s_sum, local);
    __syncthreads();
    if (tid == 0) row_sums[m] = s_sum;
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

// ---- small M: M <= MT token rows, 16 weight rows per block, K split over the 4 waves ----------
// The activation snap is fused: the block snaps its MT token rows into LDS as int8 codes (the
// 4-bit interleave per 8-code group) one K chunk at a time, so a draft-verify or small prefill
// call is one launch. The 4-bit zero point needs sum(xq) per token row: one more MFMA per step
// against an all-ones B operand gives it exactly, folded with the partials like the products. Lane (j = lane % 16, g = lane / 16)
// owns weight row n0 + j; per 128-code stage it loads 16 bytes of that row (8-bit: 32), and MFMA
// half-step s takes codes g*32 + s*16 .. +16 of the stage from both operands. The LDS rows are
// padded by 16 bytes so the 16 token rows of one A read fall on distinct banks.
template <int BITS, int MT>
__global__ __launch_bounds__(256) void qgemm_small_kernel(
    const void *__restrict__ x, int x_kind, const uint8_t *__restrict__ W,
    const float *__restrict__ scales, void *dst, int M, int N, int K, float in_scale,
    float out_scale, int out_kind) {
    constexpr int TM = MT / 16;
    constexpr int KC = 32768 / MT;     // codes of a row per LDS chunk
    constexpr int XSTR = KC + 16;      // LDS bytes per token row
    constexpr int BATCH = 4;
    constexpr int NACC = BITS == 4 ? 2 * TM : TM;  // products, then (4-bit) the row sums
    __shared__ __align__(16) int8_t xs[MT * XSTR];
    __shared__ v4i red[3][NACC][64];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int j = lane & 15;
    const int g = lane >> 4;
    const int n0 = blockIdx.x * 16;
    const int m0 = blockIdx.y * MT;
    const int n = min(n0 + j, N - 1);
    const int row_bytes = BITS == 4 ? (K >> 1) : K;
    const uint8_t *wrow = W + (int64_t)n * row_bytes;
    bool r_ok;
    const float rcp = srq_recip(in_scale, r_ok);
    v4i acc[NACC];
#pragma unroll
    for (int t = 0; t < NACC; ++t) acc[t] = v4i{0, 0, 0, 0};
    const v4i ones = v4i{0x01010101, 0x01010101, 0x01010101, 0x01010101};

    for (int kc0 = 0; kc0 < K; kc0 += KC) {
        const int kcn = min(KC, K - kc0);
        const int gpr = kcn >> 3;  // 8-code groups per row in this chunk
        lds_barrier();  // the previous chunk's codes are no longer read
        for (int q = tid; q < MT * gpr; q += 256) {
            const int r = q / gpr, gi = q - r * gpr;
            const int m = m0 + r;
            int c[8] = {0, 0, 0, 0, 0, 0, 0, 0};
            if (m < M) {
                const int64_t e = (int64_t)m * K + kc0 + gi * 8;
                if (x_kind == G4_KIND_I8) {
                    const uint2 v = *reinterpret_cast<const uint2 *>(reinterpret_cast<const int8_t *>(x) + e);
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        c[i] = (int)(int8_t)((v.x >> (8 * i)) & 0xff);
                        c[4 + i] = (int)(int8_t)((v.y >> (8 * i)) & 0xff);
                    }
                } else if (x_kind == G4_KIND_F16) {
                    const u32x4 v = *reinterpret_cast<const u32x4 *>(reinterpret_cast<const __half *>(x) + e);
                    const uint32_t h[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        c[2 * i] = (int)srq_code_fast(
                            __half2float(__ushort_as_half((unsigned short)(h[i] & 0xffff))), in_scale, rcp, r_ok);
                        c[2 * i + 1] = (int)srq_code_fast(
                            __half2float(__ushort_as_half((unsigned short)(h[i] >> 16))), in_scale, rcp, r_ok);
                    }
                } else {
                    const float4 *p4 = reinterpret_cast<const float4 *>(reinterpret_cast<const float *>(x) + e);
                    const float4 v0 = p4[0], v1 = p4[1];
                    const float v[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
#pragma unroll
                    for (int i = 0; i < 8; ++i) c[i] = (int)srq_code_fast(v[i], in_scale, rcp, r_ok);
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
        lds_barrier();
        const int ksteps = kcn / kTileBK;
        const int kbase = kc0 / kTileBK;
        for (int kb0 = wave; kb0 < ksteps; kb0 += 4 * BATCH) {
            u32x4 bw[BATCH][BITS == 4 ? 1 : 2];
#pragma unroll
            for (int u = 0; u < BATCH; ++u) {
                const int kb = min(kb0 + 4 * u, ksteps - 1);  // clamped: every load is valid
                if (BITS == 4) {
                    bw[u][0] = *reinterpret_cast<const u32x4 *>(wrow + (kbase + kb) * 64 + g * 16);
                } else {
                    bw[u][0] = *reinterpret_cast<const u32x4 *>(wrow + (kbase + kb) * 128 + g * 32);
                    bw[u][BITS == 4 ? 0 : 1] =
                        *reinterpret_cast<const u32x4 *>(wrow + (kbase + kb) * 128 + g * 32 + 16);
                }
            }
#pragma unroll
            for (int u = 0; u < BATCH; ++u) {
                const int kb = kb0 + 4 * u;
                if (kb < ksteps) {
#pragma unroll
                    for (int s = 0; s < 2; ++s) {
                        v4i b;
                        if (BITS == 4)
                            b = b_operand<4>(bw[u][0].x, bw[u][0].y, bw[u][0].z, bw[u][0].w, s);
                        else
                            b = __builtin_bit_cast(v4i, bw[u][BITS == 4 ? 0 : s]);
#pragma unroll
                        for (int t = 0; t < TM; ++t) {
                            const v4i a = *reinterpret_cast<const v4i *>(
                                &xs[(t * 16 + j) * XSTR + kb * kTileBK + g * 32 + s * 16]);
                            acc[t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, acc[t], 0, 0, 0);
                            if (BITS == 4 && s == 0)  // each code counted once: both halves
                                acc[TM + t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, ones, acc[TM + t], 0, 0, 0);
                            if (BITS == 4 && s == 1)
                                acc[TM + t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, ones, acc[TM + t], 0, 0, 0);
                        }
                    }
                }
            }
        }
    }
    // Fold the four waves' partial tiles through LDS, then wave 0 writes.
    if (wave > 0) {
#pragma unroll
        for (int t = 0; t < NACC; ++t) red[wave - 1][t][lane] = acc[t];
    }
    __syncthreads();
    if (wave == 0) {
        bool o_ok;
        const float orcp = srq_recip(out_scale, o_ok);
        const int nn = n0 + j;
        if (nn < N) {
            const float rs = __fmul_rn(in_scale, scales[nn]);
#pragma unroll
            for (int t = 0; t < TM; ++t) {
                v4i a = acc[t];
                v4i rsum = BITS == 4 ? acc[TM + t] : v4i{0, 0, 0, 0};
#pragma unroll
                for (int w = 0; w < 3; ++w) {
                    a += red[w][t][lane];
                    if (BITS == 4) rsum += red[w][TM + t][lane];
                }
                // D layout: lane l, register r -> row 4 (l / 16) + r of A, column l % 16 of B.
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int lr = t * 16 + 4 * g + r;
                    const int m = m0 + lr;
                    if (m < M) {
                        int v = a[r];
                        if (BITS == 4) v -= 8 * rsum[r];  // the ones product: sum(xq) of row lr
                        const float yv = __fmul_rn(rs, (float)v);
                        const int64_t o = (int64_t)m * N + nn;
                        if (out_kind == G4_KIND_I8) {
                            reinterpret_cast<int8_t *>(dst)[o] = (int8_t)srq_code_fast(yv, out_scale, orcp, o_ok);
                        } else if (out_kind == G4_KIND_I32) {
                            reinterpret_cast<int32_t *>(dst)[o] = v;
                        } else {
                            float f = yv;
                            if (out_scale != 0.0f) f = __fmul_rn(srq_code_fast(yv, out_scale, orcp, o_ok), out_scale);
                            reinterpret_cast<float *>(dst)[o] = f;
                        }
                    }
                }
            }
        }
    }
}

// ---- tile: 64 x 96 outputs per block, K in 128-code stages ---------------------------------------
// Block = 4 waves stacked along M; wave w owns rows m0 + 16 w .. +16 and all 96 columns (6 MFMA
// column tiles). Two blocks share a CU (two waves per SIMD), so one wave's MFMAs cover the other's
// LDS and barrier latency.
//  A (activation codes) goes straight from global memory into registers: lane (j = lane % 16,
//    g = lane / 16) loads bytes s * 64 + g * 16 .. +16 of its row for MFMA half-step s, so one
//    load instruction covers 16 rows x 64 contiguous bytes. No LDS traffic for A.
//  B (weights) is staged through double-buffered LDS once per block, expanded to int8 codes on the
//    way (4-bit: nibbles into the activation interleave [k0 k2 k4 k6 k1 k3 k5 k7]; 8-bit: as is),
//    so the inner loop is LDS reads plus MFMAs. Column stride 144 bytes keeps the 16-lane reads on
//    distinct banks.
//  Loads run D stages ahead through a register ring written out with compile-time slots, so the
//  wait counts stay partial (a load behind a branch would drain them).
// The integer sums are exact; A and B agree on the k assignment inside every MFMA, so the order
// the matrix core sums in does not matter.
constexpr int kMfmaBN = 96;
constexpr int kMfmaBM = 64;

template <int BITS>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 8))) void qgemm_mfma_kernel(
    const int8_t *__restrict__ A, const int *__restrict__ row_sums, const uint8_t *__restrict__ W,
    const float *__restrict__ scales, void *dst, int M, int N, int K, int kp, float in_scale,
    float out_scale, int out_kind, int tiles_m, int tiles_n) {
    constexpr int BN = kMfmaBN, TN = BN / 16, D = 2;
    constexpr int BROW = BITS == 4 ? 64 : 128;  // weight bytes of one column per stage
    constexpr int BSTR = 144;                   // LDS bytes per column: 128 codes + 16 pad
    constexpr int B_CHUNKS = BN * BROW / 16;
    constexpr int B_CH = (B_CHUNKS + 255) / 256;
    constexpr int CPC = BROW / 16;              // 16-byte weight chunks per column per stage
    __shared__ __align__(16) uint8_t sB[2][BN * BSTR];

    const int b = blockIdx.x;
    // Blocks are dealt to the 8 XCDs round robin: give one XCD every M tile of a run of N tiles,
    // so its L2 fetches those weight columns once.
    const int xcd = b & 7, idx = b >> 3;
    const int tm = idx % tiles_m;
    const int tn = (idx / tiles_m) * 8 + xcd;
    if (tn >= tiles_n) return;
    const int m0 = tm * kMfmaBM, n0 = tn * BN;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int j = lane & 15, g = lane >> 4;
    const int ksteps = K / 128;
    const int row_bytes = BITS == 4 ? K / 2 : K;
    const int8_t *arow = A + (int64_t)min(m0 + wave * 16 + j, M - 1) * kp + g * 16;
    const uint8_t *bsrc[B_CH];
    int bdst[B_CH];
#pragma unroll
    for (int i = 0; i < B_CH; ++i) {
        const int q = min(tid + 256 * i, B_CHUNKS - 1);
        const int col = q / CPC, c = q % CPC;
        bsrc[i] = W + (int64_t)min(n0 + col, N - 1) * row_bytes + c * 16;
        bdst[i] = col * BSTR + c * (BITS == 4 ? 32 : 16);
    }
    // The epilogue's per-row zero-point sums and per-column scales, requested before the K loop so
    // their latency is not added after it.
    int rsum[4];
#pragma unroll
    for (int r = 0; r < 4; ++r)
        rsum[r] = BITS == 4 ? 8 * row_sums[min(m0 + wave * 16 + 4 * g + r, M - 1)] : 0;
    float col_scale[TN];
#pragma unroll
    for (int y = 0; y < TN; ++y) col_scale[y] = __fmul_rn(in_scale, scales[min(n0 + y * 16 + j, N - 1)]);
    v4i acc[TN];
#pragma unroll
    for (int y = 0; y < TN; ++y) acc[y] = v4i{0, 0, 0, 0};
    u32x4 ra[D][2];
    u32x4 rb[D][B_CH];
    auto load = [&](u32x4 (&xa)[2], u32x4 (&xb)[B_CH], int st) {
        const int s_ = min(st, ksteps - 1);  // past the end: re-read the last stage, unguarded
        xa[0] = *reinterpret_cast<const u32x4 *>(arow + s_ * 128);
        xa[1] = *reinterpret_cast<const u32x4 *>(arow + s_ * 128 + 64);
#pragma unroll
        for (int i = 0; i < B_CH; ++i) xb[i] = *reinterpret_cast<const u32x4 *>(bsrc[i] + s_ * BROW);
    };
    // Threads past the last chunk hold a copy of it (clamped index) and store it to the same place.
    auto store_b = [&](const u32x4 (&xb)[B_CH], int buf) {
#pragma unroll
        for (int i = 0; i < B_CH; ++i) {
            const u32x4 w = xb[i];
            if (BITS == 4) {
                const u32x4 e0{w.x & 0x0F0F0F0Fu, (w.x >> 4) & 0x0F0F0F0Fu, w.y & 0x0F0F0F0Fu,
                               (w.y >> 4) & 0x0F0F0F0Fu};
                const u32x4 e1{w.z & 0x0F0F0F0Fu, (w.z >> 4) & 0x0F0F0F0Fu, w.w & 0x0F0F0F0Fu,
                               (w.w >> 4) & 0x0F0F0F0Fu};
                *reinterpret_cast<u32x4 *>(&sB[buf][bdst[i]]) = e0;
                *reinterpret_cast<u32x4 *>(&sB[buf][bdst[i] + 16]) = e1;
            } else {
                *reinterpret_cast<u32x4 *>(&sB[buf][bdst[i]]) = w;
            }
        }
    };
#pragma unroll
    for (int i = 0; i < D; ++i) load(ra[i], rb[i], i);
    store_b(rb[0], 0);
    lds_barrier();
    // Stage st consumes ring slot st % D and refills it with stage st + D. Whole groups of D stages
    // run unguarded (a branch around the loads would make the wait counts drain at the loop head);
    // a final odd stage is peeled.
    auto stage = [&](u32x4 (&xa)[2], u32x4 (&xb)[B_CH], const u32x4 (&xb_next)[B_CH], int st) {
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            v4i bo[TN];
#pragma unroll
            for (int y = 0; y < TN; ++y)
                bo[y] = *reinterpret_cast<const v4i *>(
                    &sB[st & 1][(y * 16 + j) * BSTR + (s * 4 + g) * 16]);
#pragma unroll
            for (int y = 0; y < TN; ++y)
                acc[y] = __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(v4i, xa[s]), bo[y],
                                                               acc[y], 0, 0, 0);
        }
        store_b(xb_next, (st + 1) & 1);
        load(xa, xb, st + D);
        lds_barrier();
    };
    static_assert(D == 2, "the ring below is written out for two slots");
    int st = 0;
    for (; st + 2 <= ksteps; st += 2) {
        stage(ra[0], rb[0], rb[1], st);
        stage(ra[1], rb[1], rb[0], st + 1);
    }
    if (st < ksteps) stage(ra[0], rb[0], rb[1], st);
    // D layout of a 16 x 16 MFMA tile: lane l, register r -> row 4 (l / 16) + r, column l % 16.
    // The outputs go through LDS so each row of the tile leaves as whole 16-byte stores (scattered
    // byte stores of 16-byte runs cost more than the contraction). Edge tiles and rows whose start
    // is not 16-byte aligned keep per-element stores.
    bool r_ok;
    const float rcp = srq_recip(out_scale, r_ok);
    const int esz = out_kind == G4_KIND_I8 ? 1 : 4;
    const bool full = m0 + kMfmaBM <= M && n0 + BN <= N && ((int64_t)N * esz) % 16 == 0;
    lds_barrier();  // every wave is done reading the last stage's weights
    uint8_t *stile = &sB[0][0];  // 64 x 96 outputs: 6 KB (int8) or 24 KB (f32 / int32) of LDS
    static_assert(2 * BN * BSTR >= kMfmaBM * BN * 4, "the output tile fits the weight buffers");
#pragma unroll
    for (int y = 0; y < TN; ++y) {
        const int n = n0 + y * 16 + j;
        const float rs = col_scale[y];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int lr = wave * 16 + 4 * g + r;
            const int m = m0 + lr;
            const int v = acc[y][r] - rsum[r];
            const float yv = __fmul_rn(rs, (float)v);
            if (full) {
                const int o = lr * BN + y * 16 + j;
                if (out_kind == G4_KIND_I8) {
                    stile[o] = (uint8_t)(int8_t)srq_code_fast(yv, out_scale, rcp, r_ok);
                } else if (out_kind == G4_KIND_I32) {
                    reinterpret_cast<int32_t *>(stile)[o] = v;
                } else {
                    float f = yv;
                    if (out_scale != 0.0f) f = __fmul_rn(srq_code_fast(yv, out_scale, rcp, r_ok), out_scale);
                    reinterpret_cast<float *>(stile)[o] = f;
                }
            } else if (m < M && n < N) {
                const int64_t o = (int64_t)m * N + n;
                if (out_kind == G4_KIND_I8) {
                    reinterpret_cast<int8_t *>(dst)[o] = (int8_t)srq_code_fast(yv, out_scale, rcp, r_ok);
                } else if (out_kind == G4_KIND_I32) {
                    reinterpret_cast<int32_t *>(dst)[o] = v;
                } else {
                    float f = yv;
                    if (out_scale != 0.0f) f = __fmul_rn(srq_code_fast(yv, out_scale, rcp, r_ok), out_scale);
                    reinterpret_cast<float *>(dst)[o] = f;
                }
            }
        }
    }
    if (!full) return;  // uniform
    lds_barrier();
    const int row_chunks = BN * esz / 16;  // 6 (int8) or 24 (f32 / int32)
    for (int q = tid; q < kMfmaBM * row_chunks; q += 256) {
        const int lr = q / row_chunks, c = q - lr * row_chunks;
        const u32x4 v = *reinterpret_cast<const u32x4 *>(stile + lr * BN * esz + c * 16);
        *reinterpret_cast<u32x4 *>(reinterpret_cast<uint8_t *>(dst) +
                                   ((int64_t)(m0 + lr) * N + n0) * esz + c * 16) = v;
    }
}

// ---- per-stream workspace for the snapped activation codes ------------------------------------

struct Workspace {
    void *ptr = nullptr;
    size_t bytes = 0;
};

static std::mutex g_ws_mu;
static std::map<std::pair<int, void *>, Workspace> g_ws;

// Returns a device buffer of at least `bytes` owned by (device, stream). Calls on one stream are
// ordered, so they may share it; calls on different streams get different buffers.
static int workspace(void *stream, size_t bytes, void **out) {
    int dev = 0;
    G4_HIP(hipGetDevice(&dev));
    std::lock_guard<std::mutex> lock(g_ws_mu);
    Workspace &ws = g_ws[{dev, stream}];
    if (ws.bytes < bytes) {
        if (ws.ptr) {
            G4_HIP(hipStreamSynchronize(as_stream(stream)));
            G4_HIP(hipFree(ws.ptr));
            ws.ptr = nullptr;
            ws.bytes = 0;
        }
        size_t grow = std::max(bytes, (size_t)4 << 20);
        G4_HIP(hipMalloc(&ws.ptr, grow));
        ws.bytes = grow;
    }
    *out = ws.ptr;
    return G4_OK;
}

enum KernelChoice { K_GEMV = 0, K_SKINNY16, K_SKINNY32, K_TILE128, K_GEMV_F32, K_GEMV_COLS };

static KernelChoice pick_kernel(int bits, int m, int n, int k, float in_scale) {
    (void)n;
    if (in_scale == 0.0f) return K_GEMV_F32;
    if (m <= 2) return K_GEMV;
    if (k % kTileBK != 0) return K_GEMV_COLS;
    if (m <= 16) return K_SKINNY16;
    if (m <= 32) return K_SKINNY32;
    (void)bits;
    return K_TILE128;
}

static const char *choice_name(KernelChoice c, int bits) {
    switch (c) {
        case K_GEMV: return bits == 4 ? "qgemv-4bit" : "qgemv-8bit";
        case K_SKINNY16: return bits == 4 ? "qgemm-4bit-mfma-small16" : "qmatmul-8bit-mfma-small16";
        case K_SKINNY32: return bits == 4 ? "qgemm-4bit-mfma-small32" : "qmatmul-8bit-mfma-small32";
        case K_TILE128: return bits == 4 ? "qgemm-4bit-mfma-tile" : "qmatmul-8bit-mfma-tile";
        case K_GEMV_F32: return bits == 4 ? "qgemv-4bit-f32" : "qgemv-8bit-f32";
        default: return bits == 4 ? "qgemv-4bit-columns" : "qgemv-8bit-columns";
    }
}

template <int BITS>
static int launch_mfma(KernelChoice c, const int8_t *codes, const int *sums, const uint8_t *w,
                       const float *scales, void *dst, int m, int n, int k, int kp,
                       float in_scale, float out_scale, int out_kind, hipStream_t stream) {
    const int tiles_m = (m + kMfmaBM - 1) / kMfmaBM;
    const int tiles_n = (n + kMfmaBN - 1) / kMfmaBN;
    const int blocks = tiles_m * ((tiles_n + 7) / 8) * 8;  // XCD-aware order: whole groups of 8
    hipLaunchKernelGGL((qgemm_mfma_kernel<BITS>), dim3(blocks), dim3(256), 0, stream, codes, sums,
                       w, scales, dst, m, n, k, kp, in_scale, out_scale, out_kind, tiles_m, tiles_n);
    G4_LAUNCHED("qgemm_mfma_kernel");
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

static int run_linear(int bits, const void *wq, const float *scales, const void *x, int x_kind,
                      void *dst, int out_kind, int k, int n, int m, float in_scale,
                      float out_scale, hipStream_t stream, const char *who) {
    const KernelChoice c = pick_kernel(bits, m, n, k, in_scale);
    if (c == K_GEMV || c == K_GEMV_F32 || c == K_GEMV_COLS)
        return gemv_columns(bits, wq, scales, x, x_kind, dst, out_kind, k, n, m, in_scale,
                            out_scale, stream, who);
    if (k > 16384)
        return set_error(G4_ERR_INVALID, "%s: K %d exceeds 16384 (the exact int32/f32 bound)", who, k);
    if (c == K_SKINNY16 || c == K_SKINNY32) {
        // One launch: the activation snap is fused into the small-M kernel.
        const int mt = c == K_SKINNY16 ? 16 : 32;
        dim3 grid((n + 15) / 16, (m + mt - 1) / mt);
        const uint8_t *w = reinterpret_cast<const uint8_t *>(wq);
#define G4_SMALL(B, T)                                                                           \
    hipLaunchKernelGGL((qgemm_small_kernel<B, T>), grid, dim3(256), 0, stream, x, x_kind, w, scales, \
                       dst, m, n, k, in_scale, out_scale, out_kind)
        if (bits == 4 && mt == 16) G4_SMALL(4, 16);
        else if (bits == 4) G4_SMALL(4, 32);
        else if (mt == 16) G4_SMALL(8, 16);
        else G4_SMALL(8, 32);
#undef G4_SMALL
        G4_LAUNCHED("qgemm_small_kernel");
        return G4_OK;
    }
    const int kp = k;  // k % 128 == 0 on the MFMA kernels
    const size_t code_bytes = (size_t)m * kp;
    const size_t sum_off = (code_bytes + 255) & ~(size_t)255;
    void *ws = nullptr;
    int rc = workspace(stream, sum_off + (size_t)m * sizeof(int), &ws);
    if (rc) return rc;
    int8_t *codes = reinterpret_cast<int8_t *>(ws);
    int *sums = reinterpret_cast<int *>(reinterpret_cast<uint8_t *>(ws) + sum_off);
    if (bits == 4)
        hipLaunchKernelGGL(quantize_rows_kernel<true>, dim3(m), dim3(kQuantThreads), 0, stream, x,
                           x_kind, k, kp, in_scale, codes, sums);
    else
        hipLaunchKernelGGL(quantize_rows_kernel<false>, dim3(m), dim3(kQuantThreads), 0, stream, x,
                           x_kind, k, kp, in_scale, codes, sums);
    G4_LAUNCHED("quantize_rows_kernel");
    const uint8_t *w = reinterpret_cast<const uint8_t *>(wq);
    if (bits == 4)
        return launch_mfma<4>(c, codes, sums, w, scales, dst, m, n, k, kp, in_scale, out_scale,
                              out_kind, stream);
    return launch_mfma<8>(c, codes, sums, w, scales, dst, m, n, k, kp, in_scale, out_scale,
                          out_kind, stream);
}

}  // namespace g4

using namespace g4;

extern "C" {

// qgemm-4bit (qgemm.ts:589-639) and qmatmul-8bit (pleMatmul.ts:257-303).
int g4_qgemm(int bits, const void *wq, const float *scales, const void *x, int x_kind, void *dst,
             int out_kind, int k, int num_rows, int m_cols, float in_scale, float out_scale,
             void *stream) {
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
    int rc = check_linear(bits, wq, scales, x, x_kind, dst, out_kind, k, num_rows, m_cols,
                          in_scale, out_scale, who);
    if (rc) return rc;
    return run_linear(bits, wq, scales, x, x_kind, dst, out_kind, k, num_rows, m_cols, in_scale,
                      out_scale, as_stream(stream), who);
}

int g4_linear(int bits, const void *wq, const float *scales, const void *x, int x_kind, void *dst,
              int out_kind, int k, int num_rows, int m_cols, float in_scale, float out_scale,
              void *stream) {
    return g4_qgemm(bits, wq, scales, x, x_kind, dst, out_kind, k, num_rows, m_cols, in_scale,
                    out_scale, stream);
}

int g4_kernel_for_shape(int bits, int m_cols, int num_rows, int k, char *buf, size_t buf_len) {
    if (!buf || buf_len == 0) return set_error(G4_ERR_INVALID, "g4_kernel_for_shape: no buffer");
    const KernelChoice c = pick_kernel(bits, m_cols, num_rows, k, 1.0f);
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

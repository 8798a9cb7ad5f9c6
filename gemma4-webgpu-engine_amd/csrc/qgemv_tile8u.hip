// qgemv-4bit over the eight-row tile layout: the `tile8u` inner loop of src/kernels/qgemv.ts:870-1015
// (the geometry the 4-bit pipeline compiles when GemvGeometry.inner is 'tile8u', qgemv.ts:440),
// with its gelu prologue (GemvPrologue 'gelu'), and the repack that builds the layout from the
// checkpoint's row layout.
//
// Layout (qgemv.ts:871-876): rows in tiles of eight; tile t holds K u32 words, and word k carries
// the unsigned code (0..15, zero point 8) of row 8t + r at bits 4r .. 4r + 3. Rows past the row
// count (a partial last tile) are written as code 8.
//
// The loop's mapping (qgemv.ts:955-989): one 32-lane group owns one tile, so here each half of a
// wave64 is that group and a 64-thread block owns two tiles. Lane l takes the 16-byte word vector
// l + 32 i, the codes of k = 128 i + 4 l + j (j = 0..3), against activations k .. k + 3.
//  - Calibrated (inScale != 0): the activations snapped to int8 codes. The per-lane sum over
//    every row is exact in int32, so any exact method gives the reference's integers; this one
//    transposes the four words into per-row byte vectors (two byte permutes per output word, and
//    a nibble mask for even and odd rows) and takes four products per v_dot4 against the lane's
//    four codes. The zero point comes off once per lane: f32(sum(u x) - 8 sum(x)), as the shader
//    does before its reduction.
//    From K = 768 up, a block of S half-waves takes one tile and splits its K loop S ways (at least
//    three iterations each), summing the lane values in int32: exact, so the same f32 result, with
//    S times the waves in flight (one half-wave per tile leaves a 1536-row projection 96 waves).
//  - Uncalibrated: the shader's f32 order, one multiply and one add per element (no FMA):
//    acc_r += f32(u_r) * x_j over i then j, the activation sum beside it, then acc_r - 8 * sum.
// Then each row's 32 lane values are summed as mmSum does on the subgroup path (qgemv.ts:311-316,
// sgSum32 of subgroupReduce.ts:49-59: x + shuffleXor(x, m) for m = 1, 2, 4, 8, 16; the workgroup
// fallback's tree differs in the last bits, subgroupReduce.ts:61-67), and lane 0 applies the
// epilogue f32(f32(xs * scale) * sum) with the output snap (xs = inScale, or 1 uncalibrated). A
// tile past the last one reads the last tile clamped, and its rows fail the store guard
// (qgemv.ts:962-965, 1004-1008).
#include "g4_internal.h"

namespace g4 {

constexpr int kT8Threads = 64;  // two tiles (one per half-wave) per block

__global__ __launch_bounds__(256) void tile8u_repack_kernel(const uint8_t *w, uint32_t *out, int k, int n,
                                                            int64_t words) {
    const int64_t row_bytes = k >> 1;
    for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < words;
         idx += (int64_t)gridDim.x * blockDim.x) {
        const int64_t t = idx / k;
        const int kk = (int)(idx - t * k);
        uint32_t word = 0;
#pragma unroll
        for (int r = 0; r < 8; ++r) {
            const int64_t row = t * 8 + r;
            const uint32_t nib = row < n ? (w[row * row_bytes + (kk >> 1)] >> (4 * (kk & 1))) & 15u : 8u;
            word |= nib << (4 * r);
        }
        out[idx] = word;
    }
}

// The activation values k .. k + 3 as f32: x (f32 or f16), or the gelu prologue's product.
__device__ __forceinline__ void t8_act4(const void *x, int x_kind, const GeluAct &act, bool gelu,
                                        int64_t e, float v[4]) {
    if (gelu) {
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = gelu_act_value(act, x, x_kind, e + j);
    } else if (x_kind == G4_KIND_F16) {
        const uint2 h = *reinterpret_cast<const uint2 *>(reinterpret_cast<const __half *>(x) + e);
        v[0] = __half2float(__ushort_as_half((unsigned short)(h.x & 0xffff)));
        v[1] = __half2float(__ushort_as_half((unsigned short)(h.x >> 16)));
        v[2] = __half2float(__ushort_as_half((unsigned short)(h.y & 0xffff)));
        v[3] = __half2float(__ushort_as_half((unsigned short)(h.y >> 16)));
    } else {
        const float4 f = *reinterpret_cast<const float4 *>(reinterpret_cast<const float *>(x) + e);
        v[0] = f.x, v[1] = f.y, v[2] = f.z, v[3] = f.w;
    }
}

// The four codes of k .. k + 3 as one word of signed bytes (k in the low byte), and their sum.
__device__ __forceinline__ uint32_t t8_codes4(const void *x, int x_kind, const GeluAct &act, bool gelu,
                                              int64_t e, float s, float rcp, bool r_ok, int &sum) {
    int c[4];
    if (!gelu && x_kind == G4_KIND_I8) {
        const uint32_t w = *reinterpret_cast<const uint32_t *>(reinterpret_cast<const int8_t *>(x) + e);
#pragma unroll
        for (int j = 0; j < 4; ++j) c[j] = (int)(int8_t)((w >> (8 * j)) & 0xff);
    } else {
        float v[4];
        t8_act4(x, x_kind, act, gelu, e, v);
#pragma unroll
        for (int j = 0; j < 4; ++j) c[j] = (int)srq_code_fast(v[j], s, rcp, r_ok);
    }
    sum += c[0] + c[1] + c[2] + c[3];
    return (uint32_t)(c[0] & 0xff) | ((uint32_t)(c[1] & 0xff) << 8) | ((uint32_t)(c[2] & 0xff) << 16) |
           ((uint32_t)(c[3] & 0xff) << 24);
}

// sgSum32 over the 32 lanes of this half-wave: the xor butterfly 1, 2, 4, 8, 16, each level adding
// the partner lane's value to the lane's own.
__device__ __forceinline__ float half_butterfly_sum(float v) {
#pragma unroll
    for (int m = 1; m < 32; m <<= 1) v = __fadd_rn(v, __shfl_xor(v, m, 32));
    return v;
}

// The calibrated loop of one lane over iterations [i0, i1): exact sum(u x) per row and sum(x).
__device__ __forceinline__ void t8_accumulate(const u32x4 *wt, int lane, int i0, int i1, const void *x,
                                              int x_kind, const GeluAct &act, bool gelu, float in_scale,
                                              float rcp, bool r_ok, int acc[8], int &sx) {
    constexpr int U = 4;  // iterations whose loads are in flight together
    for (int ib = i0; ib < i1; ib += U) {
        u32x4 v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) v[u] = wt[min(ib + u, i1 - 1) * 32 + lane];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int i = ib + u;
            if (i >= i1) break;
            const uint32_t xw = t8_codes4(x, x_kind, act, gelu, (int64_t)i * 128 + 4 * lane, in_scale, rcp,
                                          r_ok, sx);
            // byte b of word j -> byte j of T_b: T_b holds rows 2b (low nibbles) and 2b + 1 (high
            // nibbles) at k .. k + 3
            const uint32_t lo01 = __builtin_amdgcn_perm(v[u].y, v[u].x, 0x05010400u);
            const uint32_t hi01 = __builtin_amdgcn_perm(v[u].y, v[u].x, 0x07030602u);
            const uint32_t lo23 = __builtin_amdgcn_perm(v[u].w, v[u].z, 0x05010400u);
            const uint32_t hi23 = __builtin_amdgcn_perm(v[u].w, v[u].z, 0x07030602u);
            const uint32_t T[4] = {__builtin_amdgcn_perm(lo23, lo01, 0x05040100u),
                                   __builtin_amdgcn_perm(lo23, lo01, 0x07060302u),
                                   __builtin_amdgcn_perm(hi23, hi01, 0x05040100u),
                                   __builtin_amdgcn_perm(hi23, hi01, 0x07060302u)};
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                acc[2 * b] = __builtin_amdgcn_sdot4((int)(T[b] & 0x0F0F0F0Fu), (int)xw, acc[2 * b], false);
                acc[2 * b + 1] =
                    __builtin_amdgcn_sdot4((int)((T[b] >> 4) & 0x0F0F0F0Fu), (int)xw, acc[2 * b + 1], false);
            }
        }
    }
}

// The calibrated path with K split over the S half-waves of a block, one tile per block: every
// lane value and every partial of the shader's reduction is an integer of magnitude at most
// 8 * 128 * K <= 2^24 (K <= 16384), so the f32 butterfly of the shader is exact and its result is
// f32(the exact total); summing the same integers in another order in int32 gives that value.
template <int S>
__global__ __launch_bounds__(S * 32) void qgemv_tile8u_split_kernel(
    const uint32_t *__restrict__ tw, const float *__restrict__ scales, const void *x, int x_kind,
    GeluAct act, int gelu, void *dst, int out_kind, int k, int n, float in_scale, float out_scale) {
    __shared__ int red[S][8];
    const int lane = threadIdx.x & 31, h = threadIdx.x >> 5;
    const int tile = blockIdx.x;
    const u32x4 *wt = reinterpret_cast<const u32x4 *>(tw + (int64_t)tile * k);
    const int iters = k >> 7, per = (iters + S - 1) / S;
    const int i0 = min(h * per, iters), i1 = min(i0 + per, iters);
    bool r_ok;
    const float rcp = srq_recip(in_scale, r_ok);
    int acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int sx = 0;
    t8_accumulate(wt, lane, i0, i1, x, x_kind, act, gelu != 0, in_scale, rcp, r_ok, acc, sx);
#pragma unroll
    for (int r = 0; r < 8; ++r) {
        int v = acc[r] - 8 * sx;
#pragma unroll
        for (int m = 1; m < 32; m <<= 1) v += __shfl_xor(v, m, 32);
        acc[r] = v;
    }
    if (lane == 0) {
#pragma unroll
        for (int r = 0; r < 8; ++r) red[h][r] = acc[r];
    }
    __syncthreads();
    if (threadIdx.x < 8) {
        const int r = threadIdx.x, row = tile * 8 + r;
        int total = 0;
#pragma unroll
        for (int q = 0; q < S; ++q) total += red[q][r];
        if (row < n)
            store_linear_out(dst, row, out_kind, linear_epilogue(in_scale, scales[row], (float)total), total,
                             out_scale);
    }
}

template <bool CAL>
__global__ __launch_bounds__(kT8Threads) void qgemv_tile8u_kernel(
    const uint32_t *__restrict__ tw, const float *__restrict__ scales, const void *x, int x_kind,
    GeluAct act, int gelu, void *dst, int out_kind, int k, int n, float in_scale, float out_scale) {
    const int lane = threadIdx.x & 31;
    const int tiles = (n + 7) >> 3;
    const int tile = blockIdx.x * (kT8Threads / 32) + (threadIdx.x >> 5);
    const u32x4 *wt = reinterpret_cast<const u32x4 *>(tw + (int64_t)min(tile, tiles - 1) * k);
    const int iters = k >> 7;
    float part[8];
    if (CAL) {
        bool r_ok;
        const float rcp = srq_recip(in_scale, r_ok);
        int acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        int sx = 0;
        t8_accumulate(wt, lane, 0, iters, x, x_kind, act, gelu != 0, in_scale, rcp, r_ok, acc, sx);
#pragma unroll
        for (int r = 0; r < 8; ++r) part[r] = (float)(acc[r] - 8 * sx);
    } else {
        float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        float sxf = 0.0f;
        for (int i = 0; i < iters; ++i) {
            const u32x4 v = wt[i * 32 + lane];
            float xv[4];
            t8_act4(x, x_kind, act, gelu != 0, (int64_t)i * 128 + 4 * lane, xv);
            const uint32_t w4[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                sxf = __fadd_rn(sxf, xv[j]);
#pragma unroll
                for (int r = 0; r < 8; ++r)
                    acc[r] = __fadd_rn(acc[r], __fmul_rn((float)((w4[j] >> (4 * r)) & 15u), xv[j]));
            }
        }
        const float sx8f = __fmul_rn(8.0f, sxf);
#pragma unroll
        for (int r = 0; r < 8; ++r) part[r] = __fsub_rn(acc[r], sx8f);
    }
    float sum[8];
#pragma unroll
    for (int r = 0; r < 8; ++r) sum[r] = half_butterfly_sum(part[r]);
    if (lane == 0 && tile < tiles) {
        const float xs = CAL ? in_scale : 1.0f;
#pragma unroll
        for (int r = 0; r < 8; ++r) {
            const int row = tile * 8 + r;
            if (row < n) store_linear_out(dst, row, out_kind, linear_epilogue(xs, scales[row], sum[r]), 0, out_scale);
        }
    }
}

}  // namespace g4

using namespace g4;

extern "C" {

int g4_tile8u_repack(const void *wq, void *tile_wq, int k, int num_rows, void *stream) {
    if (!wq || !tile_wq) return set_error(G4_ERR_INVALID, "tile8u repack: wq and tile_wq must be given");
    if (k <= 0 || num_rows <= 0) return set_error(G4_ERR_INVALID, "tile8u repack needs K and a row count");
    if (k % 2) return set_error(G4_ERR_INVALID, "tile8u repack: K %d does not fill whole bytes", k);
    if (reinterpret_cast<uintptr_t>(tile_wq) & 3)
        return set_error(G4_ERR_INVALID, "tile8u repack: tile_wq must be 4-byte aligned");
    const int64_t words = (int64_t)((num_rows + 7) / 8) * k;
    int64_t blocks = (words + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL(tile8u_repack_kernel, dim3((unsigned)blocks), dim3(256), 0, as_stream(stream),
                       reinterpret_cast<const uint8_t *>(wq), reinterpret_cast<uint32_t *>(tile_wq), k,
                       num_rows, words);
    G4_LAUNCHED("tile8u_repack_kernel");
    return G4_OK;
}

int g4_qgemv_tile8u(const void *tile_wq, const float *scales, const void *x, int x_kind,
                    const g4_gelu_act *act, void *dst, int out_kind, int k, int num_rows,
                    float in_scale, float out_scale, void *stream) {
    const bool gelu = act != nullptr;
    const char *who = gelu ? "qgemv-4bit-gelu" : "qgemv-4bit";
    if (!tile_wq || !scales || !x || !dst)
        return set_error(G4_ERR_INVALID, gelu ? "%s needs inputs named gate and up" : "qgemv needs inputs named wq and scales", who);
    if (gelu && !act->up) return set_error(G4_ERR_INVALID, "%s needs inputs named gate and up", who);
    if (k <= 0 || num_rows <= 0) return set_error(G4_ERR_INVALID, "qgemv needs params.k and params.numRows");
    if (k % 256 != 0)
        return set_error(G4_ERR_INVALID,
                         "qgemv-4bit needs K a multiple of 256, got %d. Every text tensor satisfies this; "
                         "a caller that does not is packing the wrong tensor.", k);
    if (k > 16384) return set_error(G4_ERR_INVALID, "%s: K %d exceeds 16384 (the exact int32/f32 bound)", who, k);
    if (x_kind != G4_KIND_F32 && x_kind != G4_KIND_F16 && x_kind != G4_KIND_I8)
        return set_error(G4_ERR_INVALID, "%s: x_kind %d is not f32, f16 or int8", who, x_kind);
    if (gelu && x_kind == G4_KIND_F16) return set_error(G4_ERR_INVALID, "%s: gate must be f32 or int8 codes", who);
    if (out_kind != G4_KIND_F32 && out_kind != G4_KIND_I8)
        return set_error(G4_ERR_INVALID, "%s (tile8u): out_kind %d is not f32 or int8", who, out_kind);
    if (out_kind == G4_KIND_I8 && out_scale == 0.0f)
        return set_error(G4_ERR_INVALID, "%s: int8 output codes need a calibrated outScale", who);
    if (in_scale == 0.0f && !gelu && x_kind == G4_KIND_I8)
        return set_error(G4_ERR_INVALID, "%s: int8 activation codes need a calibrated inScale", who);
    if (!std::isfinite(in_scale) || !std::isfinite(out_scale))
        return set_error(G4_ERR_INVALID, "%s: inScale and outScale must be finite", who);
    const uintptr_t need_x = x_kind == G4_KIND_F32 ? 15 : x_kind == G4_KIND_F16 ? 7 : 3;
    if ((reinterpret_cast<uintptr_t>(tile_wq) & 15) || (reinterpret_cast<uintptr_t>(x) & need_x))
        return set_error(G4_ERR_INVALID, "%s: tile_wq must be 16-byte aligned and x aligned to 4 elements", who);
    GeluAct a = gelu ? gelu_act_of(act) : GeluAct{};
    if (gelu) {
        if (act->up_offset < 0) return set_error(G4_ERR_INVALID, "%s: upOffset must be >= 0", who);
        if (act->up_kind != G4_KIND_F32 && act->up_kind != G4_KIND_I8)
            return set_error(G4_ERR_INVALID, "%s: up must be f32 or int8 codes", who);
    }
    const int tiles = (num_rows + 7) / 8;
    const dim3 grid((unsigned)((tiles + 1) / 2));
    // calibrated: K over S half-waves of a block (at least three 128-code iterations each)
    const int iters = k / 128;
    const int S = iters >= 48 ? 16 : iters >= 24 ? 8 : iters >= 12 ? 4 : iters >= 6 ? 2 : 1;
    const uint32_t *tws = reinterpret_cast<const uint32_t *>(tile_wq);
#define G4_T8_SPLIT(SS)                                                                             \
    hipLaunchKernelGGL(qgemv_tile8u_split_kernel<SS>, dim3((unsigned)tiles), dim3(SS * 32), 0,      \
                       as_stream(stream), tws, scales, x, x_kind, a, gelu ? 1 : 0, dst, out_kind, k, \
                       num_rows, in_scale, out_scale)
    if (in_scale != 0.0f && S == 16) G4_T8_SPLIT(16);
    else if (in_scale != 0.0f && S == 8) G4_T8_SPLIT(8);
    else if (in_scale != 0.0f && S == 4) G4_T8_SPLIT(4);
    else if (in_scale != 0.0f && S == 2) G4_T8_SPLIT(2);
#undef G4_T8_SPLIT
    else if (in_scale != 0.0f)
        hipLaunchKernelGGL(qgemv_tile8u_kernel<true>, grid, dim3(kT8Threads), 0, as_stream(stream),
                           reinterpret_cast<const uint32_t *>(tile_wq), scales, x, x_kind, a, gelu ? 1 : 0,
                           dst, out_kind, k, num_rows, in_scale, out_scale);
    else
        hipLaunchKernelGGL(qgemv_tile8u_kernel<false>, grid, dim3(kT8Threads), 0, as_stream(stream),
                           reinterpret_cast<const uint32_t *>(tile_wq), scales, x, x_kind, a, gelu ? 1 : 0,
                           dst, out_kind, k, num_rows, in_scale, out_scale);
    G4_LAUNCHED("qgemv_tile8u_kernel");
    return G4_OK;
}

}  // extern "C"

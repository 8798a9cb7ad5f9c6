// Row operations of the decode glue shared by their own kernels (decode.hip) and by the streaming
// GEMV, whose blocks can run the RMS join that produces their activation row in place of its snap
// (qgemv_stream.hip).
//
// Arithmetic (the CPU restatement oracle/g4_decode_oracle.c states the same steps): a reduction is
// 256 lane-strided partial sums (lane l takes elements l, l + 256, ... ascending) followed by a
// pairwise tree (stride 128 down to 1, lane l adds lane l + stride); 1/sqrt is the IEEE square
// root then the IEEE divide. Every function here expects a block of exactly 256 threads.
#pragma once

#include "g4_internal.h"

namespace g4 {

constexpr int kRowThreads = 256;
constexpr int kJoinMaxPer = 8;  // an RMS join serves widths up to 8 * 256
// The stand-in row an RMS join reads for an absent operand (zero-initialized, never written).
static __device__ float g_join_zero_row[kJoinMaxPer * kRowThreads];

// The in-wave levels s = 32 .. 1 of the pairwise tree (lane l adds lane l + s for l < s), with
// the total in every lane: s = 32 and 16 by the gfx950 lane swaps (v_permlane32_swap hands lanes
// 0-31 the values of lanes 32-63, v_permlane16_swap row 0 those of row 1), s = 8 .. 1 by DPP
// row_shl, each a register move instead of an LDS round trip; the same adds on the same lanes as
// __shfl_down(v, s), so the same sum bit for bit.
__device__ __forceinline__ float wave_tree_sum(float v) {
    {
        const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        v = __fadd_rn(v, __uint_as_float(r[1]));
    }
    {
        const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        v = __fadd_rn(v, __uint_as_float(r[1]));
    }
    v = __fadd_rn(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x108, 0xF, 0xF, true)));
    v = __fadd_rn(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x104, 0xF, 0xF, true)));
    v = __fadd_rn(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x102, 0xF, 0xF, true)));
    v = __fadd_rn(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x101, 0xF, 0xF, true)));
    return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(v)));
}

// The same tree over each 32-lane half of the wave (levels 16 .. 1): the half's total in its
// first lane (lanes 0 and 32).
__device__ __forceinline__ float half_wave_tree_sum(float v) {
    {
        const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        v = __fadd_rn(v, __uint_as_float(r[1]));
    }
    v = __fadd_rn(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x108, 0xF, 0xF, true)));
    v = __fadd_rn(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x104, 0xF, 0xF, true)));
    v = __fadd_rn(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x102, 0xF, 0xF, true)));
    return __fadd_rn(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x101, 0xF, 0xF, true)));
}

// The wave's int32 sum in lane 0 (exact in any order), by the same lane moves.
__device__ __forceinline__ int wave_sum_i32_first(int v) {
    {
        const auto r = __builtin_amdgcn_permlane32_swap((unsigned)v, (unsigned)v, false, false);
        v += (int)r[1];
    }
    {
        const auto r = __builtin_amdgcn_permlane16_swap((unsigned)v, (unsigned)v, false, false);
        v += (int)r[1];
    }
    v += __builtin_amdgcn_update_dpp(0, v, 0x108, 0xF, 0xF, true);
    v += __builtin_amdgcn_update_dpp(0, v, 0x104, 0xF, 0xF, true);
    v += __builtin_amdgcn_update_dpp(0, v, 0x102, 0xF, 0xF, true);
    return v + __builtin_amdgcn_update_dpp(0, v, 0x101, 0xF, 0xF, true);
}

// The maximum over each 32-lane half of the wave in its first lane (lanes 0 and 32), and over the
// whole wave in lane 0, by the same lane moves (a maximum is exact in any order).
__device__ __forceinline__ float dpp_max_rows(float v) {
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x108, 0xF, 0xF, true)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x104, 0xF, 0xF, true)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x102, 0xF, 0xF, true)));
    return fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x101, 0xF, 0xF, true)));
}
__device__ __forceinline__ float half_wave_max(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return dpp_max_rows(fmaxf(v, __uint_as_float(r[1])));
}
__device__ __forceinline__ float wave_max(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return half_wave_max(fmaxf(v, __uint_as_float(r[1])));
}

// The pairwise tree over 256 lanes: level s adds lane l + s into lane l for l < s, s = 128 .. 1
// (every thread of the block calls it; returns the total). The 256 partials go through LDS once;
// then every wave evaluates the whole tree itself: lane l takes levels 128 and 64 in-lane
// ((p[l] + p[l+128]) + (p[l+64] + p[l+192])) and the six in-wave levels in registers. One barrier.
// lds: 256 floats that the block does not write again before another barrier (two trees in a row
// take two regions).
__device__ __forceinline__ float block_tree_sum(float part, float *lds) {
    const int t = threadIdx.x, lane = t & 63;
    lds[t] = part;
    __syncthreads();
    const float a = __fadd_rn(lds[lane], lds[lane + 128]);       // s = 128, lanes l < 64
    const float b = __fadd_rn(lds[lane + 64], lds[lane + 192]);  // s = 128, lanes 64 .. 127
    return wave_tree_sum(__fadd_rn(a, b));                       // s = 64, then 32 .. 1
}

// sqrtf, not __fsqrt_rn: on this toolchain __fsqrt_rn is the native (approximate) v_sqrt_f32
// unless OCML_BASIC_ROUNDED_OPERATIONS is defined, while sqrtf lowers to v_sqrt_f32 plus the
// neighbour test that makes it correctly rounded.
__device__ __forceinline__ float inv_rms(float sumsq, int width, float eps) {
    return __fdiv_rn(1.0f, sqrtf(__fadd_rn(__fdiv_rn(sumsq, (float)width), eps)));
}

__device__ __forceinline__ float load_val(const void *src, int kind, float scale, int64_t i) {
    if (kind == G4_KIND_I8) return __fmul_rn((float)reinterpret_cast<const int8_t *>(src)[i], scale);
    return reinterpret_cast<const float *>(src)[i];
}

__device__ __forceinline__ int8_t snap_code(float v, float s) { return (int8_t)srq_code_i(v, s); }

// rms-norm / norm-residual / norm-residual-norm of one row (rmsNorm.ts:131-180,
// mlpEpilogue.ts:196-230, blockJoin.ts:160-175): y = (src * inv) * gain (gain null: weightless);
// with a residual, hidden = resid + y, times alpha when alpha != 1. Outputs: hidden (f32, when
// J.hidden is set), and emit(i, code) for every element i < width with the code of either the
// second norm of hidden (gain2 given) or of hidden itself, snapped on in_scale (when J.codes is
// set). lds: 512 floats (the two reductions take one half each).
// The value of element i (flat index idx) of a join over split accumulators: the producing
// linear's epilogue f32(in_scale * scale) * f32(acc), its int8 snap, dequantized by the join.
// The int32 sum of element idx's split partials (at most SPLITS of them). Branch free (a split
// past acc_splits re-reads split 0 and adds nothing), so a caller's loads of several elements all
// go out before any sum.
template <int SPLITS>
__device__ __forceinline__ int acc_sum(const JoinTail &J, int64_t idx) {
    const int32_t *p = reinterpret_cast<const int32_t *>(J.src) + idx;
    if constexpr (SPLITS == 1) return p[0];
    int part[SPLITS];
#pragma unroll
    for (int s = 0; s < SPLITS; ++s) part[s] = p[(s < J.acc_splits ? s : 0) * J.acc_split_stride];
    int acc = 0;
#pragma unroll
    for (int s = 0; s < SPLITS; ++s) acc += s < J.acc_splits ? part[s] : 0;
    return acc;
}
__device__ __forceinline__ float acc_value(const JoinTail &J, int acc, float scale) {
    const float y = __fmul_rn(__fmul_rn(J.acc_in_scale, scale), (float)acc);
    return __fmul_rn((float)snap_code(y, J.src_scale), J.src_scale);
}

struct NoLoads {
    __device__ void operator()() const {}
};

// ACC > 0: the source is at most ACC split int32 accumulators (src_kind G4_KIND_I32).
// after_loads() runs once every operand load of the join is issued and before any is used: a
// caller's own loads issued there queue behind the join's, so the join waits for its operands only
// (a wave's loads complete in issue order) while the caller's stay in flight under its arithmetic.
// PER: elements per thread the caller provides for (width <= PER * 256; a caller that knows the
// width issues no loads past it).
// G2 false: the join has no second gain (J.gain2 null, checked by the launcher), so that operand
// is neither loaded nor tested.
template <int ACC = 0, int PER = kJoinMaxPer, bool G2 = true, typename Emit, typename Loads = NoLoads>
__device__ __forceinline__ void rms_join_row_emit(const JoinTail &J, int64_t row, float *lds,
                                                  Emit emit, Loads after_loads = Loads()) {
    static_assert(PER >= 1 && PER <= kJoinMaxPer, "an RMS join serves widths up to 8 * 256");
    const int t = threadIdx.x;
    const int width = J.width;
    const int64_t base = row * width;
    // every operand is loaded before the first barrier (a barrier also fences the compiler's
    // load scheduling, so later loads would each cost a memory latency of their own), at indices
    // clamped into the row and with no branch between them, so no load waits for another; the
    // conversions and the selects of the out-of-row elements come after all of them
    float v[PER], ga[PER], re[PER], g2[PER];
    int raw[PER];  // the source element's bits: an int8 code, an f32, or the int32 sum
    float as[ACC ? PER : 1];
    int ic[PER];
#pragma unroll
    for (int e = 0; e < PER; ++e) ic[e] = min(t + e * kRowThreads, width - 1);
    if constexpr (ACC > 0) {
#pragma unroll
        for (int e = 0; e < PER; ++e) {
            raw[e] = acc_sum<ACC>(J, base + ic[e]);
            as[e] = J.acc_scales[ic[e]];
        }
    } else if (J.src_kind == G4_KIND_I8) {
        const int8_t *src = reinterpret_cast<const int8_t *>(J.src) + base;
#pragma unroll
        for (int e = 0; e < PER; ++e) raw[e] = src[ic[e]];
    } else {
        const int *src = reinterpret_cast<const int *>(J.src) + base;
#pragma unroll
        for (int e = 0; e < PER; ++e) raw[e] = src[ic[e]];
    }
    // An absent gain, residual or second gain is read from a row of zeros in its place, so the
    // loads stay unconditional: a load in one arm of a branch and a constant in the other made the
    // compiler wait for every load in flight on the constant's path.
    const bool g2on = G2 && J.gain2 != nullptr;
    const float *gp = J.gain ? J.gain : g_join_zero_row;
    const float *rp = J.resid ? J.resid + base : g_join_zero_row;
#pragma unroll
    for (int e = 0; e < PER; ++e) {
        ga[e] = gp[ic[e]];
        re[e] = rp[ic[e]];
        g2[e] = g2on ? J.gain2[ic[e]] : 0.0f;
    }
    after_loads();
#pragma unroll
    for (int e = 0; e < PER; ++e) {
        ga[e] = J.gain ? ga[e] : 1.0f;
        re[e] = J.resid ? re[e] : 0.0f;
    }
#pragma unroll
    for (int e = 0; e < PER; ++e) {
        const bool in = t + e * kRowThreads < width;
        float x;
        if constexpr (ACC > 0) x = acc_value(J, raw[e], as[e]);
        else x = J.src_kind == G4_KIND_I8 ? __fmul_rn((float)raw[e], J.src_scale) : __int_as_float(raw[e]);
        v[e] = in ? x : 0.0f;
        ga[e] = in ? ga[e] : 1.0f;
        re[e] = in ? re[e] : 0.0f;
        g2[e] = in ? g2[e] : 0.0f;
    }
    float part = 0.0f;
#pragma unroll
    for (int e = 0; e < PER; ++e)
        if (t + e * kRowThreads < width) part = __fadd_rn(part, __fmul_rn(v[e], v[e]));
    const float inv = inv_rms(block_tree_sum(part, lds), width, J.eps);
    float part2 = 0.0f;
#pragma unroll
    for (int e = 0; e < PER; ++e) {
        const int i = t + e * kRowThreads;
        if (i >= width) continue;
        float y = __fmul_rn(v[e], inv);
        if (J.gain) y = __fmul_rn(y, ga[e]);
        if (J.resid) {
            y = __fadd_rn(re[e], y);
            if (J.alpha != 1.0f) y = __fmul_rn(y, J.alpha);
        }
        v[e] = y;
        if (J.hidden) J.hidden[base + i] = y;
        if (g2on) part2 = __fadd_rn(part2, __fmul_rn(y, y));
    }
    if (!J.codes) return;
    if (g2on) {
        const float inv2 = inv_rms(block_tree_sum(part2, lds + kRowThreads), width, J.eps);
#pragma unroll
        for (int e = 0; e < PER; ++e) {
            const int i = t + e * kRowThreads;
            if (i < width) emit(i, snap_code(__fmul_rn(__fmul_rn(v[e], inv2), g2[e]), J.in_scale));
        }
    } else {
#pragma unroll
        for (int e = 0; e < PER; ++e) {
            const int i = t + e * kRowThreads;
            if (i < width) emit(i, snap_code(v[e], J.in_scale));
        }
    }
}

// The join kernel's form: codes to J.codes[row][i]. lds: 512 floats.
template <int ACC = 0, int PER = kJoinMaxPer, bool G2 = true>
__device__ __forceinline__ void rms_join_row(const JoinTail &J, int64_t row, float *lds) {
    int8_t *codes = J.codes;
    const int64_t base = row * J.width;
    rms_join_row_emit<ACC, PER, G2>(J, row, lds, [=](int i, int8_t c) { codes[base + i] = c; });
}

// The elements per thread a launcher instantiates for a row of `width`: 6 up to 1536 (the E2B
// hidden size), else 8.
constexpr int kJoinPerNarrow = 6;
__host__ __device__ inline bool join_narrow(int width) { return width <= kJoinPerNarrow * kRowThreads; }

}  // namespace g4

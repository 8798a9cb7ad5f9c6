// The per-layer-embedding gather on gfx950: ple-gather-4bit and ple-gather-4bit-sliced
// (src/kernels/embedGather.ts:176-261, :435-485), plus one fused launch over every slice of a
// split table (the reference dispatches once per slice, embedGather.ts:403-419).
//
// One thread per 4 bytes of a gathered row: it reads 8 packed codes with one 32-bit load and
// writes 8 outputs (one 16-byte f16 store, two of f32, one 8-byte of int8), so each load and store
// instruction of a wave covers one contiguous run of the row. The arithmetic is the reference's: fold the
// embed scale 16 into the group scale in f32 (exact, a power of two), then one multiply per
// element, f32((code - 8) * f32(16 * scale)), rounded to f16 ties-to-even for the f16 output.
// The scale index follows the shader (embedGather.ts:245-248): group of col = 4 j, so a group
// size that is a multiple of 4 (required) gives every element its own group's scale.
#include "g4_internal.h"

namespace g4 {

constexpr int kGatherThreads = 256;
constexpr int kMaxSlices = 16;

struct SliceTable {
    const uint8_t *codes[kMaxSlices];
    int64_t start[kMaxSlices];
    int64_t count[kMaxSlices];
    int n;
};

__device__ __forceinline__ float scale_at(const void *scales, int kind, int64_t i) {
    if (kind == G4_KIND_F16) return __half2float(reinterpret_cast<const __half *>(scales)[i]);
    return reinterpret_cast<const float *>(scales)[i];
}

// Writes the 8 outputs of chunk `ch` (codes 8 ch .. 8 ch + 7, one packed u32) of slot `slot`.
// `src` points at the code word, or is null for an id no slice carries (written as zeros).
__device__ __forceinline__ void gather_chunk(const uint8_t *src, const void *scales, int scale_kind,
                                             int64_t row, void *dst, int out_kind, int64_t slot,
                                             int ch, int cols, int group_size, int groups_per_row) {
    const uint32_t w = src ? *reinterpret_cast<const uint32_t *>(src) : 0x88888888u;
    const int col0 = ch * 8;
    const int64_t obase = slot * (int64_t)cols + col0;
    if (out_kind == G4_KIND_I8) {
        // code - 8 per nibble, low nibble first: bytes 0..3 from nibbles 0..3, 4..7 from 4..7.
        uint32_t lo = 0, hi = 0;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            lo |= (uint32_t)((int)((w >> (4 * q)) & 0xf) - 8 & 0xff) << (8 * q);
            hi |= (uint32_t)((int)((w >> (16 + 4 * q)) & 0xf) - 8 & 0xff) << (8 * q);
        }
        *reinterpret_cast<uint2 *>(reinterpret_cast<int8_t *>(dst) + obase) = make_uint2(lo, hi);
        return;
    }
    float out[8];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        // One scale per vec4 of output, the group of its first column (embedGather.ts:245-248).
        float scale = 0.0f;
        if (src) {
            const int col = col0 + 4 * q;
            scale = __fmul_rn(16.0f, scale_at(scales, scale_kind,
                                              row * groups_per_row + col / group_size));
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int i = 4 * q + e;
            const int code = (int)((w >> (4 * i)) & 0xf) - 8;
            out[i] = __fmul_rn((float)code, scale);
        }
    }
    if (out_kind == G4_KIND_F16) {
        uint32_t h[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const unsigned short lo = __half_as_ushort(__float2half_rn(out[2 * i]));
            const unsigned short hi = __half_as_ushort(__float2half_rn(out[2 * i + 1]));
            h[i] = (uint32_t)lo | ((uint32_t)hi << 16);
        }
        *reinterpret_cast<uint4 *>(reinterpret_cast<__half *>(dst) + obase) =
            make_uint4(h[0], h[1], h[2], h[3]);
    } else {
        float4 *d = reinterpret_cast<float4 *>(reinterpret_cast<float *>(dst) + obase);
        d[0] = make_float4(out[0], out[1], out[2], out[3]);
        d[1] = make_float4(out[4], out[5], out[6], out[7]);
    }
}

// One slice (or the whole table with start 0 and count = rows): ids outside the slice are left
// untouched when `sliced`, and written as zeros when not (an id the table does not hold).
__global__ __launch_bounds__(kGatherThreads) void ple_gather_kernel(
    const uint8_t *codes, const void *scales, int scale_kind, const int32_t *ids, void *dst,
    int out_kind, int slots, int cols, int group_size, int groups_per_row, int sliced,
    int64_t start, int64_t count) {
    const int chunks = cols >> 3;
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= (int64_t)slots * chunks) return;
    const int64_t slot = t / chunks;
    const int ch = (int)(t - slot * chunks);
    const int64_t row = (int64_t)(uint32_t)ids[slot];
    const bool inside = row >= start && row - start < count;
    if (!inside && sliced) return;
    const uint8_t *src =
        inside ? codes + (row - start) * (int64_t)(cols >> 1) + (int64_t)ch * 4 : nullptr;
    gather_chunk(src, scales, scale_kind, row, dst, out_kind, slot, ch, cols, group_size,
                 groups_per_row);
}

// Every slice of a split table in one launch: each slot finds the slice that carries its id.
__global__ __launch_bounds__(kGatherThreads) void ple_gather_split_kernel(
    SliceTable tab, const void *scales, int scale_kind, const int32_t *ids, void *dst, int out_kind,
    int slots, int cols, int group_size, int groups_per_row) {
    const int chunks = cols >> 3;
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= (int64_t)slots * chunks) return;
    const int64_t slot = t / chunks;
    const int ch = (int)(t - slot * chunks);
    const int64_t row = (int64_t)(uint32_t)ids[slot];
    const uint8_t *src = nullptr;
#pragma unroll
    for (int s = 0; s < kMaxSlices; ++s) {
        if (s < tab.n && row >= tab.start[s] && row - tab.start[s] < tab.count[s])
            src = tab.codes[s] + (row - tab.start[s]) * (int64_t)(cols >> 1) + (int64_t)ch * 4;
    }
    gather_chunk(src, scales, scale_kind, row, dst, out_kind, slot, ch, cols, group_size,
                 groups_per_row);
}

static int check_gather(const void *scales, int scale_kind, const int32_t *ids, void *dst,
                        int out_kind, int slots, int cols, int group_size, int groups_per_row,
                        const char *who) {
    if (!scales || !ids || !dst)
        return set_error(G4_ERR_INVALID, "%s needs inputs named codes, scales and ids", who);
    if (slots <= 0) return set_error(G4_ERR_INVALID, "%s: params.slots must be positive", who);
    if (cols <= 0 || cols % 8 != 0)
        return set_error(G4_ERR_INVALID, "%s: %d columns do not pack evenly at 4 bits", who, cols);
    if (group_size <= 0 || group_size % 4 != 0 || cols % group_size != 0)
        return set_error(G4_ERR_INVALID, "%s: group size %d does not divide %d in vec4 steps", who,
                         group_size, cols);
    if (groups_per_row != cols / group_size)
        return set_error(G4_ERR_INVALID, "%s: groupsPerRow %d is not cols / groupSize = %d", who,
                         groups_per_row, cols / group_size);
    if (scale_kind != G4_KIND_F32 && scale_kind != G4_KIND_F16)
        return set_error(G4_ERR_INVALID, "%s: scales must be f32 or f16", who);
    if (out_kind != G4_KIND_F32 && out_kind != G4_KIND_F16 && out_kind != G4_KIND_I8)
        return set_error(G4_ERR_INVALID, "%s: output must be f32, f16 or int8 codes", who);
    if (reinterpret_cast<uintptr_t>(dst) & 15)
        return set_error(G4_ERR_INVALID, "%s: dst must be 16-byte aligned", who);
    return G4_OK;
}

}  // namespace g4

using namespace g4;

extern "C" {

int g4_ple_gather(const void *codes, const void *scales, int scale_kind, const int32_t *ids,
                  void *dst, int out_kind, int slots, int cols, int group_size,
                  int groups_per_row, int sliced, int64_t slice_start_row,
                  int64_t slice_row_count, void *stream) {
    const char *who = sliced ? "ple-gather-4bit-sliced" : "ple-gather-4bit";
    if (!codes) return set_error(G4_ERR_INVALID, "%s needs inputs named codes, scales and ids", who);
    int rc = check_gather(scales, scale_kind, ids, dst, out_kind, slots, cols, group_size,
                          groups_per_row, who);
    if (rc) return rc;
    if (slice_start_row < 0 || slice_row_count <= 0)
        return set_error(G4_ERR_INVALID,
                         sliced ? "ple-gather-4bit-sliced needs params sliceStartRow and "
                                  "sliceRowCount naming a non empty vocabulary range"
                                : "ple-gather-4bit needs the table's row count (slice_row_count) to "
                                  "bound the ids");
    if (!sliced && slice_start_row != 0)
        return set_error(G4_ERR_INVALID, "ple-gather-4bit: an unsliced table starts at row 0");
    if (reinterpret_cast<uintptr_t>(codes) & 3)
        return set_error(G4_ERR_INVALID, "%s: codes must be 4-byte aligned", who);
    const int64_t threads = (int64_t)slots * (cols / 8);
    const int64_t blocks = (threads + kGatherThreads - 1) / kGatherThreads;
    hipLaunchKernelGGL(ple_gather_kernel, dim3((unsigned)blocks), dim3(kGatherThreads), 0,
                       as_stream(stream), reinterpret_cast<const uint8_t *>(codes), scales,
                       scale_kind, ids, dst, out_kind, slots, cols, group_size, groups_per_row,
                       sliced ? 1 : 0, slice_start_row, slice_row_count);
    G4_LAUNCHED("ple_gather_kernel");
    return G4_OK;
}

int g4_ple_gather_split(const void *const *slice_codes, const int64_t *slice_starts,
                        const int64_t *slice_counts, int num_slices, const void *scales,
                        int scale_kind, const int32_t *ids, void *dst, int out_kind, int slots,
                        int cols, int group_size, int groups_per_row, void *stream) {
    const char *who = "ple-gather-4bit-sliced";
    if (!slice_codes || !slice_starts || !slice_counts || num_slices < 1 || num_slices > kMaxSlices)
        return set_error(G4_ERR_INVALID, "%s: 1..%d slices required", who, kMaxSlices);
    int rc = check_gather(scales, scale_kind, ids, dst, out_kind, slots, cols, group_size,
                          groups_per_row, who);
    if (rc) return rc;
    SliceTable tab{};
    tab.n = num_slices;
    for (int s = 0; s < num_slices; ++s) {
        if (!slice_codes[s] || (reinterpret_cast<uintptr_t>(slice_codes[s]) & 3))
            return set_error(G4_ERR_INVALID, "%s: slice %d codes missing or not 4-byte aligned", who, s);
        if (slice_starts[s] < 0 || slice_counts[s] <= 0)
            return set_error(G4_ERR_INVALID,
                             "%s needs params sliceStartRow and sliceRowCount naming a non empty "
                             "vocabulary range", who);
        tab.codes[s] = reinterpret_cast<const uint8_t *>(slice_codes[s]);
        tab.start[s] = slice_starts[s];
        tab.count[s] = slice_counts[s];
    }
    const int64_t threads = (int64_t)slots * (cols / 8);
    const int64_t blocks = (threads + kGatherThreads - 1) / kGatherThreads;
    hipLaunchKernelGGL(ple_gather_split_kernel, dim3((unsigned)blocks), dim3(kGatherThreads), 0,
                       as_stream(stream), tab, scales, scale_kind, ids, dst, out_kind, slots, cols,
                       group_size, groups_per_row);
    G4_LAUNCHED("ple_gather_split_kernel");
    return G4_OK;
}

}  // extern "C"

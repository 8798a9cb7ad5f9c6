// The per-layer-embedding gather on gfx950: ple-gather-4bit and ple-gather-4bit-sliced
// (src/kernels/embedGather.ts:176-261, :435-485), plus one fused launch over every slice of a
// split table (the reference dispatches once per slice, embedGather.ts:403-419).
//
// One block per token: each thread reads 8 packed codes with one 32-bit load and writes 8 outputs
// (one 16-byte f16 store, two of f32, one 8-byte of int8) per run, and the block's threads take
// consecutive runs, so each load and store instruction covers one contiguous stretch of the row. The arithmetic is the reference's: fold the
// embed scale 16 into the group scale in f32 (exact, a power of two), then one multiply per
// element, f32((code - 8) * f32(16 * scale)), rounded to f16 ties-to-even for the f16 output.
// The scale index follows the shader (embedGather.ts:245-248): group of col = 4 j, so a group
// size that is a multiple of 4 (required) gives every element its own group's scale.
#include "g4_internal.h"

namespace g4 {

constexpr int kMaxSlices = 16;
typedef unsigned int u32x2g __attribute__((ext_vector_type(2)));

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

// The embed scale of the vec4 starting at column `col` (the group of its first column,
// embedGather.ts:245-248), times the embed multiplier 16 (exact: a power of two).
__device__ __forceinline__ float vec4_scale(const void *scales, int scale_kind, int64_t row, int col,
                                            int group_size, int groups_per_row) {
    return __fmul_rn(16.0f, scale_at(scales, scale_kind, row * groups_per_row + col / group_size));
}

// Writes the 8 outputs of chunk `ch` (codes 8 ch .. 8 ch + 7, the packed word `w`) of slot `slot`;
// s0 / s1 are the folded scales of its two vec4s. A word of 0x88888888 with zero scales writes the
// zeros of an id no slice carries.
__device__ __forceinline__ void gather_chunk(uint32_t w, float s0, float s1, void *dst,
                                             int out_kind, int64_t slot, int ch, int cols) {
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
        __builtin_nontemporal_store(
            (u32x2g){lo, hi}, reinterpret_cast<u32x2g *>(reinterpret_cast<int8_t *>(dst) + obase));
        return;
    }
    float out[8];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        const float scale = q == 0 ? s0 : s1;
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
        __builtin_nontemporal_store(
            u32x4{h[0], h[1], h[2], h[3]},
            reinterpret_cast<u32x4 *>(reinterpret_cast<__half *>(dst) + obase));
    } else {
        u32x4 *d = reinterpret_cast<u32x4 *>(reinterpret_cast<float *>(dst) + obase);
        __builtin_nontemporal_store(u32x4{__float_as_uint(out[0]), __float_as_uint(out[1]),
                                          __float_as_uint(out[2]), __float_as_uint(out[3])}, d);
        __builtin_nontemporal_store(u32x4{__float_as_uint(out[4]), __float_as_uint(out[5]),
                                          __float_as_uint(out[6]), __float_as_uint(out[7])}, d + 1);
    }
}

// One block per token slot (the id, the slice lookup and the row base are uniform scalars). A
// thread covers the 8-code runs tid, tid + T, tid + 2T, ... of the row (T = threads of the block),
// so every load instruction reads one contiguous run of codes and every store instruction writes
// one contiguous run of the output row; outputs are written non-temporally (they are not re-read
// by this launch).
// RPT runs per thread. A large gather takes 8: a 8960-column row is then 192 threads, three waves,
// so a 2048-token gather's blocks are all resident at once (32 waves per CU), where 4 runs per
// thread needed a second round (11.9 -> 9.7 us). A small one (a decode step's few tokens) takes 4,
// which halves each thread's serial work.
constexpr int kSmallGatherSlots = 256;
constexpr int kRowScales = 128;  // scale groups of a row staged in LDS (the E2B table: 70)

template <int RPT>
__device__ __forceinline__ void gather_row(const uint8_t *row_codes, const void *scales,
                                           int scale_kind, int64_t row, void *dst, int out_kind,
                                           int64_t slot, int cols, int group_size,
                                           int groups_per_row) {
    const int runs = cols >> 3;
    const int T = blockDim.x;
    // a run of 8 codes lies in one group when the group size is a multiple of 8: one scale load
    const bool one_scale = (group_size & 7) == 0;
    // the row's folded scales, loaded once per block into LDS when they fit (one global load per
    // thread at most, in place of one per run; staging the codes the same way measured slower)
    __shared__ float srow[kRowScales];
    const bool staged = one_scale && row_codes && groups_per_row <= kRowScales && groups_per_row <= T &&
                        (int64_t)group_size * groups_per_row >= cols;
    if (staged) {  // uniform
        if ((int)threadIdx.x < groups_per_row)
            srow[threadIdx.x] = __fmul_rn(16.0f, scale_at(scales, scale_kind, row * groups_per_row + threadIdx.x));
        __syncthreads();
    }
    for (int base = threadIdx.x; base < runs; base += RPT * T) {
        // All of this thread's code words and scales are requested before any is converted.
        uint32_t w[RPT];
        float s0[RPT], s1[RPT];
#pragma unroll
        for (int u = 0; u < RPT; ++u) {
            const int ch = base + u * T;
            const bool live = row_codes && ch < runs;
            w[u] = live ? *reinterpret_cast<const uint32_t *>(row_codes + (int64_t)ch * 4)
                        : 0x88888888u;
            s0[u] = !live ? 0.0f
                    : staged ? srow[ch * 8 / group_size]
                             : vec4_scale(scales, scale_kind, row, ch * 8, group_size, groups_per_row);
            s1[u] = !live ? 0.0f
                    : one_scale ? s0[u]
                                : vec4_scale(scales, scale_kind, row, ch * 8 + 4, group_size, groups_per_row);
        }
#pragma unroll
        for (int u = 0; u < RPT; ++u) {
            const int ch = base + u * T;
            if (ch < runs) gather_chunk(w[u], s0[u], s1[u], dst, out_kind, slot, ch, cols);
        }
    }
}

// One slice (or the whole table with start 0 and count = rows): ids outside the slice are left
// untouched when `sliced`, and written as zeros when not (an id the table does not hold).
template <int RPT>
__global__ __launch_bounds__(1024) void ple_gather_kernel(
    const uint8_t *codes, const void *scales, int scale_kind, const int32_t *ids, void *dst,
    int out_kind, int slots, int cols, int group_size, int groups_per_row, int sliced,
    int64_t start, int64_t count) {
    const int64_t slot = blockIdx.x;
    const int64_t row = (int64_t)(uint32_t)ids[slot];
    const bool inside = row >= start && row - start < count;
    if (!inside && sliced) return;  // uniform
    gather_row<RPT>(inside ? codes + (row - start) * (int64_t)(cols >> 1) : nullptr, scales, scale_kind,
               row, dst, out_kind, slot, cols, group_size, groups_per_row);
}

// Every slice of a split table in one launch: each slot finds the slice that carries its id.
template <int RPT>
__global__ __launch_bounds__(1024) void ple_gather_split_kernel(
    SliceTable tab, const void *scales, int scale_kind, const int32_t *ids, void *dst, int out_kind,
    int slots, int cols, int group_size, int groups_per_row) {
    const int64_t slot = blockIdx.x;
    const int64_t row = (int64_t)(uint32_t)ids[slot];
    const uint8_t *src = nullptr;
    for (int s = 0; s < tab.n; ++s)
        if (row >= tab.start[s] && row - tab.start[s] < tab.count[s])
            src = tab.codes[s] + (row - tab.start[s]) * (int64_t)(cols >> 1);
    gather_row<RPT>(src, scales, scale_kind, row, dst, out_kind, slot, cols, group_size, groups_per_row);
}

// Threads per block: enough for rpt 8-code runs each, whole waves, at most 1024.
static int gather_threads(int cols, int rpt) {
    const int runs = cols >> 3;
    int t = (runs + rpt - 1) / rpt;
    t = ((t + 63) / 64) * 64;
    return t < 64 ? 64 : (t > 1024 ? 1024 : t);
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
    const int rpt = slots < kSmallGatherSlots ? 4 : 8;
    if (rpt == 4)
        hipLaunchKernelGGL(ple_gather_kernel<4>, dim3((unsigned)slots), dim3(gather_threads(cols, 4)),
                           0, as_stream(stream), reinterpret_cast<const uint8_t *>(codes), scales,
                           scale_kind, ids, dst, out_kind, slots, cols, group_size, groups_per_row,
                           sliced ? 1 : 0, slice_start_row, slice_row_count);
    else
        hipLaunchKernelGGL(ple_gather_kernel<8>, dim3((unsigned)slots), dim3(gather_threads(cols, 8)),
                           0, as_stream(stream), reinterpret_cast<const uint8_t *>(codes), scales,
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
    if (slots < kSmallGatherSlots)
        hipLaunchKernelGGL(ple_gather_split_kernel<4>, dim3((unsigned)slots),
                           dim3(gather_threads(cols, 4)), 0, as_stream(stream), tab, scales,
                           scale_kind, ids, dst, out_kind, slots, cols, group_size, groups_per_row);
    else
        hipLaunchKernelGGL(ple_gather_split_kernel<8>, dim3((unsigned)slots),
                           dim3(gather_threads(cols, 8)), 0, as_stream(stream), tab, scales,
                           scale_kind, ids, dst, out_kind, slots, cols, group_size, groups_per_row);
    G4_LAUNCHED("ple_gather_split_kernel");
    return G4_OK;
}

}  // extern "C"

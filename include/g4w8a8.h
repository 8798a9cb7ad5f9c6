/*
 * g4w8a8: MI355X (gfx950) wNa8o8 quantized projection path and split PLE gather.
 *
 * The drop-in C ABI for the reference's operator seam (Ar5en1c/gemma4-webgpu-engine,
 * src/kernels/registry.ts:108-119 `Kernel.bind`, fed by src/execute.ts:438 `resolveStep`).
 * Each entry point replaces one registry kernel (named in its comment, with the file:line of the
 * reference's bind it mirrors): the same named inputs, the same params and the same refusals. The
 * reference's `bind` throws an Error; here every entry point returns a status and
 * g4_last_error() gives the message, with the reference's wording where it has one.
 *
 * Conventions
 *  - Plain pointers and sizes only. Device pointers are HIP device memory (hipMalloc, or any
 *    allocator of this process such as torch); `stream` is a hipStream_t (NULL = default stream).
 *  - Every compute entry point is enqueue-only on `stream`: it returns after the launch.
 *  - Layouts are the reference's (src/kernels/qlayout.ts:12-26, src/quant.ts:11-20):
 *      weights   row-major packed rows, K contiguous; 4-bit: two codes per byte, low nibble first,
 *                zero point 8; 8-bit: the signed byte is the code.
 *      scales    f32 [N], one per output row.
 *      x         [M][K] row-major, f32 or f16 (widened exactly), or int8 codes already snapped.
 *      dst       [M][N] row-major (the reference's dst[col * N + row]).
 *  - Arithmetic (src/kernels/qgemv.ts:1131-1176): xq = clamp(RNE(f32(x / inScale)), -128, 127);
 *    acc = sum(wcode * xq) exact in int32; y = f32(f32(inScale * scale[n]) * f32(acc));
 *    q = clamp(RNE(f32(y / outScale)), -128, 127). Divides are IEEE binary32.
 *    inScale == 0 selects the uncalibrated f32 code dot (lm_head), outScale == 0 skips the output
 *    snap (quant.ts:248-357).
 */
#ifndef G4W8A8_H
#define G4W8A8_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define G4_ABI_VERSION 1

/* Status codes. */
#define G4_OK 0
#define G4_ERR_INVALID 1     /* a refused argument: the reference's bind would throw */
#define G4_ERR_UNKNOWN_KERNEL 2
#define G4_ERR_HIP 3         /* a HIP runtime call failed */
#define G4_ERR_NO_DEVICE 4
#define G4_ERR_UNSUPPORTED 5 /* a combination the path does not implement */

/* Element kinds of activations (x_kind) and outputs (out_kind). */
#define G4_KIND_F32 0 /* x: f32 activations. dst: the reference's f32 dst, q * outScale (or y) */
#define G4_KIND_F16 1 /* x: f16 activations, widened exactly. dst (gather only): f16 values */
#define G4_KIND_I8 2  /* x: int8 codes already snapped on inScale. dst: int8 codes q */
#define G4_KIND_I32 3 /* dst only: the exact int32 accumulator sum(wcode * xq) */

/* Version of this ABI (G4_ABI_VERSION). */
int g4_abi_version(void);

/* Message of the last failed call on this thread ("" when none). Owned by the library. */
const char *g4_last_error(void);

/* ---- device memory, streams, events (what the reference's BufferManager/runtime.ts own) ---- */
int g4_device_count(int *count);
int g4_set_device(int device);
int g4_malloc(void **ptr, size_t bytes);
int g4_free(void *ptr);
int g4_memcpy_h2d(void *dst, const void *src, size_t bytes, void *stream);
int g4_memcpy_d2h(void *dst, const void *src, size_t bytes, void *stream);
int g4_memcpy_d2d(void *dst, const void *src, size_t bytes, void *stream);
/* Pinned host memory (hipHostMalloc), the staging side of an asynchronous readback: the
 * reference's MAP_READ staging buffers and mapAsync (src/runtime.ts:866-878). */
int g4_host_alloc(void **ptr, size_t bytes);
int g4_host_free(void *ptr);
/* A device-to-host copy enqueued on `stream` without waiting (g4_memcpy_d2h waits): dst must be
 * g4_host_alloc memory, read only after an event recorded behind the copy has completed. */
int g4_memcpy_d2h_async(void *dst, const void *src, size_t bytes, void *stream);
/* Byte fill through a kernel (safe under graph capture). */
int g4_fill_u8(void *dst, uint8_t value, size_t bytes, void *stream);
int g4_stream_create(void **stream);
int g4_stream_destroy(void *stream);
int g4_stream_synchronize(void *stream);
int g4_device_synchronize(void);
int g4_event_create(void **event);
int g4_event_destroy(void *event);
int g4_event_record(void *event, void *stream);
int g4_event_synchronize(void *event);
int g4_event_elapsed_ms(float *ms, void *start, void *end);

/* HIP graphs: capture a sequence of enqueues on `stream` once, replay it with one launch. The
 * decode loop is launch-bound (a launch costs microseconds of host time, more than a small GEMV
 * runs); the reference caches its per-token encode the same way (runtime.ts:702-767). Kernels of
 * this library never allocate or memset inside a capture. g4_qgemm / g4_linear with f16 or f32
 * activations at M > 32 (and at M >= 3 once M * K * ceil(N / 16) reaches 4 Mi, where one snap pass
 * beats the small-M kernel snapping in every block) snap them into a per-stream workspace: it must
 * already be large enough when
 * the capture starts (run the same shape once on the stream first); a call that would grow it
 * inside a capture is refused with G4_ERR_INVALID. A workspace whose address a capture took is never
 * freed (a graph may be replayed later, on any stream); g4_stream_destroy frees the stream's
 * workspace otherwise. g4_graph_destroy waits for the graph's own last launch (an event recorded
 * after each g4_graph_launch, on the stream it was launched on), not for the whole device, and
 * releases the graph even when that wait fails. Launches of one graph on several streams must be
 * ordered by the caller (the event marks the most recent launch). g4_graph_end_capture refuses
 * (G4_ERR_INVALID, nothing instantiated, the stream out of capture) a graph holding anything but
 * kernels, device-to-device copies, events and empty nodes: a captured copy to or from host memory
 * would touch that host buffer at every replay, after the enqueuing call returned, and memset
 * nodes have given wrong results on replays after the first (clear with g4_fill_u8 instead). */
int g4_graph_begin_capture(void *stream);
int g4_graph_end_capture(void *stream, void **graph_exec);
int g4_graph_launch(void *graph_exec, void *stream);
int g4_graph_destroy(void *graph_exec);

/* ---- the quantized linears --------------------------------------------------------------- */

/*
 * qgemv-4bit / qgemv-8bit and the wide qgemv-4bit-m2 / qgemv-8bit-m2.
 * Replaces bindGemv (src/kernels/qgemv.ts:1299-1363; registry entries :1471, :1595) and
 * bindGemvWide (src/kernels/qgemvWide.ts:515-574; entries :597-712).
 * cols is the token count: 1 for a decode step, 2 for the draft-verify pass (cols > 2 refused,
 * as qgemvWide.ts:522-526). K must be a multiple of 256 (4-bit) or 128 (8-bit), qgemv.ts:1305-1310.
 */
int g4_qgemv(int bits, const void *wq, const float *scales, const void *x, int x_kind, void *dst,
             int out_kind, int k, int num_rows, int cols, float in_scale, float out_scale,
             void *stream);

/*
 * qgemm-4bit (+ -single, -prefill4) and qmatmul-8bit: M token columns, any M >= 1.
 * Replaces bindGemm (src/kernels/qgemm.ts:589-639; entries :641, :717, :725) and bindQmatmul8
 * (src/kernels/pleMatmul.ts:257-303; entry :323). bits 4 needs K % 256 == 0 (qgemm.ts:598-600);
 * bits 8 needs K % 4 == 0 (pleMatmul.ts:266-271). The calibrated path runs on int8 MFMA.
 * Uncalibrated qmatmul-8bit (bits 8, inScale 0) keeps the reference's serial per-output f32 order at
 * every M (pleMatmul.ts:139-147, oracle :212-222): one thread per output, each 4-code word summed
 * in order from 0, then added to the accumulator. Uncalibrated bits 4 is the f32 code dot of
 * qgemv-4bit per column.
 */
int g4_qgemm(int bits, const void *wq, const float *scales, const void *x, int x_kind, void *dst,
             int out_kind, int k, int num_rows, int m_cols, float in_scale, float out_scale,
             void *stream);

/*
 * The execute.ts routing (src/execute.ts:372-430 matmulKernel/gemvWide/pleKernel) folded into one
 * call: picks the kernel for (bits, M, N, K) on this GPU. M <= 2 -> the GEMV family, larger M ->
 * the MFMA GEMM. Same arguments as g4_qgemm. M <= 2 is the decode GEMV's mode: an uncalibrated
 * 8-bit call there is qgemv-8bit's f32 path (execute.ts:372-375), above two tokens qmatmul-8bit's.
 */
int g4_linear(int bits, const void *wq, const float *scales, const void *x, int x_kind, void *dst,
              int out_kind, int k, int num_rows, int m_cols, float in_scale, float out_scale,
              void *stream);

/*
 * g4_qgemm for callers that cannot allocate device memory: code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc. No counterpart in the reference. Same arguments,
 * routing and results as g4_qgemm. The one buffer g4_qgemm needs beyond its operands (the snapped
 * activation codes: f16 / f32 x on the paths that snap first, M * K bytes) is a static device array of
 * g4_qgemm_noalloc_max_codes() bytes (8 MiB) that each GPU holds until the process ends; a call
 * whose path needs more is refused with G4_ERR_INVALID before anything is enqueued. It calls no
 * hipMalloc / hipFree. Every call on one GPU shares that GPU's array: calls that overlap on one GPU
 * (other streams, other host threads) race and must be ordered by the caller.
 */
int g4_qgemm_noalloc(int bits, const void *wq, const float *scales, const void *x, int x_kind,
                     void *dst, int out_kind, int k, int num_rows, int m_cols, float in_scale,
                     float out_scale, void *stream);
size_t g4_qgemm_noalloc_max_codes(void);

/* Name of the kernel g4_linear picks for a shape, written into buf (NUL terminated). */
int g4_kernel_for_shape(int bits, int m_cols, int num_rows, int k, char *buf, size_t buf_len);

/*
 * qkv-batch-4bit (count 3) and gate-up-batch-4bit (count 2): several projections of one x in one
 * launch. Replaces bindProjectionBatch (src/kernels/projectionBatch.ts:85-128; entries :161-162).
 * w[i], scales[i], out[i], rows[i], in_scales[i], out_scales[i] per projection; K multiple of 128
 * (projectionBatch.ts:90); gate/up (count 2) needs equal row counts (:92).
 */
int g4_projection_batch(int bits, int count, const void *const *w, const float *const *scales,
                        const void *x, int x_kind, void *const *out, int out_kind, const int *rows,
                        const float *in_scales, const float *out_scales, int k, void *stream);

/*
 * The grouped GEMV: up to G4_MAX_GROUP independent M=1 linears (each its own weights, x, K, N,
 * width and scales) in one launch. The generalisation of projectionBatch.ts to a whole layer's
 * projection set (q, k, v, o, gate, up, down). No reference counterpart beyond projectionBatch.
 */
#define G4_MAX_GROUP 16
typedef struct g4_gemv_desc {
    const void *wq;
    const float *scales;
    const void *x;
    void *dst;
    int bits;     /* 4 or 8 */
    int x_kind;   /* G4_KIND_F32, _F16 or _I8 */
    int out_kind; /* G4_KIND_I8, _F32 or _I32 */
    int k;
    int num_rows;
    float in_scale;  /* non-zero: the grouped GEMV is the calibrated path only */
    float out_scale;
} g4_gemv_desc;
int g4_qgemv_grouped(const g4_gemv_desc *descs, int count, void *stream);

/*
 * A reusable grouped GEMV over any number of projections (a whole decode step's projection set):
 * the descriptors are validated and laid out once into a device-resident job table, and every
 * g4_qgemv_plan_launch replays the same launch on the buffers the descriptors name. This is the
 * reference's cached decode-step bind (src/runtime.ts:702-767: bind groups and dispatches built once,
 * replayed per token) in C-ABI form. Every projection must be calibrated (inScale != 0) and have a
 * streaming shape class (K * bits / 128 a multiple of 16, 32 or 64 with at most 4 chunks per lane,
 * or 6 at 8 bits; K <= 16384); g4_qgemv_plan_create refuses others with G4_ERR_UNSUPPORTED.
 * create allocates and copies (synchronous); launch only enqueues, so it can be graph-captured.
 */
typedef struct g4_gemv_plan g4_gemv_plan;
int g4_qgemv_plan_create(const g4_gemv_desc *descs, int count, g4_gemv_plan **plan);
int g4_qgemv_plan_launch(const g4_gemv_plan *plan, void *stream);
/* Tiles (4 waves each) and blocks of the plan's launch. */
int g4_qgemv_plan_info(const g4_gemv_plan *plan, int *tiles, int *grid);
int g4_qgemv_plan_destroy(g4_gemv_plan *plan);

/*
 * qgemv-4bit-split / qgemv-8bit-split (src/kernels/qgemv.ts:1753, :1772; band logic :521-548) and
 * qgemv-4bit-gelu-exact-split without the gelu prologue (src/kernels/exactSplit.ts:19-31).
 * Writes partials f32 [num_rows][k_splits]: exact = 0 the scaled f32(f32(xs*scale)*f32(sum_band)),
 * exact = 1 the raw integer f32(sum_band) (needs inScale > 0 and K <= 16384, exactSplit.ts:27).
 */
int g4_qgemv_split(int bits, const void *wq, const float *scales, const void *x, int x_kind,
                   float *partials, int k, int num_rows, int k_splits, int exact, float in_scale,
                   void *stream);

/* qgemv-merge (src/kernels/qgemv.ts:1405, WGSL :1027-1072): ascending f32 fold of k_splits
 * partials per row, then the output snap. Refuses k_splits < 2 (:1444-1446). */
int g4_qgemv_merge(const float *partials, void *dst, int out_kind, int num_rows, int k_splits,
                   float out_scale, void *stream);

/* qgemv-exact-merge (src/kernels/exactSplit.ts:32-72): fold, then f32(f32(in*scale)*t), snap. */
int g4_qgemv_exact_merge(const float *partials, const float *scales, void *dst, int out_kind,
                         int num_rows, int k_splits, float in_scale, float out_scale,
                         void *stream);

/*
 * The fused gelu prologue (GemvPrologue 'gelu', src/kernels/qgemv.ts:359-400): the GEMV reads
 * x[i] = gelu_tanh(gate[i]) * up[up_offset + i] in place of x, the gelu-mul kernel's expression
 * (geluMul.ts:101-116), snapped on inScale. The gate is passed where x goes (f32, the reference's
 * gate output, or int8 codes times gate_scale); `up` is f32 or int8 codes times up_scale. On a
 * calibrated site the result is bit for bit the unfused gelu-mul + GEMV chain (qgemv.ts:362-368).
 * An uncalibrated site (inScale 0, f32 gate) runs the f32 code dot over the unsnapped product, as
 * the reference's f32 path does. f32 operands need 16-byte alignment (after the offset), int8
 * codes 8-byte.
 */
typedef struct g4_gelu_act {
    const void *up;    /* NULL in a plan entry: that projection has no prologue */
    int up_kind;       /* G4_KIND_F32 or G4_KIND_I8 */
    float gate_scale;  /* the gate's int8 codes (x_kind G4_KIND_I8) times this */
    float up_scale;    /* up_kind G4_KIND_I8: the codes times this */
    int64_t up_offset; /* in ELEMENTS. The reference's params.upOffset counts vec4s
                          (qgemv.ts:398, execute.ts:886 layer * dim / 4): up_offset = 4 * upOffset */
} g4_gelu_act;

/* qgemv-4bit-gelu / qgemv-8bit-gelu (registry src/kernels/qgemv.ts:1668-1696, bindGemv(bits,
 * 'gelu')): the down_proj of a decode MLP and the per_layer_projection. */
int g4_qgemv_gelu(int bits, const void *wq, const float *scales, const void *gate, int gate_kind,
                  const g4_gelu_act *act, void *dst, int out_kind, int k, int num_rows,
                  float in_scale, float out_scale, void *stream);

/*
 * The tile8u geometry of qgemv-4bit and qgemv-4bit-gelu (src/kernels/qgemv.ts:870-1015; compiled in
 * place of the classic loop when GemvGeometry.inner is 'tile8u', qgemv.ts:440, the bind unchanged,
 * bindGemv :1299-1363). The weights are in the eight-row tile layout (qgemv.ts:871-876): tile t =
 * rows 8t .. 8t + 7, K u32 words, word k holding row 8t + r's unsigned code (0..15) at bits 4r.
 * g4_tile8u_repack builds it from the checkpoint's row layout (tile_wq: ceil(num_rows / 8) * K * 4
 * bytes; rows past num_rows padded with code 8); the reference ships no repack (the layout was
 * priced on a sweep page before anything read it, qgemv.ts:893-895). g4_qgemv_tile8u: x as for
 * g4_qgemv, or with act != NULL the gelu prologue (x is the gate, as g4_qgemv_gelu); dst f32 or
 * int8 codes; no K split (qgemv.ts:907). Results: calibrated, the classic loop's exactly (the sum
 * is the same exact integer); uncalibrated, the tile loop's own f32 order (per lane over k =
 * 128 i + 4 l + j, then the 32-lane tree). */
int g4_tile8u_repack(const void *wq, void *tile_wq, int k, int num_rows, void *stream);
int g4_qgemv_tile8u(const void *tile_wq, const float *scales, const void *x, int x_kind,
                    const g4_gelu_act *act, void *dst, int out_kind, int k, int num_rows,
                    float in_scale, float out_scale, void *stream);

/* qgemv-4bit-gelu-m2 / qgemv-8bit-gelu-m2 (src/kernels/qgemvWide.ts:660-669, 698-709; bind
 * bindGemvWide(bits, 'gelu') :515-574): the gelu prologue over `cols` token columns (1..2, the
 * draft-verify pass, execute.ts:382-390). gate and up are [cols][K] (column c at element c * K; up
 * also offset by act->up_offset), dst is [cols][num_rows]. Column for column g4_qgemv_gelu. */
int g4_qgemv_gelu_m2(int bits, const void *wq, const float *scales, const void *gate, int gate_kind,
                     const g4_gelu_act *act, void *dst, int out_kind, int k, int num_rows, int cols,
                     float in_scale, float out_scale, void *stream);

/*
 * ple-gate-split (src/kernels/pleSplit.ts:17-23, bind :50-63): per_layer_input_gate (8-bit) as
 * exact split-K integer partials (qgemv.ts:521-548 with exactPartials), written row-interleaved
 * for the fold's vec4 read: partials[(row / 4) * 4 * n + split * 4 + row % 4] = f32(sum of the
 * split's K band), n = k_splits, which is pleGateSplits() (1, 2, 4 or 8; 1 runs as 2,
 * pleSplit.ts:16). partials holds num_rows * n floats. Refuses num_rows % 4 != 0 and an
 * uncalibrated inScale with the reference's messages (pleSplit.ts:58-59).
 */
int g4_ple_gate_split(const void *wq, const float *scales, const void *x, int x_kind,
                      float *partials, int k, int num_rows, int k_splits, float in_scale,
                      void *stream);

/*
 * ple-fold-projection (src/kernels/pleSplit.ts:24-41, bind :64-84): per_layer_projection
 * (qgemv-8bit-gelu) whose gate is folded from ple-gate-split's partials (gate_parts, k_splits as
 * there): gate[i] = total = sum over s of the partials in split order from 0;
 * v = f32(f32(gate_in_scale * gate_scales[i]) * total), then clamp(RNE(v / gate_out_scale)) *
 * gate_out_scale when gate_out_scale != 0; the GEMV reads gelu_tanh(gate[i]) * up[up_offset + i].
 * act gives up (act->gate_scale is not used); gate_scales are the gate linear's row scales [K].
 * gate_parts and gate_scales need 16-byte alignment. One token (execute.ts:880-881).
 */
int g4_ple_fold_projection(const void *wq, const float *scales, const float *gate_parts,
                           const float *gate_scales, int k_splits, float gate_in_scale,
                           float gate_out_scale, const g4_gelu_act *act, void *dst, int out_kind,
                           int k, int num_rows, float in_scale, float out_scale, void *stream);

/* qgemv-4bit-gelu-exact-split (src/kernels/exactSplit.ts:19-31 with the gelu prologue; plan.ts
 * :594-597 producer down exact partials): the split-K partials of g4_qgemv_split over the gelu
 * prologue's codes; fold them with g4_qgemv_exact_merge (exact = 1) or g4_qgemv_merge. */
int g4_qgemv_gelu_split(int bits, const void *wq, const float *scales, const void *gate,
                        int gate_kind, const g4_gelu_act *act, float *partials, int k,
                        int num_rows, int k_splits, int exact, float in_scale, void *stream);

/* g4_qgemv_plan_create with a prologue per projection: acts[i] (acts may be NULL) gives
 * projection i the gelu prologue when acts[i].up is set; descs[i].x is then the gate. */
int g4_qgemv_plan_create_gelu(const g4_gemv_desc *descs, const g4_gelu_act *acts, int count,
                              g4_gemv_plan **plan);

/* quant.ts:309-334 srqCodes as a kernel: n activations (f32 or f16) to int8 codes on scale. */
int g4_srq_quantize(const void *x, int x_kind, int8_t *codes, int64_t n, float scale,
                    void *stream);

/* ---- the per-layer-embedding gather ------------------------------------------------------- */

/*
 * ple-gather-4bit (sliced = 0) and ple-gather-4bit-sliced (sliced = 1).
 * Replaces makeBind (src/kernels/embedGather.ts:435-485; entries :487, :547).
 * codes: the table (or, sliced, one vocabulary slice of it: row r of the slice is vocabulary row
 *        slice_start_row + r), cols/2 bytes per row. scales: [rows][groups_per_row], f32 or f16
 *        (scale_kind), addressed by the ABSOLUTE row (embedGather.ts:248). ids: int32 [slots].
 * dst [slots][cols]: G4_KIND_F32 = the reference's f32 (code-8)*(16*scale); G4_KIND_F16 the same
 * rounded to nearest even; G4_KIND_I8 the gathered signed codes. A sliced gather writes only the
 * slots whose id falls inside the slice (embedGather.ts:188-196) and refuses a missing or empty
 * range (:463-467).
 */
int g4_ple_gather(const void *codes, const void *scales, int scale_kind, const int32_t *ids,
                  void *dst, int out_kind, int slots, int cols, int group_size,
                  int groups_per_row, int sliced, int64_t slice_start_row,
                  int64_t slice_row_count, void *stream);

/*
 * One gather over a whole split table: every slice of `plan` in order (the reference walks
 * slicedGatherDispatches, embedGather.ts:403-419, one dispatch per slice). slice_codes[i] is the
 * device buffer of slice i. Launches one fused kernel that routes each token to its slice.
 */
int g4_ple_gather_split(const void *const *slice_codes, const int64_t *slice_starts,
                        const int64_t *slice_counts, int num_slices, const void *scales,
                        int scale_kind, const int32_t *ids, void *dst, int out_kind, int slots,
                        int cols, int group_size, int groups_per_row, void *stream);

/* ---- the split planner (pure host code) --------------------------------------------------- */

/* tableSplit.ts:51-81 TableSplitInput. max_slice_bytes 0 = DEFAULT_MAX_SLICE_BYTES (256 MiB). */
typedef struct g4_table_split_input {
    int64_t rows;
    int64_t row_bytes;
    int64_t max_storage_buffer_binding_size;
    int64_t max_buffer_size;
    int64_t max_storage_buffers_per_shader_stage;
    int64_t max_slice_bytes;
} g4_table_split_input;

/* tableSplit.ts:39-50 TableSlice. */
typedef struct g4_table_slice {
    int64_t index;
    int64_t start_row;
    int64_t row_count;
    int64_t byte_offset;
    int64_t byte_length;
} g4_table_slice;

/* tableSplit.ts:90-118 TableSplitPlan (without the note string). */
typedef struct g4_table_split_plan {
    int64_t rows;
    int64_t row_bytes;
    int64_t total_bytes;
    int64_t limit_bytes;
    int64_t rows_per_slice;
    int64_t num_slices;
    int32_t single;
    int32_t feasible;
    int64_t storage_bindings_per_dispatch;
    int64_t binding_budget;
    int64_t dispatches_per_gather;
} g4_table_split_plan;

/* tableSplit.ts:125-215 planTableSplit. Writes the plan and up to max_slices slices. */
int g4_plan_table_split(const g4_table_split_input *input, g4_table_split_plan *plan,
                        g4_table_slice *slices, int64_t max_slices);

/* tableSplit.ts:218-223 sliceForRow: the slice index carrying `row`, or -1. */
int64_t g4_slice_for_row(const g4_table_slice *slices, int64_t num_slices, int64_t row);

/* tableSplit.ts:226-230 GatherLimits: the limits half of a device profile. */
typedef struct g4_gather_limits {
    int64_t max_storage_buffer_binding_size;
    int64_t max_buffer_size;
    int64_t max_storage_buffers_per_shader_stage;
} g4_gather_limits;

/* tableSplit.ts:232-245 GatherSplitPlans (without the note string): both tables of one gather.
 * scales_single: the scale table is one buffer, which the sliced gather assumes (it addresses
 * scales by the absolute vocabulary row, embedGather.ts:248). */
typedef struct g4_gather_split_plans {
    g4_table_split_plan codes;
    g4_table_split_plan scales;
    int32_t scales_single;
} g4_gather_split_plans;

/* tableSplit.ts:257-287 planGatherSplit: plans the packed codes ([rows][code_row_bytes]) and the
 * f32 scales ([rows][scales_per_row]) with planTableSplit under the same limits and the default
 * slice cap. Up to max_code_slices / max_scale_slices slices are written (either array may be NULL
 * with a 0 count). Pure host code. */
int g4_plan_gather_split(int64_t rows, int64_t code_row_bytes, int64_t scales_per_row,
                         const g4_gather_limits *limits, g4_gather_split_plans *plans,
                         g4_table_slice *code_slices, int64_t max_code_slices,
                         g4_table_slice *scale_slices, int64_t max_scale_slices);

#ifdef __cplusplus
}
#endif

#endif /* G4W8A8_H */

// Host runtime of libg4w8a8: the last-error string, device memory, streams and events, the byte
// fill kernel and the pure table split planner (src/tableSplit.ts).
#include "g4_internal.h"

#include <cstdio>
#include <mutex>
#include <vector>

namespace g4 {

static thread_local std::string t_last_error;

int set_error(int status, const char *fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    t_last_error = buf;
    return status;
}

void clear_error() { t_last_error.clear(); }

int hip_status(hipError_t err, const char *what) {
    return set_error(err == hipErrorNoDevice ? G4_ERR_NO_DEVICE : G4_ERR_HIP, "%s failed: %s (%d)",
                     what, hipGetErrorString(err), (int)err);
}

int device_cu_count() {
    static std::mutex mu;
    static std::vector<int> cache;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 256;
    std::lock_guard<std::mutex> lock(mu);
    if ((int)cache.size() <= dev) cache.resize(dev + 1, 0);
    if (cache[dev] == 0) {
        int cus = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            cus <= 0)
            cus = 256;
        cache[dev] = cus;
    }
    return cache[dev];
}

__global__ void fill_u8_kernel(uint8_t *dst, uint8_t value, size_t bytes) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    size_t stride = (size_t)gridDim.x * blockDim.x;
    uint32_t v4 = 0x01010101u * value;
    size_t words = bytes / 4;
    if (((uintptr_t)dst & 3) == 0) {
        uint32_t *d = reinterpret_cast<uint32_t *>(dst);
        for (size_t w = i; w < words; w += stride) d[w] = v4;
        for (size_t b = words * 4 + i; b < bytes; b += stride) dst[b] = value;
    } else {
        for (size_t b = i; b < bytes; b += stride) dst[b] = value;
    }
}

}  // namespace g4

using namespace g4;

extern "C" {

int g4_abi_version(void) { return G4_ABI_VERSION; }

const char *g4_last_error(void) { return t_last_error.c_str(); }

int g4_device_count(int *count) {
    if (!count) return set_error(G4_ERR_INVALID, "g4_device_count: count is NULL");
    int n = 0;
    hipError_t err = hipGetDeviceCount(&n);
    if (err != hipSuccess) {
        *count = 0;
        return hip_status(err, "hipGetDeviceCount");
    }
    *count = n;
    return G4_OK;
}

int g4_set_device(int device) {
    G4_HIP(hipSetDevice(device));
    return G4_OK;
}

int g4_malloc(void **ptr, size_t bytes) {
    if (!ptr) return set_error(G4_ERR_INVALID, "g4_malloc: ptr is NULL");
    *ptr = nullptr;
    if (bytes == 0) bytes = 1;
    G4_HIP(hipMalloc(ptr, bytes));
    return G4_OK;
}

int g4_free(void *ptr) {
    if (ptr) G4_HIP(hipFree(ptr));
    return G4_OK;
}

int g4_memcpy_h2d(void *dst, const void *src, size_t bytes, void *stream) {
    if (bytes == 0) return G4_OK;
    if (!dst || !src) return set_error(G4_ERR_INVALID, "g4_memcpy_h2d: a NULL address");
    G4_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, as_stream(stream)));
    G4_HIP(hipStreamSynchronize(as_stream(stream)));
    return G4_OK;
}

int g4_memcpy_d2h(void *dst, const void *src, size_t bytes, void *stream) {
    if (bytes == 0) return G4_OK;
    if (!dst || !src) return set_error(G4_ERR_INVALID, "g4_memcpy_d2h: a NULL address");
    G4_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, as_stream(stream)));
    G4_HIP(hipStreamSynchronize(as_stream(stream)));
    return G4_OK;
}

int g4_host_alloc(void **ptr, size_t bytes) {
    if (!ptr) return set_error(G4_ERR_INVALID, "g4_host_alloc: ptr is NULL");
    *ptr = nullptr;
    if (bytes == 0) bytes = 1;
    G4_HIP(hipHostMalloc(ptr, bytes, hipHostMallocDefault));
    return G4_OK;
}

int g4_host_free(void *ptr) {
    if (ptr) G4_HIP(hipHostFree(ptr));
    return G4_OK;
}

int g4_memcpy_d2h_async(void *dst, const void *src, size_t bytes, void *stream) {
    if (bytes == 0) return G4_OK;
    if (!dst || !src) return set_error(G4_ERR_INVALID, "g4_memcpy_d2h_async: a NULL address");
    G4_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, as_stream(stream)));
    return G4_OK;
}

int g4_memcpy_d2d(void *dst, const void *src, size_t bytes, void *stream) {
    if (bytes == 0) return G4_OK;
    if (!dst || !src) return set_error(G4_ERR_INVALID, "g4_memcpy_d2d: a NULL address");
    G4_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, as_stream(stream)));
    return G4_OK;
}

int g4_fill_u8(void *dst, uint8_t value, size_t bytes, void *stream) {
    if (bytes == 0) return G4_OK;
    if (!dst) return set_error(G4_ERR_INVALID, "g4_fill_u8: dst is NULL");
    size_t words = (bytes + 3) / 4;
    size_t blocks = (words + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL(fill_u8_kernel, dim3((unsigned)blocks), dim3(256), 0, as_stream(stream),
                       reinterpret_cast<uint8_t *>(dst), value, bytes);
    G4_LAUNCHED("fill_u8_kernel");
    return G4_OK;
}

int g4_stream_create(void **stream) {
    if (!stream) return set_error(G4_ERR_INVALID, "g4_stream_create: stream is NULL");
    hipStream_t s = nullptr;
    // Default priority on purpose: streams of different priorities have hung on this pool.
    G4_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    *stream = s;
    return G4_OK;
}

int g4_stream_destroy(void *stream) {
    if (!stream) return G4_OK;
    // the stream's GEMM workspace goes with it (freed, or kept when a captured graph holds it), so
    // a later stream that reuses the handle does not inherit it
    int rc = workspace_forget_stream(stream);
    G4_HIP(hipStreamDestroy(as_stream(stream)));
    return rc;
}

int g4_stream_synchronize(void *stream) {
    G4_HIP(hipStreamSynchronize(as_stream(stream)));
    return G4_OK;
}

int g4_device_synchronize(void) {
    G4_HIP(hipDeviceSynchronize());
    return G4_OK;
}

int g4_event_create(void **event) {
    if (!event) return set_error(G4_ERR_INVALID, "g4_event_create: event is NULL");
    hipEvent_t e = nullptr;
    G4_HIP(hipEventCreate(&e));
    *event = e;
    return G4_OK;
}

int g4_event_destroy(void *event) {
    if (event) G4_HIP(hipEventDestroy(reinterpret_cast<hipEvent_t>(event)));
    return G4_OK;
}

int g4_event_record(void *event, void *stream) {
    G4_HIP(hipEventRecord(reinterpret_cast<hipEvent_t>(event), as_stream(stream)));
    return G4_OK;
}

int g4_event_synchronize(void *event) {
    G4_HIP(hipEventSynchronize(reinterpret_cast<hipEvent_t>(event)));
    return G4_OK;
}

int g4_event_elapsed_ms(float *ms, void *start, void *end) {
    if (!ms) return set_error(G4_ERR_INVALID, "g4_event_elapsed_ms: ms is NULL");
    G4_HIP(hipEventElapsedTime(ms, reinterpret_cast<hipEvent_t>(start),
                               reinterpret_cast<hipEvent_t>(end)));
    return G4_OK;
}

int g4_graph_begin_capture(void *stream) {
    if (!stream) return set_error(G4_ERR_INVALID, "graph capture needs a created stream, not the default stream");
    G4_HIP(hipStreamBeginCapture(as_stream(stream), hipStreamCaptureModeThreadLocal));
    return G4_OK;
}

namespace {

bool device_address(const void *p) {
    hipPointerAttribute_t a{};
    if (!p || hipPointerGetAttributes(&a, p) != hipSuccess) {
        (void)hipGetLastError();  // an address the runtime does not know is host memory
        return false;
    }
    return a.type == hipMemoryTypeDevice;
}

// G4_OK when every node of a captured graph is one a replay can run without touching host
// storage: kernels, device-to-device copies, empty, event record and event wait nodes.
int captured_node_refusal(hipGraph_t graph) {
    size_t count = 0;
    G4_HIP(hipGraphGetNodes(graph, nullptr, &count));
    std::vector<hipGraphNode_t> nodes(count);
    if (count) G4_HIP(hipGraphGetNodes(graph, nodes.data(), &count));
    for (hipGraphNode_t n : nodes) {
        hipGraphNodeType type;
        G4_HIP(hipGraphNodeGetType(n, &type));
        switch (type) {
        case hipGraphNodeTypeKernel:
        case hipGraphNodeTypeEmpty:
        case hipGraphNodeTypeEventRecord:
        case hipGraphNodeTypeWaitEvent:
            break;
        case hipGraphNodeTypeMemcpy: {
            hipMemcpy3DParms p{};
            if (hipGraphMemcpyNodeGetParams(n, &p) != hipSuccess) {
                (void)hipGetLastError();
                return set_error(G4_ERR_INVALID,
                                 "graph capture: the graph holds a copy whose ends cannot be inspected; "
                                 "enqueue host copies outside the capture");
            }
            const bool d2d = p.kind == hipMemcpyDeviceToDevice ||
                             (p.kind == hipMemcpyDefault && device_address(p.srcPtr.ptr) &&
                              device_address(p.dstPtr.ptr));
            if (!d2d)
                return set_error(G4_ERR_INVALID,
                                 "graph capture: the graph holds a copy to or from host memory, which "
                                 "every replay would touch after the enqueuing call returned; enqueue "
                                 "host copies outside the capture");
            break;
        }
        case hipGraphNodeTypeMemset:
            return set_error(G4_ERR_INVALID,
                             "graph capture: the graph holds a memset node; clear device memory "
                             "with a fill kernel (g4_fill_u8) inside a graph");
        default:
            return set_error(G4_ERR_INVALID, "graph capture: the graph holds a node of type %d; "
                             "only kernels, device copies and events are replayed", (int)type);
        }
    }
    return G4_OK;
}

}  // namespace

// The handle of a captured graph: the executable and an event recorded after each launch, so
// destroy waits for this graph's own replays and nothing else on the device.
struct G4Graph {
    hipGraphExec_t exec = nullptr;
    hipEvent_t done = nullptr;
    bool launched = false;
};

int g4_graph_end_capture(void *stream, void **graph_exec) {
    if (!stream || !graph_exec) return set_error(G4_ERR_INVALID, "g4_graph_end_capture: NULL argument");
    hipGraph_t graph = nullptr;
    G4_HIP(hipStreamEndCapture(as_stream(stream), &graph));
    // A kernel node holds copies of its arguments, so a replay reads no storage of the caller's
    // beyond the device buffers those arguments name. A copy node would read or write its host
    // buffer at every replay, long after the call that enqueued it returned (and a host buffer
    // freed by then is a host fault inside the graph launch), and memset nodes have given wrong
    // results on replays after the first. The graph keeps kernels, device-to-device copies and
    // the stream's own event and empty nodes only.
    const int bad = captured_node_refusal(graph);
    if (bad != G4_OK) {
        (void)hipGraphDestroy(graph);
        return bad;
    }
    hipGraphExec_t exec = nullptr;
    hipError_t err = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    (void)hipGraphDestroy(graph);
    if (err != hipSuccess) return hip_status(err, "hipGraphInstantiate");
    hipEvent_t done = nullptr;
    err = hipEventCreateWithFlags(&done, hipEventDisableTiming);
    if (err != hipSuccess) {
        (void)hipGraphExecDestroy(exec);
        return hip_status(err, "hipEventCreateWithFlags");
    }
    G4Graph *g = new G4Graph;
    g->exec = exec;
    g->done = done;
    *graph_exec = g;
    return G4_OK;
}

int g4_graph_launch(void *graph_exec, void *stream) {
    if (!graph_exec) return set_error(G4_ERR_INVALID, "g4_graph_launch: no graph");
    G4Graph *g = static_cast<G4Graph *>(graph_exec);
    G4_HIP(hipGraphLaunch(g->exec, as_stream(stream)));
    G4_HIP(hipEventRecord(g->done, as_stream(stream)));
    g->launched = true;
    return G4_OK;
}

int g4_graph_destroy(void *graph_exec) {
    if (!graph_exec) return G4_OK;
    G4Graph *g = static_cast<G4Graph *>(graph_exec);
    // Replays are ordered on their streams, and each launch re-records `done` after it, so the
    // event completes once the last launch (on whichever stream) has finished. Waiting on it
    // touches no other stream (a capture in progress elsewhere stays valid). The graph and the
    // event are released even when the wait reports an error.
    hipError_t wait = g->launched ? hipEventSynchronize(g->done) : hipSuccess;
    hipError_t d1 = hipGraphExecDestroy(g->exec);
    hipError_t d2 = hipEventDestroy(g->done);
    delete g;
    if (wait != hipSuccess) return hip_status(wait, "g4_graph_destroy: waiting for the last launch");
    if (d1 != hipSuccess) return hip_status(d1, "hipGraphExecDestroy");
    if (d2 != hipSuccess) return hip_status(d2, "hipEventDestroy");
    return G4_OK;
}

// tableSplit.ts:125-215 planTableSplit. Pure: limits go in as numbers.
int g4_plan_table_split(const g4_table_split_input *in, g4_table_split_plan *plan,
                        g4_table_slice *slices, int64_t max_slices) {
    if (!in || !plan) return set_error(G4_ERR_INVALID, "g4_plan_table_split: NULL argument");
    if (max_slices > 0 && !slices)
        return set_error(G4_ERR_INVALID, "g4_plan_table_split: slices is NULL");
    const int64_t kDefaultMaxSliceBytes = 256LL * 1024 * 1024;  // DEFAULT_MAX_SLICE_BYTES
    const int64_t kGatherBindings = 4;                          // GATHER_STORAGE_BINDINGS
    int64_t rows = in->rows > 0 ? in->rows : 0;
    int64_t row_bytes = in->row_bytes > 1 ? in->row_bytes : 1;
    int64_t total = rows * row_bytes;
    int64_t limit = in->max_storage_buffer_binding_size < in->max_buffer_size
                        ? in->max_storage_buffer_binding_size
                        : in->max_buffer_size;
    if (limit < 0) limit = 0;
    *plan = g4_table_split_plan{};
    plan->rows = rows;
    plan->row_bytes = row_bytes;
    plan->total_bytes = total;
    plan->limit_bytes = limit;
    plan->storage_bindings_per_dispatch = kGatherBindings;
    plan->binding_budget = in->max_storage_buffers_per_shader_stage;
    bool fits_whole = total > 0 && total <= limit;
    int64_t cap = in->max_slice_bytes > 0 ? in->max_slice_bytes : kDefaultMaxSliceBytes;
    int64_t slice_cap = limit < cap ? limit : cap;
    if (slice_cap < 1) slice_cap = 1;
    int64_t rows_per_slice = (fits_whole ? limit : slice_cap) / row_bytes;
    if (rows_per_slice < 1) {
        // One row does not fit in one binding: infeasible, no slices (tableSplit.ts:147-167).
        plan->rows_per_slice = 0;
        plan->num_slices = 0;
        plan->single = 0;
        plan->feasible = 0;
        plan->dispatches_per_gather = 0;
        return G4_OK;
    }
    // Slices start on a sixteen row boundary (tableSplit.ts:170-173).
    int64_t aligned = rows_per_slice >= 16 ? rows_per_slice - (rows_per_slice % 16) : rows_per_slice;
    int64_t per = rows < aligned ? rows : aligned;
    int64_t n = 0;
    for (int64_t start = 0; per > 0 && start < rows; start += per, ++n) {
        if (n < max_slices) {
            int64_t count = per < rows - start ? per : rows - start;
            slices[n] = g4_table_slice{n, start, count, start * row_bytes, count * row_bytes};
        }
    }
    if (n == 0) {
        if (max_slices > 0) slices[0] = g4_table_slice{0, 0, 0, 0, 0};
        n = 1;
    }
    plan->rows_per_slice = per;
    plan->num_slices = n;
    plan->single = n == 1;
    plan->dispatches_per_gather = n;
    plan->feasible = kGatherBindings <= plan->binding_budget;
    return G4_OK;
}

// tableSplit.ts:257-287 planGatherSplit: the codes and the f32 scales planned separately under
// the same limits (they reach the cap at very different sizes), scalesSingle from the scale plan.
int g4_plan_gather_split(int64_t rows, int64_t code_row_bytes, int64_t scales_per_row,
                         const g4_gather_limits *limits, g4_gather_split_plans *plans,
                         g4_table_slice *code_slices, int64_t max_code_slices,
                         g4_table_slice *scale_slices, int64_t max_scale_slices) {
    if (!limits || !plans) return set_error(G4_ERR_INVALID, "g4_plan_gather_split: NULL argument");
    g4_table_split_input in{};
    in.rows = rows;
    in.max_storage_buffer_binding_size = limits->max_storage_buffer_binding_size;
    in.max_buffer_size = limits->max_buffer_size;
    in.max_storage_buffers_per_shader_stage = limits->max_storage_buffers_per_shader_stage;
    in.max_slice_bytes = 0;
    in.row_bytes = code_row_bytes;
    int rc = g4_plan_table_split(&in, &plans->codes, code_slices, code_slices ? max_code_slices : 0);
    if (rc) return rc;
    in.row_bytes = scales_per_row * 4;
    rc = g4_plan_table_split(&in, &plans->scales, scale_slices, scale_slices ? max_scale_slices : 0);
    if (rc) return rc;
    plans->scales_single = plans->scales.single;
    return G4_OK;
}

// tableSplit.ts:218-223 sliceForRow.
int64_t g4_slice_for_row(const g4_table_slice *slices, int64_t num_slices, int64_t row) {
    if (!slices) return -1;
    for (int64_t i = 0; i < num_slices; i++) {
        if (row >= slices[i].start_row && row < slices[i].start_row + slices[i].row_count)
            return slices[i].index;
    }
    return -1;
}

}  // extern "C"

// g4_qgemm_noalloc: g4_qgemm for callers that cannot allocate device memory (code under HIP graph
// capture, tight serving loops, harnesses that forbid hipMalloc). It has no counterpart in the
// reference.
//
// The only memory g4_qgemm needs beyond its operands is the buffer of snapped activation codes on
// the tile path (f16 / f32 activations at M > 32: M * K bytes). Here that buffer is `scratch`, a
// file-scope device array of kScratchBytes that every GPU holds for the life of the process. The
// host never uses the array's name as an address: at the first call on a device (that device
// current) hipGetSymbolAddress gives that device's copy, kept per device and passed to the kernels.
// Every call on one GPU shares that GPU's array, so calls that overlap on one GPU (two streams, or
// two host threads) race on it; the array keeps the last call's codes and needs no clearing (each
// call writes every code it reads).
#include "g4_internal.h"

#include <mutex>

namespace {

constexpr size_t kScratchBytes = (size_t)8 << 20;  // 8 MiB: M * K <= 8 Mi codes
constexpr int kMaxDevices = 64;

__device__ __align__(256) int8_t scratch[kScratchBytes];

std::mutex g_mu;
int8_t *g_ptr[kMaxDevices] = {};

// This device's address of `scratch`, looked up once per device.
int scratch_ptr(int8_t **out) {
    int dev = 0;
    G4_HIP(hipGetDevice(&dev));
    if (dev < 0 || dev >= kMaxDevices)
        return g4::set_error(G4_ERR_UNSUPPORTED, "g4_qgemm_noalloc: device %d beyond %d", dev,
                             kMaxDevices);
    std::lock_guard<std::mutex> lock(g_mu);
    if (!g_ptr[dev]) {
        void *ptr = nullptr;
        G4_HIP(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
        if (!ptr) return g4::set_error(G4_ERR_HIP, "g4_qgemm_noalloc: no address for the scratch array");
        g_ptr[dev] = static_cast<int8_t *>(ptr);
    }
    *out = g_ptr[dev];
    return G4_OK;
}

}  // namespace

extern "C" {

size_t g4_qgemm_noalloc_max_codes(void) { return kScratchBytes; }

int g4_qgemm_noalloc(int bits, const void *wq, const float *scales, const void *x, int x_kind,
                     void *dst, int out_kind, int k, int num_rows, int m_cols, float in_scale,
                     float out_scale, void *stream) {
    // the call is checked and routed first (the reference's refusals come before any size
    // message); the scratch array's address is looked up only when the routed path snaps codes
    return g4::qgemm_given_codes(bits, wq, scales, x, x_kind, dst, out_kind, k, num_rows, m_cols,
                                 in_scale, out_scale, stream, scratch_ptr, kScratchBytes,
                                 "g4_qgemm_noalloc");
}

}  // extern "C"

// The per-stream activation workspace of the tile GEMM: the lifetime rules, host code only.
//
// A g4_qgemm call with f16 / f32 activations at M > 32 snaps them into a device buffer that the
// tile kernel then reads. The buffer belongs to (device, stream), so calls ordered on one stream
// share it. The rules:
//  - A call that fits the current buffer uses it. If the stream is capturing a graph, the buffer
//    is marked captured: the graph's nodes now hold its address.
//  - A call that needs a larger buffer while the stream captures is refused (allocating is not
//    allowed inside a capture, and a capture must not see a buffer that a later call could move).
//  - Growth outside a capture replaces the buffer. The old one is freed after the stream drains,
//    unless a capture took its address: then it is retired and kept until the process ends, so a
//    graph replayed later never touches freed memory.
//  - When the library destroys a stream, its buffer goes the same way (freed, or retired when
//    captured), and a new stream that reuses the handle starts without one.
// The runtime calls are passed in (WorkspaceOps) so a CPU test can drive these rules with fakes.
#ifndef G4_WORKSPACE_H
#define G4_WORKSPACE_H

#include <cstddef>
#include <cstdio>
#include <map>
#include <mutex>
#include <string>
#include <utility>
#include <vector>

namespace g4 {

struct WorkspaceOps {
    int (*alloc)(void **ptr, size_t bytes);       // 0 on success
    int (*release)(void *ptr);                    // 0 on success
    int (*drain)(void *stream);                   // waits for the stream's work; 0 on success
    int (*capturing)(void *stream, bool *yes);    // whether the stream is capturing; 0 on success
};

class WorkspaceCache {
  public:
    enum Status { kOk = 0, kRefused = 1, kRuntime = 2 };
    static constexpr size_t kMinBytes = (size_t)4 << 20;

    explicit WorkspaceCache(WorkspaceOps ops) : ops_(ops) {}

    // A buffer of at least `bytes` for (device, stream) in *out. On kRefused / kRuntime, *err says
    // why and nothing changed.
    Status get(int device, void *stream, size_t bytes, void **out, std::string *err) {
        std::lock_guard<std::mutex> lock(mu_);
        bool cap = false;
        if (ops_.capturing(stream, &cap)) return fail(err, kRuntime, "stream capture status query failed");
        Entry &e = entries_[{device, stream}];
        if (e.ptr && e.bytes >= bytes) {
            e.captured |= cap;
            *out = e.ptr;
            return kOk;
        }
        if (cap) {
            char msg[320];
            snprintf(msg, sizeof msg,
                     "the activation workspace of this stream holds %zu bytes and the call needs %zu: "
                     "growing it would allocate inside a graph capture. Run the same shape once on "
                     "this stream before capturing.",
                     e.bytes, bytes);
            return fail(err, kRefused, msg);
        }
        void *fresh = nullptr;
        const size_t grow = bytes > kMinBytes ? bytes : kMinBytes;
        if (ops_.alloc(&fresh, grow) || !fresh) return fail(err, kRuntime, "workspace allocation failed");
        if (e.ptr) {
            Status st = drop(stream, e);
            if (st != kOk) {
                (void)ops_.release(fresh);
                return fail(err, st, "draining the stream before freeing its old workspace failed");
            }
        }
        e.ptr = fresh;
        e.bytes = grow;
        e.captured = false;
        *out = fresh;
        return kOk;
    }

    // The stream is about to be destroyed: release its buffer, or retire it when captured.
    Status forget_stream(int device, void *stream) {
        std::lock_guard<std::mutex> lock(mu_);
        auto it = entries_.find({device, stream});
        if (it == entries_.end()) return kOk;
        Status st = it->second.ptr ? drop(stream, it->second) : kOk;
        entries_.erase(it);
        return st;
    }

    size_t live_buffers() {
        std::lock_guard<std::mutex> lock(mu_);
        size_t n = 0;
        for (auto &kv : entries_) n += kv.second.ptr != nullptr;
        return n;
    }
    size_t retired_buffers() {
        std::lock_guard<std::mutex> lock(mu_);
        return retired_.size();
    }

  private:
    struct Entry {
        void *ptr = nullptr;
        size_t bytes = 0;
        bool captured = false;
    };

    static Status fail(std::string *err, Status st, const char *msg) {
        if (err) *err = msg;
        return st;
    }

    // Gives up e's buffer: retired when a capture holds its address, else freed once the stream
    // has drained.
    Status drop(void *stream, Entry &e) {
        if (e.captured) {
            retired_.push_back(e.ptr);
        } else {
            if (ops_.drain(stream)) return kRuntime;
            (void)ops_.release(e.ptr);
        }
        e.ptr = nullptr;
        e.bytes = 0;
        e.captured = false;
        return kOk;
    }

    WorkspaceOps ops_;
    std::mutex mu_;
    std::map<std::pair<int, void *>, Entry> entries_;
    std::vector<void *> retired_;  // addresses held by captured graphs: never freed
};

}  // namespace g4

#endif  // G4_WORKSPACE_H

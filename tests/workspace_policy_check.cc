// CPU driver for the workspace lifetime rules (gemma4-webgpu-engine_amd/csrc/g4_workspace.h),
// with fake runtime calls that record what the cache asks for. Built and run by
// tests/test_workspace_policy.py; prints "ok" and exits 0 when every rule holds.
#include <cstdio>
#include <cstdlib>
#include <set>
#include <string>

#include "g4_workspace.h"

namespace {

std::set<void *> g_live;        // allocations not yet released
int g_drains = 0;               // drain calls
bool g_capturing = false;       // what the fake capture query answers
int g_next = 1;

int fake_alloc(void **p, size_t) {
    *p = reinterpret_cast<void *>(static_cast<uintptr_t>(0x1000 * g_next++));
    g_live.insert(*p);
    return 0;
}
int fake_release(void *p) {
    if (!g_live.erase(p)) {
        std::printf("FAIL: released %p twice or never allocated\n", p);
        std::exit(1);
    }
    return 0;
}
int fake_drain(void *) {
    ++g_drains;
    return 0;
}
int fake_capturing(void *, bool *yes) {
    *yes = g_capturing;
    return 0;
}

void expect(bool cond, const char *what) {
    if (!cond) {
        std::printf("FAIL: %s\n", what);
        std::exit(1);
    }
}

}  // namespace

int main() {
    using g4::WorkspaceCache;
    WorkspaceCache c(g4::WorkspaceOps{fake_alloc, fake_release, fake_drain, fake_capturing});
    void *s1 = reinterpret_cast<void *>(0xA1), *s2 = reinterpret_cast<void *>(0xA2);
    std::string err;
    void *p = nullptr, *q = nullptr;

    // first use allocates at least the minimum; a smaller call reuses it
    expect(c.get(0, s1, 100, &p, &err) == WorkspaceCache::kOk && p, "first get");
    expect(c.get(0, s1, 4096, &q, &err) == WorkspaceCache::kOk && q == p, "reuse on one stream");
    // another stream, or the same handle on another device, gets its own buffer
    expect(c.get(0, s2, 100, &q, &err) == WorkspaceCache::kOk && q != p, "per stream");
    expect(c.get(1, s1, 100, &q, &err) == WorkspaceCache::kOk && q != p, "per device");
    expect(c.live_buffers() == 3, "three live buffers");

    // growth outside a capture drains the stream and frees the old buffer
    int drains = g_drains;
    expect(c.get(0, s1, WorkspaceCache::kMinBytes * 2, &q, &err) == WorkspaceCache::kOk && q != p,
           "growth");
    expect(g_drains == drains + 1 && !g_live.count(p), "old buffer freed after a drain");
    p = q;

    // inside a capture: a fitting call marks the buffer captured; growth is refused
    g_capturing = true;
    expect(c.get(0, s1, 64, &q, &err) == WorkspaceCache::kOk && q == p, "fit under capture");
    err.clear();
    expect(c.get(0, s1, WorkspaceCache::kMinBytes * 8, &q, &err) == WorkspaceCache::kRefused,
           "growth under capture refused");
    expect(err.find("inside a graph capture") != std::string::npos, "refusal message");
    expect(g_live.count(p) == 1, "refusal changed nothing");
    // a stream with no workspace cannot get one inside a capture either
    void *s3 = reinterpret_cast<void *>(0xA3);
    expect(c.get(0, s3, 64, &q, &err) == WorkspaceCache::kRefused, "first allocation under capture");
    g_capturing = false;

    // growth after the capture: the captured buffer is retired, never freed
    expect(c.get(0, s1, WorkspaceCache::kMinBytes * 8, &q, &err) == WorkspaceCache::kOk && q != p,
           "growth after capture");
    expect(g_live.count(p) == 1 && c.retired_buffers() == 1, "captured buffer retired, not freed");
    void *captured_old = p;
    p = q;

    // destroying a stream frees its (uncaptured) buffer; a reused handle starts fresh
    drains = g_drains;
    expect(c.forget_stream(0, s1) == WorkspaceCache::kOk, "forget");
    expect(!g_live.count(p) && g_drains == drains + 1, "forgotten stream's buffer freed");
    expect(c.get(0, s1, 100, &q, &err) == WorkspaceCache::kOk && g_live.count(q), "handle reuse");
    // a stream whose buffer a capture holds: forgetting retires it
    g_capturing = true;
    expect(c.get(0, s2, 10, &p, &err) == WorkspaceCache::kOk, "capture on s2");
    g_capturing = false;
    expect(c.forget_stream(0, s2) == WorkspaceCache::kOk && g_live.count(p) &&
               c.retired_buffers() == 2, "captured buffer survives its stream");
    expect(g_live.count(captured_old) == 1, "retired buffers stay allocated");
    expect(c.forget_stream(0, reinterpret_cast<void *>(0xBAD)) == WorkspaceCache::kOk, "unknown");
    std::printf("ok\n");
    return 0;
}

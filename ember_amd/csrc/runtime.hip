// runtime.hip -- device memory and error handling of libember_amd.so.
//
// Replaces the reference's src/core/memory_gpu.cu:10-43 (cudaMalloc /
// cudaFree / cudaMemcpy / cudaDeviceSynchronize) and the exit()-on-error
// macros of src/core/utils_gpu.cuh:8-34 with HIP calls whose failures are
// recorded and reported instead of terminating the process.
//
// alloc_memory / free_memory keep a per-device cache of freed blocks.  The
// reference's free_memory is cudaFree, which waits for the whole device, and
// its alloc_memory a cudaMalloc per tensor; a training step of a small model
// frees and allocates hundreds of tensors, so the host stalled on every free
// and the queue of launches drained.  Here a freed block goes back to the
// cache at once and the next allocation of a similar size reuses it.  This
// is safe because every kernel and copy of the library is enqueued on the
// HIP null stream, which runs in order: work enqueued after the reuse cannot
// start before work enqueued before the free has finished.  (Memory used by
// work on other streams must be synchronised by its user before it is freed,
// as with any stream-ordered allocator.)  Sizes are rounded to 512 B below
// 1 MiB and to 2 MiB above; a cached block is reused for a request of up to
// 1.25 x smaller.  When hipMalloc runs out of memory the device's cache is
// released (after a device synchronisation) and the allocation retried.
// EMBER_AMD_NO_CACHE=1 in the environment turns the cache off (plain
// hipMalloc / hipFree per call, the reference's behaviour).
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <atomic>
#include <map>
#include <mutex>
#include <unordered_map>

#include "common.h"

namespace ember {

static thread_local int t_last_error = EMBER_OK;

int record_error(int status, const char *what, hipError_t err)
{
    if (status == EMBER_OK) return status;
    if (t_last_error == EMBER_OK) t_last_error = status;
    if (err != hipSuccess)
        fprintf(stderr, "ember_amd: %s failed: %s\n", what, hipGetErrorString(err));
    else
        fprintf(stderr, "ember_amd: %s: %s\n", what, ember_error_string(status));
    return status;
}

bool hip_ok(hipError_t err, const char *what)
{
    if (err == hipSuccess) return true;
    record_error(err == hipErrorOutOfMemory ? EMBER_ERR_OUT_OF_MEMORY : EMBER_ERR_DEVICE, what,
                 err);
    return false;
}

// Names of the kernels this thread launched since the last
// ember_launch_log_reset, comma-separated; a name that does not fit is
// dropped and the log ends in "...".
namespace {
constexpr int kLaunchLogBytes = 1024;
thread_local char t_launch_log[kLaunchLogBytes];
thread_local int t_launch_log_len = 0;
thread_local bool t_launch_log_full = false;

void log_launch(const char *kernel)
{
    if (t_launch_log_full) return;
    const size_t n = strlen(kernel);
    const int sep = t_launch_log_len ? 1 : 0;
    if (t_launch_log_len + sep + (int)n + 4 >= kLaunchLogBytes) {
        memcpy(t_launch_log + t_launch_log_len, "...", 4);
        t_launch_log_full = true;
        return;
    }
    if (sep) t_launch_log[t_launch_log_len++] = ',';
    memcpy(t_launch_log + t_launch_log_len, kernel, n + 1);
    t_launch_log_len += (int)n;
}
}  // namespace

bool launch_ok(const char *kernel)
{
    log_launch(kernel);
    return hip_ok(hipGetLastError(), kernel);
}

namespace {
constexpr int kMaxDevices = 16;
struct ScratchBuf {
    void *ptr = nullptr;
    size_t bytes = 0;
};
ScratchBuf g_scratch[kMaxDevices][kScratchSlots];
std::mutex g_scratch_mu;
}  // namespace

void *scratch(int slot, size_t bytes)
{
    int dev = 0;
    if (!hip_ok(hipGetDevice(&dev), "hipGetDevice")) return nullptr;
    if (dev < 0 || dev >= kMaxDevices || slot < 0 || slot >= kScratchSlots) {
        record_error(EMBER_ERR_INVALID_ARGUMENT, "scratch slot");
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    ScratchBuf &s = g_scratch[dev][slot];
    if (s.bytes >= bytes && s.ptr) return s.ptr;
    if (s.ptr) {
        // The old buffer may still be read by queued kernels on the null
        // stream; hipFree synchronises the device before releasing it.
        if (!hip_ok(hipFree(s.ptr), "hipFree(scratch)")) return nullptr;
        s.ptr = nullptr;
        s.bytes = 0;
    }
    size_t want = bytes < 4096 ? 4096 : bytes;
    void *p = nullptr;
    if (!hip_ok(hipMalloc(&p, want), "hipMalloc(scratch)")) return nullptr;
    s.ptr = p;
    s.bytes = want;
    return p;
}

// Frees every scratch buffer of `dev` (the current device), after the queued
// work that may still read them has finished.
void release_scratch(int dev)
{
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    bool synced = false;
    for (ScratchBuf &s : g_scratch[dev]) {
        if (!s.ptr) continue;
        if (!synced) {
            hip_ok(hipDeviceSynchronize(), "hipDeviceSynchronize(empty_cache)");
            synced = true;
        }
        hip_ok(hipFree(s.ptr), "hipFree(scratch)");
        s.ptr = nullptr;
        s.bytes = 0;
    }
}

namespace {
std::atomic<int> g_deterministic{0};
std::atomic<int> g_cu_count[kMaxDevices];
}  // namespace

int device_cu_count()
{
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    if (dev >= 0 && dev < kMaxDevices) {
        const int c = g_cu_count[dev].load(std::memory_order_relaxed);
        if (c > 0) return c;
    }
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
        return 0;
    if (dev >= 0 && dev < kMaxDevices) g_cu_count[dev].store(n, std::memory_order_relaxed);
    return n;
}

bool deterministic()
{
    return g_deterministic.load(std::memory_order_relaxed) != 0;
}

namespace {

struct LiveBlock {
    size_t bytes;  // rounded size of the hipMalloc'd block
    int dev;
};

struct DevicePool {
    std::multimap<size_t, void *> free_blocks;  // rounded size -> block
    size_t cached = 0;                          // bytes held in free_blocks
    size_t in_use = 0;                          // bytes handed out
    size_t peak = 0;                            // max of in_use
};

std::mutex g_alloc_mu;
std::unordered_map<void *, LiveBlock> g_live;  // blocks handed out by alloc_memory
DevicePool g_pool[kMaxDevices];
int g_cache_mode = -1;                         // -1 unresolved, 0 off, 1 on

bool cache_on()
{
    if (g_cache_mode < 0) {
        const char *v = getenv("EMBER_AMD_NO_CACHE");
        g_cache_mode = (v && v[0] && !(v[0] == '0' && v[1] == 0)) ? 0 : 1;
    }
    return g_cache_mode == 1;
}

size_t round_bytes(size_t b)
{
    constexpr size_t kSmall = 512, kLarge = size_t(2) << 20;
    if (b < (size_t(1) << 20)) return (b + kSmall - 1) / kSmall * kSmall;
    return (b + kLarge - 1) / kLarge * kLarge;
}

// Returns every cached block of `dev` to HIP.  Caller holds g_alloc_mu and
// has made `dev` current.
void release_cached(int dev)
{
    DevicePool &p = g_pool[dev];
    if (p.free_blocks.empty()) return;
    // Freed blocks may still be read by queued work.
    hip_ok(hipDeviceSynchronize(), "hipDeviceSynchronize(empty_cache)");
    for (auto &kv : p.free_blocks) hip_ok(hipFree(kv.second), "hipFree(empty_cache)");
    p.free_blocks.clear();
    p.cached = 0;
}

void *cached_alloc(size_t bytes)
{
    int dev = 0;
    if (!hip_ok(hipGetDevice(&dev), "hipGetDevice")) return nullptr;
    if (dev < 0 || dev >= kMaxDevices) {
        record_error(EMBER_ERR_UNSUPPORTED, "alloc_memory: device index");
        return nullptr;
    }
    const size_t want = round_bytes(bytes);
    std::lock_guard<std::mutex> lock(g_alloc_mu);
    DevicePool &p = g_pool[dev];
    void *ptr = nullptr;
    size_t got = want;
    auto it = p.free_blocks.lower_bound(want);
    if (it != p.free_blocks.end() && it->first <= want + want / 4) {
        ptr = it->second;
        got = it->first;
        p.cached -= got;
        p.free_blocks.erase(it);
    } else {
        hipError_t err = hipMalloc(&ptr, want);
        if (err == hipErrorOutOfMemory && !p.free_blocks.empty()) {
            (void)hipGetLastError();
            release_cached(dev);
            err = hipMalloc(&ptr, want);
        }
        if (err != hipSuccess) {
            // Same contract as memory_gpu.cu:15-19: report and return NULL;
            // the binding turns NULL into MemoryError.
            record_error(EMBER_ERR_OUT_OF_MEMORY, "alloc_memory", err);
            (void)hipGetLastError();
            return nullptr;
        }
    }
    g_live.emplace(ptr, LiveBlock{got, dev});
    p.in_use += got;
    if (p.in_use > p.peak) p.peak = p.in_use;
    return ptr;
}

void cached_free(void *ptr)
{
    std::lock_guard<std::mutex> lock(g_alloc_mu);
    auto it = g_live.find(ptr);
    if (it == g_live.end()) {
        // Not from alloc_memory (e.g. memory hipMalloc'd by the caller).
        hip_ok(hipFree(ptr), "free_memory");
        return;
    }
    DevicePool &p = g_pool[it->second.dev];
    p.in_use -= it->second.bytes;
    p.cached += it->second.bytes;
    p.free_blocks.emplace(it->second.bytes, ptr);
    g_live.erase(it);
}

}  // namespace

}  // namespace ember

extern "C" {

int ember_get_last_error(void)
{
    int s = ember::t_last_error;
    ember::t_last_error = EMBER_OK;
    return s;
}

const char *ember_error_string(int status)
{
    switch (status) {
        case EMBER_OK: return "success";
        case EMBER_ERR_INVALID_ARGUMENT: return "invalid argument";
        case EMBER_ERR_UNSUPPORTED: return "unsupported configuration";
        case EMBER_ERR_OUT_OF_MEMORY: return "out of device memory";
        case EMBER_ERR_DEVICE: return "HIP runtime error";
        default: return "unknown status";
    }
}

void *alloc_memory(size_t bytes)
{
    if (bytes == 0) return nullptr;  // hipMalloc(0) gives NULL without error
    if (ember::cache_on()) return ember::cached_alloc(bytes);
    void *ptr = nullptr;
    hipError_t err = hipMalloc(&ptr, bytes);
    if (err != hipSuccess) {
        // Same contract as memory_gpu.cu:15-19: report and return NULL; the
        // binding turns NULL into MemoryError.
        ember::record_error(EMBER_ERR_OUT_OF_MEMORY, "alloc_memory", err);
        (void)hipGetLastError();
        return nullptr;
    }
    return ptr;
}

void free_memory(void *ptr)
{
    if (!ptr) return;
    if (ember::cache_on())
        ember::cached_free(ptr);
    else
        ember::hip_ok(hipFree(ptr), "free_memory");
}

void ember_empty_cache(void)
{
    int dev = 0;
    if (!ember::hip_ok(hipGetDevice(&dev), "hipGetDevice")) return;
    if (dev < 0 || dev >= ember::kMaxDevices) return;
    {
        std::lock_guard<std::mutex> lock(ember::g_alloc_mu);
        ember::release_cached(dev);
    }
    ember::release_scratch(dev);
}

void ember_launch_log_reset(void)
{
    ember::t_launch_log_len = 0;
    ember::t_launch_log_full = false;
    ember::t_launch_log[0] = '\0';
}

const char *ember_launch_log(void)
{
    return ember::t_launch_log;
}

void ember_set_deterministic(int enabled)
{
    ember::g_deterministic.store(enabled ? 1 : 0, std::memory_order_relaxed);
}

int ember_get_deterministic(void)
{
    return ember::deterministic() ? 1 : 0;
}

void ember_memory_stats(size_t *in_use, size_t *cached, size_t *peak)
{
    int dev = 0;
    size_t u = 0, c = 0, pk = 0;
    if (ember::hip_ok(hipGetDevice(&dev), "hipGetDevice") && dev >= 0 && dev < ember::kMaxDevices) {
        std::lock_guard<std::mutex> lock(ember::g_alloc_mu);
        u = ember::g_pool[dev].in_use;
        c = ember::g_pool[dev].cached;
        pk = ember::g_pool[dev].peak;
    }
    if (in_use) *in_use = u;
    if (cached) *cached = c;
    if (peak) *peak = pk;
}

void copy_to_device(void *dst_device, const void *src_host, size_t bytes)
{
    if (bytes == 0) return;
    ember::hip_ok(hipMemcpy(dst_device, src_host, bytes, hipMemcpyHostToDevice), "copy_to_device");
}

void copy_from_device(void *dst_host, const void *src_device, size_t bytes)
{
    if (bytes == 0) return;
    ember::hip_ok(hipMemcpy(dst_host, src_device, bytes, hipMemcpyDeviceToHost),
                  "copy_from_device");
}

void sync_device(void)
{
    ember::hip_ok(hipDeviceSynchronize(), "sync_device");
}

}  // extern "C"

// runtime.hip -- device memory and error handling of libember_amd.so.
//
// Replaces the reference's src/core/memory_gpu.cu:10-43 (cudaMalloc /
// cudaFree / cudaMemcpy / cudaDeviceSynchronize) and the exit()-on-error
// macros of src/core/utils_gpu.cuh:8-34 with HIP calls whose failures are
// recorded and reported instead of terminating the process.
#include <stdio.h>

#include <mutex>

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

bool launch_ok(const char *kernel)
{
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
    if (ptr) ember::hip_ok(hipFree(ptr), "free_memory");
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

// distributions.hip -- uniform() and constant(), the two native entry points
// of the reference's random extension.
//
// Replaces src/random/distributions.h:8-9 as implemented for the GPU in
// src/random/distributions_gpu.cu:11-32, which src/random/random_api.c:70,88
// calls after _seed() has called srand() (random_api.c:97-105).
//
// uniform: the reference draws on the host so that srand() seeds both
// backends alike; here too.  Each value is low + (rand() / RAND_MAX) *
// (high - low) in fp32 with rand() the C library's generator, the one the
// reference binding's srand() seeds; the values are then copied to the
// device.  (This library's own binding, ember_amd._core._em_random, draws
// the same sequence from a private copy of the generator instead, because
// the HIP runtime also calls rand(); a caller of this entry point shares the
// C library's state with everything else in the process, as the reference
// does.)
//
// constant: every element is `value`; the reference fills a host buffer and
// copies it, here a kernel writes it on the null stream (same bits, no host
// buffer or PCIe transfer).
//
// Errors are recorded like every other void entry point (sticky status,
// ember_get_last_error); size <= 0 does nothing.
#include <stdlib.h>

#include "common.h"

namespace ember {
namespace {

typedef float f32x4_t __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(256) void fill_kernel(float *__restrict__ out, float value, int64_t n)
{
    const int64_t n4 = n >> 2;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    const f32x4_t v4 = {value, value, value, value};
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (((uintptr_t)out & 15) == 0) {
        for (; i < n4; i += stride) reinterpret_cast<f32x4_t *>(out)[i] = v4;
        i = (n4 << 2) + (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    }
    for (; i < n; i += stride) out[i] = value;
}

}  // namespace
}  // namespace ember

extern "C" void uniform(float low, float high, float *out, int size)
{
    if (size <= 0) return;
    if (!out) {
        ember::record_error(EMBER_ERR_INVALID_ARGUMENT, "uniform: null output");
        return;
    }
    float *host = (float *)malloc((size_t)size * sizeof(float));
    if (!host) {
        ember::record_error(EMBER_ERR_OUT_OF_MEMORY, "uniform: host buffer");
        return;
    }
    const float range = high - low;
    for (int i = 0; i < size; ++i) host[i] = low + ((float)rand() / (float)RAND_MAX) * range;
    copy_to_device(out, host, (size_t)size * sizeof(float));
    free(host);
}

extern "C" void constant(float value, float *out, int size)
{
    if (size <= 0) return;
    if (!out) {
        ember::record_error(EMBER_ERR_INVALID_ARGUMENT, "constant: null output");
        return;
    }
    const int64_t n = size;
    const int64_t groups = ((n + 3) / 4 + 255) / 256;
    const unsigned grid = (unsigned)(groups < 4096 ? groups : 4096);
    hipLaunchKernelGGL(ember::fill_kernel, dim3(grid), dim3(256), 0, 0, out, value, n);
    ember::launch_ok("constant");
}

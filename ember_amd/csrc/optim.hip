// optim.hip -- fused Adam over many parameter tensors in one launch.
//
// Replaces the reference's Adam.apply (ember/optim/adam.py:24-45), which runs
// 13 separate element-wise kernels per parameter (each allocating its
// result, ember/tensor/tensor.py:205-222).  The kernel performs exactly the
// same fp32 operations in exactly the same order, each correctly rounded and
// none contracted into an FMA, with the same fp32 scalars, so its results are
// bit-identical to Ember's composed update:
//     m = m*b1;  m = m + g*(1-b1)                 adam.py:36-37
//     v = v*b2;  v = v + (g*g)*(1-b2)             adam.py:39-40
//     mh = m / (1-b1^t);  vh = v / (1-b2^t)       adam.py:42-43
//     p = p - (mh*lr) / (sqrt(vh) + eps)          adam.py:45
// The scalars are formed in double and rounded to fp32 once, as Python
// computes them and the reference's binding converts them ("f",
// src/tensor/tensor_api.c:213).
//
// HBM-bound: 28 bytes per parameter (p, g, m, v read; p, m, v written).
// Tensors are packed kTensorsPerLaunch at a time into the kernel arguments
// (no device-side pointer table, no allocation); each workgroup handles one
// chunk of kChunk elements of one tensor, 16-byte vector loads where the
// tensor allows.
#include <math.h>

#include "common.h"

namespace ember {
namespace {

constexpr int kTensorsPerLaunch = 48;
constexpr int kBlock = 256;
constexpr int kChunk = 4 * kBlock * 4;  // elements per workgroup (4 float4 per thread)

struct AdamScalars {
    float b1, omb1, b2, omb2, bc1, bc2, lr, eps;
};

struct AdamBatch {
    float *p[kTensorsPerLaunch];
    const float *g[kTensorsPerLaunch];
    float *m[kTensorsPerLaunch];
    float *v[kTensorsPerLaunch];
    int64_t n[kTensorsPerLaunch];
    int first_chunk[kTensorsPerLaunch + 1];  // prefix sum of chunks per tensor
    int ntensors;
    AdamScalars s;
};

__device__ __forceinline__ void adam_one(float &p, float g, float &m, float &v, const AdamScalars &s)
{
#pragma clang fp contract(off)
    const float m1 = m * s.b1;
    const float m2 = m1 + g * s.omb1;
    const float v1 = v * s.b2;
    const float v2 = v1 + (g * g) * s.omb2;
    const float mh = m2 / s.bc1;
    const float vh = v2 / s.bc2;
    const float num = mh * s.lr;
    const float den = sqrtf(vh) + s.eps;
    p = p - num / den;
    m = m2;
    v = v2;
}

__global__ __launch_bounds__(kBlock) void adam_kernel(AdamBatch a)
{
    // Tensor of this workgroup: the last t with first_chunk[t] <= blockIdx.x.
    int t = 0;
    while (t + 1 < a.ntensors && a.first_chunk[t + 1] <= (int)blockIdx.x) ++t;
    const int64_t base = (int64_t)(blockIdx.x - a.first_chunk[t]) * kChunk;
    const int64_t n = a.n[t];
    float *p = a.p[t];
    const float *g = a.g[t];
    float *m = a.m[t];
    float *v = a.v[t];
    const bool vec = ((((uintptr_t)p) | ((uintptr_t)g) | ((uintptr_t)m) | ((uintptr_t)v)) & 15) == 0;
    if (vec && base + kChunk <= n) {
#pragma unroll
        for (int it = 0; it < kChunk / (4 * kBlock); ++it) {
            const int64_t i = base + 4 * ((int64_t)it * kBlock + threadIdx.x);
            float4 pv = *(const float4 *)(p + i);
            const float4 gv = *(const float4 *)(g + i);
            float4 mv = *(const float4 *)(m + i);
            float4 vv = *(const float4 *)(v + i);
            adam_one(pv.x, gv.x, mv.x, vv.x, a.s);
            adam_one(pv.y, gv.y, mv.y, vv.y, a.s);
            adam_one(pv.z, gv.z, mv.z, vv.z, a.s);
            adam_one(pv.w, gv.w, mv.w, vv.w, a.s);
            *(float4 *)(p + i) = pv;
            *(float4 *)(m + i) = mv;
            *(float4 *)(v + i) = vv;
        }
    } else {
        const int64_t end = base + kChunk < n ? base + kChunk : n;
        for (int64_t i = base + threadIdx.x; i < end; i += kBlock) {
            float pv = p[i], mv = m[i], vv = v[i];
            adam_one(pv, g[i], mv, vv, a.s);
            p[i] = pv;
            m[i] = mv;
            v[i] = vv;
        }
    }
}

}  // namespace
}  // namespace ember

extern "C" int adam_step(float *const *params, const float *const *grads, float *const *exp_avg,
                         float *const *exp_avg_sq, const int64_t *sizes, int ntensors, double lr,
                         double beta1, double beta2, double eps, int64_t step)
{
    using namespace ember;
    if (ntensors < 0 || step < 1 || (ntensors > 0 && (!params || !grads || !exp_avg || !exp_avg_sq || !sizes)))
        return record_error(EMBER_ERR_INVALID_ARGUMENT, "adam_step");
    for (int i = 0; i < ntensors; ++i) {
        if (sizes[i] < 0) return record_error(EMBER_ERR_INVALID_ARGUMENT, "adam_step");
        if (sizes[i] > 0 && (!params[i] || !grads[i] || !exp_avg[i] || !exp_avg_sq[i]))
            return record_error(EMBER_ERR_INVALID_ARGUMENT, "adam_step");
        if (sizes[i] / kChunk > (int64_t)INT32_MAX / 2)
            return record_error(EMBER_ERR_INVALID_ARGUMENT, "adam_step");
    }
    AdamScalars s;
    s.b1 = (float)beta1;
    s.omb1 = (float)(1.0 - beta1);
    s.b2 = (float)beta2;
    s.omb2 = (float)(1.0 - beta2);
    s.bc1 = (float)(1.0 - pow(beta1, (double)step));
    s.bc2 = (float)(1.0 - pow(beta2, (double)step));
    s.lr = (float)lr;
    s.eps = (float)eps;

    int i = 0;
    while (i < ntensors) {
        AdamBatch a;
        a.s = s;
        int nt = 0;
        int64_t chunks = 0;
        a.first_chunk[0] = 0;
        for (; i < ntensors && nt < kTensorsPerLaunch; ++i) {
            if (sizes[i] == 0) continue;
            const int64_t c = (sizes[i] + kChunk - 1) / kChunk;
            if (nt > 0 && chunks + c > (int64_t)INT32_MAX / 2) break;  // next launch
            a.p[nt] = params[i];
            a.g[nt] = grads[i];
            a.m[nt] = exp_avg[i];
            a.v[nt] = exp_avg_sq[i];
            a.n[nt] = sizes[i];
            chunks += c;
            a.first_chunk[++nt] = (int)chunks;
        }
        if (nt == 0) continue;
        a.ntensors = nt;
        hipLaunchKernelGGL(adam_kernel, dim3((unsigned)chunks), dim3(kBlock), 0, 0, a);
        if (!launch_ok("adam_kernel")) return EMBER_ERR_DEVICE;
    }
    return EMBER_OK;
}

// optim.hip -- fused optimiser steps (Adam, AdamW, SGD) over many parameter
// tensors in one launch.
//
// Replaces the reference's Adam.apply (ember/optim/adam.py:24-45),
// AdamW.apply (ember/optim/adamw.py:33-56) and SGD.apply
// (ember/optim/sgd.py:25-35), which run 3 to 15 separate element-wise
// kernels per parameter (each allocating its result,
// ember/tensor/tensor.py:205-222).  Each kernel performs exactly the same
// fp32 operations in exactly the same order, each correctly rounded and none
// contracted into an FMA, with the same fp32 scalars, so its results are
// bit-identical to Ember's composed update:
//   Adam:  m = m*b1;  m = m + g*(1-b1)                 adam.py:36-37
//          v = v*b2;  v = v + (g*g)*(1-b2)             adam.py:39-40
//          mh = m / (1-b1^t);  vh = v / (1-b2^t)       adam.py:42-43
//          p = p - (mh*lr) / (sqrt(vh) + eps)          adam.py:45
//   AdamW: the same m, v, mh, vh, then                 adamw.py:45-52
//          p = p - p*(lr*wd)                           adamw.py:55
//          p = p - (mh*lr) / (sqrt(vh) + eps)          adamw.py:56
//   SGD:   v = v*momentum;  v = v + g;  p = p - v*lr   sgd.py:33-35
// The scalars are formed in double and rounded to fp32 once, as Python
// computes them (lr*wd is one Python product) and the reference's binding
// converts them ("f", src/tensor/tensor_api.c:213).
//
// HBM-bound: 28 bytes per parameter for Adam / AdamW (p, g, m, v read; p, m,
// v written), 20 for SGD (p, g, v read; p, v written).
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

enum class Rule { kAdam, kAdamW, kSgd };

struct OptScalars {
    float b1, omb1, b2, omb2, bc1, bc2, lr, eps;
    float lrwd;      // AdamW: fp32(lr * weight_decay)
    float momentum;  // SGD
};

// m is Adam's first moment or SGD's velocity; v (Adam's second moment) is
// not touched by SGD.
struct OptBatch {
    float *p[kTensorsPerLaunch];
    const float *g[kTensorsPerLaunch];
    float *m[kTensorsPerLaunch];
    float *v[kTensorsPerLaunch];
    int64_t n[kTensorsPerLaunch];
    int first_chunk[kTensorsPerLaunch + 1];  // prefix sum of chunks per tensor
    int ntensors;
    OptScalars s;
};

template <Rule R>
__device__ __forceinline__ void update_one(float &p, float g, float &m, float &v, const OptScalars &s)
{
#pragma clang fp contract(off)
    if constexpr (R == Rule::kSgd) {
        const float v1 = m * s.momentum;
        const float v2 = v1 + g;
        p = p - v2 * s.lr;
        m = v2;
    } else {
        const float m1 = m * s.b1;
        const float m2 = m1 + g * s.omb1;
        const float v1 = v * s.b2;
        const float v2 = v1 + (g * g) * s.omb2;
        const float mh = m2 / s.bc1;
        const float vh = v2 / s.bc2;
        const float num = mh * s.lr;
        const float den = sqrtf(vh) + s.eps;
        float pd = p;
        if constexpr (R == Rule::kAdamW) pd = pd - pd * s.lrwd;
        p = pd - num / den;
        m = m2;
        v = v2;
    }
}

template <Rule R>
__global__ __launch_bounds__(kBlock) void opt_kernel(OptBatch a)
{
    constexpr bool kSecond = R != Rule::kSgd;  // a second-moment tensor
    // Tensor of this workgroup: the last t with first_chunk[t] <= blockIdx.x.
    int t = 0;
    while (t + 1 < a.ntensors && a.first_chunk[t + 1] <= (int)blockIdx.x) ++t;
    const int64_t base = (int64_t)(blockIdx.x - a.first_chunk[t]) * kChunk;
    const int64_t n = a.n[t];
    float *p = a.p[t];
    const float *g = a.g[t];
    float *m = a.m[t];
    float *v = a.v[t];
    const uintptr_t bits = ((uintptr_t)p) | ((uintptr_t)g) | ((uintptr_t)m) | (kSecond ? (uintptr_t)v : 0);
    if ((bits & 15) == 0 && base + kChunk <= n) {
#pragma unroll
        for (int it = 0; it < kChunk / (4 * kBlock); ++it) {
            const int64_t i = base + 4 * ((int64_t)it * kBlock + threadIdx.x);
            float4 pv = *(const float4 *)(p + i);
            const float4 gv = *(const float4 *)(g + i);
            float4 mv = *(const float4 *)(m + i);
            float4 vv = kSecond ? *(const float4 *)(v + i) : float4{0.f, 0.f, 0.f, 0.f};
            update_one<R>(pv.x, gv.x, mv.x, vv.x, a.s);
            update_one<R>(pv.y, gv.y, mv.y, vv.y, a.s);
            update_one<R>(pv.z, gv.z, mv.z, vv.z, a.s);
            update_one<R>(pv.w, gv.w, mv.w, vv.w, a.s);
            *(float4 *)(p + i) = pv;
            *(float4 *)(m + i) = mv;
            if (kSecond) *(float4 *)(v + i) = vv;
        }
    } else {
        const int64_t end = base + kChunk < n ? base + kChunk : n;
        for (int64_t i = base + threadIdx.x; i < end; i += kBlock) {
            float pv = p[i], mv = m[i], vv = kSecond ? v[i] : 0.0f;
            update_one<R>(pv, g[i], mv, vv, a.s);
            p[i] = pv;
            m[i] = mv;
            if (kSecond) v[i] = vv;
        }
    }
}

// Argument checks shared by the entry points (v may be null for SGD).
int check_opt_args(float *const *params, const float *const *grads, float *const *m,
                   float *const *v, bool need_v, const int64_t *sizes, int ntensors, const char *who)
{
    if (ntensors < 0 || (ntensors > 0 && (!params || !grads || !m || (need_v && !v) || !sizes)))
        return record_error(EMBER_ERR_INVALID_ARGUMENT, who);
    for (int i = 0; i < ntensors; ++i) {
        if (sizes[i] < 0) return record_error(EMBER_ERR_INVALID_ARGUMENT, who);
        if (sizes[i] > 0 && (!params[i] || !grads[i] || !m[i] || (need_v && !v[i])))
            return record_error(EMBER_ERR_INVALID_ARGUMENT, who);
        if (sizes[i] / kChunk > (int64_t)INT32_MAX / 2) return record_error(EMBER_ERR_INVALID_ARGUMENT, who);
    }
    return EMBER_OK;
}

// Launches opt_kernel<R> over the tensors, kTensorsPerLaunch at a time.
template <Rule R>
int launch_opt(float *const *params, const float *const *grads, float *const *m, float *const *v,
               const int64_t *sizes, int ntensors, const OptScalars &s, const char *who)
{
    int i = 0;
    while (i < ntensors) {
        OptBatch a;
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
            a.m[nt] = m[i];
            a.v[nt] = v ? v[i] : nullptr;
            a.n[nt] = sizes[i];
            chunks += c;
            a.first_chunk[++nt] = (int)chunks;
        }
        if (nt == 0) continue;
        a.ntensors = nt;
        hipLaunchKernelGGL((opt_kernel<R>), dim3((unsigned)chunks), dim3(kBlock), 0, 0, a);
        if (!launch_ok(who)) return EMBER_ERR_DEVICE;
    }
    return EMBER_OK;
}

OptScalars adam_scalars(double lr, double beta1, double beta2, double eps, int64_t step)
{
    OptScalars s{};
    s.b1 = (float)beta1;
    s.omb1 = (float)(1.0 - beta1);
    s.b2 = (float)beta2;
    s.omb2 = (float)(1.0 - beta2);
    s.bc1 = (float)(1.0 - pow(beta1, (double)step));
    s.bc2 = (float)(1.0 - pow(beta2, (double)step));
    s.lr = (float)lr;
    s.eps = (float)eps;
    return s;
}

}  // namespace
}  // namespace ember

extern "C" int adam_step(float *const *params, const float *const *grads, float *const *exp_avg,
                         float *const *exp_avg_sq, const int64_t *sizes, int ntensors, double lr,
                         double beta1, double beta2, double eps, int64_t step)
{
    using namespace ember;
    int st = check_opt_args(params, grads, exp_avg, exp_avg_sq, true, sizes, ntensors, "adam_step");
    if (st != EMBER_OK) return st;
    if (step < 1) return record_error(EMBER_ERR_INVALID_ARGUMENT, "adam_step");
    return launch_opt<Rule::kAdam>(params, grads, exp_avg, exp_avg_sq, sizes, ntensors,
                                   adam_scalars(lr, beta1, beta2, eps, step), "adam_step");
}

extern "C" int adamw_step(float *const *params, const float *const *grads, float *const *exp_avg,
                          float *const *exp_avg_sq, const int64_t *sizes, int ntensors, double lr,
                          double beta1, double beta2, double eps, double weight_decay, int64_t step)
{
    using namespace ember;
    int st = check_opt_args(params, grads, exp_avg, exp_avg_sq, true, sizes, ntensors, "adamw_step");
    if (st != EMBER_OK) return st;
    if (step < 1) return record_error(EMBER_ERR_INVALID_ARGUMENT, "adamw_step");
    OptScalars s = adam_scalars(lr, beta1, beta2, eps, step);
    s.lrwd = (float)(lr * weight_decay);
    return launch_opt<Rule::kAdamW>(params, grads, exp_avg, exp_avg_sq, sizes, ntensors, s,
                                    "adamw_step");
}

extern "C" int sgd_step(float *const *params, const float *const *grads, float *const *velocity,
                        const int64_t *sizes, int ntensors, double lr, double momentum)
{
    using namespace ember;
    int st = check_opt_args(params, grads, velocity, nullptr, false, sizes, ntensors, "sgd_step");
    if (st != EMBER_OK) return st;
    OptScalars s{};
    s.lr = (float)lr;
    s.momentum = (float)momentum;
    return launch_opt<Rule::kSgd>(params, grads, velocity, nullptr, sizes, ntensors, s, "sgd_step");
}

// softmax.hip -- softmax along one axis in one launch.
//
// Ember's softmax(a, axis) is exp(a - amax(a, axis)) / sum(exp(...), axis)
// (ember/tensor/tensor.py:430-437), run by the reference as five launches
// (max_axis, sub_broadcasted, exponent_tensor, sum_axis, truediv_broadcasted)
// and four intermediate tensors.  Here each line along the axis is read once
// or three times and written once:
//   m = max over the line (fmaxf: any order gives the same value)
//   e = expf(x - m),  s = sum of e,  out = e * (1 / s)  (within 2 ulp of e / s)
// with the composed path's fp32 operations per element, except that the
// division is a multiply by the line's reciprocal.  The order of the sum also
// differs where lines are long: the last axis is reduced
// across a wave or a workgroup in a fixed tree order (deterministic);
// other axes are summed in index order as sum_axis does.
//   * last axis, L <= 2048: a wave per row, the row held in registers;
//   * last axis, L > 2048: a workgroup per row, three passes over the row
//     (the re-reads hit L2), float4 when rows are 16-byte aligned;
//   * other axes: a thread per (outer, inner) line, three passes, loads
//     coalesced across inner.
// HBM-bound: 8 bytes per element (read + write) on the first two paths.
#include <math.h>

#include "common.h"

namespace ember {
namespace {

__device__ __forceinline__ float wave_max(float v)
{
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

__device__ __forceinline__ float wave_sum(float v)
{
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

template <int NV>
__global__ __launch_bounds__(256) void softmax_rows_wave(const float *__restrict__ a,
                                                         float *__restrict__ out, int rows, int L)
{
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    const float *p = a + (int64_t)row * L;
    float *q = out + (int64_t)row * L;
    float v[NV];
    float m = -INFINITY;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int c = 64 * j + lane;
        v[j] = c < L ? p[c] : -INFINITY;
        m = fmaxf(m, v[j]);
    }
    m = wave_max(m);
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int c = 64 * j + lane;
        const float e = c < L ? expf(v[j] - m) : 0.0f;
        v[j] = e;
        s += e;
    }
    // One correctly rounded reciprocal per row and a multiply per element
    // (within 2 ulp of the quotient) instead of an IEEE division per element.
    const float inv = 1.0f / wave_sum(s);
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int c = 64 * j + lane;
        if (c < L) q[c] = v[j] * inv;
    }
}

// Block-wide reduction of one value per thread (256 threads); every thread
// gets the result.
template <bool MAX>
__device__ __forceinline__ float block_reduce(float v, float *red)
{
    v = MAX ? wave_max(v) : wave_sum(v);
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    float r = red[0];
#pragma unroll
    for (int i = 1; i < 4; ++i) r = MAX ? fmaxf(r, red[i]) : r + red[i];
    __syncthreads();
    return r;
}

template <bool VEC4>
__global__ __launch_bounds__(256) void softmax_rows_block(const float *__restrict__ a,
                                                          float *__restrict__ out, int L)
{
    __shared__ float red[4];
    const int t = threadIdx.x;
    const float *p = a + (int64_t)blockIdx.x * L;
    float *q = out + (int64_t)blockIdx.x * L;
    float m = -INFINITY;
    if (VEC4) {
        for (int c = 4 * t; c < L; c += 1024) {
            const float4 x = *(const float4 *)&p[c];
            m = fmaxf(m, fmaxf(fmaxf(x.x, x.y), fmaxf(x.z, x.w)));
        }
    } else {
        for (int c = t; c < L; c += 256) m = fmaxf(m, p[c]);
    }
    m = block_reduce<true>(m, red);
    float s = 0.0f;
    if (VEC4) {
        for (int c = 4 * t; c < L; c += 1024) {
            const float4 x = *(const float4 *)&p[c];
            s += expf(x.x - m);
            s += expf(x.y - m);
            s += expf(x.z - m);
            s += expf(x.w - m);
        }
    } else {
        for (int c = t; c < L; c += 256) s += expf(p[c] - m);
    }
    const float inv = 1.0f / block_reduce<false>(s, red);
    if (VEC4) {
        for (int c = 4 * t; c < L; c += 1024) {
            const float4 x = *(const float4 *)&p[c];
            float4 y;
            y.x = expf(x.x - m) * inv;
            y.y = expf(x.y - m) * inv;
            y.z = expf(x.z - m) * inv;
            y.w = expf(x.w - m) * inv;
            *(float4 *)&q[c] = y;
        }
    } else {
        for (int c = t; c < L; c += 256) q[c] = expf(p[c] - m) * inv;
    }
}

__global__ __launch_bounds__(256) void softmax_lines(const float *__restrict__ a,
                                                     float *__restrict__ out, int outer, int inner,
                                                     int L)
{
    const int64_t total = (int64_t)outer * inner;
    for (int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x; idx < total;
         idx += (int64_t)gridDim.x * 256) {
        const int64_t o = idx / inner, i = idx - o * inner;
        const int64_t base = o * L * inner + i;
        float m = a[base];
        for (int r = 1; r < L; ++r) m = fmaxf(m, a[base + (int64_t)r * inner]);
        float s = 0.0f;
        for (int r = 0; r < L; ++r) s += expf(a[base + (int64_t)r * inner] - m);
        // An IEEE division per element, as Ember's composition (a strided
        // line is latency-bound, so the reciprocal would save nothing here).
        for (int r = 0; r < L; ++r) {
            const int64_t off = base + (int64_t)r * inner;
            out[off] = expf(a[off] - m) / s;
        }
    }
}

template <int NV>
void launch_wave(const float *a, float *out, int rows, int L)
{
    hipLaunchKernelGGL(softmax_rows_wave<NV>, dim3((rows + 3) / 4), dim3(256), 0, 0, a, out, rows, L);
}

}  // namespace
}  // namespace ember

extern "C" int softmax_axis(const float *a, float *out, int outer, int inner, int axis_dim)
{
    using namespace ember;
    if (outer < 0 || inner < 0 || axis_dim < 0) return record_error(EMBER_ERR_INVALID_ARGUMENT, "softmax_axis");
    if ((int64_t)outer * inner * axis_dim == 0) return EMBER_OK;
    if (!a || !out) return record_error(EMBER_ERR_INVALID_ARGUMENT, "softmax_axis");
    if (inner == 1) {
        const int L = axis_dim, rows = outer;
        if (L <= 64) launch_wave<1>(a, out, rows, L);
        else if (L <= 128) launch_wave<2>(a, out, rows, L);
        else if (L <= 256) launch_wave<4>(a, out, rows, L);
        else if (L <= 512) launch_wave<8>(a, out, rows, L);
        else if (L <= 1024) launch_wave<16>(a, out, rows, L);
        else if (L <= 2048) launch_wave<32>(a, out, rows, L);
        else if (L % 4 == 0 && (((uintptr_t)a | (uintptr_t)out) % 16) == 0)
            hipLaunchKernelGGL(softmax_rows_block<true>, dim3(rows), dim3(256), 0, 0, a, out, L);
        else
            hipLaunchKernelGGL(softmax_rows_block<false>, dim3(rows), dim3(256), 0, 0, a, out, L);
    } else {
        const int64_t total = (int64_t)outer * inner;
        int64_t blocks = (total + 255) / 256;
        if (blocks > 65536) blocks = 65536;
        hipLaunchKernelGGL(softmax_lines, dim3((unsigned)blocks), dim3(256), 0, 0, a, out, outer,
                           inner, axis_dim);
    }
    return launch_ok("softmax_axis") ? EMBER_OK : EMBER_ERR_DEVICE;
}

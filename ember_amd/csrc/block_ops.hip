// block_ops.hip -- the element-wise and reduction pieces a transformer block's
// backward needs beside the GEMMs and attention: Ember's GELU backward and
// the column sums that give bias gradients.
//
//   gelu_bwd: dx = dy * ((1 + tanh(0.8u)) * (0.5 + 0.8(u - y)))
//             (ember/nn/activations.py:61-66, evaluated in the order of
//             Ember's element-wise operators; u = GELU input, y = output,
//             recomputed from u with the forward's operations when not
//             given: 12 instead of 16 bytes per element)
//   col_sum:  out[c] = sum_r x[r][c], the bias gradient of a Linear layer
//             (ember/nn/layers.py:54, em.sum(grad_y, axis=0)).  Widths that
//             are a multiple of 4 (16-byte aligned): a workgroup owns 64
//             columns (16 float4 quads) of a 256-row slice and 16 row groups
//             sum interleaved rows, then the groups are added in order; a
//             second launch reduces the slice partials the same way.  Other
//             widths: one thread per column over 128-row slices, then the
//             slices in order.  Either way the order is fixed, so the result
//             is deterministic.
// Both HBM-bound.
#include <math.h>

#include "common.h"
#include "mfma.h"

namespace ember {
namespace {

// One element: t = 1 + tanh(0.8u); y = (0.5u) * t when recomputed (the
// forward's own operations, so the same bits as the stored output);
// dx = dy * (t * (0.8(u - y) + 0.5)).
template <bool RECOMPUTE>
__device__ __forceinline__ float gelu_bwd_one(float dyv, float x, float yv)
{
#pragma clang fp contract(off)
    const float t = tanhf(x * 0.8f) + 1.0f;
    const float y = RECOMPUTE ? (x * 0.5f) * t : yv;
    const float r = (x - y) * 0.8f + 0.5f;
    return dyv * (t * r);
}

// n % 4 == 0 and 16-byte aligned operands: float4 per thread and pass.
template <bool RECOMPUTE>
__global__ __launch_bounds__(256) void gelu_bwd_vec4(const float *__restrict__ dy, const float *__restrict__ u,
                                                     const float *__restrict__ y, float *__restrict__ dx,
                                                     int64_t n4)
{
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += (int64_t)gridDim.x * 256) {
        const f32x4 g = ((const f32x4 *)dy)[i];
        const f32x4 x = ((const f32x4 *)u)[i];
        f32x4 yv = {0.f, 0.f, 0.f, 0.f};
        if (!RECOMPUTE) yv = ((const f32x4 *)y)[i];
        f32x4 o;
#pragma unroll
        for (int j = 0; j < 4; ++j) o[j] = gelu_bwd_one<RECOMPUTE>(g[j], x[j], yv[j]);
        ((f32x4 *)dx)[i] = o;
    }
}

template <bool RECOMPUTE>
__global__ __launch_bounds__(256) void gelu_bwd_kernel(const float *__restrict__ dy,
                                                       const float *__restrict__ u,
                                                       const float *__restrict__ y,
                                                       float *__restrict__ dx, int64_t n)
{
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256)
        dx[i] = gelu_bwd_one<RECOMPUTE>(dy[i], u[i], RECOMPUTE ? 0.0f : y[i]);
}

constexpr int kRowsPerSlice = 128;

__global__ __launch_bounds__(256) void col_sum_partial(const float *__restrict__ x,
                                                       float *__restrict__ part, int64_t rows,
                                                       int cols)
{
    const int c = blockIdx.x * 256 + threadIdx.x;
    if (c >= cols) return;
    const int64_t r0 = (int64_t)blockIdx.y * kRowsPerSlice;
    const int64_t r1 = r0 + kRowsPerSlice < rows ? r0 + kRowsPerSlice : rows;
    float s = 0.0f;
    for (int64_t r = r0; r < r1; ++r) s += x[r * cols + c];
    part[(int64_t)blockIdx.y * cols + c] = s;
}

// out[y][c] = sum over rows r in [y*rpw, (y+1)*rpw) of x[r][c], c in quads.
constexpr int kQuads = 16, kGroups = 16, kSliceRows = 256;
// Row loaders for col_reduce4: a plain matrix, or the GELU backward
// evaluated on the fly (dx stored as it is summed, the same bits as
// gelu_bwd_vec4 with the output recomputed).
struct PlainRows {
    const float *x;
    __device__ __forceinline__ float4 operator()(int64_t off) const { return *(const float4 *)(x + off); }
};
struct GeluBwdRows {
    const float *dy, *u;
    float *dx;
    __device__ __forceinline__ float4 operator()(int64_t off) const
    {
        const f32x4 g = *(const f32x4 *)(dy + off);
        const f32x4 x = *(const f32x4 *)(u + off);
        f32x4 o;
#pragma unroll
        for (int j = 0; j < 4; ++j) o[j] = gelu_bwd_one<true>(g[j], x[j], 0.0f);
        *(f32x4 *)(dx + off) = o;
        return make_float4(o[0], o[1], o[2], o[3]);
    }
};

template <class LD>
__global__ __launch_bounds__(256) void col_reduce4(LD ld, float *__restrict__ out, int64_t rows, int cols,
                                                   int rpw)
{
    __shared__ float4 red[kGroups][kQuads];
    const int q = threadIdx.x % kQuads, g = threadIdx.x / kQuads;
    const int quad = blockIdx.x * kQuads + q;
    const int64_t r0 = (int64_t)blockIdx.y * rpw;
    const int64_t r1 = r0 + rpw < rows ? r0 + rpw : rows;
    float4 s = make_float4(0.f, 0.f, 0.f, 0.f);
    if (4 * quad < cols) {
        int64_t r = r0 + g;
        // Eight rows in flight, then the adds in row order (the same sums as
        // one row at a time).
        for (; r + 7 * kGroups < r1; r += 8 * kGroups) {
            float4 v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) v[u] = ld((r + u * kGroups) * cols + 4 * quad);
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                s.x += v[u].x;
                s.y += v[u].y;
                s.z += v[u].z;
                s.w += v[u].w;
            }
        }
        for (; r < r1; r += kGroups) {
            const float4 v = ld(r * cols + 4 * quad);
            s.x += v.x;
            s.y += v.y;
            s.z += v.z;
            s.w += v.w;
        }
    }
    red[g][q] = s;
    __syncthreads();
    if (g == 0 && 4 * quad < cols) {
        float4 t = red[0][q];
#pragma unroll
        for (int gg = 1; gg < kGroups; ++gg) {
            const float4 u = red[gg][q];
            t.x += u.x;
            t.y += u.y;
            t.z += u.z;
            t.w += u.w;
        }
        *(float4 *)(out + (int64_t)blockIdx.y * cols + 4 * quad) = t;
    }
}

__global__ __launch_bounds__(256) void col_sum_final(const float *__restrict__ part,
                                                     float *__restrict__ out, int slices, int cols)
{
    const int c = blockIdx.x * 256 + threadIdx.x;
    if (c >= cols) return;
    float s = 0.0f;
    for (int k = 0; k < slices; ++k) s += part[(int64_t)k * cols + c];
    out[c] = s;
}

// Column sums of a rows x cols matrix (cols % 4 == 0) read through ld: one
// pass when it fits one 256-row slice, else slice partials in scratch and a
// second pass over them in slice order.
template <class LD>
int col_sum4(LD ld, float *out, int64_t rows, int64_t cols)
{
    const unsigned cblocks = (unsigned)((cols / 4 + kQuads - 1) / kQuads);
    const int64_t slices4 = (rows + kSliceRows - 1) / kSliceRows;
    if (slices4 > 65535) return record_error(EMBER_ERR_UNSUPPORTED, "col_sum");
    if (slices4 == 1) {
        hipLaunchKernelGGL((col_reduce4<LD>), dim3(cblocks, 1), dim3(256), 0, 0, ld, out, rows, (int)cols,
                           (int)rows);
        return launch_ok("col_reduce4") ? EMBER_OK : EMBER_ERR_DEVICE;
    }
    float *part4 = (float *)scratch(kScratchColSum, (size_t)slices4 * cols * sizeof(float));
    if (!part4) return EMBER_ERR_OUT_OF_MEMORY;
    hipLaunchKernelGGL((col_reduce4<LD>), dim3(cblocks, (unsigned)slices4), dim3(256), 0, 0, ld, part4, rows,
                       (int)cols, kSliceRows);
    if (!launch_ok("col_reduce4")) return EMBER_ERR_DEVICE;
    hipLaunchKernelGGL((col_reduce4<PlainRows>), dim3(cblocks, 1), dim3(256), 0, 0, PlainRows{part4}, out,
                       slices4, (int)cols, (int)slices4);
    return launch_ok("col_reduce4") ? EMBER_OK : EMBER_ERR_DEVICE;
}

}  // namespace
}  // namespace ember

extern "C" int gelu_bwd(const float *dy, const float *u, const float *y, float *dx, int64_t n)
{
    using namespace ember;
    if (n < 0) return record_error(EMBER_ERR_INVALID_ARGUMENT, "gelu_bwd");
    if (n == 0) return EMBER_OK;
    if (!dy || !u || !dx) return record_error(EMBER_ERR_INVALID_ARGUMENT, "gelu_bwd");
    const bool vec = n % 4 == 0 && (((uintptr_t)dy | (uintptr_t)u | (uintptr_t)y | (uintptr_t)dx) % 16) == 0;
    const int64_t work = vec ? n / 4 : n;
    // About 8 workgroups per CU, each thread a few elements (grid-stride).
    int64_t blocks = (work + 255) / 256;
    const int64_t cap = 8 * 256;
    if (blocks > cap) blocks = cap;
    if (vec) {
        if (y) hipLaunchKernelGGL(gelu_bwd_vec4<false>, dim3((unsigned)blocks), dim3(256), 0, 0, dy, u, y, dx, work);
        else hipLaunchKernelGGL(gelu_bwd_vec4<true>, dim3((unsigned)blocks), dim3(256), 0, 0, dy, u, y, dx, work);
    } else {
        if (y) hipLaunchKernelGGL(gelu_bwd_kernel<false>, dim3((unsigned)blocks), dim3(256), 0, 0, dy, u, y, dx, work);
        else hipLaunchKernelGGL(gelu_bwd_kernel<true>, dim3((unsigned)blocks), dim3(256), 0, 0, dy, u, y, dx, work);
    }
    return launch_ok("gelu_bwd") ? EMBER_OK : EMBER_ERR_DEVICE;
}

extern "C" int col_sum(const float *x, float *out, int64_t rows, int64_t cols)
{
    using namespace ember;
    if (rows < 0 || cols < 0 || cols > INT32_MAX) return record_error(EMBER_ERR_INVALID_ARGUMENT, "col_sum");
    if (cols == 0) return EMBER_OK;
    if (!out || (rows > 0 && !x)) return record_error(EMBER_ERR_INVALID_ARGUMENT, "col_sum");
    if (rows > 0 && cols % 4 == 0 && (((uintptr_t)x | (uintptr_t)out) % 16) == 0)
        return col_sum4(PlainRows{x}, out, rows, cols);
    const int64_t slices = (rows + kRowsPerSlice - 1) / kRowsPerSlice;
    if (slices > 65535) return record_error(EMBER_ERR_UNSUPPORTED, "col_sum");
    float *part = nullptr;
    if (slices > 0) {
        part = (float *)scratch(kScratchColSum, (size_t)slices * cols * sizeof(float));
        if (!part) return EMBER_ERR_OUT_OF_MEMORY;
        hipLaunchKernelGGL(col_sum_partial, dim3((unsigned)((cols + 255) / 256), (unsigned)slices),
                           dim3(256), 0, 0, x, part, rows, (int)cols);
        if (!launch_ok("col_sum_partial")) return EMBER_ERR_DEVICE;
    }
    hipLaunchKernelGGL(col_sum_final, dim3((unsigned)((cols + 255) / 256)), dim3(256), 0, 0,
                       (const float *)part, out, (int)slices, (int)cols);
    return launch_ok("col_sum_final") ? EMBER_OK : EMBER_ERR_DEVICE;
}

extern "C" int gelu_bwd_col_sum(const float *dy, const float *u, float *dx, float *dbias, int64_t rows,
                                int64_t cols)
{
    using namespace ember;
    if (rows < 0 || cols < 0 || cols > INT32_MAX || rows > INT64_MAX / (cols > 0 ? cols : 1))
        return record_error(EMBER_ERR_INVALID_ARGUMENT, "gelu_bwd_col_sum");
    if (cols == 0) return EMBER_OK;
    if (!dbias || (rows > 0 && (!dy || !u || !dx))) return record_error(EMBER_ERR_INVALID_ARGUMENT, "gelu_bwd_col_sum");
    // One pass (dx written while its columns are summed) for 16-byte aligned
    // rows; otherwise the two entry points in turn (the same results).
    if (rows > 0 && cols % 4 == 0 && (((uintptr_t)dy | (uintptr_t)u | (uintptr_t)dx | (uintptr_t)dbias) % 16) == 0)
        return col_sum4(GeluBwdRows{dy, u, dx}, dbias, rows, cols);
    const int st = gelu_bwd(dy, u, nullptr, dx, rows * cols);
    return st != EMBER_OK ? st : col_sum(dx, dbias, rows, cols);
}

// elementwise.hip -- the element-wise, transpose and reduction operators of
// Ember's native ABI on HIP.
//
// These are off the attention/GEMM hot path; they exist so that the library
// exports every symbol the reference's binding links against
// (src/tensor/operators.h:10-27, implemented for CUDA in
// src/tensor/operators_gpu.cu:33-219).  Differences from that file:
//  * broadcast ops pass shape and strides to the kernel by value instead of
//    three cudaMalloc + H2D copies + a device sync + three frees per call
//    (operators_gpu.cu:94-106);
//  * transpose goes through a 32 x 33 LDS tile so loads and stores are both
//    coalesced (operators_gpu.cu:138-151 stores with a stride of n);
//  * sum() reduces on the device in double and copies one float back,
//    instead of copying the whole tensor to the host (operators_gpu.cu:153-166).
// sum_axis / max_axis keep the reference's arithmetic exactly: each output is
// folded along the axis in index order with a float accumulator (sum from
// 0.0f, max from the first element with fmaxf).  Where the axis is the last
// one (inner == 1) the reference's one-thread-per-output loads are strided by
// the row length; here a wave owns 64 rows and stages 64-column chunks
// through LDS with row-contiguous loads before each lane folds its row.
#include <math.h>

#include "common.h"
#include "lds_dma.h"
#include "mfma.h"

namespace ember {
namespace {

constexpr int kBlock = 256;
constexpr int kMaxDims = 16;

inline int grid_for(int64_t n)
{
    int64_t g = (n + kBlock - 1) / kBlock;
    return (int)(g > 1048576 ? 1048576 : (g < 1 ? 1 : g));
}

struct BcastShape {
    int ndim;
    int shape[kMaxDims];
    int sa[kMaxDims];
    int sb[kMaxDims];
};

}  // namespace
}  // namespace ember

using ember::BcastShape;
using ember::grid_for;
using ember::kBlock;

#define EMBER_BINARY_OP(name, f)                                                              \
    __global__ void k_##name##_tensor(const float *a, const float *b, float *out, int size)   \
    {                                                                                         \
        for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < size;                         \
             i += gridDim.x * blockDim.x) {                                                   \
            const float x = a[i], y = b[i];                                                   \
            out[i] = (f);                                                                     \
        }                                                                                     \
    }                                                                                         \
    extern "C" void name##_tensor(const float *a, const float *b, float *out, int size)       \
    {                                                                                         \
        if (size <= 0) return;                                                                \
        hipLaunchKernelGGL(k_##name##_tensor, dim3(grid_for(size)), dim3(kBlock), 0, 0, a, b, \
                           out, size);                                                        \
        ember::launch_ok(#name "_tensor");                                                    \
    }

#define EMBER_SCALAR_OP(name, f)                                                               \
    __global__ void k_##name##_scalar(const float *a, float y, float *out, int size)           \
    {                                                                                          \
        for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < size;                          \
             i += gridDim.x * blockDim.x) {                                                    \
            const float x = a[i];                                                              \
            out[i] = (f);                                                                      \
        }                                                                                      \
    }                                                                                          \
    extern "C" void name##_scalar(const float *a, float b, float *out, int size)               \
    {                                                                                          \
        if (size <= 0) return;                                                                 \
        hipLaunchKernelGGL(k_##name##_scalar, dim3(grid_for(size)), dim3(kBlock), 0, 0, a, b,  \
                           out, size);                                                         \
        ember::launch_ok(#name "_scalar");                                                     \
    }

#define EMBER_UNARY_OP(name, f)                                                                \
    __global__ void k_##name##_tensor(const float *a, float *out, int size)                    \
    {                                                                                          \
        for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < size;                          \
             i += gridDim.x * blockDim.x) {                                                    \
            const float x = a[i];                                                              \
            out[i] = (f);                                                                      \
        }                                                                                      \
    }                                                                                          \
    extern "C" void name##_tensor(const float *a, float *out, int size)                        \
    {                                                                                          \
        if (size <= 0) return;                                                                 \
        hipLaunchKernelGGL(k_##name##_tensor, dim3(grid_for(size)), dim3(kBlock), 0, 0, a,     \
                           out, size);                                                         \
        ember::launch_ok(#name "_tensor");                                                     \
    }

#define EMBER_BROADCAST_OP(name, f)                                                             \
    __global__ void k_##name##_broadcasted(const float *a, const float *b, float *out,          \
                                           BcastShape s, int total)                             \
    {                                                                                           \
        for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < total;                          \
             i += gridDim.x * blockDim.x) {                                                     \
            int rem = i, ia = 0, ib = 0;                                                        \
            for (int d = s.ndim - 1; d >= 0; d--) {                                             \
                const int coord = rem % s.shape[d];                                             \
                rem /= s.shape[d];                                                              \
                ia += coord * s.sa[d];                                                          \
                ib += coord * s.sb[d];                                                          \
            }                                                                                   \
            const float x = a[ia], y = b[ib];                                                   \
            out[i] = (f);                                                                       \
        }                                                                                       \
    }                                                                                           \
    extern "C" void name##_broadcasted(const float *a, const float *b, float *out,              \
                                       const int *shape, const int *strides_a,                  \
                                       const int *strides_b, int ndim)                          \
    {                                                                                           \
        if (ndim < 0 || ndim > ember::kMaxDims) {                                               \
            ember::record_error(EMBER_ERR_UNSUPPORTED, #name "_broadcasted: ndim");             \
            return;                                                                             \
        }                                                                                       \
        BcastShape s;                                                                           \
        s.ndim = ndim;                                                                          \
        int total = 1;                                                                          \
        for (int d = 0; d < ndim; d++) {                                                        \
            s.shape[d] = shape[d];                                                              \
            s.sa[d] = strides_a[d];                                                             \
            s.sb[d] = strides_b[d];                                                             \
            total *= shape[d];                                                                  \
        }                                                                                       \
        if (total <= 0) return;                                                                 \
        hipLaunchKernelGGL(k_##name##_broadcasted, dim3(grid_for(total)), dim3(kBlock), 0, 0,   \
                           a, b, out, s, total);                                                \
        ember::launch_ok(#name "_broadcasted");                                                 \
    }

#include "operators.def"

namespace {

__global__ void k_transpose(const float *a, float *out, int n, int m)
{
    __shared__ float tile[32][33];
    const int bx = blockIdx.x * 32, by = blockIdx.y * 32;
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // 32 x 8 threads
    for (int r = ty; r < 32; r += 8) {
        const int i = by + r, j = bx + tx;
        if (i < n && j < m) tile[r][tx] = a[(int64_t)i * m + j];
    }
    __syncthreads();
    for (int r = ty; r < 32; r += 8) {
        const int j = bx + r, i = by + tx;  // out[j][i]
        if (i < n && j < m) out[(int64_t)j * n + i] = tile[tx][r];
    }
}

__global__ void k_sum_partial(const float *a, int size, double *partial)
{
    __shared__ double red[kBlock];
    double s = 0.0;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < size; i += gridDim.x * blockDim.x)
        s += (double)a[i];
    red[threadIdx.x] = s;
    __syncthreads();
    for (int off = kBlock / 2; off > 0; off >>= 1) {
        if ((int)threadIdx.x < off) red[threadIdx.x] += red[threadIdx.x + off];
        __syncthreads();
    }
    if (threadIdx.x == 0) partial[blockIdx.x] = red[0];
}

// The MSE loss in one pass: d = p - t; grad = d * scale; partial sums of
// d*d exactly as k_sum_partial forms them over the product tensor (same
// grid, same strided walk, same tree), so the loss equals
// sum(diff * diff) and grad equals scale * diff bit for bit.
__global__ void k_mse_partial(const float *p, const float *t, float *grad, float scale, int size,
                              double *partial)
{
#pragma clang fp contract(off)
    __shared__ double red[kBlock];
    double s = 0.0;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < size; i += gridDim.x * blockDim.x) {
        const float d = p[i] - t[i];
        grad[i] = d * scale;
        const float sq = d * d;
        s += (double)sq;
    }
    red[threadIdx.x] = s;
    __syncthreads();
    for (int off = kBlock / 2; off > 0; off >>= 1) {
        if ((int)threadIdx.x < off) red[threadIdx.x] += red[threadIdx.x + off];
        __syncthreads();
    }
    if (threadIdx.x == 0) partial[blockIdx.x] = red[0];
}

__global__ void k_sum_final(const double *partial, int n, float *out)
{
    __shared__ double red[kBlock];
    double s = 0.0;
    for (int i = threadIdx.x; i < n; i += blockDim.x) s += partial[i];
    red[threadIdx.x] = s;
    __syncthreads();
    for (int off = kBlock / 2; off > 0; off >>= 1) {
        if ((int)threadIdx.x < off) red[threadIdx.x] += red[threadIdx.x + off];
        __syncthreads();
    }
    if (threadIdx.x == 0) *out = (float)red[0];
}

__global__ void k_sum_axis(const float *a, float *out, int outer, int inner, int axis_dim)
{
    const int total = outer * inner;
    for (int idx = blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += gridDim.x * blockDim.x) {
        const int o = idx / inner, i = idx - o * inner;
        const float *p = a + (int64_t)o * axis_dim * inner + i;
        float s = 0.0f;
        for (int r = 0; r < axis_dim; r++) s += p[(int64_t)r * inner];
        out[idx] = s;
    }
}

__global__ void k_max_axis(const float *a, float *out, int outer, int inner, int axis_dim)
{
    const int total = outer * inner;
    for (int idx = blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += gridDim.x * blockDim.x) {
        const int o = idx / inner, i = idx - o * inner;
        const float *p = a + (int64_t)o * axis_dim * inner + i;
        float mx = p[0];
        for (int r = 1; r < axis_dim; r++) mx = fmaxf(mx, p[(int64_t)r * inner]);
        out[idx] = mx;
    }
}

// Last-axis reduction of up to 64 rows per wave (see the file comment).
template <bool MAX>
__global__ __launch_bounds__(64) void k_reduce_rows(const float *a, float *out, int rows, int L)
{
    __shared__ float tile[64 * 65];
    const int lane = threadIdx.x;
    const int r0 = blockIdx.x * 64;
    const int nr = min(64, rows - r0);
    float acc = 0.0f;
    for (int c0 = 0; c0 < L; c0 += 64) {
        const int c = c0 + lane;
        if (c < L) {
#pragma unroll 16
            for (int r = 0; r < nr; ++r) tile[r * 65 + lane] = a[(int64_t)(r0 + r) * L + c];
        }
        __syncthreads();
        if (lane < nr) {
            const int nc = min(64, L - c0);
            const float *t = tile + lane * 65;
            int j = 0;
            if (MAX && c0 == 0) acc = t[j++];
            for (; j < nc; ++j) acc = MAX ? fmaxf(acc, t[j]) : acc + t[j];
        }
        __syncthreads();
    }
    if (lane < nr) out[r0 + lane] = acc;
}

// The same fold with the loads pipelined (L % 4 == 0, L < 2^24, a 16-byte
// aligned): a one-wave workgroup owns 64 rows; each 64-column chunk is copied
// HBM -> LDS by direct 16-byte copies (buffer form: the chunk's base in a
// scalar descriptor, a fixed 32-bit byte offset per lane and copy) into rows
// padded to 68 floats, kRing chunks in flight (17 copies each; vmcnt counts
// at most 63).  A piece past the row (the 17th) or past the matrix re-reads
// the chunk's first piece: valid memory, never folded.  Lane r folds row r in
// index order from 128-bit LDS reads (conflict-free: 8 consecutive rows start
// 16 bytes apart in the 128-byte bank cycle), all 16 reads of a chunk before
// its adds.  One wave, so no barriers: a chunk is consumed after this wave's
// own vmcnt wait and refilled after its fold has read it.
constexpr int kRowStr = 68;                 // floats per padded tile row
constexpr int kTileCopies = 64 * 17 / 64;   // 1 KiB copies per 64 x 64 tile
constexpr int kRing = 4;                    // chunks in flight

template <bool MAX>
__global__ __launch_bounds__(64) void k_reduce_rows_ring(const float *a, float *out, int rows, int L)
{
    using ember::f32x4;
    __shared__ float tile[kRing * 64 * kRowStr];
    const int lane = threadIdx.x;
    const int r0 = blockIdx.x * 64;
    const int nr = min(64, rows - r0);
    const int nchunk = (L + 63) / 64;
    const float *row0 = a + (int64_t)r0 * L;
    // Byte offset of this lane's piece in copy t of a chunk whose columns
    // from cend on lie past the row (0: the chunk's first piece).
    auto offset = [&](int t, int ln, int cend) {
        const int p = 64 * t + ln;
        const int r = p / 17, q = p - 17 * r;
        return q < 16 && r < nr && 4 * q < cend ? 4u * (unsigned)(r * L + 4 * q) : 0u;
    };
    unsigned off[kTileCopies];
#pragma unroll
    for (int t = 0; t < kTileCopies; ++t) off[t] = offset(t, lane, 64);
    auto issue = [&](int ch) {
        float *dst = tile + (ch % kRing) * 64 * kRowStr;
        const __amdgpu_buffer_rsrc_t rs = ember::dma_rsrc(row0 + 64 * ch);
        const int cend = L - 64 * ch;
        if (cend >= 64) {
#pragma unroll
            for (int t = 0; t < kTileCopies; ++t) ember::dma16_buf(rs, off[t], dst + 256 * t);
        } else {
            int ln = lane;
            asm volatile("" : "+v"(ln));  // the tail's offsets: recomputed, not kept live
#pragma unroll
            for (int t = 0; t < kTileCopies; ++t) ember::dma16_buf(rs, offset(t, ln, cend), dst + 256 * t);
        }
    };
    for (int ch = 0; ch < min(kRing, nchunk); ++ch) issue(ch);
    float acc = 0.0f;
    for (int ch = 0; ch < nchunk; ++ch) {
        // Chunks ch + 1 .. issued after this one may stay in flight.
        switch (min(kRing - 1, nchunk - 1 - ch)) {
            case 3: ember::wait_vmem_n<3 * kTileCopies>(); break;
            case 2: ember::wait_vmem_n<2 * kTileCopies>(); break;
            case 1: ember::wait_vmem_n<kTileCopies>(); break;
            default: ember::wait_vmem(); break;
        }
        if (lane < nr) {
            const float *t = tile + (ch % kRing) * 64 * kRowStr + lane * kRowStr;
            const int nc = min(64, L - 64 * ch);
            if (nc == 64) {
                f32x4 v[16];
#pragma unroll
                for (int q = 0; q < 16; ++q) v[q] = *(const f32x4 *)(t + 4 * q);
#pragma unroll
                for (int q = 0; q < 16; ++q)
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        if (MAX)
                            acc = (ch == 0 && q == 0 && j == 0) ? v[q][j] : fmaxf(acc, v[q][j]);
                        else
                            acc += v[q][j];
                    }
            } else {
                for (int j0 = 0; j0 < nc; j0 += 4) {
                    const f32x4 v = *(const f32x4 *)(t + j0);
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        if (j0 + j < nc) {
                            if (MAX)
                                acc = (ch == 0 && j0 + j == 0) ? v[j] : fmaxf(acc, v[j]);
                            else
                                acc += v[j];
                        }
                    }
                }
            }
        }
        if (ch + kRing < nchunk) issue(ch + kRing);
    }
    if (lane < nr) out[r0 + lane] = acc;
}

}  // namespace

extern "C" {

void transpose(const float *a, float *out, int n, int m)
{
    if (n <= 0 || m <= 0) return;
    hipLaunchKernelGGL(k_transpose, dim3((m + 31) / 32, (n + 31) / 32), dim3(256), 0, 0, a, out, n,
                       m);
    ember::launch_ok("transpose");
}

float sum(const float *a, int size)
{
    if (size <= 0) return 0.0f;
    const int nblk = grid_for(size) > 1024 ? 1024 : grid_for(size);
    char *ws = (char *)ember::scratch(ember::kScratchSum, (size_t)nblk * sizeof(double) + 16);
    if (!ws) return 0.0f;
    double *partial = (double *)ws;
    float *res = (float *)(ws + (size_t)nblk * sizeof(double));
    hipLaunchKernelGGL(k_sum_partial, dim3(nblk), dim3(kBlock), 0, 0, a, size, partial);
    hipLaunchKernelGGL(k_sum_final, dim3(1), dim3(kBlock), 0, 0, partial, nblk, res);
    if (!ember::launch_ok("sum")) return 0.0f;
    float host = 0.0f;
    ember::hip_ok(hipMemcpy(&host, res, sizeof(float), hipMemcpyDeviceToHost), "sum");
    return host;
}

int mse_loss(const float *pred, const float *target, float *grad, int size, float scale, float *loss)
{
    if (size < 0 || !loss) return ember::record_error(EMBER_ERR_INVALID_ARGUMENT, "mse_loss");
    *loss = 0.0f;
    if (size == 0) return EMBER_OK;
    if (!pred || !target || !grad) return ember::record_error(EMBER_ERR_INVALID_ARGUMENT, "mse_loss");
    const int nblk = grid_for(size) > 1024 ? 1024 : grid_for(size);  // as in sum()
    char *ws = (char *)ember::scratch(ember::kScratchSum, (size_t)nblk * sizeof(double) + 16);
    if (!ws) return EMBER_ERR_OUT_OF_MEMORY;
    double *partial = (double *)ws;
    float *res = (float *)(ws + (size_t)nblk * sizeof(double));
    hipLaunchKernelGGL(k_mse_partial, dim3(nblk), dim3(kBlock), 0, 0, pred, target, grad, scale, size, partial);
    hipLaunchKernelGGL(k_sum_final, dim3(1), dim3(kBlock), 0, 0, partial, nblk, res);
    if (!ember::launch_ok("mse_loss")) return EMBER_ERR_DEVICE;
    if (!ember::hip_ok(hipMemcpy(loss, res, sizeof(float), hipMemcpyDeviceToHost), "mse_loss"))
        return EMBER_ERR_DEVICE;
    return EMBER_OK;
}

int sum_axis_product(const int *shape, int start, int end)
{
    int p = 1;
    for (int i = start; i < end; i++) p *= shape[i];
    return p;
}

void sum_axis(const float *a, float *out, int outer_stride, int inner_stride, int axis_dim)
{
    const int total = outer_stride * inner_stride;
    if (total <= 0) return;
    if (inner_stride == 1 && axis_dim > 1) {
        if (axis_dim % 4 == 0 && axis_dim < (1 << 24) && ((uintptr_t)a & 15) == 0)
            hipLaunchKernelGGL(k_reduce_rows_ring<false>, dim3((outer_stride + 63) / 64), dim3(64), 0, 0, a,
                               out, outer_stride, axis_dim);
        else
            hipLaunchKernelGGL(k_reduce_rows<false>, dim3((outer_stride + 63) / 64), dim3(64), 0, 0, a,
                               out, outer_stride, axis_dim);
        ember::launch_ok("sum_axis");
        return;
    }
    hipLaunchKernelGGL(k_sum_axis, dim3(grid_for(total)), dim3(kBlock), 0, 0, a, out, outer_stride,
                       inner_stride, axis_dim);
    ember::launch_ok("sum_axis");
}

void max_axis(const float *a, float *out, int outer_stride, int inner_stride, int axis_dim)
{
    const int total = outer_stride * inner_stride;
    if (total <= 0 || axis_dim <= 0) return;
    if (inner_stride == 1 && axis_dim > 1) {
        if (axis_dim % 4 == 0 && axis_dim < (1 << 24) && ((uintptr_t)a & 15) == 0)
            hipLaunchKernelGGL(k_reduce_rows_ring<true>, dim3((outer_stride + 63) / 64), dim3(64), 0, 0, a,
                               out, outer_stride, axis_dim);
        else
            hipLaunchKernelGGL(k_reduce_rows<true>, dim3((outer_stride + 63) / 64), dim3(64), 0, 0, a,
                               out, outer_stride, axis_dim);
        ember::launch_ok("max_axis");
        return;
    }
    hipLaunchKernelGGL(k_max_axis, dim3(grid_for(total)), dim3(kBlock), 0, 0, a, out, outer_stride,
                       inner_stride, axis_dim);
    ember::launch_ok("max_axis");
}

}  // extern "C"

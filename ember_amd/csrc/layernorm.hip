// layernorm.hip -- LayerNorm forward / backward over the last dimension.
//
// No reference counterpart: Ember has no LayerNorm (a pre-LN decoder
// block built from Ember ops composes it from sum_axis / broadcast / sqrt).  The
// semantics are those of oracle/ember_oracle.c (oracle_layernorm_*):
//   mean = sum(x)/d;  var = sum((x - mean)^2)/d  (biased);
//   rstd = 1/sqrt(var + eps);  y = (x - mean)*rstd*gamma + beta
//   backward (xhat = (x - mean)*rstd, g = dy*gamma):
//   dx = rstd*(g - mean(g) - xhat*mean(g*xhat))  (+ dres, the gradient that
//        reaches x through a residual connection, when given);
//   dgamma = sum_rows(dy*xhat);  dbeta = sum_rows(dy)
//
// HBM-bound.  One wave per row; a row is held in registers (d <= 4096, a
// multiple of 4) as 16-byte chunks, 64 lanes wide, so x is read once; the
// row reductions are wave shuffles.  dgamma / dbeta: each workgroup (8 rows,
// so that ~1000 workgroups keep the loads in flight) sums its rows'
// contributions per column in registers and writes one partial row; a second
// launch adds the partials in a fixed tree order (16 interleaved runs per
// column, then the runs in order: deterministic, no atomics).  The partials
// live in library scratch.
#include <math.h>

#include "common.h"

namespace ember {
namespace {

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kMaxChunks = 16;  // 16-byte chunks per lane: d <= 64*4*16 = 4096

__device__ __forceinline__ float wave_sum(float v)
{
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
    return v;
}

template <int NC>
__global__ __launch_bounds__(kThreads) void ln_fwd_kernel(const float *__restrict__ x,
                                                         const float *__restrict__ gamma,
                                                         const float *__restrict__ beta,
                                                         float *__restrict__ y, float *mean_out,
                                                         float *rstd_out, int64_t rows, int d,
                                                         float eps)
{
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6);
    if (row >= rows) return;  // whole waves retire together
    const float *xr = x + row * d;
    float4 v[NC];
    float s = 0.0f;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const int col = 4 * (64 * c + lane);
        v[c] = col < d ? *(const float4 *)(xr + col) : make_float4(0.f, 0.f, 0.f, 0.f);
        s += (v[c].x + v[c].y) + (v[c].z + v[c].w);
    }
    const float mean = wave_sum(s) / (float)d;
    float q = 0.0f;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const int col = 4 * (64 * c + lane);
        if (col < d) {
            const float a = v[c].x - mean, b = v[c].y - mean, e = v[c].z - mean, f = v[c].w - mean;
            q += (a * a + b * b) + (e * e + f * f);
        }
    }
    const float rstd = 1.0f / sqrtf(wave_sum(q) / (float)d + eps);
    float *yr = y + row * d;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const int col = 4 * (64 * c + lane);
        if (col < d) {
            const float4 g = *(const float4 *)(gamma + col);
            const float4 b = *(const float4 *)(beta + col);
            float4 o;
            o.x = (v[c].x - mean) * rstd * g.x + b.x;
            o.y = (v[c].y - mean) * rstd * g.y + b.y;
            o.z = (v[c].z - mean) * rstd * g.z + b.z;
            o.w = (v[c].w - mean) * rstd * g.w + b.w;
            *(float4 *)(yr + col) = o;
        }
    }
    if (lane == 0) {
        mean_out[row] = mean;
        rstd_out[row] = rstd;
    }
}

// dx per row; per-workgroup partial column sums of dy*xhat and dy.
template <int NC>
__global__ __launch_bounds__(kThreads) void ln_bwd_kernel(const float *__restrict__ x,
                                                         const float *__restrict__ gamma,
                                                         const float *__restrict__ mean_in,
                                                         const float *__restrict__ rstd_in,
                                                         const float *__restrict__ dy,
                                                         const float *__restrict__ dres,
                                                         float *__restrict__ dx,
                                                         float *__restrict__ part, int64_t rows,
                                                         int d, int rows_per_block)
{
    const int lane = threadIdx.x & 63;
    const int w = threadIdx.x >> 6;
    float4 pg[NC], pb[NC];  // this wave's partial dgamma / dbeta per chunk
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        pg[c] = make_float4(0.f, 0.f, 0.f, 0.f);
        pb[c] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
    const int64_t r0 = (int64_t)blockIdx.x * rows_per_block;
    for (int64_t row = r0 + w; row < r0 + rows_per_block && row < rows; row += kWaves) {
        const float mean = mean_in[row], rstd = rstd_in[row];
        float4 xh[NC], gg[NC];
        float s1 = 0.0f, s2 = 0.0f;
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            const int col = 4 * (64 * c + lane);
            if (col < d) {
                const float4 xv = *(const float4 *)(x + row * d + col);
                const float4 gv = *(const float4 *)(dy + row * d + col);
                const float4 ga = *(const float4 *)(gamma + col);
                xh[c] = make_float4((xv.x - mean) * rstd, (xv.y - mean) * rstd,
                                    (xv.z - mean) * rstd, (xv.w - mean) * rstd);
                gg[c] = make_float4(gv.x * ga.x, gv.y * ga.y, gv.z * ga.z, gv.w * ga.w);
                s1 += (gg[c].x + gg[c].y) + (gg[c].z + gg[c].w);
                s2 += (gg[c].x * xh[c].x + gg[c].y * xh[c].y) + (gg[c].z * xh[c].z + gg[c].w * xh[c].w);
                pg[c].x += gv.x * xh[c].x;
                pg[c].y += gv.y * xh[c].y;
                pg[c].z += gv.z * xh[c].z;
                pg[c].w += gv.w * xh[c].w;
                pb[c].x += gv.x;
                pb[c].y += gv.y;
                pb[c].z += gv.z;
                pb[c].w += gv.w;
            }
        }
        const float m1 = wave_sum(s1) / (float)d;
        const float m2 = wave_sum(s2) / (float)d;
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            const int col = 4 * (64 * c + lane);
            if (col < d) {
                float4 o;
                o.x = rstd * (gg[c].x - m1 - xh[c].x * m2);
                o.y = rstd * (gg[c].y - m1 - xh[c].y * m2);
                o.z = rstd * (gg[c].z - m1 - xh[c].z * m2);
                o.w = rstd * (gg[c].w - m1 - xh[c].w * m2);
                if (dres) {
                    const float4 r = *(const float4 *)(dres + row * d + col);
                    o.x += r.x;
                    o.y += r.y;
                    o.z += r.z;
                    o.w += r.w;
                }
                *(float4 *)(dx + row * d + col) = o;
            }
        }
    }
    // Sum the 4 waves' partials through LDS, in wave order, and write this
    // workgroup's row of partials: part[block][0..d) = dgamma, [d..2d) = dbeta.
    __shared__ float red[kWaves][4 * 64];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const int col = 4 * (64 * c + lane);
#pragma unroll
        for (int which = 0; which < 2; ++which) {
            const float4 mine = which ? pb[c] : pg[c];
            __syncthreads();
            *(float4 *)&red[w][4 * lane] = mine;
            __syncthreads();
            if (w == 0 && col < d) {
                float4 t = *(const float4 *)&red[0][4 * lane];
#pragma unroll
                for (int ww = 1; ww < kWaves; ++ww) {
                    const float4 u = *(const float4 *)&red[ww][4 * lane];
                    t.x += u.x;
                    t.y += u.y;
                    t.z += u.z;
                    t.w += u.w;
                }
                *(float4 *)(part + ((int64_t)blockIdx.x * 2 + which) * d + col) = t;
            }
        }
    }
}

// dgamma[c] = sum_b part[b][0][c], dbeta[c] = sum_b part[b][1][c]: a
// workgroup owns 16 quads of the 2d output columns; thread group g (of 16)
// sums partial rows b = g, g+16, ... in order (float4), then the 16 group
// sums are added in g order.
constexpr int kPgQuads = 16, kPgGroups = 16;
__global__ __launch_bounds__(256) void ln_param_grad_kernel(const float *__restrict__ part,
                                                            float *__restrict__ dgamma,
                                                            float *__restrict__ dbeta, int nblk,
                                                            int d)
{
    __shared__ float4 red[kPgGroups][kPgQuads];
    const int q = threadIdx.x % kPgQuads, g = threadIdx.x / kPgQuads;
    const int quad = blockIdx.x * kPgQuads + q;  // over 2d/4 column quads
    const int nq = 2 * d / 4;
    float4 s = make_float4(0.f, 0.f, 0.f, 0.f);
    if (quad < nq) {
        const int which = (4 * quad) / d, col = 4 * quad - which * d;
        const float *src = part + (int64_t)which * d + col;
        const int64_t step = (int64_t)kPgGroups * 2 * d;  // floats between a thread's rows
        int b = g;
        // Eight loads in flight, then the adds in row order (the same sums
        // as one row at a time).
        for (; b + 7 * kPgGroups < nblk; b += 8 * kPgGroups) {
            float4 v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) v[u] = *(const float4 *)(src + (int64_t)b * 2 * d + u * step);
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                s.x += v[u].x;
                s.y += v[u].y;
                s.z += v[u].z;
                s.w += v[u].w;
            }
        }
        for (; b < nblk; b += kPgGroups) {
            const float4 v = *(const float4 *)(src + (int64_t)b * 2 * d);
            s.x += v.x;
            s.y += v.y;
            s.z += v.z;
            s.w += v.w;
        }
    }
    red[g][q] = s;
    __syncthreads();
    if (g == 0 && quad < nq) {
        float4 t = red[0][q];
#pragma unroll
        for (int gg = 1; gg < kPgGroups; ++gg) {
            const float4 u = red[gg][q];
            t.x += u.x;
            t.y += u.y;
            t.z += u.z;
            t.w += u.w;
        }
        const int which = (4 * quad) / d, col = 4 * quad - which * d;
        *(float4 *)((which ? dbeta : dgamma) + col) = t;
    }
}

// Status of the argument checks (pointers are checked even for rows == 0).
int ln_args(const void *const *ptrs, int n, int64_t rows, int64_t d, const char *who)
{
    if (rows < 0 || d <= 0 || d % 4)
        return record_error(EMBER_ERR_INVALID_ARGUMENT, who);
    if (d > 64 * 4 * kMaxChunks) return record_error(EMBER_ERR_UNSUPPORTED, who);
    for (int i = 0; i < n; ++i)
        if (!ptrs[i] || ((uintptr_t)ptrs[i] & 15)) return record_error(EMBER_ERR_INVALID_ARGUMENT, who);
    return EMBER_OK;
}

template <int NC>
void launch_fwd(const float *x, const float *g, const float *b, float *y, float *mean, float *rstd,
                int64_t rows, int d, float eps)
{
    const int64_t blocks = (rows + kWaves - 1) / kWaves;
    hipLaunchKernelGGL(ln_fwd_kernel<NC>, dim3((unsigned)blocks), dim3(kThreads), 0, 0, x, g, b, y,
                       mean, rstd, rows, d, eps);
}

template <int NC>
void launch_bwd(const float *x, const float *g, const float *mean, const float *rstd,
                const float *dy, const float *dres, float *dx, float *part, int64_t rows, int d,
                int rpb, int nblk)
{
    hipLaunchKernelGGL(ln_bwd_kernel<NC>, dim3(nblk), dim3(kThreads), 0, 0, x, g, mean, rstd, dy,
                       dres, dx, part, rows, d, rpb);
}

}  // namespace
}  // namespace ember

extern "C" int layernorm_fwd(const float *x, const float *gamma, const float *beta, float *y,
                             float *mean, float *rstd, int64_t rows, int64_t d, float eps)
{
    using namespace ember;
    const void *ptrs[] = {x, gamma, beta, y, mean, rstd};
    const int st = ln_args(ptrs, 6, rows, d, "layernorm_fwd");
    if (st != EMBER_OK) return st;
    if (!(eps >= 0.0f) || isinf(eps)) return record_error(EMBER_ERR_INVALID_ARGUMENT, "layernorm_fwd");
    if (rows == 0) return EMBER_OK;
    const int nc = (int)((d + 255) / 256);
    if (nc <= 4)
        launch_fwd<4>(x, gamma, beta, y, mean, rstd, rows, (int)d, eps);
    else if (nc <= 8)
        launch_fwd<8>(x, gamma, beta, y, mean, rstd, rows, (int)d, eps);
    else
        launch_fwd<16>(x, gamma, beta, y, mean, rstd, rows, (int)d, eps);
    return launch_ok("ln_fwd_kernel") ? EMBER_OK : EMBER_ERR_DEVICE;
}

extern "C" int layernorm_bwd(const float *x, const float *gamma, const float *mean,
                             const float *rstd, const float *dy, const float *dres, float *dx,
                             float *dgamma, float *dbeta, int64_t rows, int64_t d)
{
    using namespace ember;
    const void *ptrs[] = {x, gamma, mean, rstd, dy, dx, dgamma, dbeta};
    const int st = ln_args(ptrs, 8, rows, d, "layernorm_bwd");
    if (st != EMBER_OK) return st;
    if ((uintptr_t)dres & 15) return record_error(EMBER_ERR_INVALID_ARGUMENT, "layernorm_bwd");
    const unsigned pg_blocks = (unsigned)((2 * d / 4 + kPgQuads - 1) / kPgQuads);
    if (rows == 0) {
        // Sums over no rows: the reduction kernel over zero partials writes 0.
        hipLaunchKernelGGL(ln_param_grad_kernel, dim3(pg_blocks), dim3(256), 0, 0,
                           (const float *)nullptr, dgamma, dbeta, 0, (int)d);
        return launch_ok("ln_param_grad_kernel") ? EMBER_OK : EMBER_ERR_DEVICE;
    }
    // Workgroups of 8 rows (2 per wave), each owning a contiguous run; rows
    // beyond 2^18 take longer runs so the partials stay under 2^15 rows.
    const int64_t rpb64 = (rows + 32767) / 32768;
    const int rpb = (int)(rpb64 < 2 * kWaves ? 2 * kWaves : rpb64);
    const int nblk = (int)((rows + rpb - 1) / rpb);
    float *part = (float *)scratch(kScratchLayerNorm, (size_t)nblk * 2 * d * sizeof(float));
    if (!part) return EMBER_ERR_OUT_OF_MEMORY;
    const int nc = (int)((d + 255) / 256);
    if (nc <= 4)
        launch_bwd<4>(x, gamma, mean, rstd, dy, dres, dx, part, rows, (int)d, rpb, nblk);
    else if (nc <= 8)
        launch_bwd<8>(x, gamma, mean, rstd, dy, dres, dx, part, rows, (int)d, rpb, nblk);
    else
        launch_bwd<16>(x, gamma, mean, rstd, dy, dres, dx, part, rows, (int)d, rpb, nblk);
    if (!launch_ok("ln_bwd_kernel")) return EMBER_ERR_DEVICE;
    hipLaunchKernelGGL(ln_param_grad_kernel, dim3(pg_blocks), dim3(256), 0, 0, part, dgamma, dbeta,
                       nblk, (int)d);
    return launch_ok("ln_param_grad_kernel") ? EMBER_OK : EMBER_ERR_DEVICE;
}

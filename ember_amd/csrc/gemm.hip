// gemm.hip -- fp32 GEMM on gfx950 matrix cores behind Ember's matmul ABI.
//
// Replaces the reference's cuBLAS calls (src/tensor/operators_gpu.cu:114-136):
//   matmul(a, b, out, n, m, k):          out(n x m) = a(n x k) @ b(k x m)
//   matmul_batched(..., batch, n, m, k): the same per batch with strides
//                                        n*k, k*m, n*m
// all row-major fp32 with fp32 accumulation (v_mfma_f32_32x32x2f32; no
// reduced-precision inputs).  The CPU path of the reference accumulates in
// double (src/tensor/operators_cpu.c:47-60); agreement is to fp32 rounding
// of a length-k sum, see the parity tests.
//
// Tiling: a workgroup of 4 waves computes a 128 x 128 block of out, each
// wave a 64 x 64 quadrant as 2 x 2 MFMA accumulators.  The k dimension is
// walked in 32-wide slabs: the next slab's A (128 x 32) and B (32 x 128)
// are loaded from HBM/L2 into registers while the current one is multiplied
// out of LDS (two LDS buffers, one barrier per slab).  Lane half h of a wave
// contracts k in [16h, 16h+16) of the slab, so A is read from LDS as
// 128-bit row segments; B rows of the second half sit 32 floats further on
// so the two lane halves read disjoint banks.  Workgroups are ordered so
// that consecutive ones share B column panels in L2.
#include "common.h"
#include "mfma.h"

namespace ember {
namespace {

constexpr int kThreads = 256;
constexpr int BM = 128, BN = 128, BK = 32;
constexpr int ASTR = BK + 4;  // padded A row in LDS
constexpr int BBUF = BK * BN + 32;

struct GemmArgs {
    const float *a, *b;
    float *c;
    int n, m, k;
    int64_t sa, sb, sc;  // batch strides (elements)
    int tiles_n, tiles_m;
};

__device__ __forceinline__ int bs_index(int kr, int col)
{
    return kr * BN + (kr >= BK / 2 ? 32 : 0) + col;
}

// Loads one slab into registers: A rows row0.., cols k0..k0+31; B rows k0..,
// cols col0..col0+127.  Out-of-range elements read as 0.
template <bool VEC>
__device__ __forceinline__ void load_slab(const GemmArgs &g, const float *A, const float *B, int row0,
                                          int col0, int k0, int tid, f32x4 (&ra)[4], f32x4 (&rb)[4])
{
#pragma unroll
    for (int it = 0; it < 4; ++it) {
        const int idx = it * kThreads + tid;  // 0..1023
        {   // A: 128 rows x 8 float4
            const int r = idx >> 3, c4 = idx & 7;
            const int row = row0 + r, col = k0 + 4 * c4;
            f32x4 v = {0.f, 0.f, 0.f, 0.f};
            if (VEC) {
                if (row < g.n && col < g.k) v = *(const f32x4 *)(A + (int64_t)row * g.k + col);
            } else if (row < g.n) {
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    if (col + j < g.k) v[j] = A[(int64_t)row * g.k + col + j];
            }
            ra[it] = v;
        }
        {   // B: 32 rows x 32 float4
            const int r = idx >> 5, c4 = idx & 31;
            const int row = k0 + r, col = col0 + 4 * c4;
            f32x4 v = {0.f, 0.f, 0.f, 0.f};
            if (VEC) {
                if (row < g.k && col < g.m) v = *(const f32x4 *)(B + (int64_t)row * g.m + col);
            } else if (row < g.k) {
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    if (col + j < g.m) v[j] = B[(int64_t)row * g.m + col + j];
            }
            rb[it] = v;
        }
    }
}

__device__ __forceinline__ void store_slab(float *As, float *Bs, int tid, const f32x4 (&ra)[4],
                                           const f32x4 (&rb)[4])
{
#pragma unroll
    for (int it = 0; it < 4; ++it) {
        const int idx = it * kThreads + tid;
        {
            const int r = idx >> 3, c4 = idx & 7;
            *(f32x4 *)&As[r * ASTR + 4 * c4] = ra[it];
        }
        {
            const int r = idx >> 5, c4 = idx & 31;
            *(f32x4 *)&Bs[bs_index(r, 4 * c4)] = rb[it];
        }
    }
}

template <bool VEC>
__global__ __launch_bounds__(kThreads, 2) void gemm_f32_kernel(GemmArgs g)
{
    __shared__ float As[2][BM * ASTR];
    __shared__ float Bs[2][BBUF];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int w = tid >> 6;
    const int h32 = lane >> 5;
    const int l32 = lane & 31;
    const int wr = w >> 1, wc = w & 1;

    // Column panels vary slowest within a group of 8 row tiles so that
    // neighbouring workgroups reuse the same B panel from L2.
    const int tile = blockIdx.x;
    constexpr int GROUP = 8;
    const int per_group = GROUP * g.tiles_m;
    const int grp = tile / per_group;
    const int first_row_tile = grp * GROUP;
    const int rows_in_grp = min(GROUP, g.tiles_n - first_row_tile);
    const int in_grp = tile - grp * per_group;
    const int tn = first_row_tile + in_grp % rows_in_grp;
    const int tm = in_grp / rows_in_grp;

    const int row0 = tn * BM;
    const int col0 = tm * BN;
    const float *A = g.a + (int64_t)blockIdx.y * g.sa;
    const float *B = g.b + (int64_t)blockIdx.y * g.sb;
    float *C = g.c + (int64_t)blockIdx.y * g.sc;

    f32x16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = zero16();

    f32x4 ra[4], rb[4];
    const int nslab = (g.k + BK - 1) / BK;
    load_slab<VEC>(g, A, B, row0, col0, 0, tid, ra, rb);
    store_slab(As[0], Bs[0], tid, ra, rb);
    __syncthreads();

    for (int s = 0; s < nslab; ++s) {
        const int cur = s & 1;
        if (s + 1 < nslab) load_slab<VEC>(g, A, B, row0, col0, (s + 1) * BK, tid, ra, rb);
        const float *as = As[cur];
        const float *bs = Bs[cur];
#pragma unroll
        for (int kk = 0; kk < BK / 2; kk += 4) {
            f32x4 af[2];
#pragma unroll
            for (int rb2 = 0; rb2 < 2; ++rb2)
                af[rb2] = *(const f32x4 *)&as[(64 * wr + 32 * rb2 + l32) * ASTR + h32 * (BK / 2) + kk];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int kr = h32 * (BK / 2) + kk + j;
                float bf[2];
#pragma unroll
                for (int cb = 0; cb < 2; ++cb) bf[cb] = bs[bs_index(kr, 64 * wc + 32 * cb + l32)];
#pragma unroll
                for (int rb2 = 0; rb2 < 2; ++rb2)
#pragma unroll
                    for (int cb = 0; cb < 2; ++cb)
                        acc[rb2][cb] = mfma_32x32x2(af[rb2][j], bf[cb], acc[rb2][cb]);
            }
        }
        if (s + 1 < nslab) store_slab(As[cur ^ 1], Bs[cur ^ 1], tid, ra, rb);
        __syncthreads();
    }

#pragma unroll
    for (int rb2 = 0; rb2 < 2; ++rb2) {
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) {
            const int col = col0 + 64 * wc + 32 * cb + l32;
            if (col >= g.m) continue;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int row = row0 + 64 * wr + 32 * rb2 + acc_row(i, h32);
                if (row < g.n) C[(int64_t)row * g.m + col] = acc[rb2][cb][i];
            }
        }
    }
}

void gemm_launch(const float *a, const float *b, float *out, int batch, int n, int m, int k,
                 const char *who)
{
    if (n < 0 || m < 0 || k < 0 || batch < 0) {
        record_error(EMBER_ERR_INVALID_ARGUMENT, who);
        return;
    }
    if ((int64_t)n * m == 0 || batch == 0) return;
    GemmArgs g;
    g.a = a;
    g.b = b;
    g.c = out;
    g.n = n;
    g.m = m;
    g.k = k;
    g.sa = (int64_t)n * k;
    g.sb = (int64_t)k * m;
    g.sc = (int64_t)n * m;
    g.tiles_n = (n + BM - 1) / BM;
    g.tiles_m = (m + BN - 1) / BN;
    if (batch > 65535) {
        record_error(EMBER_ERR_UNSUPPORTED, who);
        return;
    }
    const bool vec = (k % 4 == 0) && (m % 4 == 0) && (((uintptr_t)a | (uintptr_t)b) % 16 == 0);
    const dim3 grid(g.tiles_n * g.tiles_m, batch);
    if (vec)
        hipLaunchKernelGGL(gemm_f32_kernel<true>, grid, dim3(kThreads), 0, 0, g);
    else
        hipLaunchKernelGGL(gemm_f32_kernel<false>, grid, dim3(kThreads), 0, 0, g);
    launch_ok(who);
}

}  // namespace
}  // namespace ember

extern "C" {

void matmul(const float *a, const float *b, float *out, int n, int m, int k)
{
    ember::gemm_launch(a, b, out, 1, n, m, k, "matmul");
}

void matmul_batched(const float *a, const float *b, float *out, int batch, int n, int m, int k)
{
    ember::gemm_launch(a, b, out, batch, n, m, k, "matmul_batched");
}

}  // extern "C"

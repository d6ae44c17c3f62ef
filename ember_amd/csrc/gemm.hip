// gemm.hip -- fp32 GEMM on gfx950 matrix cores behind Ember's matmul ABI.
//
// Replaces the reference's cuBLAS calls (src/tensor/operators_gpu.cu:114-136):
//   matmul(a, b, out, n, m, k):          out(n x m) = a(n x k) @ b(k x m)
//   matmul_batched(..., batch, n, m, k): the same per batch with strides
//                                        n*k, k*m, n*m
// and adds gemm_ex, which also takes either operand transposed in place
// (a stored k x n, b stored m x k: the weight- and input-gradient products of
// a Linear layer, ember/nn/layers.py:50-56, without materialising T(x)) and
// the fused epilogue of linear_fwd.
// all row-major fp32 with fp32 accumulation (v_mfma_f32_32x32x2f32; no
// reduced-precision inputs).  The CPU path of the reference accumulates in
// double (src/tensor/operators_cpu.c:47-60); agreement is to fp32 rounding
// of a length-k sum, see the parity tests.
//
// Tile-aligned shapes (n % 128, m % 256, k % 16 == 0) take the fast path
// further down (gemm_f32_dma_kernel: 128 x 256 or 256 x 256 tiles, slabs
// copied HBM -> LDS without registers).  The general path, for any other
// shape: a workgroup of 4 waves computes a 128 x 128 block of out, each
// wave a 64 x 64 quadrant as 2 x 2 MFMA accumulators.  The k dimension is
// walked in 32-wide slabs: the next slab's A (128 x 32) and B (32 x 128)
// are loaded from HBM/L2 into registers while the current one is multiplied
// out of LDS (two LDS buffers, one barrier per slab).  Lane half h of a wave
// contracts k in [16h, 16h+16) of the slab, so A is read from LDS as
// 128-bit row segments; B rows of the second half sit 32 floats further on
// so the two lane halves read disjoint banks.  Workgroups are ordered so
// that consecutive ones share B column panels in L2.
#include "common.h"
#include "lds_dma.h"
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
    int lda, ldb;        // row pitch of a and b as stored (k or n; m or k)
    int ta, tb;          // a stored k x n / b stored m x k
    int64_t sa, sb, sc;  // batch strides (elements)
    int tiles_n, tiles_m;
    int kchunk;          // split-K: k range of one blockIdx.z (multiple of 16)
    float *part;         // split-K partial sums [ksplit][batch][n][m]
    // Epilogue (all optional): out = act(acc + bias[col]) + residual, with
    // pre = acc + bias stored before the activation; residual and pre use
    // out's layout and batch stride.
    const float *bias;
    const float *residual;
    float *pre;
    int act;  // 0 none, 1 Ember's GELU
};

// Ember's GELU, 0.5*x*(1 + tanh(0.8*x)) (ember/nn/activations.py:58), in the
// order Ember's element-wise operators evaluate it.
__device__ __forceinline__ float gelu08(float x)
{
#pragma clang fp contract(off)
    return (x * 0.5f) * (tanhf(x * 0.8f) + 1.0f);
}

__device__ __forceinline__ float epilogue(const GemmArgs &g, float v, int64_t off, int col)
{
    if (g.bias) v += g.bias[col];
    if (g.pre) g.pre[off] = v;
    if (g.act == 1) v = gelu08(v);
    if (g.residual) v += g.residual[off];
    return v;
}

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
            if (VEC && !g.ta) {
                if (row < g.n && col < g.k) v = *(const f32x4 *)(A + (int64_t)row * g.lda + col);
            } else if (row < g.n) {
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    if (col + j < g.k)
                        v[j] = g.ta ? A[(int64_t)(col + j) * g.lda + row]
                                    : A[(int64_t)row * g.lda + col + j];
            }
            ra[it] = v;
        }
        {   // B: 32 rows x 32 float4
            const int r = idx >> 5, c4 = idx & 31;
            const int row = k0 + r, col = col0 + 4 * c4;
            f32x4 v = {0.f, 0.f, 0.f, 0.f};
            if (VEC && !g.tb) {
                if (row < g.k && col < g.m) v = *(const f32x4 *)(B + (int64_t)row * g.ldb + col);
            } else if (row < g.k) {
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    if (col + j < g.m)
                        v[j] = g.tb ? B[(int64_t)(col + j) * g.ldb + row]
                                    : B[(int64_t)row * g.ldb + col + j];
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
                if (row < g.n) {
                    const int64_t off = (int64_t)blockIdx.y * g.sc + (int64_t)row * g.m + col;
                    C[(int64_t)row * g.m + col] = epilogue(g, acc[rb2][cb][i], off, col);
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Fast path for tile-aligned shapes (n % 128 == 0, m % 256 == 0, k % 16 == 0,
// 16-byte aligned operands): 128 x 256 block of out per workgroup, 64 x 128
// per wave as 2 x 4 accumulators, two workgroups per CU.
//   * k is walked in slabs of 16, copied HBM -> LDS directly
//     (buffer_load_dwordx4 ... lds, no registers) one slab ahead into the
//     other of two buffers; one barrier per slab.
//   * A slab, a stored n x k: 128 tile rows padded to 20 floats, so the A
//     operand (one row per lane, 4 k per ds_read_b128) hits 16 different
//     bank groups.  a stored k x n (TA): 16 k-rows of 128 floats; a lane
//     reads two neighbouring tile rows with one ds_read_b64 and uses them as
//     the two row blocks of its wave, i.e. MFMA row r of row block rb is tile
//     row 2r + rb of the wave's 64 (undone in the store).
//   * B slab, b stored k x m: 16 rows of 256, a lane reads 4 consecutive
//     columns with one ds_read_b128, one per accumulator column block
//     (column = 4*lane + cb).  b stored m x k (TB): 256 columns padded to 20
//     floats, a lane reads 4 k of its column with one ds_read_b128 (column =
//     32*cb + lane).  Either way each B read feeds 8 MFMAs.
//   * every LDS address in the loop is a per-lane base plus a compile-time
//     offset.
//   * tiles are numbered so that the tiles one XCD runs (workgroup ids are
//     dealt to the 8 XCDs round-robin) are contiguous, and within that
//     range grouped 8 row tiles per B column panel for L2 reuse.
//   * split-K (SPLIT): blockIdx.z walks k in [z*kchunk, (z+1)*kchunk) and
//     stores its raw sums to part; gemm_splitk_reduce adds the splits in
//     order and applies the epilogue, so results do not depend on timing.
constexpr int FM = 128, FN = 256, FK = 16;
constexpr int FASTR = FK + 4;  // padded row of a k-contiguous slab

template <bool TA, int TM = FM> struct ASlab {
    static_assert(!TA || TM == 128, "a stored k x n: one 1 KiB copy is two 128-float rows");
    static constexpr int kBuf = TA ? FK * TM : TM * FASTR;     // floats
    static constexpr int kCopies = kBuf / 256;                  // 1 KiB copies
};
template <bool TB> struct BSlab {
    static constexpr int kBuf = TB ? FN * FASTR : FK * FN;
    static constexpr int kCopies = kBuf / 256;                  // 20 / 16
};

// TM = 128 (4 waves, 2 workgroups per CU) or 256 (8 waves, 1 per CU: the
// same 64 x 128 per wave, a third less L2 -> LDS traffic per flop).
// KG = 2 (TM = 128 only): two groups of 4 waves per workgroup, one per CU,
// each group with its own LDS buffers and the whole 128 x 256 tile; group 0
// multiplies the even k-slabs, group 1 the odd ones, and group 1's sums are
// added to group 0's through LDS before the store.  For outputs with no more
// tiles than CUs: two waves per SIMD instead of one, no extra HBM traffic.
template <bool TA, bool TB, bool SPLIT, int TM = FM, int KG = 1>
__global__ __launch_bounds__(TM * 2 * KG, TM == 128 && KG == 1 ? 2 : 1) void gemm_f32_dma_kernel(GemmArgs g)
{
    static_assert(KG == 1 || (KG == 2 && TM == 128 && !SPLIT), "k groups: 128-row tiles, no split-K");
    constexpr int NW = TM / 32;  // waves per group: TM/64 rows x 2 columns of 64 x 128
    constexpr int ABUF = ASlab<TA, TM>::kBuf, BBUF_ = BSlab<TB>::kBuf;
    constexpr int ACOP = ASlab<TA, TM>::kCopies, BCOP = BSlab<TB>::kCopies;
    __shared__ float As0[KG * ABUF], As1[KG * ABUF];
    __shared__ float Bs0[KG * BBUF_], Bs1[KG * BBUF_];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    // Wave index made provably uniform: the per-wave copy counts and LDS
    // destinations below then use scalar branches and registers.
    const int wg = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int grpk = KG == 1 ? 0 : wg / NW;  // k group
    const int w = KG == 1 ? wg : wg - grpk * NW;  // wave within the group
    const int h32 = lane >> 5;
    const int l32 = lane & 31;
    const int wr = w >> 1, wc = w & 1;

    const int ntiles = g.tiles_n * g.tiles_m;
    int tile = blockIdx.x;
    if (ntiles % 8 == 0) tile = (tile % 8) * (ntiles / 8) + tile / 8;
    constexpr int GROUP = 8;
    const int per_group = GROUP * g.tiles_m;
    const int grp = tile / per_group;
    const int first = grp * GROUP;
    const int rows_in_grp = min(GROUP, g.tiles_n - first);
    const int in_grp = tile - grp * per_group;
    // The tile origin is computed with vector integer division; made
    // provably uniform here, it stays in scalar registers and the buffer
    // descriptors built from it need no per-lane (waterfall) handling.
    const int row0 = __builtin_amdgcn_readfirstlane((first + in_grp % rows_in_grp) * TM);
    const int col0 = __builtin_amdgcn_readfirstlane((in_grp / rows_in_grp) * FN);

    int kbeg = 0, kend = g.k;
    if (SPLIT) {
        kbeg = blockIdx.z * g.kchunk;
        kend = min(g.k, kbeg + g.kchunk);
    }
    // Tile origins; slab k0 (absolute) is added per fetch.
    const float *A = g.a + (int64_t)blockIdx.y * g.sa + (TA ? (int64_t)row0 : (int64_t)row0 * g.lda);
    const float *B = g.b + (int64_t)blockIdx.y * g.sb + (TB ? (int64_t)col0 * g.ldb : (int64_t)col0);

    // Per-lane byte offsets of the 1 KiB copies this wave issues (copy
    // t = w + NW*s), below 2^32 because lda, ldb < 2^22 (checked on the host).
    constexpr int AS = (ACOP + NW - 1) / NW, BS = (BCOP + NW - 1) / NW;
    unsigned aoff[AS], boff[BS];
#pragma unroll
    for (int s = 0; s < AS; ++s) {
        const int t = w + NW * s;
        if (TA) {  // copy t: k-rows 2t, 2t+1, 32 chunks each
            aoff[s] = 4u * (unsigned)((2 * t + h32) * g.lda + 4 * l32);
        } else {   // row p / 5, chunk p % 5 (chunk 4 is row padding: re-read chunk 0)
            const int p = 64 * t + lane;
            const int r = p / (FASTR / 4), c = p - r * (FASTR / 4);
            aoff[s] = 4u * (unsigned)(r * g.lda + 4 * (c < 4 ? c : 0));
        }
    }
#pragma unroll
    for (int s = 0; s < BS; ++s) {
        const int t = w + NW * s;
        if (TB) {
            const int p = 64 * t + lane;
            const int r = p / (FASTR / 4), c = p - r * (FASTR / 4);
            boff[s] = 4u * (unsigned)(r * g.ldb + 4 * (c < 4 ? c : 0));
        } else {   // copy t: k-row t
            boff[s] = 4u * (unsigned)(t * g.ldb + 4 * lane);
        }
    }

    auto fetch = [&](int k0, float *__restrict__ as, float *__restrict__ bs) {
        const __amdgpu_buffer_rsrc_t ra = dma_rsrc(TA ? A + (int64_t)k0 * g.lda : A + k0);
#pragma unroll
        for (int s = 0; s < AS; ++s)
            if (w + NW * s < ACOP) dma16_buf(ra, aoff[s], as + 256 * (w + NW * s));
        const __amdgpu_buffer_rsrc_t rb = dma_rsrc(TB ? B + k0 : B + (int64_t)k0 * g.ldb);
#pragma unroll
        for (int s = 0; s < BS; ++s)
            if (w + NW * s < BCOP) dma16_buf(rb, boff[s], bs + 256 * (w + NW * s));
    };

    f32x16 acc[2][4];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = zero16();

    const int abase = TA ? 8 * h32 * TM + 64 * wr + 2 * l32 : (64 * wr + l32) * FASTR + 8 * h32;
    const int bbase = TB ? (128 * wc + l32) * FASTR + 8 * h32 : 8 * h32 * FN + 128 * wc + 4 * l32;
    auto slab = [&](const float *__restrict__ as, const float *__restrict__ bs) {
#pragma unroll
        for (int kk = 0; kk < 8; kk += 4) {
            f32x4 af[2];
            if (TA) {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const f32x2 v = *(const f32x2 *)&as[abase + (kk + j) * TM];
                    af[0][j] = v[0];
                    af[1][j] = v[1];
                }
            } else {
#pragma unroll
                for (int rb = 0; rb < 2; ++rb) af[rb] = *(const f32x4 *)&as[abase + rb * 32 * FASTR + kk];
            }
            f32x4 bt[4];
            if (TB) {
#pragma unroll
                for (int cb = 0; cb < 4; ++cb) bt[cb] = *(const f32x4 *)&bs[bbase + cb * 32 * FASTR + kk];
            }
            if (TB) {
                // Column block outermost: the MFMAs of block cb need only its
                // own B read, so the later reads overlap earlier products
                // (k-step innermost would need all four reads before the
                // first MFMA: 12 % slower with one workgroup per CU).  Each
                // accumulator still adds its k-steps in the same order.
#pragma unroll
                for (int cb = 0; cb < 4; ++cb)
#pragma unroll
                    for (int rb = 0; rb < 2; ++rb)
#pragma unroll
                        for (int j = 0; j < 4; ++j) acc[rb][cb] = mfma_32x32x2(af[rb][j], bt[cb][j], acc[rb][cb]);
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const f32x4 bf = *(const f32x4 *)&bs[bbase + (kk + j) * FN];
#pragma unroll
                    for (int rb = 0; rb < 2; ++rb)
#pragma unroll
                        for (int cb = 0; cb < 4; ++cb) acc[rb][cb] = mfma_32x32x2(af[rb][j], bf[cb], acc[rb][cb]);
                }
            }
        }
    };

    // This group's buffers and slabs: slab j of the group is slab
    // KG*j + grpk of the tile (the host launches KG = 2 only when the slab
    // count is even, so both groups meet the same barriers).
    float *const as0 = As0 + grpk * ABUF, *const as1 = As1 + grpk * ABUF;
    float *const bs0 = Bs0 + grpk * BBUF_, *const bs1 = Bs1 + grpk * BBUF_;
    const int nslab = (kend - kbeg) / FK / KG;
    auto kslab = [&](int j) { return kbeg + (KG * j + grpk) * FK; };
    if (nslab > 0) {
        fetch(kslab(0), as0, bs0);
        wait_vmem();
        __syncthreads();
    }
    // Two slabs per trip so that each buffer is a distinct LDS object: the
    // compiler then knows the copy into one does not feed reads of the other.
    for (int s = 0; s < nslab; s += 2) {
        if (s + 1 < nslab) fetch(kslab(s + 1), as1, bs1);
        slab(as0, bs0);
        wait_vmem();
        __syncthreads();
        if (s + 1 < nslab) {
            if (s + 2 < nslab) fetch(kslab(s + 2), as0, bs0);
            slab(as1, bs1);
            wait_vmem();
            __syncthreads();
        }
    }
    if constexpr (KG == 2) {
        // Group 1's sums to group 0, one row block at a time through the B
        // buffers (free after the loop's last barrier): wave w of group 1
        // writes acc[rb][0..3] lane-linearly (4096 floats) at xb, the wave
        // of group 0 with the same w reads them back.  Sums in a fixed order
        // (even slabs + odd slabs).
        static_assert(2 * BBUF_ >= 2 * 4096, "exchange area: two waves per B buffer");
        float *const xb = (w < 2 ? Bs0 : Bs1) + (w & 1) * 4096 + 4 * lane;
#pragma unroll
        for (int rb = 0; rb < 2; ++rb) {
            if (grpk == 1) {
#pragma unroll
                for (int cb = 0; cb < 4; ++cb)
#pragma unroll
                    for (int q = 0; q < 4; ++q)
                        *(f32x4 *)&xb[(cb * 4 + q) * 256] =
                            f32x4{acc[rb][cb][4 * q], acc[rb][cb][4 * q + 1], acc[rb][cb][4 * q + 2], acc[rb][cb][4 * q + 3]};
            }
            __syncthreads();
            if (grpk == 0) {
#pragma unroll
                for (int cb = 0; cb < 4; ++cb)
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const f32x4 o = *(const f32x4 *)&xb[(cb * 4 + q) * 256];
#pragma unroll
                        for (int e = 0; e < 4; ++e) acc[rb][cb][4 * q + e] += o[e];
                    }
            }
            __syncthreads();
        }
        if (grpk == 1) return;
    }

    // Output: row(rb, i) and col(cb) as the operand layouts above define them.
    const int64_t zoff = SPLIT ? ((int64_t)blockIdx.z * gridDim.y + blockIdx.y) * g.sc
                               : (int64_t)blockIdx.y * g.sc;
    const int64_t tile_off = zoff + (int64_t)row0 * g.m + col0;
    float *C = (SPLIT ? g.part : g.c) + tile_off;
    const bool epi = !SPLIT && (g.bias || g.pre || g.act || g.residual);
    // This lane's output columns (within the tile) for accumulator column
    // block cb: 4*l32 + cb (+128*wc) in the normal layout, 32*cb + l32 with
    // b transposed.  The epilogue's bias is loaded once per column.
    auto colof = [&](int cb) { return 128 * wc + (TB ? 32 * cb + l32 : 4 * l32 + cb); };
    f32x4 bv = {0.f, 0.f, 0.f, 0.f};
    if (epi && g.bias) {
#pragma unroll
        for (int cb = 0; cb < 4; ++cb) bv[cb] = g.bias[col0 + colof(cb)];
    }
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int row = TA ? 64 * wr + 2 * acc_row(i, h32) + rb : 64 * wr + 32 * rb + acc_row(i, h32);
            f32x4 v;
#pragma unroll
            for (int cb = 0; cb < 4; ++cb) v[cb] = acc[rb][cb][i];
            const int64_t roff = (int64_t)row * g.m;
            if (epi) {
                // out = act(acc + bias) + residual, pre = acc + bias.
#pragma clang fp contract(off)
                if (g.bias) v += bv;
                if (TB) {
#pragma unroll
                    for (int cb = 0; cb < 4; ++cb) {
                        if (g.pre) g.pre[tile_off + roff + colof(cb)] = v[cb];
                        if (g.act == 1) v[cb] = gelu08(v[cb]);
                        if (g.residual) v[cb] += g.residual[tile_off + roff + colof(cb)];
                    }
                } else {
                    if (g.pre) *(f32x4 *)&g.pre[tile_off + roff + colof(0)] = v;
                    if (g.act == 1) {
#pragma unroll
                        for (int cb = 0; cb < 4; ++cb) v[cb] = gelu08(v[cb]);
                    }
                    if (g.residual) v += *(const f32x4 *)&g.residual[tile_off + roff + colof(0)];
                }
            }
            if (TB) {
#pragma unroll
                for (int cb = 0; cb < 4; ++cb) C[roff + colof(cb)] = v[cb];
            } else {
                *(f32x4 *)&C[roff + colof(0)] = v;
            }
        }
    }
}

// out = epilogue(sum over z of part[z]), z in order; m % 4 == 0.
__global__ __launch_bounds__(256) void gemm_splitk_reduce(GemmArgs g, int ksplit, int64_t total)
{
    const int64_t n4 = total / 4;
    for (int64_t q = (int64_t)blockIdx.x * 256 + threadIdx.x; q < n4; q += (int64_t)gridDim.x * 256) {
        const int64_t off = 4 * q;
        f32x4 s = *(const f32x4 *)&g.part[off];
        for (int z = 1; z < ksplit; ++z) {
            const f32x4 v = *(const f32x4 *)&g.part[(int64_t)z * total + off];
#pragma unroll
            for (int c = 0; c < 4; ++c) s[c] += v[c];
        }
        if (g.bias || g.pre || g.act || g.residual) {
            const int col = (int)(off % g.m);
#pragma unroll
            for (int c = 0; c < 4; ++c) s[c] = epilogue(g, s[c], off + c, col + c);
        }
        *(f32x4 *)&g.c[off] = s;
    }
}

// Tile-shape choice only: an unknown CU count falls back to MI355X's 256.
int num_cus()
{
    const int n = device_cu_count();
    return n > 0 ? n : 256;
}

template <bool TA, bool TB>
void launch_fast(const GemmArgs &g, dim3 grid, bool split)
{
    // 256-row tiles when their count fills whole waves of CUs (or leaves a
    // small tail): a 256 x 256 tile per CU reads a third less per flop, but
    // a partly idle last wave costs more than that saves.
    if constexpr (!TA) {
        if (!split && g.n % 256 == 0) {
            const int cus = num_cus();
            const int tiles = (g.n / 256) * g.tiles_m * (int)grid.y;
            if (tiles % cus == 0 || tiles >= 4 * cus) {
                GemmArgs g2 = g;
                g2.tiles_n = g.n / 256;
                const dim3 grid2(g2.tiles_n * g2.tiles_m, grid.y, 1);
                hipLaunchKernelGGL((gemm_f32_dma_kernel<TA, TB, false, 256>), grid2, dim3(512), 0, 0, g2);
                return;
            }
        }
    }
    if (split) {
        hipLaunchKernelGGL((gemm_f32_dma_kernel<TA, TB, true>), grid, dim3(kThreads), 0, 0, g);
        return;
    }
    // No more tiles than CUs: one workgroup per CU either way, so give it two
    // k groups (two waves per SIMD); needs an even slab count.
    if ((int)(grid.x * grid.y) <= num_cus() && (g.k / FK) % 2 == 0 && g.k >= 4 * FK) {
        hipLaunchKernelGGL((gemm_f32_dma_kernel<TA, TB, false, FM, 2>), grid, dim3(2 * kThreads), 0, 0, g);
        return;
    }
    hipLaunchKernelGGL((gemm_f32_dma_kernel<TA, TB, false>), grid, dim3(kThreads), 0, 0, g);
}

int gemm_launch(const float *a, const float *b, float *out, int batch, int n, int m, int k,
                const char *who, const float *bias = nullptr, const float *residual = nullptr,
                float *pre = nullptr, int act = 0, int ta = 0, int tb = 0)
{
    if (n < 0 || m < 0 || k < 0 || batch < 0) return record_error(EMBER_ERR_INVALID_ARGUMENT, who);
    if ((int64_t)n * m == 0 || batch == 0) return EMBER_OK;
    // k == 0: a and b are empty (null from alloc_memory(0)) and every output
    // is an empty sum, i.e. 0 before the epilogue, as in the reference's CPU
    // loop; the generic kernel below never reads a or b then.
    if (!out || (k > 0 && (!a || !b))) return record_error(EMBER_ERR_INVALID_ARGUMENT, who);
    GemmArgs g;
    g.a = a;
    g.b = b;
    g.c = out;
    g.n = n;
    g.m = m;
    g.k = k;
    g.ta = ta;
    g.tb = tb;
    g.lda = ta ? n : k;
    g.ldb = tb ? k : m;
    g.sa = (int64_t)n * k;
    g.sb = (int64_t)k * m;
    g.sc = (int64_t)n * m;
    g.tiles_n = (n + BM - 1) / BM;
    g.tiles_m = (m + BN - 1) / BN;
    g.kchunk = k;
    g.part = nullptr;
    g.bias = bias;
    g.residual = residual;
    g.pre = pre;
    g.act = act;
    if (batch > 65535) return record_error(EMBER_ERR_UNSUPPORTED, who);
    const bool vec = (k % 4 == 0) && (m % 4 == 0) && (n % 4 == 0 || !ta) &&
                     (((uintptr_t)a | (uintptr_t)b) % 16 == 0);
    // The fast kernel moves out, pre and residual as 16-byte vectors, and
    // addresses a tile's rows with 32-bit byte offsets (row pitch < 2^22).
    if (vec && n % FM == 0 && m % FN == 0 && k % FK == 0 && k > 0 && g.lda < (1 << 22) &&
        g.ldb < (1 << 22) &&
        (((uintptr_t)out | (uintptr_t)pre | (uintptr_t)residual) % 16) == 0) {
        g.tiles_n = n / FM;
        g.tiles_m = m / FN;
        const int work = g.tiles_n * g.tiles_m * batch;
        // Fewer tiles than CUs: split k so that about two workgroups run per
        // CU, each over at least 512 of k.
        int ksplit = 1;
        const int cus = num_cus();
        if (work < cus && k >= 1024) {
            ksplit = min(2 * cus / work, k / 512);
            if (ksplit > 64) ksplit = 64;
            if (ksplit > 1) {
                g.kchunk = ((k + ksplit - 1) / ksplit + FK - 1) / FK * FK;
                ksplit = (k + g.kchunk - 1) / g.kchunk;
            }
        }
        dim3 grid(g.tiles_n * g.tiles_m, batch, ksplit);
        const bool split = ksplit > 1;
        if (split) {
            const int64_t total = (int64_t)batch * n * m;
            g.part = (float *)scratch(kScratchGemmSplit, (size_t)ksplit * total * sizeof(float));
            if (!g.part) return EMBER_ERR_OUT_OF_MEMORY;
        }
        if (ta)
            tb ? launch_fast<true, true>(g, grid, split) : launch_fast<true, false>(g, grid, split);
        else
            tb ? launch_fast<false, true>(g, grid, split) : launch_fast<false, false>(g, grid, split);
        if (!launch_ok(who)) return EMBER_ERR_DEVICE;
        if (split) {
            const int64_t total = (int64_t)batch * n * m;
            int64_t blocks = (total / 4 + 255) / 256;
            if (blocks > 8 * cus) blocks = 8 * cus;
            hipLaunchKernelGGL(gemm_splitk_reduce, dim3((unsigned)blocks), dim3(256), 0, 0, g,
                               ksplit, total);
            if (!launch_ok("gemm_splitk_reduce")) return EMBER_ERR_DEVICE;
        }
        return EMBER_OK;
    }
    const dim3 grid(g.tiles_n * g.tiles_m, batch);
    if (vec)
        hipLaunchKernelGGL(gemm_f32_kernel<true>, grid, dim3(kThreads), 0, 0, g);
    else
        hipLaunchKernelGGL(gemm_f32_kernel<false>, grid, dim3(kThreads), 0, 0, g);
    return launch_ok(who) ? EMBER_OK : EMBER_ERR_DEVICE;
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

int linear_fwd(const float *a, const float *b, const float *bias, const float *residual,
               float *out, float *pre, int n, int m, int k, int act)
{
    if (act < 0 || act > 1) return ember::record_error(EMBER_ERR_INVALID_ARGUMENT, "linear_fwd");
    return ember::gemm_launch(a, b, out, 1, n, m, k, "linear_fwd", bias, residual, pre, act);
}

int gemm_ex(const float *a, const float *b, float *out, int batch, int n, int m, int k,
            int trans_a, int trans_b, const float *bias, const float *residual, float *pre, int act)
{
    if (act < 0 || act > 1 || (trans_a != 0 && trans_a != 1) || (trans_b != 0 && trans_b != 1))
        return ember::record_error(EMBER_ERR_INVALID_ARGUMENT, "gemm_ex");
    return ember::gemm_launch(a, b, out, batch, n, m, k, "gemm_ex", bias, residual, pre, act,
                              trans_a, trans_b);
}

}  // extern "C"

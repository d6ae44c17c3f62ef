// attention_bwd.hip -- entry point of the fused flash-attention backward
// (fp32, gfx950); the short-sequence kernels (S <= 64: one workgroup per head
// with Q, K, V, dO staged in LDS) are below; 64 < S <= 128 at D = 64 and 128
// runs attn_bwd_s128 (attention_bwd_s128.hip), longer D = 64 attn_bwd_w16
// (attention_bwd_w16.hip), and the rest the key-block workgroup kernel of
// attention_bwd_kernels.h.
//
// No reference counterpart (pawel002/ember has no attention): the operator is
// new, slotted beside matmul in src/tensor/operators.h:20-27.  Its semantics
// are those of oracle/ember_oracle.c (oracle_attention_bwd).
//
// Build note.  This file is compiled with -mllvm -amdgpu-mfma-vgpr-form=1
// (MFMA accumulators in VGPRs); the causal D = 128 instantiation lives in
// attention_bwd_c128.hip, compiled with the default (AGPR) form.  Measured
// at config shapes on MI355X: the AGPR form is 1.7 % faster for causal
// D = 128, while for non-causal D = 128 the default allocation cycles the
// 128 dK/dV accumulators between AGPRs and VGPRs every query block and runs
// 2x slower than the VGPR form (and D = 64 causal is 6 % faster in VGPR form).
#include <mutex>

#include <algorithm>

#include "attention_bwd_kernels.h"

namespace ember {
namespace {

// Compute units of the current device: the grid of the persistent kernels
// below.
int device_cus(int *out)
{
    *out = device_cu_count();
    return *out > 0 ? EMBER_OK : record_error(EMBER_ERR_DEVICE, "hipDeviceGetAttribute(CU count)");
}

// 32 < S <= 64 at D = 128: a workgroup of 8 waves stages one head's Q, K,
// dO and V in LDS as 64 padded rows of D+4 floats (132 KB: one workgroup
// per CU), forms delta = <dO, O> per row and lse2 = lse * log2(e) while
// staging, and never leaves the CU for intermediate results.  Rows past S
// are staged as row S-1 and carry lse2 = +inf (P = 0), delta = 0.  P^T and
// dS^T (64 x 68 floats each) overlay the V tile once every wave is past its
// dP products, so P and dS wait in registers across one barrier.
//   wave w: S / dP quadrants w and w + 8 of the 4 x 4 grid of 16 x 16
//   quadrants on v_mfma_f32_16x16x4f32 over all of D (causally: the lower
//   triangle, dealt as below);
//   wave w: rows 32(w/4).. and columns 32(w%4).. of dV, dK and dQ on
//   v_mfma_f32_32x32x2f32 over the 64 queries / keys (a causal head skips
//   the half that is all zeros: keys 32.. see only queries 32.., queries
//   0..31 only keys 0..31), contracting in the order
//   q = 4 (s & 1) + 8 h + 16 (s >> 1) + j for k-step s, lane half h and
//   MFMA j, which puts the two lane halves' LDS rows 8 apart, in disjoint
//   banks.
struct ShortLds64 {
    static constexpr int D = 128;
    static constexpr int R = 64;                         // rows per tile
    static constexpr int NW = 8;                         // waves
    static constexpr int STR = D + 4;
    static constexpr int ROWCH = STR / 4;
    static constexpr int COP = (R * ROWCH + 63) / 64;    // 33 copies per tile
    static constexpr int TILE = COP * 256;
    static constexpr int PSTR = R + 4;                   // P^T / dS^T row
    static constexpr int VP = TILE > 2 * R * PSTR ? TILE : 2 * R * PSTR;
};

// Quadrant e of an N x N grid of 16 x 16 S / dP blocks: row-major, or
// causally the lower triangle row by row, (0,0), (1,0), (1,1), (2,0), ...
// Dealing the causal triangle's quadrants in this order to waves
// e mod NW evens out the SIMDs (waves w and w + 4 share one): at N = 4 and
// 8 waves, 3, 3, 2, 2 products against 4, 3, 2, 1 for the full grid's
// quadrants w and w + 8 with the masked ones skipped.
template <int N, bool CAUSAL>
__device__ __forceinline__ void quad_of(int e, int &qm, int &qn)
{
    if (CAUSAL) {
        qm = 0;
#pragma unroll
        for (int m = 1; m < N; ++m) qm += e >= m * (m + 1) / 2;
        qn = e - qm * (qm + 1) / 2;
    } else {
        qm = e / N;
        qn = e - qm * N;
    }
}

// The kernel is persistent: one workgroup per CU walks heads blockIdx.x,
// blockIdx.x + gridDim.x, ...  The tiles take the whole LDS, so no second
// workgroup can overlap one head's HBM traffic with another's products;
// instead each thread prefetches its row share of the next head (Q, K, V,
// dO and O: 8 lanes per row, 16 floats of each) into registers while the
// current head is multiplied (+13-23 % against one workgroup per head,
// which loaded, then multiplied).  Per iteration:
//   barrier (the previous head's products are done with LDS);
//   prefetched rows -> LDS tiles, delta and lse2 from them; barrier;
//   prefetch the next head's rows;
//   S / dP of the quadrants, P / dS, then dV / dK / dQ; store them.
// Causally the 10 quadrants of the lower triangle are dealt in quad_of's
// order (SIMDs 3, 3, 2, 2; +3-4 % at S = 48-64 against quadrants w and
// w + 8 of the full grid, 4, 3, 2, 1).
// Vector-memory operations retire in issue order and the stores are the
// last ones of an iteration, so the wait for the prefetched rows at the
// next iteration's top is vmcnt(stores): it does not wait for the stores.
template <bool CAUSAL>
__global__ __launch_bounds__(512, 1) void attn_bwd_short_lds64p(BwdArgs a, int nbh)
{
    typedef ShortLds64 L;
    constexpr int D = L::D, R = L::R;
    __shared__ float tiles[3 * L::TILE + L::VP];  // Q, K, dO, then V (later P^T, dS^T)
    __shared__ float L2s[R], DLs[R];
    float *__restrict__ Qs = tiles;
    float *__restrict__ Ks = tiles + L::TILE;
    float *__restrict__ Gs = tiles + 2 * L::TILE;
    float *__restrict__ Vs = tiles + 3 * L::TILE;
    float *__restrict__ PT = Vs;
    float *__restrict__ DT = Vs + R * L::PSTR;

    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int S = a.S;
    const int in_ss = (int)a.in_ss, out_ss = (int)a.out_ss;  // < 2^24 (checked on the host)
    // Staging and row statistics: row j, 8 lanes per row, columns 32 it + 4 s8.
    const int j = 8 * w + (lane >> 3), s8 = lane & 7;
    const int jr = j < S ? j : S - 1;  // rows past S re-read row S-1 (masked later)
    auto in_base_of = [&](int bh) {
        const int b = bh / a.H;
        return (int64_t)b * a.in_sb + (int64_t)(bh - b * a.H) * a.in_sh;
    };
    auto out_base_of = [&](int bh) {
        const int b = bh / a.H;
        return (int64_t)b * a.out_sb + (int64_t)(bh - b * a.H) * a.out_sh;
    };
    f32x4 rq[D / 32], rk[D / 32], rv[D / 32], rg[D / 32], ro[D / 32];
    float lse_v = 0.0f;
    auto prefetch = [&](int bh) {
        const int64_t ib = in_base_of(bh) + (int64_t)jr * in_ss + 4 * s8;
        const int64_t ob = out_base_of(bh) + (int64_t)jr * out_ss + 4 * s8;
#pragma unroll
        for (int it = 0; it < D / 32; ++it) {
            rq[it] = *(const f32x4 *)(a.q + ib + 32 * it);
            rk[it] = *(const f32x4 *)(a.k + ib + 32 * it);
            rv[it] = *(const f32x4 *)(a.v + ib + 32 * it);
            rg[it] = *(const f32x4 *)(a.dout + ob + 32 * it);
            ro[it] = *(const f32x4 *)(a.o + ob + 32 * it);
        }
        lse_v = a.lse[(int64_t)bh * S + jr];
    };

    const int h32 = lane >> 5, l32 = lane & 31;
    const int rb = w >> 2;
    const int col = 32 * (w & 3) + l32;
    const int row = 32 * rb + l32;

    const int stride = (int)gridDim.x;
    int bh = blockIdx.x;
    prefetch(bh);
    // The first head's rows are waited for here, so that the loop's head,
    // where this path and the previous iteration's meet, waits only for the
    // prefetched rows and not for the stores issued after them.
    wait_vmem();
    for (; bh < nbh; bh += stride) {
        __syncthreads();  // the previous head's products are done with the tiles
        {
            float part = 0.0f;
#pragma unroll
            for (int c = 0; c < D / 32; ++c) {
                const int off = j * L::STR + 32 * c + 4 * s8;
                *(f32x4 *)&Qs[off] = rq[c];
                *(f32x4 *)&Ks[off] = rk[c];
                *(f32x4 *)&Vs[off] = rv[c];
                *(f32x4 *)&Gs[off] = rg[c];
                part += ro[c][0] * rg[c][0] + ro[c][1] * rg[c][1] + ro[c][2] * rg[c][2] + ro[c][3] * rg[c][3];
            }
            part += __shfl_xor(part, 1);
            part += __shfl_xor(part, 2);
            part += __shfl_xor(part, 4);
            if (s8 == 0) {
                L2s[j] = j < S ? lse_v * kLog2e : INFINITY;
                DLs[j] = j < S ? part : 0.0f;
            }
        }
        __syncthreads();
        // The next head's loads are issued after the barrier, so that no wave
        // waits at it for the others' issue (+5.6 % at S = 64, +7.7 % at 48).
        prefetch(bh + stride < nbh ? bh + stride : bh);  // one path: the last head re-reads itself

        // ---- S, dP, P, dS of quadrants w and w + 8 ----
        const int l16 = lane & 15, g4 = lane >> 4;
        // Causal: the 10 quadrants of the lower triangle (quad_of's order)
        // with products, then (0,1) and (2,3), all masked, which the 32-row
        // blocks below read and which are written as zeros.
        constexpr int NQD = CAUSAL ? 12 : 16;
        float pv[2][4], dv4[2][4];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int e = w + L::NW * u;
            if (e >= NQD) break;
            int qm, qn;
            if (CAUSAL && e >= 10) {
                qm = e == 10 ? 0 : 2;
                qn = qm + 1;
            } else {
                quad_of<4, CAUSAL>(e, qm, qn);
            }
            const int key = 16 * qn + l16;
            f32x4 sacc = {0.f, 0.f, 0.f, 0.f}, pacc = {0.f, 0.f, 0.f, 0.f};
            if (!CAUSAL || e < 10) {
                const int arow = (16 * qm + l16) * L::STR + 4 * g4;
                const int brow = key * L::STR + 4 * g4;
#pragma unroll
                for (int c0 = 0; c0 < D; c0 += 16) {
                    const f32x4 qf = *(const f32x4 *)&Qs[arow + c0];
                    const f32x4 kf = *(const f32x4 *)&Ks[brow + c0];
                    const f32x4 gf = *(const f32x4 *)&Gs[arow + c0];
                    const f32x4 vf = *(const f32x4 *)&Vs[brow + c0];
#pragma unroll
                    for (int jj = 0; jj < 4; ++jj) {
                        sacc = __builtin_amdgcn_mfma_f32_16x16x4f32(qf[jj], kf[jj], sacc, 0, 0, 0);
                        pacc = __builtin_amdgcn_mfma_f32_16x16x4f32(gf[jj], vf[jj], pacc, 0, 0, 0);
                    }
                }
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int qi = 16 * qm + 4 * g4 + r;
                float p = __builtin_amdgcn_exp2f(fmaf(sacc[r], a.c, -L2s[qi]));
                const bool vis = key < S && (!CAUSAL || key <= qi);
                p = vis ? p : 0.0f;
                pv[u][r] = p;
                dv4[u][r] = p * (pacc[r] - DLs[qi]);
            }
        }
        __syncthreads();  // every wave is past its dP products: V's space is free
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int e = w + L::NW * u;
            if (e >= NQD) break;
            int qm, qn;
            if (CAUSAL && e >= 10) {
                qm = e == 10 ? 0 : 2;
                qn = qm + 1;
            } else {
                quad_of<4, CAUSAL>(e, qm, qn);
            }
            const int key = 16 * qn + l16;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int qi = 16 * qm + 4 * g4 + r;
                PT[key * L::PSTR + qi] = pv[u][r];
                DT[key * L::PSTR + qi] = dv4[u][r];
            }
        }
        __syncthreads();

        // ---- rows 32 rb.., columns 32 cb.. of dV, dK (rows: keys) and dQ (rows: queries) ----
        f32x16 dv = zero16(), dk = zero16(), dq = zero16();
        auto kstep = [&](int t) {
            const int q0 = 4 * (t & 1) + 8 * h32 + 16 * (t >> 1);
            const bool kv_live = !CAUSAL || rb == 0 || t >= 4;
            const bool q_live = !CAUSAL || rb == 1 || t < 4;
            if (kv_live) {
                const f32x4 pt = *(const f32x4 *)&PT[row * L::PSTR + q0];
                const f32x4 dt = *(const f32x4 *)&DT[row * L::PSTR + q0];
#pragma unroll
                for (int jj = 0; jj < 4; ++jj) {
                    dv = mfma_32x32x2(pt[jj], Gs[(q0 + jj) * L::STR + col], dv);
                    dk = mfma_32x32x2(dt[jj], Qs[(q0 + jj) * L::STR + col], dk);
                }
            }
            if (q_live) {
#pragma unroll
                for (int jj = 0; jj < 4; ++jj)
                    dq = mfma_32x32x2(DT[(q0 + jj) * L::PSTR + row], Ks[(q0 + jj) * L::STR + col], dq);
            }
        };
        // Half the k-steps unrolled, which keeps the kernel within 256
        // registers next to the prefetched rows (fully unrolled, the
        // non-causal kernel spills 12).
#pragma unroll 4
        for (int t = 0; t < 8; ++t) kstep(t);
        // Branch-free bounded stores (rows past S pushed out of the
        // descriptors' range), so that every path issues the same stores and
        // the next head's wait for its prefetched rows does not wait for them.
        const int64_t ib = in_base_of(bh);
        const unsigned range = 4u * (unsigned)((S - 1) * in_ss + 128);
        const __amdgpu_buffer_rsrc_t rdv = store_rsrc(a.dv + ib, range);
        const __amdgpu_buffer_rsrc_t rdk = store_rsrc(a.dk + ib, range);
        const __amdgpu_buffer_rsrc_t rdq = store_rsrc(a.dq + ib, range);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int r = 32 * rb + acc_row(i, h32);
            const unsigned off = r < S ? 4u * (unsigned)(r * in_ss + col) : kStoreNone;
            store1_bounded(rdv, off, dv[i]);
            store1_bounded(rdk, off, dk[i] * a.scale);
            store1_bounded(rdq, off, dq[i] * a.scale);
        }
    }
}

template <bool CAUSAL>
int launch_bwd_short_lds64p(const BwdArgs &args, int nbh)
{
    int ncu = 0;
    const int st = device_cus(&ncu);
    if (st != EMBER_OK) return st;
    const int grid = nbh < ncu ? nbh : ncu;
    hipLaunchKernelGGL((attn_bwd_short_lds64p<CAUSAL>), dim3((unsigned)grid), dim3(512), 0, 0, args, nbh);
    return launch_ok("attn_bwd_short_lds64p") ? EMBER_OK : EMBER_ERR_DEVICE;
}


// Short sequences (S <= R; R = 32 or 64 rows at D <= 64, R = 32 at
// D = 128): one workgroup of R/8 waves per head, the head's Q, K, V, dO
// staged in LDS in padded rows (D+4 floats; rows past S staged as row S-1,
// with lse2 = +inf and delta = 0), every product on v_mfma_f32_16x16x4f32
// so that the work splits evenly over the waves at any D and R:
//   wave w: S and dP of the 16 x 16 quadrants w, w + NW, ... of the
//   (R/16)^2 grid (causal: quadrants above the diagonal are skipped; at
//   R = 64 only the 10 of the lower triangle are dealt, in quad_of's order,
//   so the SIMDs take 3, 3, 2, 2 of them: +6-7 % causal at S = 48-64), P
//   and dS stored transposed ([key][query], rows of R+4) in LDS;
//   wave w: the 16 x 16 output blocks w, w + NW, ... of dV, dK (rows: keys)
//   and dQ (rows: queries), 3 (R/16)(D/16) blocks in all, each contracting
//   16 queries or keys per group of 4 MFMAs (causal: only the groups that
//   can be nonzero: keys 16rb.. see queries >= 16rb, queries 16rb.. keys
//   <= 16rb + 15).
// A 16 x 16 product's A operand [m][k] is lane m + 16k and its B operand
// [k][n] lane n + 16k: with k = 4 g + j (g = lane / 16, MFMA j of a group
// of 4), P^T / dS^T rows are read as 128-bit segments, the other operand
// one float per lane from rows 4 apart (disjoint banks for rows of D+4 or
// R+4 floats).  R = 32: 46 KB of LDS at D = 64 (three workgroups per CU),
// 79 KB at D = 128 (two); R = 64: 104 KB at D = 64 (one per CU).
template <int D, int R>
struct LdsBwdShape {
    static constexpr int NW = R / 8;
    static constexpr int STR = D + 4;
    static constexpr int ROWCH = STR / 4;
    static constexpr int COP = (R * ROWCH + 63) / 64;
    static constexpr int TILE = COP * 256;
    static constexpr int PSTR = R + 4;
    static constexpr int NBO = (R / 16) * (D / 16);        // 16 x 16 blocks per output
    static constexpr int NB = 3 * NBO / NW;                // output blocks per wave
    static_assert(NB * NW == 3 * NBO, "even split");
    // S / dP quadrants, dealt to the waves in order: wave w takes w,
    // w + NW, ...  Causal 64-row tiles deal only the lower triangle (the
    // quadrants the dV / dK / dQ products read) for even SIMDs; at 32 rows
    // (three workgroups per CU) the full grid with the masked quadrant
    // written as zeros measured 1 % faster.
    template <bool CAUSAL> struct Quads {
        static constexpr bool TRI = CAUSAL && R == 64;
        static constexpr int N = TRI ? (R / 16) * (R / 16 + 1) / 2 : (R / 16) * (R / 16);
        static constexpr int PER_WAVE = (N + NW - 1) / NW;
    };
};

// R = 64 at D = 64 is persistent (one workgroup per CU walks heads
// blockIdx.x, blockIdx.x + gridDim.x, ...), as attn_bwd_short_lds64p: each
// thread prefetches its row share of the next head (Q, K, V, dO, O: 8 lanes
// per row) into registers while the current head is multiplied, because the
// 104 KB of LDS leave no room for a second workgroup to overlap the loads
// (+11-15 % at S = 48 and 64).  At D = 32 (72 KB) two workgroups per CU
// already overlap each other and the persistent form measured 0 to -6 %.
// R = 32 at D = 64 (three workgroups per CU) takes the persistent form
// (PERS, three per CU) for S < 32 and non-causally: +27 % at S = 17, +5 %
// at S = 25, +3.7 % non-causal at S = 32; causal S = 32 measured -1.5 %
// and keeps one workgroup per head.  R = 32 at D = 128 is persistent with
// two workgroups per CU (S <= 32; against a one-head-per-workgroup kernel
// with direct HBM -> LDS copies and 32 x 32 products: +14 % at S = 17,
// +8 % at S = 25, +1.6 % causal and +2.8 % non-causal at S = 32).
template <int D, int R, bool CAUSAL, bool PERS>
__global__ __launch_bounds__(R * 8, R == 32 ? 2 : 1) void attn_bwd_lds16(BwdArgs a, int nbh)
{
    typedef LdsBwdShape<D, R> L;
    constexpr bool kPersistent = PERS;
    static_assert(!PERS || D == 64 || (D == 128 && R == 32), "persistent forms: D = 64, or D = 128 with 32 rows");
    constexpr int CH = D / 32;  // 16-byte chunks per lane and row
    __shared__ float tiles[4 * L::TILE];  // Q, K, V, dO
    __shared__ float PT[R * L::PSTR], DT[R * L::PSTR];
    __shared__ float L2s[R], DLs[R];
    float *__restrict__ Qs = tiles;
    float *__restrict__ Ks = tiles + L::TILE;
    float *__restrict__ Vs = tiles + 2 * L::TILE;
    float *__restrict__ Gs = tiles + 3 * L::TILE;

    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int S = a.S;
    const int in_ss = (int)a.in_ss, out_ss = (int)a.out_ss;  // < 2^24 (checked on the host)
    // Row statistics (and, persistent, staging): row j, 8 lanes per row.
    const int j = 8 * w + (lane >> 3);
    const int s8 = lane & 7;
    const int jr = j < S ? j : S - 1;  // rows past S re-read row S-1 (masked later)
    auto in_base_of = [&](int bh) {
        const int b = bh / a.H;
        return (int64_t)b * a.in_sb + (int64_t)(bh - b * a.H) * a.in_sh;
    };
    auto out_base_of = [&](int bh) {
        const int b = bh / a.H;
        return (int64_t)b * a.out_sb + (int64_t)(bh - b * a.H) * a.out_sh;
    };
    auto put_stats = [&](float part, float lse) {
        part += __shfl_xor(part, 1);
        part += __shfl_xor(part, 2);
        part += __shfl_xor(part, 4);
        if (s8 == 0) {
            L2s[j] = j < S ? lse * kLog2e : INFINITY;
            DLs[j] = j < S ? part : 0.0f;
        }
    };

    const int l16 = lane & 15, g4 = lane >> 4;
    // S / dP / P / dS of this wave's quadrants, then its 16 x 16 blocks of
    // dV, dK, dQ, stored.  Q, K, V, dO and the statistics are in LDS.
    auto compute = [&](int bh) {
        const int64_t in_base = in_base_of(bh);
        auto quadrant = [&](int qm, int qn, bool live) {
            const int key = 16 * qn + l16;
            f32x4 sacc = {0.f, 0.f, 0.f, 0.f}, pacc = {0.f, 0.f, 0.f, 0.f};
            if (live) {
                const int arow = (16 * qm + l16) * L::STR + 4 * g4;
                const int brow = key * L::STR + 4 * g4;
#pragma unroll
                for (int c0 = 0; c0 < D; c0 += 16) {
                    const f32x4 qf = *(const f32x4 *)&Qs[arow + c0];
                    const f32x4 kf = *(const f32x4 *)&Ks[brow + c0];
                    const f32x4 gf = *(const f32x4 *)&Gs[arow + c0];
                    const f32x4 vf = *(const f32x4 *)&Vs[brow + c0];
#pragma unroll
                    for (int jj = 0; jj < 4; ++jj) {
                        sacc = __builtin_amdgcn_mfma_f32_16x16x4f32(qf[jj], kf[jj], sacc, 0, 0, 0);
                        pacc = __builtin_amdgcn_mfma_f32_16x16x4f32(gf[jj], vf[jj], pacc, 0, 0, 0);
                    }
                }
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int qi = 16 * qm + 4 * g4 + r;
                float p = __builtin_amdgcn_exp2f(fmaf(sacc[r], a.c, -L2s[qi]));
                const bool vis = key < S && (!CAUSAL || key <= qi);
                p = vis ? p : 0.0f;
                PT[key * L::PSTR + qi] = p;
                DT[key * L::PSTR + qi] = p * (pacc[r] - DLs[qi]);
            }
        };
        if constexpr (L::template Quads<CAUSAL>::TRI) {
#pragma unroll
            for (int u = 0; u < L::template Quads<CAUSAL>::PER_WAVE; ++u) {
                const int e = w + L::NW * u;
                if (e >= L::template Quads<CAUSAL>::N) break;
                int qm, qn;
                quad_of<R / 16, true>(e, qm, qn);
                quadrant(qm, qn, true);
            }
        } else {
#pragma unroll
            for (int u = 0; u < (R / 16) * (R / 16) / L::NW; ++u) {
                const int quad = w + L::NW * u;
                const int qm = quad / (R / 16), qn = quad - qm * (R / 16);
                quadrant(qm, qn, !CAUSAL || qn <= qm);
            }
        }
        __syncthreads();

#pragma unroll
        for (int u = 0; u < L::NB; ++u) {
            const int blk = w + L::NW * u;
            const int o = blk / L::NBO;  // 0 dV, 1 dK, 2 dQ
            const int rem = blk - o * L::NBO;
            const int rb = rem / (D / 16), cb = rem - rb * (D / 16);
            const int col = 16 * cb + l16;
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
            if (o < 2) {
                // dV[k][n] = sum_q P^T[k][q] dO[q][n];  dK[k][n] = sum_q dS^T[k][q] Q[q][n]
                const float *__restrict__ A = o == 0 ? PT : DT;
                const float *__restrict__ Bt = o == 0 ? Gs : Qs;
#pragma unroll
                for (int c = 0; c < R / 16; ++c) {
                    if (CAUSAL && c < rb) continue;
                    const f32x4 af = *(const f32x4 *)&A[(16 * rb + l16) * L::PSTR + 16 * c + 4 * g4];
#pragma unroll
                    for (int jj = 0; jj < 4; ++jj)
                        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(
                            af[jj], Bt[(16 * c + 4 * g4 + jj) * L::STR + col], acc, 0, 0, 0);
                }
            } else {
                // dQ[m][n] = sum_k dS[m][k] K[k][n] = sum_k dS^T[k][m] K[k][n]
#pragma unroll
                for (int c = 0; c < R / 16; ++c) {
                    if (CAUSAL && c > rb) continue;
#pragma unroll
                    for (int jj = 0; jj < 4; ++jj) {
                        const int kk = 16 * c + 4 * g4 + jj;
                        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(DT[kk * L::PSTR + 16 * rb + l16],
                                                                  Ks[kk * L::STR + col], acc, 0, 0, 0);
                    }
                }
            }
            float *__restrict__ dst = o == 0 ? a.dv : (o == 1 ? a.dk : a.dq);
            const float mul = o == 0 ? 1.0f : a.scale;
            if constexpr (kPersistent) {
                // Branch-free bounded stores (rows past S pushed out of the
                // descriptor's range; lds_dma.h): every path issues the same
                // stores, and the next head's wait skips them.
                const __amdgpu_buffer_rsrc_t rs = store_rsrc(dst + in_base, 4u * (unsigned)((S - 1) * in_ss + D));
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int row = 16 * rb + 4 * g4 + r;
                    store1_bounded(rs, row < S ? 4u * (unsigned)(row * in_ss + col) : kStoreNone, acc[r] * mul);
                }
            } else {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int row = 16 * rb + 4 * g4 + r;
                    if (row < S) dst[in_base + (int64_t)row * in_ss + col] = acc[r] * mul;
                }
            }
        }
    };

    if constexpr (!kPersistent) {
        const int bh = blockIdx.x;
        const int64_t in_base = in_base_of(bh), out_base = out_base_of(bh);
        {
            const __amdgpu_buffer_rsrc_t rq = dma_rsrc(a.q + in_base);
            const __amdgpu_buffer_rsrc_t rk = dma_rsrc(a.k + in_base);
            const __amdgpu_buffer_rsrc_t rv = dma_rsrc(a.v + in_base);
            const __amdgpu_buffer_rsrc_t rg = dma_rsrc(a.dout + out_base);
#pragma unroll
            for (int sl = 0; sl < (L::COP + L::NW - 1) / L::NW; ++sl) {  // copy t = w + NW sl
                const int t = w + L::NW * sl;
                if (t >= L::COP) break;
                const int p = 64 * t + lane;
                int r = p / L::ROWCH;
                const int c = p - r * L::ROWCH;
                const bool real = r < R && c < D / 4;
                r = r < S ? r : S - 1;
                const unsigned oi = real ? 4u * (unsigned)(r * in_ss + 4 * c) : 0u;
                const unsigned og = real ? 4u * (unsigned)(r * out_ss + 4 * c) : 0u;
                dma16_buf(rq, oi, Qs + 256 * t);
                dma16_buf(rk, oi, Ks + 256 * t);
                dma16_buf(rv, oi, Vs + 256 * t);
                dma16_buf(rg, og, Gs + 256 * t);
            }
        }
        {
            const float *__restrict__ orow = a.o + out_base + (int64_t)jr * out_ss;
            const float *__restrict__ grow = a.dout + out_base + (int64_t)jr * out_ss;
            float part = 0.0f;
#pragma unroll
            for (int it = 0; it < CH; ++it) {
                const f32x4 o4 = *(const f32x4 *)(orow + 32 * it + 4 * s8);
                const f32x4 g4v = *(const f32x4 *)(grow + 32 * it + 4 * s8);
                part += o4[0] * g4v[0] + o4[1] * g4v[1] + o4[2] * g4v[2] + o4[3] * g4v[3];
            }
            put_stats(part, a.lse[(int64_t)bh * S + jr]);
        }
        wait_vmem();
        __syncthreads();
        compute(bh);
    } else {
        f32x4 rq[CH], rk[CH], rv[CH], rg[CH], ro[CH];
        float lse_v = 0.0f;
        auto prefetch = [&](int bh) {
            const int64_t ib = in_base_of(bh) + (int64_t)jr * in_ss + 4 * s8;
            const int64_t ob = out_base_of(bh) + (int64_t)jr * out_ss + 4 * s8;
#pragma unroll
            for (int it = 0; it < CH; ++it) {
                rq[it] = *(const f32x4 *)(a.q + ib + 32 * it);
                rk[it] = *(const f32x4 *)(a.k + ib + 32 * it);
                rv[it] = *(const f32x4 *)(a.v + ib + 32 * it);
                rg[it] = *(const f32x4 *)(a.dout + ob + 32 * it);
                ro[it] = *(const f32x4 *)(a.o + ob + 32 * it);
            }
            lse_v = a.lse[(int64_t)bh * S + jr];
        };
        const int stride = (int)gridDim.x;
        int bh = blockIdx.x;
        prefetch(bh);
        // The first head's rows are waited for here, so that the loop's
        // head, where this path and the previous iteration's meet, waits only
        // for those rows and not for the stores behind them.
        wait_vmem();
        for (; bh < nbh; bh += stride) {
            __syncthreads();  // the previous head's products are done with LDS
            float part = 0.0f;
#pragma unroll
            for (int c = 0; c < CH; ++c) {
                const int off = j * L::STR + 32 * c + 4 * s8;
                *(f32x4 *)&Qs[off] = rq[c];
                *(f32x4 *)&Ks[off] = rk[c];
                *(f32x4 *)&Vs[off] = rv[c];
                *(f32x4 *)&Gs[off] = rg[c];
                part += ro[c][0] * rg[c][0] + ro[c][1] * rg[c][1] + ro[c][2] * rg[c][2] + ro[c][3] * rg[c][3];
            }
            put_stats(part, lse_v);
            __syncthreads();
            // Issued after the barrier, so that no wave waits at it for the
            // others' issue (+6.7 % at S = 64, +10.5 % at 48, causal).
            prefetch(bh + stride < nbh ? bh + stride : bh);  // one path: the last head re-reads itself
            compute(bh);
        }
    }
}

template <int D, int R, bool CAUSAL>
int launch_bwd_lds16(const BwdArgs &args, int nbh)
{
    if constexpr (D == 64 || (D == 128 && R == 32)) {
        if (D == 128 || R == 64 || !CAUSAL || args.S < 32) {
            int ncu = 0;
            const int st = device_cus(&ncu);
            if (st != EMBER_OK) return st;
            const int slots = ncu * (D == 128 ? 2 : (R == 32 ? 3 : 1));
            const int grid = nbh < slots ? nbh : slots;
            hipLaunchKernelGGL((attn_bwd_lds16<D, R, CAUSAL, true>), dim3((unsigned)grid), dim3(R * 8), 0, 0, args,
                               nbh);
            return launch_ok(R == 32 ? "attn_bwd_lds16_r32" : "attn_bwd_lds16_r64") ? EMBER_OK : EMBER_ERR_DEVICE;
        }
    }
    if constexpr (!((D == 64 && R == 64) || D == 128))  // (always persistent)
        hipLaunchKernelGGL((attn_bwd_lds16<D, R, CAUSAL, false>), dim3((unsigned)nbh), dim3(R * 8), 0, 0, args,
                           nbh);
    return launch_ok(R == 32 ? "attn_bwd_lds16_r32" : "attn_bwd_lds16_r64") ? EMBER_OK : EMBER_ERR_DEVICE;
}


}  // namespace
}  // namespace ember

// Scratch of the no-allocation entry point: a fixed device array, one per
// GPU (each device that loads this library holds its own copy until the
// process ends).  2^22 floats (16 MiB) of row statistics, i.e. lse2 and
// delta for up to 2^21 padded rows (B * H * S_pad), then 2^17 ints for
// deterministic mode's tile counters (rows_pad / 16).
// Host code never uses this name as an address: the device address comes
// from hipGetSymbolAddress, once per device (noalloc_scratch below).
constexpr size_t kNoAllocStatsFloats = size_t(1) << 22;
constexpr size_t kNoAllocOrderInts = size_t(1) << 17;
static __device__ __align__(256) float scratch[kNoAllocStatsFloats + kNoAllocOrderInts];

// Deterministic mode's count of tile waits that gave up (see
// attention_bwd_kernels.h), one per GPU, zero when the library loads.
static __device__ int order_timeouts[1];

namespace ember {
namespace {

constexpr int kNoAllocDevices = 16;

// Where attention_bwd_rows puts the row statistics (2 * rows_pad floats)
// and, when `ordered`, deterministic mode's tile counters (rows_pad / 16
// ints): sets *stats (and *order) and returns EMBER_OK, or returns the
// status it recorded.
using StatsSource = int (*)(int64_t rows_pad, bool ordered, float **stats, int **order);

int library_stats(int64_t rows_pad, bool ordered, float **stats, int **order)
{
    *stats = (float *)scratch(kScratchAttnDelta, (size_t)rows_pad * 2 * sizeof(float));
    if (!*stats) return EMBER_ERR_OUT_OF_MEMORY;  // scratch() recorded the cause
    if (ordered) {
        *order = (int *)scratch(kScratchAttnOrder, (size_t)(rows_pad / 16) * sizeof(int));
        if (!*order) return EMBER_ERR_OUT_OF_MEMORY;
    }
    return EMBER_OK;
}

// The device address of a __device__ array on the current device, looked up
// once per device and symbol.
std::mutex g_symbol_mu;

template <typename T>
int symbol_address(T **cache, const void *symbol, const char *what, T **out)
{
    int dev = 0;
    if (!hip_ok(hipGetDevice(&dev), "hipGetDevice")) return EMBER_ERR_DEVICE;
    if (dev < 0 || dev >= kNoAllocDevices) return record_error(EMBER_ERR_UNSUPPORTED, what);
    std::lock_guard<std::mutex> lock(g_symbol_mu);
    T **slot = &cache[dev];
    if (!*slot) {
        T *ptr = nullptr;
        const hipError_t err = hipGetSymbolAddress((void **)&ptr, symbol);
        if (err != hipSuccess || !ptr) return record_error(EMBER_ERR_DEVICE, what, err);
        *slot = ptr;
    }
    *out = *slot;
    return EMBER_OK;
}

float *g_noalloc_ptr[kNoAllocDevices];
int *g_timeouts_ptr[kNoAllocDevices];

int timeouts_ptr(int **out)
{
    return symbol_address(g_timeouts_ptr, HIP_SYMBOL(::order_timeouts),
                          "hipGetSymbolAddress(attention_bwd order_timeouts)", out);
}

int noalloc_stats(int64_t rows_pad, bool ordered, float **stats, int **order)
{
    if ((size_t)rows_pad * 2 > kNoAllocStatsFloats)
        return record_error(EMBER_ERR_INVALID_ARGUMENT,
                            "attention_bwd_noalloc: B*H*S_pad (S rounded up to 32) exceeds 2^21 rows");
    float *base = nullptr;
    const int st = symbol_address(g_noalloc_ptr, HIP_SYMBOL(::scratch),
                                  "hipGetSymbolAddress(attention_bwd_noalloc scratch)", &base);
    if (st != EMBER_OK) return st;
    *stats = base;
    if (ordered) *order = (int *)(base + kNoAllocStatsFloats);  // rows_pad / 16 <= 2^21 / 16
    return EMBER_OK;
}

int attention_bwd_rows(const float *q, const float *k, const float *v, const float *o,
                       const float *lse, const float *d_o, float *dq, float *dk, float *dv, int64_t B,
                       int64_t H, int64_t S, int64_t D, float scale, int causal, int64_t in_sb,
                       int64_t in_sh, int64_t in_ss, int64_t out_sb, int64_t out_sh, int64_t out_ss,
                       StatsSource stats_source, const char *who)
{
    const void *ptrs[] = {q, k, v, o, lse, d_o, dq, dk, dv};
    const int64_t strides[] = {in_sb, in_sh, in_ss, out_sb, out_sh, out_ss};
    int st = check_attention_args(ptrs, 9, B, H, S, D, scale, strides, 6, who);
    if (st != EMBER_OK || B * H * S == 0) return st;

    // S <= 64: a workgroup stages one head's Q, K, V and dO in LDS and forms
    // the row statistics itself (no scratch, no atomics):
    // attn_bwd_lds16 with 32- or 64-row tiles at D <= 64 and 32-row tiles
    // at D = 128 (S <= 32), attn_bwd_short_lds64p at D = 128 (S <= 64); the
    // 64-row kernels at D = 64 and 128, which fill a CU's LDS, and most
    // 32-row launches at D = 64 and 128 are persistent and prefetch the next
    // head into registers.  Measured with 2^20
    // query rows: 4.6-4.9 TB/s at S = 32 and 3.7-4.3 TB/s at S = 64 (causal),
    // where the register-fed kernels they replaced (one wave per head or
    // per key block, rows read one per lane from HBM) moved 2.8-3.5 and
    // 2.0-2.1 TB/s.  64 < S <= 128 at D = 64 and 128: attn_bwd_s128, one
    // workgroup per head with 16-key chunks dealt out so that a causal
    // head's waves have equal work, the row statistics formed in the kernel
    // and dQ stored directly (no scratch, no atomics, reproducible).
    if (S <= 2 * kBq || (S <= kBk && D >= 64)) {
        BwdArgs sa;
        sa.q = q;
        sa.k = k;
        sa.v = v;
        sa.o = o;
        sa.lse = lse;
        sa.dout = d_o;
        sa.dq = dq;
        sa.dk = dk;
        sa.dv = dv;
        sa.lse2 = sa.delta = nullptr;
        sa.order = sa.order_timeouts = nullptr;
        sa.order_group = 1;
        sa.H = (int)H;
        sa.S = (int)S;
        sa.S_pad = sa.nkb = 0;
        sa.c = scale * kLog2e;
        sa.scale = scale;
        sa.in_sb = in_sb;
        sa.in_sh = in_sh;
        sa.in_ss = in_ss;
        sa.out_sb = out_sb;
        sa.out_sh = out_sh;
        sa.out_ss = out_ss;
        const int nbh = (int)(B * H);
        if (S > 2 * kBq) return launch_bwd_s128(sa, (int)D, causal != 0, nbh);
        const int key = (S <= kBq ? 0 : 8) + (int)(D / 32) * 2 + (causal ? 1 : 0);
        switch (key) {
            case 2: return launch_bwd_lds16<32, 32, false>(sa, nbh);
            case 3: return launch_bwd_lds16<32, 32, true>(sa, nbh);
            case 4: return launch_bwd_lds16<64, 32, false>(sa, nbh);
            case 5: return launch_bwd_lds16<64, 32, true>(sa, nbh);
            case 8: return launch_bwd_lds16<128, 32, false>(sa, nbh);
            case 9: return launch_bwd_lds16<128, 32, true>(sa, nbh);
            case 10: return launch_bwd_lds16<32, 64, false>(sa, nbh);
            case 11: return launch_bwd_lds16<32, 64, true>(sa, nbh);
            case 12: return launch_bwd_lds16<64, 64, false>(sa, nbh);
            case 13: return launch_bwd_lds16<64, 64, true>(sa, nbh);
            case 16: return launch_bwd_short_lds64p<false>(sa, nbh);
            default: return launch_bwd_short_lds64p<true>(sa, nbh);
        }
    }
    const int64_t S_pad = (S + kBq - 1) / kBq * kBq;
    const int64_t rows_pad = B * H * S_pad;
    const int64_t nkb = (S + kBk - 1) / kBk;
    // Deterministic dq: tile counters (ordered dQ, attention_bwd_kernels.h).
    const bool ordered = deterministic();
    int *order = nullptr, *timeouts = nullptr;
    float *stats = nullptr;
    st = stats_source(rows_pad, ordered, &stats, &order);
    if (st != EMBER_OK) return st;
    if (ordered && (st = timeouts_ptr(&timeouts)) != EMBER_OK) return st;

    BwdArgs args;
    args.q = q;
    args.k = k;
    args.v = v;
    args.o = o;
    args.lse = lse;
    args.dout = d_o;
    args.dq = dq;
    args.dk = dk;
    args.dv = dv;
    args.lse2 = stats;
    args.delta = stats + rows_pad;
    args.order = order;
    args.order_timeouts = timeouts;
    args.order_group = 1;
    if (ordered && causal) {
        // Key blocks per group of the dQ order (attention_bwd_kernels.h): as
        // many as run at once per head, R = slots / heads (B * H rounded up
        // to the 8 XCDs), while the lower R - 1 key blocks of a group leave
        // room for its top key block with a sixteenth of the slots spare.
        // Non-causal walks all start at the first tile, where no key block
        // is ahead of another: R = 1 (ascending).
        const int ncu = device_cu_count();
        const int per_cu = D == 64 ? 4 : D == 32 ? 2 : 1;  // workgroups per CU (LDS, registers)
        const int64_t slots = (int64_t)ncu * per_cu;
        const int64_t heads8 = (B * H + 7) / 8 * 8;
        int64_t R = std::min<int64_t>(nkb, slots / heads8);
        while (R > 1 && (R - 1) * heads8 + 1 > slots - slots / 16) --R;
        args.order_group = (int)std::max<int64_t>(1, R);
    }
    args.H = (int)H;
    args.S = (int)S;
    args.S_pad = (int)S_pad;
    args.nkb = (int)nkb;
    args.c = scale * kLog2e;
    args.scale = scale;
    args.in_sb = in_sb;
    args.in_sh = in_sh;
    args.in_ss = in_ss;
    args.out_sb = out_sb;
    args.out_sh = out_sh;
    args.out_ss = out_ss;
    const int nblocks = args.nkb * (int)(B * H);
    // D = 64: 16-key chunks, four workgroups per CU (attention_bwd_w16.hip);
    // D = 32 and 128: the key-block workgroup kernel.
    if (D == 64) return launch_bwd_w16(args, rows_pad, causal != 0, (int)(B * H));
    switch (D * 2 + (causal ? 1 : 0)) {
        case 64: return launch_bwd<32, false>(args, rows_pad, nblocks);
        case 65: return launch_bwd<32, true>(args, rows_pad, nblocks);
        case 256: return launch_bwd<128, false>(args, rows_pad, nblocks);
        default: return launch_bwd_causal_d128(args, rows_pad, nblocks);
    }
}

}  // namespace
}  // namespace ember

extern "C" int attention_bwd(const float *q, const float *k, const float *v, const float *o,
                             const float *lse, const float *d_o, float *dq, float *dk, float *dv,
                             int64_t B, int64_t H, int64_t S, int64_t D, float scale, int causal,
                             int64_t in_sb, int64_t in_sh, int64_t in_ss, int64_t out_sb,
                             int64_t out_sh, int64_t out_ss)
{
    return ember::attention_bwd_rows(q, k, v, o, lse, d_o, dq, dk, dv, B, H, S, D, scale, causal, in_sb,
                                     in_sh, in_ss, out_sb, out_sh, out_ss, ember::library_stats,
                                     "attention_bwd");
}

// The same computation with the row statistics (and deterministic mode's
// counters) in the fixed array above: no hipMalloc, hipFree or other
// allocating call on any path (the first call on a device looks up the
// array's device address).  Every thread and call on one device shares that
// device's array; the library enqueues all work on the null stream, so calls
// run one after another, and launches of this entry point that overlap on one
// device would race on the array.  Each call writes every statistic and
// counter it reads (attn_bwd_pre fills all 2 * rows_pad floats, padding rows
// included, and zeroes the counters) before reading it, so nothing needs
// clearing.
extern "C" int attention_bwd_noalloc(const float *q, const float *k, const float *v, const float *o,
                                     const float *lse, const float *d_o, float *dq, float *dk,
                                     float *dv, int64_t B, int64_t H, int64_t S, int64_t D,
                                     float scale, int causal, int64_t in_sb, int64_t in_sh,
                                     int64_t in_ss, int64_t out_sb, int64_t out_sh, int64_t out_ss)
{
    return ember::attention_bwd_rows(q, k, v, o, lse, d_o, dq, dk, dv, B, H, S, D, scale, causal, in_sb,
                                     in_sh, in_ss, out_sb, out_sh, out_ss, ember::noalloc_stats,
                                     "attention_bwd_noalloc");
}

// Deterministic mode's tile waits that gave up on the current device since
// the library was loaded (attention_bwd_kernels.h); synchronises the device.
extern "C" int ember_deterministic_timeouts(void)
{
    int *ptr = nullptr;
    if (ember::timeouts_ptr(&ptr) != EMBER_OK) return -1;
    int v = 0;
    if (!ember::hip_ok(hipMemcpy(&v, ptr, sizeof(int), hipMemcpyDeviceToHost), "ember_deterministic_timeouts"))
        return -1;
    return v;
}

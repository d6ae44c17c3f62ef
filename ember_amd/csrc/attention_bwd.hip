// attention_bwd.hip -- fused flash-attention backward (fp32) for gfx950.
//
// No reference counterpart (pawel002/ember has no attention); semantics are
// those of oracle/ember_oracle.c (oracle_attention_bwd): P is recomputed from
// the forward's LSE, never stored.
//
// Two launches on the null stream:
//  1. attn_bwd_pre: delta[i] = <dO_i, O_i> per query row (HBM-bound, one
//     pass over O and dO) and dQ := 0 (dQ is accumulated with atomics).
//  2. attn_bwd_kernel, K/V-stationary: one workgroup = 4 waves = 128 keys
//     of one (b, h); each wave keeps K^T and V^T of its 32 keys resident in
//     registers as MFMA B operands and accumulates dK, dV for them in
//     registers.  The workgroup walks query blocks of 32 (causal: only the
//     blocks at or below its keys), staging Q and dO in LDS:
//        S  = Q K^T, dP = dO V^T           (C[m][n], keys on lanes)
//        P  = exp2(S*c - lse2[m]), dS = P * (dP - delta[m])
//        dV += P^T dO,  dK += dS^T Q       (P / dS registers are the A
//                                           operands directly)
//     dS of all 4 waves goes through LDS so that dQ(32 x D) = dS . K over the
//     workgroup's 128 keys is one more MFMA product per wave, added to the
//     global dQ with hardware fp32 atomics (dq must be device memory).
#include <math.h>

#include "common.h"
#include "mfma.h"

namespace ember {

int check_attention_args(const void *const *ptrs, int nptrs, int64_t B, int64_t H, int64_t S,
                         int64_t D, const int64_t *strides, int nstrides, const char *who);

namespace {

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kBkw = 32;            // keys per wave
constexpr int kBk = kBkw * kWaves;  // keys per workgroup
constexpr int kBq = 32;             // queries per step
constexpr float kLog2e = 1.4426950408889634f;

struct BwdArgs {
    const float *q, *k, *v, *o, *lse, *dout;
    float *dq, *dk, *dv, *delta;
    int H, S, nkb;
    float c;      // scale * log2(e)
    float scale;
    int64_t in_sb, in_sh, in_ss, out_sb, out_sh, out_ss;
};

// delta = rowsum(dO * O); dQ row := 0.  D/4 threads per row.
template <int D>
__global__ __launch_bounds__(256) void attn_bwd_pre(BwdArgs a, int64_t rows)
{
    constexpr int TPR = D / 4;
    constexpr int RPB = 256 / TPR;
    const int sub = threadIdx.x % TPR;
    const int64_t row = (int64_t)blockIdx.x * RPB + threadIdx.x / TPR;
    if (row >= rows) return;  // whole TPR-lane groups retire together
    const int64_t bh = row / a.S;
    const int m = (int)(row - bh * a.S);
    const int b = (int)(bh / a.H);
    const int hh = (int)(bh - (int64_t)b * a.H);
    const int64_t ooff = (int64_t)b * a.out_sb + (int64_t)hh * a.out_sh + (int64_t)m * a.out_ss + 4 * sub;
    const f32x4 ov = *(const f32x4 *)(a.o + ooff);
    const f32x4 gv = *(const f32x4 *)(a.dout + ooff);
    float s = ov[0] * gv[0] + ov[1] * gv[1] + ov[2] * gv[2] + ov[3] * gv[3];
#pragma unroll
    for (int off = TPR / 2; off > 0; off >>= 1) s += __shfl_xor(s, off);
    if (sub == 0) a.delta[row] = s;
    const int64_t qoff = (int64_t)b * a.in_sb + (int64_t)hh * a.in_sh + (int64_t)m * a.in_ss + 4 * sub;
    *(f32x4 *)(a.dq + qoff) = f32x4{0.f, 0.f, 0.f, 0.f};
}

template <int D, bool CAUSAL>
__global__ __launch_bounds__(kThreads, 1) void attn_bwd_kernel(BwdArgs a)
{
    constexpr int DH = D / 2;
    constexpr int DB = D / 32;
    constexpr int QSTR = D + 4;        // padded Q / dO rows
    constexpr int SSTR = kBk + 4;      // padded dS rows
    constexpr int NSPLIT = 4 / DB;     // waves sharing one 32-wide d block of dQ
    constexpr int NK = kBk / NSPLIT;   // keys each wave contracts for dQ
    constexpr int NKH = NK / 2;        // ... per lane half
    // K of the workgroup for the dQ product.  Row n starts at
    // n*D + (n/NKH)*32: rows NKH apart (read by the two lane halves at the
    // same k-step) land 32 banks apart, and the shift never decreases, so
    // rows do not overlap.
    constexpr int KALL = kBk * D + (kBk / NKH) * 32;
    __shared__ float Kall[KALL];
    __shared__ float Qs[kBq * QSTR];
    __shared__ float dOs[kBq * QSTR];
    __shared__ float dSs[kBq * SSTR];
    __shared__ float lse2s[kBq];
    __shared__ float dlts[kBq];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int w = tid >> 6;
    const int h32 = lane >> 5;
    const int l32 = lane & 31;

    const int BH = (int)(gridDim.x / a.nkb);
    const int kb = blockIdx.x / BH;  // ascending: the longest causal rows first
    const int bh = blockIdx.x - kb * BH;
    const int b = bh / a.H;
    const int hh = bh - b * a.H;
    const int S = a.S;
    const int n0 = kb * kBk;
    const int n0w = n0 + kBkw * w;
    const int nl = n0w + l32;

    const int64_t in_base = (int64_t)b * a.in_sb + (int64_t)hh * a.in_sh;
    const int64_t out_base = (int64_t)b * a.out_sb + (int64_t)hh * a.out_sh;

    // Resident B operands: lane holds K[nl][h32*DH + kk] and V[nl][...].
    float kr[DH], vr[DH];
    {
        const int nrow = nl < S ? nl : S - 1;
        const float *ks = a.k + in_base + (int64_t)nrow * a.in_ss + h32 * DH;
        const float *vs = a.v + in_base + (int64_t)nrow * a.in_ss + h32 * DH;
#pragma unroll
        for (int kk = 0; kk < DH; kk += 4) {
            const f32x4 t = *(const f32x4 *)(ks + kk);
            const f32x4 u = *(const f32x4 *)(vs + kk);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                kr[kk + j] = t[j];
                vr[kk + j] = u[j];
            }
        }
    }
    // K tile of the whole workgroup into LDS (zeros past the sequence end).
#pragma unroll
    for (int it = 0; it < kBk * D / 4 / kThreads; ++it) {
        const int idx = it * kThreads + tid;
        const int r = idx / (D / 4);
        const int c4 = idx - r * (D / 4);
        const int n = n0 + r;
        f32x4 kv = {0.f, 0.f, 0.f, 0.f};
        if (n < S) kv = *(const f32x4 *)(a.k + in_base + (int64_t)n * a.in_ss + 4 * c4);
        *(f32x4 *)&Kall[r * D + (r / NKH) * 32 + 4 * c4] = kv;
    }

    f32x16 dvacc[DB], dkacc[DB];
#pragma unroll
    for (int db = 0; db < DB; ++db) {
        dvacc[db] = zero16();
        dkacc[db] = zero16();
    }

    const int nq = (S + kBq - 1) / kBq;
    const int qstart = CAUSAL ? n0 / kBq : 0;
    const bool key_tail = n0w + kBkw > S;
    const int dblk = w % DB;
    const int nbase = (w / DB) * NK;

    for (int qb = qstart; qb < nq; ++qb) {
        const int m0 = qb * kBq;
        __syncthreads();
#pragma unroll
        for (int it = 0; it < kBq * D / 4 / kThreads; ++it) {
            const int idx = it * kThreads + tid;
            const int r = idx / (D / 4);
            const int c4 = idx - r * (D / 4);
            const int m = m0 + r;
            f32x4 qv = {0.f, 0.f, 0.f, 0.f}, gv = {0.f, 0.f, 0.f, 0.f};
            if (m < S) {
                qv = *(const f32x4 *)(a.q + in_base + (int64_t)m * a.in_ss + 4 * c4);
                gv = *(const f32x4 *)(a.dout + out_base + (int64_t)m * a.out_ss + 4 * c4);
            }
            *(f32x4 *)&Qs[r * QSTR + 4 * c4] = qv;
            *(f32x4 *)&dOs[r * QSTR + 4 * c4] = gv;
        }
        if (tid < kBq) {
            const int m = m0 + tid;
            // Rows past the end get lse = +inf, so their P is exactly 0.
            lse2s[tid] = m < S ? a.lse[(int64_t)bh * S + m] * kLog2e : INFINITY;
            dlts[tid] = m < S ? a.delta[(int64_t)bh * S + m] : 0.0f;
        }
        __syncthreads();

        const bool active = !CAUSAL || n0w <= m0 + kBq - 1;
        if (active) {
            f32x16 sacc = zero16(), pacc = zero16();
#pragma unroll
            for (int kk = 0; kk < DH; kk += 4) {
                const f32x4 qf = *(const f32x4 *)&Qs[l32 * QSTR + h32 * DH + kk];
                const f32x4 gf = *(const f32x4 *)&dOs[l32 * QSTR + h32 * DH + kk];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    sacc = mfma_32x32x2(qf[j], kr[kk + j], sacc);
                    pacc = mfma_32x32x2(gf[j], vr[kk + j], pacc);
                }
            }
            const bool need_mask = key_tail || (CAUSAL && n0w + kBkw - 1 > m0);
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int r = acc_row(i, h32);
                float p = exp2f(sacc[i] * a.c - lse2s[r]);
                if (need_mask && (nl >= S || (CAUSAL && nl > m0 + r))) p = 0.0f;
                sacc[i] = p;                      // P[m][n]
                pacc[i] = p * (pacc[i] - dlts[r]);  // dS[m][n]
            }
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int r = acc_row(i, h32);
                const typename VecN<DB>::T gf = *(const typename VecN<DB>::T *)&dOs[r * QSTR + DB * l32];
                const typename VecN<DB>::T qf = *(const typename VecN<DB>::T *)&Qs[r * QSTR + DB * l32];
#pragma unroll
                for (int db = 0; db < DB; ++db) {
                    dvacc[db] = mfma_32x32x2(sacc[i], vget<DB>(gf, db), dvacc[db]);
                    dkacc[db] = mfma_32x32x2(pacc[i], vget<DB>(qf, db), dkacc[db]);
                }
            }
#pragma unroll
            for (int i = 0; i < 16; ++i) dSs[acc_row(i, h32) * SSTR + kBkw * w + l32] = pacc[i];
        } else {
#pragma unroll
            for (int i = 0; i < 16; ++i) dSs[acc_row(i, h32) * SSTR + kBkw * w + l32] = 0.0f;
        }
        __syncthreads();

        // dQ[m0:m0+32, 32*dblk : 32*dblk+32] += scale * dS . K over this wave's key range.
        f32x16 qacc = zero16();
#pragma unroll
        for (int kk = 0; kk < NKH; kk += 4) {
            const f32x4 sf = *(const f32x4 *)&dSs[l32 * SSTR + nbase + h32 * NKH + kk];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int n = nbase + h32 * NKH + kk + j;
                const float kf = Kall[n * D + (n / NKH) * 32 + 32 * dblk + l32];
                qacc = mfma_32x32x2(sf[j], kf, qacc);
            }
        }
        float *dqb = a.dq + in_base + 32 * dblk + l32;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int m = m0 + acc_row(i, h32);
            if (m < S) unsafeAtomicAdd(dqb + (int64_t)m * a.in_ss, qacc[i] * a.scale);
        }
    }

    // dK (scaled) and dV rows of this wave's keys: register i -> key
    // n0w + acc_row(i, h32), lane -> d = DB*l32 + db.
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int n = n0w + acc_row(i, h32);
        if (n >= S) continue;
        float *dkrow = a.dk + in_base + (int64_t)n * a.in_ss + DB * l32;
        float *dvrow = a.dv + in_base + (int64_t)n * a.in_ss + DB * l32;
        typename VecN<DB>::T kout, vout;
        if constexpr (DB == 1) {
            kout = dkacc[0][i] * a.scale;
            vout = dvacc[0][i];
        } else {
#pragma unroll
            for (int db = 0; db < DB; ++db) {
                kout[db] = dkacc[db][i] * a.scale;
                vout[db] = dvacc[db][i];
            }
        }
        *(typename VecN<DB>::T *)dkrow = kout;
        *(typename VecN<DB>::T *)dvrow = vout;
    }
}

template <int D, bool CAUSAL>
int launch_bwd(const BwdArgs &args, int64_t rows, int nblocks)
{
    constexpr int RPB = 256 / (D / 4);
    const int pre_blocks = (int)((rows + RPB - 1) / RPB);
    hipLaunchKernelGGL((attn_bwd_pre<D>), dim3(pre_blocks), dim3(256), 0, 0, args, rows);
    if (!launch_ok("attn_bwd_pre")) return EMBER_ERR_DEVICE;
    hipLaunchKernelGGL((attn_bwd_kernel<D, CAUSAL>), dim3(nblocks), dim3(kThreads), 0, 0, args);
    return launch_ok("attn_bwd_kernel") ? EMBER_OK : EMBER_ERR_DEVICE;
}

}  // namespace
}  // namespace ember

extern "C" int attention_bwd(const float *q, const float *k, const float *v, const float *o,
                             const float *lse, const float *d_o, float *dq, float *dk, float *dv,
                             int64_t B, int64_t H, int64_t S, int64_t D, float scale, int causal,
                             int64_t in_sb, int64_t in_sh, int64_t in_ss, int64_t out_sb,
                             int64_t out_sh, int64_t out_ss)
{
    using namespace ember;
    const void *ptrs[] = {q, k, v, o, lse, d_o, dq, dk, dv};
    const int64_t strides[] = {in_sb, in_sh, in_ss, out_sb, out_sh, out_ss};
    int st = check_attention_args(ptrs, 9, B, H, S, D, strides, 6, "attention_bwd");
    if (st != EMBER_OK || B * H * S == 0) return st;

    const int64_t rows = B * H * S;
    float *delta = (float *)scratch(kScratchAttnDelta, (size_t)rows * sizeof(float));
    if (!delta) return EMBER_ERR_OUT_OF_MEMORY;

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
    args.delta = delta;
    args.H = (int)H;
    args.S = (int)S;
    args.nkb = (int)((S + kBk - 1) / kBk);
    args.c = scale * kLog2e;
    args.scale = scale;
    args.in_sb = in_sb;
    args.in_sh = in_sh;
    args.in_ss = in_ss;
    args.out_sb = out_sb;
    args.out_sh = out_sh;
    args.out_ss = out_ss;
    const int nblocks = args.nkb * (int)(B * H);
    switch (D * 2 + (causal ? 1 : 0)) {
        case 64: return launch_bwd<32, false>(args, rows, nblocks);
        case 65: return launch_bwd<32, true>(args, rows, nblocks);
        case 128: return launch_bwd<64, false>(args, rows, nblocks);
        case 129: return launch_bwd<64, true>(args, rows, nblocks);
        case 256: return launch_bwd<128, false>(args, rows, nblocks);
        default: return launch_bwd<128, true>(args, rows, nblocks);
    }
}

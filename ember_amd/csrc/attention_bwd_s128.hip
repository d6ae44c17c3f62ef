// attention_bwd_s128.hip -- the fused attention backward for sequences of 65
// to 128 rows at head_dim 64 and 128 (attn_bwd_s128).
//
// No reference counterpart (pawel002/ember has no attention); semantics are
// those of oracle/ember_oracle.c (oracle_attention_bwd).
//
// Why a kernel of its own.  The key-block workgroup kernel
// (attention_bwd_kernels.h) gives each of its 4 waves 32 keys and walks
// 32-query blocks in lockstep; at S = 128 that is one workgroup per head in
// which, causally, wave 0 has work in all 4 steps and wave 3 in one, so a
// causal head costs as much as a non-causal one (measured 1.98 against
// 2.00 ms at B128 H64 D128).  Here the keys are cut into 16-row chunks and
// every product runs on v_mfma_f32_16x16x4f32, so that masked work is cut at
// 16 x 16 and the chunks can be dealt out evenly: a causal chunk j is seen
// by 8 - j of the 8 query chunks, and the chunks j and 7 - j together by 9,
// so each wave (or each SIMD) holds such a pair.
//
// One workgroup per head; wave w keeps K and V of its key chunks resident in
// registers (B operands of S = Q K^T and dP = dO V^T) and accumulates dK, dV
// for them in registers:
//   D = 128: 8 waves, one chunk each; waves w and w + 4 share a SIMD and
//     hold chunks w and 7 - w (2 waves per SIMD, one workgroup per CU,
//     136 KB of LDS);
//   D = 64: 4 waves, chunks w and 7 - w each (76 KB of LDS, two workgroups
//     per CU, which also overlap one head's loads with another's products).
// The workgroup walks 16-query chunks qc in lockstep, with the next chunk's
// Q, dO and O rows copied HBM -> LDS (global_load_lds_dwordx4, no registers)
// into the second of two buffers while the current one is multiplied:
//   S, dP of each active (key chunk, qc) pair; delta = <dO, O> of the 16
//     rows, formed by every wave from the LDS rows (no separate pass, no
//     extra barrier); P = exp2(S*c - lse2), dS = P * (dP - delta), masked at
//     the diagonal and past S;
//   dV += P^T dO, dK += dS^T Q (the P / dS accumulators are the A operands
//     directly); dS to LDS;
//   barrier; dQ of chunk qc = scale * dS . K over all keys at or before it,
//     one 16-column block per wave, K read transposed from LDS; stored
//     straight to dq (every element written once: no atomics, no scratch,
//     reproducible).
// lse2 of all rows is formed once per head into LDS (rows past S: +inf, so
// their P is exactly 0; their Q, dO, O rows re-read row S-1).
#include "attention_bwd_kernels.h"

namespace ember {
namespace {

template <int D>
struct S128Shape {
    static constexpr int NW = D == 128 ? 8 : 4;          // waves per workgroup
    static constexpr int NC = 8 / NW;                    // 16-key chunks per wave
    static constexpr int DH = D / 4;                     // k-steps of an S block per lane group
    static constexpr int STR = D + 4;                    // padded row of a chunk tile
    static constexpr int ROWCH = STR / 4;                // 16-byte pieces per padded row
    static constexpr int COP = (48 * ROWCH + 63) / 64;   // 1 KiB copies per chunk set (Q, dO, O)
    static constexpr int SET = COP * 256;                // floats per chunk set
    static constexpr int SLOTS = (COP + NW - 1) / NW;    // copies per wave
    static constexpr int XSTR = 128 + 4;                 // padded row of dS (16 x 128) and K^T (D x 128)
    static constexpr int NH = D / 64;                    // 64-column halves of a row
};

// Sum over the 16 lanes of a row (lanes 16g .. 16g + 15).
__device__ __forceinline__ float row16_sum(float x)
{
    x += __shfl_xor(x, 1);
    x += __shfl_xor(x, 2);
    x += __shfl_xor(x, 4);
    x += __shfl_xor(x, 8);
    return x;
}

__device__ __forceinline__ f32x4 mfma16(float a, float b, f32x4 c)
{
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// 16 x 16 x 4 operand placement (lane l = n + 16 g, n = l % 16, g = l / 16):
// A[m][k] is lane m + 16k, B[k][n] lane n + 16k, and C[m][n] lane n + 16(m/4),
// register m % 4.  The contraction index of a k-step is free, so:
//   S = Q K^T:  lane (n, g) supplies Q[n][DH g + s] and K[n][DH g + s] at
//     k-step s (Q rows read as 128-bit LDS segments, K resident);
//   dV += P^T dO: register r of the P accumulator (P[4g + r][n]) is the A
//     operand of the k-step that contracts query 4g + r; lane (n, g) reads
//     dO[4g + r][64h + 4n + j] as the B operand of column block 4h + j, so
//     column n of accumulator block 4h + j is d = 64h + 4n + j (four blocks
//     from one 128-bit read, and a 128-bit store per row at the end);
//   dQ = dS K: lane (n, g) reads dS[n][16c + 4g + j] and K^T[16w + n][16c + 4g + j]
//     for k-step j of key chunk c (both 128-bit reads).
template <int D, bool CAUSAL>
__global__ __launch_bounds__(S128Shape<D>::NW * 64, D == 128 ? 1 : 2) void attn_bwd_s128(BwdArgs a)
{
    typedef S128Shape<D> L;
    constexpr int NW = L::NW, NC = L::NC, DH = L::DH, STR = L::STR, XSTR = L::XSTR, NH = L::NH;
    constexpr int NB = D / 16;  // 16-column blocks of dV / dK
    __shared__ float sets[2 * L::SET];      // chunk tiles: rows 0-15 Q, 16-31 dO, 32-47 O
    __shared__ float dsb[2 * 16 * XSTR];    // dS of a query chunk, alternate chunks alternate halves
    __shared__ float Kt[D * XSTR];          // K^T of the head
    __shared__ float L2s[128];              // lse2 per row

    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n = lane & 15, g = lane >> 4;
    const int S = a.S;
    const int nch = (S + 15) >> 4;
    const int bh = blockIdx.x;
    const int b = bh / a.H, hh = bh - b * a.H;
    const int64_t in_base = (int64_t)b * a.in_sb + (int64_t)hh * a.in_sh;
    const int64_t out_base = (int64_t)b * a.out_sb + (int64_t)hh * a.out_sh;
    const int in_ss = (int)a.in_ss, out_ss = (int)a.out_ss;  // < 2^24 (checked on the host)

    // This wave's key chunks, ascending (so the active ones form a prefix).
    int kc[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) kc[c] = NC == 1 ? (w < 4 ? w : 11 - w) : (c == 0 ? w : 7 - w);

    // Resident K and V: lane (n, g) holds K[16 kc + n][DH g + s], s < DH.
    float kr[NC][DH], vr[NC][DH];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const int row = min(16 * kc[c] + n, S - 1);
        const float *__restrict__ ks = a.k + in_base + (int64_t)row * in_ss + DH * g;
        const float *__restrict__ vs = a.v + in_base + (int64_t)row * in_ss + DH * g;
#pragma unroll
        for (int s = 0; s < DH; s += 4) {
            const f32x4 t = *(const f32x4 *)(ks + s);
            const f32x4 u = *(const f32x4 *)(vs + s);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                kr[c][s + j] = t[j];
                vr[c][s + j] = u[j];
            }
        }
    }
    // K^T for the dQ product (chunks past S are never read).
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        if (16 * kc[c] < S) {
#pragma unroll
            for (int s = 0; s < DH; ++s) Kt[(DH * g + s) * XSTR + 16 * kc[c] + n] = kr[c][s];
        }
    }
    for (int t = threadIdx.x; t < 128; t += NW * 64)
        L2s[t] = t < S ? a.lse[(int64_t)bh * S + t] * kLog2e : INFINITY;

    // Copies chunk qc's Q, dO and O rows into a set: copy t fills 16-byte
    // pieces 64t .. 64t + 63 of the 48 padded rows; a padding or slack piece
    // re-reads the head's first Q piece (valid memory, never used).
    auto fetch = [&](int qc, float *dst) {
        const int m0 = 16 * qc;
#pragma unroll
        for (int sl = 0; sl < L::SLOTS; ++sl) {
            const int t = w + NW * sl;
            if (t < L::COP) {
                const int p = 64 * t + lane;
                const int row = p / L::ROWCH, c4 = p - row * L::ROWCH;
                const int tensor = row >> 4;  // 0 Q, 1 dO, 2 O, 3 slack
                const int r = min(m0 + (row & 15), S - 1);
                const float *src = a.q + in_base;
                if (tensor < 3 && c4 < D / 4) {
                    if (tensor == 0)
                        src += (int64_t)r * in_ss + 4 * c4;
                    else
                        src = (tensor == 1 ? a.dout : a.o) + out_base + (int64_t)r * out_ss + 4 * c4;
                }
                dma16(src, dst + 256 * t);
            }
        }
    };

    f32x4 dvacc[NC][NB], dkacc[NC][NB];
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
        for (int db = 0; db < NB; ++db) {
            dvacc[c][db] = f32x4{0.f, 0.f, 0.f, 0.f};
            dkacc[c][db] = f32x4{0.f, 0.f, 0.f, 0.f};
        }

    // delta of rows 4g + r of the chunk set: each lane of a row group sums
    // its D/16 columns (the pieces of dO it reads again for dV), then the
    // group sums.
    auto row_delta = [&](const float *__restrict__ cur, float (&dl)[4]) {
        const float *__restrict__ Gs = cur + 16 * STR;
        const float *__restrict__ Os = cur + 32 * STR;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            float part = 0.0f;
#pragma unroll
            for (int h = 0; h < NH; ++h) {
                const int off = (4 * g + r) * STR + 64 * h + 4 * n;
                const f32x4 o4 = *(const f32x4 *)&Os[off];
                const f32x4 g4 = *(const f32x4 *)&Gs[off];
                part += o4[0] * g4[0] + o4[1] * g4[1] + o4[2] * g4[2] + o4[3] * g4[3];
            }
            dl[r] = row16_sum(part);
        }
    };

    // The products of query chunk qc with key chunk slot C (one slot at a
    // time: at D = 64 a wave holding both slots' operands at once spills).
    auto products = [&](auto slot, int qc, const float *__restrict__ cur, float *__restrict__ ds,
                        const float (&dl)[4], const f32x4 &l2) {
        constexpr int C = decltype(slot)::value;
        const float *__restrict__ Qs = cur;
        const float *__restrict__ Gs = cur + 16 * STR;
        f32x4 sacc = {0.f, 0.f, 0.f, 0.f}, pacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s0 = 0; s0 < DH; s0 += 4) {
            const f32x4 qf = *(const f32x4 *)&Qs[n * STR + DH * g + s0];
            const f32x4 gf = *(const f32x4 *)&Gs[n * STR + DH * g + s0];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                sacc = mfma16(qf[j], kr[C][s0 + j], sacc);
                pacc = mfma16(gf[j], vr[C][s0 + j], pacc);
            }
        }
        // P and dS; masked (P = 0) where key > query on the diagonal chunk
        // and for keys past S: an integer threshold per lane, row r masked
        // when thr > r.
        int thr = CAUSAL && kc[C] == qc ? n - 4 * g : -1;
        if (16 * kc[C] + n >= S) thr = 1 << 20;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            float p = __builtin_amdgcn_exp2f(fmaf(sacc[r], a.c, -l2[r]));
            p = thr > r ? 0.0f : p;
            sacc[r] = p;
            pacc[r] = p * (pacc[r] - dl[r]);
            ds[(4 * g + r) * XSTR + 16 * kc[C] + n] = pacc[r];
        }
        // dV += P^T dO, dK += dS^T Q.
#pragma unroll
        for (int r = 0; r < 4; ++r) {
#pragma unroll
            for (int h = 0; h < NH; ++h) {
                const int off = (4 * g + r) * STR + 64 * h + 4 * n;
                const f32x4 gb = *(const f32x4 *)&Gs[off];
                const f32x4 qb = *(const f32x4 *)&Qs[off];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    dvacc[C][4 * h + j] = mfma16(sacc[r], gb[j], dvacc[C][4 * h + j]);
                    dkacc[C][4 * h + j] = mfma16(pacc[r], qb[j], dkacc[C][4 * h + j]);
                }
            }
        }
    };

    fetch(0, sets);
    wait_vmem();
    __syncthreads();

    for (int qc = 0; qc < nch; ++qc) {
        const int st = qc & 1;
        const float *__restrict__ cur = sets + st * L::SET;
        float *__restrict__ ds = dsb + st * 16 * XSTR;
        if (qc + 1 < nch) fetch(qc + 1, sets + (st ^ 1) * L::SET);
        // Active chunks: inside the sequence and (causal) at or before qc.
        int nact = 0;
#pragma unroll
        for (int c = 0; c < NC; ++c)
            if (16 * kc[c] < S && (!CAUSAL || kc[c] <= qc)) nact = c + 1;
        if (nact > 0) {
            float dl[4];
            row_delta(cur, dl);
            const f32x4 l2 = *(const f32x4 *)&L2s[16 * qc + 4 * g];
            products(std::integral_constant<int, 0>{}, qc, cur, ds, dl, l2);
            if constexpr (NC == 2) {
                if (nact == 2) products(std::integral_constant<int, 1>{}, qc, cur, ds, dl, l2);
            }
        }
        wait_vmem();      // this wave's copies of chunk qc + 1 have landed
        __syncthreads();  // dS of chunk qc and all of chunk qc + 1 are in LDS

        // dQ rows 16 qc .. of columns 16w .. 16w + 15, over key chunks
        // 0 .. qc (causal) or all of them.
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
        const int klast = CAUSAL ? qc : nch - 1;
        for (int c = 0; c <= klast; ++c) {
            const f32x4 af = *(const f32x4 *)&ds[n * XSTR + 16 * c + 4 * g];
            const f32x4 bf = *(const f32x4 *)&Kt[(16 * w + n) * XSTR + 16 * c + 4 * g];
#pragma unroll
            for (int j = 0; j < 4; ++j) acc = mfma16(af[j], bf[j], acc);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int row = 16 * qc + 4 * g + r;
            if (row < S) a.dq[in_base + (int64_t)row * in_ss + 16 * w + n] = acc[r] * a.scale;
        }
    }

    // dK (scaled) and dV rows of this wave's keys: register r of block
    // 4h + j holds key 16 kc + 4g + r, column 64h + 4n + j.
#pragma unroll
    for (int c = 0; c < NC; ++c) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int key = 16 * kc[c] + 4 * g + r;
            if (key >= S) continue;
            float *dkrow = a.dk + in_base + (int64_t)key * in_ss + 4 * n;
            float *dvrow = a.dv + in_base + (int64_t)key * in_ss + 4 * n;
#pragma unroll
            for (int h = 0; h < NH; ++h) {
                f32x4 ko, vo;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    ko[j] = dkacc[c][4 * h + j][r] * a.scale;
                    vo[j] = dvacc[c][4 * h + j][r];
                }
                *(f32x4 *)(dkrow + 64 * h) = ko;
                *(f32x4 *)(dvrow + 64 * h) = vo;
            }
        }
    }
}

template <int D, bool CAUSAL>
int launch_s128(const BwdArgs &args, int nbh)
{
    hipLaunchKernelGGL((attn_bwd_s128<D, CAUSAL>), dim3((unsigned)nbh), dim3(S128Shape<D>::NW * 64), 0, 0,
                       args);
    return launch_ok("attn_bwd_s128") ? EMBER_OK : EMBER_ERR_DEVICE;
}

}  // namespace

int launch_bwd_s128(const BwdArgs &args, int D, bool causal, int nbh)
{
    if (D == 128) return causal ? launch_s128<128, true>(args, nbh) : launch_s128<128, false>(args, nbh);
    return causal ? launch_s128<64, true>(args, nbh) : launch_s128<64, false>(args, nbh);
}

}  // namespace ember

// attention_bwd_w16.hip -- the fused attention backward for S > 128 at
// head_dim 64, in 16-key chunks (attn_bwd_w16).
//
// No reference counterpart (pawel002/ember has no attention); semantics are
// those of oracle/ember_oracle.c (oracle_attention_bwd).
//
// The key-block kernel (attention_bwd_kernels.h) gives each of its 4 waves 32
// keys on v_mfma_f32_32x32x2f32 and walks 32-query blocks; at D = 64 it takes
// 272 registers per lane and 104 KB of LDS, so a CU runs one workgroup, one
// wave per SIMD, every wait in a step (barriers, LDS latency, the atomics'
// issue) idles the matrix core, and causally each workgroup computes 128 x
// 128 diagonal scores of which half are masked.  Here a workgroup holds 64
// keys, one 16-key chunk per wave on v_mfma_f32_16x16x4f32 (the same rate per
// flop): K, V, dK, dV of a chunk take 4 x 16 registers per lane (126 in
// all), and the LDS holds two 16-query chunk sets, the dS of one chunk and
// K^T of the 64 keys (39 KB), so four independent workgroups share a CU and
// fill each other's waits, and masked work is cut at 16 x 16.  (Three per CU
// with a second dS buffer and one barrier per step measured 3-6 % slower.)  At D = 128 the same design
// (188 registers, 79 KB, two workgroups per CU) measured 5-7 % slower than
// the key-block kernel, which keeps that case.
//
// Per step qc (16 query rows), as attn_bwd_s128:
//   dQ of chunk qc - 2 (formed in the previous step) added into dq;
//   chunk qc + 1 (Q, dO rows; lse2, delta from attn_bwd_pre) copied HBM ->
//     LDS into the other set;
//   dQ of chunk qc - 1 = dS . K over the workgroup's keys at or before it,
//     D/4 columns per wave, dS and K^T from LDS;
//   barrier (every wave has read dS of chunk qc - 1);
//   S, dP of this wave's (key chunk, qc) pair when active; P = exp2(S*c -
//     lse2), dS = P * (dP - delta), masked at the diagonal and past S; dS to
//     LDS; dV += P^T dO, dK += dS^T Q with the P / dS accumulators as the A
//     operands;
//   barrier.
// dQ goes out with atomics; in deterministic mode with the same atomics in a
// fixed key-block order per 16-row chunk (ordered dQ,
// attention_bwd_kernels.h): the chunk's counter is polled a step before the
// adds, which wait for it to show the key blocks before this one.
#include "attention_bwd_kernels.h"

namespace ember {
namespace {

template <int D>
struct W16Shape {
    static constexpr int NW = 4;                          // waves per workgroup, one 16-key chunk each
    static constexpr int KB = 16 * NW;                    // keys per workgroup
    static constexpr int DH = D / 4;                      // k-steps of an S block per lane group
    static constexpr int STR = D + 4;                     // padded row of a chunk tile
    static constexpr int ROWCH = STR / 4;                 // 16-byte pieces per padded row
    static constexpr int TCOP = (16 * ROWCH + 63) / 64;   // 1 KiB copies per 16-row tile
    static constexpr int TILE = 16 * STR;                 // floats per tile (a copy's lanes past it are masked)
    static constexpr int SET = 2 * TILE + 32;             // Q and dO tiles, then lse2 and delta of 16 rows
    static constexpr int SL = (TCOP + 1) / 2;             // copies per wave (two waves per tile)
    static constexpr int XSTR = KB + 4;                   // padded row of dS (16 x KB) and K^T (D x KB)
    static constexpr int NH = D / 64;                     // 64-column halves of a row
    static constexpr int NB = D / 16;                     // 16-column blocks of dV / dK
    static constexpr int QB = NB / NW;                    // 16-column blocks of dQ per wave
};

__device__ __forceinline__ f32x4 mfma16(float a, float b, f32x4 c)
{
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// 16 x 16 x 4 operand placement (lane l = n + 16 g): A[m][k] is lane m + 16k,
// B[k][n] lane n + 16k, C[m][n] lane n + 16(m/4), register m % 4.
//   S = Q K^T: lane (n, g) supplies Q[n][DH g + s] and K[n][DH g + s] at k-step s;
//   dV += P^T dO: register r of the P accumulator (P[4g + r][n]) is the A
//     operand of the k-step that contracts query 4g + r; lane (n, g) reads
//     dO[4g + r][64h + 4n + j] as the B operand of column block 4h + j;
//   dQ = dS K: lane (n, g) reads dS[n][16c + 4g + j] and K^T[d][16c + 4g + j].
template <int D, bool CAUSAL, int DQ, bool PAIRK>
__global__ __launch_bounds__(256, 4) void attn_bwd_w16(BwdArgs a, int nkb)
{
    typedef W16Shape<D> L;
    constexpr int NW = L::NW, DH = L::DH, STR = L::STR, XSTR = L::XSTR, NH = L::NH, NB = L::NB,
                  QB = L::QB, CPW = L::KB / 16;
    __shared__ float sets[2 * L::SET];    // two chunk sets
    __shared__ float dsb[16 * XSTR];      // dS of a query chunk
    __shared__ float Kt[D * XSTR];        // K^T of the workgroup's keys

    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n = lane & 15, g = lane >> 4;
    const int S = a.S;
    const int nch = (S + 15) >> 4;
    // PAIRK (causal, atomic dQ): key blocks p and nkb - 1 - p of a head, one
    // after the other, so that every workgroup walks about 2 nch - 4 nkb
    // query chunks (the middle block of an odd nkb alone, dispatched last).
    static_assert(!PAIRK || DQ == kDqAtomic, "the ordered dQ follows single key blocks");
    const int per_head = PAIRK ? (nkb + 1) / 2 : nkb;
    const int BH = (int)(gridDim.x / per_head);
    const int kb0 = blockIdx.x / BH;  // ascending: the longest causal walks first
    const int bh = blockIdx.x - kb0 * BH;
    const int b = bh / a.H;
    const int hh = bh - b * a.H;
    const int64_t in_base = (int64_t)b * a.in_sb + (int64_t)hh * a.in_sh;
    const int64_t out_base = (int64_t)b * a.out_sb + (int64_t)hh * a.out_sh;
    const int in_ss = (int)a.in_ss, out_ss = (int)a.out_ss;  // < 2^24 (checked on the host)
    // Key block kb of head bh.
    auto run = [&](int kb) {
    const int c0 = CPW * kb;                   // the workgroup's first key chunk
    const int kc = c0 + w;                     // this wave's key chunk
    const bool kvalid = 16 * kc < S;           // the chunk holds keys of the sequence
    const int qstart = CAUSAL ? c0 : 0;        // first query chunk that sees a key of the workgroup
    const int clim = min(NW - 1, (S - 1) / 16 - c0);  // last chunk of the workgroup inside S
    const float *__restrict__ l2p = a.lse2 + (int64_t)bh * a.S_pad;
    const float *__restrict__ dlp = a.delta + (int64_t)bh * a.S_pad;

    // Resident K and V of the chunk: lane (n, g) holds K[16 kc + n][DH g + s]
    // (rows past S re-read row S - 1; their products are masked).
    float kr[DH], vr[DH];
    {
        const int row = min(16 * kc + n, S - 1);
        const float *__restrict__ ks = a.k + in_base + (int64_t)row * in_ss + DH * g;
        const float *__restrict__ vs = a.v + in_base + (int64_t)row * in_ss + DH * g;
#pragma unroll
        for (int s = 0; s < DH; s += 4) {
            const f32x4 t = *(const f32x4 *)(ks + s);
            const f32x4 u = *(const f32x4 *)(vs + s);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                kr[s + j] = t[j];
                vr[s + j] = u[j];
            }
        }
    }

    // Copies of a chunk set: waves 0, 1 copy the Q tile, waves 2, 3 the dO
    // tile (one tensor per wave: its base in a scalar buffer descriptor, a
    // fixed 32-bit byte offset per lane), every other copy each; wave 0 also
    // copies the 16 rows' lse2 and delta.  A padding or slack piece re-reads
    // the chunk's first piece (valid memory, never used).
    const int tw = w >> 1;
    const int tss = tw == 0 ? in_ss : out_ss;
    const float *__restrict__ tptr = tw == 0 ? a.q + in_base : a.dout + out_base;
    auto piece = [&](int u, int ln, int rmax) {
        const int p = 64 * u + ln;
        const int r = p / L::ROWCH, c4 = p - r * L::ROWCH;
        return r < 16 && c4 < D / 4 ? 4u * (unsigned)(min(r, rmax) * tss + 4 * c4) : 0u;
    };
    unsigned coff[L::SL];
#pragma unroll
    for (int sl = 0; sl < L::SL; ++sl) coff[sl] = piece((w & 1) + 2 * sl, lane, 15);
    // Chunk qc into set dst; the sequence's last chunk clamps its rows to
    // S - 1 (offsets recomputed from an opaque lane index).  Its lse2 rows
    // past S are +inf (attn_bwd_pre), so those rows contribute exactly 0.
    auto fetch = [&](int qc, float *dst) {
        const int m0 = 16 * qc;
        const bool full = m0 + 15 < S;
        const __amdgpu_buffer_rsrc_t rsrc = dma_rsrc(tptr + (int64_t)m0 * tss);
        float *tdst = dst + tw * L::TILE;
        int ln = lane;
        asm volatile("" : "+v"(ln));
#pragma unroll
        for (int sl = 0; sl < L::SL; ++sl) {
            const int u = (w & 1) + 2 * sl;
            if (u < L::TCOP && 64 * u + lane < 16 * L::ROWCH)
                dma16_buf(rsrc, full ? coff[sl] : piece(u, ln, S - 1 - m0), tdst + 256 * u);
        }
        if (w == 0 && lane < 8) dma16(lane < 4 ? l2p + m0 + 4 * lane : dlp + m0 + 4 * (lane - 4), dst + 2 * L::TILE);
    };

    f32x4 dvacc[NB], dkacc[NB];
#pragma unroll
    for (int i = 0; i < NB; ++i) {
        dvacc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
        dkacc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    }

    // The products of query chunk qc with this wave's key chunk.
    auto products = [&](int qc, const float *__restrict__ cur, float *__restrict__ ds) {
        const float *__restrict__ Qs = cur;
        const float *__restrict__ Gs = cur + L::TILE;
        f32x4 sacc = {0.f, 0.f, 0.f, 0.f}, pacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s0 = 0; s0 < DH; s0 += 4) {
            const f32x4 qf = *(const f32x4 *)&Qs[n * STR + DH * g + s0];
            const f32x4 gf = *(const f32x4 *)&Gs[n * STR + DH * g + s0];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                sacc = mfma16(qf[j], kr[s0 + j], sacc);
                pacc = mfma16(gf[j], vr[s0 + j], pacc);
            }
        }
        // lse2 and delta of rows 4g + r; P and dS, masked (P = 0) where key >
        // query on the diagonal chunk and for keys past S: an integer
        // threshold per lane, row r masked when thr > r.
        const f32x4 l2 = *(const f32x4 *)&cur[2 * L::TILE + 4 * g];
        const f32x4 dl = *(const f32x4 *)&cur[2 * L::TILE + 16 + 4 * g];
        int thr = CAUSAL && kc == qc ? n - 4 * g : -1;
        if (16 * kc + n >= S) thr = 1 << 20;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            float p = __builtin_amdgcn_exp2f(fmaf(sacc[r], a.c, -l2[r]));
            p = thr > r ? 0.0f : p;
            sacc[r] = p;
            pacc[r] = p * (pacc[r] - dl[r]);
            ds[(4 * g + r) * XSTR + 16 * w + n] = pacc[r];
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
                    dvacc[4 * h + j] = mfma16(sacc[r], gb[j], dvacc[4 * h + j]);
                    dkacc[4 * h + j] = mfma16(pacc[r], qb[j], dkacc[4 * h + j]);
                }
            }
        }
    };

    // dQ of query chunk qc (rows 16 qc .., column blocks QB w ..) from its dS
    // (in the dS half ds) and K^T, over the workgroup's key chunks inside S
    // and (causal) at or before qc.
    auto dq_product = [&](int qc, const float *__restrict__ ds, f32x4 (&acc)[QB]) {
#pragma unroll
        for (int q = 0; q < QB; ++q) acc[q] = f32x4{0.f, 0.f, 0.f, 0.f};
        const int clast = CAUSAL ? min(clim, qc - c0) : clim;
        for (int c = 0; c <= clast; ++c) {
            const f32x4 af = *(const f32x4 *)&ds[n * XSTR + 16 * c + 4 * g];
#pragma unroll
            for (int q = 0; q < QB; ++q) {
                const f32x4 bf = *(const f32x4 *)&Kt[(16 * (QB * w + q) + n) * XSTR + 16 * c + 4 * g];
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[q] = mfma16(af[j], bf[j], acc[q]);
            }
        }
    };
    // dQ of chunk qc added into dq (register r of block q: row 16 qc + 4g + r,
    // column 16 (QB w + q) + n).  Deterministic mode (kDqOrdered): first wait
    // until the chunk's counter (polled: an earlier read) shows the four
    // waves of every key block before kb in the order; the caller counts the
    // adds.
    int *const turns = DQ == kDqOrdered ? a.order + (int64_t)bh * (a.S_pad / 16) : nullptr;
    // Increments chunk qc's counter must show before this wave adds (ordered
    // dQ, attention_bwd_kernels.h): four per key block before kb.
    auto expect = [&](int qc) {
        const int last = CAUSAL ? min(nkb - 1, qc >> 2) : nkb - 1;  // key blocks of 64 = 4 chunks
        return 4 * order_before(kb, last, a.order_group);
    };
    auto store_dq = [&](auto mode, int qc, const f32x4 (&acc)[QB], int polled) {
        constexpr int Q = decltype(mode)::value;
        if constexpr (Q == kDqOrdered)
            order_wait(turns + qc, expect(qc), polled, a.order_timeouts);
        else if constexpr (Q == kDqOrderedFree)
            asm volatile("" ::: "memory");
        float *__restrict__ dqb = a.dq + in_base + 16 * QB * w + n;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int row = 16 * qc + 4 * g + r;
            if (row < S) {
#pragma unroll
                for (int q = 0; q < QB; ++q)
                    unsafeAtomicAdd(dqb + (int64_t)row * in_ss + 16 * q, acc[q][r] * a.scale);  // row * in_ss may pass 2^31
            }
        }
    };

    // K^T of the workgroup's keys for the dQ product (chunks past S are never read).
#pragma unroll
    for (int s = 0; s < DH; ++s) Kt[(DH * g + s) * XSTR + 16 * w + n] = kr[s];
    fetch(qstart, sets);
    wait_vmem();
    __syncthreads();

    // The walk over query chunks; mode: kDqAtomic, or in deterministic mode
    // kDqOrdered (poll and wait) or kDqOrderedFree (every key block before
    // kb has added all its chunks: no polls or waits).
    auto walk = [&](auto mode) {
        constexpr int Q = decltype(mode)::value;
        constexpr bool POLL = Q == kDqOrdered, COUNT = Q != kDqAtomic;
        f32x4 qa[QB];  // dQ of chunk qc - 1, added in step qc + 1
#pragma unroll
        for (int q = 0; q < QB; ++q) qa[q] = f32x4{0.f, 0.f, 0.f, 0.f};
        int polled = 0;  // kDqOrdered: the counter of the chunk added next
        if (POLL) polled = order_poll(turns + qstart);
        for (int qc = qstart; qc < nch; ++qc) {
            const int st = (qc - qstart) & 1;
            if (qc >= qstart + 2) store_dq(mode, qc - 2, qa, polled);
            if (POLL && qc >= qstart + 1) polled = order_poll(turns + qc - 1);
            if (qc + 1 < nch) fetch(qc + 1, sets + (st ^ 1) * L::SET);
            if (qc >= qstart + 1) dq_product(qc - 1, dsb, qa);
            __syncthreads();  // every wave has read dS of chunk qc - 1
            if (kvalid && (!CAUSAL || kc <= qc)) products(qc, sets + st * L::SET, dsb);
            wait_vmem();      // this wave's copies of chunk qc + 1 have landed
            if (COUNT && qc >= qstart + 2) order_done(turns + qc - 2);
            __syncthreads();  // dS of chunk qc and all of chunk qc + 1 in LDS
        }
        if (nch - qstart >= 2) {
            store_dq(mode, nch - 2, qa, polled);
            if (COUNT) order_done(turns + nch - 2);
        }
        {
            f32x4 ql[QB];
            if (POLL) polled = order_poll(turns + nch - 1);
            dq_product(nch - 1, dsb, ql);
            store_dq(mode, nch - 1, ql, polled);
            if (COUNT) order_done(turns + nch - 1);
        }
    };
    if constexpr (DQ == kDqAtomic) {
        walk(std::integral_constant<int, kDqAtomic>{});
    } else {
        // Whether the key blocks before this one have added their share of
        // its last chunk, and so of all its chunks (each walks upward).
        if (__builtin_amdgcn_readfirstlane(order_poll(turns + nch - 1)) >= expect(nch - 1))
            walk(std::integral_constant<int, kDqOrderedFree>{});
        else
            walk(std::integral_constant<int, kDqOrdered>{});
    }

    // dK (scaled) and dV of this wave's keys: register r of block 4h + j
    // holds key 16 kc + 4g + r, column 64h + 4n + j.
    if (kvalid) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int key = 16 * kc + 4 * g + r;
        if (key >= S) continue;
        float *dkrow = a.dk + in_base + (int64_t)key * in_ss + 4 * n;
        float *dvrow = a.dv + in_base + (int64_t)key * in_ss + 4 * n;
#pragma unroll
        for (int h = 0; h < NH; ++h) {
            f32x4 ko, vo;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                ko[j] = dkacc[4 * h + j][r] * a.scale;
                vo[j] = dvacc[4 * h + j][r];
            }
            *(f32x4 *)(dkrow + 64 * h) = ko;
            *(f32x4 *)(dvrow + 64 * h) = vo;
        }
    }
    }
    };
    if constexpr (PAIRK) {
        for (int pi = 0; pi < 2; ++pi) {
            const int kb = pi == 0 ? kb0 : nkb - 1 - kb0;
            if (pi == 1) {
                if (kb == kb0) break;
                __syncthreads();  // every wave is done with the first block's K^T and dS
            }
            run(kb);
        }
    } else {
        run(kb0);
    }
}

template <bool CAUSAL>
int launch_w16(const BwdArgs &args, int64_t rows_pad, int nbh)
{
    constexpr int D = 64;
    constexpr int RPB = 256 / (D / 4);
    const int pre_blocks = (int)((rows_pad + RPB - 1) / RPB);
    hipLaunchKernelGGL((attn_bwd_pre<D>), dim3(pre_blocks), dim3(256), 0, 0, args, rows_pad);
    if (!launch_ok("attn_bwd_pre")) return EMBER_ERR_DEVICE;
    const int nkb = (args.S + W16Shape<D>::KB - 1) / W16Shape<D>::KB;
    const dim3 grid((unsigned)(nkb * nbh));
    if (!args.order) {
        // Causal launches whose key-block pairs all fit one round of resident
        // workgroups take the blocks in pairs of about equal walks: measured
        // +4 % at B4 H16 S = 1024, +8-9 % at B2 H16 S = 2048 and B1 H16
        // S = 4096, +-0 at B8 H16 S = 1024; at S = 512 (short walks, which do
        // not cover the second block's prologue) -2.5 %, so from 16 blocks.
        if constexpr (CAUSAL) {
            const int ncu = device_cu_count();
            const int64_t pairs = (int64_t)(nkb + 1) / 2 * nbh;
            if (nkb >= 16 && pairs <= (int64_t)(ncu > 0 ? ncu : 256) * 4) {
                hipLaunchKernelGGL((attn_bwd_w16<D, CAUSAL, kDqAtomic, true>), dim3((unsigned)pairs), dim3(256), 0,
                                   0, args, nkb);
                return launch_ok("attn_bwd_w16_pairs") ? EMBER_OK : EMBER_ERR_DEVICE;
            }
        }
        hipLaunchKernelGGL((attn_bwd_w16<D, CAUSAL, kDqAtomic, false>), grid, dim3(256), 0, 0, args, nkb);
    } else {
        hipLaunchKernelGGL((attn_bwd_w16<D, CAUSAL, kDqOrdered, false>), grid, dim3(256), 0, 0, args, nkb);
    }
    return launch_ok("attn_bwd_w16") ? EMBER_OK : EMBER_ERR_DEVICE;
}

}  // namespace

int launch_bwd_w16(const BwdArgs &args, int64_t rows_pad, bool causal, int nbh)
{
    return causal ? launch_w16<true>(args, rows_pad, nbh) : launch_w16<false>(args, rows_pad, nbh);
}

}  // namespace ember

// attention_bwd_kernels.h -- kernels of the fused attention backward,
// included by attention_bwd.hip and attention_bwd_c128.hip.
//
// No reference counterpart (pawel002/ember has no attention); semantics are
// those of oracle/ember_oracle.c (oracle_attention_bwd): P is recomputed from
// the forward's LSE, never stored.
//
// Two launches on the null stream:
//  1. attn_bwd_pre (HBM-bound, one pass over O and dO): per query row
//     lse2 = lse * log2(e) and delta = <dO, O> into a row-statistics scratch
//     whose rows are padded per (b, h) to a multiple of 32 (padding rows get
//     lse2 = +inf, delta = 0, so every P they enter is exactly 0); and
//     dQ := 0 (dQ is accumulated with atomics).
//  2. attn_bwd_kernel, K/V-stationary: one workgroup = 4 waves = 128 keys of
//     one (b, h).  Each wave keeps K and V of its 32 keys resident in
//     registers as MFMA B operands and accumulates dK, dV for them in
//     registers.  The workgroup walks query blocks of 32 (causal: only the
//     blocks at or below its keys) with Q, dO and the block's lse2 / delta
//     staged in LDS:
//        S  = Q K^T, dP = dO V^T           (C[m][n], keys on lanes)
//        P  = exp2(S*c - lse2[m]), dS = P * (dP - delta[m])
//        dV += P^T dO,  dK += dS^T Q       (P / dS registers are the A
//                                           operands directly)
//     dS of all 4 waves goes through LDS so that dQ(32 x D) = dS . K over the
//     workgroup's 128 keys is one more MFMA product per wave, added to the
//     global dQ with hardware fp32 atomics (dq must be device memory).
//     Deterministic mode (ember_set_deterministic) adds the same values with
//     the same atomics, but in a fixed order: a tile's contributions come in
//     ascending key-block order, each wave waiting for the tile's counter
//     to show that the key blocks before its own have added theirs (see
//     "Ordered dQ" below).
//     That product is software-pipelined by one block: block j's step runs
//     the dQ MFMAs of block j-1 in between block j's softmax instructions,
//     so the matrix core keeps working while the softmax's VALU and
//     transcendental instructions issue (one wave per SIMD: no other wave
//     could fill the gap), and the step ends with one pair of barriers
//     around the dS exchange instead of two separated phases.
//
// Pipelining and instruction economy.  The next query block's Q, dO, lse2
// and delta are copied HBM -> LDS directly (gfx950 buffer_load_dwordx4 ... lds,
// no registers) into the second of two buffers while the current block is
// multiplied.  All LDS tiles use padded rows (Q/dO: D+4 floats, dS: 128+4;
// K: rows of D with the second half of the keys shifted by 32 floats) rather
// than XOR swizzles, chosen so that every LDS access in the loop is a per-lane
// base register plus a compile-time offset: the loop then spends its VALU
// issue slots on the softmax and not on address arithmetic.  The causal and
// key-tail mask is an integer compare per element against a per-lane
// threshold (no branches inside a step); workgroups with neither run a
// mask-free copy of the loop.
#pragma once

#include <math.h>

#include <type_traits>

#include "common.h"
#include "lds_dma.h"
#include "mfma.h"

namespace ember {

int check_attention_args(const void *const *ptrs, int nptrs, int64_t B, int64_t H, int64_t S,
                         int64_t D, float scale, const int64_t *strides, int nstrides,
                         const char *who);

struct BwdArgs {
    const float *q, *k, *v, *o, *lse, *dout;
    float *dq, *dk, *dv;
    float *lse2, *delta;  // row statistics, (B*H, S_pad) each
    // Deterministic mode (ember_set_deterministic), null otherwise:
    // order[bh * (S_pad / 16) + m / 16] counts the contributions added so
    // far to the dQ rows of head bh from row m (16-row granularity);
    // attn_bwd_pre zeroes them.  order_timeouts counts waits that gave up (a
    // device counter that is never reset).
    int *order;
    int *order_timeouts;
    int order_group;  // key blocks per group of the order (see "Ordered dQ")
    int H, S, S_pad, nkb;
    float c;      // scale * log2(e)
    float scale;
    int64_t in_sb, in_sh, in_ss, out_sb, out_sh, out_ss;
};

// attention_bwd_c128.hip: the causal D = 128 launch (a translation unit of
// its own, see the file comment).
int launch_bwd_causal_d128(const BwdArgs &args, int64_t rows_pad, int nblocks);

// attention_bwd_s128.hip: 64 < S <= 128 at D = 64 or 128, one workgroup
// per head (no row statistics and no atomics: args.lse2, delta, order
// unused).
int launch_bwd_s128(const BwdArgs &args, int D, bool causal, int nbh);
// attention_bwd_w16.hip: D = 64 at S > 128 (attn_bwd_pre, then attn_bwd_w16,
// ordered when args.order is set).
int launch_bwd_w16(const BwdArgs &args, int64_t rows_pad, bool causal, int nbh);

namespace {

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kBkw = 32;            // keys per wave
constexpr int kBk = kBkw * kWaves;  // keys per workgroup
constexpr int kBq = 32;             // queries per step
constexpr float kLog2e = 1.4426950408889634f;

// Row statistics and dQ := 0 (and, in deterministic mode, the tile
// counters := 0).  D/4 threads per (padded) row.
template <int D>
__global__ __launch_bounds__(256) void attn_bwd_pre(BwdArgs a, int64_t rows_pad)
{
    constexpr int TPR = D / 4;
    constexpr int RPB = 256 / TPR;
    const int sub = threadIdx.x % TPR;
    const int64_t row = (int64_t)blockIdx.x * RPB + threadIdx.x / TPR;
    if (row >= rows_pad) return;  // whole TPR-lane groups retire together
    if (a.order && sub == 0 && (row & 15) == 0) a.order[row >> 4] = 0;
    const int64_t bh = row / a.S_pad;
    const int m = (int)(row - bh * a.S_pad);
    if (m >= a.S) {
        if (sub == 0) {
            a.lse2[row] = INFINITY;
            a.delta[row] = 0.0f;
        }
        return;
    }
    const int b = (int)(bh / a.H);
    const int hh = (int)(bh - (int64_t)b * a.H);
    const int64_t ooff = (int64_t)b * a.out_sb + (int64_t)hh * a.out_sh + (int64_t)m * a.out_ss + 4 * sub;
    const f32x4 ov = *(const f32x4 *)(a.o + ooff);
    const f32x4 gv = *(const f32x4 *)(a.dout + ooff);
    float s = ov[0] * gv[0] + ov[1] * gv[1] + ov[2] * gv[2] + ov[3] * gv[3];
#pragma unroll
    for (int off = TPR / 2; off > 0; off >>= 1) s += __shfl_xor(s, off);
    if (sub == 0) {
        a.delta[row] = s;
        a.lse2[row] = a.lse[bh * a.S + m] * kLog2e;
    }
    const int64_t qoff = (int64_t)b * a.in_sb + (int64_t)hh * a.in_sh + (int64_t)m * a.in_ss + 4 * sub;
    *(f32x4 *)(a.dq + qoff) = f32x4{0.f, 0.f, 0.f, 0.f};
}

// ---- Ordered dQ (deterministic mode) ----
// fp32 addition is not associative, so dQ added with atomics in arrival
// order differs in its last bits from run to run.  In deterministic mode each
// dQ tile receives its key blocks' contributions in a fixed order: the wave
// that adds key block kb's share of a tile first waits until the tile's
// counter shows that every key block before kb in that order has added
// its share, then adds its own with the same atomics, waits for their
// acknowledgement and increments the counter.
// The order follows the hardware's schedule.  Work items keep the default
// mode's numbering (key block major, heaviest causal walks first, each
// head's workgroups on one XCD), and the workgroups of each XCD start in
// index order.  Key blocks come in groups of R (args.order_group): the
// groups in ascending order, and within a group descending, because the R
// key blocks of a group run at the same time and, causally, key block kb + 1
// starts its walk at the tile key block kb reaches four steps later, so
// that it is ahead at every tile they share.  A workgroup waits only for
// lower groups, which started earlier, and for higher key blocks of its own
// group; the host picks R so that the groups below the top key block of a
// group fit in the device at once, R <= 1 + (slots - 1) / (B * H) (slots:
// workgroups resident at once, an eighth kept spare), so the top key blocks,
// which wait on lower groups only, always start, and no wait can deadlock.
// The counter is polled a step ahead of its use.  A workgroup first reads
// the counter of the last tile it adds to: if every key block before it has
// added its share there, it has added all its tiles (each walks its tiles
// upward, and a key block that sees one of this workgroup's tiles sees its
// last one), and the workgroup walks without polls or waits
// (kDqOrderedFree), only counting its own adds.
// The adds are released by waiting for their acknowledgement (vmcnt), not by
// an agent-scope release fence: these atomics are performed where every XCD's
// atomics on the address meet (adds into one tile from several XCDs are
// exact), and an acknowledged atomic has been performed there; the fence
// would add an L2 write-back per wave and step (3.8x the time at B4 H32
// S4096 D128), and with it and without it dQ came out the same bits in
// every case measured (causal and not, D = 32, 64, 128).
// Each wait is still bounded, should those start-order assumptions ever not
// hold: after ~2 s (s_memrealtime runs at 100 MHz) it gives up, counts
// itself in order_timeouts, and from then on no wait blocks; the sum stays
// correct, only its order is lost, which ember_deterministic_timeouts()
// reports.
constexpr int kDqAtomic = 0, kDqOrdered = 1, kDqOrderedFree = 2;
constexpr uint64_t kOrderTimeoutTicks = 200000000ull;

// A tile counter (relaxed, device scope: the load bypasses this XCD's L2,
// so it sees increments made on other XCDs).
__device__ __forceinline__ int order_poll(const int *p)
{
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Waits until *turn >= expect (polled: an earlier read of *turn).
__device__ __forceinline__ void order_wait(const int *turn, int expect, int polled, int *timeouts)
{
    if (__builtin_amdgcn_readfirstlane(polled) < expect) {
        const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
        for (;;) {
            __builtin_amdgcn_s_sleep(2);
            if (__builtin_amdgcn_readfirstlane(order_poll(turn)) >= expect) break;
            if (__builtin_amdgcn_readfirstlane(order_poll(timeouts)) != 0) break;
            if (__builtin_amdgcn_s_memrealtime() - t0 > kOrderTimeoutTicks) {
                if ((threadIdx.x & 63) == 0)
                    __hip_atomic_fetch_add(timeouts, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
        }
    }
    asm volatile("" ::: "memory");  // the adds that follow stay after the wait
}

// This wave's adds into the tile have been acknowledged (vmcnt 0: every
// vector memory operation of the wave has completed); count them.
__device__ __forceinline__ void order_done(int *turn)
{
    __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8));  // vmcnt(0)
    asm volatile("" ::: "memory");
    if ((threadIdx.x & 63) == 0) __hip_atomic_fetch_add(turn, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int D>
struct BwdLayout {
    static constexpr int DB = D / 32;
    static constexpr int QSTR = D + 4;                // padded Q / dO row
    static constexpr int QROWCH = QSTR / 4;           // 16-byte chunks per padded row
    static constexpr int QCHUNKS = kBq * QROWCH;      // chunks per Q / dO tile
    static constexpr int QDMA = (QCHUNKS + 63) / 64;  // 1 KiB copies per tile
    static constexpr int QBUF = QDMA * 256;           // floats reserved per tile
    static constexpr int SLOTS = (QDMA + kWaves - 1) / kWaves;  // copies per wave
    static constexpr int SSTR = kBk + 4;              // padded dS row
    static constexpr int NSPLIT = 4 / DB;             // waves sharing a 32-wide d block of dQ
    static constexpr int NK = kBk / NSPLIT;           // keys each wave contracts for dQ
    static constexpr int NKH = NK / 2;                // ... per lane half
    // K row n at n*D + (n / NKH)*32: the two lane halves of the dQ product
    // read rows NKH apart, which the shift puts 32 banks apart.
    static constexpr int KALL = kBk * D + (kBk / NKH) * 32;
};

constexpr int kMaxSlots = 5;  // BwdLayout<128>::SLOTS

// Buffers for a block's dS: two at D = 64, used by alternate blocks, which
// saves one barrier per block (bwd_step; +2-3 % at D = 64); one at D = 128
// (no LDS left) and at D = 32 (two measured -1 to -4 % causal).  The
// library instantiates this kernel at D = 32 and 128; D = 64 runs
// attn_bwd_w16 (attention_bwd_w16.hip), which measured faster there.
template <int D>
constexpr int kDsBufs = D == 64 ? 2 : 1;

// Loop-invariant state of one workgroup.
struct BwdBlock {
    const float *qp, *gp;      // q, dO at (b, h)
    const float *l2p, *dlp;    // lse2, delta at (b, h)
    float *dqp;                // dq at (b, h)
    int *turns;                // deterministic mode: tile counters of (b, h)
    int S, nq, n0w, w, kb;
    int in_ss, out_ss;
    // Per copy slot s (copy t = w + 4s of a tile): this lane's chunk as a
    // byte offset within the block for q and dO (0 for padding or slack:
    // the block's first chunk, never read).
    unsigned qoff[kMaxSlots], goff[kMaxSlots];
    bool key_tail;
};

// This lane's chunk of copy t of a Q / dO tile (padded rows): its row, and
// whether it holds data (not row padding or slack past the tile).
template <int D>
__device__ __forceinline__ void bwd_chunk(int t, int lane, int &r, int &c4, bool &real)
{
    typedef BwdLayout<D> L;
    const int p = 64 * t + lane;
    r = p / L::QROWCH;
    c4 = p - r * L::QROWCH;
    real = p < L::QCHUNKS && c4 < D / 4;
}

// Copies query block m0's Q and dO tiles (padded rows) and its lse2 / delta
// into one set of buffers (buffer-form copies: the block base in a scalar
// descriptor, a 32-bit byte offset per lane).  Copy t of a tile fills chunks
// 64t .. 64t+63; a padding or slack chunk reads row m0's first chunk (valid
// memory, never used).  Rows past the end re-read row S-1; their lse2 is
// +inf, so they contribute exactly 0.  On that (last) block the offsets are
// recomputed from an opaque lane index, so that the compiler keeps no
// second set live across the loop.
template <int D>
__device__ __forceinline__ void bwd_fetch(const BwdBlock &k, int m0, float *__restrict__ qn,
                                          float *__restrict__ gn, float *__restrict__ stn)
{
    typedef BwdLayout<D> L;
    const __amdgpu_buffer_rsrc_t rq = dma_rsrc(k.qp + (int64_t)m0 * k.in_ss);
    const __amdgpu_buffer_rsrc_t rg = dma_rsrc(k.gp + (int64_t)m0 * k.out_ss);
    const int rmax = k.S - 1 - m0;  // rows beyond it are clamped to it
    if (rmax >= kBq - 1) {
#pragma unroll
        for (int s = 0; s < L::SLOTS; ++s) {
            const int t = k.w + kWaves * s;
            if (t < L::QDMA) {
                dma16_buf(rq, k.qoff[s], qn + 256 * t);
                dma16_buf(rg, k.goff[s], gn + 256 * t);
            }
        }
    } else {
        int ln = threadIdx.x & 63;
        asm volatile("" : "+v"(ln));
#pragma unroll
        for (int s = 0; s < L::SLOTS; ++s) {
            const int t = k.w + kWaves * s;
            if (t < L::QDMA) {
                int r, c4;
                bool real;
                bwd_chunk<D>(t, ln, r, c4, real);
                r = min(r, rmax);
                dma16_buf(rq, real ? 4u * (unsigned)(r * k.in_ss + 4 * c4) : 0u, qn + 256 * t);
                dma16_buf(rg, real ? 4u * (unsigned)(r * k.out_ss + 4 * c4) : 0u, gn + 256 * t);
            }
        }
    }
    if (k.w == 0) {
        const int lane = threadIdx.x & 63;
        if (lane < 16) dma16(lane < 8 ? k.l2p + m0 + 4 * lane : k.dlp + m0 + 4 * (lane - 8), stn);
    }
}

// dQ of one query block: dQ[m0:m0+32, 32*dblk:+32] += scale * dS . K over
// this wave's share of the workgroup's keys, dS read from LDS.  The dQ
// product of the previous block is issued in the middle of the next block's
// step, interleaved with that block's softmax (see bwd_step).
template <int D>
struct DqState {
    int sa, kbase;
};

template <int D>
__device__ __forceinline__ DqState<D> dq_state(int w)
{
    typedef BwdLayout<D> L;
    constexpr int DB = L::DB;
    const int lane = threadIdx.x & 63;
    const int h32 = lane >> 5;
    const int l32 = lane & 31;
    const int dblk = w % DB;
    const int nbase = (w / DB) * L::NK;
    DqState<D> st;
    st.sa = l32 * L::SSTR + nbase + h32 * L::NKH;
    st.kbase = (nbase + h32 * L::NKH) * D + (nbase / L::NKH + h32) * 32 + 32 * dblk + l32;
    return st;
}

// Deterministic mode: the contributions that come before key block kb's at
// a tile whose last contributing key block is `last` (ordered dQ above):
// every key block of the lower groups, and those after kb in its own group.
__device__ __forceinline__ int order_before(int kb, int last, int R)
{
    const int g0 = kb - kb % R;
    return g0 + min(g0 + R - 1, last) - kb;
}

// How many increments this wave must see on the counter of the tile of rows
// m0.. before adding: four per key block before kb in the order (one per
// wave), and, where waves share dQ columns (D < 128), those of the lower
// waves of its own key block.
template <int D, bool CAUSAL>
__device__ __forceinline__ int dq_turn_expect(const BwdArgs &a, const BwdBlock &k, int m0)
{
    constexpr int DB = BwdLayout<D>::DB;
    const int last = CAUSAL ? min(a.nkb - 1, (m0 / kBq) >> 2) : a.nkb - 1;  // key blocks of 128 = 4 tiles
    return 4 * order_before(k.kb, last, a.order_group) + (k.w / DB) * DB;
}

// Deterministic mode: whether a wave counts its adds into a tile at once
// (waves that share dQ columns wait for each other within the step) or
// after the step's wait for its copies, which then costs no extra wait.
template <int D>
constexpr bool kDoneAtOnce = BwdLayout<D>::DB < 4;

// The finished dQ block (rows m0..m0+31) added into dq with atomics;
// deterministic mode (kDqOrdered) first waits for its turn (polled: an
// earlier read of the tile counter) and counts its adds (kDoneAtOnce) or
// leaves that to the caller.
template <int D, bool CAUSAL, int DQ>
__device__ __forceinline__ void dq_store(const BwdArgs &a, const BwdBlock &k, int m0, const f32x16 &qacc,
                                         int polled)
{
    constexpr int DB = BwdLayout<D>::DB;
    const int lane = threadIdx.x & 63;
    const int h32 = lane >> 5;
    const int l32 = lane & 31;
    const int dblk = k.w % DB;
    if constexpr (DQ == kDqOrdered)
        order_wait(k.turns + (m0 >> 4), dq_turn_expect<D, CAUSAL>(a, k, m0), polled, a.order_timeouts);
    else if constexpr (DQ == kDqOrderedFree)
        asm volatile("" ::: "memory");
    // Row i of the block: wave-uniform row base + unsigned lane offset.
    float *dqb = k.dqp + (int64_t)m0 * k.in_ss + 32 * dblk;
    const unsigned qoff = (unsigned)(4 * h32 * k.in_ss + l32);
    if (m0 + kBq <= k.S) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            float *rowp = dqb + (int64_t)(((i >> 2) * 8 + (i & 3)) * k.in_ss);
            unsafeAtomicAdd(rowp + qoff, qacc[i] * a.scale);
        }
    } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            float *rowp = dqb + (int64_t)(((i >> 2) * 8 + (i & 3)) * k.in_ss);
            if (m0 + acc_row(i, h32) < k.S) unsafeAtomicAdd(rowp + qoff, qacc[i] * a.scale);
        }
    }
    if constexpr (DQ != kDqAtomic && kDoneAtOnce<D>) order_done(k.turns + (m0 >> 4));
}

// The dQ product of the previous block (when PREV) fused with this block's
// softmax: P = exp2(S*c - lse2), masked where t > 8(i/4) + i%4 (when MASK),
// dS = P * (dP - delta).  sacc / pacc hold S / dP on entry, P / dS on exit.
template <int D, bool PREV, bool MASK>
__device__ __forceinline__ void dq_softmax(const BwdArgs &a, const float *__restrict__ ds,
                                           const float *__restrict__ kall, const DqState<D> &dqs,
                                           const f32x4 (&l2v)[4], const f32x4 (&dlv)[4], int t,
                                           f32x16 &sacc, f32x16 &pacc, f32x16 &qacc)
{
    typedef BwdLayout<D> L;
    constexpr int NIT = L::NKH / 4;  // dQ k-steps of 4 MFMAs
    constexpr int EPI = 16 / NIT;    // softmax elements per k-step
#pragma unroll
    for (int it = 0; it < NIT; ++it) {
        if (PREV) {
            const f32x4 sf = *(const f32x4 *)&ds[dqs.sa + 4 * it];
#pragma unroll
            for (int j = 0; j < 4; ++j)
                qacc = mfma_32x32x2(sf[j], kall[dqs.kbase + (4 * it + j) * D], qacc);
        }
#pragma unroll
        for (int e = 0; e < EPI; ++e) {
            const int i = it * EPI + e;
            float p = __builtin_amdgcn_exp2f(fmaf(sacc[i], a.c, -l2v[i >> 2][i & 3]));
            if (MASK) p = t > 8 * (i >> 2) + (i & 3) ? 0.0f : p;
            sacc[i] = p;                                   // P[m][n]
            pacc[i] = p * (pacc[i] - dlv[i >> 2][i & 3]);  // dS[m][n]
        }
    }
}

// One query block qb, software-pipelined with the previous one:
//   1. copy block qb+1 into (qn, gn, stn);
//   2. S = Q K^T and dP = dO V^T of block qb (MFMA);
//   3. the dQ product of block qb-1 (dS in LDS since the last barrier),
//      interleaved with the softmax of block qb: its VALU work issues while
//      the dQ MFMAs run, instead of leaving the matrix core idle;
//   4. dQ of block qb-1 to memory (dq_store: atomics or partial slab);
//   5. dV += P^T dO, dK += dS^T Q of block qb;
//   6. barrier (every wave has read dS of block qb-1; not needed with two
//      dS buffers, see kDsBufs), dS of block qb to LDS, wait for the
//      copies, barrier.
// The mask is applied branch-free (an integer compare per element against a
// per-lane threshold), so steps 2 and 3 are one basic block.  Keys a wave
// cannot see in this block (causal, above the diagonal) get P = 0 by the same
// compare, so no wave skips the block.
template <int D, bool CAUSAL, bool PREV, bool MASK, int DQ>
__device__ __forceinline__ void bwd_step(const BwdArgs &a, const BwdBlock &k, int qb,
                                         const float *__restrict__ qs,
                                         const float *__restrict__ gs,
                                         const float *__restrict__ st, float *__restrict__ dsb,
                                         int parity,
                                         float *__restrict__ qn, float *__restrict__ gn,
                                         float *__restrict__ stn,
                                         const float *__restrict__ kall, const float *kr,
                                         const float *vr, f32x16 *dvacc, f32x16 *dkacc,
                                         int tail_bias)
{
    typedef BwdLayout<D> L;
    constexpr int DH = D / 2;
    constexpr int DB = L::DB;
    const int lane = threadIdx.x & 63;
    const int h32 = lane >> 5;
    const int l32 = lane & 31;
    const int m0 = qb * kBq;
    // dS buffers (kDsBufs): this block's dS goes to buffer `parity`, the
    // previous block's is read from the other one (the same one at D = 128).
    constexpr int kDsStride = (kDsBufs<D> - 1) * kBq * L::SSTR;
    const float *const ds = dsb + (parity ^ 1) * kDsStride;
    float *const ds_out = dsb + parity * kDsStride;

    // Deterministic mode: the previous block's tile counter, read a step ahead of its use.
    int polled = 0;
    if (PREV && DQ == kDqOrdered) polled = order_poll(k.turns + ((m0 - kBq) >> 4));
    if (qb + 1 < k.nq) bwd_fetch<D>(k, m0 + kBq, qn, gn, stn);

    // ---- S, dP ----
    f32x16 sacc = zero16(), pacc = zero16();
    {
        const int abase = l32 * L::QSTR + h32 * DH;
#pragma unroll
        for (int kk = 0; kk < DH; kk += 4) {
            const f32x4 qf = *(const f32x4 *)&qs[abase + kk];
            const f32x4 gf = *(const f32x4 *)&gs[abase + kk];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                sacc = mfma_32x32x2(qf[j], kr[kk + j], sacc);
                pacc = mfma_32x32x2(gf[j], vr[kk + j], pacc);
            }
        }
    }
    // Row statistics of rows acc_row(4g + 0..3, h32) = 8g + 4*h32 + 0..3.
    f32x4 l2v[4], dlv[4];
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        l2v[g] = *(const f32x4 *)&st[8 * g + 4 * h32];
        dlv[g] = *(const f32x4 *)&st[kBq + 8 * g + 4 * h32];
    }
    // ---- dQ of the previous block, interleaved with this block's softmax ----
    // Blocks that cross the diagonal or the last key take the masked copy of
    // the loop; each copy is one basic block.
    f32x16 qacc = zero16();
    const DqState<D> dqs = dq_state<D>(k.w);
    // P[m][n] = 0 where t > 8(i/4) + i%4 (see the mask note above).
    const int t = (CAUSAL ? k.n0w + l32 - m0 - 4 * h32 : -1) + tail_bias;
    dq_softmax<D, PREV, MASK>(a, ds, kall, dqs, l2v, dlv, t, sacc, pacc, qacc);
    // D < 128: P and dS are pinned here (an empty asm that reads and writes
    // them), so that the compiler computes them interleaved with the dQ
    // MFMAs above instead of sinking them past the dQ store's branches into
    // the dV/dK block, where nothing hides them (measured +3.7 % at D = 64;
    // at D = 128 the sunk form is 0.8 % faster).
    if constexpr (D < 128) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            float x = sacc[i], y = pacc[i];
            asm volatile("" : "+v"(x), "+v"(y));
            sacc[i] = x;
            pacc[i] = y;
        }
    }
    if (PREV) dq_store<D, CAUSAL, DQ>(a, k, m0 - kBq, qacc, polled);

    // ---- dV += P^T dO, dK += dS^T Q ----
    {
        typedef typename VecN<DB>::T OpT;
        const int bbase = 4 * h32 * L::QSTR + DB * l32;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int off = bbase + ((i >> 2) * 8 + (i & 3)) * L::QSTR;
            const OpT gf = *(const OpT *)&gs[off];
            const OpT qf = *(const OpT *)&qs[off];
#pragma unroll
            for (int db = 0; db < DB; ++db) {
                dvacc[db] = mfma_32x32x2(sacc[i], vget<DB>(gf, db), dvacc[db]);
                dkacc[db] = mfma_32x32x2(pacc[i], vget<DB>(qf, db), dkacc[db]);
            }
        }
    }
    // Every wave has read the previous block's dS (with one dS buffer; with
    // two, this block's dS goes to the other one, which nobody has read since
    // the last step's closing barrier).
    if constexpr (kDsBufs<D> == 1) __syncthreads();
    {
        const int sbase = 4 * h32 * L::SSTR + kBkw * k.w + l32;
#pragma unroll
        for (int i = 0; i < 16; ++i) ds_out[sbase + ((i >> 2) * 8 + (i & 3)) * L::SSTR] = pacc[i];
    }
    wait_vmem();  // this wave's copies into (qn, gn, stn) have landed
    if (PREV && DQ != kDqAtomic && !kDoneAtOnce<D>) order_done(k.turns + ((m0 - kBq) >> 4));
    __syncthreads();
}

// dQ of the last block (its dS is in LDS after the last step's barrier).
template <int D, bool CAUSAL, int DQ>
__device__ __forceinline__ void bwd_last_dq(const BwdArgs &a, const BwdBlock &k, int m0,
                                            const float *__restrict__ ds,
                                            const float *__restrict__ kall)
{
    typedef BwdLayout<D> L;
    int polled = 0;
    if (DQ == kDqOrdered) polled = order_poll(k.turns + (m0 >> 4));
    const DqState<D> dqs = dq_state<D>(k.w);
    f32x16 qacc = zero16();
#pragma unroll
    for (int kk = 0; kk < L::NKH; kk += 4) {
        const f32x4 sf = *(const f32x4 *)&ds[dqs.sa + kk];
#pragma unroll
        for (int j = 0; j < 4; ++j) qacc = mfma_32x32x2(sf[j], kall[dqs.kbase + (kk + j) * D], qacc);
    }
    dq_store<D, CAUSAL, DQ>(a, k, m0, qacc, polled);
    if (DQ != kDqAtomic && !kDoneAtOnce<D>) order_done(k.turns + (m0 >> 4));
}

template <int D, bool CAUSAL, int DQ>
__global__ __launch_bounds__(kThreads, 1) void attn_bwd_kernel(BwdArgs a)
{
    typedef BwdLayout<D> L;
    constexpr int DH = D / 2;
    constexpr int DB = L::DB;
    static_assert(L::SLOTS <= kMaxSlots, "copy slots");
    __shared__ float Kall[L::KALL];
    __shared__ float Qs0[L::QBUF], Qs1[L::QBUF];
    __shared__ float dOs0[L::QBUF], dOs1[L::QBUF];
    __shared__ float St0[2 * kBq], St1[2 * kBq];
    __shared__ float dSs[kDsBufs<D> * kBq * L::SSTR];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    // Wave index, made provably uniform for D < 128 (scalar copy branches
    // and LDS bases); at D = 128 the kernel is short of scalar registers and
    // the plain form measured faster (2 % non-causal).
    const int w = D == 128 ? tid >> 6 : __builtin_amdgcn_readfirstlane(tid >> 6);
    const int h32 = lane >> 5;
    const int l32 = lane & 31;

    const int BH = (int)(gridDim.x / a.nkb);
    const int kb = blockIdx.x / BH;  // ascending: the longest causal rows first
    const int bh = blockIdx.x - kb * BH;
    const int b = bh / a.H;
    const int hh = bh - b * a.H;
    const int S = a.S;
    const int n0 = kb * kBk;

    BwdBlock k;
    const int64_t in_base = (int64_t)b * a.in_sb + (int64_t)hh * a.in_sh;
    const int64_t out_base = (int64_t)b * a.out_sb + (int64_t)hh * a.out_sh;
    k.qp = a.q + in_base;
    k.gp = a.dout + out_base;
    k.l2p = a.lse2 + (int64_t)bh * a.S_pad;
    k.dlp = a.delta + (int64_t)bh * a.S_pad;
    k.dqp = a.dq + in_base;
    k.turns = DQ == kDqOrdered ? a.order + (int64_t)bh * (a.S_pad / 16) : nullptr;
    k.S = S;
    k.nq = (S + kBq - 1) / kBq;
    k.w = w;
    k.kb = kb;
    k.n0w = n0 + kBkw * w;
    k.in_ss = (int)a.in_ss;  // row strides < 2^24, checked on the host
    k.out_ss = (int)a.out_ss;
    k.key_tail = k.n0w + kBkw > S;
#pragma unroll
    for (int s = 0; s < kMaxSlots; ++s) {
        int r, c4;
        bool real;
        bwd_chunk<D>(w + kWaves * s, lane, r, c4, real);
        k.qoff[s] = real ? 4u * (unsigned)(r * k.in_ss + 4 * c4) : 0u;
        k.goff[s] = real ? 4u * (unsigned)(r * k.out_ss + 4 * c4) : 0u;
    }

    // Resident B operands: lane holds K[nl][h32*DH + kk] and V[nl][...].
    float kr[DH], vr[DH];
    {
        const int nl = k.n0w + l32;
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
        *(f32x4 *)&Kall[r * D + (r / L::NKH) * 32 + 4 * c4] = kv;
    }

    f32x16 dvacc[DB], dkacc[DB];
#pragma unroll
    for (int db = 0; db < DB; ++db) {
        dvacc[db] = zero16();
        dkacc[db] = zero16();
    }

    // First block into buffer set 0; afterwards every step copies the next
    // block into the other set while it computes.
    const int qstart = CAUSAL ? n0 / kBq : 0;
    bwd_fetch<D>(k, qstart * kBq, Qs0, dOs0, St0);
    wait_vmem();
    __syncthreads();

    // Keys past the sequence end: P = 0 whatever the row (see bwd_step).
    // Without a causal mask or such keys no block needs the mask.
    const int tail_bias = k.n0w + l32 >= S ? (1 << 24) : 0;
    auto walk = [&](auto mask, auto mode) {
        constexpr bool M = decltype(mask)::value;
        constexpr int Q = decltype(mode)::value;
        bwd_step<D, CAUSAL, false, M, Q>(a, k, qstart, Qs0, dOs0, St0, dSs, 0, Qs1, dOs1, St1, Kall, kr,
                                         vr, dvacc, dkacc, tail_bias);
        for (int qb = qstart + 1; qb < k.nq; qb += 2) {
            bwd_step<D, CAUSAL, true, M, Q>(a, k, qb, Qs1, dOs1, St1, dSs, 1, Qs0, dOs0, St0, Kall, kr,
                                            vr, dvacc, dkacc, tail_bias);
            if (qb + 1 < k.nq)
                bwd_step<D, CAUSAL, true, M, Q>(a, k, qb + 1, Qs0, dOs0, St0, dSs, 0, Qs1, dOs1, St1,
                                                Kall, kr, vr, dvacc, dkacc, tail_bias);
        }
    };
    const float *const ds_last = dSs + ((k.nq - 1 - qstart) & 1) * (kDsBufs<D> - 1) * kBq * L::SSTR;
    auto walk_all = [&](auto mode) {
        if (CAUSAL || k.key_tail)
            walk(std::true_type{}, mode);
        else
            walk(std::false_type{}, mode);
        bwd_last_dq<D, CAUSAL, decltype(mode)::value>(a, k, (k.nq - 1) * kBq, ds_last, Kall);
    };
    if constexpr (DQ == kDqAtomic) {
        walk_all(std::integral_constant<int, kDqAtomic>{});
    } else {
        // Deterministic mode: whether the key blocks before this one have
        // added their share of its last tile, and so of all its tiles
        // (ordered dQ above); waves that share dQ columns (D < 128) always
        // wait for each other.
        const int m_last = (k.nq - 1) * kBq;
        const int seen = order_poll(k.turns + (m_last >> 4));
        if (!kDoneAtOnce<D> && __builtin_amdgcn_readfirstlane(seen) >= dq_turn_expect<D, CAUSAL>(a, k, m_last))
            walk_all(std::integral_constant<int, kDqOrderedFree>{});
        else
            walk_all(std::integral_constant<int, kDqOrdered>{});
    }

    // dK (scaled) and dV rows of this wave's keys: register i -> key
    // n0w + acc_row(i, h32), lane -> d = DB*l32 + db.
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int n = k.n0w + acc_row(i, h32);
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

// Launches the backward for args: attn_bwd_pre, then the workgroup kernel,
// whose dQ is added with atomics in arrival order or (args.order set) in
// key-block order.
template <int D, bool CAUSAL>
int launch_bwd(const BwdArgs &args, int64_t rows_pad, int nblocks)
{
    constexpr int RPB = 256 / (D / 4);
    const int pre_blocks = (int)((rows_pad + RPB - 1) / RPB);
    hipLaunchKernelGGL((attn_bwd_pre<D>), dim3(pre_blocks), dim3(256), 0, 0, args, rows_pad);
    if (!launch_ok("attn_bwd_pre")) return EMBER_ERR_DEVICE;
    if (!args.order) {
        hipLaunchKernelGGL((attn_bwd_kernel<D, CAUSAL, kDqAtomic>), dim3(nblocks), dim3(kThreads), 0, 0,
                           args);
        return launch_ok("attn_bwd_kernel") ? EMBER_OK : EMBER_ERR_DEVICE;
    }
    hipLaunchKernelGGL((attn_bwd_kernel<D, CAUSAL, kDqOrdered>), dim3(nblocks), dim3(kThreads), 0, 0, args);
    return launch_ok("attn_bwd_kernel") ? EMBER_OK : EMBER_ERR_DEVICE;
}

}  // namespace
}  // namespace ember


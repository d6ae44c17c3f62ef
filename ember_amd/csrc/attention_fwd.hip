// attention_fwd.hip -- fused flash-attention forward (fp32) for gfx950.
//
// No reference counterpart: pawel002/ember has no attention; the operator is
// new, slotted beside matmul in src/tensor/operators.h:20-27.  Its semantics
// are those of oracle/ember_oracle.c (oracle_attention_fwd).
//
// Work decomposition.  One workgroup = 4 waves = 128 queries of one (b, h);
// each wave owns 32 queries for the whole kernel.  The workgroup walks the
// keys in tiles of 64: every tile of K and V is read from HBM once and
// staged in LDS, where the 4 waves share it.  The copies go HBM -> LDS
// directly (buffer_load_dwordx4 ... lds, no registers) and overlap the
// products: V of tile t lands while S of tile t is computed, K of tile t+1
// while V of tile t is multiplied; two barriers per tile.
// Short sequences (S <= 64, HBM-bound) use one wave per 32-query block
// instead, with no barriers (attn_fwd_wave, D >= 64), or pack heads
// (attn_fwd_packed, D = 32): S <= 32 puts 4 heads in a workgroup (one per
// wave, tiles of 32 keys) and S <= 64 puts 2 (two waves each), so that no
// wave idles and every wave keeps loading.
// 64 < S <= 96, and causal S <= 128, at D >= 64 take attn_fwd_wave with one
// wave per pair of query blocks.
//
// Per tile and wave (all products on v_mfma_f32_32x32x2f32):
//   S^T (64 keys x 32 queries) = K_tile . Q^T   -- K from LDS, Q^T resident in
//                                                  registers for the kernel
//   online softmax over keys: each lane holds one query column, so the row
//   max is an in-lane max over 32 registers plus one exchange with lane^32,
//   and the row sum stays a per-lane partial until the end
//   O^T (D x 32 queries) += V_tile^T . P^T      -- P^T straight from the S^T
//                                                  accumulator registers
// The softmax runs in base 2 with scale*log2(e) folded into one FMA per
// score, on v_exp_f32, with lazy rescaling of O (see the loop); LSE is
// stored in natural log.  Causal: tiles wholly above a wave's
// diagonal are skipped per wave, the mask (key <= query, integer compare) is
// applied only on tiles that cross the diagonal or the sequence end.
#include <math.h>

#include <type_traits>

#include "common.h"
#include "lds_dma.h"
#include "mfma.h"

namespace ember {
namespace {

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kBr = 32 * kWaves;  // queries per workgroup (one head per workgroup)
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

struct FwdArgs {
    const float *q, *k, *v;
    float *o, *lse;
    int H, S, nqb, nbh;
    float c;  // scale * log2(e)
    int64_t in_sb, in_sh, in_ss, out_sb, out_sh, out_ss;
};

// Copy layout of one 64-key tile for the direct HBM -> LDS copies.  A copy is
// 64 lanes x 16 bytes = 1 KiB of LDS; copy t of a tile fills 16-byte chunks
// 64t .. 64t+63.  K rows are padded to D+4 floats (conflict-free reads of a
// column of chunks by 32 lanes): a padding chunk re-reads the tile's first
// chunk (valid memory, never used).  V rows are dense.
template <int D> struct FwdTile {
    static constexpr int KSTR = D + 4;                       // floats per K row
    static constexpr int KCH = KSTR / 4;                     // chunks per K row
    static constexpr int KCOP = KCH;                         // copies per K tile: 64 rows * KCH / 64
    static constexpr int VCOP = D / 4;                       // copies per V tile
    static constexpr int KSL = (KCOP + kWaves - 1) / kWaves; // K copy slots per wave
    static constexpr int VSL = VCOP / kWaves;                // V copy slots per wave
    static constexpr int VROWS = kWaves * 256 / D;           // V rows between a wave's slots
};

// One head per workgroup, S > 64 (see the file comment).  Per tile t:
//   wait for this wave's K copies, barrier (K(t) complete, Vs free)
//   copy V(t) -> Vs;  S^T = K . Q^T;  mask, softmax
//   wait for this wave's V copies, barrier (V(t) complete, Ks free)
//   copy K(t+1) -> Ks;  O^T += V^T . P^T
// A wave whose queries all precede the tile (causal) skips the products
// but still issues its copies and meets both barriers.
// Workgroups per CU: two, or three at D = 64 (LDS fits three there; the
// causal D = 64 kernel fits three in registers thanks to its split loop,
// see the end of the kernel).
template <int D, bool CAUSAL, bool PAIRQ>
__global__ __launch_bounds__(kThreads, D == 64 ? 3 : 2) void attn_fwd_kernel(FwdArgs a)
{
    typedef FwdTile<D> T;
    constexpr int DH = D / 2;   // contraction length per lane half (k-steps)
    constexpr int DB = D / 32;  // 32-row blocks of O^T
    constexpr int KSTR = T::KSTR;
    constexpr int kBc = 64;
    // D = 128 keeps one offset register per V copy slot (it has the
    // registers, and it saves the per-slot descriptor arithmetic); smaller D
    // keeps one and moves the descriptor base per slot.
    constexpr bool kVoffRegs = D == 128;
    __shared__ float Ks[kBc * KSTR];
    __shared__ float Vs[kBc * D];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int h32 = lane >> 5;
    const int l32 = lane & 31;

    // Heavy (late) query blocks first so the causal triangle load-balances.
    // PAIRQ (causal): the workgroup takes query blocks nqb - 1 - p and p of
    // its head, one after the other: 2 (nqb + 1) key tiles for every
    // workgroup (the middle block of an odd nqb alone, dispatched last).
    const int per_head = PAIRQ ? (a.nqb + 1) / 2 : a.nqb;
    const int BH = (int)(gridDim.x / per_head);
    const int qbr = blockIdx.x / BH;
    const int bh = blockIdx.x - qbr * BH;
    const int qb_first = CAUSAL ? (a.nqb - 1 - qbr) : qbr;
    const int b = bh / a.H;
    const int hh = bh - b * a.H;
    const int S = a.S;
    const int64_t in_base = (int64_t)b * a.in_sb + (int64_t)hh * a.in_sh;
    const int in_ss = (int)a.in_ss;  // < 2^24 (checked on the host)
    const float *__restrict__ kbase = a.k + in_base;
    const float *__restrict__ vbase = a.v + in_base;

    // Byte offsets of this wave's copy slots within a tile (slot s is copy
    // t = w + 4s, chunk p = 64t + lane).  The element offset r * in_ss + 4c
    // (r < 64, in_ss < 2^24) fits an int; the byte offset, up to
    // 4 * 63 * 2^24 + 4 * D, only fits 32 bits unsigned.
    unsigned koff[T::KSL];
#pragma unroll
    for (int s = 0; s < T::KSL; ++s) {
        const int p = 64 * (w + kWaves * s) + lane;
        const int r = p / T::KCH, c = p - r * T::KCH;
        koff[s] = c < D / 4 ? 4u * (unsigned)(r * in_ss + 4 * c) : 0u;
    }
    unsigned voff[kVoffRegs ? T::VSL : 1];
#pragma unroll
    for (int s = 0; s < (kVoffRegs ? T::VSL : 1); ++s) {
        const int p = 64 * (w + kWaves * s) + lane;
        const int r = p / (D / 4), c = p - r * (D / 4);
        voff[s] = 4u * (unsigned)(r * in_ss + 4 * c);
    }

    // Rows past the sequence end re-read row S-1: their scores are masked,
    // so they contribute exactly 0.  On that (last) tile the offsets are
    // recomputed from an opaque lane index, so that the compiler does not
    // keep a second set live across the loop.
    auto fetch_k = [&](int n0) {
        const __amdgpu_buffer_rsrc_t src = dma_rsrc(kbase + (int64_t)n0 * in_ss);
        const int rmax = S - 1 - n0;
        if (rmax >= kBc - 1) {
#pragma unroll
            for (int s = 0; s < T::KSL; ++s)
                if (w + kWaves * s < T::KCOP) dma16_buf(src, koff[s], Ks + 256 * (w + kWaves * s));
        } else {
            int ln = lane;
            asm volatile("" : "+v"(ln));
#pragma unroll
            for (int s = 0; s < T::KSL; ++s) {
                const int t = w + kWaves * s;
                if (t < T::KCOP) {
                    const int p = 64 * t + ln;
                    const int r = p / T::KCH, c = p - r * T::KCH;
                    const unsigned off = c < D / 4 ? 4u * (unsigned)(min(r, rmax) * in_ss + 4 * c) : 0u;
                    dma16_buf(src, off, Ks + 256 * t);
                }
            }
        }
    };
    auto fetch_v = [&](int n0) {
        const int rmax = S - 1 - n0;
        if (rmax >= kBc - 1) {
#pragma unroll
            for (int s = 0; s < T::VSL; ++s) {
                if constexpr (kVoffRegs)
                    dma16_buf(dma_rsrc(vbase + (int64_t)n0 * in_ss), voff[s],
                              Vs + 256 * (w + kWaves * s));
                else
                    dma16_buf(dma_rsrc(vbase + (int64_t)(n0 + T::VROWS * s) * in_ss), voff[0],
                              Vs + 256 * (w + kWaves * s));
            }
        } else {
            const __amdgpu_buffer_rsrc_t src = dma_rsrc(vbase + (int64_t)n0 * in_ss);
            int ln = lane;
            asm volatile("" : "+v"(ln));
#pragma unroll
            for (int s = 0; s < T::VSL; ++s) {
                const int t = w + kWaves * s;
                const int p = 64 * t + ln;
                const int r = p / (D / 4), c = p - r * (D / 4);
                dma16_buf(src, 4u * (unsigned)(min(r, rmax) * in_ss + 4 * c), Vs + 256 * t);
            }
        }
    };

    // Query block qb; K tile 0 already requested unless first; next: a
    // second block follows (its K tile 0, the same head's, is requested
    // during this block's last tile).
    auto run_block = [&](int qb, bool first, bool next) {
    const int q0 = qb * kBr;
    const int m0 = q0 + 32 * w;
    const int mq = m0 + l32;
    const int kend = CAUSAL ? min(S, q0 + kBr) : S;
    const int ntiles = (kend + kBc - 1) / kBc;
    if (first) fetch_k(0);

    // Q^T operand: lane holds Q[mq][h32*DH + kk] for k-step kk.
    float qr[DH];
    {
        const int mrow = mq < S ? mq : S - 1;
        const float *src = a.q + in_base + (int64_t)mrow * a.in_ss + h32 * DH;
#pragma unroll
        for (int kk = 0; kk < DH; kk += 4) {
            f32x4 t = *(const f32x4 *)(src + kk);
#pragma unroll
            for (int j = 0; j < 4; ++j) qr[kk + j] = t[j];
        }
    }

    f32x16 oacc[DB];
#pragma unroll
    for (int db = 0; db < DB; ++db) oacc[db] = zero16();
    float mrun = -INFINITY;  // reference max of s*c for query mq (see below)
    float lrun = 0.0f;       // this lane half's share of the running sum

    auto tile = [&](int t, auto masked) {
        constexpr bool MASKED = decltype(masked)::value;
        const int n0 = t * kBc;
        wait_vmem();      // this wave's copies of K tile t have landed
        __syncthreads();  // all of K tile t is in LDS; every wave is done with Vs
        fetch_v(n0);
        const bool active = !MASKED || !(CAUSAL && n0 > m0 + 31);  // some key at or before a query
        f32x16 sacc[kBc / 32];
        if (active) {
            // S^T = K . Q^T for two 32-key blocks.
#pragma unroll
            for (int blk = 0; blk < kBc / 32; ++blk) sacc[blk] = zero16();
#pragma unroll
            for (int kk = 0; kk < DH; kk += 4) {
#pragma unroll
                for (int blk = 0; blk < kBc / 32; ++blk) {
                    const f32x4 kf = *(const f32x4 *)&Ks[(32 * blk + l32) * KSTR + h32 * DH + kk];
#pragma unroll
                    for (int j = 0; j < 4; ++j) sacc[blk] = mfma_32x32x2(kf[j], qr[kk + j], sacc[blk]);
                }
            }

            // Mask (diagonal and tail tiles only), tile max of the raw scores.
            const bool need_mask = MASKED && ((n0 + kBc > S) || (CAUSAL && n0 + kBc - 1 > m0));
            if (need_mask) {
#pragma unroll
                for (int blk = 0; blk < kBc / 32; ++blk) {
#pragma unroll
                    for (int i = 0; i < 16; ++i) {
                        const int n = n0 + 32 * blk + acc_row(i, h32);
                        const bool vis = (n < S) & (!CAUSAL | (n <= mq));
                        sacc[blk][i] = vis ? sacc[blk][i] : -INFINITY;
                    }
                }
            }
            float tmax = -INFINITY;
#pragma unroll
            for (int blk = 0; blk < kBc / 32; ++blk)
#pragma unroll
                for (int i = 0; i < 16; ++i) tmax = fmaxf(tmax, sacc[blk][i]);
            tmax = fmaxf(tmax, __shfl_xor(tmax, 32));
            // Scaled tile max (scale >= 0, checked on the host).  The
            // reference max mrun is raised only when some lane's scores would
            // otherwise exceed it by more than 2^8 (lazy rescaling): the
            // result is the same softmax, and most tiles skip the rescale of
            // O.  Tile 0 holds key 0, visible to every query, so it always
            // sets a finite mrun.
            const float tm2 = tmax * a.c;
            if (__ballot(tm2 > mrun + 8.0f) != 0) {
                const float mnew = fmaxf(mrun, tm2);
                const float alpha = __builtin_amdgcn_exp2f(mrun - mnew);
                mrun = mnew;
                lrun *= alpha;
#pragma unroll
                for (int db = 0; db < DB; ++db) oacc[db] *= alpha;
            }
            if (need_mask) {
#pragma unroll
                for (int blk = 0; blk < kBc / 32; ++blk) {
#pragma unroll
                    for (int i = 0; i < 16; ++i) {
                        const float sv = sacc[blk][i];
                        const float p = sv == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(fmaf(sv, a.c, -mrun));
                        sacc[blk][i] = p;
                        lrun += p;
                    }
                }
            } else {
#pragma unroll
                for (int blk = 0; blk < kBc / 32; ++blk) {
#pragma unroll
                    for (int i = 0; i < 16; ++i) {
                        const float p = __builtin_amdgcn_exp2f(fmaf(sacc[blk][i], a.c, -mrun));
                        sacc[blk][i] = p;
                        lrun += p;
                    }
                }
            }
        }
        wait_vmem();      // this wave's copies of V tile t have landed
        __syncthreads();  // all of V tile t is in LDS; every wave is done with Ks
        if (t + 1 < ntiles)
            fetch_k(n0 + kBc);
        else if (next)
            fetch_k(0);
        if (active) {
            // O^T += V^T . P^T; lane l32 covers O^T rows d = DB*l32 + db.
#pragma unroll
            for (int blk = 0; blk < kBc / 32; ++blk) {
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const int nr = 32 * blk + acc_row(i, h32);
                    const typename VecN<DB>::T vf = *(const typename VecN<DB>::T *)&Vs[nr * D + DB * l32];
#pragma unroll
                    for (int db = 0; db < DB; ++db)
                        oacc[db] = mfma_32x32x2(vget<DB>(vf, db), sacc[blk][i], oacc[db]);
                }
            }
        }
    };
    // Causal D = 64: the tiles wholly before the workgroup's first query need
    // no mask for any wave and run a mask-free copy of the loop body; with
    // only the last (diagonal) tiles carrying the mask the kernel fits three
    // workgroups per CU without spilling (146 VGPRs; one loop with the mask
    // test inside needed 178, or spilled 8-10 at three per CU).  Measured:
    // +1 % at config 2, +3 % at S = 4096.  The other instantiations keep one
    // loop (splitting measured -1 % at D = 128 and -2 % for non-causal D = 64).
    int t = 0;
    if constexpr (D == 64 && CAUSAL) {
        for (const int nfull = min(q0 / kBc, ntiles); t < nfull; ++t) tile(t, std::false_type{});
    }
    for (; t < ntiles; ++t) tile(t, std::true_type{});

    const float ltot = lrun + __shfl_xor(lrun, 32);
    if (mq < S) {
        const float inv = 1.0f / ltot;
        float *orow = a.o + (int64_t)b * a.out_sb + (int64_t)hh * a.out_sh + (int64_t)mq * a.out_ss;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int r = acc_row(i, h32);  // O^T row block index -> d = DB*r + db
            typename VecN<DB>::T outv;
            if constexpr (DB == 1) {
                outv = oacc[0][i] * inv;
            } else {
#pragma unroll
                for (int db = 0; db < DB; ++db) outv[db] = oacc[db][i] * inv;
            }
            *(typename VecN<DB>::T *)(orow + DB * r) = outv;
        }
        if (h32 == 0) a.lse[(int64_t)bh * S + mq] = (mrun + log2f(ltot)) * kLn2;
    }
    };
    if constexpr (PAIRQ) {
        const int second = a.nqb - 1 - qb_first;
        run_block(qb_first, true, second != qb_first);
        if (second != qb_first) run_block(second, false, false);
    } else {
        run_block(qb_first, true, false);
    }
}

// S <= 64 (D = 64 and 128, see launch_fwd): one
// wave per (head, 32-query block), four independent
// waves per workgroup (consecutive query blocks of a head share one) and no
// barriers, so that two waves per SIMD overlap one's copies with another's
// products in this HBM-bound regime.  PAIR (64 < S <= 128, D >= 64; see
// launch_fwd): one wave per pair of blocks p and nqb - 1 - p of a head,
// taken one after the other, so that causally every wave has the same
// number of key tiles.  Each wave stages its Q tile, then each 32-key K
// tile, through a private padded LDS slice with coalesced copies
// (buffer_load ... lds: an MFMA operand puts one row per lane, which read
// straight from HBM would touch 64 lines per load), and loads V straight
// into registers in operand order (already row-contiguous across lanes).
// Per tile: S^T = K.Q^T, the online softmax of attn_fwd_kernel,
// O^T += V^T.P^T.  Rows past the sequence end re-read row S-1 (masked).
// Once a tile's K reads are done, the slice takes the next K tile, or after
// a pair's first block the second block's Q rows, while the softmax and
// the V products run (+0.5-3 % at S = 48-128; the V loads, into registers
// still in use, wait for the tile's start, and are waited for only by the
// V products: +1-4 % at S = 32-128).
template <int D>
struct WaveSlice {
    static constexpr int STR = D + 4;                // padded row (floats)
    static constexpr int CH = STR / 4;               // 16-byte chunks per row
    static constexpr int COP = (32 * CH + 63) / 64;  // 1 KiB copies per 32-row tile
    static constexpr int BUF = COP * 256;            // floats per wave slice
};

template <int D, bool CAUSAL, bool PAIR>
__global__ __launch_bounds__(kThreads, 2) void attn_fwd_wave(FwdArgs a)
{
    typedef WaveSlice<D> T;
    constexpr int DH = D / 2;
    constexpr int DB = D / 32;
    typedef typename VecN<DB>::T VT;
    __shared__ float slab[kWaves * T::BUF];
    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int h32 = lane >> 5;
    const int l32 = lane & 31;
    float *__restrict__ buf = slab + w * T::BUF;

    // PAIR: a wave takes query blocks p and nqb - 1 - p of its head (p + 1
    // and nqb - p key tiles causally: the same nqb + 1 for every wave);
    // otherwise one block.
    const int per_head = PAIR ? (a.nqb + 1) / 2 : a.nqb;
    const int item = blockIdx.x * kWaves + w;  // query block (pair) fastest
    if (item >= a.nbh * per_head) return;      // no barriers below: safe to leave
    const int bh = item / per_head;
    const int p0 = item - bh * per_head;
    const int b = bh / a.H;
    const int hh = bh - b * a.H;
    const int S = a.S;
    const int in_ss = (int)a.in_ss;  // < 2^24 (checked on the host)
    const int64_t in_base = (int64_t)b * a.in_sb + (int64_t)hh * a.in_sh;
    const float *__restrict__ vb = a.v + in_base;
    // Query block qb of head bh; q_ready: its Q rows are already being
    // copied into buf; next_qb >= 0: the block that follows, whose Q rows
    // are copied into buf during this block's last tile, once its K reads
    // are done.
    auto block = [&](int qb, bool q_ready, int next_qb) {
    const int m0 = 32 * qb;
    const int mq = m0 + l32;

    // Copies rows r0 .. r0+31 (clamped to S-1) of a (S, D) slab into buf;
    // copy t fills chunks 64t .. 64t+63, a padding or slack chunk re-reads
    // the first chunk.  Offsets are recomputed per call from an opaque lane
    // index, so that they do not stay live in registers.
    auto stage = [&](const float *base, int r0) {
        const __amdgpu_buffer_rsrc_t rs = dma_rsrc(base + (int64_t)r0 * in_ss);
        const int rmax = S - 1 - r0;
        int ln = lane;
        asm volatile("" : "+v"(ln));
#pragma unroll
        for (int t = 0; t < T::COP; ++t) {
            const int p = 64 * t + ln;
            const int r = p / T::CH, c = p - r * T::CH;
            const unsigned off = c < D / 4 ? 4u * (unsigned)(min(r, rmax) * in_ss + 4 * c) : 0u;
            dma16_buf(rs, off, buf + 256 * t);
        }
    };

    // Q^T operand: lane holds Q[mq][h32*DH + kk] for k-step kk.
    if (!q_ready) stage(a.q + in_base, m0);
    wait_vmem();
    float qr[DH];
#pragma unroll
    for (int kk = 0; kk < DH; kk += 4) {
        const f32x4 t = *(const f32x4 *)&buf[l32 * T::STR + h32 * DH + kk];
#pragma unroll
        for (int j = 0; j < 4; ++j) qr[kk + j] = t[j];
    }

    f32x16 oacc[DB];
#pragma unroll
    for (int db = 0; db < DB; ++db) oacc[db] = zero16();
    float mrun = -INFINITY, lrun = 0.0f;

    const int kend = CAUSAL ? min(S, m0 + 32) : S;
    wait_lds();  // this wave's reads of Q are complete before the copy overwrites them
    stage(a.k + in_base, 0);
    for (int n0 = 0; n0 < kend; n0 += 32) {
        VT vr[16];   // V operand for k-step i: V[n0 + acc_row(i, h32)][DB*l32 .. +DB)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            int nv = n0 + acc_row(i, h32);
            nv = nv < S ? nv : S - 1;
            vr[i] = *(const VT *)(vb + (int64_t)nv * a.in_ss + DB * l32);
        }
        // The K tile, copied before these 16 V loads, has landed; the V
        // rows are waited for one by one before the products that read them
        // (the compiler's waits), so the S products and the softmax run
        // while they arrive.
        wait_vmem_n<16>();
        f32x16 sacc = zero16();
#pragma unroll
        for (int kk = 0; kk < DH; kk += 4) {
            const f32x4 kf = *(const f32x4 *)&buf[l32 * T::STR + h32 * DH + kk];
#pragma unroll
            for (int j = 0; j < 4; ++j) sacc = mfma_32x32x2(kf[j], qr[kk + j], sacc);
        }
        if (n0 + 32 < kend) {
            wait_lds();  // this wave's reads of the K tile are complete
            stage(a.k + in_base, n0 + 32);
        } else if (next_qb >= 0) {
            wait_lds();  // the same, before the next block's Q rows
            stage(a.q + in_base, 32 * next_qb);
        }
        const bool need_mask = n0 + 32 > S || (CAUSAL && n0 + 31 > m0);
        if (need_mask) {
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int n = n0 + acc_row(i, h32);
                const bool vis = (n < S) & (!CAUSAL | (n <= mq));
                sacc[i] = vis ? sacc[i] : -INFINITY;
            }
        }
        float tmax = -INFINITY;
#pragma unroll
        for (int i = 0; i < 16; ++i) tmax = fmaxf(tmax, sacc[i]);
        tmax = fmaxf(tmax, __shfl_xor(tmax, 32));
        // Lazy rescaling as in attn_fwd_kernel; tile 0 holds key 0, visible
        // to every query, so it sets a finite mrun.
        const float tm2 = tmax * a.c;
        if (__ballot(tm2 > mrun + 8.0f) != 0) {
            const float mnew = fmaxf(mrun, tm2);
            const float alpha = __builtin_amdgcn_exp2f(mrun - mnew);
            mrun = mnew;
            lrun *= alpha;
#pragma unroll
            for (int db = 0; db < DB; ++db) oacc[db] *= alpha;
        }
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const float sv = sacc[i];
            const float p = need_mask && sv == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(fmaf(sv, a.c, -mrun));
            sacc[i] = p;
            lrun += p;
        }
#pragma unroll
        for (int i = 0; i < 16; ++i)
#pragma unroll
            for (int db = 0; db < DB; ++db) oacc[db] = mfma_32x32x2(vget<DB>(vr[i], db), sacc[i], oacc[db]);
    }

    const float ltot = lrun + __shfl_xor(lrun, 32);
    if (mq < S) {
        const float inv = 1.0f / ltot;
        float *orow = a.o + (int64_t)b * a.out_sb + (int64_t)hh * a.out_sh + (int64_t)mq * a.out_ss;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int r = acc_row(i, h32);  // O^T row block index -> d = DB*r + db
            VT outv;
            if constexpr (DB == 1) {
                outv = oacc[0][i] * inv;
            } else {
#pragma unroll
                for (int db = 0; db < DB; ++db) outv[db] = oacc[db][i] * inv;
            }
            *(VT *)(orow + DB * r) = outv;
        }
        if (h32 == 0) a.lse[(int64_t)bh * S + mq] = (mrun + log2f(ltot)) * kLn2;
    }
    };
    if constexpr (PAIR) {
        const int second = a.nqb - 1 - p0;  // odd nqb: the middle block alone
        block(p0, false, second != p0 ? second : -1);
        if (second != p0) block(second, true, -1);
    } else {
        block(p0, false, -1);
    }
}

// Short sequences (S <= 64): HP heads per workgroup (2 or 4), each with 4/HP
// waves of 32 queries, and key tiles of BC (64, or 32 when HP = 4); the
// tiles of all HP heads sit side by side in LDS and are loaded through
// registers (a sequence has one or two tiles, so there is nothing to
// overlap the copies with).
template <int D, bool CAUSAL, int HP, int BC>
__global__ __launch_bounds__(kThreads, 1) void attn_fwd_packed(FwdArgs a)
{
    static_assert(HP == 2 || HP == 4, "one-head workgroups use attn_fwd_kernel");
    constexpr int DH = D / 2;   // contraction length per lane half (k-steps)
    constexpr int DB = D / 32;  // 32-row blocks of O^T
    constexpr int KSTR = D + 4; // padded K row: conflict-free column reads
    constexpr int QB = kWaves / HP;  // waves (32-query blocks) per head
    constexpr int kBc = BC;
    __shared__ float Ks[HP * kBc * KSTR];
    __shared__ float Vs[HP * kBc * D];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int w = tid >> 6;
    const int h32 = lane >> 5;
    const int l32 = lane & 31;

    const int bh0 = blockIdx.x * HP;
    int bh = bh0 + w / QB;
    // A wave past the last head computes on the last head's data and stores
    // nothing (it still takes part in every barrier).
    const bool head_ok = bh < a.nbh;
    if (!head_ok) bh = a.nbh - 1;
    const int b = bh / a.H;
    const int hh = bh - b * a.H;
    const int S = a.S;
    const int m0 = 32 * (w % QB);
    const int mq = m0 + l32;
    const float *__restrict__ kslab = Ks + (w / QB) * kBc * KSTR;
    const float *__restrict__ vslab = Vs + (w / QB) * kBc * D;

    const int64_t in_base = (int64_t)b * a.in_sb + (int64_t)hh * a.in_sh;
    const float *__restrict__ qp = a.q + in_base;

    // Q^T operand: lane holds Q[mq][h32*DH + kk] for k-step kk.
    float qr[DH];
    {
        const int mrow = mq < S ? mq : S - 1;
        const float *src = qp + (int64_t)mrow * a.in_ss + h32 * DH;
#pragma unroll
        for (int kk = 0; kk < DH; kk += 4) {
            f32x4 t = *(const f32x4 *)(src + kk);
#pragma unroll
            for (int j = 0; j < 4; ++j) qr[kk + j] = t[j];
        }
    }

    f32x16 oacc[DB];
#pragma unroll
    for (int db = 0; db < DB; ++db) oacc[db] = zero16();
    float mrun = -INFINITY;  // reference max of s*c for query mq (see below)
    float lrun = 0.0f;       // this lane half's share of the running sum

    const int kend = CAUSAL ? min(S, 32 * QB) : S;
    const int ntiles = (kend + kBc - 1) / kBc;
    constexpr int kLoads = HP * kBc * D / 4 / kThreads;
    constexpr int kRowsPerLoad = kThreads / (D / 4);
    static_assert(kBc % kRowsPerLoad == 0, "a load row block must lie in one head");
    // Base of the head each tile row block belongs to (head bh0 + hp,
    // clamped to the last head).
    auto head_base = [&](int hp) -> int64_t {
        int h = bh0 + hp;
        if (h >= a.nbh) h = a.nbh - 1;
        const int hb = h / a.H;
        return (int64_t)hb * a.in_sb + (int64_t)(h - hb * a.H) * a.in_sh;
    };

    for (int t = 0; t < ntiles; ++t) {
        // Per-lane offsets below derive from `tid`, which the empty asm makes
        // opaque per tile, so that the compiler recomputes them (a few VALU
        // ops) instead of hoisting them out of the loop and spilling.
        int tid = threadIdx.x;
        asm volatile("" : "+v"(tid));
        const int n0 = t * kBc;
        __syncthreads();
        if (n0 + kBc <= S) {
#pragma unroll
            for (int it = 0; it < kLoads; ++it) {
                const int hp = it * kRowsPerLoad / kBc;  // compile-time
                const int64_t hbase = head_base(hp) + (int64_t)n0 * a.in_ss;
                const int idx = it * kThreads + tid;
                const int r = idx / (D / 4);
                const int c4 = idx - r * (D / 4);
                const int rr = r - hp * kBc;
                const unsigned off = (unsigned)(rr * (int)a.in_ss + 4 * c4);
                *(f32x4 *)&Ks[r * KSTR + 4 * c4] = *(const f32x4 *)(a.k + hbase + off);
                *(f32x4 *)&Vs[r * D + 4 * c4] = *(const f32x4 *)(a.v + hbase + off);
            }
        } else {
#pragma unroll
            for (int it = 0; it < kLoads; ++it) {
                const int hp = it * kRowsPerLoad / kBc;
                const int64_t hbase = head_base(hp) + (int64_t)n0 * a.in_ss;
                const int idx = it * kThreads + tid;
                const int r = idx / (D / 4);
                const int c4 = idx - r * (D / 4);
                const int rr = r - hp * kBc;
                f32x4 kv = {0.f, 0.f, 0.f, 0.f}, vv = {0.f, 0.f, 0.f, 0.f};
                if (n0 + rr < S) {
                    const unsigned off = (unsigned)(rr * (int)a.in_ss + 4 * c4);
                    kv = *(const f32x4 *)(a.k + hbase + off);
                    vv = *(const f32x4 *)(a.v + hbase + off);
                }
                *(f32x4 *)&Ks[r * KSTR + 4 * c4] = kv;
                *(f32x4 *)&Vs[r * D + 4 * c4] = vv;
            }
        }
        __syncthreads();
        if (CAUSAL && n0 > m0 + 31) continue;  // tile wholly above this wave's diagonal

        // S^T = K . Q^T for two 32-key blocks.
        f32x16 sacc[kBc / 32];
#pragma unroll
        for (int blk = 0; blk < kBc / 32; ++blk) sacc[blk] = zero16();
#pragma unroll
        for (int kk = 0; kk < DH; kk += 4) {
#pragma unroll
            for (int blk = 0; blk < kBc / 32; ++blk) {
                const f32x4 kf = *(const f32x4 *)&kslab[(32 * blk + l32) * KSTR + h32 * DH + kk];
#pragma unroll
                for (int j = 0; j < 4; ++j) sacc[blk] = mfma_32x32x2(kf[j], qr[kk + j], sacc[blk]);
            }
        }

        // Mask (diagonal and tail tiles only), tile max of the raw scores.
        const bool need_mask = (n0 + kBc > S) || (CAUSAL && n0 + kBc - 1 > m0);
        if (need_mask) {
#pragma unroll
            for (int blk = 0; blk < kBc / 32; ++blk) {
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const int n = n0 + 32 * blk + acc_row(i, h32);
                    const bool vis = (n < S) & (!CAUSAL | (n <= mq));
                    sacc[blk][i] = vis ? sacc[blk][i] : -INFINITY;
                }
            }
        }
        float tmax = -INFINITY;
#pragma unroll
        for (int blk = 0; blk < kBc / 32; ++blk)
#pragma unroll
            for (int i = 0; i < 16; ++i) tmax = fmaxf(tmax, sacc[blk][i]);
        tmax = fmaxf(tmax, __shfl_xor(tmax, 32));
        // Scaled tile max (scale >= 0, checked on the host).  The reference
        // max mrun is raised only when some lane's scores would otherwise
        // exceed it by more than 2^8 (lazy rescaling): the result is the same
        // softmax, and most tiles skip the rescale of O.  Tile 0 holds key 0,
        // visible to every query, so it always sets a finite mrun.
        const float tm2 = tmax * a.c;
        if (__ballot(tm2 > mrun + 8.0f) != 0) {
            const float mnew = fmaxf(mrun, tm2);
            const float alpha = __builtin_amdgcn_exp2f(mrun - mnew);
            mrun = mnew;
            lrun *= alpha;
#pragma unroll
            for (int db = 0; db < DB; ++db) oacc[db] *= alpha;
        }
        if (need_mask) {
#pragma unroll
            for (int blk = 0; blk < kBc / 32; ++blk) {
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const float sv = sacc[blk][i];
                    const float p = sv == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(fmaf(sv, a.c, -mrun));
                    sacc[blk][i] = p;
                    lrun += p;
                }
            }
        } else {
#pragma unroll
            for (int blk = 0; blk < kBc / 32; ++blk) {
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const float p = __builtin_amdgcn_exp2f(fmaf(sacc[blk][i], a.c, -mrun));
                    sacc[blk][i] = p;
                    lrun += p;
                }
            }
        }

        // O^T += V^T . P^T; lane l32 covers O^T rows d = DB*l32 + db.
#pragma unroll
        for (int blk = 0; blk < kBc / 32; ++blk) {
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int nr = 32 * blk + acc_row(i, h32);
                const typename VecN<DB>::T vf = *(const typename VecN<DB>::T *)&vslab[nr * D + DB * l32];
#pragma unroll
                for (int db = 0; db < DB; ++db)
                    oacc[db] = mfma_32x32x2(vget<DB>(vf, db), sacc[blk][i], oacc[db]);
            }
        }
    }

    const float ltot = lrun + __shfl_xor(lrun, 32);
    if (mq < S && head_ok) {
        const float inv = 1.0f / ltot;
        float *orow = a.o + (int64_t)b * a.out_sb + (int64_t)hh * a.out_sh + (int64_t)mq * a.out_ss;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int r = acc_row(i, h32);  // O^T row block index -> d = DB*r + db
            typename VecN<DB>::T outv;
            if constexpr (DB == 1) {
                outv = oacc[0][i] * inv;
            } else {
#pragma unroll
                for (int db = 0; db < DB; ++db) outv[db] = oacc[db][i] * inv;
            }
            *(typename VecN<DB>::T *)(orow + DB * r) = outv;
        }
        if (h32 == 0) a.lse[(int64_t)bh * S + mq] = (mrun + log2f(ltot)) * kLn2;
    }
}

// Split-key forward for launches too small to fill the GPU (few heads of
// moderate length, config 1's shape): a workgroup owns 32 queries of one
// head and its 4 waves walk interleaved 32-key tiles (wave w takes tiles
// w, w+4, ...).  A wave loads its tile's K and V straight into registers in
// MFMA operand order (no LDS, no barriers in the loop; the next tile's loads
// are issued before the current tile's products), runs the same online
// softmax as attn_fwd_kernel, and the four partial states are merged at the
// end through LDS:  M = max_w m_w,  L = sum_w l_w 2^(m_w - M),
// O = sum_w O_w 2^(m_w - M) / L.  A wave that sees no key ends with
// m = -inf, l = 0, O = 0 and drops out of the merge; wave 0's first tile
// holds key 0, visible to every query, so M is finite.
template <int D, bool CAUSAL>
__global__ __launch_bounds__(kThreads, 1) void attn_fwd_split(FwdArgs a)
{
    constexpr int DH = D / 2;
    constexpr int DB = D / 32;
    typedef typename VecN<DB>::T VT;
    __shared__ float part[kWaves * D * 32];  // O^T partials [w][d][query]
    __shared__ float mst[kWaves * 32], lst[kWaves * 32];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int w = tid >> 6;
    const int h32 = lane >> 5;
    const int l32 = lane & 31;

    const int nqb = a.nqb;  // 32-query blocks per head
    const int bh = blockIdx.x / nqb;
    const int qb = blockIdx.x - bh * nqb;
    const int b = bh / a.H;
    const int hh = bh - b * a.H;
    const int S = a.S;
    const int m0 = 32 * qb;
    const int mq = m0 + l32;
    const int64_t in_base = (int64_t)b * a.in_sb + (int64_t)hh * a.in_sh;

    float qr[DH];
    {
        const int mrow = mq < S ? mq : S - 1;
        const float *src = a.q + in_base + (int64_t)mrow * a.in_ss + 4 * h32;
#pragma unroll
        for (int kk = 0; kk < DH; kk += 4) {
            const f32x4 t = *(const f32x4 *)(src + 2 * kk);
#pragma unroll
            for (int j = 0; j < 4; ++j) qr[kk + j] = t[j];
        }
    }

    // K operand: lane holds K[n0 + l32][d] for k-step kk, with
    // d = 8 (kk / 4) + 4 h32 + kk % 4 (Q^T likewise), so that the two lanes
    // of a row read 32 contiguous bytes per load (32 cache lines per load
    // instruction rather than 64); V operand for k-step i:
    // V[n0 + acc_row(i, h32)][DB*l32 .. +DB).  Rows past S are clamped
    // (their scores are masked).
    float kr[DH];
    VT vr[16];
    auto load_tile = [&](int n0, float (&kd)[DH], VT (&vd)[16]) {
        const int nk = n0 + l32 < S ? n0 + l32 : S - 1;
        const float *ks = a.k + in_base + (int64_t)nk * a.in_ss + 4 * h32;
#pragma unroll
        for (int kk = 0; kk < DH; kk += 4) {
            const f32x4 t = *(const f32x4 *)(ks + 2 * kk);
#pragma unroll
            for (int j = 0; j < 4; ++j) kd[kk + j] = t[j];
        }
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            int nv = n0 + acc_row(i, h32);
            nv = nv < S ? nv : S - 1;
            vd[i] = *(const VT *)(a.v + in_base + (int64_t)nv * a.in_ss + DB * l32);
        }
    };

    f32x16 oacc[DB];
#pragma unroll
    for (int db = 0; db < DB; ++db) oacc[db] = zero16();
    float mrun = -INFINITY, lrun = 0.0f;

    const int kend = CAUSAL ? min(S, m0 + 32) : S;
    const int ntiles = (kend + 31) / 32;
    int t = w;
    if (t < ntiles) load_tile(32 * t, kr, vr);
    for (; t < ntiles; t += kWaves) {
        const int n0 = 32 * t;
        float kn[DH];
        VT vn[16];
        const bool more = t + kWaves < ntiles;
        if (more) load_tile(n0 + 32 * kWaves, kn, vn);

        f32x16 sacc = zero16();
#pragma unroll
        for (int kk = 0; kk < DH; ++kk) sacc = mfma_32x32x2(kr[kk], qr[kk], sacc);
        if (n0 + 32 > S || (CAUSAL && n0 + 31 > m0)) {
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int n = n0 + acc_row(i, h32);
                const bool vis = (n < S) & (!CAUSAL | (n <= mq));
                sacc[i] = vis ? sacc[i] : -INFINITY;
            }
        }
        float tmax = -INFINITY;
#pragma unroll
        for (int i = 0; i < 16; ++i) tmax = fmaxf(tmax, sacc[i]);
        tmax = fmaxf(tmax, __shfl_xor(tmax, 32));
        const float tm2 = tmax * a.c;
        // Same lazy rescaling as attn_fwd_kernel; a wave's first tile may be
        // wholly masked for some queries (tm2 = -inf), which leaves mrun
        // unchanged.
        if (__ballot(tm2 > mrun + 8.0f) != 0) {
            const float mnew = fmaxf(mrun, tm2);
            const float alpha = mrun == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mrun - mnew);
            mrun = mnew;
            lrun *= alpha;
#pragma unroll
            for (int db = 0; db < DB; ++db) oacc[db] *= alpha;
        }
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const float sv = sacc[i];
            const float p = sv == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(fmaf(sv, a.c, -mrun));
            sacc[i] = p;
            lrun += p;
        }
#pragma unroll
        for (int i = 0; i < 16; ++i)
#pragma unroll
            for (int db = 0; db < DB; ++db) oacc[db] = mfma_32x32x2(vget<DB>(vr[i], db), sacc[i], oacc[db]);
        if (more) {
#pragma unroll
            for (int kk = 0; kk < DH; ++kk) kr[kk] = kn[kk];
#pragma unroll
            for (int i = 0; i < 16; ++i) vr[i] = vn[i];
        }
    }

    // Publish this wave's state: m (in scaled log2 units), l, O^T.
    const float ltot = lrun + __shfl_xor(lrun, 32);
    if (h32 == 0) {
        mst[w * 32 + l32] = mrun;
        lst[w * 32 + l32] = ltot;
    }
#pragma unroll
    for (int i = 0; i < 16; ++i)
#pragma unroll
        for (int db = 0; db < DB; ++db)
            part[(w * D + DB * acc_row(i, h32) + db) * 32 + l32] = oacc[db][i];
    __syncthreads();

    // Merge: wave w writes d in [w*D/4, (w+1)*D/4) of query l32; lane half
    // h32 takes the first or second half of that range.
    float M = -INFINITY;
#pragma unroll
    for (int v = 0; v < kWaves; ++v) M = fmaxf(M, mst[v * 32 + l32]);
    float f[kWaves], L = 0.0f;
#pragma unroll
    for (int v = 0; v < kWaves; ++v) {
        const float mv = mst[v * 32 + l32];
        f[v] = mv == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mv - M);
        L += f[v] * lst[v * 32 + l32];
    }
    if (mq < S) {
        const float inv = 1.0f / L;
        constexpr int DQ = D / 8;  // d values per lane
        const int d0 = w * (D / 4) + h32 * DQ;
        float *orow = a.o + (int64_t)b * a.out_sb + (int64_t)hh * a.out_sh + (int64_t)mq * a.out_ss + d0;
#pragma unroll
        for (int d4 = 0; d4 < DQ; d4 += 4) {
            f32x4 o4;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                float acc = 0.0f;
#pragma unroll
                for (int v = 0; v < kWaves; ++v) acc += f[v] * part[(v * D + d0 + d4 + j) * 32 + l32];
                o4[j] = acc * inv;
            }
            *(f32x4 *)(orow + d4) = o4;
        }
        if (w == 0 && h32 == 0) a.lse[(int64_t)bh * S + mq] = (M + log2f(L)) * kLn2;
    }
}

__device__ __forceinline__ f32x4 mfma16(float a, float b, f32x4 c)
{
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// attn_fwd_split at 16 queries per workgroup, for launches with at most one
// such workgroup per CU (config 1's B1 H4 S256: 64 workgroups against 32):
// every product on v_mfma_f32_16x16x4f32, so a wave's 16 x 32 tile costs
// half the matrix-core time of the 32 x 32 one and a query block spreads
// over twice the CUs, with no exchange between workgroups.
// 16 x 16 x 4 placement (lane l = n + 16 g): A[m][k] from lane m + 16k,
// B[k][n] from lane n + 16k, C[m][n] in lane n + 16(m/4), register m % 4.
//   S^T (keys x queries) = K . Q^T, per 16-key block: lane (n, g) supplies
//     K[key n][d] and Q[query n][d] at k-step s, d = 16 (s / 4) + 4g + s % 4
//     (see load_tile);  C: lane (query n, g), register r <-> key 4g + r of
//     the block.
//   O^T (d x queries) += V^T . P^T, per 16-key block and k-step r: the
//     B operand is P^T[key 4g + r][query n], i.e. register r of the S^T
//     accumulator; the A operand of column block j is V[key 4g + r][E n + j]
//     (E = D/16: lane n loads E consecutive floats of the row), so that
//     output register r of block j in lane (n, g) is O[query n][E(4g + r) + j].
// The online softmax, lazy rescaling and final merge are attn_fwd_split's.
template <int D, bool CAUSAL, int NW>
__global__ __launch_bounds__(64 * NW, 1) void attn_fwd_split16(FwdArgs a)
{
    constexpr int DQ = D / 4;   // k-steps of S per 16-key block
    constexpr int E = D / 16;   // column blocks of O^T; floats of a V row per lane
    __shared__ float part[NW * D * 16];  // O^T partials [w][d][query]
    __shared__ float mst[NW * 16], lst[NW * 16];
    __shared__ float qs[NW == 4 ? 16 * (D + 4) : 1];  // the block's Q rows, read once for all waves

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n = lane & 15;
    const int g = lane >> 4;

    const int nqb = a.nqb;  // 16-query blocks per head
    const int bh = blockIdx.x / nqb;
    const int qb = blockIdx.x - bh * nqb;
    const int b = bh / a.H;
    const int hh = bh - b * a.H;
    const int S = a.S;
    const int m0 = 16 * qb;
    const int mq = m0 + n;
    const int64_t in_base = (int64_t)b * a.in_sb + (int64_t)hh * a.in_sh;

    // Four waves: the block's Q rows (16 x D) are read once, 16 bytes per
    // thread, into LDS ahead of the key tiles' loads, and every wave takes
    // its operand from there after one barrier (each wave reading them
    // itself made a quarter of a CU's loads repeats): -3.5 to -5 % at
    // S = 128-300.  Eight waves read their own (the barrier measured +5 %
    // at config 1).
    constexpr bool kQShared = NW == 4;
    constexpr int QPIECES = 16 * D / 4;
    constexpr int QPT = (QPIECES + 64 * NW - 1) / (64 * NW);  // pieces per thread
    f32x4 qpiece[QPT];
    float qr[DQ];
    if constexpr (kQShared) {
#pragma unroll
        for (int u = 0; u < QPT; ++u) {
            // Unconditional (a thread past the pieces re-reads one), so that
            // the wait for them below counts exactly the key tile's loads.
            const int pc = (tid + 64 * NW * u) % QPIECES;
            const int qrow = pc / (D / 4), qcol = 4 * (pc - qrow * (D / 4));
            qpiece[u] = *(const f32x4 *)(a.q + in_base + (int64_t)min(m0 + qrow, S - 1) * a.in_ss + qcol);
        }
    } else {
        const int mrow = mq < S ? mq : S - 1;
        const float *src = a.q + in_base + (int64_t)mrow * a.in_ss + 4 * g;
#pragma unroll
        for (int s4 = 0; s4 < DQ; s4 += 4) {
            const f32x4 t = *(const f32x4 *)(src + 4 * s4);
#pragma unroll
            for (int j = 0; j < 4; ++j) qr[s4 + j] = t[j];
        }
    }

    // A 32-key tile: K rows n0 + 16c + n, V rows n0 + 16c + 4g + r (columns
    // E n ..); rows past S clamped (masked).  K-step s of lane group g
    // contracts d = 16 (s / 4) + 4g + s % 4, for Q as for K, so that the
    // four lanes of a row read 64 contiguous bytes per load: 16 cache lines
    // per load instruction, where a contiguous quarter of d per lane group
    // touches up to 64.
    float kr[2][DQ];
    float vr[2][4][E];
    auto load_tile = [&](int n0, float (&kd)[2][DQ], float (&vd)[2][4][E]) {
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            const int nk = min(n0 + 16 * c + n, S - 1);
            const float *ks = a.k + in_base + (int64_t)nk * a.in_ss + 4 * g;
#pragma unroll
            for (int s4 = 0; s4 < DQ; s4 += 4) {
                const f32x4 t = *(const f32x4 *)(ks + 4 * s4);
#pragma unroll
                for (int j = 0; j < 4; ++j) kd[c][s4 + j] = t[j];
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int nv = min(n0 + 16 * c + 4 * g + r, S - 1);
                const float *vs = a.v + in_base + (int64_t)nv * a.in_ss + E * n;
#pragma unroll
                for (int j4 = 0; j4 < E; j4 += 4) {
                    const f32x4 t = *(const f32x4 *)(vs + j4);
#pragma unroll
                    for (int j = 0; j < 4; ++j) vd[c][r][j4 + j] = t[j];
                }
            }
        }
    };

    f32x4 oacc[E];
#pragma unroll
    for (int j = 0; j < E; ++j) oacc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
    float mrun = -INFINITY, lrun = 0.0f;

    const int kend = CAUSAL ? min(S, m0 + 16) : S;
    const int ntiles = (kend + 31) / 32;
    int t = w;
    if constexpr (kQShared) {
        load_tile(32 * min(t, ntiles - 1), kr, vr);  // a wave without a tile re-reads the last (unused)
#pragma unroll
        for (int u = 0; u < QPT; ++u) {
            // Every thread writes (one past the pieces writes the same bits
            // to the same place), so the load is not sunk behind the tile's.
            const int pc = (tid + 64 * NW * u) % QPIECES;
            const int qrow = pc / (D / 4), qcol = 4 * (pc - qrow * (D / 4));
            *(f32x4 *)&qs[qrow * (D + 4) + qcol] = qpiece[u];
        }
        __syncthreads();
#pragma unroll
        for (int s4 = 0; s4 < DQ; s4 += 4) {
            const f32x4 tq = *(const f32x4 *)&qs[n * (D + 4) + 4 * s4 + 4 * g];
#pragma unroll
            for (int j = 0; j < 4; ++j) qr[s4 + j] = tq[j];
        }
    } else {
        if (t < ntiles) load_tile(32 * t, kr, vr);
    }
    for (; t < ntiles; t += NW) {
        const int n0 = 32 * t;
        float kn[2][DQ];
        float vn[2][4][E];
        const bool more = t + NW < ntiles;
        if (more) load_tile(n0 + 32 * NW, kn, vn);

        f32x4 sacc[2];
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            sacc[c] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int s = 0; s < DQ; ++s) sacc[c] = mfma16(kr[c][s], qr[s], sacc[c]);
        }
        if (n0 + 32 > S || (CAUSAL && n0 + 31 > m0)) {
#pragma unroll
            for (int c = 0; c < 2; ++c)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int key = n0 + 16 * c + 4 * g + r;
                    const bool vis = (key < S) & (!CAUSAL | (key <= mq));
                    sacc[c][r] = vis ? sacc[c][r] : -INFINITY;
                }
        }
        float tmax = -INFINITY;
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
            for (int r = 0; r < 4; ++r) tmax = fmaxf(tmax, sacc[c][r]);
        tmax = fmaxf(tmax, __shfl_xor(tmax, 16));
        tmax = fmaxf(tmax, __shfl_xor(tmax, 32));
        const float tm2 = tmax * a.c;
        if (__ballot(tm2 > mrun + 8.0f) != 0) {
            const float mnew = fmaxf(mrun, tm2);
            const float alpha = mrun == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mrun - mnew);
            mrun = mnew;
            lrun *= alpha;
#pragma unroll
            for (int j = 0; j < E; ++j) oacc[j] *= alpha;
        }
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float sv = sacc[c][r];
                const float p = sv == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(fmaf(sv, a.c, -mrun));
                sacc[c][r] = p;
                lrun += p;
            }
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
            for (int r = 0; r < 4; ++r)
#pragma unroll
                for (int j = 0; j < E; ++j) oacc[j] = mfma16(vr[c][r][j], sacc[c][r], oacc[j]);
        if (more) {
#pragma unroll
            for (int c = 0; c < 2; ++c) {
#pragma unroll
                for (int s = 0; s < DQ; ++s) kr[c][s] = kn[c][s];
#pragma unroll
                for (int r = 0; r < 4; ++r)
#pragma unroll
                    for (int j = 0; j < E; ++j) vr[c][r][j] = vn[c][r][j];
            }
        }
    }

    // Publish this wave's state: m (scaled log2 units), l summed over the
    // four lane groups, O^T.
    float ltot = lrun + __shfl_xor(lrun, 16);
    ltot += __shfl_xor(ltot, 32);
    if (g == 0) {
        mst[w * 16 + n] = mrun;
        lst[w * 16 + n] = ltot;
    }
#pragma unroll
    for (int j = 0; j < E; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) part[(w * D + E * (4 * g + r) + j) * 16 + n] = oacc[j][r];
    __syncthreads();

    // Merge: thread (w, g) writes d in [DPT (4w + g), DPT (4w + g) + DPT)
    // of query n.
    constexpr int DPT = D / (4 * NW);
    static_assert(DPT == 2 || DPT % 4 == 0, "merge stores are 8 or 16 bytes");
    float M = -INFINITY;
#pragma unroll
    for (int v = 0; v < NW; ++v) M = fmaxf(M, mst[v * 16 + n]);
    float f[NW], L = 0.0f;
#pragma unroll
    for (int v = 0; v < NW; ++v) {
        const float mv = mst[v * 16 + n];
        f[v] = mv == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mv - M);
        L += f[v] * lst[v * 16 + n];
    }
    if (mq < S) {
        const float inv = 1.0f / L;
        const int d0 = DPT * (4 * w + g);
        float *orow = a.o + (int64_t)b * a.out_sb + (int64_t)hh * a.out_sh + (int64_t)mq * a.out_ss + d0;
        constexpr int VW = DPT == 2 ? 2 : 4;
#pragma unroll
        for (int d4 = 0; d4 < DPT; d4 += VW) {
            typename VecN<VW>::T ov;
#pragma unroll
            for (int j = 0; j < VW; ++j) {
                float acc = 0.0f;
#pragma unroll
                for (int v = 0; v < NW; ++v) acc += f[v] * part[(v * D + d0 + d4 + j) * 16 + n];
                ov[j] = acc * inv;
            }
            *(typename VecN<VW>::T *)(orow + d4) = ov;
        }
        if (w == 0 && g == 0) a.lse[(int64_t)bh * S + mq] = (M + log2f(L)) * kLn2;
    }
}

// 64 < S <= 128 at D = 64 and 128 over many heads: one persistent
// workgroup of 8 waves per CU walks whole heads.  A head's K and V (at most
// 128 rows) are staged in LDS once, from registers that were filled with
// that head's rows while the previous head was multiplied (4 threads per
// row, coalesced), so each of Q, K, V is read from HBM once.  A wave owns
// one 16-query chunk; causally the hardware's placement of waves w and
// w + 4 on one SIMD gives SIMD j the chunks j and nch - 1 - j, which see
// nch + 1 key chunks together (9 at S = 128 on every SIMD), with no
// lockstep between waves (one barrier pair per head, around the staging).
// The products are attn_fwd_split16's (v_mfma_f32_16x16x4f32; placement
// documented there) with K and V read from LDS: per key chunk,
// S^T = K . Q^T (16 keys x 16 queries), the online softmax with lazy
// rescaling, O^T += V^T . P^T; masked work is cut at 16 x 16.
template <int D>
struct HeadTile {
    static constexpr int KSTR = D + 4;  // padded K row
    static constexpr int PER = D / 4;   // floats of a K or V row per staging thread
};

template <int D, bool CAUSAL>
__global__ __launch_bounds__(512, D == 64 ? 2 : 1) void attn_fwd_head(FwdArgs a)
{
    typedef HeadTile<D> T;
    constexpr int DQ = D / 4;  // k-steps of S per key chunk
    constexpr int E = D / 16;  // column blocks of O^T; floats of a V row per lane
    constexpr int KSTR = T::KSTR, PER = T::PER;
    __shared__ float Ks[128 * KSTR];
    __shared__ float Vs[128 * D];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n = lane & 15;
    const int g = lane >> 4;
    const int S = a.S;
    const int nch = (S + 15) >> 4;
    // This wave's query chunk.  Waves w and w + 4 share a SIMD.  Causal:
    // SIMD j < ceil(nch / 2) takes chunks j and nch - 1 - j, which see
    // nch + 1 key chunks together.  Non-causal: chunk w.
    const int sj = w & 3, second = w >> 2;
    int c;
    bool active;
    if (CAUSAL) {
        c = second ? nch - 1 - sj : sj;
        active = 2 * sj < nch && (!second || nch - 1 - sj > sj);
    } else {
        c = w;
        active = w < nch;
    }
    const int m0 = 16 * c;
    const int mq = m0 + n;
    const int srow = tid >> 2, spart = tid & 3;  // staging: K / V row and quarter
    const int srow_c = min(srow, S - 1);          // rows past S re-read row S - 1 (masked)
    const int qrow_c = min(mq, S - 1);

    f32x4 kp[PER / 4], vp[PER / 4], qp[DQ / 4];
    auto prefetch_kv = [&](int bh) {
        const int b = bh / a.H;
        const int64_t base = (int64_t)b * a.in_sb + (int64_t)(bh - b * a.H) * a.in_sh;
        const float *ks = a.k + base + (int64_t)srow_c * a.in_ss + PER * spart;
        const float *vs = a.v + base + (int64_t)srow_c * a.in_ss + PER * spart;
#pragma unroll
        for (int i = 0; i < PER / 4; ++i) {
            kp[i] = *(const f32x4 *)(ks + 4 * i);
            vp[i] = *(const f32x4 *)(vs + 4 * i);
        }
    };
    auto prefetch_q = [&](int bh) {
        const int b = bh / a.H;
        const int64_t base = (int64_t)b * a.in_sb + (int64_t)(bh - b * a.H) * a.in_sh;
        const float *qs = a.q + base + (int64_t)qrow_c * a.in_ss + DQ * g;
#pragma unroll
        for (int i = 0; i < DQ / 4; ++i) qp[i] = *(const f32x4 *)(qs + 4 * i);
    };
    auto prefetch = [&](int bh) {
        prefetch_kv(bh);
        if (active) prefetch_q(bh);
    };

    const int nbh = a.nbh;
    int bh = blockIdx.x;
    if (bh < nbh) prefetch(bh);
    for (; bh < nbh; bh += gridDim.x) {
        __syncthreads();  // the previous head's products are done with Ks, Vs
#pragma unroll
        for (int i = 0; i < PER / 4; ++i) {
            *(f32x4 *)&Ks[srow * KSTR + PER * spart + 4 * i] = kp[i];
            *(f32x4 *)&Vs[srow * D + PER * spart + 4 * i] = vp[i];
        }
        float qr[DQ];
#pragma unroll
        for (int i = 0; i < DQ / 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) qr[4 * i + j] = qp[i][j];
        __syncthreads();
        // The next head's K and V rows are requested after the barrier, so
        // that no wave waits at it for the others' issue (+1-3 % at
        // S = 72-112); its Q rows only after this wave's last key chunk
        // (+2-7 % at S = 80-128: fewer loads queued while every wave starts
        // its products, and the waves, whose chunk counts differ, issue
        // them at different times).
        const bool has_next = bh + (int)gridDim.x < nbh;
        if (has_next) prefetch_kv(bh + gridDim.x);
        if (!active) continue;

        f32x4 oacc[E];
#pragma unroll
        for (int j = 0; j < E; ++j) oacc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
        float mrun = -INFINITY, lrun = 0.0f;
        const int kc_end = CAUSAL ? c : nch - 1;
        for (int kc = 0; kc <= kc_end; ++kc) {
            const int k0 = 16 * kc;
            f32x4 sacc = {0.f, 0.f, 0.f, 0.f};
            const float *krow = &Ks[(k0 + n) * KSTR + DQ * g];
#pragma unroll
            for (int s4 = 0; s4 < DQ; s4 += 4) {
                const f32x4 kf = *(const f32x4 *)(krow + s4);
#pragma unroll
                for (int j = 0; j < 4; ++j) sacc = mfma16(kf[j], qr[s4 + j], sacc);
            }
            if ((CAUSAL && kc == c) || k0 + 16 > S) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int key = k0 + 4 * g + r;
                    const bool vis = (key < S) & (!CAUSAL | (key <= mq));
                    sacc[r] = vis ? sacc[r] : -INFINITY;
                }
            }
            float tmax = fmaxf(fmaxf(sacc[0], sacc[1]), fmaxf(sacc[2], sacc[3]));
            tmax = fmaxf(tmax, __shfl_xor(tmax, 16));
            tmax = fmaxf(tmax, __shfl_xor(tmax, 32));
            const float tm2 = tmax * a.c;
            if (__ballot(tm2 > mrun + 8.0f) != 0) {
                const float mnew = fmaxf(mrun, tm2);
                const float alpha = mrun == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mrun - mnew);
                mrun = mnew;
                lrun *= alpha;
#pragma unroll
                for (int j = 0; j < E; ++j) oacc[j] *= alpha;
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float sv = sacc[r];
                const float p = sv == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(fmaf(sv, a.c, -mrun));
                sacc[r] = p;
                lrun += p;
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float *vrow = &Vs[(k0 + 4 * g + r) * D + E * n];
#pragma unroll
                for (int j4 = 0; j4 < E; j4 += 4) {
                    const f32x4 vf = *(const f32x4 *)(vrow + j4);
#pragma unroll
                    for (int j = 0; j < 4; ++j) oacc[j4 + j] = mfma16(vf[j], sacc[r], oacc[j4 + j]);
                }
            }
        }
        if (has_next) prefetch_q(bh + gridDim.x);

        float ltot = lrun + __shfl_xor(lrun, 16);
        ltot += __shfl_xor(ltot, 32);
        if (mq < S) {
            const int b = bh / a.H;
            const int hh = bh - b * a.H;
            const float inv = 1.0f / ltot;
            float *orow = a.o + (int64_t)b * a.out_sb + (int64_t)hh * a.out_sh + (int64_t)mq * a.out_ss;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
#pragma unroll
                for (int j4 = 0; j4 < E; j4 += 4) {
                    f32x4 o4;
#pragma unroll
                    for (int j = 0; j < 4; ++j) o4[j] = oacc[j4 + j][r] * inv;
                    *(f32x4 *)(orow + E * (4 * g + r) + j4) = o4;
                }
            }
            if (g == 0) a.lse[(int64_t)bh * S + mq] = (mrun + log2f(ltot)) * kLn2;
        }
    }
}

template <int D, bool CAUSAL>
int launch_fwd(FwdArgs args, int64_t nbh)
{
    // A launch that would leave most CUs idle (and is longer than the
    // packed short-sequence case) splits the keys across waves instead, at
    // 16 queries per workgroup where that still fits one workgroup per CU.
    const int64_t regular = (args.S + kBr - 1) / kBr * nbh;
    if (args.S > 64 && regular * 4 <= 256) {
        if constexpr (D >= 64) {
            const int64_t nqb16 = (args.S + 15) / 16;
            const int ncu = device_cu_count();
            if (nqb16 * nbh <= (ncu > 0 ? ncu : 256)) {
                args.nqb = (int)nqb16;
                // Eight waves (one 32-key tile each at config 1's S = 256)
                // where a D = 64 wave would otherwise walk two or more tiles.
                if constexpr (D == 64) {
                    if (args.S > 4 * 32) {
                        hipLaunchKernelGGL((attn_fwd_split16<D, CAUSAL, 8>), dim3((unsigned)(args.nqb * nbh)),
                                           dim3(512), 0, 0, args);
                        return launch_ok("attn_fwd_split16_w8") ? EMBER_OK : EMBER_ERR_DEVICE;
                    }
                }
                hipLaunchKernelGGL((attn_fwd_split16<D, CAUSAL, 4>), dim3((unsigned)(args.nqb * nbh)),
                                   dim3(kThreads), 0, 0, args);
                return launch_ok("attn_fwd_split16") ? EMBER_OK : EMBER_ERR_DEVICE;
            }
        }
        args.nqb = (args.S + 31) / 32;
        hipLaunchKernelGGL((attn_fwd_split<D, CAUSAL>), dim3((unsigned)(args.nqb * nbh)), dim3(kThreads),
                           0, 0, args);
        return launch_ok("attn_fwd_split") ? EMBER_OK : EMBER_ERR_DEVICE;
    }
    // D = 64, causal 64 < S <= 128 and non-causal 64 < S <= 80: persistent
    // workgroups over whole heads (K, V read once).  Measured at 2^20 query
    // rows against the paired-wave kernel: causal S = 128 3.71 -> 4.30 TB/s,
    // S = 112 3.36 -> 4.26, S = 80 3.69 -> 4.03, S = 96 4.12 -> 4.15;
    // non-causal S = 72 2.62 -> 3.19, S = 80 2.81 -> 3.55; non-causal S = 96
    // (3.06 against 3.21) and S = 128 (3.06 against the workgroup kernel's
    // 3.29) keep the kernels below.  At D = 128 the staged head fills a CU's
    // LDS alone and measured 14 % slower than the paired waves.
    if constexpr (D == 64) {
        if (args.S > 64 && (CAUSAL ? args.S <= 128 : args.S <= 80)) {
            const int ncu = device_cu_count();
            const int64_t slots = (int64_t)(ncu > 0 ? ncu : 256) * (D == 64 ? 2 : 1);
            hipLaunchKernelGGL((attn_fwd_head<D, CAUSAL>), dim3((unsigned)(nbh < slots ? nbh : slots)), dim3(512),
                               0, 0, args);
            return launch_ok("attn_fwd_head") ? EMBER_OK : EMBER_ERR_DEVICE;
        }
    }
    // 64 < S <= 96, and causal S <= 128 (D >= 64): one wave per pair of
    // 32-query blocks.  The 128-query workgroups leave a quarter or more of
    // their waves without rows at S <= 96, and causally their waves have 1
    // to 4 key tiles (in lockstep) where a pair has the same 5.  Measured
    // (B*H = 8192 heads at S = 80 and 96): +32-36 % causal, +15-17 %
    // non-causal; causal S = 112 and 128: +3 % and equal; non-causal
    // S = 128: -14 to -22 %, so that case stays with the workgroups.
    if constexpr (D >= 64) {
        if (args.S > 64 && (args.S <= 96 || (CAUSAL && args.S <= 128))) {
            args.nqb = (args.S + 31) / 32;
            const int64_t items = (int64_t)(args.nqb + 1) / 2 * nbh;
            hipLaunchKernelGGL((attn_fwd_wave<D, CAUSAL, true>), dim3((unsigned)((items + kWaves - 1) / kWaves)),
                               dim3(kThreads), 0, 0, args);
            return launch_ok("attn_fwd_wave_pair") ? EMBER_OK : EMBER_ERR_DEVICE;
        }
    }
    if (args.S > 64) {
        args.nqb = (args.S + kBr - 1) / kBr;
        // Causal launches whose block pairs all fit one round of resident
        // workgroups take the blocks in pairs of equal work (no tail of
        // light blocks): measured +15-24 % at B2-B4 H16 S = 1024-2048, +0.6 %
        // at B8 H16 S = 1024 D = 64.  Larger ones keep single blocks, heavy
        // first (pairs there measured -0.6 to -2 %).
        if constexpr (CAUSAL) {
            const int ncu = device_cu_count();
            const int64_t slots = (int64_t)(ncu > 0 ? ncu : 256) * (D == 64 ? 3 : 2);
            const int64_t pairs = (int64_t)(args.nqb + 1) / 2 * nbh;
            if (args.nqb >= 4 && pairs <= slots) {
                hipLaunchKernelGGL((attn_fwd_kernel<D, CAUSAL, true>), dim3((unsigned)pairs), dim3(kThreads), 0, 0,
                                   args);
                return launch_ok("attn_fwd_kernel_pairs") ? EMBER_OK : EMBER_ERR_DEVICE;
            }
        }
        const int nblocks = args.nqb * (int)nbh;
        hipLaunchKernelGGL((attn_fwd_kernel<D, CAUSAL, false>), dim3(nblocks), dim3(kThreads), 0, 0, args);
        return launch_ok("attn_fwd_kernel") ? EMBER_OK : EMBER_ERR_DEVICE;
    }
    // S <= 64: the wave kernel at D = 128 (4.7 TB/s at S = 32 and 4.0 at
    // S = 64, where the packed kernel moves 3.8 and 2.9) and at D = 64
    // (against the packed kernel: causal +9-13 % at S = 32, +25 % at S = 48,
    // +5-11 % at S = 64; non-causal +6 % at S = 32, +25-33 % at S = 33-48,
    // equal at S = 64; 8192-32768 heads); D = 32 keeps the packed kernel.
    if constexpr (D >= 64) {
        args.nqb = (args.S + 31) / 32;
        const int64_t items = (int64_t)args.nqb * nbh;
        hipLaunchKernelGGL((attn_fwd_wave<D, CAUSAL, false>), dim3((unsigned)((items + kWaves - 1) / kWaves)),
                           dim3(kThreads), 0, 0, args);
        return launch_ok("attn_fwd_wave") ? EMBER_OK : EMBER_ERR_DEVICE;
    }
    if constexpr (D == 32) {
        args.nqb = 1;
        if (args.S <= 32) {
            hipLaunchKernelGGL((attn_fwd_packed<D, CAUSAL, 4, 32>), dim3((unsigned)((nbh + 3) / 4)),
                               dim3(kThreads), 0, 0, args);
            return launch_ok("attn_fwd_packed_hp4") ? EMBER_OK : EMBER_ERR_DEVICE;
        }
        hipLaunchKernelGGL((attn_fwd_packed<D, CAUSAL, 2, 64>), dim3((unsigned)((nbh + 1) / 2)),
                           dim3(kThreads), 0, 0, args);
        return launch_ok("attn_fwd_packed_hp2") ? EMBER_OK : EMBER_ERR_DEVICE;
    }
    return EMBER_OK;  // not reached: every head size returns above
}

}  // namespace

// Shared argument checks for attention_fwd / attention_bwd.
int check_attention_args(const void *const *ptrs, int nptrs, int64_t B, int64_t H, int64_t S,
                         int64_t D, float scale, const int64_t *strides, int nstrides,
                         const char *who)
{
    if (B < 0 || H < 0 || S < 0 || D <= 0 || !(scale >= 0.0f) || isinf(scale))
        return record_error(EMBER_ERR_INVALID_ARGUMENT, who);
    if (D != 32 && D != 64 && D != 128) return record_error(EMBER_ERR_UNSUPPORTED, who);
    // Each factor is bounded before any product is formed (B, H < 2^31 keep
    // B * H below 2^62).
    if (B > INT32_MAX || H > INT32_MAX || S > (int64_t)INT32_MAX / 2 || B * H > (int64_t)INT32_MAX / 1024)
        return record_error(EMBER_ERR_INVALID_ARGUMENT, who);
    // At most 2^33 elements (32 GiB) per tensor: the backward's nine tensors
    // then fill an MI355X's 288 GB, and every launch's grid stays below 2^32
    // work-items (the largest, attn_bwd_pre, runs D/4 per padded row).
    if (B * H * S * D > (int64_t(1) << 33)) return record_error(EMBER_ERR_INVALID_ARGUMENT, who);
    for (int i = 0; i < nstrides; ++i)
        if (strides[i] < 0 || (strides[i] & 3)) return record_error(EMBER_ERR_INVALID_ARGUMENT, who);
    // Row strides (the third of each triple) index rows with 32-bit offsets.
    if (strides[2] >= (int64_t(1) << 24) || strides[5] >= (int64_t(1) << 24))
        return record_error(EMBER_ERR_INVALID_ARGUMENT, who);
    if (B * H * S == 0) return EMBER_OK;
    for (int i = 0; i < nptrs; ++i)
        if (!ptrs[i] || ((uintptr_t)ptrs[i] & 15)) return record_error(EMBER_ERR_INVALID_ARGUMENT, who);
    return EMBER_OK;
}

}  // namespace ember

extern "C" int attention_fwd(const float *q, const float *k, const float *v, float *o, float *lse,
                             int64_t B, int64_t H, int64_t S, int64_t D, float scale, int causal,
                             int64_t in_sb, int64_t in_sh, int64_t in_ss, int64_t out_sb,
                             int64_t out_sh, int64_t out_ss)
{
    using namespace ember;
    const void *ptrs[] = {q, k, v, o, lse};
    const int64_t strides[] = {in_sb, in_sh, in_ss, out_sb, out_sh, out_ss};
    int st = check_attention_args(ptrs, 5, B, H, S, D, scale, strides, 6, "attention_fwd");
    if (st != EMBER_OK || B * H * S == 0) return st;

    FwdArgs args;
    args.q = q;
    args.k = k;
    args.v = v;
    args.o = o;
    args.lse = lse;
    args.H = (int)H;
    args.S = (int)S;
    args.nbh = (int)(B * H);
    args.c = scale * kLog2e;
    args.in_sb = in_sb;
    args.in_sh = in_sh;
    args.in_ss = in_ss;
    args.out_sb = out_sb;
    args.out_sh = out_sh;
    args.out_ss = out_ss;
    const int64_t nbh = B * H;
    switch (D * 2 + (causal ? 1 : 0)) {
        case 64: return launch_fwd<32, false>(args, nbh);
        case 65: return launch_fwd<32, true>(args, nbh);
        case 128: return launch_fwd<64, false>(args, nbh);
        case 129: return launch_fwd<64, true>(args, nbh);
        case 256: return launch_fwd<128, false>(args, nbh);
        default: return launch_fwd<128, true>(args, nbh);
    }
}

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
//   D = 128: 8 waves, one chunk each, chunks w and 7 - w on waves w and
//     w + 4 (the hardware's round-robin placement puts those on one SIMD;
//     2 waves per SIMD, 137 KB of LDS, one workgroup per CU), persistent
//     (below);
//   D = 64: 4 waves, chunks w and 7 - w each (80 KB of LDS, two workgroups
//     per CU, which also overlap one head's loads with another's products).
// The workgroup walks 16-query chunks qc in lockstep, with the next chunk's
// Q, dO and O rows copied HBM -> LDS (buffer_load ... lds, no registers)
// into the second of two buffers while the current one is multiplied.
// Step qc:
//   dQ of chunk qc - 1 = scale * dS . K over all keys at or before it, one
//     16-column block per wave, dS and K^T from LDS; stored straight to dq in
//     the next step (every element written once: no atomics, no scratch,
//     reproducible);
//   S, dP of each active (key chunk, qc) pair; delta = <dO, O> of the 16
//     rows, formed by every wave from the LDS rows (no separate pass, no
//     extra barrier); P = exp2(S*c - lse2), dS = P * (dP - delta), masked at
//     the diagonal and past S;
//   dS to LDS; dV += P^T dO, dK += dS^T Q (the P / dS accumulators are the
//     A operands directly);
//   barrier.
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
    static constexpr int TCOP = (16 * ROWCH + 63) / 64;  // 1 KiB copies per 16-row tile
    static constexpr int TILE = TCOP * 256;              // floats per tile
    static constexpr int SET = 3 * TILE;                 // a chunk set: Q, dO, O tiles
    // Copies: the waves are split over the three tiles (wave w copies tile
    // 3w / NW), each wave taking every NWT-th copy of its tile.
    static constexpr int NWT_MIN = NW == 8 ? 2 : 1;      // fewest waves on a tile
    static constexpr int SLOTS = (TCOP + NWT_MIN - 1) / NWT_MIN;  // copies per wave, at most
    static constexpr int XSTR = 128 + 4;                 // padded row of dS (16 x 128) and K^T (D x 128)
    static constexpr int NH = D / 64;                    // 64-column halves of a row
    // Persistent at D = 128 (one workgroup per CU, nothing else to overlap
    // a head's loads with); at D = 64 two resident workgroups overlap each
    // other and the persistent form would not fit the registers.
    static constexpr bool PERSIST = D == 128;
};

// x of another lane of the same 16-lane row, by DPP control CTRL.
template <int CTRL>
__device__ __forceinline__ float row_dpp(float x)
{
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), CTRL, 0xF, 0xF, false));
}

// Sum over the 16 lanes of a row (lanes 16g .. 16g + 15), on DPP moves (no
// LDS round trip): pairs (quad_perm 1,0,3,2), quads (2,3,0,1), the two
// quads of each half (row_half_mirror), the two halves (row_mirror).  Every
// step adds the same two values on both lanes of a pair, so all 16 lanes end
// with the same bits.
__device__ __forceinline__ float row16_sum(float x)
{
    x += row_dpp<0xB1>(x);
    x += row_dpp<0x4E>(x);
    x += row_dpp<0x141>(x);
    x += row_dpp<0x140>(x);
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
__global__ __launch_bounds__(S128Shape<D>::NW * 64, D == 128 ? 1 : 2) void attn_bwd_s128(BwdArgs a, int nbh)
{
    typedef S128Shape<D> L;
    constexpr int NW = L::NW, NC = L::NC, DH = L::DH, STR = L::STR, XSTR = L::XSTR, NH = L::NH;
    constexpr int NB = D / 16;  // 16-column blocks of dV / dK
    constexpr bool kPersist = L::PERSIST;
    __shared__ float sets[2 * L::SET];      // chunk sets: Q, dO, O tiles of 16 padded rows
    __shared__ float dsb[2 * 16 * XSTR];    // dS of a query chunk, alternate chunks alternate halves
    // K^T of the head, rows of 128 keys + 4 padding floats; the padding of
    // rows 0-31 holds lse2 of the head's 128 rows (row r at r/4, 128 + r%4),
    // which keeps two D = 64 workgroups within a CU's LDS.
    __shared__ float Kt[D * XSTR];

    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n = lane & 15, g = lane >> 4;
    const int S = a.S;
    const int nch = (S + 15) >> 4;
    const int in_ss = (int)a.in_ss, out_ss = (int)a.out_ss;  // < 2^24 (checked on the host)
    auto in_base_of = [&](int bh) {
        const int b = bh / a.H;
        return (int64_t)b * a.in_sb + (int64_t)(bh - b * a.H) * a.in_sh;
    };
    auto out_base_of = [&](int bh) {
        const int b = bh / a.H;
        return (int64_t)b * a.out_sb + (int64_t)(bh - b * a.H) * a.out_sh;
    };

    // This wave's key chunks, ascending (so the active ones form a prefix).
    int kc[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) kc[c] = NC == 1 ? (w < 4 ? w : 11 - w) : (c == 0 ? w : 7 - w);

    // Resident K and V of head bh: lane (n, g) holds K[16 kc + n][DH g + s].
    float kr[NC][DH], vr[NC][DH];
    auto load_kv = [&](int bh) {
        const int64_t base = in_base_of(bh);
        int ln = lane;  // opaque: no address kept live across the chunk loop
        asm volatile("" : "+v"(ln));
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            const int row = min(16 * kc[c] + (ln & 15), S - 1);
            const float *__restrict__ ks = a.k + base + (int64_t)row * in_ss + DH * (ln >> 4);
            const float *__restrict__ vs = a.v + base + (int64_t)row * in_ss + DH * (ln >> 4);
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
    };
    // lse of row threadIdx.x (< 128) of head bh, kept in a register until
    // the head starts.
    float lse_r = 0.0f;
    auto load_lse = [&](int bh) {
        const int t = threadIdx.x;
        if (t < 128) lse_r = a.lse[(int64_t)bh * S + min(t, S - 1)];
    };

    // Copies of a chunk set.  Copy u of a tile fills its 16-byte pieces
    // 64u .. 64u + 63; wave w copies tile tw = 3w / NW (Q, dO, O), copies
    // u = w - w0 + NWT s, so all of a wave's copies read one tensor: its base
    // lives in a scalar buffer descriptor and each lane supplies a 32-bit
    // byte offset, fixed for the kernel (row m0 + r of the chunk at m0).  A
    // padding or slack piece re-reads the chunk's first piece (valid memory,
    // never used).
    const int tw = 3 * w / NW;                      // this wave's tile
    const int w0 = (tw * NW + 2) / 3;               // first wave of that tile
    const int nwt = ((tw + 1) * NW + 2) / 3 - w0;   // waves on that tile
    const int tss = tw == 0 ? in_ss : out_ss;       // row stride of its tensor
    auto piece = [&](int u, int ln, int rmax) {
        const int p = 64 * u + ln;
        const int r = p / L::ROWCH, c4 = p - r * L::ROWCH;
        return r < 16 && c4 < D / 4 ? 4u * (unsigned)(min(r, rmax) * tss + 4 * c4) : 0u;
    };
    unsigned coff[L::SLOTS];
#pragma unroll
    for (int sl = 0; sl < L::SLOTS; ++sl) coff[sl] = piece(w - w0 + nwt * sl, lane, 15);
    // Chunk qc of the head with bases ib (q) and ob (dO, O) into set dst.
    // The sequence's last chunk clamps its rows to S - 1 (offsets recomputed
    // from an opaque lane index, so no second set stays live).
    auto fetch = [&](int64_t ib, int64_t ob, int qc, float *dst) {
        const int m0 = 16 * qc;
        const bool full = m0 + 15 < S;
        const float *tbase = tw == 0 ? a.q + ib : (tw == 1 ? a.dout : a.o) + ob;
        const __amdgpu_buffer_rsrc_t rsrc = dma_rsrc(tbase + (int64_t)m0 * tss);
        float *tdst = dst + tw * L::TILE;
        int ln = lane;
        asm volatile("" : "+v"(ln));
#pragma unroll
        for (int sl = 0; sl < L::SLOTS; ++sl) {
            const int u = w - w0 + nwt * sl;
            if (u < L::TCOP) dma16_buf(rsrc, full ? coff[sl] : piece(u, ln, S - 1 - m0), tdst + 256 * u);
        }
    };

    f32x4 dvacc[NC][NB], dkacc[NC][NB];

    // delta of rows 4g + r of the chunk set: each lane of a row group sums
    // its D/16 columns (the pieces of dO it reads again for dV), then the
    // group sums.
    auto row_delta = [&](const float *__restrict__ cur, float (&dl)[4]) {
        const float *__restrict__ Gs = cur + L::TILE;
        const float *__restrict__ Os = cur + 2 * L::TILE;
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
        const float *__restrict__ Gs = cur + L::TILE;
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

    // Stores of a finished head: its last dQ chunk (rows 16 qc ..,
    // columns 16w ..) and dK (scaled), dV of this wave's keys (register r
    // of block 4h + j holds key 16 kc + 4g + r, column 64h + 4n + j).
    auto store_dq = [&](int64_t base, int qc, const f32x4 &acc) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int row = 16 * qc + 4 * g + r;
            if (row < S) a.dq[base + (int64_t)row * in_ss + 16 * w + n] = acc[r] * a.scale;
        }
    };
    auto store_dkdv = [&](int64_t base) {
#pragma unroll
        for (int c = 0; c < NC; ++c) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int key = 16 * kc[c] + 4 * g + r;
                if (key >= S) continue;
                float *dkrow = a.dk + base + (int64_t)key * in_ss + 4 * n;
                float *dvrow = a.dv + base + (int64_t)key * in_ss + 4 * n;
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
    };

    // dQ of query chunk qc (rows 16 qc .., columns 16w .. 16w + 15) from
    // its dS (in the dS half ds) and K^T, over key chunks 0 .. qc (causal)
    // or all of them.
    auto dq_product = [&](int qc, const float *__restrict__ ds) {
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
        const int klast = CAUSAL ? qc : nch - 1;
        for (int c = 0; c <= klast; ++c) {
            const f32x4 af = *(const f32x4 *)&ds[n * XSTR + 16 * c + 4 * g];
            const f32x4 bf = *(const f32x4 *)&Kt[(16 * w + n) * XSTR + 16 * c + 4 * g];
#pragma unroll
            for (int j = 0; j < 4; ++j) acc = mfma16(af[j], bf[j], acc);
        }
        return acc;
    };

    // Step qc: store dQ of chunk qc - 2 (formed in the previous step), copy
    // chunk qc + 1, form dQ of chunk qc - 1 (its dS is in LDS since the last
    // barrier) ahead of chunk qc's products, so that each wave's dQ MFMAs and
    // its products' latencies overlap; one barrier.  dQ of the last two
    // chunks is left to the head's end.
    //
    // Persistent (D = 128): workgroup i walks heads i, i + gridDim.x, ...
    // During a head's last step the next head's K, V (into the registers the
    // last S and dP products have just released), lse and first chunk are
    // loaded; the finished head's last two dQ chunks, dK and dV are stored
    // after the next head's first barrier, so that the wait before that
    // barrier covers only loads.
    const int stride = (int)gridDim.x;
    int bh = blockIdx.x;
    load_kv(bh);
    load_lse(bh);
    fetch(in_base_of(bh), out_base_of(bh), 0, sets);
    int sbase = 0;  // set / dS half of the head's chunk 0
    int prev = -1;  // the finished head whose stores are pending
    f32x4 dq_a = {0.f, 0.f, 0.f, 0.f}, dq_b = {0.f, 0.f, 0.f, 0.f};  // its dQ chunks nch-2, nch-1
    // Head bh; next: the workgroup's next head (nbh if none).
    auto head = [&](int bh, int next) {
        const int64_t in_base = in_base_of(bh), out_base = out_base_of(bh);
        wait_vmem();  // this head's K, V, lse and this wave's copies of chunk 0
        {
            const int t = threadIdx.x;
            if (t < 128) Kt[(t >> 2) * XSTR + 128 + (t & 3)] = t < S ? lse_r * kLog2e : INFINITY;
        }
        __syncthreads();  // chunk 0 and lse2 in LDS; every wave is done with the previous head
        if (prev >= 0) {
            const int64_t pb = in_base_of(prev);
            store_dq(pb, nch - 2, dq_a);
            store_dq(pb, nch - 1, dq_b);
            store_dkdv(pb);
        }
#pragma unroll
        for (int c = 0; c < NC; ++c)
#pragma unroll
            for (int db = 0; db < NB; ++db) {
                dvacc[c][db] = f32x4{0.f, 0.f, 0.f, 0.f};
                dkacc[c][db] = f32x4{0.f, 0.f, 0.f, 0.f};
            }
        // K^T for the dQ product (chunks past S are never read).
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            if (16 * kc[c] < S) {
#pragma unroll
                for (int s = 0; s < DH; ++s) Kt[(DH * g + s) * XSTR + 16 * kc[c] + n] = kr[c][s];
            }
        }

        f32x4 qa = {0.f, 0.f, 0.f, 0.f};  // dQ of chunk qc - 1, stored in step qc + 1
        for (int qc = 0; qc < nch; ++qc) {
            const int st = (qc + sbase) & 1;
            const float *__restrict__ cur = sets + st * L::SET;
            float *__restrict__ ds = dsb + st * 16 * XSTR;
            const bool last = qc + 1 == nch;
            if (qc >= 2) store_dq(in_base, qc - 2, qa);
            if (!last)
                fetch(in_base, out_base, qc + 1, sets + (st ^ 1) * L::SET);
            else if (kPersist && next < nbh)
                fetch(in_base_of(next), out_base_of(next), 0, sets + (st ^ 1) * L::SET);
            if (qc >= 1) qa = dq_product(qc - 1, dsb + (st ^ 1) * 16 * XSTR);
            // Active chunks: inside the sequence and (causal) at or before qc.
            int nact = 0;
#pragma unroll
            for (int c = 0; c < NC; ++c)
                if (16 * kc[c] < S && (!CAUSAL || kc[c] <= qc)) nact = c + 1;
            if (nact > 0) {
                float dl[4];
                row_delta(cur, dl);
                const f32x4 l2 = *(const f32x4 *)&Kt[(4 * qc + g) * XSTR + 128];  // lse2 of rows 4g + r
                products(std::integral_constant<int, 0>{}, qc, cur, ds, dl, l2);
                if constexpr (NC == 2) {
                    if (nact == 2) products(std::integral_constant<int, 1>{}, qc, cur, ds, dl, l2);
                }
            }
            if (!last) {
                wait_vmem();  // this wave's copies of chunk qc + 1 have landed
            } else if (kPersist && next < nbh) {
                load_kv(next);
                load_lse(next);
            }
            __syncthreads();  // dS of chunk qc (and, but last, all of chunk qc + 1) in LDS
        }
        const f32x4 qb = dq_product(nch - 1, dsb + ((nch - 1 + sbase) & 1) * 16 * XSTR);
        if constexpr (kPersist) {
            dq_a = qa;
            dq_b = qb;
            sbase ^= nch & 1;
            prev = bh;
        } else {
            store_dq(in_base, nch - 2, qa);
            store_dq(in_base, nch - 1, qb);
            store_dkdv(in_base);
        }
    };
    if constexpr (kPersist) {
        for (; bh < nbh; bh += stride) head(bh, bh + stride);
        const int64_t pb = in_base_of(prev);
        store_dq(pb, nch - 2, dq_a);
        store_dq(pb, nch - 1, dq_b);
        store_dkdv(pb);
    } else {
        head(bh, nbh);
    }
}

template <int D, bool CAUSAL>
int launch_s128(const BwdArgs &args, int nbh)
{
    int grid = nbh;  // one workgroup per head, or (persistent) one per CU
    if constexpr (S128Shape<D>::PERSIST) {
        const int ncu = device_cu_count();
        if (ncu <= 0) return record_error(EMBER_ERR_DEVICE, "hipDeviceGetAttribute(CU count)");
        if (ncu < nbh) grid = ncu;
    }
    hipLaunchKernelGGL((attn_bwd_s128<D, CAUSAL>), dim3((unsigned)grid), dim3(S128Shape<D>::NW * 64), 0, 0,
                       args, nbh);
    return launch_ok("attn_bwd_s128") ? EMBER_OK : EMBER_ERR_DEVICE;
}

}  // namespace

int launch_bwd_s128(const BwdArgs &args, int D, bool causal, int nbh)
{
    if (D == 128) return causal ? launch_s128<128, true>(args, nbh) : launch_s128<128, false>(args, nbh);
    return causal ? launch_s128<64, true>(args, nbh) : launch_s128<64, false>(args, nbh);
}

}  // namespace ember

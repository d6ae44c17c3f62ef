// attention_bwd.hip -- entry point of the fused flash-attention backward
// (fp32, gfx950); the kernels are in attention_bwd_kernels.h.
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
#include "attention_bwd_kernels.h"

extern "C" int attention_bwd(const float *q, const float *k, const float *v, const float *o,
                             const float *lse, const float *d_o, float *dq, float *dk, float *dv,
                             int64_t B, int64_t H, int64_t S, int64_t D, float scale, int causal,
                             int64_t in_sb, int64_t in_sh, int64_t in_ss, int64_t out_sb,
                             int64_t out_sh, int64_t out_ss)
{
    using namespace ember;
    const void *ptrs[] = {q, k, v, o, lse, d_o, dq, dk, dv};
    const int64_t strides[] = {in_sb, in_sh, in_ss, out_sb, out_sh, out_ss};
    int st = check_attention_args(ptrs, 9, B, H, S, D, scale, strides, 6, "attention_bwd");
    if (st != EMBER_OK || B * H * S == 0) return st;

    const int64_t S_pad = (S + kBq - 1) / kBq * kBq;
    const int64_t rows_pad = B * H * S_pad;
    float *stats = (float *)scratch(kScratchAttnDelta, (size_t)rows_pad * 2 * sizeof(float));
    if (!stats) return EMBER_ERR_OUT_OF_MEMORY;

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
    args.H = (int)H;
    args.S = (int)S;
    args.S_pad = (int)S_pad;
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
        case 64: return launch_bwd<32, false>(args, rows_pad, nblocks);
        case 65: return launch_bwd<32, true>(args, rows_pad, nblocks);
        case 128: return launch_bwd<64, false>(args, rows_pad, nblocks);
        case 129: return launch_bwd<64, true>(args, rows_pad, nblocks);
        case 256: return launch_bwd<128, false>(args, rows_pad, nblocks);
        default: return launch_bwd_causal_d128(args, rows_pad, nblocks);
    }
}

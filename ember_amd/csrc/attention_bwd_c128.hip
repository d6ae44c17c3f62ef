// attention_bwd_c128.hip -- the causal, head_dim 128 instantiation of the
// fused attention backward (attention_bwd_kernels.h), in a translation unit
// of its own so that it is compiled with the default MFMA register form (see
// attention_bwd.hip).
#include "attention_bwd_kernels.h"

namespace ember {

int launch_bwd_causal_d128(const BwdArgs &args, int64_t rows_pad, int nblocks)
{
    return launch_bwd<128, true>(args, rows_pad, nblocks);
}

}  // namespace ember

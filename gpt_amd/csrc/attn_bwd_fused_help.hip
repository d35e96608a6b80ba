// The HELP instantiation of the one-launch head_dim-64 backward
// (bwd_fused_d64_kernel<true, true>, attn_bwd_fused_kernel.h), taken for grids
// of at most 2 workgroups per CU. A translation unit of its own, compiled with
// the default machine scheduler (the max-ILP one that attn_bwd_fused.hip uses
// measured 0.9 % slower for this instantiation at B = 8, T = 256).
#include "attn_bwd_fused_kernel.h"

namespace gpt_attn {

hipError_t launch_bwd_fused_d64_help(dim3 g, float *grad_x, float *ws, int *ctl, const float *lse, float *D,
                                     const float *dy, const float *y, const float *qkv, int T, int C, int H,
                                     int BH, int n_qb, float c2, float scale, int n_cu, const FusedSync &sync,
                                     hipStream_t st)
{
    launch_timed(kKindFused, bwd_fused_d64_kernel<true, true>, g, dim3(256), st, grad_x, ws, ctl, lse, D, dy, y, qkv,
                 T, C, H, 0, BH, n_qb, c2, scale, n_cu, sync);
    return hipGetLastError();
}

}  // namespace gpt_attn

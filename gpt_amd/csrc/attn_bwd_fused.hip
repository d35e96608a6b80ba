// Causal self-attention backward for gfx950, head_dim 64, one launch: the
// host side (occupancy, which grids take it, the launch) and the instantiation
// for full grids. The kernel and its design are in attn_bwd_fused_kernel.h.
//
// This translation unit is compiled with the max-ILP machine scheduler
// (gpt_amd/Makefile): for bwd_fused_d64_kernel<true, false> it measured 0.6-0.7
// % faster per 12-layer C3 step (A/B on one box: 0.9224 / 0.9221 vs 0.9290 /
// 0.9290 ms, outputs bitwise unchanged), while the HELP instantiation lost
// 0.9 % at B = 8 with it and stays in attn_bwd_fused_help.hip under the
// default scheduler.
#include "attn_bwd_fused_kernel.h"

namespace gpt_attn {

// Workgroups of the fused kernel one CU holds at once (registers and LDS),
// from the runtime's occupancy calculator; cached per device.
static int fused_per_cu()
{
    static int cached[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64)
        return 0;
    if (cached[dev] == 0)
    {
        int n = 0;
        const hipError_t e =
            hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, bwd_fused_d64_kernel<true, false>, 256, 0);
        cached[dev] = e == hipSuccess && n > 0 ? n : -1;
    }
    return cached[dev] > 0 ? cached[dev] : 0;
}

bool bwd_fused_d64_fits(const Shape &s, int bh_per_chunk, int n_cu)
{
    // Correct at any grid size (no wait depends on residency); taken where it
    // measured fastest, grids that one round of the CUs holds, with one chunk
    // and a control block that holds its counters and flags.
    const long n_kg = (s.T + 63) / 64, n_qb = (s.T + 31) / 32;
    return n_cu > 0 && s.T <= 64 * kMaxFusedKeyGroups && bh_per_chunk >= s.B * s.H &&
           (long)s.B * s.H * n_qb <= kCtlItems && (long)s.B * s.H * n_kg <= (long)fused_per_cu() * n_cu;
}

int bwd_fused_d64_main_workgroups(const Shape &s) { return (s.T + 63) / 64 * s.B * s.H; }

hipError_t launch_bwd_fused_d64(float *grad_x, float *D, const float *lse, const float *dy, const float *y,
                                const float *qkv, float *ws, int *ctl, int n_cu, const FusedSync &sync,
                                const Shape &s, hipStream_t st)
{
    const int n_qb = (s.T + 31) / 32;
    const int BH = s.B * s.H;
    const float scale = 1.0f / sqrtf(64.f);
    const int n_main = bwd_fused_d64_main_workgroups(s);
    const dim3 g((unsigned)(n_main + kOrphanRunners));
    // T <= 256 (bwd_fused_d64_fits): the D rows are computed in the kernel;
    // grids of at most 2 workgroups per CU share the last step's work out
    if (n_main <= 2 * n_cu)
        return launch_bwd_fused_d64_help(g, grad_x, ws, ctl, lse, D, dy, y, qkv, s.T, s.C, s.H, BH, n_qb,
                                         scale * kLog2e, scale, n_cu, sync, st);
    else
        launch_timed(kKindFused, bwd_fused_d64_kernel<true, false>, g, dim3(256), st, grad_x, ws, ctl, lse, D, dy, y,
                     qkv, s.T, s.C, s.H, 0, BH, n_qb, scale * kLog2e, scale, n_cu, sync);
    return hipGetLastError();
}

}  // namespace gpt_attn

// Internal launchers of the attention kernels (called by attn_capi.hip after
// argument validation). Each returns the hipError_t of its launches.
#pragma once

#include <hip/hip_runtime.h>

namespace gpt_attn {

struct Shape
{
    int B, T, C, H, d;
};

// Forward, head_dim 64, fp32 MFMA. Pointers 16-byte aligned.
hipError_t launch_fwd_d64(float *y, float *lse, const float *qkv, const Shape &s, hipStream_t st);

// Forward, any head_dim in 1..256, scalar HIP kernel.
hipError_t launch_fwd_general(float *y, float *lse, const float *qkv, const Shape &s, hipStream_t st);

// Backward, head_dim 64, fp32 MFMA (D rows + dQ zeroing, then the fused
// dK/dV/dQ kernel with atomic dQ accumulation).
hipError_t launch_bwd_d64(float *grad_x, float *D, const float *lse, const float *dy,
                          const float *y, const float *qkv, const Shape &s, hipStream_t st);

// Backward, any head_dim in 1..256, scalar HIP kernels (no atomics).
hipError_t launch_bwd_general(float *grad_x, float *D, const float *lse, const float *dy,
                              const float *y, const float *qkv, const Shape &s, hipStream_t st);

}  // namespace gpt_attn

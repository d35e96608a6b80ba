/*
 * CPU oracle for the causal self-attention op pair of Filipeak/gpt.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker that the HIP product
 * path (gpt_amd/) is compared against. Only tests/, __graft_entry__.smoke()
 * and bench.py's cpu_baseline leg may load it; the product never calls it and
 * has no CPU fallback.
 *
 * Layouts (reference src/backend/backend_interface.h:161-184):
 *   qkv     [B, T, 3C]   Q at column h*d, K at C + h*d, V at 2C + h*d
 *   y       [B, T, C]    head h in columns h*d .. h*d + d - 1
 *   lse     [B, T, H]    token-major, natural-log log-sum-exp of scaled scores
 *   grad_x  [B, T, 3C]   dQ / dK / dV in the qkv layout (overwritten)
 *   D       [B, T, H]    sum_d dO * O (written by the backward)
 */
#ifndef GPT_ATTN_ORACLE_H
#define GPT_ATTN_ORACLE_H

#ifdef __cplusplus
extern "C" {
#endif

/* fp32 restatement of CPUBackend::device_flash_attention_forward
 * (src/backend/cpu/cpu_backend.cpp:289-356), same loop and summation order. */
void oracle_attn_forward_f32(float *y, float *lse, const float *qkv,
                             int B, int T, int C, int H);

/* fp32 restatement of CPUBackend::device_flash_attention_backward
 * (src/backend/cpu/cpu_backend.cpp:358-437), same loop and summation order. */
void oracle_attn_backward_f32(float *grad_x, float *D, const float *lse,
                              const float *grad_y, const float *y,
                              const float *qkv, int B, int T, int C, int H);

/* The same two algorithms carried out in double precision on fp64 buffers.
 * They serve as the "exact" answer when an fp32 result's own rounding error
 * has to be separated from an implementation error. */
void oracle_attn_forward_f64(double *y, double *lse, const double *qkv,
                             int B, int T, int C, int H);
void oracle_attn_backward_f64(double *grad_x, double *D, const double *lse,
                              const double *grad_y, const double *y,
                              const double *qkv, int B, int T, int C, int H);

#ifdef __cplusplus
}
#endif

#endif

// Internal launchers of the GPT-2 op kernels (ops_kernels.hip), called by
// ops_capi.hip after argument validation. Each returns the hipError_t of its
// launches. Row-major shapes; rows = B * T.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>

namespace gpt_ops {

// Number of partial-sum rows the two-stage column reductions write, for a
// matrix of `rows` rows (each workgroup of the first stage folds a fixed
// stripe of rows; the second stage adds the partials in stripe order).
int colsum_parts(long rows);

hipError_t launch_embedding_fwd(float *y, const float *wte, const float *wpe, const int *tok, int B, int T, int C,
                                int vocab_rows, hipStream_t st);
hipError_t launch_embedding_bwd(float *grad_wte, float *grad_wpe, const float *gy, const int *tok, int B, int T,
                                int C, int vocab_rows, hipStream_t st);

// ws: 2 * colsum_parts(rows) * C floats
hipError_t launch_layernorm_fwd(float *y, float *means, float *vars, float *x, const float *res,
                                const float *gamma, const float *beta, long rows, int C, hipStream_t st);
hipError_t launch_layernorm_bwd(float *gx, float *ggamma, float *gbeta, const float *gy, const float *gres,
                                const float *x, const float *means, const float *vars, const float *gamma, long rows,
                                int C, float *ws, hipStream_t st);

// y[r, o] += b[o]; act = GELU(y) when act != NULL
hipError_t launch_bias_gelu(float *y, float *act, const float *b, long rows, int N, hipStream_t st);
// act = GELU(y)
hipError_t launch_gelu(float *act, const float *y, long rows, int N, hipStream_t st);
// gb[o] += sum_r gy[r, o]; ws: colsum_parts(rows) * N floats
hipError_t launch_bias_grad(float *gb, const float *gy, long rows, int N, float *ws, hipStream_t st);
hipError_t launch_gelu_bwd(float *gx, const float *gy, const float *x, long n, hipStream_t st);

hipError_t launch_softmax_fwd(float *y, const float *x, long rows, int V, int Vp, hipStream_t st);
hipError_t launch_ce_bwd(float *gx, const float *y, const int *labels, long rows, int V, int Vp, hipStream_t st);
hipError_t launch_ce_loss(float *loss, const float *y, const int *labels, long rows, int Vp, hipStream_t st);

hipError_t launch_adamw(float *p, const float *g, float *m, float *v, long n, float lr, float beta1, float beta2,
                        float eps, float wd, float one_m_b1p, float one_m_b2p, hipStream_t st);
// ws: clip_parts() floats
int clip_parts();
hipError_t launch_scale_clip(float *g, long n, float max_norm, float accum, float *ws, hipStream_t st);

hipError_t launch_fill_normal(float *p, size_t n, float mean, float stddev, unsigned long long seed, hipStream_t st);
hipError_t launch_fill_const(float *p, size_t n, float value, hipStream_t st);

}  // namespace gpt_ops

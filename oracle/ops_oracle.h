/*
 * ops_oracle.h - CPU restatement of the reference CPU backend's GPT-2 ops
 * other than attention (reference src/backend/cpu/cpu_backend.cpp:65-287,
 * 439-557). TEST INFRASTRUCTURE ONLY: the checker of the HIP ops library,
 * never part of the product path.
 *
 * Same arguments as the IGPTBackend methods (backend_interface.h:26-237),
 * host pointers. Every accumulation runs in the reference's order, so with
 * the same compiler flags (-O2, no FMA contraction) the results equal the
 * reference's bit for bit (pinned against the reference's own code in
 * tests/test_ops_oracle.py).
 */
#ifndef OPS_ORACLE_H
#define OPS_ORACLE_H

#ifdef __cplusplus
extern "C" {
#endif

void ops_oracle_embedding_forward(float *y, const float *wte, const float *wpe, const int *tok, int B, int T, int C);
void ops_oracle_unembedding_forward(float *y, const float *x, const float *wte, int B, int T, int C, int Vp);
void ops_oracle_embedding_backward(float *gwte, float *gwpe, const float *gy, const int *tok, int B, int T, int C);
void ops_oracle_unembedding_backward(float *gx, float *gwte, const float *gy, const float *x, const float *wte,
                                     int B, int T, int C, int Vp);
void ops_oracle_layernorm_forward(float *y, float *means, float *vars, float *x, const float *res,
                                  const float *gamma, const float *beta, int B, int T, int C);
void ops_oracle_layernorm_backward(float *gx, float *ggamma, float *gbeta, const float *gy, const float *gres,
                                   const float *x, const float *means, const float *vars, const float *gamma, int B,
                                   int T, int C);
void ops_oracle_linear_forward(float *y, float *act, const float *x, const float *w, const float *b, int activation,
                               int B, int T, int in, int out);
void ops_oracle_linear_backward(float *gx, float *gw, float *gb, const float *gy, const float *x, const float *w,
                                int B, int T, int in, int out);
void ops_oracle_activation_backward(float *gx, const float *gy, const float *x, int B, int T, int n);
void ops_oracle_softmax_forward(float *y, const float *x, int B, int T, int V, int Vp);
void ops_oracle_ce_backward(float *gx, const float *y, const int *labels, int B, int T, int V, int Vp);
void ops_oracle_ce_loss(float *loss, const float *y, const int *labels, int B, int T, int Vp);
void ops_oracle_adamw(float *p, const float *g, float *m, float *v, int n, float lr, float beta1, float beta2,
                      float eps, float wd, int step);
void ops_oracle_scale_clip(float *g, int n, float max_norm, int accum);

#ifdef __cplusplus
}
#endif

#endif

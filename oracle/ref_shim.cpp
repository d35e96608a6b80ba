// C entry points over the reference's own CPUBackend attention ops, so that
// tests can call the reference implementation compiled from its sources in
// /root/reference (see oracle/Makefile; output goes to oracle/_ref/ only).
//
// TEST INFRASTRUCTURE ONLY: the result is a checker and a CPU baseline,
// never part of the product path.
//
// Wrapped methods (reference src/backend/cpu/cpu_backend.h:9-32):
//   CPUBackend::device_flash_attention_forward   cpu_backend.cpp:289-356
//   CPUBackend::device_flash_attention_backward  cpu_backend.cpp:358-437
// and, as ref_op_*, every other compute method (cpu_backend.cpp:65-287,
// 439-557), the reference side of the ops library's parity tests.
#include "cpu_backend.h"

extern "C" {

void ref_attn_forward_f32(float *y, float *lse, const float *qkv, int B, int T, int C, int H)
{
    CPUBackend be;
    be.device_flash_attention_forward(y, lse, qkv, B, T, C, H);
}

void ref_attn_backward_f32(float *grad_x, float *D, const float *lse, const float *grad_y,
                           const float *y, const float *qkv, int B, int T, int C, int H)
{
    CPUBackend be;
    be.device_flash_attention_backward(grad_x, D, lse, grad_y, y, qkv, B, T, C, H);
}

void ref_op_embedding_forward(float *y, const float *wte, const float *wpe, const int *tok, int B, int T, int C)
{
    CPUBackend().device_embedding_forward(y, wte, wpe, tok, B, T, C);
}

void ref_op_unembedding_forward(float *y, const float *x, const float *wte, int B, int T, int C, int Vp)
{
    CPUBackend().device_unembedding_forward(y, x, wte, B, T, C, Vp);
}

void ref_op_embedding_backward(float *gwte, float *gwpe, const float *gy, const int *tok, int B, int T, int C)
{
    CPUBackend().device_embedding_backward(gwte, gwpe, gy, tok, B, T, C);
}

void ref_op_unembedding_backward(float *gx, float *gwte, const float *gy, const float *x, const float *wte, int B,
                                 int T, int C, int Vp)
{
    CPUBackend().device_unembedding_backward(gx, gwte, gy, x, wte, B, T, C, Vp);
}

void ref_op_layernorm_forward(float *y, float *means, float *vars, float *x, const float *res, const float *gamma,
                              const float *beta, int B, int T, int C)
{
    CPUBackend().device_layernorm_residual_fused_forward(y, means, vars, x, res, gamma, beta, B, T, C);
}

void ref_op_layernorm_backward(float *gx, float *ggamma, float *gbeta, const float *gy, const float *gres,
                               const float *x, const float *means, const float *vars, const float *gamma, int B,
                               int T, int C)
{
    CPUBackend().device_layernorm_residual_fused_backward(gx, ggamma, gbeta, gy, gres, x, means, vars, gamma, B, T,
                                                          C);
}

void ref_op_linear_forward(float *y, float *act, const float *x, const float *w, const float *b, int activation,
                           int B, int T, int in, int out)
{
    CPUBackend().device_linear_activation_fused_forward(y, act, x, w, b, activation != 0, B, T, in, out);
}

void ref_op_linear_backward(float *gx, float *gw, float *gb, const float *gy, const float *x, const float *w, int B,
                            int T, int in, int out)
{
    CPUBackend().device_linear_backward(gx, gw, gb, gy, x, w, B, T, in, out);
}

void ref_op_activation_backward(float *gx, const float *gy, const float *x, int B, int T, int n)
{
    CPUBackend().device_activation_backward(gx, gy, x, B, T, n);
}

void ref_op_softmax_forward(float *y, const float *x, int B, int T, int V, int Vp)
{
    CPUBackend().device_softmax_forward(y, x, B, T, V, Vp);
}

void ref_op_ce_backward(float *gx, const float *y, const int *labels, int B, int T, int V, int Vp)
{
    CPUBackend().device_cross_entropy_softmax_fused_backward(gx, y, labels, B, T, V, Vp);
}

void ref_op_ce_loss(float *loss, const float *y, const int *labels, int B, int T, int Vp)
{
    CPUBackend().device_cross_entropy_loss(loss, y, labels, B, T, Vp);
}

void ref_op_adamw(float *p, float *g, float *m, float *v, int n, float lr, float beta1, float beta2, float eps,
                  float wd, int step)
{
    CPUBackend().device_adamw_step(p, g, m, v, n, lr, beta1, beta2, eps, wd, step);
}

void ref_op_scale_clip(float *g, int n, float max_norm, int accum)
{
    CPUBackend().device_scale_and_clip_grad(g, n, max_norm, accum);
}

}

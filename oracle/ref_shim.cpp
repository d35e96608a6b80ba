// C entry points over the reference's own CPUBackend attention ops, so that
// tests can call the reference implementation compiled from its sources in
// /root/reference (see oracle/Makefile; output goes to oracle/_ref/ only).
//
// TEST INFRASTRUCTURE ONLY: the result is a checker and a CPU baseline,
// never part of the product path.
//
// Wrapped methods (reference src/backend/cpu/cpu_backend.h:25-26):
//   CPUBackend::device_flash_attention_forward   cpu_backend.cpp:289-356
//   CPUBackend::device_flash_attention_backward  cpu_backend.cpp:358-437
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

}

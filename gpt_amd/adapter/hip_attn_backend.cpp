// HipAttnBackend: the reference's IGPTBackend attention ops bound to the
// gfx950 HIP library's C ABI. See hip_attn_backend.h.
#include "hip_attn_backend.h"

#include "gpt_hip_attn.h"

#include <hip/hip_runtime_api.h>

#include <cstdio>
#include <cstdlib>

namespace {

void die_hip(hipError_t e, const char *what)
{
    if (e == hipSuccess)
        return;
    std::fprintf(stderr, "[hip_attn_backend] %s failed: %s\n", what, hipGetErrorString(e));
    std::abort();
}

void die_attn(int rc)
{
    if (rc == 0)
        return;
    std::fprintf(stderr, "[hip_attn_backend] gpt_hip_attn error %d: %s\n", rc, gpt_hip_attn_last_error());
    std::abort();
}

size_t round4(size_t n) { return (n + 3) & ~size_t(3); }

}  // namespace

HipAttnBackend::HipAttnBackend()
{
    if (!gpt_hip_attn_device_ok())
    {
        std::fprintf(stderr, "[hip_attn_backend] no usable HIP device\n");
        std::abort();
    }
}

HipAttnBackend::~HipAttnBackend()
{
    if (dev_)
        (void)hipFree(dev_);
}

float *HipAttnBackend::reserve(size_t floats)
{
    const size_t bytes = floats * sizeof(float);
    if (bytes > dev_bytes_)
    {
        if (dev_)
            die_hip(hipFree(dev_), "hipFree");
        dev_ = nullptr;
        die_hip(hipMalloc(&dev_, bytes), "hipMalloc");
        dev_bytes_ = bytes;
    }
    return static_cast<float *>(dev_);
}

void HipAttnBackend::device_flash_attention_forward(float *y, float *logsumexp, const float *qkv, int batch_size,
                                                    int seq_len, int hidden_size, int num_heads)
{
    const size_t n_qkv = (size_t)batch_size * seq_len * 3 * hidden_size;
    const size_t n_y = (size_t)batch_size * seq_len * hidden_size;
    const size_t n_l = (size_t)batch_size * seq_len * num_heads;
    float *d_qkv = reserve(round4(n_qkv) + round4(n_y) + round4(n_l));
    float *d_y = d_qkv + round4(n_qkv);
    float *d_l = d_y + round4(n_y);
    die_hip(hipMemcpy(d_qkv, qkv, n_qkv * sizeof(float), hipMemcpyHostToDevice), "hipMemcpy H2D");
    die_attn(gpt_hip_attn_fwd_f32(d_y, d_l, d_qkv, batch_size, seq_len, hidden_size, num_heads, nullptr));
    die_hip(hipMemcpy(y, d_y, n_y * sizeof(float), hipMemcpyDeviceToHost), "hipMemcpy D2H");
    die_hip(hipMemcpy(logsumexp, d_l, n_l * sizeof(float), hipMemcpyDeviceToHost), "hipMemcpy D2H");
}

void HipAttnBackend::device_flash_attention_backward(float *grad_x, float *D_cache, const float *logsumexp,
                                                     const float *grad_y, const float *y, const float *qkv,
                                                     int batch_size, int seq_len, int hidden_size, int num_heads)
{
    const size_t n_qkv = (size_t)batch_size * seq_len * 3 * hidden_size;
    const size_t n_y = (size_t)batch_size * seq_len * hidden_size;
    const size_t n_l = (size_t)batch_size * seq_len * num_heads;
    float *d_qkv = reserve(2 * round4(n_qkv) + 2 * round4(n_y) + 2 * round4(n_l));
    float *d_gx = d_qkv + round4(n_qkv);
    float *d_y = d_gx + round4(n_qkv);
    float *d_gy = d_y + round4(n_y);
    float *d_l = d_gy + round4(n_y);
    float *d_D = d_l + round4(n_l);
    die_hip(hipMemcpy(d_qkv, qkv, n_qkv * sizeof(float), hipMemcpyHostToDevice), "hipMemcpy H2D");
    die_hip(hipMemcpy(d_y, y, n_y * sizeof(float), hipMemcpyHostToDevice), "hipMemcpy H2D");
    die_hip(hipMemcpy(d_gy, grad_y, n_y * sizeof(float), hipMemcpyHostToDevice), "hipMemcpy H2D");
    die_hip(hipMemcpy(d_l, logsumexp, n_l * sizeof(float), hipMemcpyHostToDevice), "hipMemcpy H2D");
    die_attn(gpt_hip_attn_bwd_f32(d_gx, d_D, d_l, d_gy, d_y, d_qkv, batch_size, seq_len, hidden_size, num_heads,
                                  nullptr));
    die_hip(hipMemcpy(grad_x, d_gx, n_qkv * sizeof(float), hipMemcpyDeviceToHost), "hipMemcpy D2H");
    die_hip(hipMemcpy(D_cache, d_D, n_l * sizeof(float), hipMemcpyDeviceToHost), "hipMemcpy D2H");
}

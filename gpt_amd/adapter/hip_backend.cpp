// HipBackend: every IGPTBackend op on the gfx950 GPU through the two C-ABI
// libraries. See hip_backend.h.
#include "hip_backend.h"

#include "gpt_hip_attn.h"
#include "gpt_hip_ops.h"

#include <hip/hip_runtime_api.h>

#include <cstdio>
#include <cstdlib>
#include <cstring>

namespace {

void die_hip(hipError_t e, const char *what)
{
    if (e == hipSuccess)
        return;
    std::fprintf(stderr, "[hip_backend] %s failed: %s\n", what, hipGetErrorString(e));
    std::abort();
}

void die_attn(int rc)
{
    if (rc == 0)
        return;
    std::fprintf(stderr, "[hip_backend] gpt_hip_attn error %d: %s\n", rc, gpt_hip_attn_last_error());
    std::abort();
}

void die_ops(int rc)
{
    if (rc == 0)
        return;
    std::fprintf(stderr, "[hip_backend] gpt_hip_ops error %d: %s\n", rc, gpt_hip_ops_last_error());
    std::abort();
}

}  // namespace

HipBackend::HipBackend(unsigned long seed) : seed_(seed), pool_(new Pool)
{
    if (!gpt_hip_attn_device_ok())
    {
        std::fprintf(stderr, "[hip_backend] no usable HIP device\n");
        std::abort();
    }
}

HipBackend::~HipBackend()
{
    // the pooled blocks go back to the runtime; blocks still handed out
    // belong to the caller, whose later device_free calls go straight to
    // hipFree (the pool object itself is kept for them)
    pool_->released = true;
    if (hipDeviceSynchronize() != hipSuccess)
        return;
    for (auto &kv : pool_->free_blocks)
        (void)hipFree(kv.second);
    pool_->free_blocks.clear();
    if (pool_->stage)
        (void)hipHostFree(pool_->stage);
    pool_->stage = nullptr;
    pool_->stage_bytes = 0;
}

void HipBackend::device_get_memory_info(float *free_mb, float *total_mb)
{
    size_t f = 0, t = 0;
    die_hip(hipMemGetInfo(&f, &t), "hipMemGetInfo");
    *free_mb = (float)(f / (1024.0 * 1024.0));
    *total_mb = (float)(t / (1024.0 * 1024.0));
}

// Caching allocation pool. The reference's generator re-sizes the model every
// token: GPT::set_size frees every activation buffer and allocates it again
// for the new prefix length (src/model/gpt.cpp:399-424, called from
// src/infer/infer.cpp:116-118). On the HIP runtime each hipFree waits for the
// device and each hipMalloc maps fresh memory, so here a freed block goes to a
// free list by its bucket size and the next request of that bucket takes it
// back: sizes are rounded up to a power of two from 256 bytes to 1 GiB (a
// prefix that grows by one token stays in its buckets), to a multiple of
// 256 MiB beyond. Reuse is safe without waiting: every op of this backend runs
// on the legacy default stream, in order, so work queued on a block before it
// was freed runs before work queued after it was handed out again. Memory goes
// back to the runtime only when the backend is destroyed.
static size_t pool_bucket(size_t n)
{
    constexpr size_t kMinBucket = 256, kPow2Max = size_t(1) << 30, kLargeStep = size_t(256) << 20;
    if (n <= kMinBucket)
        return kMinBucket;
    if (n > kPow2Max)
        return (n + kLargeStep - 1) / kLargeStep * kLargeStep;
    size_t b = kMinBucket;
    while (b < n)
        b <<= 1;
    return b;
}

void HipBackend::device_malloc(void **ptr, size_t size)
{
    Pool &p = *pool_;
    ++p.mallocs;
    if (p.released)
    {
        die_hip(hipMalloc(ptr, size), "hipMalloc");
        return;
    }
    const size_t b = pool_bucket(size);
    auto it = p.free_blocks.find(b);
    if (it != p.free_blocks.end())
    {
        *ptr = it->second;
        p.free_blocks.erase(it);
        ++p.reused;
    }
    else
    {
        die_hip(hipMalloc(ptr, b), "hipMalloc");
        p.held += b;
    }
    p.block_bytes[*ptr] = b;
}

void HipBackend::device_free(void *ptr)
{
    if (!ptr)
        return;
    Pool &p = *pool_;
    auto it = p.block_bytes.find(ptr);
    if (it == p.block_bytes.end() || p.released)
    {
        // after the destructor (or a block from before it): straight back
        if (it != p.block_bytes.end())
            p.block_bytes.erase(it);
        die_hip(hipFree(ptr), "hipFree");
        return;
    }
    p.free_blocks.emplace(it->second, ptr);
    p.block_bytes.erase(it);
}

void HipBackend::device_memset(void *ptr, int value, size_t size) { die_hip(hipMemset(ptr, value, size), "hipMemset"); }

void HipBackend::device_fill_normal(float *ptr, float mean, float stddev, size_t size)
{
    // a fresh counter-based stream per call: seed, then the call index
    const unsigned long long s = seed_ * 0x9E3779B97F4A7C15ull + (++fills_ << 40);
    die_ops(gpt_hip_fill_normal_f32(ptr, mean, stddev, size, s, nullptr));
}

void HipBackend::device_fill_const(float *ptr, float value, size_t size)
{
    die_ops(gpt_hip_fill_const_f32(ptr, value, size, nullptr));
}

// Host copies of up to kStageMax bytes (the generator's row of logits per
// token, the trainer's token batches) go through a pinned buffer the backend
// owns: a DMA into page-locked memory plus a host memcpy, instead of the
// runtime's pageable-memory path, whose first use in a process can stall a
// call for milliseconds. Larger copies (checkpoints) go straight through.
void *HipBackend::stage(size_t size)
{
    Pool &p = *pool_;
    if (p.released || size == 0 || size > kStageMax)
        return nullptr;
    if (size > p.stage_bytes)
    {
        size_t n = 1 << 16;
        while (n < size)
            n <<= 1;
        if (p.stage)
            die_hip(hipHostFree(p.stage), "hipHostFree");
        p.stage = nullptr;
        die_hip(hipHostMalloc(&p.stage, n, hipHostMallocDefault), "hipHostMalloc");
        p.stage_bytes = n;
    }
    return p.stage;
}

void HipBackend::device_memcpy_d2h(void *dst, const void *src, size_t size)
{
    void *b = stage(size);
    if (!b)
    {
        die_hip(hipMemcpy(dst, src, size, hipMemcpyDeviceToHost), "hipMemcpy D2H");
        return;
    }
    die_hip(hipMemcpy(b, src, size, hipMemcpyDeviceToHost), "hipMemcpy D2H");
    std::memcpy(dst, b, size);
}

void HipBackend::device_memcpy_h2d(void *dst, const void *src, size_t size)
{
    void *b = stage(size);
    if (!b)
    {
        die_hip(hipMemcpy(dst, src, size, hipMemcpyHostToDevice), "hipMemcpy H2D");
        return;
    }
    std::memcpy(b, src, size);
    die_hip(hipMemcpy(dst, b, size, hipMemcpyHostToDevice), "hipMemcpy H2D");
}

void HipBackend::device_embedding_forward(float *y, const float *wte, const float *wpe, const int *input_tokens,
                                          int batch_size, int seq_len, int hidden_size)
{
    // the interface does not pass the vocabulary size: ids unchecked, as in the reference
    die_ops(gpt_hip_embedding_forward_f32(y, wte, wpe, input_tokens, batch_size, seq_len, hidden_size, 0, nullptr));
}

void HipBackend::device_unembedding_forward(float *y, const float *x, const float *wte, int batch_size, int seq_len,
                                            int hidden_size, int vocab_size_padded)
{
    die_ops(gpt_hip_unembedding_forward_f32(y, x, wte, batch_size, seq_len, hidden_size, vocab_size_padded, nullptr));
}

void HipBackend::device_embedding_backward(float *grad_wte, float *grad_wpe, const float *grad_y,
                                           const int *input_tokens, int batch_size, int seq_len, int hidden_size)
{
    die_ops(gpt_hip_embedding_backward_f32(grad_wte, grad_wpe, grad_y, input_tokens, batch_size, seq_len,
                                           hidden_size, 0, nullptr));
}

void HipBackend::device_unembedding_backward(float *grad_x, float *grad_wte, const float *grad_y, const float *x,
                                             const float *wte, int batch_size, int seq_len, int hidden_size,
                                             int vocab_size_padded)
{
    die_ops(gpt_hip_unembedding_backward_f32(grad_x, grad_wte, grad_y, x, wte, batch_size, seq_len, hidden_size,
                                             vocab_size_padded, nullptr));
}

void HipBackend::device_layernorm_residual_fused_forward(float *y, float *means, float *vars, float *x,
                                                         const float *residual, const float *gamma,
                                                         const float *beta, int batch_size, int seq_len,
                                                         int hidden_size)
{
    die_ops(gpt_hip_layernorm_residual_forward_f32(y, means, vars, x, residual, gamma, beta, batch_size, seq_len,
                                                   hidden_size, nullptr));
}

void HipBackend::device_layernorm_residual_fused_backward(float *grad_x, float *grad_gamma, float *grad_beta,
                                                          const float *grad_y, const float *grad_residual,
                                                          const float *x, const float *means, const float *vars,
                                                          const float *gamma, int batch_size, int seq_len,
                                                          int hidden_size)
{
    die_ops(gpt_hip_layernorm_residual_backward_f32(grad_x, grad_gamma, grad_beta, grad_y, grad_residual, x, means,
                                                    vars, gamma, batch_size, seq_len, hidden_size, nullptr));
}

void HipBackend::device_linear_activation_fused_forward(float *y, float *act, const float *x, const float *w,
                                                        const float *b, bool activation, int batch_size,
                                                        int seq_len, int input_size, int output_size)
{
    die_ops(gpt_hip_linear_activation_forward_f32(y, act, x, w, b, activation ? 1 : 0, batch_size, seq_len,
                                                  input_size, output_size, nullptr));
}

void HipBackend::device_linear_backward(float *grad_x, float *grad_w, float *grad_b, const float *grad_y,
                                        const float *x, const float *w, int batch_size, int seq_len, int input_size,
                                        int output_size)
{
    die_ops(gpt_hip_linear_backward_f32(grad_x, grad_w, grad_b, grad_y, x, w, batch_size, seq_len, input_size,
                                        output_size, nullptr));
}

void HipBackend::device_activation_backward(float *grad_x, const float *grad_y, const float *x, int batch_size,
                                            int seq_len, int output_size)
{
    die_ops(gpt_hip_activation_backward_f32(grad_x, grad_y, x, batch_size, seq_len, output_size, nullptr));
}

void HipBackend::device_flash_attention_forward(float *y, float *logsumexp, const float *qkv, int batch_size,
                                                int seq_len, int hidden_size, int num_heads)
{
    die_attn(gpt_hip_attn_fwd_f32(y, logsumexp, qkv, batch_size, seq_len, hidden_size, num_heads, nullptr));
}

void HipBackend::device_flash_attention_backward(float *grad_x, float *D_cache, const float *logsumexp,
                                                 const float *grad_y, const float *y, const float *qkv,
                                                 int batch_size, int seq_len, int hidden_size, int num_heads)
{
    die_attn(gpt_hip_attn_bwd_f32(grad_x, D_cache, logsumexp, grad_y, y, qkv, batch_size, seq_len, hidden_size,
                                  num_heads, nullptr));
}

void HipBackend::device_softmax_forward(float *y, const float *x, int batch_size, int seq_len, int vocab_size,
                                        int vocab_size_padded)
{
    die_ops(gpt_hip_softmax_forward_f32(y, x, batch_size, seq_len, vocab_size, vocab_size_padded, nullptr));
}

void HipBackend::device_cross_entropy_softmax_fused_backward(float *grad_x, const float *y_softmax,
                                                             const int *tokens_labels, int batch_size, int seq_len,
                                                             int vocab_size, int vocab_size_padded)
{
    die_ops(gpt_hip_cross_entropy_softmax_backward_f32(grad_x, y_softmax, tokens_labels, batch_size, seq_len,
                                                       vocab_size, vocab_size_padded, nullptr));
}

void HipBackend::device_cross_entropy_loss(float *loss, const float *y_softmax, const int *tokens_labels,
                                           int batch_size, int seq_len, int vocab_size_padded)
{
    die_ops(gpt_hip_cross_entropy_loss_f32(loss, y_softmax, tokens_labels, batch_size, seq_len, vocab_size_padded,
                                           nullptr));
}

void HipBackend::device_adamw_step(float *params, float *g, float *m, float *v, int size, float lr, float beta1,
                                   float beta2, float eps, float weight_decay, int step)
{
    die_ops(gpt_hip_adamw_step_f32(params, g, m, v, size, lr, beta1, beta2, eps, weight_decay, step, nullptr));
}

void HipBackend::device_scale_and_clip_grad(float *g, int size, float max_norm, int accum_steps)
{
    die_ops(gpt_hip_scale_and_clip_grad_f32(g, size, max_norm, accum_steps, nullptr));
}

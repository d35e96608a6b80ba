// IGPTBackend with every op on the gfx950 GPU: the reference's full op
// interface (src/backend/backend_interface.h:5-238) bound to the two C-ABI
// libraries of this project,
//   attention  gpt_amd/libgpt_hip_attn.so  (include/gpt_hip_attn.h)
//   the rest   gpt_amd/libgpt_hip_ops.so   (include/gpt_hip_ops.h)
// plus the HIP runtime for memory. It has the shape of the reference's own
// GPU backend (src/backend/cuda/cuda_backend.h:8-46): device pointers
// throughout, the legacy default stream, abort with a message on any error
// (src/backend/cuda/utils/cuda_utils.cuh:21-34).
#pragma once

#include "backend_interface.h"

#include <cstddef>
#include <map>
#include <unordered_map>

class HipBackend : public IGPTBackend
{
public:
    explicit HipBackend(unsigned long seed = 42);
    ~HipBackend() override;

    void device_get_memory_info(float *free_mb, float *total_mb) override;
    void device_malloc(void **ptr, size_t size) override;
    void device_free(void *ptr) override;
    void device_memset(void *ptr, int value, size_t size) override;
    void device_fill_normal(float *ptr, float mean, float stddev, size_t size) override;
    void device_fill_const(float *ptr, float value, size_t size) override;
    void device_memcpy_d2h(void *dst, const void *src, size_t size) override;
    void device_memcpy_h2d(void *dst, const void *src, size_t size) override;
    void device_embedding_forward(float *y, const float *wte, const float *wpe, const int *input_tokens,
                                  int batch_size, int seq_len, int hidden_size) override;
    void device_unembedding_forward(float *y, const float *x, const float *wte, int batch_size, int seq_len,
                                    int hidden_size, int vocab_size_padded) override;
    void device_embedding_backward(float *grad_wte, float *grad_wpe, const float *grad_y, const int *input_tokens,
                                   int batch_size, int seq_len, int hidden_size) override;
    void device_unembedding_backward(float *grad_x, float *grad_wte, const float *grad_y, const float *x,
                                     const float *wte, int batch_size, int seq_len, int hidden_size,
                                     int vocab_size_padded) override;
    void device_layernorm_residual_fused_forward(float *y, float *means, float *vars, float *x, const float *residual,
                                                 const float *gamma, const float *beta, int batch_size, int seq_len,
                                                 int hidden_size) override;
    void device_layernorm_residual_fused_backward(float *grad_x, float *grad_gamma, float *grad_beta,
                                                  const float *grad_y, const float *grad_residual, const float *x,
                                                  const float *means, const float *vars, const float *gamma,
                                                  int batch_size, int seq_len, int hidden_size) override;
    void device_linear_activation_fused_forward(float *y, float *act, const float *x, const float *w, const float *b,
                                                bool activation, int batch_size, int seq_len, int input_size,
                                                int output_size) override;
    void device_linear_backward(float *grad_x, float *grad_w, float *grad_b, const float *grad_y, const float *x,
                                const float *w, int batch_size, int seq_len, int input_size,
                                int output_size) override;
    void device_activation_backward(float *grad_x, const float *grad_y, const float *x, int batch_size, int seq_len,
                                    int output_size) override;
    void device_flash_attention_forward(float *y, float *logsumexp, const float *qkv, int batch_size, int seq_len,
                                        int hidden_size, int num_heads) override;
    void device_flash_attention_backward(float *grad_x, float *D_cache, const float *logsumexp,
                                         const float *grad_y, const float *y, const float *qkv, int batch_size,
                                         int seq_len, int hidden_size, int num_heads) override;
    void device_softmax_forward(float *y, const float *x, int batch_size, int seq_len, int vocab_size,
                                int vocab_size_padded) override;
    void device_cross_entropy_softmax_fused_backward(float *grad_x, const float *y_softmax, const int *tokens_labels,
                                                     int batch_size, int seq_len, int vocab_size,
                                                     int vocab_size_padded) override;
    void device_cross_entropy_loss(float *loss, const float *y_softmax, const int *tokens_labels, int batch_size,
                                   int seq_len, int vocab_size_padded) override;
    void device_adamw_step(float *params, float *g, float *m, float *v, int size, float lr, float beta1, float beta2,
                           float eps, float weight_decay, int step) override;
    void device_scale_and_clip_grad(float *g, int size, float max_norm, int accum_steps) override;

    // Allocation pool statistics: device_malloc calls, of which served from
    // the pool, and the bytes the pool holds from the HIP runtime.
    struct PoolStats
    {
        size_t mallocs, reused, bytes_held;
    };
    PoolStats pool_stats() const { return {pool_->mallocs, pool_->reused, pool_->held}; }

private:
    unsigned long long seed_;
    unsigned long long fills_ = 0;  // fill_normal calls so far: each draws a fresh stream
    // Caching allocation pool (see device_malloc): freed blocks by bucket
    // size, and the bucket size of every block handed out. On the heap and
    // never deleted: the reference's trainer and generator delete their
    // backend (src/train/train.cpp:165, src/infer/infer.cpp:166) before their
    // model and data objects go out of scope and free their buffers through
    // it (src/model/gpt.cpp:92, src/infer/data_manager.cpp:22), so the pool
    // must outlive this object; after the destructor it passes every call
    // straight to the HIP runtime.
    struct Pool
    {
        std::multimap<size_t, void *> free_blocks;
        std::unordered_map<void *, size_t> block_bytes;
        size_t mallocs = 0, reused = 0, held = 0;
        bool released = false;
        // pinned bounce buffer for host copies up to kStageMax bytes
        // (grown to the largest such copy, hipHostMalloc)
        void *stage = nullptr;
        size_t stage_bytes = 0;
    };
    static constexpr size_t kStageMax = size_t(64) << 20;
    void *stage(size_t size);
    Pool *pool_;
};

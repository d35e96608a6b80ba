// IGPTBackend whose attention op pair runs on the gfx950 HIP library
// (include/gpt_hip_attn.h) and whose other ops are the reference's own
// CPUBackend (reference src/backend/cpu/cpu_backend.h:5-32).
//
// This is the reference-side binding of the C ABI: it overrides exactly the
// two methods the library replaces,
//   IGPTBackend::device_flash_attention_forward   backend_interface.h:161-170
//   IGPTBackend::device_flash_attention_backward  backend_interface.h:172-184
// with the same arguments. Because the inherited ops keep tensors in host
// memory (CPUBackend::device_malloc is malloc), each attention call stages
// its tensors into device buffers it owns, calls the library, and copies the
// outputs back; the attention arithmetic itself always runs on the GPU (there
// is no CPU fallback: a library error aborts, as the reference's CUDA backend
// does on any runtime error, src/backend/cuda/utils/cuda_utils.cuh:21-34).
#pragma once

#include "cpu_backend.h"

#include <cstddef>

class HipAttnBackend : public CPUBackend
{
public:
    HipAttnBackend();
    ~HipAttnBackend() override;

    void device_flash_attention_forward(float *y, float *logsumexp, const float *qkv, int batch_size, int seq_len,
                                        int hidden_size, int num_heads) override;
    void device_flash_attention_backward(float *grad_x, float *D_cache, const float *logsumexp,
                                         const float *grad_y, const float *y, const float *qkv, int batch_size,
                                         int seq_len, int hidden_size, int num_heads) override;

private:
    // Grow-only device staging area, carved into 16-byte aligned tensors.
    float *reserve(size_t floats);
    void *dev_ = nullptr;
    size_t dev_bytes_ = 0;
};

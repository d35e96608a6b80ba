/*
 * gpt_hip_ops.h - C ABI of the MI355X (gfx950) GPT-2 ops around the attention
 * path: the reference backend interface's other compute methods (embedding,
 * unembedding, LayerNorm + residual, linear + GELU, GELU backward, vocabulary
 * softmax, cross-entropy, AdamW, gradient scale + clip) and the two fill
 * initialisers. Library: gpt_amd/libgpt_hip_ops.so.
 *
 * Each entry point replaces one virtual method of the reference's op
 * interface IGPTBackend (src/backend/backend_interface.h) with the same
 * arguments in the same order, plus a stream; the CPU backend method it is
 * checked against (src/backend/cpu/cpu_backend.cpp) is cited per function.
 *
 * Conventions (as in gpt_hip_attn.h):
 *   - Every pointer is a DEVICE pointer: fp32 tensors, C-contiguous, int32
 *     token ids, in the reference's layouts (B = batch_size, T = seq_len).
 *   - `stream` is a hipStream_t passed as void*; NULL is the default stream.
 *     Work is enqueued asynchronously; nothing is copied to the host.
 *   - Return 0 or a negative GPT_HIP_OPS_E* code; the message of the last
 *     failure on the calling thread is kept for gpt_hip_ops_last_error().
 *     Validation happens before any device work. Empty shapes are no-ops.
 *   - Accumulating outputs (the reference's "+=": grad_wte, grad_wpe,
 *     grad_gamma, grad_beta, grad_w, grad_b) are added to; every other
 *     output is overwritten. Reductions run in a fixed order, so results are
 *     bitwise reproducible run to run (no floating-point atomics).
 *   - Matrix products run on rocBLAS fp32 GEMMs (MFMA, fp32 in, fp32
 *     accumulate; the reference's CUDA backend uses TF32 tensor cores); the
 *     element-wise, normalisation and reduction work runs on this library's
 *     own HIP kernels. Reductions that need partial sums (LayerNorm and bias
 *     gradients, the gradient norm) use a workspace the library allocates on
 *     first use, one per (device, stream), grown when a call needs more (at
 *     most 256 partial rows: a few MB) and kept until the process ends.
 *   - Token ids must lie in [0, vocab_rows) where the entry point takes
 *     vocab_rows > 0; the reference's methods do not receive the vocabulary
 *     size and do not check, and vocab_rows = 0 keeps that behaviour.
 */
#ifndef GPT_HIP_OPS_H
#define GPT_HIP_OPS_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GPT_HIP_OPS_OK 0
#define GPT_HIP_OPS_EINVAL (-1)   /* bad shape or argument */
#define GPT_HIP_OPS_ENULL (-2)    /* a required pointer is NULL */
#define GPT_HIP_OPS_ENODEV (-4)   /* no usable HIP device */
#define GPT_HIP_OPS_ELAUNCH (-5)  /* a kernel launch or library call failed */
#define GPT_HIP_OPS_ERANGE (-6)   /* tensor too large for the index types */
#define GPT_HIP_OPS_ENOMEM (-7)   /* a workspace could not be allocated */

/* y[b,t,:] = wte[tok[b,t],:] + wpe[t,:].
 * Replaces IGPTBackend::device_embedding_forward (backend_interface.h:26-40;
 * CPU cpu_backend.cpp:65-79; CUDA kernels/embedding.cu:29-45). A token id
 * outside [0, vocab_rows) (vocab_rows > 0) gives a row of NaN. */
int gpt_hip_embedding_forward_f32(float *y, const float *wte, const float *wpe, const int *input_tokens,
                                  int batch_size, int seq_len, int hidden_size, int vocab_rows, void *stream);

/* y[b,t,v] = sum_h x[b,t,h] wte[v,h] for v < vocab_size_padded.
 * Replaces IGPTBackend::device_unembedding_forward (backend_interface.h:42-51;
 * CPU cpu_backend.cpp:81-100; CUDA kernels/embedding.cu:47-63). */
int gpt_hip_unembedding_forward_f32(float *y, const float *x, const float *wte, int batch_size, int seq_len,
                                    int hidden_size, int vocab_size_padded, void *stream);

/* grad_wte[tok[b,t],:] += grad_y[b,t,:] and grad_wpe[t,:] += grad_y[b,t,:],
 * added in the reference's order (b, then t), so the sums are the CPU
 * backend's bit for bit. Replaces IGPTBackend::device_embedding_backward
 * (backend_interface.h:53-68; CPU cpu_backend.cpp:102-117; CUDA
 * kernels/embedding.cu:112-138). Rows with a token id outside
 * [0, vocab_rows) (vocab_rows > 0) are left out of grad_wte. */
int gpt_hip_embedding_backward_f32(float *grad_wte, float *grad_wpe, const float *grad_y, const int *input_tokens,
                                   int batch_size, int seq_len, int hidden_size, int vocab_rows, void *stream);

/* grad_x = grad_y @ wte (overwrite); grad_wte += grad_y^T @ x.
 * Replaces IGPTBackend::device_unembedding_backward (backend_interface.h:70-82;
 * CPU cpu_backend.cpp:119-140; CUDA kernels/embedding.cu:140-170). */
int gpt_hip_unembedding_backward_f32(float *grad_x, float *grad_wte, const float *grad_y, const float *x,
                                     const float *wte, int batch_size, int seq_len, int hidden_size,
                                     int vocab_size_padded, void *stream);

/* x += residual (in place, when residual is not NULL); means, vars = mean and
 * biased variance of each row of x; y = (x - mean) / sqrt(var + 1e-5) * gamma
 * + beta. Replaces IGPTBackend::device_layernorm_residual_fused_forward
 * (backend_interface.h:84-99; CPU cpu_backend.cpp:142-175; CUDA
 * kernels/layernorm.cu:146-164). */
int gpt_hip_layernorm_residual_forward_f32(float *y, float *means, float *vars, float *x, const float *residual,
                                           const float *gamma, const float *beta, int batch_size, int seq_len,
                                           int hidden_size, void *stream);

/* grad_x = LayerNorm input gradient (+ grad_residual when not NULL)
 * (overwrite); grad_gamma += sum over rows of grad_y * x_hat; grad_beta +=
 * sum over rows of grad_y. Replaces
 * IGPTBackend::device_layernorm_residual_fused_backward
 * (backend_interface.h:101-118; CPU cpu_backend.cpp:177-211; CUDA
 * kernels/layernorm.cu:358-394). */
int gpt_hip_layernorm_residual_backward_f32(float *grad_x, float *grad_gamma, float *grad_beta, const float *grad_y,
                                            const float *grad_residual, const float *x, const float *means,
                                            const float *vars, const float *gamma, int batch_size, int seq_len,
                                            int hidden_size, void *stream);

/* y = x @ w + b; act = GELU(y) (tanh form) when activation != 0, else act is
 * not touched (may be NULL). w is [input_size, output_size].
 * Replaces IGPTBackend::device_linear_activation_fused_forward
 * (backend_interface.h:120-132; CPU cpu_backend.cpp:213-239; CUDA
 * kernels/linear.cu:36-66). */
int gpt_hip_linear_activation_forward_f32(float *y, float *act, const float *x, const float *w, const float *b,
                                          int activation, int batch_size, int seq_len, int input_size,
                                          int output_size, void *stream);

/* grad_x = grad_y @ w^T (overwrite); grad_w += x^T @ grad_y; grad_b +=
 * column sums of grad_y. Replaces IGPTBackend::device_linear_backward
 * (backend_interface.h:134-148; CPU cpu_backend.cpp:241-266; CUDA
 * kernels/linear.cu:116-159). */
int gpt_hip_linear_backward_f32(float *grad_x, float *grad_w, float *grad_b, const float *grad_y, const float *x,
                                const float *w, int batch_size, int seq_len, int input_size, int output_size,
                                void *stream);

/* grad_x = grad_y * GELU'(x) (tanh form). Replaces
 * IGPTBackend::device_activation_backward (backend_interface.h:150-159; CPU
 * cpu_backend.cpp:268-287; CUDA kernels/linear.cu:189-203). */
int gpt_hip_activation_backward_f32(float *grad_x, const float *grad_y, const float *x, int batch_size,
                                    int seq_len, int output_size, void *stream);

/* y = softmax over the first vocab_size columns of each row of x; columns
 * vocab_size .. vocab_size_padded - 1 of y are set to 0. Replaces
 * IGPTBackend::device_softmax_forward (backend_interface.h:186-194; CPU
 * cpu_backend.cpp:439-478; CUDA kernels/softmax.cu:112-123). */
int gpt_hip_softmax_forward_f32(float *y, const float *x, int batch_size, int seq_len, int vocab_size,
                                int vocab_size_padded, void *stream);

/* grad_x[r,v] = (y_softmax[r,v] - [v == label_r]) / (B T) for v < vocab_size
 * (columns past vocab_size are not written). Labels outside [0, vocab_size)
 * match no column. Replaces
 * IGPTBackend::device_cross_entropy_softmax_fused_backward
 * (backend_interface.h:196-205; CPU cpu_backend.cpp:480-497; CUDA
 * kernels/cross_entropy.cu:60-76). */
int gpt_hip_cross_entropy_softmax_backward_f32(float *grad_x, const float *y_softmax, const int *tokens_labels,
                                               int batch_size, int seq_len, int vocab_size, int vocab_size_padded,
                                               void *stream);

/* *loss = -(1 / (B T)) sum_r log(y_softmax[r, label_r] + 1e-8), one float in
 * device memory. Labels must lie in [0, vocab_size_padded) (checked on the
 * device: an out-of-range label makes *loss NaN). Replaces
 * IGPTBackend::device_cross_entropy_loss (backend_interface.h:207-216; CPU
 * cpu_backend.cpp:499-515; CUDA kernels/cross_entropy.cu:104-121). */
int gpt_hip_cross_entropy_loss_f32(float *loss, const float *y_softmax, const int *tokens_labels, int batch_size,
                                   int seq_len, int vocab_size_padded, void *stream);

/* One AdamW step over `size` parameters, bias corrections beta^step as the
 * CPU backend computes them (powf on the host), the update in the CPU
 * backend's operation order. Replaces IGPTBackend::device_adamw_step
 * (backend_interface.h:218-228; CPU cpu_backend.cpp:517-532; CUDA
 * kernels/adamw.cu:71-97). */
int gpt_hip_adamw_step_f32(float *params, float *g, float *m, float *v, int size, float lr, float beta1,
                           float beta2, float eps, float weight_decay, int step, void *stream);

/* g /= accum_steps; norm = ||g||_2; if norm > max_norm, g *= max_norm /
 * (norm + 1e-6). The CPU backend's semantics (norm of the scaled gradient);
 * the reference CUDA backend instead takes the norm before scaling.
 * Replaces IGPTBackend::device_scale_and_clip_grad (backend_interface.h:
 * 230-237; CPU cpu_backend.cpp:534-557; CUDA kernels/gradient_clip.cu:
 * 35-59). */
int gpt_hip_scale_and_clip_grad_f32(float *g, int size, float max_norm, int accum_steps, void *stream);

/* Initialisers behind IGPTBackend::device_fill_normal / device_fill_const
 * (backend_interface.h:18-20; CPU cpu_backend.cpp:34-53). fill_normal draws
 * from this library's counter-based generator (splitmix64 of seed and index,
 * Box-Muller), not the CPU backend's rand(): same distribution, different
 * numbers. */
int gpt_hip_fill_normal_f32(float *ptr, float mean, float stddev, size_t size, unsigned long long seed,
                            void *stream);
int gpt_hip_fill_const_f32(float *ptr, float value, size_t size, void *stream);

/* Message for the last non-zero return on the calling thread ("" if none).
 * No reference counterpart (the reference prints and aborts). */
const char *gpt_hip_ops_last_error(void);

/* GEMM planning state, for tests and tuning: *plans = hipBLASLt plans in use
 * (one per shape, transposes and epilogue taken so far in this process),
 * *tuned = how many of them run the kernel this library's tuning table names
 * for the shape (GPT-2 124M's linear layers at 4096 rows, on the two
 * hipBLASLt builds the table covers), *blaslt_version = the loaded hipBLASLt's
 * hipblasLtGetVersion (0 before the first plan). No reference counterpart. */
int gpt_hip_ops_gemm_info(int *plans, int *tuned, int *blaslt_version);

#ifdef __cplusplus
}
#endif

#endif /* GPT_HIP_OPS_H */

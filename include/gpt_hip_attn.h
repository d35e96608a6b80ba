/*
 * gpt_hip_attn.h - C ABI of the MI355X (gfx950) causal self-attention backend.
 *
 * This is the drop-in boundary for the reference's attention op pair. The
 * reference exposes it as two virtual methods of its op-level interface
 * IGPTBackend; a backend adapter implements each method by calling the entry
 * point below with the same arguments in the same order (plus a stream).
 *
 * Conventions shared by every entry point:
 *   - All tensor pointers are DEVICE pointers (hipMalloc'd or equivalent),
 *     fp32, C-contiguous, in the reference's layouts:
 *       qkv     [B, T, 3C]  Q | K | V; head h occupies columns h*d .. h*d+d-1
 *                           of each third, d = C / H
 *       y       [B, T, C]
 *       lse     [B, T, H]   token-major, natural log, of the scaled scores
 *       grad_y  [B, T, C]
 *       grad_x  [B, T, 3C]  dQ | dK | dV
 *       D_cache [B, T, H]
 *   - Softmax scale is 1/sqrt(d); the causal mask keeps key j <= query i.
 *   - `stream` is a hipStream_t passed as void*; NULL means the default stream.
 *     Work is enqueued asynchronously. The forward allocates nothing. The
 *     head_dim-64 backward uses a workspace (a 1 MiB control block, then the
 *     dS tiles: 4 KiB per 32x32 causal tile, 28 MiB at B=16 T=256 H=12, at
 *     most 2 GiB per call: larger problems run in (b, h) chunks) that the
 *     library allocates on first use, one buffer per (device, stream), grows
 *     when a call needs more (after waiting for that stream) and keeps until
 *     the process ends; steady-state calls do not allocate. A call that
 *     would allocate while its stream is capturing a graph returns
 *     GPT_HIP_ATTN_ENOMEM instead (make one call before capturing, or use
 *     gpt_hip_attn_bwd_f32_noalloc).
 *   - Return 0 on success or a negative GPT_HIP_ATTN_E* code; the message of
 *     the last failure on the calling thread is kept for
 *     gpt_hip_attn_last_error(). Inputs are never modified.
 *   - B == 0 or T == 0 is a successful no-op.
 *   - head_dim 64 runs the fp32-MFMA kernels (pointers must be 16-byte
 *     aligned, which the reference's 4-float tensor padding guarantees);
 *     any other head_dim in 1..256, or a misaligned pointer, runs the
 *     general-d HIP kernels. Results are bitwise reproducible run to run
 *     (no atomics) unless path 2 is selected.
 */
#ifndef GPT_HIP_ATTN_H
#define GPT_HIP_ATTN_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GPT_HIP_ATTN_OK 0
#define GPT_HIP_ATTN_EINVAL (-1)     /* bad shape: B,T < 0, C,H <= 0, C % H != 0 */
#define GPT_HIP_ATTN_ENULL (-2)      /* a required pointer is NULL */
#define GPT_HIP_ATTN_EHEADDIM (-3)   /* head_dim outside 1..256 */
#define GPT_HIP_ATTN_ENODEV (-4)     /* no usable HIP device */
#define GPT_HIP_ATTN_ELAUNCH (-5)    /* a kernel launch failed */
#define GPT_HIP_ATTN_ERANGE (-6)     /* tensor too large for the index types */
#define GPT_HIP_ATTN_ENOMEM (-7)     /* the backward's workspace could not be allocated */

/* Causal attention forward: writes every element of y and lse.
 * Replaces IGPTBackend::device_flash_attention_forward
 * (reference src/backend/backend_interface.h:161-170; CUDA implementation
 * src/backend/cuda/kernels/attention.cu:249-268; CPU oracle
 * src/backend/cpu/cpu_backend.cpp:289-356). Same argument order. */
int gpt_hip_attn_fwd_f32(float *y, float *lse, const float *qkv,
                         int batch_size, int seq_len, int hidden_size, int num_heads,
                         void *stream);

/* Causal attention backward: OVERWRITES grad_x with dQ | dK | dV and writes
 * D_cache[b,t,h] = sum_d grad_y * y. `lse` and `y` are the forward's outputs.
 * Replaces IGPTBackend::device_flash_attention_backward
 * (reference src/backend/backend_interface.h:172-184; CUDA implementation
 * src/backend/cuda/kernels/attention.cu:545-577; CPU oracle
 * src/backend/cpu/cpu_backend.cpp:358-437). Same argument order. */
int gpt_hip_attn_bwd_f32(float *grad_x, float *D_cache, const float *lse,
                         const float *grad_y, const float *y, const float *qkv,
                         int batch_size, int seq_len, int hidden_size, int num_heads,
                         void *stream);

/* Causal attention backward that allocates nothing: the same arguments,
 * results (bit for bit) and status codes as gpt_hip_attn_bwd_f32, but the
 * head_dim-64 path keeps its dS tiles (64 MiB) and control block (1 MiB) in a
 * fixed 65 MiB device array of the
 * library (one copy per device, allocated when the library's code object is
 * loaded on that device and held until the process ends) instead of the
 * per-stream workspace, and no call makes a hipMalloc / hipFree. Returns
 * GPT_HIP_ATTN_ERANGE, before launching anything, when one (b, h)'s dS tiles
 * exceed the array (head_dim 64 and T > 5760). Calls that take the general-d
 * kernels (other head sizes, misaligned pointers) use no dS tiles and run as
 * in gpt_hip_attn_bwd_f32; path 2 of gpt_hip_attn_set_path does not apply
 * here (this entry point always takes the deterministic kernels). All calls on one
 * device share the array: calls that overlap in time on one device (another
 * stream, another host thread) race and must not be issued; calls ordered on
 * one stream are safe. The array's contents are left from the last call.
 * No counterpart in the reference: for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc). */
int gpt_hip_attn_bwd_f32_noalloc(float *grad_x, float *D_cache, const float *lse,
                                 const float *grad_y, const float *y, const float *qkv,
                                 int batch_size, int seq_len, int hidden_size, int num_heads,
                                 void *stream);

/* Number of waits in the one-launch backward (T <= 256) that reached their
 * safety time limit, on the calling thread's current device, since the last
 * call; the counts are cleared. Waits for all work queued on the device
 * first (hipDeviceSynchronize). The owner of a dQ item waits for its dS tiles
 * only a bounded time (about 50 us) and otherwise hands the item to extra
 * workgroups at the end of the grid, which wait only for work that waits for
 * nothing itself; so a correct run returns 0 whatever else shares the GPU. A
 * nonzero count means that many dQ items read incomplete tiles (wrong dQ
 * rows); when there was one, the control blocks are also cleared here, so
 * that later calls start clean. Returns the count (>= 0), or
 * GPT_HIP_ATTN_ENODEV / GPT_HIP_ATTN_ELAUNCH. No reference counterpart (the
 * reference's dQ uses atomics and never waits). */
int gpt_hip_attn_wait_timeouts(void);

/* Test hook for the one-launch backward's dQ waits (process-wide, read at
 * each launch; not thread-safe). `microseconds` limits the owners' wait
 * before they hand an item over (default 50) and the wait of the workgroups
 * that take handed-over items for those items' counts (a safety limit,
 * default 1000000); a negative value restores both defaults. (Those
 * workgroups' wait for every owner's decision keeps its one-second limit.) `extra_need` is added to every count
 * a dQ item waits for (default 0), so that with extra_need > 0 every owner
 * hands its item over and every taker's wait runs to the limit: this is how
 * tests drive the timeout path without stalling the GPU. Results of a launch
 * made with extra_need > 0 are undefined (its waits time out); the next
 * launch with the defaults is correct. Returns 0, or GPT_HIP_ATTN_EINVAL for
 * extra_need < 0. No reference counterpart. */
int gpt_hip_attn_set_wait_limit(long long microseconds, int extra_need);

/* Frees the default backward's dS workspaces on the calling thread's current
 * device. gpt_hip_attn_bwd_f32 keeps one grow-only workspace per (device,
 * stream) that it first ran on (up to 64 of them per process), so that calls
 * allocate nothing after the first. This call waits for all work queued on
 * the device (hipDeviceSynchronize), frees every workspace there and forgets
 * its stream; the next backward call on a stream allocates again. For
 * long-lived processes that retire streams or want the memory back. Backward
 * calls on other host threads must not overlap it. Returns 0, or
 * GPT_HIP_ATTN_ENODEV / GPT_HIP_ATTN_ELAUNCH with the HIP error in
 * gpt_hip_attn_last_error(). No reference counterpart (the reference
 * backward allocates no memory of its own). */
int gpt_hip_attn_release_workspaces(void);

/* Message for the last non-zero return on the calling thread ("" if none).
 * No reference counterpart: the reference prints and aborts instead
 * (src/backend/cuda/utils/cuda_utils.cuh:21-34); adapters that keep that
 * behaviour print this string before abort(). */
const char *gpt_hip_attn_last_error(void);

/* 1 if a HIP device is present and usable, else 0. No reference counterpart
 * (the reference assumes a device). */
int gpt_hip_attn_device_ok(void);

/* Launch timer, for benchmarks and tracing. gpt_hip_attn_timing_enable(1)
 * makes every later kernel launch of the library time itself with a HIP event
 * pair (head_dim-64 kernels: events set from the dispatch's own start and end
 * timestamps; others: events recorded on the stream around the launches), up
 * to 8192 launches between reads; (0) turns it off.
 * gpt_hip_attn_timing_read() waits for the recorded events, writes the summed
 * milliseconds and the launch count per kernel kind into ms[k] / count[k] for
 * k < n_kinds, forgets the recorded launches and returns how many there were.
 * Kinds: 0 head_dim-64 forward, 1 backward D rows (T > 256; up to T = 256
 * the backward kernels compute them), 2 backward dK/dV (+ dS tiles) of the
 * two-launch form, 3 its dQ kernel, 4 everything else (general-d kernels, the
 * atomic variant), 5 the fused one-launch backward (T <= 256). Not
 * thread-safe. No reference counterpart (the reference times
 * whole training steps with a host clock, src/core/benchmark.h:5-16). */
int gpt_hip_attn_timing_enable(int on);
int gpt_hip_attn_timing_read(double *ms, int *count, int n_kinds);

/* Kernel selection, for tests and tuning only (not thread-safe; process-wide).
 *   path 0  automatic (default): MFMA kernels for head_dim 64, general-d
 *           kernels otherwise and for head_dim-64 calls beyond the MFMA
 *           kernels' 32-bit buffer ranges (T * 3 * hidden_size * 4 bytes
 *           per batch slice >= 2^31; backward also T > 32736)
 *   path 1  always the general-d kernels (a second, independent HIP
 *           implementation used to cross-check the MFMA kernels)
 *   path 2  as 0, but the head_dim-64 backward accumulates dQ with fp32
 *           global atomics (no workspace, not bitwise reproducible); kept to
 *           measure that design against the default
 *   path 3  as 0, but the head_dim-64 backward always takes the two-launch
 *           form (dK/dV + dS tiles, then dQ) instead of the single fused
 *           launch that path 0 takes for T <= 256; kept to measure the two
 *           against each other (both deterministic)
 * Returns the previous path, or GPT_HIP_ATTN_EINVAL for an unknown path.
 * No reference counterpart. */
int gpt_hip_attn_set_path(int path);

#ifdef __cplusplus
}
#endif

#endif /* GPT_HIP_ATTN_H */

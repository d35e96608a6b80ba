// Internal launchers of the attention kernels (called by attn_capi.hip after
// argument validation). Each returns the hipError_t of its launches.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stddef.h>

namespace gpt_attn {

struct Shape
{
    int B, T, C, H, d;
};

// Kernel kinds reported by the optional launch timer (gpt_hip_attn_timing_*).
enum KernelKind
{
    kKindFwd = 0,       // fwd_qs_d64_kernel / fwd_d64_kernel
    kKindRowdot = 1,    // bwd_rowdot_d64_kernel
    kKindDkdv = 2,      // bwd_dkdv_d64_kernel
    kKindDq = 3,        // bwd_dq_d64_kernel
    kKindOther = 4,     // general-d kernels, atomic-variant kernels
    kKindFused = 5,     // bwd_fused_d64_kernel (dK/dV + dS tiles + dQ, one launch)
    kNumKinds = 6
};

// Brackets the launches between begin and end with HIP events on `st` when the
// timer is enabled; no-ops otherwise.
void timer_begin(int kind, hipStream_t st);
void timer_end(hipStream_t st);

// Takes a timer slot for one launch of `kind` when the timer is enabled and
// returns its two events; false (and null events) otherwise.
bool timer_slot(int kind, hipEvent_t *e0, hipEvent_t *e1);

// One kernel launch; with the timer enabled the slot's events go to
// hipExtLaunchKernelGGL, which sets them from the dispatch's own start and end
// timestamps, so the timed span is the kernel alone (no launch gap, no event
// packets between kernels).
template <typename K, typename... Args>
inline void launch_timed(int kind, K kernel, dim3 grid, dim3 block, hipStream_t st, Args... args)
{
    hipEvent_t e0 = nullptr, e1 = nullptr;
    if (timer_slot(kind, &e0, &e1))
        hipExtLaunchKernelGGL(kernel, grid, block, 0, st, e0, e1, 0, args...);
    else
        hipLaunchKernelGGL(kernel, grid, block, 0, st, args...);
}

// Largest dS workspace one backward call asks for; bigger problems are
// processed in chunks of (b, h) pairs that fit.
constexpr size_t kWorkspaceCap = size_t(2) << 30;

// Forward, head_dim 64, fp32 MFMA. Pointers 16-byte aligned.
hipError_t launch_fwd_d64(float *y, float *lse, const float *qkv, const Shape &s, hipStream_t st);

// Forward, any head_dim in 1..256, scalar HIP kernel.
hipError_t launch_fwd_general(float *y, float *lse, const float *qkv, const Shape &s, hipStream_t st);

// D = rowsum(dO * O) for any head_dim; optionally zeroes the dQ third of grad_x.
hipError_t launch_bwd_prep(float *grad_x, float *D, const float *dy, const float *y, const Shape &s,
                           hipStream_t st, int zero_dq);

// Bytes of dS workspace launch_bwd_d64 needs when it may use at most `cap`
// bytes, and the number of (b, h) pairs processed per chunk with it (0 when
// one (b, h)'s dS tiles alone exceed `cap`; the return value is then that
// one (b, h)'s size).
size_t bwd_d64_workspace_bytes(const Shape &s, size_t cap, int *bh_per_chunk);

// Backward, head_dim 64, fp32 MFMA, deterministic (D rows, dK/dV + dS tiles,
// dQ from the dS tiles). `ws` holds bwd_d64_workspace_bytes(s) bytes.
hipError_t launch_bwd_d64(float *grad_x, float *D, const float *lse, const float *dy, const float *y,
                          const float *qkv, float *ws, int bh_per_chunk, const Shape &s, hipStream_t st);

// Control block of the one-launch fused backward (layout in
// attn_bwd_fused_kernel.h): a word of expired safety waits, then per (b, h, query
// block) a completion counter, per (b, h, key group) an orphan flag and per
// (b, h) a done counter. It sits at the start of the workspace and is zeroed
// when the workspace is allocated; every launch leaves its counters at 0,
// and flags of earlier launches are told apart by the launch epoch.
constexpr size_t kCtlBytes = size_t(1) << 20;
// Control-block word that counts the fused backward's waits that reached
// their safety time limit.
constexpr int kCtlWaitErrors = 16;
// Counters from word kCtlCounters, orphan flags from kCtlCounters +
// kCtlItems, done counters from kCtlCounters + 2 kCtlItems, each region at a
// fixed place whatever the shape.
constexpr int kCtlCounters = 32;
constexpr int kCtlItems = (int)((kCtlBytes / 4 - kCtlCounters) / 3) & ~1;
// Extra workgroups at the end of the fused backward's grid that run orphaned
// dQ items (one per XCD).
constexpr int kOrphanRunners = 8;

// Per-launch parameters of the fused backward's dQ claims.
struct FusedSync
{
    unsigned epoch;          // never 0; differs between consecutive launches on one control block
    int n_main;              // main workgroups (the grid holds kOrphanRunners more)
    int need_extra;          // test hook: added to every awaited count (0 in normal use)
    long long wait_ticks;    // wall-clock ticks (wall_clock64) an owner waits before orphaning its item
    long long safety_ticks;  // wall-clock ticks after which a runner's wait for an item's counts is an error
    long long done_ticks;    // the same for a runner's wait for the main workgroups' decisions
};

// Backward, head_dim 64, fp32 MFMA, deterministic, one launch for T <= 256:
// one dK/dV item per main workgroup, then the dQ of its diagonal blocks once
// their dS tiles are complete (or, after a bounded wait, by an orphan runner).
// Correct whatever part of the grid is resident; taken for grids one round
// of the CUs holds, needing one chunk (bwd_fused_d64_fits). `ws` holds the dS
// tiles of all B * H (b, h), `ctl` the control block; n_cu = compute units.
bool bwd_fused_d64_fits(const Shape &s, int bh_per_chunk, int n_cu);
int bwd_fused_d64_main_workgroups(const Shape &s);
hipError_t launch_bwd_fused_d64(float *grad_x, float *D, const float *lse, const float *dy, const float *y,
                                const float *qkv, float *ws, int *ctl, int n_cu, const FusedSync &sync,
                                const Shape &s, hipStream_t st);

// D = rowsum(dO * O) for head_dim 64 (bwd_rowdot_d64_kernel).
hipError_t launch_bwd_rowdot_d64(float *D, const float *dy, const float *y, const Shape &s, hipStream_t st);

// Compute units of the current device (cached per device; 0 if unknown).
int device_cu_count();

// Backward, head_dim 64, fp32 MFMA with fp32-atomic dQ accumulation (D rows +
// dQ zeroing, then the fused dK/dV/dQ kernel).
hipError_t launch_bwd_d64_atomic(float *grad_x, float *D, const float *lse, const float *dy, const float *y,
                                 const float *qkv, const Shape &s, hipStream_t st);

// Backward, any head_dim in 1..256, scalar HIP kernels (no atomics).
hipError_t launch_bwd_general(float *grad_x, float *D, const float *lse, const float *dy, const float *y,
                              const float *qkv, const Shape &s, hipStream_t st);

}  // namespace gpt_attn

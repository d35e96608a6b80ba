// C ABI of the gfx950 causal-attention backend (declared in
// include/gpt_hip_attn.h): argument validation, kernel selection, status codes.
//
// The reference's op methods return void and abort on any runtime error
// (src/backend/cuda/utils/cuda_utils.cuh:21-34, 64-77); here every entry point
// returns a status and keeps a per-thread message, and the reference-side
// adapter turns a non-zero status back into print + abort.
#include "../../include/gpt_hip_attn.h"
#include "attn_kernels.h"

#include <hip/hip_runtime.h>

#include <atomic>
#include <climits>
#include <mutex>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>

// 65 MiB: the backward's control block (1 MiB) and 64 MiB of dS tiles (one
// (b, h)'s tiles fit up to T = 5760).
static __device__ __align__(256) float scratch[(size_t(65) << 20) / sizeof(float)];

namespace {

thread_local char g_err[512] = "";
// kernel selection (gpt_hip_attn_set_path): 0 automatic, 1 general-d kernels
// only, 2 atomic-dQ backward, 3 two-launch backward at every T; read once per
// call
std::atomic<int> g_path{0};
// Time limits of the fused backward's dQ waits, in microseconds, and the test
// hook's extra count (gpt_hip_attn_set_wait_limit).
// Default limits: how long the owner of a dQ item waits before it hands the
// item to the orphan runners, and the runners' safety limit.
constexpr long long kDefaultOwnerWaitUs = 50;
constexpr long long kDefaultSafetyUs = 1000000;
std::atomic<long long> g_owner_wait_us{kDefaultOwnerWaitUs};
std::atomic<long long> g_safety_us{kDefaultSafetyUs};
std::atomic<int> g_need_extra{0};

// Wall-clock ticks (wall_clock64) per microsecond of the current device.
long long wall_ticks_per_us()
{
    static long long cached[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64)
        return 100;
    if (cached[dev] == 0)
    {
        int khz = 0;
        if (hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev) != hipSuccess || khz <= 0)
            khz = 100000;  // 100 MHz, the gfx9 real-time counter
        cached[dev] = (khz + 999) / 1000;
    }
    return cached[dev];
}


int fail(int code, const char *fmt, ...)
{
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// The head_dim-64 kernels address one batch slice of qkv through a 32-bit
// buffer range and use offsets at or above 2^31 as "no block"; larger slices
// take the general-d kernels.
bool slice_fits_buffer(const gpt_attn::Shape &s) { return (long long)s.T * 3LL * s.C * 4LL < (1LL << 31); }

// The head_dim-64 backward reads one (b, h)'s dS tiles through a buffer range
// too: n (n + 1) / 2 tiles of 4 KiB for n = ceil(T / 32) query blocks, below
// 2^31 bytes up to T = 32736. Longer rows take the general-d kernels.
bool ds_fits_buffer(const gpt_attn::Shape &s)
{
    const long long n = (s.T + 31) / 32;
    return n * (n + 1) / 2 * 4096LL < (1LL << 31);
}

int check_shape(const char *op, int B, int T, int C, int H, gpt_attn::Shape *s)
{
    if (B < 0 || T < 0 || C <= 0 || H <= 0)
        return fail(GPT_HIP_ATTN_EINVAL, "%s: invalid shape B=%d T=%d C=%d H=%d", op, B, T, C, H);
    if (C % H != 0)
        return fail(GPT_HIP_ATTN_EINVAL, "%s: hidden_size %d is not a multiple of num_heads %d", op, C, H);
    const int d = C / H;
    if (d > 256)
        return fail(GPT_HIP_ATTN_EHEADDIM, "%s: head_dim %d is not supported (1..256)", op, d);
    // Element offsets are computed in 64-bit; the grid uses one block per
    // (tile, b, h) or per 128 rows, which must fit a 32-bit grid dimension.
    const long long rows = (long long)B * T * H;
    if ((long long)B * T * 3LL * C >= (1LL << 40) || rows >= (1LL << 31))
        return fail(GPT_HIP_ATTN_ERANGE, "%s: tensor too large (B=%d T=%d C=%d)", op, B, T, C);
    *s = gpt_attn::Shape{B, T, C, H, d};
    return 0;
}

int check_device(const char *op)
{
    int n = 0;
    const hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n <= 0)
        return fail(GPT_HIP_ATTN_ENODEV, "%s: no HIP device (%s)", op,
                    e != hipSuccess ? hipGetErrorString(e) : "device count is 0");
    return 0;
}

// Optional launch timer: when enabled, each head_dim-64 kernel launch takes
// two HIP events (from a fixed pool, reused after every read) that
// hipExtLaunchKernelGGL sets from the dispatch's start and end; the other
// launches are bracketed by two events recorded on their stream.
// gpt_hip_attn_timing_read() waits for them and sums the elapsed time per
// kernel kind. Not thread-safe; meant for one benchmarking thread.
constexpr int kTimerSlots = 8192;
struct LaunchTimer
{
    bool on = false;
    bool ready = false;
    int used = 0;
    int open = -1;
    hipEvent_t ev0[kTimerSlots], ev1[kTimerSlots];
    int kind[kTimerSlots];
};
LaunchTimer g_timer;

// dS workspace of the deterministic backward: one grow-only buffer per
// (device, stream), allocated on first use and kept until the process ends.
// Calls on one stream run in order and share its buffer; calls on different
// streams get different buffers. (A stream-ordered hipMallocAsync /
// hipFreeAsync pair per call measured about 13 us of GPU time per call on
// MI355X, even with the pool keeping its memory.)
struct Workspace
{
    int dev;
    hipStream_t st;
    void *p;
    size_t bytes;
    unsigned epoch;  // of the last fused-backward launch on this control block
};
constexpr int kMaxWorkspaces = 64;
std::mutex g_ws_mu;
Workspace g_ws[kMaxWorkspaces];
int g_ws_n = 0;

// Next launch epoch of a control block: never 0 (the value of a zeroed
// block), different from the previous one.
unsigned next_epoch(unsigned e) { return e + 1 == 0 ? 1 : e + 1; }

// Zeroes n ints (the control block of a new workspace). A kernel rather than
// hipMemsetAsync, so that no memset node is ever recorded into a graph.
__global__ void zero_ints_kernel(int *p, int n)
{
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x)
        p[i] = 0;
}

// Device buffer of at least `bytes` bytes for the backward on `st`, and the
// epoch of its next fused launch (advanced when `fused`). Refuses
// (hipErrorStreamCaptureUnsupported) to allocate while `st` is capturing a
// graph: such callers take gpt_hip_attn_bwd_f32_noalloc, or make one call
// before capturing.
hipError_t workspace_get(void **out, unsigned *epoch, bool fused, size_t bytes, hipStream_t st)
{
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess)
        return e;
    std::lock_guard<std::mutex> lock(g_ws_mu);
    Workspace *w = nullptr;
    for (int i = 0; i < g_ws_n; ++i)
        if (g_ws[i].dev == dev && g_ws[i].st == st)
            w = &g_ws[i];
    if (!w)
    {
        if (g_ws_n == kMaxWorkspaces)
            return hipErrorOutOfMemory;
        w = &g_ws[g_ws_n++];
        *w = Workspace{dev, st, nullptr, 0, 0};
    }
    if (w->bytes < bytes)
    {
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        e = hipStreamIsCapturing(st, &cs);
        if (e != hipSuccess)
            return e;
        if (cs != hipStreamCaptureStatusNone)
            return hipErrorStreamCaptureUnsupported;
        if (w->p)
        {
            // the old buffer may still be read by work queued on this stream
            e = hipStreamSynchronize(st);
            if (e == hipSuccess)
                e = hipFree(w->p);
            if (e != hipSuccess)
                return e;
            w->p = nullptr;
            w->bytes = 0;
        }
        w->epoch = 0;  // a new control block is zeroed below
        e = hipMalloc(&w->p, bytes);
        if (e == hipSuccess)  // the fused backward's control block starts out zeroed
        {
            hipLaunchKernelGGL(zero_ints_kernel, dim3(256), dim3(256), 0, st, static_cast<int *>(w->p),
                               (int)(gpt_attn::kCtlBytes / sizeof(int)));
            e = hipGetLastError();
        }
        if (e != hipSuccess)
        {
            if (w->p)
                (void)hipFree(w->p);
            w->p = nullptr;
            return e;
        }
        w->bytes = bytes;
    }
    *out = w->p;
    if (fused)
        w->epoch = next_epoch(w->epoch);
    *epoch = w->epoch;
    return hipSuccess;
}

// Frees the workspaces of the current device once all its queued work is done.
hipError_t workspace_release_device()
{
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess)
        return e;
    std::lock_guard<std::mutex> lock(g_ws_mu);
    e = hipDeviceSynchronize();
    if (e != hipSuccess)
        return e;
    int n = 0;
    for (int i = 0; i < g_ws_n; ++i)
    {
        if (g_ws[i].dev == dev)
        {
            if (g_ws[i].p)
            {
                const hipError_t f = hipFree(g_ws[i].p);
                if (f != hipSuccess && e == hipSuccess)
                    e = f;
            }
            continue;
        }
        g_ws[n++] = g_ws[i];
    }
    g_ws_n = n;
    return e;
}

// Scratch of the no-allocation backward (gpt_hip_attn_bwd_f32_noalloc): a
// fixed device array that holds the dS tiles in place of the per-stream
// workspace. Each device the library runs on has its own copy, allocated when
// the code object is loaded there and held until the process ends. Host code
// never uses the array's name as an address: the device address of this
// device's copy is looked up once per device (hipGetSymbolAddress) and kept
// in g_scratch.
constexpr size_t kScratchBytes = sizeof(scratch) - gpt_attn::kCtlBytes;  // for dS tiles

constexpr int kMaxDevices = 64;
struct ScratchAddr
{
    std::once_flag once;
    hipError_t err = hipSuccess;
    float *p = nullptr;
    std::mutex mu;
    unsigned epoch = 0;  // of the last fused-backward launch on its control block
};
ScratchAddr g_scratch[kMaxDevices];

// Device address of the current device's scratch array (looked up on the
// first call per device, with that device current) and, when `epoch` is
// given, the epoch of its control block's next fused launch (advanced when
// `fused`).
hipError_t scratch_addr(float **out, unsigned *epoch = nullptr, bool fused = false)
{
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess)
        return e;
    if (dev < 0 || dev >= kMaxDevices)
        return hipErrorInvalidDevice;
    ScratchAddr &s = g_scratch[dev];
    std::call_once(s.once, [&s]() {
        void *p = nullptr;
        s.err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        s.p = s.err == hipSuccess ? static_cast<float *>(p) : nullptr;
    });
    if (s.err != hipSuccess)
        return s.err;
    *out = s.p;
    if (epoch)
    {
        std::lock_guard<std::mutex> lock(s.mu);
        if (fused)
            s.epoch = next_epoch(s.epoch);
        *epoch = s.epoch;
    }
    return hipSuccess;
}

}  // namespace

namespace gpt_attn {

void timer_begin(int kind, hipStream_t st)
{
    LaunchTimer &t = g_timer;
    if (!t.on || t.used >= kTimerSlots)
        return;
    t.open = t.used++;
    t.kind[t.open] = kind;
    (void)hipEventRecord(t.ev0[t.open], st);
}

void timer_end(hipStream_t st)
{
    LaunchTimer &t = g_timer;
    if (!t.on || t.open < 0)
        return;
    (void)hipEventRecord(t.ev1[t.open], st);
    t.open = -1;
}

bool timer_slot(int kind, hipEvent_t *e0, hipEvent_t *e1)
{
    LaunchTimer &t = g_timer;
    *e0 = *e1 = nullptr;
    if (!t.on || t.used >= kTimerSlots)
        return false;
    const int i = t.used++;
    t.kind[i] = kind;
    *e0 = t.ev0[i];
    *e1 = t.ev1[i];
    return true;
}

}  // namespace gpt_attn

namespace {

// Body of both backward entry points. The default one takes its dS workspace
// from the per-(device, stream) buffers above; the no-allocation one
// (noalloc) uses the device's scratch array, allocates nothing and refuses a
// call in which one (b, h)'s dS tiles exceed it.
int backward(const char *op, bool noalloc, float *grad_x, float *D_cache, const float *lse, const float *grad_y,
             const float *y, const float *qkv, int batch_size, int seq_len, int hidden_size, int num_heads,
             void *stream)
{
    gpt_attn::Shape s;
    if (int rc = check_shape(op, batch_size, seq_len, hidden_size, num_heads, &s))
        return rc;
    if (batch_size == 0 || seq_len == 0)
        return 0;
    if (!grad_x || !D_cache || !lse || !grad_y || !y || !qkv)
        return fail(GPT_HIP_ATTN_ENULL, "%s: NULL tensor pointer", op);
    if (int rc = check_device(op))
        return rc;
    const hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    const int path = g_path.load(std::memory_order_relaxed);
    const bool mfma = path != 1 && s.d == 64 && slice_fits_buffer(s) && ds_fits_buffer(s) &&
                      aligned16(grad_x) && aligned16(grad_y) && aligned16(y) && aligned16(qkv);
    if (!mfma)
    {
        const hipError_t e = gpt_attn::launch_bwd_general(grad_x, D_cache, lse, grad_y, y, qkv, s, st);
        if (e != hipSuccess)
            return fail(GPT_HIP_ATTN_ELAUNCH, "%s: launch failed: %s", op, hipGetErrorString(e));
        return 0;
    }
    if (path == 2 && !noalloc)
    {
        const hipError_t e = gpt_attn::launch_bwd_d64_atomic(grad_x, D_cache, lse, grad_y, y, qkv, s, st);
        if (e != hipSuccess)
            return fail(GPT_HIP_ATTN_ELAUNCH, "%s: launch failed: %s", op, hipGetErrorString(e));
        return 0;
    }
    int chunk = 0;
    const size_t bytes =
        gpt_attn::bwd_d64_workspace_bytes(s, noalloc ? kScratchBytes : gpt_attn::kWorkspaceCap, &chunk);
    void *ws = nullptr;
    unsigned epoch = 0;
    hipError_t e = hipSuccess;
    // the fused kernel for grids one round of the CUs holds (T <= 256), unless
    // path 3 asks for the two-launch split
    const int n_cu = gpt_attn::device_cu_count();
    const bool fused = path != 3 && gpt_attn::bwd_fused_d64_fits(s, chunk, n_cu);
    if (noalloc)
    {
        if (chunk == 0)
            return fail(GPT_HIP_ATTN_ERANGE,
                        "%s: one (b, h) needs %zu bytes of dS scratch at T=%d, more than the %zu-byte scratch "
                        "array (T <= 5760 fits)",
                        op, bytes, s.T, kScratchBytes);
        float *p = nullptr;
        e = scratch_addr(&p, &epoch, fused);
        if (e != hipSuccess)
            return fail(GPT_HIP_ATTN_ELAUNCH, "%s: hipGetSymbolAddress(scratch) failed: %s", op,
                        hipGetErrorString(e));
        ws = p;
    }
    else
    {
        e = workspace_get(&ws, &epoch, fused, gpt_attn::kCtlBytes + bytes, st);
        if (e == hipErrorStreamCaptureUnsupported)
            return fail(GPT_HIP_ATTN_ENOMEM,
                        "%s: the stream is capturing a graph and its dS workspace (%zu bytes) is not allocated "
                        "yet: make one call on the stream before capturing, or use gpt_hip_attn_bwd_f32_noalloc",
                        op, gpt_attn::kCtlBytes + bytes);
        if (e != hipSuccess)
            return fail(GPT_HIP_ATTN_ENOMEM, "%s: workspace of %zu bytes: %s", op, gpt_attn::kCtlBytes + bytes,
                        hipGetErrorString(e));
    }
    // workspace layout: [control block | dS tiles]
    int *ctl = static_cast<int *>(ws);
    float *dsw = reinterpret_cast<float *>(static_cast<char *>(ws) + gpt_attn::kCtlBytes);
    if (fused)
    {
        const long long tpu = wall_ticks_per_us();
        const gpt_attn::FusedSync sync{epoch,
                                       gpt_attn::bwd_fused_d64_main_workgroups(s),
                                       g_need_extra.load(std::memory_order_relaxed),
                                       g_owner_wait_us.load(std::memory_order_relaxed) * tpu,
                                       g_safety_us.load(std::memory_order_relaxed) * tpu,
                                       kDefaultSafetyUs * tpu};
        e = gpt_attn::launch_bwd_fused_d64(grad_x, D_cache, lse, grad_y, y, qkv, dsw, ctl, n_cu, sync, s, st);
    }
    else
        e = gpt_attn::launch_bwd_d64(grad_x, D_cache, lse, grad_y, y, qkv, dsw, chunk, s, st);
    if (e != hipSuccess)
        return fail(GPT_HIP_ATTN_ELAUNCH, "%s: launch failed: %s", op, hipGetErrorString(e));
    return 0;
}

}  // namespace

extern "C" {

int gpt_hip_attn_fwd_f32(float *y, float *lse, const float *qkv, int batch_size, int seq_len,
                         int hidden_size, int num_heads, void *stream)
{
    static const char *op = "gpt_hip_attn_fwd_f32";
    gpt_attn::Shape s;
    if (int rc = check_shape(op, batch_size, seq_len, hidden_size, num_heads, &s))
        return rc;
    if (batch_size == 0 || seq_len == 0)
        return 0;
    if (!y || !lse || !qkv)
        return fail(GPT_HIP_ATTN_ENULL, "%s: NULL tensor pointer", op);
    if (int rc = check_device(op))
        return rc;
    const hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    const bool mfma = g_path.load(std::memory_order_relaxed) != 1 && s.d == 64 && slice_fits_buffer(s) &&
                      aligned16(y) && aligned16(qkv);
    const hipError_t e = mfma ? gpt_attn::launch_fwd_d64(y, lse, qkv, s, st)
                              : gpt_attn::launch_fwd_general(y, lse, qkv, s, st);
    if (e != hipSuccess)
        return fail(GPT_HIP_ATTN_ELAUNCH, "%s: launch failed: %s", op, hipGetErrorString(e));
    return 0;
}

int gpt_hip_attn_bwd_f32(float *grad_x, float *D_cache, const float *lse, const float *grad_y,
                         const float *y, const float *qkv, int batch_size, int seq_len, int hidden_size,
                         int num_heads, void *stream)
{
    return backward("gpt_hip_attn_bwd_f32", false, grad_x, D_cache, lse, grad_y, y, qkv, batch_size, seq_len,
                    hidden_size, num_heads, stream);
}

int gpt_hip_attn_bwd_f32_noalloc(float *grad_x, float *D_cache, const float *lse, const float *grad_y,
                                 const float *y, const float *qkv, int batch_size, int seq_len,
                                 int hidden_size, int num_heads, void *stream)
{
    return backward("gpt_hip_attn_bwd_f32_noalloc", true, grad_x, D_cache, lse, grad_y, y, qkv, batch_size,
                    seq_len, hidden_size, num_heads, stream);
}

const char *gpt_hip_attn_last_error(void) { return g_err; }

int gpt_hip_attn_timing_enable(int on)
{
    LaunchTimer &t = g_timer;
    if (on && !t.ready)
    {
        if (int rc = check_device("gpt_hip_attn_timing_enable"))
            return rc;
        for (int i = 0; i < kTimerSlots; ++i)
        {
            if (hipEventCreate(&t.ev0[i]) != hipSuccess || hipEventCreate(&t.ev1[i]) != hipSuccess)
                return fail(GPT_HIP_ATTN_ELAUNCH, "gpt_hip_attn_timing_enable: hipEventCreate failed");
        }
        t.ready = true;
    }
    t.on = on != 0;
    t.used = 0;
    t.open = -1;
    return 0;
}

int gpt_hip_attn_timing_read(double *ms, int *count, int n_kinds)
{
    LaunchTimer &t = g_timer;
    if (!ms || !count || n_kinds <= 0)
        return fail(GPT_HIP_ATTN_ENULL, "gpt_hip_attn_timing_read: NULL output or n_kinds <= 0");
    for (int k = 0; k < n_kinds; ++k)
    {
        ms[k] = 0.0;
        count[k] = 0;
    }
    for (int i = 0; i < t.used; ++i)
    {
        if (hipEventSynchronize(t.ev1[i]) != hipSuccess)
            return fail(GPT_HIP_ATTN_ELAUNCH, "gpt_hip_attn_timing_read: hipEventSynchronize failed");
        float e = 0.f;
        if (hipEventElapsedTime(&e, t.ev0[i], t.ev1[i]) != hipSuccess)
            return fail(GPT_HIP_ATTN_ELAUNCH, "gpt_hip_attn_timing_read: hipEventElapsedTime failed");
        if (t.kind[i] < n_kinds)
        {
            ms[t.kind[i]] += e;
            count[t.kind[i]] += 1;
        }
    }
    const int n = t.used;
    t.used = 0;
    return n;
}

int gpt_hip_attn_device_ok(void)
{
    int n = 0;
    return hipGetDeviceCount(&n) == hipSuccess && n > 0 ? 1 : 0;
}

int gpt_hip_attn_wait_timeouts(void)
{
    static const char *op = "gpt_hip_attn_wait_timeouts";
    if (int rc = check_device(op))
        return rc;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    // every control block of this device: the per-stream workspaces and, once
    // looked up, the no-allocation entry point's scratch array
    // (the lock is held throughout, so that no workspace is freed meanwhile)
    std::lock_guard<std::mutex> lock(g_ws_mu);
    int *blocks[kMaxWorkspaces + 1];
    int ws_index[kMaxWorkspaces];
    int n = 0;
    for (int i = 0; i < g_ws_n && e == hipSuccess; ++i)
        if (g_ws[i].dev == dev && g_ws[i].p)
        {
            ws_index[n] = i;
            blocks[n++] = static_cast<int *>(g_ws[i].p);
        }
    const int n_ws = n;
    float *sp = nullptr;
    if (e == hipSuccess && scratch_addr(&sp) == hipSuccess && sp)
        blocks[n++] = reinterpret_cast<int *>(sp);
    if (e == hipSuccess)
        e = hipDeviceSynchronize();
    long total = 0;
    for (int i = 0; i < n && e == hipSuccess; ++i)
    {
        int v = 0;
        e = hipMemcpy(&v, blocks[i] + gpt_attn::kCtlWaitErrors, sizeof(int), hipMemcpyDeviceToHost);
        if (e == hipSuccess && v != 0)
        {
            // a launch with an expired wait may have left counters or its
            // done count off: start this control block afresh
            e = hipMemset(blocks[i], 0, gpt_attn::kCtlBytes);
            if (i < n_ws)
                g_ws[ws_index[i]].epoch = 0;
            else
            {
                std::lock_guard<std::mutex> sl(g_scratch[dev].mu);
                g_scratch[dev].epoch = 0;
            }
        }
        total += v;
    }
    if (e != hipSuccess)
        return fail(GPT_HIP_ATTN_ELAUNCH, "%s: %s", op, hipGetErrorString(e));
    return total > INT_MAX ? INT_MAX : (int)total;
}

int gpt_hip_attn_release_workspaces(void)
{
    static const char *op = "gpt_hip_attn_release_workspaces";
    if (int rc = check_device(op))
        return rc;
    const hipError_t e = workspace_release_device();
    if (e != hipSuccess)
        return fail(GPT_HIP_ATTN_ELAUNCH, "%s: %s", op, hipGetErrorString(e));
    return 0;
}

int gpt_hip_attn_set_wait_limit(long long microseconds, int extra_need)
{
    if (extra_need < 0)
        return fail(GPT_HIP_ATTN_EINVAL, "gpt_hip_attn_set_wait_limit: extra_need %d < 0", extra_need);
    g_owner_wait_us.store(microseconds < 0 ? kDefaultOwnerWaitUs : microseconds, std::memory_order_relaxed);
    g_safety_us.store(microseconds < 0 ? kDefaultSafetyUs : microseconds, std::memory_order_relaxed);
    g_need_extra.store(extra_need, std::memory_order_relaxed);
    return 0;
}

int gpt_hip_attn_set_path(int path)
{
    if (path < 0 || path > 3)
        return fail(GPT_HIP_ATTN_EINVAL, "gpt_hip_attn_set_path: unknown path %d", path);
    return g_path.exchange(path);
}

}  // extern "C"

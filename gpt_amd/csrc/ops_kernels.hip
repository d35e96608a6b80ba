// gfx950 kernels of the GPT-2 ops around the attention path (C ABI in
// include/gpt_hip_ops.h, entry points in ops_capi.hip).
//
// All of these are HBM-bound: one pass over their operands where the op
// allows it, 16-byte loads and stores when rows are multiples of 4 floats and
// the pointers are 16-byte aligned (scalar variants otherwise), one wave per
// row for the hidden-size rows (C floats) and one 1024-thread workgroup per
// row for the vocabulary rows. Every reduction runs in a fixed order (wave
// sums via DPP / permlane, then waves in index order, then partial rows in
// stripe order), so results are bitwise reproducible; no floating-point
// atomics. Element-wise arithmetic is written in the reference CPU backend's
// operation order and compiled without FMA contraction, so the element-wise
// ops (embedding, AdamW, cross-entropy backward, gradient scaling) reproduce
// that backend's fp32 results exactly; reductions differ from its sequential
// sums only by rounding.
#include "attn_common.h"
#include "ops_internal.h"

#include <float.h>
#include <math.h>
#include <stdint.h>

#pragma clang fp contract(off)

namespace gpt_ops {
namespace {

using gpt_attn::dpp_row;

constexpr float kLnEps = 1e-5f;     // cpu_backend.cpp:173, 186
constexpr float kGeluC = 0.79788456f;  // sqrt(2/pi) as the reference writes it (cpu_backend.cpp:234)
constexpr float kGeluA = 0.044715f;
constexpr float kGeluD = 0.107032f;  // 3 * 0.044715 * sqrt(2/pi) (cpu_backend.cpp:281)
constexpr float kCeEps = 1e-8f;    // cpu_backend.cpp:511
constexpr float kClipEps = 1e-6f;  // cpu_backend.cpp:550

// Sum / max over the 64 lanes of a wave, returned as lane 0's value in every
// lane (the DPP steps add in lane-dependent orders; broadcasting one lane's
// result keeps the row statistics identical across the row).
__device__ __forceinline__ float wave_sum(float x)
{
    x = gpt_attn::row16_sum(x);
    x = gpt_attn::rows16_sum(x);
    x = gpt_attn::halves_sum(x);
    return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(x)));
}

__device__ __forceinline__ float wave_max(float x)
{
    x = fmaxf(x, dpp_row<0x140>(x));
    x = fmaxf(x, dpp_row<0x141>(x));
    x = fmaxf(x, dpp_row<0x4E>(x));
    x = fmaxf(x, dpp_row<0xB1>(x));
    x = gpt_attn::rows16_max(x);
    x = gpt_attn::halves_max(x);
    return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(x)));
}

// Workgroup sum / max for NW waves: wave results through LDS, combined in
// wave order by every thread (same value everywhere). `red` holds NW floats.
template <int NW>
__device__ __forceinline__ float block_sum(float x, float *red)
{
    const float s = wave_sum(x);
    if ((threadIdx.x & 63) == 0)
        red[threadIdx.x >> 6] = s;
    __syncthreads();
    float t = red[0];
#pragma unroll
    for (int k = 1; k < NW; ++k)
        t += red[k];
    __syncthreads();
    return t;
}

template <int NW>
__device__ __forceinline__ float block_max(float x, float *red)
{
    const float s = wave_max(x);
    if ((threadIdx.x & 63) == 0)
        red[threadIdx.x >> 6] = s;
    __syncthreads();
    float t = red[0];
#pragma unroll
    for (int k = 1; k < NW; ++k)
        t = fmaxf(t, red[k]);
    __syncthreads();
    return t;
}

__device__ __forceinline__ float gelu(float s)
{
    return 0.5f * s * (1.0f + tanhf(kGeluC * (s + kGeluA * s * s * s)));
}

__device__ __forceinline__ float gelu_grad(float x)
{
    const float tanh_out = tanhf(kGeluC * (x + kGeluA * x * x * x));
    return 0.5f * (1.0f + tanh_out) + 0.5f * x * (1.0f - tanh_out * tanh_out) * (kGeluC + kGeluD * x * x);
}

__device__ __forceinline__ float4 f4(float a) { return make_float4(a, a, a, a); }
__device__ __forceinline__ float4 add4(float4 a, float4 b)
{
    return make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
}

unsigned grid_for(long n, int per_block, long cap = 16384)
{
    long g = (n + per_block - 1) / per_block;
    if (g < 1)
        g = 1;
    return (unsigned)(g < cap ? g : cap);
}

bool al16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// ---------------------------------------------------------------- embedding

// y[r, :] = wte[tok[r], :] + wpe[r % T, :], one wave per row
// (cpu_backend.cpp:65-79).
template <bool V4>
__global__ __launch_bounds__(256) void embedding_fwd_kernel(float *__restrict__ y, const float *__restrict__ wte,
                                                            const float *__restrict__ wpe,
                                                            const int *__restrict__ tok, int T, int C, long rows,
                                                            int vocab_rows)
{
    const long r = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= rows)
        return;
    const int lane = threadIdx.x & 63;
    const int t = (int)(r % T);
    const int id = tok[r];
    const bool bad = vocab_rows > 0 && (id < 0 || id >= vocab_rows);
    if (V4)
    {
        const int C4 = C >> 2;
        float4 *y4 = reinterpret_cast<float4 *>(y + r * C);
        const float4 *p4 = reinterpret_cast<const float4 *>(wpe + (long)t * C);
        if (bad)
        {
            for (int i = lane; i < C4; i += 64)
                y4[i] = f4(NAN);
            return;
        }
        const float4 *e4 = reinterpret_cast<const float4 *>(wte + (long)id * C);
        for (int i = lane; i < C4; i += 64)
            y4[i] = add4(e4[i], p4[i]);
    }
    else
    {
        float *yr = y + r * C;
        const float *pr = wpe + (long)t * C;
        if (bad)
        {
            for (int i = lane; i < C; i += 64)
                yr[i] = NAN;
            return;
        }
        const float *er = wte + (long)id * C;
        for (int i = lane; i < C; i += 64)
            yr[i] = er[i] + pr[i];
    }
}

// grad_wpe[t, c] += sum over b (ascending) of grad_y[b, t, c]: one thread per
// element (or float4) of grad_wpe, the CPU backend's order for each element
// (cpu_backend.cpp:102-117).
template <bool V4>
__global__ __launch_bounds__(256) void embedding_bwd_wpe_kernel(float *__restrict__ gwpe,
                                                                const float *__restrict__ gy, int B, long tc)
{
    const long i = (long)blockIdx.x * 256 + threadIdx.x;
    if (V4)
    {
        const long n4 = tc >> 2;
        if (i >= n4)
            return;
        float4 *g4 = reinterpret_cast<float4 *>(gwpe);
        const float4 *y4 = reinterpret_cast<const float4 *>(gy);
        float4 acc = g4[i];
        for (int b = 0; b < B; ++b)
            acc = add4(acc, y4[(long)b * n4 + i]);
        g4[i] = acc;
    }
    else
    {
        if (i >= tc)
            return;
        float acc = gwpe[i];
        for (int b = 0; b < B; ++b)
            acc += gy[(long)b * tc + i];
        gwpe[i] = acc;
    }
}

// grad_wte[id, :] += grad_y[r, :] for every row r with token id, added in
// row order: one workgroup per row; the workgroup of a token's first row
// collects the token's rows in ascending order (ballot + prefix count per
// 256-row chunk) and adds them to the grad_wte row it owns alone; the other
// rows' workgroups exit. The result equals the CPU backend's sequential
// accumulation bit for bit (cpu_backend.cpp:102-117) without atomics.
template <bool V4>
__global__ __launch_bounds__(256) void embedding_bwd_wte_kernel(float *__restrict__ gwte,
                                                                const float *__restrict__ gy,
                                                                const int *__restrict__ tok, long rows, int C,
                                                                int vocab_rows)
{
    __shared__ int list[256];
    __shared__ int cnt[4];
    const long r = blockIdx.x;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int id = tok[r];
    if (vocab_rows > 0 && (id < 0 || id >= vocab_rows))
        return;
    int seen = 0;
    for (long q = tid; q < r; q += 256)
        seen |= tok[q] == id;
    if (__syncthreads_or(seen))
        return;
    constexpr int VW = V4 ? 4 : 1;
    for (int c0 = 0; c0 < C; c0 += 256 * VW)
    {
        const int c = c0 + VW * tid;
        const bool own = c < C;
        float *dst = gwte + (long)id * C + c;
        float4 acc4 = f4(0.f);
        float acc = 0.f;
        if (own)
        {
            if (V4)
                acc4 = *reinterpret_cast<const float4 *>(dst);
            else
                acc = *dst;
        }
        for (long q0 = r; q0 < rows; q0 += 256)
        {
            const long q = q0 + tid;
            const bool m = q < rows && tok[q] == id;
            const uint64_t mask = __ballot(m);
            if (lane == 0)
                cnt[w] = __popcll(mask);
            __syncthreads();
            int base = 0;
            for (int k = 0; k < w; ++k)
                base += cnt[k];
            const int total = cnt[0] + cnt[1] + cnt[2] + cnt[3];
            if (m)
                list[base + __popcll(mask & ((1ull << lane) - 1ull))] = (int)(q - q0);
            __syncthreads();
            if (own)
            {
                for (int j = 0; j < total; ++j)
                {
                    const float *src = gy + (q0 + list[j]) * C + c;
                    if (V4)
                        acc4 = add4(acc4, *reinterpret_cast<const float4 *>(src));
                    else
                        acc += *src;
                }
            }
            __syncthreads();
        }
        if (own)
        {
            if (V4)
                *reinterpret_cast<float4 *>(dst) = acc4;
            else
                *dst = acc;
        }
    }
}

// ---------------------------------------------------------------- layernorm

// One wave per row, the row in registers (NV float4 per lane, C <= 256 NV):
// x += residual (written back), mean and biased variance (two passes over the
// registers), y = (x - mean) / sqrt(var + eps) * gamma + beta
// (cpu_backend.cpp:142-175).
template <int NV>
__global__ __launch_bounds__(256) void layernorm_fwd_kernel(float *__restrict__ y, float *__restrict__ means,
                                                            float *__restrict__ vars, float *__restrict__ x,
                                                            const float *__restrict__ res,
                                                            const float *__restrict__ gamma,
                                                            const float *__restrict__ beta, long rows, int C)
{
    const long r = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= rows)
        return;
    const int lane = threadIdx.x & 63, C4 = C >> 2;
    float4 *x4 = reinterpret_cast<float4 *>(x + r * C);
    float4 v[NV];
    float s = 0.f;
#pragma unroll
    for (int k = 0; k < NV; ++k)
    {
        const int i = lane + 64 * k;
        v[k] = f4(0.f);
        if (i < C4)
        {
            v[k] = x4[i];
            if (res)
                v[k] = add4(v[k], reinterpret_cast<const float4 *>(res + r * C)[i]);
        }
        s += (v[k].x + v[k].y) + (v[k].z + v[k].w);
    }
    if (res)
    {
#pragma unroll
        for (int k = 0; k < NV; ++k)
            if (lane + 64 * k < C4)
                x4[lane + 64 * k] = v[k];
    }
    const float mean = wave_sum(s) / (float)C;
    float q = 0.f;
#pragma unroll
    for (int k = 0; k < NV; ++k)
    {
        if (lane + 64 * k < C4)
        {
            const float a = v[k].x - mean, b = v[k].y - mean, c = v[k].z - mean, d = v[k].w - mean;
            q += (a * a + b * b) + (c * c + d * d);
        }
    }
    const float var = wave_sum(q) / (float)C;
    const float den = sqrtf(var + kLnEps);
    if (lane == 0)
    {
        means[r] = mean;
        vars[r] = var;
    }
    float4 *y4 = reinterpret_cast<float4 *>(y + r * C);
    const float4 *g4 = reinterpret_cast<const float4 *>(gamma);
    const float4 *b4 = reinterpret_cast<const float4 *>(beta);
#pragma unroll
    for (int k = 0; k < NV; ++k)
    {
        const int i = lane + 64 * k;
        if (i < C4)
        {
            const float4 g = g4[i], b = b4[i];
            y4[i] = make_float4((v[k].x - mean) / den * g.x + b.x, (v[k].y - mean) / den * g.y + b.y,
                                (v[k].z - mean) / den * g.z + b.z, (v[k].w - mean) / den * g.w + b.w);
        }
    }
}

// Any C / alignment: one 256-thread workgroup per row, three passes over
// memory (each thread re-reads only the elements it wrote).
__global__ __launch_bounds__(256) void layernorm_fwd_generic_kernel(float *__restrict__ y, float *__restrict__ means,
                                                                    float *__restrict__ vars, float *__restrict__ x,
                                                                    const float *__restrict__ res,
                                                                    const float *__restrict__ gamma,
                                                                    const float *__restrict__ beta, int C)
{
    __shared__ float red[4];
    const long r = blockIdx.x;
    float *xr = x + r * C;
    float s = 0.f;
    for (int h = threadIdx.x; h < C; h += 256)
    {
        float v = xr[h];
        if (res)
        {
            v += res[r * C + h];
            xr[h] = v;
        }
        s += v;
    }
    const float mean = block_sum<4>(s, red) / (float)C;
    float q = 0.f;
    for (int h = threadIdx.x; h < C; h += 256)
    {
        const float d = xr[h] - mean;
        q += d * d;
    }
    const float var = block_sum<4>(q, red) / (float)C;
    const float den = sqrtf(var + kLnEps);
    if (threadIdx.x == 0)
    {
        means[r] = mean;
        vars[r] = var;
    }
    for (int h = threadIdx.x; h < C; h += 256)
        y[r * C + h] = (xr[h] - mean) / den * gamma[h] + beta[h];
}

// LayerNorm backward for the rows of one stripe (NW waves x rpw rows, one
// wave per row, the row in registers), CPU backend cpu_backend.cpp:177-211:
//   x_hat = (x - mean) * inv_std, a = grad_y * gamma,
//   grad_x = inv_std * (a - sum(a) / C - x_hat * sum(a * x_hat) / C)
//            (+ grad_residual).
// A wave takes its rows two at a time, issuing both rows' loads before the
// first row's sums. Each lane also sums grad_y * x_hat and grad_y over its
// rows for its columns; the NW waves' sums are added in wave order through
// LDS and stored as the stripe's partial row part[stripe] = [gamma sums |
// beta sums].
template <int NV, int NW>
__global__ __launch_bounds__(NW * 64) void layernorm_bwd_kernel(float *__restrict__ gx,
                                                                const float *__restrict__ gy,
                                                                const float *__restrict__ gres,
                                                                const float *__restrict__ x,
                                                                const float *__restrict__ means,
                                                                const float *__restrict__ vars,
                                                                const float *__restrict__ gamma,
                                                                float *__restrict__ part, long rows, int C, int rpw)
{
    extern __shared__ float4 lds4[];  // [NW][2][C / 4]
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, C4 = C >> 2;
    const float4 *gm4 = reinterpret_cast<const float4 *>(gamma);
    float4 gm[NV], pg[NV], pb[NV];
#pragma unroll
    for (int k = 0; k < NV; ++k)
    {
        const int i = lane + 64 * k;
        gm[k] = i < C4 ? gm4[i] : f4(0.f);
        pg[k] = pb[k] = f4(0.f);
    }
    auto load = [&](long r, float4(&g)[NV], float4(&xv)[NV], float4(&e)[NV]) {
#pragma unroll
        for (int k = 0; k < NV; ++k)
        {
            const int i = lane + 64 * k;
            g[k] = xv[k] = e[k] = f4(0.f);
            if (i < C4)
            {
                g[k] = reinterpret_cast<const float4 *>(gy + r * C)[i];
                xv[k] = reinterpret_cast<const float4 *>(x + r * C)[i];
                if (gres)
                    e[k] = reinterpret_cast<const float4 *>(gres + r * C)[i];
            }
        }
    };
    auto row = [&](long r, float mean, float var, const float4(&g)[NV], const float4(&xv)[NV],
                   const float4(&e)[NV]) {
        const float inv_std = 1.0f / sqrtf(var + kLnEps);
        float4 xh[NV];
        float s1 = 0.f, s2 = 0.f;
#pragma unroll
        for (int k = 0; k < NV; ++k)
        {
            xh[k] = make_float4((xv[k].x - mean) * inv_std, (xv[k].y - mean) * inv_std, (xv[k].z - mean) * inv_std,
                                (xv[k].w - mean) * inv_std);
            if (lane + 64 * k >= C4)
                xh[k] = f4(0.f);
            const float ax = g[k].x * gm[k].x, ay = g[k].y * gm[k].y, az = g[k].z * gm[k].z, aw = g[k].w * gm[k].w;
            s1 += (ax + ay) + (az + aw);
            s2 += (ax * xh[k].x + ay * xh[k].y) + (az * xh[k].z + aw * xh[k].w);
            pg[k] = add4(pg[k], make_float4(g[k].x * xh[k].x, g[k].y * xh[k].y, g[k].z * xh[k].z, g[k].w * xh[k].w));
            pb[k] = add4(pb[k], g[k]);
        }
        const float m1 = wave_sum(s1) / (float)C, m2 = wave_sum(s2) / (float)C;
        float4 *gx4 = reinterpret_cast<float4 *>(gx + r * C);
#pragma unroll
        for (int k = 0; k < NV; ++k)
        {
            const int i = lane + 64 * k;
            if (i < C4)
            {
                float4 o = make_float4(inv_std * (g[k].x * gm[k].x - m1 - xh[k].x * m2),
                                       inv_std * (g[k].y * gm[k].y - m1 - xh[k].y * m2),
                                       inv_std * (g[k].z * gm[k].z - m1 - xh[k].z * m2),
                                       inv_std * (g[k].w * gm[k].w - m1 - xh[k].w * m2));
                if (gres)
                    o = add4(o, e[k]);
                gx4[i] = o;
            }
        }
    };
    const long r0 = ((long)blockIdx.x * NW + w) * rpw;
    for (int j = 0; j < rpw; j += 2)
    {
        const long ra = r0 + j, rb = ra + 1;
        if (ra >= rows)
            break;
        const bool has_b = j + 1 < rpw && rb < rows;
        float4 ga[NV], xa[NV], ea[NV], gb[NV], xb[NV], eb[NV];
        load(ra, ga, xa, ea);
        const float mean_a = means[ra], var_a = vars[ra];
        float mean_b = 0.f, var_b = 0.f;
        if (has_b)
        {
            load(rb, gb, xb, eb);
            mean_b = means[rb];
            var_b = vars[rb];
        }
        row(ra, mean_a, var_a, ga, xa, ea);
        if (has_b)
            row(rb, mean_b, var_b, gb, xb, eb);
    }
#pragma unroll
    for (int k = 0; k < NV; ++k)
    {
        const int i = lane + 64 * k;
        if (i < C4)
        {
            lds4[(w * 2 + 0) * C4 + i] = pg[k];
            lds4[(w * 2 + 1) * C4 + i] = pb[k];
        }
    }
    __syncthreads();
    float4 *p4 = reinterpret_cast<float4 *>(part + (long)blockIdx.x * 2 * C);
    for (int i = threadIdx.x; i < 2 * C4; i += NW * 64)
    {
        const int which = i / C4, c = i % C4;
        float4 t = lds4[(0 * 2 + which) * C4 + c];
        for (int ww = 1; ww < NW; ++ww)
            t = add4(t, lds4[(ww * 2 + which) * C4 + c]);
        p4[i] = t;
    }
}

// Any C / alignment: one 256-thread workgroup per stripe of rpw4 rows, a
// thread owning columns h = tid + 256 k; the stripe's partial row is
// accumulated in place in `part` (each element by one thread only).
__global__ __launch_bounds__(256) void layernorm_bwd_generic_kernel(
    float *__restrict__ gx, const float *__restrict__ gy, const float *__restrict__ gres, const float *__restrict__ x,
    const float *__restrict__ means, const float *__restrict__ vars, const float *__restrict__ gamma,
    float *__restrict__ part, long rows, int C, int rpw4)
{
    __shared__ float red[4];
    float *pg = part + (long)blockIdx.x * 2 * C, *pb = pg + C;
    for (int h = threadIdx.x; h < C; h += 256)
        pg[h] = pb[h] = 0.f;
    const long r0 = (long)blockIdx.x * rpw4;
    for (int j = 0; j < rpw4; ++j)
    {
        const long r = r0 + j;
        if (r >= rows)
            break;
        const float mean = means[r];
        const float inv_std = 1.0f / sqrtf(vars[r] + kLnEps);
        float s1 = 0.f, s2 = 0.f;
        for (int h = threadIdx.x; h < C; h += 256)
        {
            const float g = gy[r * C + h], xh = (x[r * C + h] - mean) * inv_std, a = g * gamma[h];
            s1 += a;
            s2 += a * xh;
            pg[h] += g * xh;
            pb[h] += g;
        }
        const float m1 = block_sum<4>(s1, red) / (float)C, m2 = block_sum<4>(s2, red) / (float)C;
        for (int h = threadIdx.x; h < C; h += 256)
        {
            const float g = gy[r * C + h], xh = (x[r * C + h] - mean) * inv_std;
            float o = inv_std * (g * gamma[h] - m1 - xh * m2);
            if (gres)
                o += gres[r * C + h];
            gx[r * C + h] = o;
        }
    }
}

// ------------------------------------------------------- column reductions

// out0[c] += sum_p part[p][c] (c < N0), out1[c - N0] += ... (N0 <= c < N):
// one workgroup of 16 waves per 64 columns; wave k adds partial rows
// p = k, k + 16, ... (at most 16 of them: parts <= 256) in order, all loads
// issued first, then the 16 wave sums are added in wave order.
__global__ __launch_bounds__(1024) void colsum_final_kernel(float *__restrict__ out0, float *__restrict__ out1,
                                                            const float *__restrict__ part, int parts, int N, int N0)
{
    __shared__ float red[16][64];
    const int lane = threadIdx.x & 63, k = threadIdx.x >> 6;
    const int c = blockIdx.x * 64 + lane;
    float v[16];
#pragma unroll
    for (int j = 0; j < 16; ++j)
    {
        const int p = k + 16 * j;
        v[j] = (c < N && p < parts) ? part[(long)p * N + c] : 0.f;
    }
    float s = v[0];
#pragma unroll
    for (int j = 1; j < 16; ++j)
        if (k + 16 * j < parts)
            s += v[j];
    red[k][lane] = s;
    __syncthreads();
    if (k == 0 && c < N)
    {
        float t = red[0][lane];
        for (int q = 1; q < 16; ++q)
            t += red[q][lane];
        if (c < N0)
            out0[c] += t;
        else
            out1[c - N0] += t;
    }
}

// part[p][c] = sum of gy[r][c] over the rows r of stripe p (ascending), one
// thread per column (float4 when V4), one workgroup per (stripe, 256-thread
// column block).
template <bool V4>
__global__ __launch_bounds__(256) void colsum_partial_kernel(float *__restrict__ part, const float *__restrict__ gy,
                                                             long rows, int N, int rps, int col_blocks)
{
    const int p = blockIdx.x / col_blocks, cb = blockIdx.x % col_blocks;
    const long r0 = (long)p * rps;
    long r1 = r0 + rps;
    if (r1 > rows)
        r1 = rows;
    if (V4)
    {
        const int c4 = cb * 256 + threadIdx.x, N4 = N >> 2;
        if (c4 >= N4)
            return;
        float4 s = f4(0.f);
        for (long r = r0; r < r1; ++r)
            s = add4(s, reinterpret_cast<const float4 *>(gy + r * N)[c4]);
        reinterpret_cast<float4 *>(part + (long)p * N)[c4] = s;
    }
    else
    {
        const int c = cb * 256 + threadIdx.x;
        if (c >= N)
            return;
        float s = 0.f;
        for (long r = r0; r < r1; ++r)
            s += gy[r * N + c];
        part[(long)p * N + c] = s;
    }
}

// ------------------------------------------------------- linear epilogues

// y = y + b[col]; act = GELU(y) (cpu_backend.cpp:213-239), grid-stride.
template <bool V4>
__global__ __launch_bounds__(256) void bias_gelu_kernel(float *__restrict__ y, float *__restrict__ act,
                                                        const float *__restrict__ b, long n, int N)
{
    const long stride = (long)gridDim.x * 256;
    if (V4)
    {
        const long n4 = n >> 2;
        const int N4 = N >> 2;
        float4 *y4 = reinterpret_cast<float4 *>(y);
        float4 *a4 = reinterpret_cast<float4 *>(act);
        const float4 *b4 = reinterpret_cast<const float4 *>(b);
        for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < n4; i += stride)
        {
            const float4 s = add4(y4[i], b4[i % N4]);
            y4[i] = s;
            if (act)
                a4[i] = make_float4(gelu(s.x), gelu(s.y), gelu(s.z), gelu(s.w));
        }
    }
    else
    {
        for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < n; i += stride)
        {
            const float s = y[i] + b[i % N];
            y[i] = s;
            if (act)
                act[i] = gelu(s);
        }
    }
}

// act = GELU(y) (cpu_backend.cpp:234), grid-stride.
template <bool V4>
__global__ __launch_bounds__(256) void gelu_fwd_kernel(float *__restrict__ act, const float *__restrict__ y, long n)
{
    const long stride = (long)gridDim.x * 256;
    if (V4)
    {
        for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < (n >> 2); i += stride)
        {
            const float4 s = reinterpret_cast<const float4 *>(y)[i];
            reinterpret_cast<float4 *>(act)[i] = make_float4(gelu(s.x), gelu(s.y), gelu(s.z), gelu(s.w));
        }
    }
    else
    {
        for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < n; i += stride)
            act[i] = gelu(y[i]);
    }
}

// grad_x = grad_y * GELU'(x) (cpu_backend.cpp:268-287), grid-stride.
template <bool V4>
__global__ __launch_bounds__(256) void gelu_bwd_kernel(float *__restrict__ gx, const float *__restrict__ gy,
                                                       const float *__restrict__ x, long n)
{
    const long stride = (long)gridDim.x * 256;
    if (V4)
    {
        const long n4 = n >> 2;
        for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < n4; i += stride)
        {
            const float4 g = reinterpret_cast<const float4 *>(gy)[i], v = reinterpret_cast<const float4 *>(x)[i];
            reinterpret_cast<float4 *>(gx)[i] =
                make_float4(g.x * gelu_grad(v.x), g.y * gelu_grad(v.y), g.z * gelu_grad(v.z), g.w * gelu_grad(v.w));
        }
    }
    else
    {
        for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < n; i += stride)
            gx[i] = gy[i] * gelu_grad(x[i]);
    }
}

// ------------------------------------------------------ softmax and loss

// Softmax over the first V of Vp columns, one 1024-thread workgroup per row
// holding the row in registers (NPT float4 per thread, Vp <= 4096 NPT): one
// read and one write of the row (cpu_backend.cpp:439-478: max, exp, sum,
// divide; padding columns set to 0).
template <int NPT>
__global__ __launch_bounds__(1024) void softmax_fwd_kernel(float *__restrict__ y, const float *__restrict__ x, int V,
                                                           int Vp)
{
    __shared__ float red[16];
    const long r = blockIdx.x;
    const int tid = threadIdx.x, Vp4 = Vp >> 2;
    const float4 *x4 = reinterpret_cast<const float4 *>(x + r * Vp);
    float4 v[NPT];
    float m = -FLT_MAX;
#pragma unroll
    for (int k = 0; k < NPT; ++k)
    {
        const int i = tid + 1024 * k;
        v[k] = i < Vp4 ? x4[i] : f4(-FLT_MAX);
        const int c = 4 * i;
        if (c + 0 < V)
            m = fmaxf(m, v[k].x);
        if (c + 1 < V)
            m = fmaxf(m, v[k].y);
        if (c + 2 < V)
            m = fmaxf(m, v[k].z);
        if (c + 3 < V)
            m = fmaxf(m, v[k].w);
    }
    const float mx = block_max<16>(m, red);
    float s = 0.f;
#pragma unroll
    for (int k = 0; k < NPT; ++k)
    {
        const int c = 4 * (tid + 1024 * k);
        v[k].x = c + 0 < V ? expf(v[k].x - mx) : 0.f;
        v[k].y = c + 1 < V ? expf(v[k].y - mx) : 0.f;
        v[k].z = c + 2 < V ? expf(v[k].z - mx) : 0.f;
        v[k].w = c + 3 < V ? expf(v[k].w - mx) : 0.f;
        s += (v[k].x + v[k].y) + (v[k].z + v[k].w);
    }
    const float sum = block_sum<16>(s, red);
    float4 *y4 = reinterpret_cast<float4 *>(y + r * Vp);
#pragma unroll
    for (int k = 0; k < NPT; ++k)
    {
        const int i = tid + 1024 * k;
        if (i < Vp4)
        {
            const int c = 4 * i;
            y4[i] = make_float4(c + 0 < V ? v[k].x / sum : 0.f, c + 1 < V ? v[k].y / sum : 0.f,
                                c + 2 < V ? v[k].z / sum : 0.f, c + 3 < V ? v[k].w / sum : 0.f);
        }
    }
}

// Any Vp / alignment: three passes over memory, one workgroup per row.
__global__ __launch_bounds__(1024) void softmax_fwd_generic_kernel(float *__restrict__ y,
                                                                   const float *__restrict__ x, int V, int Vp)
{
    __shared__ float red[16];
    const long r = blockIdx.x;
    const float *xr = x + r * Vp;
    float *yr = y + r * Vp;
    float m = -FLT_MAX;
    for (int c = threadIdx.x; c < V; c += 1024)
        m = fmaxf(m, xr[c]);
    const float mx = block_max<16>(m, red);
    float s = 0.f;
    for (int c = threadIdx.x; c < V; c += 1024)
    {
        const float e = expf(xr[c] - mx);
        yr[c] = e;
        s += e;
    }
    const float sum = block_sum<16>(s, red);
    for (int c = threadIdx.x; c < Vp; c += 1024)
        yr[c] = c < V ? yr[c] / sum : 0.f;
}

// grad_x[r, c] = (y[r, c] - [c == label]) / n for c < V (cpu_backend.cpp:
// 480-497); one workgroup per (row, 1024 columns); columns >= V untouched.
template <bool V4>
__global__ __launch_bounds__(256) void ce_bwd_kernel(float *__restrict__ gx, const float *__restrict__ y,
                                                     const int *__restrict__ labels, int V, int Vp, int col_blocks,
                                                     float n)
{
    const long r = blockIdx.x / col_blocks;
    const int cb = blockIdx.x % col_blocks;
    const int label = labels[r];
    if (V4)
    {
        const int c = 4 * (cb * 256 + threadIdx.x);
        if (c >= V)
            return;
        const float4 v = reinterpret_cast<const float4 *>(y + r * Vp)[c >> 2];
        const float4 o = make_float4((v.x - (c + 0 == label ? 1.0f : 0.0f)) / n,
                                     (v.y - (c + 1 == label ? 1.0f : 0.0f)) / n,
                                     (v.z - (c + 2 == label ? 1.0f : 0.0f)) / n,
                                     (v.w - (c + 3 == label ? 1.0f : 0.0f)) / n);
        float *dst = gx + r * Vp + c;
        if (c + 3 < V)
        {
            // non-temporal: the 824 MB of logit gradients of a GPT-2 step
            // stream out without taking cache lines (341 -> 272 us per call;
            // the hint on softmax's and AdamW's outputs changed nothing)
            typedef float f4v __attribute__((ext_vector_type(4)));
            const f4v ov = {o.x, o.y, o.z, o.w};
            __builtin_nontemporal_store(ov, reinterpret_cast<f4v *>(dst));
        }
        else
        {
            dst[0] = o.x;
            if (c + 1 < V)
                dst[1] = o.y;
            if (c + 2 < V)
                dst[2] = o.z;
        }
    }
    else
    {
        for (int c = cb * 1024 + threadIdx.x; c < V && c < (cb + 1) * 1024; c += 256)
            gx[r * Vp + c] = (y[r * Vp + c] - (c == label ? 1.0f : 0.0f)) / n;
    }
}

// *loss = -(sum_r log(y[r, label_r] + 1e-8)) / rows (cpu_backend.cpp:499-515),
// one workgroup; an out-of-range label contributes NaN.
__global__ __launch_bounds__(1024) void ce_loss_kernel(float *__restrict__ loss, const float *__restrict__ y,
                                                       const int *__restrict__ labels, long rows, int Vp)
{
    __shared__ float red[16];
    float s = 0.f;
    for (long r = threadIdx.x; r < rows; r += 1024)
    {
        const int l = labels[r];
        const float p = (l >= 0 && l < Vp) ? y[r * Vp + l] : NAN;
        s += logf(p + kCeEps);
    }
    const float t = block_sum<16>(s, red);
    if (threadIdx.x == 0)
        *loss = -t / (float)rows;
}

// ------------------------------------------------------ optimizer, clipping

// One AdamW step in the CPU backend's operation order (cpu_backend.cpp:
// 517-532); one_m_b1p = 1 - beta1^step, one_m_b2p = 1 - beta2^step.
__device__ __forceinline__ void adamw_one(float &p, float g, float &m, float &v, float lr, float beta1, float beta2,
                                          float eps, float wd, float one_m_b1p, float one_m_b2p)
{
    m = beta1 * m + (1.0f - beta1) * g;
    v = beta2 * v + (1.0f - beta2) * g * g;
    const float m_hat = m / one_m_b1p;
    const float v_hat = v / one_m_b2p;
    p -= lr * (m_hat / (sqrtf(v_hat) + eps) + wd * p);
}

template <bool V4>
__global__ __launch_bounds__(256) void adamw_kernel(float *__restrict__ p, const float *__restrict__ g,
                                                    float *__restrict__ m, float *__restrict__ v, long n, float lr,
                                                    float beta1, float beta2, float eps, float wd, float one_m_b1p,
                                                    float one_m_b2p)
{
    const long stride = (long)gridDim.x * 256;
    if (V4)
    {
        // two float4 of each stream per iteration, all eight loads issued first
        float4 *p4 = reinterpret_cast<float4 *>(p), *m4 = reinterpret_cast<float4 *>(m),
               *v4 = reinterpret_cast<float4 *>(v);
        const float4 *g4 = reinterpret_cast<const float4 *>(g);
        const long n4 = n >> 2;
        for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < n4; i += 2 * stride)
        {
            const long i2 = i + stride;
            const bool two = i2 < n4;
            float4 pa = p4[i], ma = m4[i], va = v4[i];
            const float4 ga = g4[i];
            float4 pb = f4(0.f), mb = f4(0.f), vb = f4(0.f), gb = f4(0.f);
            if (two)
            {
                pb = p4[i2];
                mb = m4[i2];
                vb = v4[i2];
                gb = g4[i2];
            }
            adamw_one(pa.x, ga.x, ma.x, va.x, lr, beta1, beta2, eps, wd, one_m_b1p, one_m_b2p);
            adamw_one(pa.y, ga.y, ma.y, va.y, lr, beta1, beta2, eps, wd, one_m_b1p, one_m_b2p);
            adamw_one(pa.z, ga.z, ma.z, va.z, lr, beta1, beta2, eps, wd, one_m_b1p, one_m_b2p);
            adamw_one(pa.w, ga.w, ma.w, va.w, lr, beta1, beta2, eps, wd, one_m_b1p, one_m_b2p);
            p4[i] = pa;
            m4[i] = ma;
            v4[i] = va;
            if (two)
            {
                adamw_one(pb.x, gb.x, mb.x, vb.x, lr, beta1, beta2, eps, wd, one_m_b1p, one_m_b2p);
                adamw_one(pb.y, gb.y, mb.y, vb.y, lr, beta1, beta2, eps, wd, one_m_b1p, one_m_b2p);
                adamw_one(pb.z, gb.z, mb.z, vb.z, lr, beta1, beta2, eps, wd, one_m_b1p, one_m_b2p);
                adamw_one(pb.w, gb.w, mb.w, vb.w, lr, beta1, beta2, eps, wd, one_m_b1p, one_m_b2p);
                p4[i2] = pb;
                m4[i2] = mb;
                v4[i2] = vb;
            }
        }
    }
    else
    {
        for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < n; i += stride)
        {
            float pp = p[i], mm = m[i], vv = v[i];
            adamw_one(pp, g[i], mm, vv, lr, beta1, beta2, eps, wd, one_m_b1p, one_m_b2p);
            p[i] = pp;
            m[i] = mm;
            v[i] = vv;
        }
    }
}

constexpr int kClipParts = 4096;

// Partial sums of (g / accum)^2 over fixed stripes: workgroup p covers
// elements [p * stripe, (p + 1) * stripe) (stripe a multiple of 4); g is not
// written here (cpu_backend.cpp:534-557 scales first, then takes the norm of
// the scaled values; the same scaled values are formed here and again when
// they are written).
template <bool V4>
__global__ __launch_bounds__(256) void clip_partial_kernel(float *__restrict__ part, const float *__restrict__ g,
                                                           long n, long stripe, float accum)
{
    __shared__ float red[4];
    const long i0 = (long)blockIdx.x * stripe;
    long i1 = i0 + stripe;
    if (i1 > n)
        i1 = n;
    float s = 0.f;
    if (V4)
    {
        for (long i = i0 + 4L * threadIdx.x; i < i1; i += 1024)
        {
            const float4 v = *reinterpret_cast<const float4 *>(g + i);
            const float a = v.x / accum, b = v.y / accum, c = v.z / accum, d = v.w / accum;
            s += (a * a + b * b) + (c * c + d * d);
        }
    }
    else
    {
        for (long i = i0 + threadIdx.x; i < i1; i += 256)
        {
            const float a = g[i] / accum;
            s += a * a;
        }
    }
    const float t = block_sum<4>(s, red);
    if (threadIdx.x == 0)
        part[blockIdx.x] = t;
}

// norm = sqrt(sum of the partials, in order); g = g / accum, times
// max_norm / (norm + 1e-6) when norm > max_norm. Every workgroup forms the
// same norm from the same partials.
template <bool V4>
__global__ __launch_bounds__(256) void clip_apply_kernel(float *__restrict__ g, const float *__restrict__ part,
                                                         int parts, long n, float max_norm, float accum)
{
    __shared__ float red[4];
    float s = 0.f;
    for (int p = threadIdx.x; p < parts; p += 256)
        s += part[p];
    const float norm = sqrtf(block_sum<4>(s, red));
    const bool clip = !(norm <= max_norm);
    const float scale = max_norm / (norm + kClipEps);
    const long stride = (long)gridDim.x * 256;
    if (V4)
    {
        float4 *g4 = reinterpret_cast<float4 *>(g);
        for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < (n >> 2); i += stride)
        {
            float4 v = g4[i];
            v = make_float4(v.x / accum, v.y / accum, v.z / accum, v.w / accum);
            if (clip)
                v = make_float4(v.x * scale, v.y * scale, v.z * scale, v.w * scale);
            g4[i] = v;
        }
    }
    else
    {
        for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < n; i += stride)
        {
            float v = g[i] / accum;
            if (clip)
                v *= scale;
            g[i] = v;
        }
    }
}

// ------------------------------------------------------------ initialisers

__device__ __forceinline__ uint64_t splitmix64(uint64_t z)
{
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

// Element i: two 24-bit uniforms from splitmix64(seed + 2i), splitmix64(seed
// + 2i + 1); Box-Muller z = sqrt(-2 ln u1) cos(2 pi u2), u1 in (0, 1].
__global__ __launch_bounds__(256) void fill_normal_kernel(float *__restrict__ p, size_t n, float mean, float stddev,
                                                          uint64_t seed)
{
    const size_t stride = (size_t)gridDim.x * 256;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += stride)
    {
        const uint64_t a = splitmix64(seed + 2 * (uint64_t)i), b = splitmix64(seed + 2 * (uint64_t)i + 1);
        const float u1 = (float)((a >> 40) + 1) * 0x1p-24f;
        const float u2 = (float)(b >> 40) * 0x1p-24f;
        const float z = sqrtf(-2.0f * logf(u1)) * cosf(6.2831853071795865f * u2);
        p[i] = z * stddev + mean;
    }
}

__global__ __launch_bounds__(256) void fill_const_kernel(float *__restrict__ p, size_t n, float value)
{
    const size_t stride = (size_t)gridDim.x * 256;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += stride)
        p[i] = value;
}

// Stripe of rows per partial for the column reductions: at most 256
// partials, at least 16 rows per stripe, a multiple of 8 (equal shares for
// the 8 or 4 waves of a LayerNorm-backward workgroup).
long colsum_rows_per_part(long rows)
{
    long rps = (rows + 255) / 256;
    rps = (rps + 7) & ~7L;
    return rps < 16 ? 16 : rps;
}

}  // namespace

int colsum_parts(long rows)
{
    const long rps = colsum_rows_per_part(rows);
    return (int)((rows + rps - 1) / rps);
}

hipError_t launch_embedding_fwd(float *y, const float *wte, const float *wpe, const int *tok, int B, int T, int C,
                                int vocab_rows, hipStream_t st)
{
    const long rows = (long)B * T;
    const bool v4 = C % 4 == 0 && al16(y) && al16(wte) && al16(wpe);
    const dim3 grid((unsigned)((rows + 3) / 4));
    if (v4)
        hipLaunchKernelGGL(embedding_fwd_kernel<true>, grid, dim3(256), 0, st, y, wte, wpe, tok, T, C, rows,
                           vocab_rows);
    else
        hipLaunchKernelGGL(embedding_fwd_kernel<false>, grid, dim3(256), 0, st, y, wte, wpe, tok, T, C, rows,
                           vocab_rows);
    return hipGetLastError();
}

hipError_t launch_embedding_bwd(float *grad_wte, float *grad_wpe, const float *gy, const int *tok, int B, int T,
                                int C, int vocab_rows, hipStream_t st)
{
    const long rows = (long)B * T, tc = (long)T * C;
    const bool v4 = C % 4 == 0 && al16(grad_wte) && al16(grad_wpe) && al16(gy);
    if (v4)
        hipLaunchKernelGGL(embedding_bwd_wpe_kernel<true>, dim3(grid_for(tc / 4, 256, 1L << 30)), dim3(256), 0, st,
                           grad_wpe, gy, B, tc);
    else
        hipLaunchKernelGGL(embedding_bwd_wpe_kernel<false>, dim3(grid_for(tc, 256, 1L << 30)), dim3(256), 0, st,
                           grad_wpe, gy, B, tc);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess)
        return e;
    if (v4)
        hipLaunchKernelGGL(embedding_bwd_wte_kernel<true>, dim3((unsigned)rows), dim3(256), 0, st, grad_wte, gy, tok,
                           rows, C, vocab_rows);
    else
        hipLaunchKernelGGL(embedding_bwd_wte_kernel<false>, dim3((unsigned)rows), dim3(256), 0, st, grad_wte, gy,
                           tok, rows, C, vocab_rows);
    return hipGetLastError();
}

hipError_t launch_layernorm_fwd(float *y, float *means, float *vars, float *x, const float *res,
                                const float *gamma, const float *beta, long rows, int C, hipStream_t st)
{
    const bool v4 = C % 4 == 0 && C <= 4096 && al16(y) && al16(x) && al16(gamma) && al16(beta) &&
                    (!res || al16(res));
    const dim3 grid((unsigned)((rows + 3) / 4)), blk(256);
    if (!v4)
        hipLaunchKernelGGL(layernorm_fwd_generic_kernel, dim3((unsigned)rows), blk, 0, st, y, means, vars, x, res,
                           gamma, beta, C);
    else if (C <= 256)
        hipLaunchKernelGGL(layernorm_fwd_kernel<1>, grid, blk, 0, st, y, means, vars, x, res, gamma, beta, rows, C);
    else if (C <= 512)
        hipLaunchKernelGGL(layernorm_fwd_kernel<2>, grid, blk, 0, st, y, means, vars, x, res, gamma, beta, rows, C);
    else if (C <= 768)
        hipLaunchKernelGGL(layernorm_fwd_kernel<3>, grid, blk, 0, st, y, means, vars, x, res, gamma, beta, rows, C);
    else if (C <= 1024)
        hipLaunchKernelGGL(layernorm_fwd_kernel<4>, grid, blk, 0, st, y, means, vars, x, res, gamma, beta, rows, C);
    else if (C <= 2048)
        hipLaunchKernelGGL(layernorm_fwd_kernel<8>, grid, blk, 0, st, y, means, vars, x, res, gamma, beta, rows, C);
    else
        hipLaunchKernelGGL(layernorm_fwd_kernel<16>, grid, blk, 0, st, y, means, vars, x, res, gamma, beta, rows,
                           C);
    return hipGetLastError();
}

hipError_t launch_layernorm_bwd(float *gx, float *ggamma, float *gbeta, const float *gy, const float *gres,
                                const float *x, const float *means, const float *vars, const float *gamma, long rows,
                                int C, float *ws, hipStream_t st)
{
    const long rps = colsum_rows_per_part(rows);
    const int parts = colsum_parts(rows);
    const bool v4 = C % 4 == 0 && C <= 2048 && al16(gx) && al16(gy) && al16(x) && al16(gamma) &&
                    (!gres || al16(gres));
    const dim3 grid((unsigned)parts);
    if (!v4)
    {
        hipLaunchKernelGGL(layernorm_bwd_generic_kernel, grid, dim3(256), 0, st, gx, gy, gres, x, means, vars, gamma,
                           ws, rows, C, (int)rps);
    }
    else if (C <= 1024)
    {
        // 8 waves per stripe (rps is a multiple of 8): 2 rows a wave at B*T = 4096
        const int rpw = (int)(rps / 8);
        const size_t lds = (size_t)16 * C * sizeof(float);
        const dim3 blk(512);
        if (C <= 256)
            hipLaunchKernelGGL((layernorm_bwd_kernel<1, 8>), grid, blk, lds, st, gx, gy, gres, x, means, vars, gamma,
                               ws, rows, C, rpw);
        else if (C <= 512)
            hipLaunchKernelGGL((layernorm_bwd_kernel<2, 8>), grid, blk, lds, st, gx, gy, gres, x, means, vars, gamma,
                               ws, rows, C, rpw);
        else if (C <= 768)
            hipLaunchKernelGGL((layernorm_bwd_kernel<3, 8>), grid, blk, lds, st, gx, gy, gres, x, means, vars, gamma,
                               ws, rows, C, rpw);
        else
            hipLaunchKernelGGL((layernorm_bwd_kernel<4, 8>), grid, blk, lds, st, gx, gy, gres, x, means, vars, gamma,
                               ws, rows, C, rpw);
    }
    else
    {
        const int rpw = (int)(rps / 4);
        hipLaunchKernelGGL((layernorm_bwd_kernel<8, 4>), grid, dim3(256), (size_t)8 * C * sizeof(float), st, gx, gy,
                           gres, x, means, vars, gamma, ws, rows, C, rpw);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess)
        return e;
    hipLaunchKernelGGL(colsum_final_kernel, dim3((unsigned)((2 * C + 63) / 64)), dim3(1024), 0, st, ggamma, gbeta,
                       ws, parts, 2 * C, C);
    return hipGetLastError();
}

hipError_t launch_bias_gelu(float *y, float *act, const float *b, long rows, int N, hipStream_t st)
{
    const long n = rows * N;
    const bool v4 = N % 4 == 0 && al16(y) && al16(b) && (!act || al16(act));
    if (v4)
        hipLaunchKernelGGL(bias_gelu_kernel<true>, dim3(grid_for(n / 4, 256)), dim3(256), 0, st, y, act, b, n, N);
    else
        hipLaunchKernelGGL(bias_gelu_kernel<false>, dim3(grid_for(n, 256)), dim3(256), 0, st, y, act, b, n, N);
    return hipGetLastError();
}

hipError_t launch_gelu(float *act, const float *y, long rows, int N, hipStream_t st)
{
    const long n = rows * N;
    if (n % 4 == 0 && al16(act) && al16(y))
        hipLaunchKernelGGL(gelu_fwd_kernel<true>, dim3(grid_for(n / 4, 256)), dim3(256), 0, st, act, y, n);
    else
        hipLaunchKernelGGL(gelu_fwd_kernel<false>, dim3(grid_for(n, 256)), dim3(256), 0, st, act, y, n);
    return hipGetLastError();
}

hipError_t launch_bias_grad(float *gb, const float *gy, long rows, int N, float *ws, hipStream_t st)
{
    const long rps = colsum_rows_per_part(rows);
    const int parts = colsum_parts(rows);
    const bool v4 = N % 4 == 0 && al16(gy);
    const int cb = v4 ? (N / 4 + 255) / 256 : (N + 255) / 256;
    if (v4)
        hipLaunchKernelGGL(colsum_partial_kernel<true>, dim3((unsigned)(parts * cb)), dim3(256), 0, st, ws, gy, rows,
                           N, (int)rps, cb);
    else
        hipLaunchKernelGGL(colsum_partial_kernel<false>, dim3((unsigned)(parts * cb)), dim3(256), 0, st, ws, gy,
                           rows, N, (int)rps, cb);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess)
        return e;
    hipLaunchKernelGGL(colsum_final_kernel, dim3((unsigned)((N + 63) / 64)), dim3(1024), 0, st, gb, gb, ws, parts,
                       N, N);
    return hipGetLastError();
}

hipError_t launch_gelu_bwd(float *gx, const float *gy, const float *x, long n, hipStream_t st)
{
    const bool v4 = n % 4 == 0 && al16(gx) && al16(gy) && al16(x);
    if (v4)
        hipLaunchKernelGGL(gelu_bwd_kernel<true>, dim3(grid_for(n / 4, 256)), dim3(256), 0, st, gx, gy, x, n);
    else
        hipLaunchKernelGGL(gelu_bwd_kernel<false>, dim3(grid_for(n, 256)), dim3(256), 0, st, gx, gy, x, n);
    return hipGetLastError();
}

hipError_t launch_softmax_fwd(float *y, const float *x, long rows, int V, int Vp, hipStream_t st)
{
    const bool v4 = Vp % 4 == 0 && Vp <= 65536 && al16(y) && al16(x);
    const dim3 grid((unsigned)rows), blk(1024);
    if (!v4)
        hipLaunchKernelGGL(softmax_fwd_generic_kernel, grid, blk, 0, st, y, x, V, Vp);
    else if (Vp <= 4096)
        hipLaunchKernelGGL(softmax_fwd_kernel<1>, grid, blk, 0, st, y, x, V, Vp);
    else if (Vp <= 16384)
        hipLaunchKernelGGL(softmax_fwd_kernel<4>, grid, blk, 0, st, y, x, V, Vp);
    else if (Vp <= 32768)
        hipLaunchKernelGGL(softmax_fwd_kernel<8>, grid, blk, 0, st, y, x, V, Vp);
    else if (Vp <= 53248)
        hipLaunchKernelGGL(softmax_fwd_kernel<13>, grid, blk, 0, st, y, x, V, Vp);
    else
        hipLaunchKernelGGL(softmax_fwd_kernel<16>, grid, blk, 0, st, y, x, V, Vp);
    return hipGetLastError();
}

hipError_t launch_ce_bwd(float *gx, const float *y, const int *labels, long rows, int V, int Vp, hipStream_t st)
{
    const bool v4 = Vp % 4 == 0 && al16(gx) && al16(y);
    const int cb = (V + 1023) / 1024;
    const dim3 grid((unsigned)(rows * cb));
    if (v4)
        hipLaunchKernelGGL(ce_bwd_kernel<true>, grid, dim3(256), 0, st, gx, y, labels, V, Vp, cb, (float)rows);
    else
        hipLaunchKernelGGL(ce_bwd_kernel<false>, grid, dim3(256), 0, st, gx, y, labels, V, Vp, cb, (float)rows);
    return hipGetLastError();
}

hipError_t launch_ce_loss(float *loss, const float *y, const int *labels, long rows, int Vp, hipStream_t st)
{
    hipLaunchKernelGGL(ce_loss_kernel, dim3(1), dim3(1024), 0, st, loss, y, labels, rows, Vp);
    return hipGetLastError();
}

hipError_t launch_adamw(float *p, const float *g, float *m, float *v, long n, float lr, float beta1, float beta2,
                        float eps, float wd, float one_m_b1p, float one_m_b2p, hipStream_t st)
{
    const bool v4 = n % 4 == 0 && al16(p) && al16(g) && al16(m) && al16(v);
    if (v4)
        hipLaunchKernelGGL(adamw_kernel<true>, dim3(grid_for(n / 4, 256)), dim3(256), 0, st, p, g, m, v, n, lr,
                           beta1, beta2, eps, wd, one_m_b1p, one_m_b2p);
    else
        hipLaunchKernelGGL(adamw_kernel<false>, dim3(grid_for(n, 256)), dim3(256), 0, st, p, g, m, v, n, lr, beta1,
                           beta2, eps, wd, one_m_b1p, one_m_b2p);
    return hipGetLastError();
}

int clip_parts() { return kClipParts; }

hipError_t launch_scale_clip(float *g, long n, float max_norm, float accum, float *ws, hipStream_t st)
{
    const bool v4 = n % 4 == 0 && al16(g);
    long stripe = (n + kClipParts - 1) / kClipParts;
    stripe = (stripe + 3) & ~3L;
    if (v4)
        hipLaunchKernelGGL(clip_partial_kernel<true>, dim3(kClipParts), dim3(256), 0, st, ws, g, n, stripe, accum);
    else
        hipLaunchKernelGGL(clip_partial_kernel<false>, dim3(kClipParts), dim3(256), 0, st, ws, g, n, stripe, accum);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess)
        return e;
    if (v4)
        hipLaunchKernelGGL(clip_apply_kernel<true>, dim3(grid_for(n / 4, 256, 8192)), dim3(256), 0, st, g, ws,
                           kClipParts, n, max_norm, accum);
    else
        hipLaunchKernelGGL(clip_apply_kernel<false>, dim3(grid_for(n, 256, 8192)), dim3(256), 0, st, g, ws,
                           kClipParts, n, max_norm, accum);
    return hipGetLastError();
}

hipError_t launch_fill_normal(float *p, size_t n, float mean, float stddev, unsigned long long seed, hipStream_t st)
{
    hipLaunchKernelGGL(fill_normal_kernel, dim3(grid_for((long)(n < (size_t)1 << 40 ? n : (size_t)1 << 40), 256)),
                       dim3(256), 0, st, p, n, mean, stddev, (uint64_t)seed);
    return hipGetLastError();
}

hipError_t launch_fill_const(float *p, size_t n, float value, hipStream_t st)
{
    hipLaunchKernelGGL(fill_const_kernel, dim3(grid_for((long)(n < (size_t)1 << 40 ? n : (size_t)1 << 40), 256)),
                       dim3(256), 0, st, p, n, value);
    return hipGetLastError();
}

}  // namespace gpt_ops

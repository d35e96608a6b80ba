// Causal self-attention forward for gfx950.
//
// Computes, per (b, h) and query row i,
//   y[i]   = sum_{j<=i} softmax_j(q_i . k_j / sqrt(d)) v_j
//   lse[i] = log sum_{j<=i} exp(q_i . k_j / sqrt(d))
// matching the reference CPU backend (src/backend/cpu/cpu_backend.cpp:289-356)
// and replacing the reference's CUDA kernel (src/backend/cuda/kernels/
// attention.cu:6-268).
//
// head_dim 64 kernel (fwd_d64_kernel). Work unit = one 32-query block x one
// 32-key block of the causal triangle. One workgroup per (b, h, query block);
// its NW waves split the query block's key blocks (wave w takes blocks
// w, w + NW, ...), each keeping its own online-softmax state, and merge the NW
// partial (max, sum, O) triples through LDS at the end. Splitting the key
// range keeps the longest wave at ceil(T / 32 / NW) units, so the causal
// triangle's uneven rows balance across the chip even at T = 256.
//
// Both products run on v_mfma_f32_32x32x2_f32 in the transposed orientation
//     S^T = K Q^T   (32 keys x 32 queries, 32 MFMAs over d = 64)
//     O^T += V^T P^T (64 dims x 32 queries, 2 x 16 MFMAs over 32 keys)
// so that each lane owns ONE query column: the row max / row sum of the online
// softmax are 15 in-lane VALU ops plus one v_permlane32_swap, and the
// probabilities already sit where P^T's B operand needs them (the key order of
// the PV contraction is permuted to the accumulator's row order, so P never
// goes through LDS). K and V go from L2 straight into MFMA operand registers.
// Q is held in registers pre-multiplied by log2(e)/sqrt(d), so the softmax runs
// on v_exp_f32 (2^x) directly.
//
// Workgroup order: query blocks from the last (most key blocks) to the first,
// (b, h) fastest. Workgroups go to the 8 XCDs round-robin, so when B*H is a
// multiple of 8 every workgroup of one (b, h) lands on the same XCD and its
// K/V stay in that XCD's L2.
#include "attn_common.h"
#include "attn_kernels.h"

#include <math.h>

namespace gpt_attn {

template <int NW>
__global__ __launch_bounds__(NW * 64) void fwd_d64_kernel(float *__restrict__ y,
                                                          float *__restrict__ lse,
                                                          const float *__restrict__ qkv,
                                                          int T, int C, int H, int BH, int n_qb,
                                                          float qscale)
{
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int n = lane & 31, hf = lane >> 5;
    const int qb = n_qb - 1 - (int)(blockIdx.x / BH);
    const int bh = (int)(blockIdx.x % BH);
    const int b = bh / H, h = bh % H;
    const long W = 3L * C;
    const float *base = qkv + (long)b * T * W + (long)h * 64;
    const int q0 = 32 * qb;

    // B operand of S^T = K Q^T: lane (n, hf) holds Q[q0 + n][32 hf + s].
    // Rows at or beyond T are read from row T - 1; their outputs are dropped.
    float qreg[32];
    {
        const float4 *src = reinterpret_cast<const float4 *>(base + (long)min(q0 + n, T - 1) * W + 32 * hf);
#pragma unroll
        for (int t = 0; t < 8; ++t)
        {
            const float4 v = src[t];
            qreg[4 * t + 0] = v.x * qscale;
            qreg[4 * t + 1] = v.y * qscale;
            qreg[4 * t + 2] = v.z * qscale;
            qreg[4 * t + 3] = v.w * qscale;
        }
    }

    v16f o0 = zero16(), o1 = zero16();  // O^T rows d = 2 * row + 0 / + 1
    float m = -INFINITY, l = 0.f;       // running max (log2 units) and sum

    for (int j = w; j <= qb; j += NW)
    {
        const int k0 = 32 * j;
        // A operand of S^T: lane (n, hf) holds K[k0 + n][32 hf + s].
        float4 kv[8];
        {
            const float4 *src =
                reinterpret_cast<const float4 *>(base + (long)min(k0 + n, T - 1) * W + C + 32 * hf);
#pragma unroll
            for (int t = 0; t < 8; ++t)
                kv[t] = src[t];
        }
        // A operand of O^T += V^T P^T, step st: V[k0 + row(st, hf)][2n, 2n + 1].
        float2 vv[16];
#pragma unroll
        for (int st = 0; st < 16; ++st)
            vv[st] = *reinterpret_cast<const float2 *>(base + (long)min(k0 + mfma_row(st, hf), T - 1) * W +
                                                      2 * C + 2 * n);

        // S^T[key k0 + row(r)][query q0 + n], in log2 units.
        v16f s = zero16();
#pragma unroll
        for (int t = 0; t < 8; ++t)
        {
            s = mfma32(kv[t].x, qreg[4 * t + 0], s);
            s = mfma32(kv[t].y, qreg[4 * t + 1], s);
            s = mfma32(kv[t].z, qreg[4 * t + 2], s);
            s = mfma32(kv[t].w, qreg[4 * t + 3], s);
        }
        if (j == qb)
        {
            // diagonal block: key k0 + row > query q0 + n is masked out (this
            // also masks keys at or beyond T for every valid query)
#pragma unroll
            for (int r = 0; r < 16; ++r)
                if (mfma_row(r, hf) > n)
                    s[r] = -INFINITY;
        }
        float mt = s[0];
#pragma unroll
        for (int r = 1; r < 16; ++r)
            mt = fmaxf(mt, s[r]);
        mt = halves_max(mt);
        const float mn = fmaxf(m, mt);
        const float corr = fast_exp2(m - mn);
        float ps = 0.f;
#pragma unroll
        for (int r = 0; r < 16; ++r)
        {
            s[r] = fast_exp2(s[r] - mn);
            ps += s[r];
        }
        l = l * corr + halves_sum(ps);
        m = mn;
        o0 *= corr;
        o1 *= corr;

        // O^T += V^T P^T: step st contracts key k0 + row(st, hf) for this
        // half, which is exactly the key of accumulator register st.
#pragma unroll
        for (int st = 0; st < 16; ++st)
        {
            o0 = mfma32(vv[st].x, s[st], o0);
            o1 = mfma32(vv[st].y, s[st], o1);
        }
    }

    if constexpr (NW > 1)
    {
        // Merge the waves' partial states; wave 0 finishes. Layout
        // [wave][register][lane] keeps every LDS access lane-contiguous.
        __shared__ float sm_m[NW][32], sm_l[NW][32];
        __shared__ float sm_o[NW - 1][32][64];
        if (w > 0)
        {
#pragma unroll
            for (int r = 0; r < 16; ++r)
            {
                sm_o[w - 1][r][lane] = o0[r];
                sm_o[w - 1][16 + r][lane] = o1[r];
            }
        }
        if (hf == 0)
        {
            sm_m[w][n] = m;
            sm_l[w][n] = l;
        }
        __syncthreads();
        if (w > 0)
            return;
        float mw[NW], M = m;
#pragma unroll
        for (int v = 0; v < NW; ++v)
        {
            mw[v] = sm_m[v][n];
            M = fmaxf(M, mw[v]);
        }
        // wave 0 always holds key block 0, so M is finite
        const float f0 = fast_exp2(m - M);
        l *= f0;
        o0 *= f0;
        o1 *= f0;
#pragma unroll
        for (int v = 1; v < NW; ++v)
        {
            const float f = fast_exp2(mw[v] - M);  // 0 for a wave that saw no key block
            l += f * sm_l[v][n];
#pragma unroll
            for (int r = 0; r < 16; ++r)
            {
                o0[r] += f * sm_o[v - 1][r][lane];
                o1[r] += f * sm_o[v - 1][16 + r][lane];
            }
        }
        m = M;
    }

    const int row = q0 + n;
    if (row < T)
    {
        const float inv = 1.f / l;
        float *dst = y + ((long)b * T + row) * C + (long)h * 64;
#pragma unroll
        for (int g = 0; g < 4; ++g)
        {
            // registers 4g..4g+3 of o0/o1 hold d = 16g + 8hf + 2j + {0, 1}
            const float4 lo = make_float4(o0[4 * g + 0] * inv, o1[4 * g + 0] * inv,
                                          o0[4 * g + 1] * inv, o1[4 * g + 1] * inv);
            const float4 hi = make_float4(o0[4 * g + 2] * inv, o1[4 * g + 2] * inv,
                                          o0[4 * g + 3] * inv, o1[4 * g + 3] * inv);
            *reinterpret_cast<float4 *>(dst + 16 * g + 8 * hf) = lo;
            *reinterpret_cast<float4 *>(dst + 16 * g + 8 * hf + 4) = hi;
        }
        if (hf == 0)
            lse[((long)b * T + row) * H + h] = (m + fast_log2(l)) * kLn2;
    }
}

// General head_dim (1..DM): one thread per (b, h, query row), online softmax
// over keys 0..i, q and the output row in registers.
template <int DM>
__global__ __launch_bounds__(128) void fwd_general_kernel(float *__restrict__ y,
                                                          float *__restrict__ lse,
                                                          const float *__restrict__ qkv,
                                                          int B, int T, int C, int H, int d,
                                                          float qscale)
{
    const long gid = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= (long)B * H * T)
        return;
    const int i = (int)(gid % T);
    const long bh = gid / T;
    const int h = (int)(bh % H), b = (int)(bh / H);
    const long W = 3L * C;
    const float *base = qkv + (long)b * T * W + (long)h * d;

    float q[DM], o[DM];
#pragma unroll
    for (int e = 0; e < DM; ++e)
    {
        q[e] = e < d ? base[(long)i * W + e] * qscale : 0.f;
        o[e] = 0.f;
    }
    float m = -INFINITY, l = 0.f;
    for (int j = 0; j <= i; ++j)
    {
        const float *kr = base + (long)j * W + C;
        const float *vr = base + (long)j * W + 2L * C;
        float s = 0.f;
#pragma unroll
        for (int e = 0; e < DM; ++e)
            if (e < d)
                s += q[e] * kr[e];
        const float mn = fmaxf(m, s);
        const float corr = fast_exp2(m - mn);
        const float p = fast_exp2(s - mn);
        l = l * corr + p;
#pragma unroll
        for (int e = 0; e < DM; ++e)
            if (e < d)
                o[e] = o[e] * corr + p * vr[e];
        m = mn;
    }
    const float inv = 1.f / l;
    float *dst = y + ((long)b * T + i) * C + (long)h * d;
#pragma unroll
    for (int e = 0; e < DM; ++e)
        if (e < d)
            dst[e] = o[e] * inv;
    lse[((long)b * T + i) * H + h] = (m + fast_log2(l)) * kLn2;
}

static float softmax_scale(int d) { return 1.0f / sqrtf((float)d); }

hipError_t launch_fwd_d64(float *y, float *lse, const float *qkv, const Shape &s, hipStream_t st)
{
    constexpr int NW = 4;
    const int n_qb = (s.T + 31) / 32;
    const int BH = s.B * s.H;
    const long blocks = (long)n_qb * BH;
    const float qscale = softmax_scale(64) * kLog2e;
    hipLaunchKernelGGL((fwd_d64_kernel<NW>), dim3((unsigned)blocks), dim3(NW * 64), 0, st, y, lse, qkv, s.T,
                       s.C, s.H, BH, n_qb, qscale);
    return hipGetLastError();
}

hipError_t launch_fwd_general(float *y, float *lse, const float *qkv, const Shape &s, hipStream_t st)
{
    const long rows = (long)s.B * s.H * s.T;
    const dim3 grid((unsigned)((rows + 127) / 128)), block(128);
    const float qscale = softmax_scale(s.d) * kLog2e;
    if (s.d <= 16)
        hipLaunchKernelGGL(fwd_general_kernel<16>, grid, block, 0, st, y, lse, qkv, s.B, s.T, s.C, s.H, s.d, qscale);
    else if (s.d <= 32)
        hipLaunchKernelGGL(fwd_general_kernel<32>, grid, block, 0, st, y, lse, qkv, s.B, s.T, s.C, s.H, s.d, qscale);
    else if (s.d <= 64)
        hipLaunchKernelGGL(fwd_general_kernel<64>, grid, block, 0, st, y, lse, qkv, s.B, s.T, s.C, s.H, s.d, qscale);
    else if (s.d <= 128)
        hipLaunchKernelGGL(fwd_general_kernel<128>, grid, block, 0, st, y, lse, qkv, s.B, s.T, s.C, s.H, s.d, qscale);
    else
        hipLaunchKernelGGL(fwd_general_kernel<256>, grid, block, 0, st, y, lse, qkv, s.B, s.T, s.C, s.H, s.d, qscale);
    return hipGetLastError();
}

}  // namespace gpt_attn

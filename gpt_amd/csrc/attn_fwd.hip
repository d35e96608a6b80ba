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
// 32-key block of the causal triangle; query block i has i + 1 units. Each
// workgroup takes a heavy/light pair of query blocks (n - 1 - p, p) of one
// (b, h), i.e. n + 1 units for n query blocks, so every workgroup carries the
// same work. Its NW waves split each query block's key blocks round-robin
// (rotated per workgroup so the spare unit lands on a different wave), each
// keeping its own online-softmax state, and merge the NW partial
// (max, sum, O) triples through LDS; wave 0 writes the row.
//
// Both products run on v_mfma_f32_32x32x2_f32 in the transposed orientation
//     S^T = K Q^T   (32 keys x 32 queries, 32 MFMAs over d = 64)
//     O^T += V^T P^T (64 dims x 32 queries, 2 x 16 MFMAs over 32 keys)
// so that each lane owns ONE query column: the row max / row sum of the online
// softmax are 15 in-lane VALU ops plus one v_permlane32_swap, and the
// probabilities already sit where P^T's B operand needs them (the key order of
// the PV contraction is permuted to the accumulator's row order, so P never
// goes through LDS). Q, K and V go from L2 straight into MFMA operand
// registers through buffer loads: rows past T read as zeros (the hardware
// range check), so there are no clamps and no per-row 64-bit address math.
// Q is held pre-multiplied by log2(e)/sqrt(d), so the softmax runs on
// v_exp_f32 (2^x) directly.
//
// Workgroup order: pair-major, (b, h) fastest. Workgroups go to the 8 XCDs
// round-robin, so when B*H is a multiple of 8 every workgroup of one (b, h)
// lands on the same XCD and its K/V stay in that XCD's L2.
#include "attn_common.h"
#include "attn_kernels.h"

#include <math.h>

namespace gpt_attn {

template <int NW>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(3))) void fwd_d64_kernel(float *__restrict__ y,
                                                          float *__restrict__ lse,
                                                          const float *__restrict__ qkv,
                                                          int T, int C, int H, int BH, int n_qb,
                                                          float qscale)
{
    const int lane = threadIdx.x & 63, w = wave_id();
    const int n = lane & 31, hf = lane >> 5;
    const int pr = (int)(blockIdx.x / BH);
    const int bh = (int)(blockIdx.x % BH);
    const int b = bh / H, h = bh % H;
    const uint32_t Wb = 12u * (uint32_t)C;  // bytes per token row of qkv
    const rsrc_t rs = make_rsrc(qkv + (long)b * T * 3L * C + (long)h * 64,
                                (uint32_t)(((long)T * 3 * C - (long)h * 64) * 4));
    // byte offsets of this lane's operands inside a 32-row block
    const uint32_t q_lane = (uint32_t)n * Wb + 128u * hf;                  // Q[n][32 hf ..]
    const uint32_t k_lane = q_lane + 4u * C;                               // K[n][32 hf ..]
    const uint32_t v_lane = 4u * hf * Wb + 8u * C + 8u * (uint32_t)n;      // V[4 hf + ..][2n ..]

    __shared__ float sm_m[2][NW][32], sm_l[2][NW][32];
    __shared__ float sm_o[2][NW > 1 ? NW - 1 : 1][32][64];  // [item][wave - 1][register][lane]

    const int qa = n_qb - 1 - pr;  // heavy query block; the light one is pr
    for (int it = 0; it < 2; ++it)
    {
        const int qb = it == 0 ? qa : pr;
        if (it == 1 && pr == qa)
            break;  // odd n_qb: the middle query block has no partner
        const int q0 = 32 * qb;
        // wave w takes key blocks j with (j + rot) % NW == w
        const int rot = (pr + (it == 0 ? 0 : qa + 1)) % NW;
        const int j0 = (w - rot + NW) % NW;

        // B operand of S^T = K Q^T: lane (n, hf) holds Q[q0 + n][32 hf + s]
        float qreg[32];
#pragma unroll
        for (int t = 0; t < 8; ++t)
        {
            const float4 v = bload4(rs, (uint32_t)q0 * Wb + q_lane + 16u * t);
            qreg[4 * t + 0] = v.x * qscale;
            qreg[4 * t + 1] = v.y * qscale;
            qreg[4 * t + 2] = v.z * qscale;
            qreg[4 * t + 3] = v.w * qscale;
        }

        v16f o0 = zero16(), o1 = zero16();  // O^T rows d = 2 * row + 0 / + 1
        float m = -INFINITY, l = 0.f;       // running max (log2 units) and sum

        // Software pipeline over this wave's key blocks j0, j0 + NW, ...:
        // K of the next block is loaded while this block's softmax and PV run,
        // V of the next block while the next block's S^T runs. A block that
        // does not exist is "loaded" from offset kNoBlock, past the end of the
        // buffer range: the hardware returns zeros without touching memory,
        // so every iteration issues the same loads and no wait depends on a
        // branch.
        // A operands: K[32j + n][32 hf + s] for S^T, and for step st of
        // O^T += V^T P^T, V[32j + row(st, hf)][2n, 2n + 1].
        float4 kv[8];
        float2 vv[16];
        {
            const uint32_t kb = j0 <= qb ? 32u * (uint32_t)j0 * Wb : kNoBlock;
#pragma unroll
            for (int t = 0; t < 8; ++t)
                kv[t] = bload4s(rs, k_lane + 16u * t, kb);
#pragma unroll
            for (int st = 0; st < 16; ++st)
                vv[st] = bload2s(rs, v_lane, kb + (uint32_t)(8 * (st >> 2) + (st & 3)) * Wb);
        }

        for (int j = j0; j <= qb; j += NW)
        {
            const uint32_t kn = j + NW <= qb ? 32u * (uint32_t)(j + NW) * Wb : kNoBlock;

            // S^T[key 32j + row(r)][query q0 + n], in log2 units
            v16f s = zero16();
#pragma unroll
            for (int t = 0; t < 8; ++t)
            {
                s = mfma32(kv[t].x, qreg[4 * t + 0], s);
                s = mfma32(kv[t].y, qreg[4 * t + 1], s);
                s = mfma32(kv[t].z, qreg[4 * t + 2], s);
                s = mfma32(kv[t].w, qreg[4 * t + 3], s);
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int t = 0; t < 8; ++t)
                kv[t] = bload4s(rs, k_lane + 16u * t, kn);
            __builtin_amdgcn_sched_barrier(0);

            if (j == qb)
            {
                // diagonal block: key row(r) > query n is masked out (this also
                // masks keys at or past T for every valid query)
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
            __builtin_amdgcn_sched_barrier(0);

            // O^T += V^T P^T: step st contracts key 32j + row(st, hf) for this
            // half, which is exactly the key of accumulator register st
#pragma unroll
            for (int st = 0; st < 16; ++st)
            {
                o0 = mfma32(vv[st].x, s[st], o0);
                o1 = mfma32(vv[st].y, s[st], o1);
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int st = 0; st < 16; ++st)
                vv[st] = bload2s(rs, v_lane, kn + (uint32_t)(8 * (st >> 2) + (st & 3)) * Wb);
            __builtin_amdgcn_sched_barrier(0);
        }

        if constexpr (NW > 1)
        {
            // Merge the waves' partial states into wave 0. Each item has its
            // own LDS buffer, so no barrier is needed after the merge.
            if (w > 0)
            {
#pragma unroll
                for (int r = 0; r < 16; ++r)
                {
                    sm_o[it][w - 1][r][lane] = o0[r];
                    sm_o[it][w - 1][16 + r][lane] = o1[r];
                }
            }
            if (hf == 0)
            {
                sm_m[it][w][n] = m;
                sm_l[it][w][n] = l;
            }
            __syncthreads();
            if (w > 0)
                continue;
            float M = m;
#pragma unroll
            for (int v = 1; v < NW; ++v)
                M = fmaxf(M, sm_m[it][v][n]);
            // some wave saw key block 0, so M is finite; a wave that saw no
            // key block has m = -inf and contributes 0
            const float f0 = fast_exp2(m - M);
            l *= f0;
            o0 *= f0;
            o1 *= f0;
#pragma unroll
            for (int v = 1; v < NW; ++v)
            {
                const float f = fast_exp2(sm_m[it][v][n] - M);
                l += f * sm_l[it][v][n];
#pragma unroll
                for (int r = 0; r < 16; ++r)
                {
                    o0[r] += f * sm_o[it][v - 1][r][lane];
                    o1[r] += f * sm_o[it][v - 1][16 + r][lane];
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
    const long blocks = (long)((n_qb + 1) / 2) * BH;  // heavy/light pairs
    const float qscale = softmax_scale(64) * kLog2e;
    timer_begin(kKindFwd, st);
    hipLaunchKernelGGL((fwd_d64_kernel<NW>), dim3((unsigned)blocks), dim3(NW * 64), 0, st, y, lse, qkv, s.T,
                       s.C, s.H, BH, n_qb, qscale);
    timer_end(st);
    return hipGetLastError();
}

hipError_t launch_fwd_general(float *y, float *lse, const float *qkv, const Shape &s, hipStream_t st)
{
    const long rows = (long)s.B * s.H * s.T;
    const dim3 grid((unsigned)((rows + 127) / 128)), block(128);
    const float qscale = softmax_scale(s.d) * kLog2e;
    timer_begin(kKindOther, st);
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
    timer_end(st);
    return hipGetLastError();
}

}  // namespace gpt_attn

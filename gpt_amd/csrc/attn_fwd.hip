// Causal self-attention forward for gfx950.
//
// Computes, per (b, h) and query row i,
//   y[i]   = sum_{j<=i} softmax_j(q_i . k_j / sqrt(d)) v_j
//   lse[i] = log sum_{j<=i} exp(q_i . k_j / sqrt(d))
// matching the reference CPU backend (src/backend/cpu/cpu_backend.cpp:289-356)
// and replacing the reference's CUDA kernel (src/backend/cuda/kernels/
// attention.cu:6-268).
//
// head_dim 64 kernel (fwd_d64_kernel): one wave owns 32 query rows; NW waves
// of a workgroup share K/V tiles of BK keys staged in LDS. Both products run
// on v_mfma_f32_32x32x2_f32 in the transposed orientation
//     S^T = K Q^T   (32 keys x 32 queries, 32 MFMAs over d = 64)
//     O^T += V^T P^T (64 dims x 32 queries, 2 x 16 MFMAs over 32 keys)
// so that each lane owns ONE query column: the row max / row sum of the online
// softmax are 15 in-lane VALU ops plus one exchange with the other half-wave,
// and the probabilities already sit where P^T's B operand needs them (the
// key order of the PV contraction is permuted to the accumulator's row order,
// so P never goes through LDS).
// Q is held in registers pre-multiplied by log2(e)/sqrt(d), so the softmax
// runs on v_exp_f32 (2^x) directly.
#include "attn_common.h"
#include "attn_kernels.h"

#include <math.h>

namespace gpt_attn {

// float4 number `idx` of a 64-wide K/V tile starting at key k0 (16 per row).
// Rows at or beyond T are read from row T-1 (always mapped) and replaced by
// zeros with a select, which keeps the load unconditional.
__device__ __forceinline__ void load_kv_f4(float4 &k, float4 &v, const float *base, int idx, int k0, int T,
                                           int C, long W)
{
    const int key = k0 + (idx >> 4), c4 = (idx & 15) * 4;
    const float *src = base + (long)min(key, T - 1) * W + c4;
    const float4 kk = *reinterpret_cast<const float4 *>(src + C);
    const float4 vv = *reinterpret_cast<const float4 *>(src + 2 * C);
    const bool ok = key < T;
    k = make_float4(ok ? kk.x : 0.f, ok ? kk.y : 0.f, ok ? kk.z : 0.f, ok ? kk.w : 0.f);
    v = make_float4(ok ? vv.x : 0.f, ok ? vv.y : 0.f, ok ? vv.z : 0.f, ok ? vv.w : 0.f);
}

template <int NW, int BK>
__global__ __launch_bounds__(NW * 64) void fwd_d64_kernel(float *__restrict__ y,
                                                          float *__restrict__ lse,
                                                          const float *__restrict__ qkv,
                                                          int B, int T, int C, int H,
                                                          float qscale, int n_qt)
{
    constexpr int D = 64, ST = kRowStride, NT = NW * 64;
    constexpr int LOADS = BK * 16 / NT;  // float4 of one K (or V) tile per thread
    static_assert((BK * 16) % NT == 0 && BK % 32 == 0, "tile shape");
    __shared__ __attribute__((aligned(16))) float ks[BK * ST];
    __shared__ __attribute__((aligned(16))) float vs[BK * ST];

    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int n = lane & 31, hf = lane >> 5;
    const int BH = B * H;
    // Heaviest query tiles (most key tiles under the causal mask) go first.
    const int qt = n_qt - 1 - (int)(blockIdx.x / BH);
    const int bh = blockIdx.x % BH;
    const int b = bh / H, h = bh % H;
    const long W = 3L * C;
    const float *base = qkv + (long)b * T * W + (long)h * D;
    const int q0 = qt * 32 * NW;
    const int qw = q0 + 32 * w;  // first query row of this wave

    // B operand of S^T = K Q^T: lane (n, hf) holds Q[qw+n][32*hf + s], s = 0..31.
    // Rows at or beyond T read as zeros.
    float qreg[32];
    {
        const int row = qw + n;
        const float4 *src =
            reinterpret_cast<const float4 *>(base + (long)min(row, T - 1) * W + 32 * hf);
#pragma unroll
        for (int t = 0; t < 8; ++t)
        {
            const float4 v = src[t];
            qreg[4 * t + 0] = row < T ? v.x * qscale : 0.f;
            qreg[4 * t + 1] = row < T ? v.y * qscale : 0.f;
            qreg[4 * t + 2] = row < T ? v.z * qscale : 0.f;
            qreg[4 * t + 3] = row < T ? v.w * qscale : 0.f;
        }
    }

    v16f o0 = zero16(), o1 = zero16();  // O^T rows d = 2*row + 0 / + 1
    float m = -INFINITY, l = 0.f;       // running max (log2 units) and sum

    const int kend = min(T, q0 + 32 * NW);  // keys [0, kend) are visible to the tile
    const int ntiles = (kend + BK - 1) / BK;

    // Next tile's K/V, loaded into registers while the current tile is used.
    float4 kpre[LOADS], vpre[LOADS];
#pragma unroll
    for (int i = 0; i < LOADS; ++i)
        load_kv_f4(kpre[i], vpre[i], base, tid + i * NT, 0, T, C, W);
    for (int kt = 0; kt < ntiles; ++kt)
    {
        __syncthreads();  // every wave is done reading the previous tile
#pragma unroll
        for (int i = 0; i < LOADS; ++i)
        {
            const int idx = tid + i * NT, r = idx >> 4, c4 = (idx & 15) * 4;
            *reinterpret_cast<float4 *>(&ks[r * ST + c4]) = kpre[i];
            *reinterpret_cast<float4 *>(&vs[r * ST + c4]) = vpre[i];
        }
        __syncthreads();
        if (kt + 1 < ntiles)
        {
#pragma unroll
            for (int i = 0; i < LOADS; ++i)
                load_kv_f4(kpre[i], vpre[i], base, tid + i * NT, (kt + 1) * BK, T, C, W);
        }

#pragma unroll
        for (int sub = 0; sub < BK / 32; ++sub)
        {
            const int kk0 = kt * BK + 32 * sub;
            if (kk0 > qw + 31)
                continue;  // keys all above this wave's queries (wave-uniform)

            // S^T[key kk0 + row(r)][query qw + n], in log2 units.
            v16f s = zero16();
            const float *krow = &ks[(32 * sub + n) * ST + 32 * hf];
#pragma unroll
            for (int t = 0; t < 8; ++t)
            {
                const float4 kv = *reinterpret_cast<const float4 *>(krow + 4 * t);
                s = mfma32(kv.x, qreg[4 * t + 0], s);
                s = mfma32(kv.y, qreg[4 * t + 1], s);
                s = mfma32(kv.z, qreg[4 * t + 2], s);
                s = mfma32(kv.w, qreg[4 * t + 3], s);
            }
            if (kk0 + 31 > qw)
            {
                // diagonal tile: key kk0 + row > query qw + n is masked out
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    if (kk0 + mfma_row(r, hf) > qw + n)
                        s[r] = -INFINITY;
            }
            float mt = s[0];
#pragma unroll
            for (int r = 1; r < 16; ++r)
                mt = fmaxf(mt, s[r]);
            mt = fmaxf(mt, swap_halves(mt));
            const float mn = fmaxf(m, mt);
            const float corr = fast_exp2(m - mn);
            float ps = 0.f;
#pragma unroll
            for (int r = 0; r < 16; ++r)
            {
                s[r] = fast_exp2(s[r] - mn);
                ps += s[r];
            }
            ps += swap_halves(ps);
            l = l * corr + ps;
            m = mn;
            o0 *= corr;
            o1 *= corr;

            // O^T += V^T P^T: step st contracts key kk0 + row(st, hf) for this
            // half, which is exactly the key of accumulator register st.
#pragma unroll
            for (int st = 0; st < 16; ++st)
            {
                const float2 vv =
                    *reinterpret_cast<const float2 *>(&vs[(32 * sub + mfma_row(st, hf)) * ST + 2 * n]);
                o0 = mfma32(vv.x, s[st], o0);
                o1 = mfma32(vv.y, s[st], o1);
            }
        }
    }

    const int row = qw + n;
    if (row < T)
    {
        const float inv = 1.f / l;
        float *dst = y + ((long)b * T + row) * C + (long)h * D;
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

// General head_dim (1..DM): one thread per (b, h, query row), two-pass-free
// online softmax over keys 0..i, q and the output row in registers.
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
    constexpr int NW = 4, BK = 64;
    const int n_qt = (s.T + 32 * NW - 1) / (32 * NW);
    const long blocks = (long)n_qt * s.B * s.H;
    const float qscale = softmax_scale(64) * kLog2e;
    hipLaunchKernelGGL((fwd_d64_kernel<NW, BK>), dim3((unsigned)blocks), dim3(NW * 64), 0, st, y, lse,
                       qkv, s.B, s.T, s.C, s.H, qscale, n_qt);
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

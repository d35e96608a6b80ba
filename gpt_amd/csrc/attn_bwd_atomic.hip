// Causal self-attention backward for gfx950, atomic-dQ variant.
//
// The library's default head_dim-64 backward (attn_bwd.hip) is deterministic;
// this variant accumulates dQ with fp32 global atomics instead and is kept as
// the measured alternative of that design choice (gpt_hip_attn_set_path(2)).
//
// Matches the reference CPU backend (src/backend/cpu/cpu_backend.cpp:358-437)
// and replaces the reference's CUDA path (src/backend/cuda/kernels/
// attention.cu:270-577):
//   D[i]  = sum_e dO[i][e] O[i][e]
//   P_ij  = exp(q_i . k_j / sqrt(d) - lse_i)            (j <= i)
//   dS_ij = P_ij (dO_i . v_j - D_i) / sqrt(d)
//   dQ_i  = sum_j dS_ij k_j,  dK_j = sum_i dS_ij q_i,  dV_j = sum_i P_ij dO_i
// grad_x is overwritten (dQ | dK | dV in the qkv layout) and D is written.
//
// Two launches:
//   bwd_prep_kernel        D rows, and zeroes the dQ third of grad_x
//                          (attn_bwd.hip)
//   bwd_d64_atomic_kernel  one workgroup of NW = 2*QS waves owns BKV = 32*NW keys and
//                    walks the query blocks (BQ = 32*QS rows) from its diagonal
//                    to T. Each wave keeps its 32 keys' K and V as MFMA
//                    operands in registers and accumulates dK, dV in
//                    registers (written once, with plain stores, at the end).
//                    Per query block:
//                      S  = Q K^T, dP = dO V^T        (queries x keys)
//                      dV += P^T dO, dK += dS^T Q     (accumulators of S/dP
//                                                      are used directly as
//                                                      the A operand)
//                      dS -> LDS; after a barrier every wave computes one
//                      32x32 tile of dQ = dS K over all BKV keys of the
//                      workgroup and adds it to grad_x with fp32 atomics.
//                    The LDS round trip transposes dS into the A layout and
//                    reduces the NW waves' key ranges before anything touches
//                    global memory, so each workgroup issues one atomic per
//                    dQ element per query block.
#include "attn_common.h"
#include "attn_kernels.h"

#include <math.h>

namespace gpt_attn {

template <int QS>
__global__ __launch_bounds__(128 * QS) void bwd_d64_atomic_kernel(float *__restrict__ grad_x,
                                                           const float *__restrict__ lse,
                                                           const float *__restrict__ Dv,
                                                           const float *__restrict__ dy,
                                                           const float *__restrict__ qkv,
                                                           int B, int T, int C, int H,
                                                           float scale, float c2)
{
    constexpr int NW = 2 * QS, NT = NW * 64, BKV = 32 * NW, BQ = 32 * QS;
    constexpr int ST = kRowStride, DSST = BKV + 4;  // both = 4 (mod 32) words
    __shared__ __attribute__((aligned(16))) float k_lds[BKV * ST];   // keys of the workgroup
    __shared__ __attribute__((aligned(16))) float q_lds[BQ * ST];    // Q of the query block
    __shared__ __attribute__((aligned(16))) float o_lds[BQ * ST];    // dO of the query block
    __shared__ __attribute__((aligned(16))) float s_lds[BQ * DSST];  // dS (queries x keys)
    __shared__ __attribute__((aligned(16))) float l_lds[BQ];         // lse * log2(e)
    __shared__ __attribute__((aligned(16))) float d_lds[BQ];         // D

    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int n = lane & 31, hf = lane >> 5;
    const int BH = B * H;
    // Key block 0 sees every query block: lowest key blocks go first.
    const int kb = (int)(blockIdx.x / BH);
    const int bh = blockIdx.x % BH;
    const int b = bh / H, h = bh % H;
    const long W = 3L * C;
    const float *qb = qkv + (long)b * T * W + (long)h * 64;
    const float *dob = dy + (long)b * T * C + (long)h * 64;
    const float *lb = lse + (long)b * T * H + h;
    const float *db_ = Dv + (long)b * T * H + h;
    float *gq = grad_x + (long)b * T * W + (long)h * 64;
    const int kb0 = kb * BKV;
    const int kw = kb0 + 32 * w;  // first key of this wave

    // B operands of S = Q K^T and dP = dO V^T: lane (n, hf) holds
    // K[kw+n][32hf + s] and V[kw+n][32hf + s], s = 0..31.
    float kop[32], vop[32];
    {
        const int key = kw + n;
        if (key < T)
        {
            const float4 *ks = reinterpret_cast<const float4 *>(qb + (long)key * W + C + 32 * hf);
            const float4 *vs = reinterpret_cast<const float4 *>(qb + (long)key * W + 2 * C + 32 * hf);
#pragma unroll
            for (int t = 0; t < 8; ++t)
            {
                const float4 a = ks[t], v = vs[t];
                kop[4 * t + 0] = a.x;
                kop[4 * t + 1] = a.y;
                kop[4 * t + 2] = a.z;
                kop[4 * t + 3] = a.w;
                vop[4 * t + 0] = v.x;
                vop[4 * t + 1] = v.y;
                vop[4 * t + 2] = v.z;
                vop[4 * t + 3] = v.w;
            }
        }
        else
        {
#pragma unroll
            for (int s = 0; s < 32; ++s)
                kop[s] = vop[s] = 0.f;
        }
    }
    // K of all BKV keys, row-major, for the B operand of dQ = dS K.
    for (int idx = tid; idx < BKV * 16; idx += NT)
    {
        const int r = idx >> 4, c4 = (idx & 15) * 4, key = kb0 + r;
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (key < T)
            v = *reinterpret_cast<const float4 *>(qb + (long)key * W + C + c4);
        *reinterpret_cast<float4 *>(&k_lds[r * ST + c4]) = v;
    }

    v16f dk0 = zero16(), dk1 = zero16(), dv0 = zero16(), dv1 = zero16();

    for (int q0 = kb0; q0 < T; q0 += BQ)
    {
        __syncthreads();  // previous block's LDS reads are done
        for (int idx = tid; idx < BQ * 16; idx += NT)
        {
            const int r = idx >> 4, c4 = (idx & 15) * 4, row = q0 + r;
            float4 qv = make_float4(0.f, 0.f, 0.f, 0.f), ov = qv;
            if (row < T)
            {
                qv = *reinterpret_cast<const float4 *>(qb + (long)row * W + c4);
                ov = *reinterpret_cast<const float4 *>(dob + (long)row * C + c4);
            }
            *reinterpret_cast<float4 *>(&q_lds[r * ST + c4]) = qv;
            *reinterpret_cast<float4 *>(&o_lds[r * ST + c4]) = ov;
        }
        if (tid < BQ)
        {
            const int row = q0 + tid;
            l_lds[tid] = row < T ? lb[(long)row * H] * kLog2e : 0.f;
            d_lds[tid] = row < T ? db_[(long)row * H] : 0.f;
        }
        __syncthreads();

#pragma unroll
        for (int sb = 0; sb < QS; ++sb)
        {
            const int qs0 = q0 + 32 * sb;  // first query of the sub-block
            if (kw <= qs0 + 31)
            {
                // S[query qs0 + row(r)][key kw + n] and dP likewise.
                v16f s = zero16(), dp = zero16();
                const float *qr = &q_lds[(32 * sb + n) * ST + 32 * hf];
                const float *orow = &o_lds[(32 * sb + n) * ST + 32 * hf];
#pragma unroll
                for (int t = 0; t < 8; ++t)
                {
                    const float4 qv = *reinterpret_cast<const float4 *>(qr + 4 * t);
                    const float4 ov = *reinterpret_cast<const float4 *>(orow + 4 * t);
                    s = mfma32(qv.x, kop[4 * t + 0], s);
                    dp = mfma32(ov.x, vop[4 * t + 0], dp);
                    s = mfma32(qv.y, kop[4 * t + 1], s);
                    dp = mfma32(ov.y, vop[4 * t + 1], dp);
                    s = mfma32(qv.z, kop[4 * t + 2], s);
                    dp = mfma32(ov.z, vop[4 * t + 2], dp);
                    s = mfma32(qv.w, kop[4 * t + 3], s);
                    dp = mfma32(ov.w, vop[4 * t + 3], dp);
                }
                const bool diag = kw + 31 > qs0;
#pragma unroll
                for (int g = 0; g < 4; ++g)
                {
                    const float4 lv = *reinterpret_cast<const float4 *>(&l_lds[32 * sb + 8 * g + 4 * hf]);
                    const float4 dv = *reinterpret_cast<const float4 *>(&d_lds[32 * sb + 8 * g + 4 * hf]);
                    const float lj[4] = {lv.x, lv.y, lv.z, lv.w};
                    const float dj[4] = {dv.x, dv.y, dv.z, dv.w};
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                    {
                        const int r = 4 * g + j;
                        float p = fast_exp2(s[r] * c2 - lj[j]);
                        if (diag && kw + n > qs0 + 8 * g + 4 * hf + j)
                            p = 0.f;
                        s[r] = p;
                        dp[r] = p * (dp[r] - dj[j]);  // dS without the 1/sqrt(d)
                    }
                }
                // dV += P^T dO and dK += dS^T Q; step st contracts query
                // qs0 + row(st, hf), the query of accumulator register st.
#pragma unroll
                for (int st = 0; st < 16; ++st)
                {
                    const int rr = 32 * sb + mfma_row(st, hf);
                    const float2 g = *reinterpret_cast<const float2 *>(&o_lds[rr * ST + 2 * n]);
                    const float2 qq = *reinterpret_cast<const float2 *>(&q_lds[rr * ST + 2 * n]);
                    dv0 = mfma32(s[st], g.x, dv0);
                    dv1 = mfma32(s[st], g.y, dv1);
                    dk0 = mfma32(dp[st], qq.x, dk0);
                    dk1 = mfma32(dp[st], qq.y, dk1);
                }
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    s_lds[(32 * sb + mfma_row(r, hf)) * DSST + 32 * w + n] = dp[r];
            }
            else
            {
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    s_lds[(32 * sb + mfma_row(r, hf)) * DSST + 32 * w + n] = 0.f;
            }
        }
        __syncthreads();

        // dQ tile (query sub-block w/2, dims 32*(w%2) .. +31) over all BKV keys.
        {
            const int sbq = w >> 1, dblk = w & 1;
            v16f acc = zero16();
            const float *arow = &s_lds[(32 * sbq + n) * DSST + hf * (BKV / 2)];
            const float *bcol = &k_lds[(hf * (BKV / 2)) * ST + 32 * dblk + n];
#pragma unroll
            for (int t = 0; t < BKV / 8; ++t)
            {
                const float4 a = *reinterpret_cast<const float4 *>(arow + 4 * t);
                acc = mfma32(a.x, bcol[(4 * t + 0) * ST], acc);
                acc = mfma32(a.y, bcol[(4 * t + 1) * ST], acc);
                acc = mfma32(a.z, bcol[(4 * t + 2) * ST], acc);
                acc = mfma32(a.w, bcol[(4 * t + 3) * ST], acc);
            }
#pragma unroll
            for (int r = 0; r < 16; ++r)
            {
                const int row = q0 + 32 * sbq + mfma_row(r, hf);
                if (row < T)
                    unsafeAtomicAdd(&gq[(long)row * W + 32 * dblk + n], acc[r] * scale);
            }
        }
    }

    // dK (scaled) and dV rows of this wave's keys: register r holds key
    // kw + row(r, hf), dims 2n and 2n + 1.
#pragma unroll
    for (int r = 0; r < 16; ++r)
    {
        const int key = kw + mfma_row(r, hf);
        if (key < T)
        {
            float *dst = gq + (long)key * W + 2 * n;
            *reinterpret_cast<float2 *>(dst + C) = make_float2(dk0[r] * scale, dk1[r] * scale);
            *reinterpret_cast<float2 *>(dst + 2 * C) = make_float2(dv0[r], dv1[r]);
        }
    }
}

static float softmax_scale(int d) { return 1.0f / sqrtf((float)d); }

hipError_t launch_bwd_d64_atomic(float *grad_x, float *D, const float *lse, const float *dy, const float *y,
                                 const float *qkv, const Shape &s, hipStream_t st)
{
    constexpr int QS = 2, BKV = 64 * QS;
    timer_begin(kKindOther, st);
    hipError_t e = launch_bwd_prep(grad_x, D, dy, y, s, st, 1);
    if (e != hipSuccess)
    {
        timer_end(st);
        return e;
    }
    const int n_kb = (s.T + BKV - 1) / BKV;
    const float scale = softmax_scale(64);
    hipLaunchKernelGGL((bwd_d64_atomic_kernel<QS>), dim3((unsigned)((long)n_kb * s.B * s.H)), dim3(128 * QS), 0,
                       st, grad_x, lse, D, dy, qkv, s.B, s.T, s.C, s.H, scale, scale * kLog2e);
    timer_end(st);
    return hipGetLastError();
}

}  // namespace gpt_attn

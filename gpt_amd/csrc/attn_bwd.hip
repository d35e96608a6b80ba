// Causal self-attention backward for gfx950.
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
// head_dim 64 path: deterministic, three launches, no atomics, no memset.
// Work unit = one 32-query block i x one 32-key block j with j <= i.
//   bwd_rowdot_d64_kernel  D rows; one wave per token row, 16 lanes per head.
//   bwd_dkdv_d64_kernel    one workgroup per (b, h, key block j); its NW waves
//                          split the query blocks i >= j (wave w takes
//                          j + w, j + w + NW, ...). Per unit, on
//                          v_mfma_f32_32x32x2_f32:
//                            S  = Q K^T, dP = dO V^T   (queries x keys)
//                            P = 2^(S c - L), dS = P (dP - D)
//                            dV += P^T dO, dK += dS^T Q (the S / dP
//                              accumulators are the A operands as they are)
//                          and the dS tile is stored to a workspace. The NW
//                          partial dK, dV are summed through LDS in a fixed
//                          order and written once with plain stores.
//   bwd_dq_d64_kernel      one wave per (b, h, heavy/light query-block pair):
//                          dQ_i = sum_{j<=i} dS_ij K_j from the workspace,
//                          written once with plain stores.
// Materialising dS costs 4 KiB of workspace per unit (28 MiB per layer at
// B=16, T=256, H=12), written and read once; in exchange no dQ element is
// accumulated by more than one wave, the result is bitwise reproducible, and
// the dK/dV and dQ work both split into units small enough to balance the
// causal triangle over 256 CUs. The atomic alternative is attn_bwd_atomic.hip.
#include "attn_common.h"
#include "attn_kernels.h"

#include <math.h>

namespace gpt_attn {

// D[b,t,h] = sum_e dO*O over the head's d columns, any head_dim; optionally
// zero the dQ third of grad_x for the same (b, t, h) slice (used by the atomic
// variant). One thread per (b, t, h).
__global__ __launch_bounds__(256) void bwd_prep_kernel(float *__restrict__ grad_x,
                                                       float *__restrict__ Dout,
                                                       const float *__restrict__ dy,
                                                       const float *__restrict__ y,
                                                       int B, int T, int C, int H, int d,
                                                       int zero_dq, int vec4)
{
    const long gid = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= (long)B * T * H)
        return;
    const int h = (int)(gid % H);
    const long bt = gid / H;
    const long off = bt * C + (long)h * d;
    float acc = 0.f;
    if (vec4)
    {
        const float4 *a = reinterpret_cast<const float4 *>(dy + off);
        const float4 *o = reinterpret_cast<const float4 *>(y + off);
        for (int e = 0; e < d / 4; ++e)
        {
            const float4 u = a[e], v = o[e];
            acc += u.x * v.x;
            acc += u.y * v.y;
            acc += u.z * v.z;
            acc += u.w * v.w;
        }
    }
    else
    {
        for (int e = 0; e < d; ++e)
            acc += dy[off + e] * y[off + e];
    }
    Dout[gid] = acc;
    if (zero_dq)
    {
        float *dq = grad_x + bt * 3L * C + (long)h * d;
        if (vec4)
        {
            float4 *z = reinterpret_cast<float4 *>(dq);
            for (int e = 0; e < d / 4; ++e)
                z[e] = make_float4(0.f, 0.f, 0.f, 0.f);
        }
        else
        {
            for (int e = 0; e < d; ++e)
                dq[e] = 0.f;
        }
    }
}

// D rows for head_dim 64: one wave per token row (all H heads), lane l reads
// float4s l, l + 64, ... of the row; the 16 lanes of one head sum their
// products in 4 butterfly steps.
__global__ __launch_bounds__(256) void bwd_rowdot_d64_kernel(float *__restrict__ Dout,
                                                             const float *__restrict__ dy,
                                                             const float *__restrict__ y,
                                                             long rows, int H)
{
    const long row = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows)
        return;
    const int lane = threadIdx.x & 63;
    const long C = 64L * H;
    const float4 *a = reinterpret_cast<const float4 *>(dy + row * C);
    const float4 *o = reinterpret_cast<const float4 *>(y + row * C);
    for (int f = lane; f < 16 * H; f += 64)  // uniform within each 16-lane group
    {
        const float4 u = a[f], v = o[f];
        float s = u.x * v.x + u.y * v.y + u.z * v.z + u.w * v.w;
        s += __shfl_xor(s, 8, 16);
        s += __shfl_xor(s, 4, 16);
        s += __shfl_xor(s, 2, 16);
        s += __shfl_xor(s, 1, 16);
        if ((lane & 15) == 0)
            Dout[row * H + (f >> 4)] = s;
    }
}

// Offset (floats) of dS tile (i, j), j <= i, inside one (b, h)'s workspace.
__device__ __forceinline__ long ds_tile(int i, int j) { return ((long)i * (i + 1) / 2 + j) * 1024; }

// Sum one 64-register-per-lane partial (v0..v3, 16 registers each) over the
// NW = 4 waves of the workgroup in the fixed order (w0 + w1) + (w2 + w3);
// wave 0 ends with the total. `red` holds two [64][64] partials.
__device__ __forceinline__ void reduce4(v16f &v0, v16f &v1, v16f &v2, v16f &v3, float (*red)[64][64], int w,
                                        int lane)
{
    if (w & 1)
    {
#pragma unroll
        for (int r = 0; r < 16; ++r)
        {
            red[w >> 1][r][lane] = v0[r];
            red[w >> 1][16 + r][lane] = v1[r];
            red[w >> 1][32 + r][lane] = v2[r];
            red[w >> 1][48 + r][lane] = v3[r];
        }
    }
    __syncthreads();
    if (!(w & 1))
    {
#pragma unroll
        for (int r = 0; r < 16; ++r)
        {
            v0[r] += red[w >> 1][r][lane];
            v1[r] += red[w >> 1][16 + r][lane];
            v2[r] += red[w >> 1][32 + r][lane];
            v3[r] += red[w >> 1][48 + r][lane];
        }
    }
    __syncthreads();
    if (w == 2)
    {
#pragma unroll
        for (int r = 0; r < 16; ++r)
        {
            red[0][r][lane] = v0[r];
            red[0][16 + r][lane] = v1[r];
            red[0][32 + r][lane] = v2[r];
            red[0][48 + r][lane] = v3[r];
        }
    }
    __syncthreads();
    if (w == 0)
    {
#pragma unroll
        for (int r = 0; r < 16; ++r)
        {
            v0[r] += red[0][r][lane];
            v1[r] += red[0][16 + r][lane];
            v2[r] += red[0][32 + r][lane];
            v3[r] += red[0][48 + r][lane];
        }
    }
}

// dK, dV and the dS tiles. One workgroup per (b, h, key-block pair
// (p, n - 1 - p)): key block j has n - j units (query blocks j .. n - 1), so
// each pair carries n + 1 units. The pair's two key blocks are done one after
// the other; for each, K and V are staged once in LDS (row stride
// kRowStride) and the 4 waves split its query blocks round-robin (rotated per
// workgroup), accumulating partial dK / dV in registers that are summed
// through LDS in a fixed order and stored by wave 0.
//
// Per unit (query block i) a wave runs two MFMA phases:
//   phase 1  S = Q K^T, dP = dO V^T: 8 chunks of 4 + 4 MFMAs; A operands
//            Q / dO[q0 + n][32 hf + 4c ..] (one float4 each per chunk, from
//            L2), B operands K / V from LDS
//   phase 2  dV += P^T dO, dK += dS^T Q: 8 chunks of 2 steps x 4 MFMAs; B
//            operands dO / Q[q0 + row(st, hf)][2n, 2n + 1] (float2, from L2)
// Every global operand is loaded one chunk ahead, and the first chunk of each
// phase one phase ahead: phase 2's while P and dS are formed, the next unit's
// phase 1 (and its lse / D rows) during this unit's phase 2. All row and block
// offsets are wave-uniform and go in the buffer loads' scalar offset; rows past
// T read as zeros through the buffer range check. 3 waves per SIMD keep all
// workgroups of a B=16, T=256, H=12 call resident at once.
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3))) void bwd_dkdv_d64_kernel(
    float *__restrict__ grad_x, float *__restrict__ dsw, const float *__restrict__ lse,
    const float *__restrict__ Dv, const float *__restrict__ dy, const float *__restrict__ qkv, int T, int C, int H,
    int bh0, int BHc, int n_qb, float c2, float scale)
{
    constexpr int NW = 4, ST = kRowStride;
    const int tid = threadIdx.x, lane = tid & 63, w = wave_id();
    const int n = lane & 31, hf = lane >> 5;
    const int pr = (int)(blockIdx.x / BHc);
    const int bhl = (int)(blockIdx.x % BHc), bh = bh0 + bhl;
    const int b = bh / H, h = bh % H;
    const uint32_t Wb = 12u * (uint32_t)C, Cb = 4u * (uint32_t)C, Hb = 4u * (uint32_t)H;
    const rsrc_t rq = make_rsrc(qkv + (long)b * T * 3L * C + (long)h * 64,
                                (uint32_t)(((long)T * 3 * C - (long)h * 64) * 4));
    const rsrc_t ro = make_rsrc(dy + (long)b * T * C + (long)h * 64, (uint32_t)(((long)T * C - (long)h * 64) * 4));
    const rsrc_t rl = make_rsrc(lse + (long)b * T * H + h, (uint32_t)(((long)T * H - h) * 4));
    const rsrc_t rd = make_rsrc(Dv + (long)b * T * H + h, (uint32_t)(((long)T * H - h) * 4));
    float *ws = dsw + (long)bhl * ((long)n_qb * (n_qb + 1) / 2) * 1024;
    float *gx = grad_x + (long)b * T * 3L * C + (long)h * 64;

    // lane-dependent parts of the operand offsets (bytes)
    const uint32_t q1_lane = (uint32_t)n * Wb + 128u * hf;      // phase 1: Q[n][32 hf ..]
    const uint32_t o1_lane = (uint32_t)n * Cb + 128u * hf;      // phase 1: dO[n][32 hf ..]
    const uint32_t q2_lane = 4u * hf * Wb + 8u * (uint32_t)n;   // phase 2: Q[4 hf + ..][2n ..]
    const uint32_t o2_lane = 4u * hf * Cb + 8u * (uint32_t)n;   // phase 2: dO[4 hf + ..][2n ..]
    const uint32_t l_lane = (uint32_t)n * Hb;                    // lse / D row n

    __shared__ __attribute__((aligned(16))) float kv_lds[2][32 * ST];  // K, V of the key block
    __shared__ __attribute__((aligned(16))) float ld_lds[NW][2][32];   // per wave: L * log2(e), D
    __shared__ float red[2][64][64];

    for (int it = 0; it < 2; ++it)
    {
        const int j = it == 0 ? pr : n_qb - 1 - pr;
        if (it == 1 && j == pr)
            break;  // odd n_qb: the middle key block has no partner
        const int k0 = 32 * j;
        // wave w takes query blocks i = j + u with (u + rot) % NW == w
        const int rot = (pr + (it == 0 ? 0 : n_qb - pr)) % NW;
        const int i_first = j + (w - rot + NW) % NW;

        // first unit's phase-1 chunk 0 and lse / D rows, in flight while K / V
        // are staged
        float4 qa[2], oa[2];
        float lrow, drow;
        {
            const uint32_t rq0 = i_first < n_qb ? 32u * (uint32_t)i_first * Wb : kNoBlock;
            const uint32_t ro0 = i_first < n_qb ? 32u * (uint32_t)i_first * Cb : kNoBlock;
            const uint32_t rl0 = i_first < n_qb ? 32u * (uint32_t)i_first * Hb : kNoBlock;
            qa[0] = bload4s(rq, q1_lane, rq0);
            oa[0] = bload4s(ro, o1_lane, ro0);
            lrow = bload1s(rl, l_lane, rl0);
            drow = bload1s(rd, l_lane, rl0);
        }

        __syncthreads();  // the previous key block's LDS reads are done
#pragma unroll
        for (int u = 0; u < 4; ++u)
        {
            const int idx = tid + 256 * u, which = idx >> 9, r = (idx >> 4) & 31, c4 = idx & 15;
            const float4 v = bload4s(rq, (uint32_t)r * Wb + (1u + which) * Cb + 16u * c4, (uint32_t)k0 * Wb);
            *reinterpret_cast<float4 *>(&kv_lds[which][r * ST + 4 * c4]) = v;
        }
        __syncthreads();

        const float *kr = &kv_lds[0][n * ST + 32 * hf];
        const float *vr = &kv_lds[1][n * ST + 32 * hf];
        v16f dk0 = zero16(), dk1 = zero16(), dv0 = zero16(), dv1 = zero16();
        for (int i = i_first; i < n_qb; i += NW)
        {
            const int q0 = 32 * i;
            const bool more = i + NW < n_qb;
            const uint32_t rqn = more ? 32u * (uint32_t)(i + NW) * Wb : kNoBlock;
            const uint32_t ron = more ? 32u * (uint32_t)(i + NW) * Cb : kNoBlock;
            const uint32_t rln = more ? 32u * (uint32_t)(i + NW) * Hb : kNoBlock;
            if (hf == 0)
            {
                ld_lds[w][0][n] = lrow * kLog2e;
                ld_lds[w][1][n] = drow;
            }

            // phase 1: S[query q0 + row(r)][key k0 + n], dP likewise
            v16f s = zero16(), dp = zero16();
#pragma unroll
            for (int c = 0; c < 8; ++c)
            {
                if (c < 7)
                {
                    qa[(c + 1) & 1] = bload4s(rq, q1_lane + 16u * (c + 1), (uint32_t)q0 * Wb);
                    oa[(c + 1) & 1] = bload4s(ro, o1_lane + 16u * (c + 1), (uint32_t)q0 * Cb);
                }
                __builtin_amdgcn_sched_barrier(0);
                const float4 q4 = qa[c & 1], o4 = oa[c & 1];
                const float4 kb = *reinterpret_cast<const float4 *>(kr + 4 * c);
                const float4 vb = *reinterpret_cast<const float4 *>(vr + 4 * c);
                s = mfma32(q4.x, kb.x, s);
                dp = mfma32(o4.x, vb.x, dp);
                s = mfma32(q4.y, kb.y, s);
                dp = mfma32(o4.y, vb.y, dp);
                s = mfma32(q4.z, kb.z, s);
                dp = mfma32(o4.z, vb.z, dp);
                s = mfma32(q4.w, kb.w, s);
                dp = mfma32(o4.w, vb.w, dp);
                __builtin_amdgcn_sched_barrier(0);
            }

            // phase 2's chunk 0 (query rows 4 hf + {0, 1}), in flight while P and
            // dS are formed
            float2 gb[2][2], qb[2][2];
#pragma unroll
            for (int e = 0; e < 2; ++e)
            {
                gb[0][e] = bload2s(ro, o2_lane, (uint32_t)(q0 + e) * Cb);
                qb[0][e] = bload2s(rq, q2_lane, (uint32_t)(q0 + e) * Wb);
            }
            wave_lds_sync();
            __builtin_amdgcn_sched_barrier(0);
            // P and dS (without the 1/sqrt(d)); zero where key > query or the
            // query row is past T.
#pragma unroll
            for (int g = 0; g < 4; ++g)
            {
                const float4 l4 = *reinterpret_cast<const float4 *>(&ld_lds[w][0][8 * g + 4 * hf]);
                const float4 d4 = *reinterpret_cast<const float4 *>(&ld_lds[w][1][8 * g + 4 * hf]);
                const float lj[4] = {l4.x, l4.y, l4.z, l4.w};
                const float dj[4] = {d4.x, d4.y, d4.z, d4.w};
#pragma unroll
                for (int jj = 0; jj < 4; ++jj)
                {
                    const int r = 4 * g + jj;
                    const int qrow = q0 + 8 * g + 4 * hf + jj;  // = q0 + row(r, hf)
                    const bool keep = (k0 + n <= qrow) && (qrow < T);
                    const float p = fast_exp2(s[r] * c2 - lj[jj]);
                    s[r] = keep ? p : 0.f;
                    dp[r] = keep ? p * (dp[r] - dj[jj]) : 0.f;
                }
            }
            // dS tile, query-major (row = query, column = key)
            {
                float *tile = ws + ds_tile(i, j) + (4 * hf) * 32 + n;
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    tile[(8 * (r >> 2) + (r & 3)) * 32] = dp[r];
            }
            __builtin_amdgcn_sched_barrier(0);

            // phase 2: step st contracts query q0 + row(st, hf), the query of
            // accumulator register st; chunk c = steps 2c, 2c + 1
#pragma unroll
            for (int c = 0; c < 8; ++c)
            {
                if (c < 7)
                {
#pragma unroll
                    for (int e = 0; e < 2; ++e)
                    {
                        const int st = 2 * (c + 1) + e;
                        const uint32_t row = (uint32_t)(q0 + 8 * (st >> 2) + (st & 3));
                        gb[(c + 1) & 1][e] = bload2s(ro, o2_lane, row * Cb);
                        qb[(c + 1) & 1][e] = bload2s(rq, q2_lane, row * Wb);
                    }
                }
                if (c == 3)
                {
                    // next unit's phase-1 chunk 0 and lse / D rows
                    qa[0] = bload4s(rq, q1_lane, rqn);
                    oa[0] = bload4s(ro, o1_lane, ron);
                    lrow = bload1s(rl, l_lane, rln);
                    drow = bload1s(rd, l_lane, rln);
                }
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int e = 0; e < 2; ++e)
                {
                    const int st = 2 * c + e;
                    const float2 g2 = gb[c & 1][e], q2 = qb[c & 1][e];
                    dv0 = mfma32(s[st], g2.x, dv0);
                    dv1 = mfma32(s[st], g2.y, dv1);
                    dk0 = mfma32(dp[st], q2.x, dk0);
                    dk1 = mfma32(dp[st], q2.y, dk1);
                }
                __builtin_amdgcn_sched_barrier(0);
            }
            wave_lds_sync();
        }

        reduce4(dk0, dk1, dv0, dv1, red, w, lane);
        if (w == 0)
        {
            // register r of lane (n, hf): key k0 + row(r, hf), dims 2n, 2n + 1
#pragma unroll
            for (int r = 0; r < 16; ++r)
            {
                const int key = k0 + mfma_row(r, hf);
                if (key < T)
                {
                    float *dst = gx + (long)key * 3 * C + 2 * n;
                    *reinterpret_cast<float2 *>(dst + C) = make_float2(dk0[r] * scale, dk1[r] * scale);
                    *reinterpret_cast<float2 *>(dst + 2 * C) = make_float2(dv0[r], dv1[r]);
                }
            }
        }
    }
}

// dQ_i = scale * sum_{j<=i} dS_ij K_j. One WAVE per (b, h, query-block pair
// (n - 1 - p, p)): n + 1 units, run as one stream (the heavy block's key
// blocks 0..n-1-p, then the light block's 0..p), so no wave ever waits for
// another and nothing is merged. A unit's operands (the dS tile and the K
// block, 12 KiB) are loaded one unit ahead into a second register set while
// the current unit's 32 MFMAs run. Workgroups hold 4 waves = 4 pairs of one
// (b, h), ordered (chunk of pairs)-major with (b, h) fastest, the same
// (b, h) -> XCD mapping as the dK/dV kernel, so a (b, h)'s dS tiles are read
// from the L2 they were written to.
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void bwd_dq_d64_kernel(float *__restrict__ grad_x,
                                                         const float *__restrict__ dsw,
                                                         const float *__restrict__ qkv,
                                                         int T, int C, int H, int bh0, int BHc, int n_qb,
                                                         float scale)
{
    const int lane = threadIdx.x & 63, w = wave_id();
    const int n = lane & 31, hf = lane >> 5;
    const int chunk = (int)(blockIdx.x / BHc);
    const int bhl = (int)(blockIdx.x % BHc), bh = bh0 + bhl;
    const int b = bh / H, h = bh % H;
    const int pr = 4 * chunk + w;  // this wave's pair
    const int n_pairs = (n_qb + 1) / 2;
    if (pr >= n_pairs)
        return;
    const int qa = n_qb - 1 - pr;
    const bool two = qa != pr;
    const uint32_t Wb = 12u * (uint32_t)C;
    const rsrc_t rk = make_rsrc(qkv + (long)b * T * 3L * C + C + (long)h * 64,
                                (uint32_t)(((long)T * 3 * C - C - (long)h * 64) * 4));
    const long tiles = (long)n_qb * (n_qb + 1) / 2;
    const rsrc_t rw = make_rsrc(dsw + (long)bhl * tiles * 1024, (uint32_t)(tiles * 4096));
    float *gx = grad_x + (long)b * T * 3L * C + (long)h * 64;
    // lane parts of the offsets: dS[n][16 hf ..] of a tile, K[16 hf + t][2n ..] of a block
    const uint32_t w_lane = (uint32_t)n * 128u + 64u * hf;
    const uint32_t k_lane = 16u * hf * Wb + 8u * (uint32_t)n;

    // unit u of the stream: query block i(u), key block j(u)
    const int cnt0 = qa + 1, total = cnt0 + (two ? pr + 1 : 0);
    auto tile_off = [&](int u) -> uint32_t {
        if (u >= total)
            return kNoBlock;
        const int i = u < cnt0 ? qa : pr, j = u < cnt0 ? u : u - cnt0;
        return (uint32_t)(((long)i * (i + 1) / 2 + j) * 4096);
    };
    auto key_off = [&](int u) -> uint32_t {
        if (u >= total)
            return kNoBlock;
        return 32u * (uint32_t)(u < cnt0 ? u : u - cnt0) * Wb;
    };

    // Two operand sets, A and B: unit u uses set u % 2; the next unit's set
    // is loaded while this unit's MFMAs run. (Deeper prefetch does not pay at
    // B=16, T=256: the kernel is bound by the dS / K reads, not by latency.)
    float4 dsA[4], dsB[4];   // A operand dS[n][16 hf + t], t = 0..15
    float2 kkA[16], kkB[16]; // B operand K[32j + 16 hf + t][2n, 2n + 1]
#define DQ_LOAD(DS, KK, u)                                                        \
    do                                                                            \
    {                                                                             \
        const uint32_t to_ = tile_off(u), ko_ = key_off(u);                       \
        _Pragma("unroll") for (int e = 0; e < 4; ++e) DS[e] = bload4s(rw, w_lane + 16u * e, to_); \
        _Pragma("unroll") for (int t = 0; t < 16; ++t) KK[t] = bload2s(rk, k_lane, ko_ + (uint32_t)t * Wb); \
    } while (0)
#define DQ_MFMA(DS, KK)                                                           \
    do                                                                            \
    {                                                                             \
        _Pragma("unroll") for (int e = 0; e < 4; ++e)                             \
        {                                                                         \
            a0 = mfma32(DS[e].x, KK[4 * e + 0].x, a0);                            \
            a1 = mfma32(DS[e].x, KK[4 * e + 0].y, a1);                            \
            a0 = mfma32(DS[e].y, KK[4 * e + 1].x, a0);                            \
            a1 = mfma32(DS[e].y, KK[4 * e + 1].y, a1);                            \
            a0 = mfma32(DS[e].z, KK[4 * e + 2].x, a0);                            \
            a1 = mfma32(DS[e].z, KK[4 * e + 2].y, a1);                            \
            a0 = mfma32(DS[e].w, KK[4 * e + 3].x, a0);                            \
            a1 = mfma32(DS[e].w, KK[4 * e + 3].y, a1);                            \
        }                                                                         \
    } while (0)
    v16f a0 = zero16(), a1 = zero16();
    // last unit of a query block: register r of lane (n, hf) holds
    // dQ[32 i + row(r, hf)][2n, 2n + 1]
    auto flush = [&](int u) {
        if (u == cnt0 - 1 || u == total - 1)
        {
            const int i = u < cnt0 ? qa : pr;
#pragma unroll
            for (int r = 0; r < 16; ++r)
            {
                const int row = 32 * i + mfma_row(r, hf);
                if (row < T)
                    *reinterpret_cast<float2 *>(gx + (long)row * 3 * C + 2 * n) =
                        make_float2(a0[r] * scale, a1[r] * scale);
            }
            a0 = zero16();
            a1 = zero16();
        }
    };

    DQ_LOAD(dsA, kkA, 0);
    for (int u = 0; u < total; u += 2)
    {
        DQ_LOAD(dsB, kkB, u + 1);
        __builtin_amdgcn_sched_barrier(0);
        DQ_MFMA(dsA, kkA);
        __builtin_amdgcn_sched_barrier(0);
        flush(u);
        if (u + 1 >= total)
            break;
        DQ_LOAD(dsA, kkA, u + 2);
        __builtin_amdgcn_sched_barrier(0);
        DQ_MFMA(dsB, kkB);
        __builtin_amdgcn_sched_barrier(0);
        flush(u + 1);
    }
#undef DQ_LOAD
#undef DQ_MFMA
}

// General head_dim: dQ rows, one thread per (b, h, query i), keys j <= i.
template <int DM>
__global__ __launch_bounds__(128) void bwd_dq_general_kernel(float *__restrict__ grad_x,
                                                             const float *__restrict__ lse,
                                                             const float *__restrict__ Dv,
                                                             const float *__restrict__ dy,
                                                             const float *__restrict__ qkv,
                                                             int B, int T, int C, int H, int d,
                                                             float scale, float c2)
{
    const long gid = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= (long)B * H * T)
        return;
    const int i = (int)(gid % T);
    const long bh = gid / T;
    const int h = (int)(bh % H), b = (int)(bh / H);
    const long W = 3L * C;
    const float *base = qkv + (long)b * T * W + (long)h * d;
    const float *g = dy + ((long)b * T + i) * C + (long)h * d;
    const float Li = lse[((long)b * T + i) * H + h] * kLog2e;
    const float Di = Dv[((long)b * T + i) * H + h];
    float q[DM], go[DM], acc[DM];
#pragma unroll
    for (int e = 0; e < DM; ++e)
    {
        q[e] = e < d ? base[(long)i * W + e] : 0.f;
        go[e] = e < d ? g[e] : 0.f;
        acc[e] = 0.f;
    }
    for (int j = 0; j <= i; ++j)
    {
        const float *kr = base + (long)j * W + C;
        const float *vr = base + (long)j * W + 2L * C;
        float s = 0.f, dp = 0.f;
#pragma unroll
        for (int e = 0; e < DM; ++e)
            if (e < d)
            {
                s += q[e] * kr[e];
                dp += go[e] * vr[e];
            }
        const float p = fast_exp2(s * c2 - Li);
        const float ds = p * (dp - Di) * scale;
#pragma unroll
        for (int e = 0; e < DM; ++e)
            if (e < d)
                acc[e] += ds * kr[e];
    }
    float *dst = grad_x + ((long)b * T + i) * W + (long)h * d;
#pragma unroll
    for (int e = 0; e < DM; ++e)
        if (e < d)
            dst[e] = acc[e];
}

// General head_dim: dK and dV rows, one thread per (b, h, key j), queries i >= j.
template <int DM>
__global__ __launch_bounds__(128) void bwd_dkdv_general_kernel(float *__restrict__ grad_x,
                                                               const float *__restrict__ lse,
                                                               const float *__restrict__ Dv,
                                                               const float *__restrict__ dy,
                                                               const float *__restrict__ qkv,
                                                               int B, int T, int C, int H, int d,
                                                               float scale, float c2)
{
    const long gid = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= (long)B * H * T)
        return;
    const int j = (int)(gid % T);
    const long bh = gid / T;
    const int h = (int)(bh % H), b = (int)(bh / H);
    const long W = 3L * C;
    const float *base = qkv + (long)b * T * W + (long)h * d;
    float k[DM], v[DM], dk[DM], dv[DM];
#pragma unroll
    for (int e = 0; e < DM; ++e)
    {
        k[e] = e < d ? base[(long)j * W + C + e] : 0.f;
        v[e] = e < d ? base[(long)j * W + 2L * C + e] : 0.f;
        dk[e] = dv[e] = 0.f;
    }
    for (int i = j; i < T; ++i)
    {
        const float *qr = base + (long)i * W;
        const float *g = dy + ((long)b * T + i) * C + (long)h * d;
        const float Li = lse[((long)b * T + i) * H + h] * kLog2e;
        const float Di = Dv[((long)b * T + i) * H + h];
        float s = 0.f, dp = 0.f;
#pragma unroll
        for (int e = 0; e < DM; ++e)
            if (e < d)
            {
                s += qr[e] * k[e];
                dp += g[e] * v[e];
            }
        const float p = fast_exp2(s * c2 - Li);
        const float ds = p * (dp - Di) * scale;
#pragma unroll
        for (int e = 0; e < DM; ++e)
            if (e < d)
            {
                dk[e] += ds * qr[e];
                dv[e] += p * g[e];
            }
    }
    float *dst = grad_x + ((long)b * T + j) * W + (long)h * d;
#pragma unroll
    for (int e = 0; e < DM; ++e)
        if (e < d)
        {
            dst[C + e] = dk[e];
            dst[2L * C + e] = dv[e];
        }
}

static float softmax_scale(int d) { return 1.0f / sqrtf((float)d); }

hipError_t launch_bwd_prep(float *grad_x, float *D, const float *dy, const float *y, const Shape &s,
                           hipStream_t st, int zero_dq)
{
    const long items = (long)s.B * s.T * s.H;
    const int vec4 = (s.d % 4 == 0) && ((reinterpret_cast<uintptr_t>(dy) | reinterpret_cast<uintptr_t>(y) |
                                         reinterpret_cast<uintptr_t>(grad_x)) %
                                            16 ==
                                        0);
    hipLaunchKernelGGL(bwd_prep_kernel, dim3((unsigned)((items + 255) / 256)), dim3(256), 0, st, grad_x, D,
                       dy, y, s.B, s.T, s.C, s.H, s.d, zero_dq, vec4);
    return hipGetLastError();
}

size_t bwd_d64_workspace_bytes(const Shape &s, int *bh_per_chunk)
{
    const long n_qb = (s.T + 31) / 32;
    const size_t per_bh = (size_t)(n_qb * (n_qb + 1) / 2) * 4096;
    const long BH = (long)s.B * s.H;
    long chunk = (long)(kWorkspaceCap / per_bh);
    chunk = chunk < 1 ? 1 : (chunk > BH ? BH : chunk);
    if (bh_per_chunk)
        *bh_per_chunk = (int)chunk;
    return per_bh * (size_t)chunk;
}

hipError_t launch_bwd_d64(float *grad_x, float *D, const float *lse, const float *dy, const float *y,
                          const float *qkv, float *ws, int bh_per_chunk, const Shape &s, hipStream_t st)
{
    const long rows = (long)s.B * s.T;
    timer_begin(kKindRowdot, st);
    hipLaunchKernelGGL(bwd_rowdot_d64_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, st, D, dy, y,
                       rows, s.H);
    timer_end(st);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess)
        return e;
    const int n_qb = (s.T + 31) / 32;
    const int BH = s.B * s.H;
    const float scale = softmax_scale(64);
    for (int bh0 = 0; bh0 < BH; bh0 += bh_per_chunk)
    {
        const int cnt = BH - bh0 < bh_per_chunk ? BH - bh0 : bh_per_chunk;
        const unsigned blocks = (unsigned)((long)((n_qb + 1) / 2) * cnt);  // heavy/light pairs
        timer_begin(kKindDkdv, st);
        hipLaunchKernelGGL(bwd_dkdv_d64_kernel, dim3(blocks), dim3(256), 0, st, grad_x, ws, lse, D, dy, qkv, s.T,
                           s.C, s.H, bh0, cnt, n_qb, scale * kLog2e, scale);
        timer_end(st);
        const unsigned dq_blocks = (unsigned)((long)((n_qb + 1) / 2 + 3) / 4 * cnt);  // 4 pairs per workgroup
        timer_begin(kKindDq, st);
        hipLaunchKernelGGL(bwd_dq_d64_kernel, dim3(dq_blocks), dim3(256), 0, st, grad_x, ws, qkv, s.T, s.C, s.H,
                           bh0, cnt, n_qb, scale);
        timer_end(st);
        e = hipGetLastError();
        if (e != hipSuccess)
            return e;
    }
    return hipSuccess;
}

template <int DM>
static void launch_bwd_general_dm(float *grad_x, const float *lse, const float *D, const float *dy,
                                  const float *qkv, const Shape &s, hipStream_t st)
{
    const long rows = (long)s.B * s.H * s.T;
    const dim3 grid((unsigned)((rows + 127) / 128)), block(128);
    const float scale = softmax_scale(s.d);
    hipLaunchKernelGGL(bwd_dq_general_kernel<DM>, grid, block, 0, st, grad_x, lse, D, dy, qkv, s.B, s.T, s.C,
                       s.H, s.d, scale, scale * kLog2e);
    hipLaunchKernelGGL(bwd_dkdv_general_kernel<DM>, grid, block, 0, st, grad_x, lse, D, dy, qkv, s.B, s.T,
                       s.C, s.H, s.d, scale, scale * kLog2e);
}

hipError_t launch_bwd_general(float *grad_x, float *D, const float *lse, const float *dy, const float *y,
                              const float *qkv, const Shape &s, hipStream_t st)
{
    timer_begin(kKindOther, st);
    hipError_t e = launch_bwd_prep(grad_x, D, dy, y, s, st, 0);
    if (e != hipSuccess)
    {
        timer_end(st);
        return e;
    }
    if (s.d <= 16)
        launch_bwd_general_dm<16>(grad_x, lse, D, dy, qkv, s, st);
    else if (s.d <= 32)
        launch_bwd_general_dm<32>(grad_x, lse, D, dy, qkv, s, st);
    else if (s.d <= 64)
        launch_bwd_general_dm<64>(grad_x, lse, D, dy, qkv, s, st);
    else if (s.d <= 128)
        launch_bwd_general_dm<128>(grad_x, lse, D, dy, qkv, s, st);
    else
        launch_bwd_general_dm<256>(grad_x, lse, D, dy, qkv, s, st);
    timer_end(st);
    return hipGetLastError();
}

}  // namespace gpt_attn

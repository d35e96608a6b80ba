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
// same work. Its NW waves (2 for large problems, 4 for small ones, 1 for a
// single query block) split each query block's key blocks round-robin; the rotation of the second block is chosen
// so its spare units go to the waves that got none in the first, which bounds
// every wave at ceil((n + 1) / NW) units. Each wave runs its units of both query blocks as ONE software-
// pipelined stream: while a unit's softmax and PV run, the next unit's K (and,
// at the switch to the second block, that block's Q) is loaded; a unit's V
// loads during its own S^T and softmax. A wave's partial (max, sum, O) of a query block
// goes to LDS and bumps that block's counter; the block's merging wave waits
// (bounded) for the other NW - 1 and writes the row. There is no workgroup
// barrier after start-up, so no wave waits for the slowest one between blocks.
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
// range check), so there are no clamps, and every block / row offset is
// wave-uniform (scalar offset). The softmax works in log2 units: the scale
// log2(e)/sqrt(d) is applied by the FMA that forms each exponent, so
// v_exp_f32 (2^x) evaluates it directly.
//
// Workgroup order: pair-major, (b, h) fastest. Workgroups go to the 8 XCDs
// round-robin, so when B*H is a multiple of 8 every workgroup of one (b, h)
// lands on the same XCD and its K/V stay in that XCD's L2.
#include "attn_common.h"
#include "attn_kernels.h"

#include <math.h>

namespace gpt_attn {

// Spin limit of a merging wave waiting for the other waves' partials (each
// spin sleeps ~64 cycles). The partials always arrive, since no wave waits for
// anything before publishing; the limit only guarantees that the wait ends.
constexpr int kMergeSpinLimit = 1 << 24;

template <int NW>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(3))) void fwd_d64_kernel(
    float *__restrict__ y, float *__restrict__ lse, const float *__restrict__ qkv, int T, int C, int H, int BH,
    int n_qb, float c2)
{
    const int lane = threadIdx.x & 63, w = NW > 1 ? wave_id() : 0;
    const int n = lane & 31, hf = lane >> 5;
    const int pr = (int)(blockIdx.x / BH);
    const int bh = (int)(blockIdx.x % BH);
    const int b = bh / H, h = bh % H;
    const uint32_t Wb = 12u * (uint32_t)C;  // bytes per token row of qkv
    const rsrc_t rs = make_rsrc(qkv + (long)b * T * 3L * C + (long)h * 64,
                                (uint32_t)(((long)T * 3 * C - (long)h * 64) * 4));
    // lane-dependent byte offsets of the operands inside a 32-row block
    const uint32_t q_lane = (uint32_t)n * Wb + 128u * hf;                  // Q[n][32 hf ..]
    const uint32_t k_lane = q_lane + 4u * C;                               // K[n][32 hf ..]
    const uint32_t v_lane = 4u * hf * Wb + 8u * C + 8u * (uint32_t)n;      // V[4 hf + ..][2n ..]

    // partials of the non-merging waves, per query block of the pair
    constexpr int NS = NW > 1 ? NW - 1 : 1;
    __shared__ float sm_o[2][NS][32][64];  // [block][slot][register][lane]
    __shared__ float sm_m[2][NS][32], sm_l[2][NS][32];
    __shared__ int sm_cnt[2];
    if constexpr (NW > 1)
    {
        if (threadIdx.x == 0)
        {
            sm_cnt[0] = 0;
            sm_cnt[1] = 0;
        }
        __syncthreads();
    }

    // The pair: block 0 = query block qa (qa + 1 key blocks), block 1 = pr.
    // Wave w takes key blocks j = j0[k], j0[k] + NW, ... of block k.
    const int qa = n_qb - 1 - pr;
    const bool two = qa != pr;  // odd n_qb: the middle block has no partner
    const int cnt0 = qa + 1, cnt1 = two ? pr + 1 : 0;
    const int s1 = (NW - 1 - cnt0 % NW) % NW;  // block 1's spare units go where block 0 had none
    const int j00 = (w + NW - 1) % NW, j01 = (w + s1) % NW;
    const bool has0 = j00 < cnt0, has1 = j01 < cnt1;
    // merging waves: wave 0 for block 0 (never given a spare unit there), and
    // for block 1 the lowest-numbered other wave with the fewest units
    auto units = [&](int ww) {
        const int a = (ww + NW - 1) % NW, c = (ww + s1) % NW;
        return (a < cnt0 ? (cnt0 - 1 - a) / NW + 1 : 0) + (c < cnt1 ? (cnt1 - 1 - c) / NW + 1 : 0);
    };
    int merger1 = NW > 1 ? 1 : 0;
    for (int ww = 2; ww < NW; ++ww)
        if (units(ww) < units(merger1))
            merger1 = ww;
    const int merger[2] = {0, merger1};

    v16f o0 = zero16(), o1 = zero16();  // O^T rows d = 2 * row + 0 / + 1
    float m = -INFINITY, l = 0.f;       // running max (log2 units) and sum

    // Partial of block k by a non-merging wave: to LDS, then count it.
    auto publish = [&](int k) {
        const int slot = w < merger[k] ? w : w - 1;
#pragma unroll
        for (int r = 0; r < 16; ++r)
        {
            sm_o[k][slot][r][lane] = o0[r];
            sm_o[k][slot][16 + r][lane] = o1[r];
        }
        if (hf == 0)
        {
            sm_m[k][slot][n] = m;
            sm_l[k][slot][n] = l;
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
        if (lane == 0)
            __hip_atomic_fetch_add(&sm_cnt[k], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    };
    // Block k by its merging wave: wait for the three partials, combine them
    // with the wave's own state and write y and lse.
    auto merge_store = [&](int k) {
        if constexpr (NW > 1)
        {
            for (int spin = 0; spin < kMergeSpinLimit; ++spin)
            {
                if (__hip_atomic_load(&sm_cnt[k], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) >= NW - 1)
                    break;
                __builtin_amdgcn_s_sleep(1);
            }
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
        }
        float M = m;
#pragma unroll
        for (int v = 0; v < NW - 1; ++v)
            M = fmaxf(M, sm_m[k][v][n]);
        // some wave saw key block 0, so M is finite; a wave that saw no key
        // block has m = -inf and contributes 0
        const float f0 = fast_exp2(m - M);
        float L = l * f0;
        o0 *= f0;
        o1 *= f0;
#pragma unroll
        for (int v = 0; v < NW - 1; ++v)
        {
            const float f = fast_exp2(sm_m[k][v][n] - M);
            L += f * sm_l[k][v][n];
#pragma unroll
            for (int r = 0; r < 16; ++r)
            {
                o0[r] += f * sm_o[k][v][r][lane];
                o1[r] += f * sm_o[k][v][16 + r][lane];
            }
        }
        const int row = 32 * (k == 0 ? qa : pr) + n;
        if (row < T)
        {
            const float inv = 1.f / L;
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
                lse[((long)b * T + row) * H + h] = (M + fast_log2(L)) * kLn2;
        }
    };

    // A wave with no unit in a block still publishes its (empty) partial.
    if (!has0 && w != merger[0])
        publish(0);
    if (two && !has1 && w != merger[1])
        publish(1);

    // first unit of the stream
    int it = has0 ? 0 : (has1 ? 1 : -1);
    int j = it == 0 ? j00 : j01;

    // B operand of S^T = K Q^T: lane (n, hf) holds Q[q0 + n][32 hf + s]
    float qreg[32];
    float4 kv[8];  // A operand of S^T: K[32j + n][32 hf + s]
    float2 vv[16]; // A operand of step st of O^T += V^T P^T: V[32j + row(st, hf)][2n, 2n + 1]
    {
        const uint32_t qo = it >= 0 ? 32u * (uint32_t)(it == 0 ? qa : pr) * Wb : kNoBlock;
        const uint32_t kb = it >= 0 ? 32u * (uint32_t)j * Wb : kNoBlock;
#pragma unroll
        for (int t = 0; t < 8; ++t)
        {
            const float4 v = bload4s(rs, q_lane + 16u * t, qo);
            qreg[4 * t + 0] = v.x;
            qreg[4 * t + 1] = v.y;
            qreg[4 * t + 2] = v.z;
            qreg[4 * t + 3] = v.w;
        }
#pragma unroll
        for (int t = 0; t < 8; ++t)
            kv[t] = bload4s(rs, k_lane + 16u * t, kb);
    }

    while (it >= 0)
    {
        const int qb = it == 0 ? qa : pr;
        const int cnt = it == 0 ? cnt0 : cnt1;
        int nit = -1, nj = 0;  // next unit of the stream
        if (j + NW < cnt)
        {
            nit = it;
            nj = j + NW;
        }
        else if (it == 0 && has1)
        {
            nit = 1;
            nj = j01;
        }
        const uint32_t kn = nit >= 0 ? 32u * (uint32_t)nj * Wb : kNoBlock;
        const uint32_t qn = nit == 1 && it == 0 ? 32u * (uint32_t)pr * Wb : kNoBlock;

        // S^T[key 32j + row(r)][query 32 qb + n] (unscaled); this unit's V
        // loads go out with the first MFMAs and land during S^T and the softmax
        const uint32_t kc = 32u * (uint32_t)j * Wb;
        v16f s = zero16();
#pragma unroll
        for (int t = 0; t < 8; ++t)
        {
            s = mfma32(kv[t].x, qreg[4 * t + 0], s);
            s = mfma32(kv[t].y, qreg[4 * t + 1], s);
            s = mfma32(kv[t].z, qreg[4 * t + 2], s);
            s = mfma32(kv[t].w, qreg[4 * t + 3], s);
            if (t == 0)
            {
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int st = 0; st < 16; ++st)
                    vv[st] = bload2s(rs, v_lane, kc + (uint32_t)(8 * (st >> 2) + (st & 3)) * Wb);
                __builtin_amdgcn_sched_barrier(0);
            }
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
        const float mn = fmaxf(m, mt * c2);
        const float corr = fast_exp2(m - mn);
        float ps = 0.f;
#pragma unroll
        for (int r = 0; r < 16; ++r)
        {
            s[r] = fast_exp2(fmaf(s[r], c2, -mn));
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
        if (qn != kNoBlock)
        {
            // switching to block 1: its Q replaces this block's (issued after
            // the next unit's K, so only this one switch waits for it)
#pragma unroll
            for (int t = 0; t < 8; ++t)
            {
                const float4 v = bload4s(rs, q_lane + 16u * t, qn);
                qreg[4 * t + 0] = v.x;
                qreg[4 * t + 1] = v.y;
                qreg[4 * t + 2] = v.z;
                qreg[4 * t + 3] = v.w;
            }
        }
        __builtin_amdgcn_sched_barrier(0);

        if (nit != it)
        {
            // this wave's last unit of block `it`
            if (w == merger[it])
                merge_store(it);
            else
                publish(it);
            o0 = zero16();
            o1 = zero16();
            m = -INFINITY;
            l = 0.f;
        }
        it = nit;
        j = nj;
    }

    // merging waves that had no unit in their block
    if (w == merger[0] && !has0)
        merge_store(0);
    if (two && w == merger[1] && !has1)
        merge_store(1);
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
    const int n_qb = (s.T + 31) / 32;
    const int BH = s.B * s.H;
    const long blocks = (long)((n_qb + 1) / 2) * BH;  // heavy/light pairs
    const float c2 = softmax_scale(64) * kLog2e;
    // Waves per pair: 4 while the pairs alone leave most of the 1024 SIMDs
    // idle, else 2 (fewer, longer streams, one partial to merge per block;
    // equal at B=16 T=256, 5-15 % faster at T >= 1024 or B = 64); never more
    // waves than the pair has units (one query block: no merge at all).
    int nw = blocks > 256 ? 2 : 4;
    while (nw > 1 && nw > n_qb + 1)
        nw >>= 1;
    if (n_qb == 1)
        nw = 1;
    timer_begin(kKindFwd, st);
    const dim3 grid((unsigned)blocks);
    switch (nw)
    {
    case 4:
        hipLaunchKernelGGL(fwd_d64_kernel<4>, grid, dim3(256), 0, st, y, lse, qkv, s.T, s.C, s.H, BH, n_qb, c2);
        break;
    case 2:
        hipLaunchKernelGGL(fwd_d64_kernel<2>, grid, dim3(128), 0, st, y, lse, qkv, s.T, s.C, s.H, BH, n_qb, c2);
        break;
    default:
        hipLaunchKernelGGL(fwd_d64_kernel<1>, grid, dim3(64), 0, st, y, lse, qkv, s.T, s.C, s.H, BH, n_qb, c2);
        break;
    }
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

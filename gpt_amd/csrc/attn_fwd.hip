// Causal self-attention forward for gfx950.
//
// Computes, per (b, h) and query row i,
//   y[i]   = sum_{j<=i} softmax_j(q_i . k_j / sqrt(d)) v_j
//   lse[i] = log sum_{j<=i} exp(q_i . k_j / sqrt(d))
// matching the reference CPU backend (src/backend/cpu/cpu_backend.cpp:289-356)
// and replacing the reference's CUDA kernel (src/backend/cuda/kernels/
// attention.cu:6-268).
//
// head_dim 64 kernels. fwd_qs_d64_kernel (below) for calls with at least 256
// 64-query groups, fwd_split_d64_kernel (below) for very small calls, and:
//
// fwd_d64_kernel (the calls in between). Work unit = one 32-query block x one
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

// Q-stationary head_dim-64 forward (fwd_qs_d64_kernel). One workgroup per
// (b, h, 64-query group J); wave w owns the 16 query rows qw0 = 64 J + 16 w ..
// qw0 + 15: their Q stays in registers as the MFMA B operand and their O, row
// max and row sum accumulate in registers, so no wave shares a row and nothing
// is merged. The 4 waves walk the key blocks 0 .. 2J + 1 together; each
// block's K and V (32 x 64) are staged once in LDS for all 4 waves (double
// buffered: block kb + 1 is loaded into registers while block kb is computed,
// then written to the other buffer; one barrier per block). Per wave and key
// block, on v_mfma_f32_16x16x4_f32 (two 16-key tiles kt):
//   S^T_kt = K_kt Q^T          (16 keys x 16 queries, 16 MFMAs each)
//   online softmax per query column in log2 units, the scale folded into the
//   exponent FMA, with a lazily updated reference max m: while no score of
//   the block exceeds m + kLazyRescale (checked with one wave vote), P is taken
//   against the stale m (so P <= 2^kLazyRescale) and neither O nor the row
//   sums are rescaled; otherwise m is raised to the block's row max (reduced
//   across the 4 lane groups) and O and the sums are rescaled. The quotient
//   O / l and lse = m + log2 l do not depend on which m was used.
//   O^T += V^T P^T             (4 accumulators of 16 x 16 over 32 keys; the
//                              S^T accumulators are the B operands as they are)
// Each lane keeps the row sum over its own keys; the 4 lane groups' sums are
// added once, after the last block.
// Workgroups are ordered heaviest first (J descending), (b, h) fastest; when
// the whole grid is resident the middle round is reversed (in blocks of 8, one
// XCD per (b, h)) so that every CU gets one heavy, one light and one middle
// group; grids of 1 to 2 workgroups per CU pair them (paired_item).
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3))) void fwd_qs_d64_kernel(
    float *__restrict__ y, float *__restrict__ lse, const float *__restrict__ qkv, int T, int C, int H, int BH,
    int n_qg, float c2, int n_cu)
{
    constexpr int ST = kTileRow;
    const int tid = threadIdx.x, lane = tid & 63, w = wave_id();
    const int c16 = lane & 15, g4 = lane >> 4;
    int item = (int)blockIdx.x;
    {
        const int G = (int)gridDim.x;
        if (n_cu > 0 && n_cu % 8 == 0 && G % n_cu == 0 && G / n_cu <= 3)
        {
            const int r = item / n_cu;
            int c = item % n_cu;
            if (r & 1)
                c = (n_cu / 8 - 1 - c / 8) * 8 + (c & 7);
            item = r * n_cu + c;
        }
    }
    int J = n_qg - 1 - item / BH;
    int bh = item % BH;
    {
        int cls = 0, idx = 0;
        if (paired_item((int)blockIdx.x, (int)gridDim.x, n_cu, BH, &cls, &idx))
        {
            J = n_qg - 1 - cls;
            bh = idx;
        }
    }
    const int b = bh / H, h = bh % H;
    if (J == 0 && n_qg == 4 && (int)gridDim.x > 2 * n_cu && (int)gridDim.x <= 3 * n_cu)
    {
        // Whole grid resident at 3 per CU (C3): the J = 0 workgroups are the
        // youngest on their CUs and get no MFMA time until about 13 us in,
        // while every workgroup's Q and first K/V arrive at once from HBM.
        // Their first loads wait about 3.4 us (127 x 64 cycles), so that
        // the heavier groups' start-up data arrives first: C3 forward
        // 21.62-21.78 -> 21.37-21.45 us (A/B on one box, outputs unchanged;
        // 1.7 us: 21.54-21.58 us, 6.8 us: no gain).
        __builtin_amdgcn_s_sleep(127);
    }
    const int qw0 = 64 * J + 16 * w;
    const uint32_t Wb = 12u * (uint32_t)C, Cb = 4u * (uint32_t)C;
    const rsrc_t rs = make_rsrc(qkv + (long)b * T * 3L * C + (long)h * 64,
                                (uint32_t)(((long)T * 3 * C - (long)h * 64) * 4));

    // K tiles swizzled (tile_off), V tiles plain 64-word rows: the V reads
    // (row 4 (l/16) + r, column group l%16) are conflict-free unswizzled. One
    // array per buffer, so that the compiler sees that loads landing in one
    // buffer do not alias reads of the other.
    __shared__ __attribute__((aligned(16))) float sk0[32 * ST], sv0[32 * ST], sk1[32 * ST], sv1[32 * ST];
    auto bufs = [&](auto buf_c) {
        constexpr int buf = decltype(buf_c)::value;
        struct B
        {
            float *k, *v;
        };
        return buf == 0 ? B{sk0, sv0} : B{sk1, sv1};
    };

    // stationary B operand: lane l holds Q[qw0 + l%16][16 (l/16) + m], m = 0..15
    // (MFMA m contracts d = m + 16 kk, kk = l/16)
    float qreg[16];
    {
        const uint32_t off = (uint32_t)c16 * Wb + 64u * g4;
#pragma unroll
        for (int c = 0; c < 4; ++c)
        {
            const float4 q4 = bload4s(rs, off + 16u * c, (uint32_t)qw0 * Wb);
            qreg[4 * c + 0] = q4.x;
            qreg[4 * c + 1] = q4.y;
            qreg[4 * c + 2] = q4.z;
            qreg[4 * c + 3] = q4.w;
        }
    }

    // Staging goes straight from memory into LDS (buffer loads to LDS, no
    // registers). A 32 x 64 tile is 8 chunks of 1 KiB, chunk k = rows
    // 4k .. 4k + 3; wave w moves chunks w and w + 4 of the K and of the V
    // tile. Lane l lands at row 4k + l/16, physical column group l%16: for the
    // swizzled K tile it fetches the logical group (l%16) ^ tile_swz(row),
    // tile_swz(row) = (l/16) << 2 | w for both of its chunks.
    const uint32_t dma_row = (uint32_t)(4 * w + (lane >> 4));
    const uint32_t k_lane = dma_row * Wb + Cb + 16u * (uint32_t)((lane & 15) ^ (((lane >> 4) << 2) | w));
    const uint32_t v_lane = dma_row * Wb + 2u * Cb + 16u * (uint32_t)(lane & 15);
    const int kb_end = min(2 * J + 2, (T + 31) / 32);  // key blocks 0 .. kb_end - 1
    auto issue = [&](int kb, auto buf_c) {
        const auto B = bufs(buf_c);
        const uint32_t ko = kb < kb_end ? 32u * (uint32_t)kb * Wb : kNoBlock;
        dma16(rs, B.k + 256 * w, k_lane, ko);
        dma16(rs, B.k + 256 * (w + 4), k_lane + 16u * Wb, ko);
        dma16(rs, B.v + 256 * w, v_lane, ko);
        dma16(rs, B.v + 256 * (w + 4), v_lane + 16u * Wb, ko);
    };

    v4f o0 = zero4(), o1 = zero4(), o2 = zero4(), o3 = zero4();  // O^T, d = 16 g4 + 4 r + e
    // reference max (log2 units, the same in the 4 lane groups of a query) of
    // query qw0 + c16 and this lane's part of its row sum
    float m = -INFINITY, l = 0.f;

    // One key block, in LDS buffer buf (a compile-time constant, so that it
    // folds into the ds_read offsets). Only the last two blocks (2J, 2J + 1)
    // can hold keys past queries; only they (GEN) test for a skipped block,
    // a fully masked second 16-key half (HALF: k0 = qw0) and the causal mask.
    auto block = [&](const int kb, auto buf_c, auto gen_c) {
        constexpr int buf = decltype(buf_c)::value;
        constexpr bool GEN = decltype(gen_c)::value;
        issue(kb + 1, BufIdx<buf ^ 1>{});
        __builtin_amdgcn_sched_barrier(0);
        const int k0 = 32 * kb;
        const auto B = bufs(buf_c);
        const float *Ks = B.k, *Vs = B.v;
        auto tile = [&](auto half_c) {
            constexpr bool HALF = decltype(half_c)::value;
            // S^T_kt[key k0 + 16 kt + 4 g4 + r][query qw0 + c16] (unscaled)
            v4f s0 = zero4(), s1 = zero4();
#pragma unroll
            for (int c = 0; c < 4; ++c)
            {
                const int ko = tile_off(c16, 4 * g4 + c);
                const float4 ka = *reinterpret_cast<const float4 *>(Ks + ko);
                const float kav[4] = {ka.x, ka.y, ka.z, ka.w};
                if constexpr (!HALF)
                {
                    const float4 kb4 = *reinterpret_cast<const float4 *>(Ks + 16 * ST + ko);
                    const float kbv[4] = {kb4.x, kb4.y, kb4.z, kb4.w};
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                    {
                        s0 = mfma16(kav[e], qreg[4 * c + e], s0);
                        s1 = mfma16(kbv[e], qreg[4 * c + e], s1);
                    }
                }
                else
                {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        s0 = mfma16(kav[e], qreg[4 * c + e], s0);
                }
            }
            if (GEN && k0 + 31 > qw0)
            {
                // diagonal block: key > query is masked out
                const int q = qw0 + c16;
#pragma unroll
                for (int r = 0; r < 4; ++r)
                {
                    if (k0 + 4 * g4 + r > q)
                        s0[r] = -INFINITY;
                    if (HALF || k0 + 16 + 4 * g4 + r > q)
                        s1[r] = -INFINITY;
                }
            }
            // exponent arguments against the current reference max
            float e0[4], e1[4];
#pragma unroll
            for (int r = 0; r < 4; ++r)
            {
                e0[r] = fmaf(s0[r], c2, -m);
                e1[r] = fmaf(s1[r], c2, -m);
            }
            const float emax = fmaxf(fmaxf(fmaxf(e0[0], e0[1]), fmaxf(e0[2], e0[3])),
                                     fmaxf(fmaxf(e1[0], e1[1]), fmaxf(e1[2], e1[3])));
            // The first block always takes this branch: with m = -inf every
            // lane holding an unmasked score has emax = +inf, and key 0 is
            // unmasked for every query (lanes with only masked scores get
            // NaN arguments here, which the branch recomputes). m is finite
            // afterwards.
            if (__any(emax > kLazyRescale))
            {
                const float mt = fmaxf(fmaxf(fmaxf(s0[0], s0[1]), fmaxf(s0[2], s0[3])),
                                       fmaxf(fmaxf(s1[0], s1[1]), fmaxf(s1[2], s1[3]))) * c2;
                const float mn = fmaxf(m, halves_max(rows16_max(mt)));
                const float corr = fast_exp2(m - mn);
                l *= corr;
                m = mn;
                o0 *= corr;
                o1 *= corr;
                o2 *= corr;
                o3 *= corr;
#pragma unroll
                for (int r = 0; r < 4; ++r)
                {
                    e0[r] = fmaf(s0[r], c2, -m);
                    e1[r] = fmaf(s1[r], c2, -m);
                }
            }
#pragma unroll
            for (int r = 0; r < 4; ++r)
            {
                s0[r] = fast_exp2(e0[r]);
                s1[r] = fast_exp2(e1[r]);
            }
            l += ((s0[0] + s1[0]) + (s0[1] + s1[1])) + ((s0[2] + s1[2]) + (s0[3] + s1[3]));
            // O^T += V^T P^T: step (kt, r) contracts keys k0 + 16 kt + 4 kk + r
            // (kk = l/16); A operand V[that key][4 c16 + e]
#pragma unroll
            for (int r = 0; r < 4; ++r)
            {
                const float4 va = *reinterpret_cast<const float4 *>(Vs + (4 * g4 + r) * ST + 4 * c16);
                o0 = mfma16(va.x, s0[r], o0);
                o1 = mfma16(va.y, s0[r], o1);
                o2 = mfma16(va.z, s0[r], o2);
                o3 = mfma16(va.w, s0[r], o3);
                if constexpr (!HALF)
                {
                    const float4 vb = *reinterpret_cast<const float4 *>(Vs + (16 + 4 * g4 + r) * ST + 4 * c16);
                    o0 = mfma16(vb.x, s1[r], o0);
                    o1 = mfma16(vb.y, s1[r], o1);
                    o2 = mfma16(vb.z, s1[r], o2);
                    o3 = mfma16(vb.w, s1[r], o3);
                }
            }
        };
        if constexpr (GEN)
        {
            if (k0 == qw0)
                tile(BufIdx<1>{});
            else if (k0 <= qw0 + 15)  // else every key of the block lies past this wave's queries
                tile(BufIdx<0>{});
        }
        else
            tile(BufIdx<0>{});
        __builtin_amdgcn_sched_barrier(0);
        lds_dma_wait();  // block kb + 1 has landed in the other buffer
        lds_barrier();
    };

    issue(0, BufIdx<0>{});
    lds_dma_wait();
    lds_barrier();
    // blocks 0 .. kb_end - 3 lie wholly before this workgroup's queries
    const int kb_gen = kb_end > 2 ? kb_end - 2 : 0;
    int kb = 0;
    for (; kb + 1 < kb_gen; kb += 2)
    {
        block(kb, BufIdx<0>{}, BufIdx<0>{});
        block(kb + 1, BufIdx<1>{}, BufIdx<0>{});
    }
    if (kb < kb_gen)  // odd count: one more plain block, the others start in buffer 1
    {
        block(kb, BufIdx<0>{}, BufIdx<0>{});
        block(kb + 1, BufIdx<1>{}, BufIdx<1>{});
        if (kb + 2 < kb_end)
            block(kb + 2, BufIdx<0>{}, BufIdx<1>{});
    }
    else
    {
        if (kb < kb_end)
            block(kb, BufIdx<0>{}, BufIdx<1>{});
        if (kb + 1 < kb_end)
            block(kb + 1, BufIdx<1>{}, BufIdx<1>{});
    }

    // register r of accumulator e: O[qw0 + c16][16 g4 + 4 r + e]
    l = halves_sum(rows16_sum(l));
    const float inv = 1.f / l;
    {
        // The wave's 16 x 64 O tile goes through LDS (the K/V buffers are
        // free after the last block's barrier: one buffer per wave, rows of
        // 68 words), so that each store instruction writes 4 whole 256-byte
        // rows, and the rows are written through to memory (device scope,
        // sc1). Lines left dirty in the XCD's L2 would be written back when
        // the launch ends, after the last workgroup: C3 forward 24.1 ->
        // 21.8 us (23.5 us with the staging alone).
        float *stg = w == 0 ? sk0 : w == 1 ? sv0 : w == 2 ? sk1 : sv1;
#pragma unroll
        for (int r = 0; r < 4; ++r)
            *reinterpret_cast<float4 *>(stg + c16 * 68 + 16 * g4 + 4 * r) =
                make_float4(o0[r] * inv, o1[r] * inv, o2[r] * inv, o3[r] * inv);
        const rsrc_t ry =
            make_rsrc(y + (long)b * T * C + (long)h * 64, (uint32_t)(((long)T * C - (long)h * 64) * 4));
#pragma unroll
        for (int i = 0; i < 4; ++i)
        {
            const int rr = (lane >> 4) + 4 * i;
            const float4 v = *reinterpret_cast<const float4 *>(stg + rr * 68 + 4 * (lane & 15));
            if (qw0 + rr < T)
                store4_sc1(ry, (uint32_t)(qw0 + rr) * 4u * (uint32_t)C + 16u * (uint32_t)(lane & 15), v);
        }
    }
    const int row = qw0 + c16;
    if (row < T && g4 == 0)
        lse[((long)b * T + row) * H + h] = (m + fast_log2(l)) * kLn2;
}

// Split-key head_dim-64 forward for calls too small to fill the GPU with
// 64-query groups (fwd_split_d64_kernel: B = 1 generation prefixes, C1). One
// workgroup per (b, h, 16-query group g), heaviest groups first; its NW waves
// take the group's 32-key blocks round-robin (one block each up to T = 16 NW
// ... 32 NW), so a call's latency is about one block instead of the whole
// row. Each wave keeps the group's Q in registers (the MFMA B operand, as in
// the Q-stationary kernel), loads its K and V blocks straight from memory as
// MFMA operands, and runs the same S^T / online-softmax / O^T += V^T P^T steps
// on v_mfma_f32_16x16x4_f32. The waves' partials (row max m, row sum l, O)
// then meet in LDS: O = sum_w 2^(m_w - M) O_w / sum_w 2^(m_w - M) l_w with
// M = max_w m_w, in wave order.
template <int NW>
__global__ __launch_bounds__(NW * 64) void fwd_split_d64_kernel(float *__restrict__ y, float *__restrict__ lse,
                                                                const float *__restrict__ qkv, int T, int C, int H,
                                                                int BH, int n_g, float c2)
{
    const int tid = threadIdx.x, lane = tid & 63, w = NW > 1 ? wave_id() : 0;
    const int c16 = lane & 15, g4 = lane >> 4;
    const int g = n_g - 1 - (int)(blockIdx.x / BH);
    const int bh = (int)(blockIdx.x % BH), b = bh / H, h = bh % H;
    const int q0 = 16 * g;
    const int n_kb = (q0 + 15) / 32 + 1;  // key blocks 0 .. n_kb - 1 hold the keys <= q0 + 15
    const uint32_t Wb = 12u * (uint32_t)C, Cb = 4u * (uint32_t)C;
    const rsrc_t rs = make_rsrc(qkv + (long)b * T * 3L * C + (long)h * 64,
                                (uint32_t)(((long)T * 3 * C - (long)h * 64) * 4));

    // B operand: lane l holds Q[q0 + l%16][16 (l/16) + m], m = 0..15
    float qreg[16];
    {
        const uint32_t off = (uint32_t)c16 * Wb + 64u * g4;
#pragma unroll
        for (int c = 0; c < 4; ++c)
        {
            const float4 q4 = bload4s(rs, off + 16u * c, (uint32_t)q0 * Wb);
            qreg[4 * c + 0] = q4.x;
            qreg[4 * c + 1] = q4.y;
            qreg[4 * c + 2] = q4.z;
            qreg[4 * c + 3] = q4.w;
        }
    }
    // lane parts of a block's operand offsets: K[c16 (+16)][16 g4 + 4c ..],
    // V[4 g4 + r (+16)][4 c16 ..]
    const uint32_t k_lane = (uint32_t)c16 * Wb + Cb + 64u * g4;
    const uint32_t v_lane = 4u * g4 * Wb + 2u * Cb + 16u * c16;

    v4f o0 = zero4(), o1 = zero4(), o2 = zero4(), o3 = zero4();  // O^T, d = 16 g4 + 4 r + e
    float m = -INFINITY, l = 0.f;  // max (log2 units) of query q0 + c16, this lane's part of its sum
    for (int kb = w; kb < n_kb; kb += NW)
    {
        const int k0 = 32 * kb;
        const uint32_t ko = (uint32_t)k0 * Wb;
        float4 ka[4], kb4[4], va[4], vb[4];
#pragma unroll
        for (int c = 0; c < 4; ++c)
        {
            ka[c] = bload4s(rs, k_lane + 16u * c, ko);
            kb4[c] = bload4s(rs, k_lane + 16u * c + 16u * Wb, ko);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r)
        {
            va[r] = bload4s(rs, v_lane + (uint32_t)r * Wb, ko);
            vb[r] = bload4s(rs, v_lane + (uint32_t)(16 + r) * Wb, ko);
        }
        // S^T_kt[key k0 + 16 kt + 4 g4 + r][query q0 + c16] (unscaled)
        v4f s0 = zero4(), s1 = zero4();
#pragma unroll
        for (int c = 0; c < 4; ++c)
        {
            const float kav[4] = {ka[c].x, ka[c].y, ka[c].z, ka[c].w};
            const float kbv[4] = {kb4[c].x, kb4[c].y, kb4[c].z, kb4[c].w};
#pragma unroll
            for (int e = 0; e < 4; ++e)
            {
                s0 = mfma16(kav[e], qreg[4 * c + e], s0);
                s1 = mfma16(kbv[e], qreg[4 * c + e], s1);
            }
        }
        if (k0 + 31 > q0)
        {
            // diagonal block: key > query is masked out
            const int q = q0 + c16;
#pragma unroll
            for (int r = 0; r < 4; ++r)
            {
                if (k0 + 4 * g4 + r > q)
                    s0[r] = -INFINITY;
                if (k0 + 16 + 4 * g4 + r > q)
                    s1[r] = -INFINITY;
            }
        }
        // online softmax over this wave's blocks; its first block holds an
        // unmasked key for every query (block w <= the diagonal), so m is
        // finite from then on
        float mt = fmaxf(fmaxf(fmaxf(s0[0], s0[1]), fmaxf(s0[2], s0[3])),
                         fmaxf(fmaxf(s1[0], s1[1]), fmaxf(s1[2], s1[3])));
        mt = halves_max(rows16_max(mt));
        const float mn = fmaxf(m, mt * c2);
        const float corr = fast_exp2(m - mn);
#pragma unroll
        for (int r = 0; r < 4; ++r)
        {
            s0[r] = fast_exp2(fmaf(s0[r], c2, -mn));
            s1[r] = fast_exp2(fmaf(s1[r], c2, -mn));
        }
        l = l * corr + (((s0[0] + s1[0]) + (s0[1] + s1[1])) + ((s0[2] + s1[2]) + (s0[3] + s1[3])));
        m = mn;
        o0 *= corr;
        o1 *= corr;
        o2 *= corr;
        o3 *= corr;
        // O^T += V^T P^T: step (kt, r) contracts keys k0 + 16 kt + 4 kk + r (kk = l/16)
#pragma unroll
        for (int r = 0; r < 4; ++r)
        {
            o0 = mfma16(va[r].x, s0[r], o0);
            o1 = mfma16(va[r].y, s0[r], o1);
            o2 = mfma16(va[r].z, s0[r], o2);
            o3 = mfma16(va[r].w, s0[r], o3);
            o0 = mfma16(vb[r].x, s1[r], o0);
            o1 = mfma16(vb[r].y, s1[r], o1);
            o2 = mfma16(vb[r].z, s1[r], o2);
            o3 = mfma16(vb[r].w, s1[r], o3);
        }
    }
    l = halves_sum(rows16_sum(l));

    const int row_base = q0;
    if constexpr (NW == 1)
    {
        const int row = row_base + c16;
        if (row < T)
        {
            const float inv = 1.f / l;
            float *dst = y + ((long)b * T + row) * C + (long)h * 64 + 16 * g4;
#pragma unroll
            for (int r = 0; r < 4; ++r)
                *reinterpret_cast<float4 *>(dst + 4 * r) =
                    make_float4(o0[r] * inv, o1[r] * inv, o2[r] * inv, o3[r] * inv);
            if (g4 == 0)
                lse[((long)b * T + row) * H + h] = (m + fast_log2(l)) * kLn2;
        }
    }
    else
    {
        // partials to LDS (a wave without blocks contributes m = -inf, l = 0, O = 0)
        __shared__ __attribute__((aligned(16))) float sm_o[NW][16 * 64];
        __shared__ float sm_m[NW][16], sm_l[NW][16];
#pragma unroll
        for (int r = 0; r < 4; ++r)
            *reinterpret_cast<float4 *>(&sm_o[w][c16 * 64 + 16 * g4 + 4 * r]) = make_float4(o0[r], o1[r], o2[r], o3[r]);
        if (g4 == 0)
        {
            sm_m[w][c16] = m;
            sm_l[w][c16] = l;
        }
        __syncthreads();
        // thread tid: query row tid / (NW * 4), float4 columns strided by NW * 4
        constexpr int TPR = NW * 4;  // threads per row
        const int q = tid / TPR, part = tid % TPR;
        float M = -INFINITY;
#pragma unroll
        for (int ww = 0; ww < NW; ++ww)
            M = fmaxf(M, sm_m[ww][q]);
        float L = 0.f, f[NW];
#pragma unroll
        for (int ww = 0; ww < NW; ++ww)
        {
            f[ww] = fast_exp2(sm_m[ww][q] - M);
            L += f[ww] * sm_l[ww][q];
        }
        const float inv = 1.f / L;
        const int row = row_base + q;
        if (row < T)
        {
            float *dst = y + ((long)b * T + row) * C + (long)h * 64;
            for (int c4 = part; c4 < 16; c4 += TPR)
            {
                float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
                for (int ww = 0; ww < NW; ++ww)
                {
                    const float4 x = *reinterpret_cast<const float4 *>(&sm_o[ww][q * 64 + 4 * c4]);
                    acc.x += f[ww] * x.x;
                    acc.y += f[ww] * x.y;
                    acc.z += f[ww] * x.z;
                    acc.w += f[ww] * x.w;
                }
                *reinterpret_cast<float4 *>(dst + 4 * c4) = make_float4(acc.x * inv, acc.y * inv, acc.z * inv, acc.w * inv);
            }
            if (part == 0)
                lse[((long)b * T + row) * H + h] = (M + fast_log2(L)) * kLn2;
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

static int fwd_cu_count()
{
    static int cached[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64)
        return 0;
    if (cached[dev] == 0)
    {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
            n = -1;
        cached[dev] = n;
    }
    return cached[dev] > 0 ? cached[dev] : 0;
}

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
    const int n_qg = (s.T + 63) / 64;
    const int n_g = (s.T + 15) / 16;
    const long groups = (long)n_qg * BH;
    // Long rows over few (b, h): below 512 64-query groups the Q-stationary
    // kernel's heaviest group (2 T / 32 key blocks on one workgroup) sets its
    // time, and the split-key kernel, 8 waves per 16-query group, is faster
    // (B=1 T=2048: 78.6 vs 98.7 us; B=2 T=1024: 50.4 vs 55.6 us; at 768
    // groups and more it is not: B=1 T=4096 257 vs 224 us, B=4 T=1024 90.9 vs
    // 69.3 us).
    const bool long_rows = groups >= 256 && groups < 512 && s.T >= 1024;
    if (groups >= 256 && !long_rows)
    {
        // enough 64-query groups to fill the GPU: the Q-stationary kernel
        launch_timed(kKindFwd, fwd_qs_d64_kernel, dim3((unsigned)groups), dim3(256), st, y, lse, qkv, s.T, s.C, s.H,
                     BH, n_qg, c2, fwd_cu_count());
        return hipGetLastError();
    }
    if (long_rows || (long)n_g * BH <= 512)
    {
        // very small call (at most 2 workgroups per CU), or long rows over few
        // (b, h): the split-key kernel, one workgroup per 16-query group, up
        // to 8 waves splitting its key blocks (one block each up to T = 256). Measured faster than the pair
        // kernel up to this size (B=1 T=256: 9.6 vs 15.0 us; B=1 T=512: 15.5
        // vs 19.8 us; B=2 T=256: 11.7 vs 15.4 us), slower past it (B=2 T=512:
        // 22.3 vs 20.8 us; B=1 T=1024: 31.6 vs 30.3 us).
        const int kb_max = (16 * (n_g - 1) + 15) / 32 + 1;
        int sw = 1;
        while (sw < kb_max && sw < 8)
            sw <<= 1;
        const dim3 g2((unsigned)((long)n_g * BH));
        switch (sw)
        {
        case 8:
            launch_timed(kKindFwd, fwd_split_d64_kernel<8>, g2, dim3(512), st, y, lse, qkv, s.T, s.C, s.H, BH, n_g, c2);
            break;
        case 4:
            launch_timed(kKindFwd, fwd_split_d64_kernel<4>, g2, dim3(256), st, y, lse, qkv, s.T, s.C, s.H, BH, n_g, c2);
            break;
        case 2:
            launch_timed(kKindFwd, fwd_split_d64_kernel<2>, g2, dim3(128), st, y, lse, qkv, s.T, s.C, s.H, BH, n_g, c2);
            break;
        default:
            launch_timed(kKindFwd, fwd_split_d64_kernel<1>, g2, dim3(64), st, y, lse, qkv, s.T, s.C, s.H, BH, n_g, c2);
            break;
        }
        return hipGetLastError();
    }
    const dim3 grid((unsigned)blocks);
    switch (nw)
    {
    case 4:
        launch_timed(kKindFwd, fwd_d64_kernel<4>, grid, dim3(256), st, y, lse, qkv, s.T, s.C, s.H, BH, n_qb, c2);
        break;
    case 2:
        launch_timed(kKindFwd, fwd_d64_kernel<2>, grid, dim3(128), st, y, lse, qkv, s.T, s.C, s.H, BH, n_qb, c2);
        break;
    default:
        launch_timed(kKindFwd, fwd_d64_kernel<1>, grid, dim3(64), st, y, lse, qkv, s.T, s.C, s.H, BH, n_qb, c2);
        break;
    }
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

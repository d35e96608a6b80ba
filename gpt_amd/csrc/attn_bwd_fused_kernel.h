// Causal self-attention backward for gfx950, head_dim 64: one persistent
// launch that computes dK, dV, the dS tiles and dQ.
//
// Matches the reference CPU backend (src/backend/cpu/cpu_backend.cpp:358-437)
// and replaces the reference's CUDA path (src/backend/cuda/kernels/
// attention.cu:270-577), whose dQ is added with one fp32 atomicAdd per element
// and tile (attention.cu:501-523). Here dQ is formed without atomics from dS
// tiles that the dK/dV work stores, as in the two-launch backward of
// attn_bwd.hip, but inside the same launch: the dQ of a query block starts as
// soon as all of its dS tiles exist, on workgroups that have run out of dK/dV
// work, instead of after a kernel boundary. Every sum has a fixed order, so
// the result is bitwise reproducible.
//
// Work (one workgroup of 4 waves each):
//   dK/dV item (b, h, 64-key group J), one per workgroup, taken by its index
//     (J-major, heaviest first, as bwd_dkdv_d64_kernel): K/V-stationary, as
//     that kernel, but walking its query blocks from the last (n - 1) down
//     to its diagonal blocks (2J + 1, 2J), so that all key groups of a (b, h)
//     finish the high blocks (the ones with the most dQ work) first. After
//     the barrier that ends the step of block i, each wave's dS stores of the
//     block before (i + 1) are complete (the step's vm_wait covered them),
//     and one thread adds 1 to the completion counter of (b, h, i + 1); the
//     last block's counter is bumped after a final wait.
//   dQ work of query blocks, done by the workgroups of the same
//     (b, h) once their dK/dV item is done: key group J forms dQ of its own
//     diagonal blocks 2J + 1 and 2J. Those are the last blocks it walks, and
//     the lower key groups reach them at about the same step count, so they
//     are complete about when J's dK/dV item ends and the dQ work needs no
//     waiting; the light key groups, which finish first, take the big
//     blocks. dQ items run at the lowest wave priority, behind the dK/dV
//     items still in flight. (12-layer step, A/B on one box: 1.006 ms with the
//     blocks dealt to the key groups by dQ work alone and the dK/dV
//     priorities kept, 1.001 ms diagonal blocks, 0.985 ms diagonal blocks at
//     priority 0; dealing the blocks by dK/dV plus dQ work, which gave all of
//     them to the two lightest key groups, 1.044 ms.)
//     The two blocks form one dQ item (one wait, one stream of units, see
//     dq_both below; 12-layer step 0.972 -> 0.959 ms against one item per
//     block, A/B on one box).
// The dS tiles are stored and loaded with the sc1 cache policy (coherent at
// device scope: written through to memory and read from there, whichever
// XCD's L2 the two sides sit behind), and a counter is bumped only after the
// stores it covers have completed, so a dQ item that sees a complete count
// reads complete tiles.
//
// Forward progress does not depend on which workgroups are resident. The
// owner of a dQ item waits for its counts only for a bounded time (tens of
// microseconds; in a launch whose grid is resident at once the counts are
// complete long before). If a contributing key group has not run yet
// (another kernel or process holds CUs, or the dispatcher placed work in
// another order), the owner marks its item an orphan and ends, which frees
// its slot. A few extra workgroups at the end of the grid (kOrphanRunners)
// wait until every main workgroup of their (b, h) pairs has made its
// decision (done counters), then run the orphans. No main workgroup ever waits for them, so every wait
// ends; an orphan's counts are complete by then (its contributors walked
// before deciding), and its dQ sums run in the same order, so the result is
// the same bits whoever runs an item. Each counter is released by
// subtracting its need once the item has run, so every launch leaves the
// counters at 0 once its own bumps have landed. The runners' waits carry a
// long time limit as a safety net that no schedule reaches; when it expires
// it counts an error in the control block and the item computes from
// whatever is there.
//
// Control block (int32 words, zeroed when the workspace is allocated; each
// region at a fixed place whatever the shape, M = kCtlItems):
//   [16] expired safety waits
//   [32, 32 + M) completion counters, (b, h) * n_qb + block
//   [32 + M, 32 + 2M) orphan flags, (b, h) * key groups + J: the epoch of
//   the launch that made item J of (b, h) an orphan
//   [32 + 2M, 32 + 3M) done counters, (b, h): its main workgroups that have
//   decided (one counter per (b, h), so that these atomics do not all meet
//   on one word); released by the runners
#pragma once
#include "attn_common.h"
#include "attn_kernels.h"

#include <math.h>

namespace gpt_attn {

namespace {

// The fused kernel computes the D rows itself, which pays only up to T = 256
// (at most 4 key groups; beyond it the two-launch form and a separate D-row
// pass measure as fast or faster).
constexpr int kMaxFusedKeyGroups = 4;


// dS tile stores / loads coherent at device scope (sc1).
constexpr int kSc1 = 16;

__device__ __forceinline__ void store_sc1(float *p, float v)
{
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float4 bload4s_sc1(rsrc_t r, uint32_t voff, uint32_t soff)
{
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, kSc1);
    return make_float4(__uint_as_float(v[0]), __uint_as_float(v[1]), __uint_as_float(v[2]), __uint_as_float(v[3]));
}
__device__ __forceinline__ int load_agent(const int *p)
{
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace

template <bool FUSE_D, bool HELP>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3))) void bwd_fused_d64_kernel(
    float *__restrict__ grad_x, float *__restrict__ dsw, int *__restrict__ ctl, const float *__restrict__ lse,
    float *__restrict__ Dv, const float *__restrict__ dy, const float *__restrict__ y, const float *__restrict__ qkv,
    int T, int C, int H, int bh0, int BHc, int n_qb, float c2, float scale, int n_cu, FusedSync sync)
{
    constexpr int ST = kTileRow;
    const int tid = threadIdx.x, lane = tid & 63, w = wave_id();
    const int c16 = lane & 15, g4 = lane >> 4;
    const int n_kg = (n_qb + 1) / 2;
    const uint32_t Wb = 12u * (uint32_t)C, Cb = 4u * (uint32_t)C, Hb = 4u * (uint32_t)H;
    const long tiles = (long)n_qb * (n_qb + 1) / 2;
    int *cnt = ctl + kCtlCounters;
    unsigned *orphan = reinterpret_cast<unsigned *>(ctl + kCtlCounters + kCtlItems);
    int *done = ctl + kCtlCounters + 2 * kCtlItems;

    // LDS: the dK/dV item's staging buffers (one array per buffer, so that
    // the compiler sees that loads landing in one buffer do not alias reads of
    // the other); the dQ item's 4 partials (32 x 64 each) reuse the Q and dO
    // tiles of both buffers
    constexpr int YT = FUSE_D ? 32 * ST : 4;
    __shared__ __attribute__((aligned(16))) float sq0[32 * ST], so0[32 * ST], sy0[YT], sld0[128];
    __shared__ __attribute__((aligned(16))) float sq1[32 * ST], so1[32 * ST], sy1[YT], sld1[128];

    // ------------------------------------------------------------ dK/dV item
    auto dkdv_item = [&](const int J, const int bhl) {
        const int bh = bh0 + bhl;
        const int b = bh / H, h = bh % H;
        const int kw0 = 64 * J + 16 * w;
        const rsrc_t rq = make_rsrc(qkv + (long)b * T * 3L * C + (long)h * 64,
                                    (uint32_t)(((long)T * 3 * C - (long)h * 64) * 4));
        const rsrc_t ro =
            make_rsrc(dy + (long)b * T * C + (long)h * 64, (uint32_t)(((long)T * C - (long)h * 64) * 4));
        const rsrc_t rl = make_rsrc(lse + (long)b * T * H + h, (uint32_t)(((long)T * H - h) * 4));
        // O (for the D rows, FUSE_D) or the D rows themselves
        const rsrc_t ryd = FUSE_D ? make_rsrc(y + (long)b * T * C + (long)h * 64,
                                              (uint32_t)(((long)T * C - (long)h * 64) * 4))
                                  : make_rsrc(Dv + (long)b * T * H + h, (uint32_t)(((long)T * H - h) * 4));
        float *ws = dsw + (long)bhl * tiles * 1024;
        float *gx_out = grad_x + (long)b * T * 3L * C + (long)h * 64;
        int *cnt_bh = cnt + (long)bhl * n_qb;

        auto bufs = [&](auto buf_c) {
            constexpr int buf = decltype(buf_c)::value;
            struct B
            {
                float *q, *o, *y, *ld;
            };
            return buf == 0 ? B{sq0, so0, sy0, sld0} : B{sq1, so1, sy1, sld1};
        };

        // stationary B operands: lane l holds K / V[kw0 + l%16][16 (l/16) + m]
        // K is requested first and V after the first block's staging, so that
        // the wait for that staging (vm_wait<4> below: all but the 4 V loads)
        // does not also wait for V, which the first dP MFMAs need only later
        // (C3 12-layer step, A/B: 0.9249 vs 0.9285 ms on one box, 0.9396 /
        // 0.9397 vs 0.9380 / 0.9433 ms on another)
        float kreg[16], vreg[16];
        const uint32_t kv_off = (uint32_t)c16 * Wb + 64u * g4;
#pragma unroll
        for (int c = 0; c < 4; ++c)
        {
            const float4 k4 = bload4s(rq, kv_off + Cb + 16u * c, (uint32_t)kw0 * Wb);
            kreg[4 * c + 0] = k4.x;
            kreg[4 * c + 1] = k4.y;
            kreg[4 * c + 2] = k4.z;
            kreg[4 * c + 3] = k4.w;
        }
        auto load_v = [&]() {
            __builtin_amdgcn_sched_barrier(0);  // after the staging loads, in issue order
#pragma unroll
            for (int c = 0; c < 4; ++c)
            {
                const float4 v4 = bload4s(rq, kv_off + 2u * Cb + 16u * c, (uint32_t)kw0 * Wb);
                vreg[4 * c + 0] = v4.x;
                vreg[4 * c + 1] = v4.y;
                vreg[4 * c + 2] = v4.z;
                vreg[4 * c + 3] = v4.w;
            }
            __builtin_amdgcn_sched_barrier(0);
        };

        // staging straight into LDS, as bwd_dkdv_d64_kernel: wave w moves chunks
        // w and w + 4 of Q and dO (and O with FUSE_D); wave 0 the lse (and D) rows
        const uint32_t dma_row = (uint32_t)(4 * w + (lane >> 4));
        const uint32_t dma_col = 16u * (uint32_t)((lane & 15) ^ (((lane >> 4) << 2) | w));
        const uint32_t dq_lane = dma_row * Wb + dma_col, do_lane = dma_row * Cb + dma_col;
        const uint32_t ld_lane = lane < 32 ? (uint32_t)lane * Hb : kNoBlock;
        const int i_lo = 2 * J;
        auto issue = [&](int i, auto buf_c) {
            const auto B = bufs(buf_c);
            const bool ok = i >= i_lo;
            const uint32_t qo = ok ? 32u * (uint32_t)i * Wb : kNoBlock, oo = ok ? 32u * (uint32_t)i * Cb : kNoBlock;
            dma16(rq, B.q + 256 * w, dq_lane, qo);
            dma16(rq, B.q + 256 * (w + 4), dq_lane + 16u * Wb, qo);
            dma16(ro, B.o + 256 * w, do_lane, oo);
            dma16(ro, B.o + 256 * (w + 4), do_lane + 16u * Cb, oo);
            if constexpr (FUSE_D)
            {
                dma16(ryd, B.y + 256 * w, do_lane, oo);
                dma16(ryd, B.y + 256 * (w + 4), do_lane + 16u * Cb, oo);
            }
            if (w == 0)
            {
                const uint32_t lo = ok ? 32u * (uint32_t)i * Hb : kNoBlock;
                dma4(rl, B.ld, ld_lane, lo);
                if constexpr (!FUSE_D)
                    dma4(ryd, B.ld + 64, ld_lane, lo);
            }
        };
        // D rows of block i from its staged dO and O (FUSE_D), as in
        // bwd_dkdv_d64_kernel; the key group whose diagonal blocks include i
        // (J = i / 2) also stores them.
        auto d_rows = [&](const int i, auto buf_c) {
            const auto B = bufs(buf_c);
            float dsum[2];
#pragma unroll
            for (int k = 0; k < 2; ++k)
            {
                const float4 o = *reinterpret_cast<const float4 *>(B.o + 256 * (w + 4 * k) + 4 * lane);
                const float4 u = *reinterpret_cast<const float4 *>(B.y + 256 * (w + 4 * k) + 4 * lane);
                dsum[k] = row16_sum(o.x * u.x + o.y * u.y + o.z * u.z + o.w * u.w);
            }
            if ((lane & 15) == 0)
            {
                const int r0 = 4 * w + (lane >> 4);
                B.ld[64 + r0] = dsum[0];
                B.ld[80 + r0] = dsum[1];
                if (i <= 2 * J + 1)
                {
                    const int q = 32 * i + r0;
                    if (q < T)
                        Dv[((long)b * T + q) * H + h] = dsum[0];
                    if (q + 16 < T)
                        Dv[((long)b * T + q + 16) * H + h] = dsum[1];
                }
            }
        };

        v4f dk0 = zero4(), dk1 = zero4(), dk2 = zero4(), dk3 = zero4();
        v4f dv0 = zero4(), dv1 = zero4(), dv2 = zero4(), dv3 = zero4();
        // blocks in walk order: n_qb - 1 down to i_lo; block i uses buffer
        // (i - i_lo) & 1, so the diagonal blocks (i_lo + 1, i_lo) always use
        // buffers 1 and 0
        const int i_top = n_qb - 1;
        if (((i_top - i_lo) & 1) == 0)
        {
            issue(i_top, BufIdx<0>{});
            load_v();
            vm_wait<4>();
            if constexpr (FUSE_D)
                d_rows(i_top, BufIdx<0>{});
        }
        else
        {
            issue(i_top, BufIdx<1>{});
            load_v();
            vm_wait<4>();
            if constexpr (FUSE_D)
                d_rows(i_top, BufIdx<1>{});
        }
        __syncthreads();
        int done_prev = -1;  // block whose dS stores the next barrier covers
        // One query block. GEN: a diagonal block (i = 2J, 2J + 1), which tests
        // for skipped tiles and zero halves and applies the causal mask.
        // Keys whose units a wave computes in a diagonal step, and halves it
        // leaves out: in the last step (block 2J) wave 2 takes wave 0's
        // second half (see below); otherwise every wave computes its own keys.
        int kwe_m = kw0;
        bool skip0_m = false, skip1_m = false;
        auto step = [&](const int i, auto buf_c, auto gen_c) {
            constexpr int buf = decltype(buf_c)::value;
            constexpr bool GEN = decltype(gen_c)::value;
            const int kwe = HELP ? kwe_m : kw0;
            const bool skip0 = HELP && skip0_m, skip1 = HELP && skip1_m;
            issue(i - 1, BufIdx<buf ^ 1>{});
            __builtin_amdgcn_sched_barrier(0);
            const int q0 = 32 * i;
            const auto Bf = bufs(buf_c);
            const float *Qs = Bf.q, *Os = Bf.o, *LDs = Bf.ld;
            float *tile = ws + ((long)i * (i + 1) / 2 + (kwe >> 5)) * 1024 + (kwe & 31) + c16 + (4 * g4) * 32;
            auto half = [&](auto t_c) {
                constexpr int t = decltype(t_c)::value;
                v4f sa = zero4(), pa = zero4();
#pragma unroll
                for (int c = 0; c < 4; ++c)
                {
                    const int ta = 16 * t * ST + tile_off(c16, 4 * g4 + c);
                    const float4 qa = *reinterpret_cast<const float4 *>(Qs + ta);
                    const float4 oa = *reinterpret_cast<const float4 *>(Os + ta);
                    const float qv[4] = {qa.x, qa.y, qa.z, qa.w}, ov[4] = {oa.x, oa.y, oa.z, oa.w};
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                    {
                        sa = mfma16(qv[e], kreg[4 * c + e], sa);
                        pa = mfma16(ov[e], vreg[4 * c + e], pa);
                    }
                }
                {
                    const float4 L = *reinterpret_cast<const float4 *>(LDs + 16 * t + 4 * g4);
                    const float4 D = *reinterpret_cast<const float4 *>(LDs + 64 + 16 * t + 4 * g4);
                    const float lv[4] = {L.x * kLog2e, L.y * kLog2e, L.z * kLog2e, L.w * kLog2e};
                    const float dv[4] = {D.x, D.y, D.z, D.w};
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                    {
                        const float p = fast_exp2(fmaf(sa[r], c2, -lv[r]));
                        sa[r] = p;
                        pa[r] = p * (pa[r] - dv[r]);
                    }
                    if (GEN && q0 + 16 * t < kwe + 15)
                    {
                        const int key = kwe + c16;
#pragma unroll
                        for (int r = 0; r < 4; ++r)
                            if (key > q0 + 16 * t + 4 * g4 + r)
                                sa[r] = pa[r] = 0.f;
                    }
                }
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    store_sc1(tile + (16 * t + r) * 32, pa[r]);
#pragma unroll
                for (int r = 0; r < 4; ++r)
                {
                    const int tb = tile_off(16 * t + 4 * g4 + r, c16);
                    const float4 ob = *reinterpret_cast<const float4 *>(Os + tb);
                    const float4 qb = *reinterpret_cast<const float4 *>(Qs + tb);
                    dv0 = mfma16(sa[r], ob.x, dv0);
                    dv1 = mfma16(sa[r], ob.y, dv1);
                    dv2 = mfma16(sa[r], ob.z, dv2);
                    dv3 = mfma16(sa[r], ob.w, dv3);
                    dk0 = mfma16(pa[r], qb.x, dk0);
                    dk1 = mfma16(pa[r], qb.y, dk1);
                    dk2 = mfma16(pa[r], qb.z, dk2);
                    dk3 = mfma16(pa[r], qb.w, dk3);
                }
            };
            // Both 16-query halves of the block at once, four interleaved
            // accumulator chains (S and dP of each half); MASK applies the
            // causal mask, for a diagonal block where this wave has units in
            // both halves.
            auto four = [&](auto mask_c) {
                constexpr bool MASK = decltype(mask_c)::value;
                v4f s0 = zero4(), s1 = zero4(), p0 = zero4(), p1 = zero4();
#pragma unroll
                for (int c = 0; c < 4; ++c)
                {
                    const int ta = tile_off(c16, 4 * g4 + c);
                    const float4 qa0 = *reinterpret_cast<const float4 *>(Qs + ta);
                    const float4 qa1 = *reinterpret_cast<const float4 *>(Qs + 16 * ST + ta);
                    const float4 oa0 = *reinterpret_cast<const float4 *>(Os + ta);
                    const float4 oa1 = *reinterpret_cast<const float4 *>(Os + 16 * ST + ta);
                    const float q0v[4] = {qa0.x, qa0.y, qa0.z, qa0.w}, q1v[4] = {qa1.x, qa1.y, qa1.z, qa1.w};
                    const float o0v[4] = {oa0.x, oa0.y, oa0.z, oa0.w}, o1v[4] = {oa1.x, oa1.y, oa1.z, oa1.w};
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                    {
                        s0 = mfma16(q0v[e], kreg[4 * c + e], s0);
                        s1 = mfma16(q1v[e], kreg[4 * c + e], s1);
                        p0 = mfma16(o0v[e], vreg[4 * c + e], p0);
                        p1 = mfma16(o1v[e], vreg[4 * c + e], p1);
                    }
                }
                {
                    const float4 L0 = *reinterpret_cast<const float4 *>(LDs + 4 * g4);
                    const float4 L1 = *reinterpret_cast<const float4 *>(LDs + 16 + 4 * g4);
                    const float4 D0 = *reinterpret_cast<const float4 *>(LDs + 64 + 4 * g4);
                    const float4 D1 = *reinterpret_cast<const float4 *>(LDs + 80 + 4 * g4);
                    const float l0v[4] = {L0.x * kLog2e, L0.y * kLog2e, L0.z * kLog2e, L0.w * kLog2e};
                    const float l1v[4] = {L1.x * kLog2e, L1.y * kLog2e, L1.z * kLog2e, L1.w * kLog2e};
                    const float d0v[4] = {D0.x, D0.y, D0.z, D0.w}, d1v[4] = {D1.x, D1.y, D1.z, D1.w};
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                    {
                        const float pa = fast_exp2(fmaf(s0[r], c2, -l0v[r])), pb = fast_exp2(fmaf(s1[r], c2, -l1v[r]));
                        s0[r] = pa;
                        p0[r] = pa * (p0[r] - d0v[r]);
                        s1[r] = pb;
                        p1[r] = pb * (p1[r] - d1v[r]);
                    }
                    if (MASK)
                    {
                        const int key = kwe + c16;
#pragma unroll
                        for (int r = 0; r < 4; ++r)
                        {
                            if (key > q0 + 4 * g4 + r)
                                s0[r] = p0[r] = 0.f;
                            if (key > q0 + 16 + 4 * g4 + r)
                                s1[r] = p1[r] = 0.f;
                        }
                    }
                }
#pragma unroll
                for (int r = 0; r < 4; ++r)
                {
                    store_sc1(tile + r * 32, p0[r]);
                    store_sc1(tile + (16 + r) * 32, p1[r]);
                }
#pragma unroll
                for (int t = 0; t < 2; ++t)
                {
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                    {
                        const int tb = tile_off(16 * t + 4 * g4 + r, c16);
                        const float4 ob = *reinterpret_cast<const float4 *>(Os + tb);
                        const float4 qb = *reinterpret_cast<const float4 *>(Qs + tb);
                        const float ap = t == 0 ? s0[r] : s1[r], ad = t == 0 ? p0[r] : p1[r];
                        dv0 = mfma16(ap, ob.x, dv0);
                        dv1 = mfma16(ap, ob.y, dv1);
                        dv2 = mfma16(ap, ob.z, dv2);
                        dv3 = mfma16(ap, ob.w, dv3);
                        dk0 = mfma16(ad, qb.x, dk0);
                        dk1 = mfma16(ad, qb.y, dk1);
                        dk2 = mfma16(ad, qb.z, dk2);
                        dk3 = mfma16(ad, qb.w, dk3);
                    }
                }
                __builtin_amdgcn_sched_barrier(0);
                vm_wait<8>();
            };
            if constexpr (GEN)
            {
                // A wave with units in both halves runs them as one step
                // (full grids: 12-layer C3 step 0.9189 / 0.9184 vs 0.9215 /
                // 0.9209 ms, outputs bitwise unchanged); the HELP instantiation
                // keeps the half-by-half form (with this form it spilled a
                // VGPR and lost 1 % at B = 8).
                if (!HELP && kwe < q0 + 16)
                {
                    if constexpr (!HELP)
                        four(BufIdx<1>{});
                }
                else if (kwe <= q0 + 31)
                {
                    if (kwe < q0 + 16)
                    {
                        if (!skip0)
                            half(BufIdx<0>{});
                    }
                    else
                    {
#pragma unroll
                        for (int r = 0; r < 4; ++r)
                            store_sc1(tile + r * 32, 0.f);
                    }
                    __builtin_amdgcn_sched_barrier(0);
                    if (!skip1)
                        half(BufIdx<1>{});
                    __builtin_amdgcn_sched_barrier(0);
                    vm_wait<8>();
                }
                else
                    lds_dma_wait();
            }
            else
                four(BufIdx<0>{});
            if constexpr (FUSE_D)
            {
                if (i - 1 >= i_lo)
                    d_rows(i - 1, BufIdx<buf ^ 1>{});
            }
            lds_barrier();
            // every wave's dS stores of the previous block are complete
            if (tid == 0 && done_prev >= 0)
                __hip_atomic_fetch_add(cnt_bh + done_prev, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            done_prev = i;
        };
        for (int i = i_top; i >= i_lo + 2; --i)
        {
            if ((i - i_lo) & 1)
                step(i, BufIdx<1>{}, BufIdx<0>{});
            else
                step(i, BufIdx<0>{}, BufIdx<0>{});
        }
        if (i_lo + 1 < n_qb)
            step(i_lo + 1, BufIdx<1>{}, BufIdx<1>{});
        if constexpr (HELP)
        {
            // register r of lane l: key kw0 + 4 g4 + r, dims 4 c16 + e
            auto store_rows = [&]() {
#pragma unroll
                for (int r = 0; r < 4; ++r)
                {
                    const int key = kw0 + 4 * g4 + r;
                    if (key < T)
                    {
                        float *dst = gx_out + (long)key * 3 * C + 4 * c16;
                        store4_nt(dst + C, make_float4(dk0[r] * scale, dk1[r] * scale, dk2[r] * scale, dk3[r] * scale));
                        store4_nt(dst + 2 * C, make_float4(dv0[r], dv1[r], dv2[r], dv3[r]));
                    }
                }
            };
            // Last step (block 2J, queries 64J .. 64J + 31): wave 0 (keys 64J ..
            // + 15) has two halves of work, wave 1 one, waves 2 and 3 (keys past
            // the block's queries) none. With HELP (the launcher takes it for
            // grids of at most 2 workgroups per CU, where no other workgroup's
            // waves fill that idle time), wave 2, whose keys are finished, stores
            // them, takes wave 0's K and V rows and computes wave 0's second half
            // from zero; wave 0 adds that partial after the step. (Step at B=8
            // T=256, 12 layers: 0.6684 vs 0.6762 ms; on full grids the same code
            // lost 0.6 % at C3 even switched off, so it is an instantiation of
            // its own.)
                if (w == 2)
            {
                store_rows();
                const uint32_t off = (uint32_t)c16 * Wb + 64u * g4;
                kwe_m = kw0 - 32;
#pragma unroll
                for (int c = 0; c < 4; ++c)
                {
                    const float4 k4 = bload4s(rq, off + Cb + 16u * c, (uint32_t)kwe_m * Wb);
                    const float4 v4 = bload4s(rq, off + 2u * Cb + 16u * c, (uint32_t)kwe_m * Wb);
                    kreg[4 * c + 0] = k4.x;
                    kreg[4 * c + 1] = k4.y;
                    kreg[4 * c + 2] = k4.z;
                    kreg[4 * c + 3] = k4.w;
                    vreg[4 * c + 0] = v4.x;
                    vreg[4 * c + 1] = v4.y;
                    vreg[4 * c + 2] = v4.z;
                    vreg[4 * c + 3] = v4.w;
                }
                dk0 = dk1 = dk2 = dk3 = zero4();
                dv0 = dv1 = dv2 = dv3 = zero4();
                skip0_m = true;
            }
            else if (w == 0)
                skip1_m = true;
            step(i_lo, BufIdx<0>{}, BufIdx<1>{});
            lds_dma_wait();
            lds_barrier();
            if (tid == 0)
                __hip_atomic_fetch_add(cnt_bh + done_prev, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            // wave 2's partial through buffer 1's Q tile (free: the last step
            // read buffer 0, and every wave's staging loads have landed)
            float4 *part = reinterpret_cast<float4 *>(sq1) + lane;
            if (w == 2)
            {
                const v4f acc[8] = {dk0, dk1, dk2, dk3, dv0, dv1, dv2, dv3};
#pragma unroll
                for (int k = 0; k < 8; ++k)
                    part[64 * k] = make_float4(acc[k][0], acc[k][1], acc[k][2], acc[k][3]);
            }
            lds_barrier();
            if (w == 0)
            {
                v4f *acc[8] = {&dk0, &dk1, &dk2, &dk3, &dv0, &dv1, &dv2, &dv3};
#pragma unroll
                for (int k = 0; k < 8; ++k)
                {
                    const float4 u = part[64 * k];
                    (*acc[k])[0] += u.x;
                    (*acc[k])[1] += u.y;
                    (*acc[k])[2] += u.z;
                    (*acc[k])[3] += u.w;
                }
            }
            if (w != 2)
                store_rows();
        }
        else
        {
            step(i_lo, BufIdx<0>{}, BufIdx<1>{});
            lds_dma_wait();
            lds_barrier();
            if (tid == 0)
                __hip_atomic_fetch_add(cnt_bh + done_prev, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

            // register r of lane l: key kw0 + 4 g4 + r, dims 4 c16 + e
#pragma unroll
            for (int r = 0; r < 4; ++r)
            {
                const int key = kw0 + 4 * g4 + r;
                if (key < T)
                {
                    float *dst = gx_out + (long)key * 3 * C + 4 * c16;
                    store4_nt(dst + C, make_float4(dk0[r] * scale, dk1[r] * scale, dk2[r] * scale, dk3[r] * scale));
                    store4_nt(dst + 2 * C, make_float4(dv0[r], dv1[r], dv2[r], dv3[r]));
                }
            }
        }
    };

    // --------------------------------------------------------------- dQ item
    // dQ of key group J's two diagonal blocks (2J + 1, 2J) as one item, once
    // both blocks' counters have reached the number of key groups that cover
    // them (J + 1; see the schedule): dQ_i = scale * sum_{j<=i} dS_ij K_j on
    // v_mfma_f32_32x32x2_f32, the units of block 2J + 1 then those of block
    // 2J split over the 4 waves in contiguous ranges (a wave's range may cover
    // both blocks: two sets of accumulators), one half-unit of operands ahead;
    // each block's 4 partials added through LDS in wave order.
    auto dq_both = [&](const int J, const int bhl) {
        const int bh = bh0 + bhl;
        const int b = bh / H, h = bh % H;
        const int n = lane & 31, hf = lane >> 5;
        const rsrc_t rk = make_rsrc(qkv + (long)b * T * 3L * C + C + (long)h * 64,
                                    (uint32_t)(((long)T * 3 * C - C - (long)h * 64) * 4));
        const rsrc_t rw = make_rsrc(dsw + (long)bhl * tiles * 1024, (uint32_t)(tiles * 4096));
        float *gq = grad_x + (long)b * T * 3L * C + (long)h * 64;
        const uint32_t w_lane = (uint32_t)n * 128u + 64u * hf;
        const uint32_t k_lane = 16u * hf * Wb + 8u * (uint32_t)n;
        const int qhi = 2 * J + 1, qlo = 2 * J;
        const int nhi = qhi < n_qb ? qhi + 1 : 0, nlo = qlo + 1;
        const int U = nhi + nlo, qd = U / 4, rm = U % 4;
        const int u0 = w * qd + (w < rm ? w : rm), nu = qd + (w < rm ? 1 : 0);
        // unit u of the combined list: block, key block
        auto tile_at = [&](int v) -> uint32_t {
            if (v >= nu)
                return kNoBlock;
            const int u = u0 + v;
            const int q = u < nhi ? qhi : qlo, j = u < nhi ? u : u - nhi;
            return ((uint32_t)q * (uint32_t)(q + 1) / 2u + (uint32_t)j) * 4096u;
        };
        auto key_at = [&](int v) -> uint32_t {
            if (v >= nu)
                return kNoBlock;
            const int u = u0 + v;
            const int j = u < nhi ? u : u - nhi;
            return 32u * (uint32_t)j * Wb;
        };
        float4 dsA[2], dsB[2];
        float2 kkA[8], kkB[8];
#define DQ_LOAD(DS, KK, v)                                                                                   \
    do                                                                                                       \
    {                                                                                                        \
        const int x_ = (v) & 1;                                                                              \
        const uint32_t to_ = tile_at((v) >> 1), ko_ = key_at((v) >> 1) + 8u * (uint32_t)x_ * Wb;             \
        _Pragma("unroll") for (int e = 0; e < 2; ++e) DS[e] = bload4s_sc1(rw, w_lane + 32u * x_ + 16u * e, to_); \
        _Pragma("unroll") for (int t = 0; t < 8; ++t) KK[t] = bload2s(rk, k_lane, ko_ + (uint32_t)t * Wb);    \
    } while (0)
#define DQ_MFMA(DS, KK, A0, A1)                                                                              \
    do                                                                                                       \
    {                                                                                                        \
        _Pragma("unroll") for (int e = 0; e < 2; ++e)                                                        \
        {                                                                                                    \
            A0 = mfma32(DS[e].x, KK[4 * e + 0].x, A0);                                                       \
            A1 = mfma32(DS[e].x, KK[4 * e + 0].y, A1);                                                       \
            A0 = mfma32(DS[e].y, KK[4 * e + 1].x, A0);                                                       \
            A1 = mfma32(DS[e].y, KK[4 * e + 1].y, A1);                                                       \
            A0 = mfma32(DS[e].z, KK[4 * e + 2].x, A0);                                                       \
            A1 = mfma32(DS[e].z, KK[4 * e + 2].y, A1);                                                       \
            A0 = mfma32(DS[e].w, KK[4 * e + 3].x, A0);                                                       \
            A1 = mfma32(DS[e].w, KK[4 * e + 3].y, A1);                                                       \
        }                                                                                                    \
    } while (0)
        v16f a0 = zero16(), a1 = zero16(), c0 = zero16(), c1 = zero16();
        DQ_LOAD(dsA, kkA, 0);
        __builtin_amdgcn_sched_barrier(0);
        for (int v = 0; v < 2 * nu; v += 2)
        {
            const bool hi = u0 + (v >> 1) < nhi;
            DQ_LOAD(dsB, kkB, v + 1);
            __builtin_amdgcn_sched_barrier(0);
            if (hi)
                DQ_MFMA(dsA, kkA, a0, a1);
            else
                DQ_MFMA(dsA, kkA, c0, c1);
            __builtin_amdgcn_sched_barrier(0);
            DQ_LOAD(dsA, kkA, v + 2);
            __builtin_amdgcn_sched_barrier(0);
            if (hi)
                DQ_MFMA(dsB, kkB, a0, a1);
            else
                DQ_MFMA(dsB, kkB, c0, c1);
            __builtin_amdgcn_sched_barrier(0);
        }
#undef DQ_LOAD
#undef DQ_MFMA
        // partials of the 4 waves added in a fixed order: register r of lane
        // (n, hf) holds dQ[32 qa + row(r, hf)][2n, 2n + 1]
        static_assert(32 * ST == 2048, "a partial fills one Q or dO tile");
        float *red = w == 0 ? sq0 : w == 1 ? so0 : w == 2 ? sq1 : so1;
        const float *parts[4] = {sq0, so0, sq1, so1};
        auto reduce = [&](const int qa, const v16f &x0, const v16f &x1) {
#pragma unroll
            for (int r = 0; r < 16; ++r)
                *reinterpret_cast<float2 *>(&red[mfma_row(r, hf) * 64 + 2 * n]) = make_float2(x0[r], x1[r]);
            __syncthreads();
#pragma unroll
            for (int k = 0; k < 2; ++k)
            {
                const int e = tid + 256 * k, row = 32 * qa + (e >> 4);
                float4 s = reinterpret_cast<const float4 *>(parts[0])[e];
#pragma unroll
                for (int ww = 1; ww < 4; ++ww)
                {
                    const float4 u = reinterpret_cast<const float4 *>(parts[ww])[e];
                    s.x += u.x;
                    s.y += u.y;
                    s.z += u.z;
                    s.w += u.w;
                }
                if (row < T)
                    store4_nt(gq + (long)row * 3 * C + 4 * (e & 15),
                              make_float4(s.x * scale, s.y * scale, s.z * scale, s.w * scale));
            }
            __syncthreads();
        };
        if (nhi > 0)
            reduce(qhi, a0, a1);
        reduce(qlo, c0, c1);
    };

    // ---------------------------------------------------------- dQ claims
    // Whether a dQ item's counts are complete, by thread 0 of the workgroup:
    // both blocks' counters (block 2J + 1 only if it exists) at `need` or
    // more, waiting at most `ticks` of wall-clock time (then false).
    auto counts_complete = [&](const int *cnt_b, const int J, const int need, const long long ticks) {
        const int qhi = 2 * J + 1, qlo = 2 * J;
        const long long t0 = (long long)wall_clock64();
        for (;;)
        {
            const int c_lo = load_agent(cnt_b + qlo);
            const int c_hi = qhi < n_qb ? load_agent(cnt_b + qhi) : need;
            if (c_lo >= need && c_hi >= need)
                return true;
            if ((long long)wall_clock64() - t0 > ticks)
                return false;
            __builtin_amdgcn_s_sleep(2);
        }
    };
    // back to 0 once every bump of this launch has landed
    auto release = [&](int *cnt_b, const int J) {
        if (tid == 0)
        {
            const int qhi = 2 * J + 1, qlo = 2 * J;
            __hip_atomic_fetch_add(cnt_b + qlo, -(J + 1), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (qhi < n_qb)
                __hip_atomic_fetch_add(cnt_b + qhi, -(J + 1), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    };
    __shared__ int s_run;

    // ------------------------------------------------------------ schedule
    if ((int)blockIdx.x >= sync.n_main)
    {
        // Orphan runner r of the grid's last kOrphanRunners workgroups, for
        // (b, h) pairs bh_lo .. bh_hi - 1: once every main workgroup of them
        // has decided (their done counters reach the key-group count), run
        // their orphans, then release the done counters.
        __shared__ int s_list[256], s_n;
        const int runners = (int)gridDim.x - sync.n_main, r = (int)blockIdx.x - sync.n_main;
        const int per = (BHc + runners - 1) / runners;
        const int bh_lo = r * per, bh_hi = bh_lo + per < BHc ? bh_lo + per : BHc;
        for (int bh = bh_lo + tid; bh < bh_hi; bh += 256)
        {
            const long long t0 = (long long)wall_clock64();
            while (load_agent(done + bh) < n_kg)
            {
                if ((long long)wall_clock64() - t0 > sync.done_ticks)
                {
                    __hip_atomic_fetch_add(ctl + kCtlWaitErrors, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    break;
                }
                __builtin_amdgcn_s_sleep(8);
            }
        }
        if (tid == 0)
            s_n = 0;
        __syncthreads();
        for (int base = bh_lo * n_kg; base < bh_hi * n_kg; base += 256)
        {
            const int idx = base + tid;
            if (idx < bh_hi * n_kg &&
                __hip_atomic_load(orphan + idx, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == sync.epoch)
                s_list[atomicAdd(&s_n, 1)] = idx;
            __syncthreads();
            const int n = s_n;
            for (int k = 0; k < n; ++k)
            {
                const int item = s_list[k], J = item % n_kg, bhl = item / n_kg;
                int *cnt_b = cnt + (long)bhl * n_qb;
                if (tid == 0 && !counts_complete(cnt_b, J, J + 1 + sync.need_extra, sync.safety_ticks))
                    __hip_atomic_fetch_add(ctl + kCtlWaitErrors, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                __syncthreads();
                dq_both(J, bhl);
                release(cnt_b, J);
            }
            __syncthreads();
            if (tid == 0)
                s_n = 0;
            __syncthreads();
        }
        // back to 0 once every main workgroup's count has landed
        for (int bh = bh_lo + tid; bh < bh_hi; bh += 256)
            __hip_atomic_fetch_add(done + bh, -n_kg, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return;
    }
    // Main workgroup: the dK/dV item of this workgroup: J-major, heaviest
    // first, (b, h) fastest; when the whole grid is resident at 3 per CU,
    // CU c hosts workgroups c, c + n_cu, c + 2 n_cu, and the middle round
    // takes its items in reverse (in blocks of 8, which keeps each (b, h) on
    // one XCD), so that every CU gets one heavy, one light and one middle
    // item; grids of 1 to 2 workgroups per CU pair them (paired_item: the
    // heaviest key groups alone on their CUs, the others heavy with light)
    {
        int item = (int)blockIdx.x;
        const int G = sync.n_main;
        if (n_cu > 0 && n_cu % 8 == 0 && G % n_cu == 0 && G / n_cu <= 3)
        {
            const int r = item / n_cu;
            int c = item % n_cu;
            if (r & 1)
                c = (n_cu / 8 - 1 - c / 8) * 8 + (c & 7);
            item = r * n_cu + c;
        }
        int J = item / BHc, bhl = item % BHc;
        if constexpr (HELP)  // grids of at most 2 workgroups per CU
        {
            int cls = 0, idx = 0;
            if (paired_item((int)blockIdx.x, G, n_cu, BHc, &cls, &idx))
            {
                J = cls;
                bhl = idx;
            }
        }
        // Wave priority by weight: the heaviest key groups (the longest chains
        // of steps) issue first, so that their chains run at about a lone
        // wave's speed while the lighter items fill the gaps (12-layer step,
        // A/B on one box: heavy first 1.052 ms, no priorities 1.055 ms, light
        // first 1.121 ms).
        {
            const int pr = n_kg - 1 - J;
            if (pr >= 3)
                __builtin_amdgcn_s_setprio(3);
            else if (pr == 2)
                __builtin_amdgcn_s_setprio(2);
            else if (pr == 1)
                __builtin_amdgcn_s_setprio(1);
        }
        dkdv_item(J, bhl);
        // dQ of this key group's own diagonal blocks (2J + 1, then 2J), at
        // the lowest priority (see above). Key group 0's blocks 0 and 1 take
        // dS from key group 0 alone, whose stores completed before the
        // barrier that ended its walk: no wait. Otherwise thread 0 waits a
        // bounded time for the counts; if they are still short, the item
        // becomes an orphan (flag stored, its completion awaited, before the
        // done counter moves, so a runner that sees the count sees the flag).
        __builtin_amdgcn_s_setprio(0);
        int *cnt_b = cnt + (long)bhl * n_qb;
        if (tid == 0)
        {
            bool run = true;
            if (J > 0 && !counts_complete(cnt_b, J, J + 1 + sync.need_extra, sync.wait_ticks))
            {
                run = false;
                const unsigned old =
                    __hip_atomic_exchange(orphan + (long)bhl * n_kg + J, sync.epoch, __ATOMIC_RELAXED,
                                          __HIP_MEMORY_SCOPE_AGENT);
                asm volatile("" ::"v"(old));  // the flag is in place before the done counter moves
            }
            __hip_atomic_fetch_add(done + bhl, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            s_run = run;
        }
        __syncthreads();  // the decision is out; the dK/dV item's LDS is free
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        if (__builtin_amdgcn_readfirstlane(s_run))
        {
            dq_both(J, bhl);
            release(cnt_b, J);
        }
    }
}

// Launches the HELP instantiation (grids of at most 2 workgroups per CU); in
// attn_bwd_fused_help.hip, a translation unit of its own so that each
// instantiation is compiled with the scheduling that measured fastest for it.
hipError_t launch_bwd_fused_d64_help(dim3 g, float *grad_x, float *ws, int *ctl, const float *lse, float *D,
                                     const float *dy, const float *y, const float *qkv, int T, int C, int H,
                                     int BH, int n_qb, float c2, float scale, int n_cu, const FusedSync &sync,
                                     hipStream_t st);

}  // namespace gpt_attn

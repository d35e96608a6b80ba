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
// head_dim 64 path: deterministic, no atomics, no memset; two launches up to
// T = 256, three beyond. Work unit = one 32-query block i x one 32-key block
// j with j <= i.
//   bwd_rowdot_d64_kernel  (T > 256) D rows, one float4 per thread, 16 lanes
//                          per (row, head).
//   bwd_dkdv_d64_kernel    one workgroup per (b, h, 64-key group); each of its
//                          4 waves keeps 16 keys' K, V rows in registers and
//                          walks the query blocks i >= its group on
//                          v_mfma_f32_16x16x4_f32:
//                            S  = Q K^T, dP = dO V^T   (queries x keys)
//                            P = 2^(S c - L), dS = P (dP - D)
//                            dV += P^T dO, dK += dS^T Q
//                          stores its part of the dS tiles to a workspace and
//                          writes its dK, dV rows once (nothing to reduce).
//                          Up to T = 256 it also computes the D rows.
//   bwd_dq_d64_kernel      one workgroup per (b, h, heavy/light query-block
//                          pair): dQ_i = sum_{j<=i} dS_ij K_j from the
//                          workspace on v_mfma_f32_32x32x2_f32, written once.
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

// D rows for head_dim 64: D[r, h] = sum over the head's 64 columns of
// dO * O. The [rows, 64 H] tensors are read as one flat stream of float4s,
// one per thread: the 16 lanes of a DPP row cover one (row, head) (64
// columns) and sum their products with 4 DPP adds.
__global__ __launch_bounds__(256) void bwd_rowdot_d64_kernel(float *__restrict__ Dout,
                                                             const float *__restrict__ dy,
                                                             const float *__restrict__ y, long n4)
{
    const long f = (long)blockIdx.x * 256 + threadIdx.x;  // float4 index; n4 is a multiple of 16
    if (f >= n4)
        return;
    const float4 u = reinterpret_cast<const float4 *>(dy)[f], v = reinterpret_cast<const float4 *>(y)[f];
    const float s = row16_sum(u.x * v.x + u.y * v.y + u.z * v.z + u.w * v.w);
    if ((threadIdx.x & 15) == 0)
        Dout[f >> 4] = s;
}

// Offset (floats) of dS tile (i, j), j <= i, inside one (b, h)'s workspace.
__device__ __forceinline__ long ds_tile(int i, int j) { return ((long)i * (i + 1) / 2 + j) * 1024; }

// dK, dV and the dS tiles, K/V-stationary. One workgroup per (b, h, 64-key
// group J); wave w owns the 16 keys kw0 = 64 J + 16 w .. kw0 + 15: their K and
// V rows stay in registers as MFMA B operands and their dK, dV accumulate in
// registers, so no wave shares an output with another and nothing is reduced.
// The 4 waves walk the query blocks i = 2J .. n - 1 together; each block's Q,
// dO (32 x 64) and lse, D rows are staged once in LDS for all 4 waves (double
// buffered: block i + 1 is loaded into registers while block i is computed,
// then written to the other buffer; one barrier per block). Per wave and query
// block, on v_mfma_f32_16x16x4_f32 (two 16-row query halves t):
//   S_t = Q_t K^T, dP_t = dO_t V^T          (16 queries x 16 keys, 16 MFMAs each)
//   P = 2^(S c - L), dS = P (dP - D)        (masked past the diagonal and T)
//   dV += P^T dO, dK += dS^T Q              (S / dP accumulators are the A
//                                            operands as they are; 4 d-tiles)
// and the wave's 32 x 16 half of dS tile (i, kw0 / 32) is stored. Workgroups
// are ordered key-group-major (heaviest first), (b, h) fastest.
template <bool FUSE_D>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3))) void bwd_dkdv_d64_kernel(
    float *__restrict__ grad_x, float *__restrict__ dsw, const float *__restrict__ lse,
    float *__restrict__ Dv, const float *__restrict__ dy, const float *__restrict__ y, const float *__restrict__ qkv,
    int T, int C, int H, int bh0, int BHc, int n_qb, float c2, float scale, int n_cu)
{
    constexpr int ST = kTileRow;
    const int tid = threadIdx.x, lane = tid & 63, w = wave_id();
    const int c16 = lane & 15, g4 = lane >> 4;
    // Work item = (key group J, (b, h)), heaviest first: J-major, (b, h)
    // fastest. When the whole grid is resident (at most 3 workgroups per CU),
    // workgroup c, c + n_cu and c + 2 n_cu share a CU (round-robin dispatch),
    // so the middle round takes the items in reverse order (in blocks of 8,
    // which keeps every (b, h) on one XCD): each CU then gets one heavy, one
    // light and one middle item instead of three of a kind.
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
    const int J = item / BHc;
    const int bhl = item % BHc, bh = bh0 + bhl;
    const int b = bh / H, h = bh % H;
    // Key slice of this wave. The 16-key slices do unequal work on the
    // diagonal blocks (slice 0 computes 4 of the 16-query halves there, slice
    // 3 one). When the grid is resident, each SIMD of a CU hosts one wave of
    // each of the CU's workgroups (c, c + n_cu, c + 2 n_cu), and choosing
    // the slice by the wave's SIMD with a different table per round evens
    // the SIMDs' diagonal work (7 or 8 halves each, instead of anything from
    // 3 to 12 when slices follow wave indices); measured 44.1 -> 43.7 us at
    // C3, no gain on larger grids, which keep slices = wave indices. The
    // choice needs the workgroup's 4 waves on 4 different SIMDs, which is
    // checked through LDS; otherwise slices follow wave indices too.
    int slice = w;
    if (n_cu > 0 && (int)gridDim.x <= 3 * n_cu)
    {
        __shared__ int sid[4];
        if (lane == 0)
            sid[w] = (__builtin_amdgcn_s_getreg(4 | (4 << 6) | (1 << 11))) & 3;  // HW_ID[5:4] = SIMD id
        lds_barrier();
        const int simd = sid[w];
        if (((1 << sid[0]) | (1 << sid[1]) | (1 << sid[2]) | (1 << sid[3])) == 0xF)
        {
            // slice per SIMD for rounds 0, 1, 2 (diagonal halves 4, 3, 2, 1 by slice):
            // per-SIMD sums 4+1+2, 3+2+3, 2+4+1, 1+3+4
            const int r = (int)blockIdx.x / n_cu;
            constexpr int kSlice[3][4] = {{0, 1, 2, 3}, {3, 2, 0, 1}, {2, 1, 3, 0}};
            slice = kSlice[r][simd];
        }
    }
    const int kw0 = 64 * J + 16 * slice;
    const uint32_t Wb = 12u * (uint32_t)C, Cb = 4u * (uint32_t)C, Hb = 4u * (uint32_t)H;
    const rsrc_t rq = make_rsrc(qkv + (long)b * T * 3L * C + (long)h * 64,
                                (uint32_t)(((long)T * 3 * C - (long)h * 64) * 4));
    const rsrc_t ro = make_rsrc(dy + (long)b * T * C + (long)h * 64, (uint32_t)(((long)T * C - (long)h * 64) * 4));
    const rsrc_t rl = make_rsrc(lse + (long)b * T * H + h, (uint32_t)(((long)T * H - h) * 4));
    const rsrc_t ry = make_rsrc(y + (long)b * T * C + (long)h * 64, (uint32_t)(((long)T * C - (long)h * 64) * 4));
    const rsrc_t rd = make_rsrc(Dv + (long)b * T * H + h, (uint32_t)(((long)T * H - h) * 4));
    float *ws = dsw + (long)bhl * ((long)n_qb * (n_qb + 1) / 2) * 1024;
    float *gx = grad_x + (long)b * T * 3L * C + (long)h * 64;

    // Q, dO of the block, swizzled (tile_off), with FUSE_D O of the block
    // (laid out as dO, read only by the lane that staged it), and its lse
    // (0..31) and D (64..95) rows; one array per buffer, so that the compiler
    // sees that loads landing in one buffer do not alias reads of the other
    constexpr int YT = FUSE_D ? 32 * ST : 4;
    __shared__ __attribute__((aligned(16))) float sq0[32 * ST], so0[32 * ST], sy0[YT], sld0[128];
    __shared__ __attribute__((aligned(16))) float sq1[32 * ST], so1[32 * ST], sy1[YT], sld1[128];
    auto bufs = [&](auto buf_c) {
        constexpr int buf = decltype(buf_c)::value;
        struct B
        {
            float *q, *o, *y, *ld;
        };
        return buf == 0 ? B{sq0, so0, sy0, sld0} : B{sq1, so1, sy1, sld1};
    };

    // stationary B operands: lane l holds K / V[kw0 + l%16][16 (l/16) + m],
    // m = 0..15 (MFMA m contracts d = m + 16 kk, kk = l/16)
    float kreg[16], vreg[16];
    {
        const uint32_t off = (uint32_t)c16 * Wb + 64u * g4;
#pragma unroll
        for (int c = 0; c < 4; ++c)
        {
            const float4 k4 = bload4s(rq, off + Cb + 16u * c, (uint32_t)kw0 * Wb);
            const float4 v4 = bload4s(rq, off + 2u * Cb + 16u * c, (uint32_t)kw0 * Wb);
            kreg[4 * c + 0] = k4.x;
            kreg[4 * c + 1] = k4.y;
            kreg[4 * c + 2] = k4.z;
            kreg[4 * c + 3] = k4.w;
            vreg[4 * c + 0] = v4.x;
            vreg[4 * c + 1] = v4.y;
            vreg[4 * c + 2] = v4.z;
            vreg[4 * c + 3] = v4.w;
        }
    }

    // Staging goes straight from memory into LDS (buffer loads to LDS, no
    // registers). A 32 x 64 tile is 8 chunks of 1 KiB, chunk k = rows
    // 4k .. 4k + 3; wave w moves chunks w and w + 4 of Q and of dO. Lane l
    // lands at row 4k + l/16, physical column group l%16, so it fetches the
    // logical group (l%16) ^ tile_swz(row), tile_swz(row) = (l/16) << 2 | w for
    // both of its chunks. With FUSE_D, O moves like dO (for the D rows);
    // otherwise wave 0 moves the block's D rows (from bwd_rowdot_d64_kernel).
    // Wave 0 also moves the lse rows of the block.
    const uint32_t dma_row = (uint32_t)(4 * w + (lane >> 4));
    const uint32_t dma_col = 16u * (uint32_t)((lane & 15) ^ (((lane >> 4) << 2) | w));
    const uint32_t dq_lane = dma_row * Wb + dma_col, do_lane = dma_row * Cb + dma_col;
    // lse / D rows: lanes 0..31 fetch rows 0..31, lanes 32..63 land zeros
    const uint32_t ld_lane = lane < 32 ? (uint32_t)lane * Hb : kNoBlock;
    auto issue = [&](int i, auto buf_c) {
        const auto B = bufs(buf_c);
        const bool ok = i < n_qb;
        const uint32_t qo = ok ? 32u * (uint32_t)i * Wb : kNoBlock, oo = ok ? 32u * (uint32_t)i * Cb : kNoBlock;
        dma16(rq, B.q + 256 * w, dq_lane, qo);
        dma16(rq, B.q + 256 * (w + 4), dq_lane + 16u * Wb, qo);
        dma16(ro, B.o + 256 * w, do_lane, oo);
        dma16(ro, B.o + 256 * (w + 4), do_lane + 16u * Cb, oo);
        if constexpr (FUSE_D)
        {
            dma16(ry, B.y + 256 * w, do_lane, oo);
            dma16(ry, B.y + 256 * (w + 4), do_lane + 16u * Cb, oo);
        }
        if (w == 0)
        {
            const uint32_t lo = ok ? 32u * (uint32_t)i * Hb : kNoBlock;
            dma4(rl, B.ld, ld_lane, lo);
            if constexpr (!FUSE_D)
                dma4(rd, B.ld + 64, ld_lane, lo);
        }
    };
    // D rows of block i, D = rowsum(dO * O), once its staging has landed:
    // each lane multiplies the dO and O float4s it staged itself (rows
    // 4 w + l/16 and 16 + 4 w + l/16, so no barrier is needed before the
    // reads), the 16 lanes of a row add them up, and the row's lane 0 writes
    // D into the buffer's D rows (made visible by the barrier that ends the
    // step). Every workgroup of a (b, h) computes a block's D the same way;
    // the one whose first two blocks include it (J = i / 2) also stores it.
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
    const int i_lo = 2 * J;
    issue(i_lo, BufIdx<0>{});
    lds_dma_wait();
    if constexpr (FUSE_D)
        d_rows(i_lo, BufIdx<0>{});
    __syncthreads();
    // One query block; the LDS buffer index is a compile-time constant (the
    // loop below is unrolled by two) so that it folds into the ds_read offsets.
    // Only a workgroup's first two blocks (i = 2J, 2J + 1) can hold keys past
    // queries, so only they (GEN) test for skipped tiles, zero halves and the
    // causal mask; every later block is a full unmasked tile for every wave,
    // a loop without branches (a branch around the dS stores would also make
    // the compiler's waits for the staging loads pessimistic).
    auto step = [&](const int i, auto buf_c, auto gen_c) {
        constexpr int buf = decltype(buf_c)::value;
        constexpr bool GEN = decltype(gen_c)::value;
        issue(i + 1, BufIdx<buf ^ 1>{});
        __builtin_amdgcn_sched_barrier(0);
        const int q0 = 32 * i;
        const auto Bf = bufs(buf_c);
        const float *Qs = Bf.q, *Os = Bf.o, *LDs = Bf.ld;
        // (dS tiles with the non-temporal hint: the dQ kernel reads each once;
        // C4 -0.5 %, C5a -0.9 %, while non-temporal loads of them in the dQ
        // kernel measured 5 % slower)
        float *tile = ws + ds_tile(i, kw0 >> 5) + (kw0 & 31) + c16 + (4 * g4) * 32;
        // Half t of the tile: queries q0 + 16 t .. + 15 against this wave's
        // 16 keys, done start to end (S, dP, P, dS, its dS rows, dV and dK)
        // before the other half, so only one half's accumulators are live.
        auto half = [&](auto t_c) {
            constexpr int t = decltype(t_c)::value;
            // S[query q0 + 16t + 4 g4 + r][key kw0 + c16], dP likewise
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
            // P and dS (without the 1/sqrt(d)); zero where key > query. Rows
            // past T need no mask: their Q, dO, lse and D load as zeros, so
            // P = 1 and dS = 0 there and they add nothing to dK, dV or dQ.
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
                if (GEN && q0 + 16 * t < kw0 + 15)  // some key of this wave lies past some query of the half
                {
                    const int key = kw0 + c16;
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        if (key > q0 + 16 * t + 4 * g4 + r)
                            sa[r] = pa[r] = 0.f;
                }
            }
            // this wave's 16 x 16 quarter of dS tile (i, kw0 / 32), query-major
#pragma unroll
            for (int r = 0; r < 4; ++r)
                __builtin_nontemporal_store(pa[r], &tile[(16 * t + r) * 32]);
            // dV += P^T dO, dK += dS^T Q: step r contracts queries
            // q0 + 16t + 4kk + r (kk = l/16); B operands dO / Q[that query][4 c16 + e]
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
        // then wait until block i + 1 has landed in the other buffer: its
        // loads were issued before this block's 8 dS stores, if any
        if constexpr (GEN)
        {
            if (kw0 <= q0 + 31)  // else all 16 keys lie past this block's last query: no tile
            {
                if (kw0 < q0 + 16)
                    half(BufIdx<0>{});
                else  // kw0 = q0 + 16: every key lies past the first 16 queries, whose dS rows are zero
                {
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        __builtin_nontemporal_store(0.f, &tile[r * 32]);
                }
                __builtin_amdgcn_sched_barrier(0);
                half(BufIdx<1>{});
                __builtin_amdgcn_sched_barrier(0);
                vm_wait<8>();
            }
            else
                lds_dma_wait();
        }
        else
        {
            // full unmasked tile, both halves at once (four independent
            // S / dP accumulator chains)
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
            }
#pragma unroll
            for (int r = 0; r < 4; ++r)
            {
                __builtin_nontemporal_store(p0[r], &tile[r * 32]);
                __builtin_nontemporal_store(p1[r], &tile[(16 + r) * 32]);
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
        }
        if constexpr (FUSE_D)
        {
            if (i + 1 < n_qb)
                d_rows(i + 1, BufIdx<buf ^ 1>{});
        }
        lds_barrier();
    };
    step(i_lo, BufIdx<0>{}, BufIdx<1>{});
    if (i_lo + 1 < n_qb)
        step(i_lo + 1, BufIdx<1>{}, BufIdx<1>{});
    int i = i_lo + 2;
    for (; i + 1 < n_qb; i += 2)
    {
        step(i, BufIdx<0>{}, BufIdx<0>{});
        step(i + 1, BufIdx<1>{}, BufIdx<0>{});
    }
    if (i < n_qb)
        step(i, BufIdx<0>{}, BufIdx<0>{});

    // register r of lane l: key kw0 + 4 g4 + r, dims 4 c16 + e (accumulator e)
#pragma unroll
    for (int r = 0; r < 4; ++r)
    {
        const int key = kw0 + 4 * g4 + r;
        if (key < T)
        {
            float *dst = gx + (long)key * 3 * C + 4 * c16;
            store4_nt(dst + C, make_float4(dk0[r] * scale, dk1[r] * scale, dk2[r] * scale, dk3[r] * scale));
            store4_nt(dst + 2 * C, make_float4(dv0[r], dv1[r], dv2[r], dv3[r]));
        }
    }
}

// dQ_i = scale * sum_{j<=i} dS_ij K_j. One workgroup per (b, h, query-block
// pair (n - 1 - p, p)). Each block's units (its key blocks 0..i) are split
// into 4 contiguous ranges, one per wave (spare units of the heavy block go to
// the first waves, of the light block to the last, so that no wave gets two),
// and every dS tile and K block is loaded once. A wave walks its heavy range,
// then its light range, as one stream on v_mfma_f32_32x32x2_f32 (16 MFMAs
// per half-unit of 16 keys, whose operands are loaded one half-unit ahead),
// keeping its partial dQ (32 x 64) of the current block in registers; the 4
// waves' partials are added through LDS at the end, in a fixed order, and
// the blocks' rows are stored. Workgroups are ordered pair-major with
// (b, h) fastest, the same (b, h) -> XCD mapping as the dK/dV kernel, so a
// (b, h)'s dS tiles are read from the L2 they were written to.
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3))) void bwd_dq_d64_kernel(float *__restrict__ grad_x,
                                                         const float *__restrict__ dsw,
                                                         const float *__restrict__ qkv,
                                                         int T, int C, int H, int bh0, int BHc, int n_qb,
                                                         float scale)
{
    const int tid = threadIdx.x, lane = tid & 63, w = wave_id();
    const int n = lane & 31, hf = lane >> 5;
    const int pr = (int)(blockIdx.x / BHc);  // this workgroup's pair
    const int bhl = (int)(blockIdx.x % BHc), bh = bh0 + bhl;
    const int b = bh / H, h = bh % H;
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

    // this wave's key blocks: [ja0, ja1) of block qa, then [jb0, jb1) of block pr
    auto range = [](int cnt, int slot, int &j0, int &j1) {
        const int q = cnt / 4, r = cnt % 4;
        j0 = slot * q + (slot < r ? slot : r);
        j1 = j0 + q + (slot < r ? 1 : 0);
    };
    int ja0, ja1, jb0 = 0, jb1 = 0;
    range(qa + 1, w, ja0, ja1);
    if (two)
        range(pr + 1, 3 - w, jb0, jb1);
    const int na = ja1 - ja0, nu = na + (jb1 - jb0);
    // unit v of the wave's stream (branch-free, wave-uniform, in SGPRs)
    const uint32_t base_a = ((uint32_t)qa * (uint32_t)(qa + 1) / 2u + (uint32_t)ja0) * 4096u;
    const uint32_t base_b = ((uint32_t)pr * (uint32_t)(pr + 1) / 2u + (uint32_t)jb0 - (uint32_t)na) * 4096u;
    auto tile_at = [&](int v) -> uint32_t {
        const uint32_t o = (v < na ? base_a : base_b) + (uint32_t)v * 4096u;
        return v < nu ? o : kNoBlock;
    };
    auto key_at = [&](int v) -> uint32_t {
        const int j = v < na ? ja0 + v : jb0 + v - na;
        return v < nu ? 32u * (uint32_t)j * Wb : kNoBlock;
    };

    // Half-units: half x (x = 0, 1) of a unit contracts keys 16 hf + 8 x + t
    // (t = 0..7) for k-slot hf, in 16 MFMAs; its operands are
    //   ds[e] = dS[n][16 hf + 8 x + 4 e ..]  (e = 0, 1; MFMA A operand)
    //   kk[t] = K[32 j + 16 hf + 8 x + t][2n, 2n + 1]  (B operand)
    // and are prefetched one half-unit ahead (two sets, 24 VGPRs each).
    float4 dsA[2], dsB[2];
    float2 kkA[8], kkB[8];
#define DQ_LOAD(DS, KK, v)                                                        \
    do                                                                            \
    {                                                                             \
        const int x_ = (v) & 1;                                                   \
        const uint32_t to_ = tile_at((v) >> 1), ko_ = key_at((v) >> 1) + 8u * (uint32_t)x_ * Wb; \
        _Pragma("unroll") for (int e = 0; e < 2; ++e) DS[e] = bload4s(rw, w_lane + 32u * x_ + 16u * e, to_); \
        _Pragma("unroll") for (int t = 0; t < 8; ++t) KK[t] = bload2s(rk, k_lane, ko_ + (uint32_t)t * Wb); \
    } while (0)
#define DQ_MFMA(DS, KK)                                                           \
    do                                                                            \
    {                                                                             \
        _Pragma("unroll") for (int e = 0; e < 2; ++e)                             \
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
    // half-units [v0, v1) of the stream (v1 - v0 even); the first is already
    // loaded into set A, and the one after the last is left loaded in set A
    auto run = [&](int v0, int v1) {
        for (int v = v0; v < v1; v += 2)
        {
            DQ_LOAD(dsB, kkB, v + 1);
            __builtin_amdgcn_sched_barrier(0);
            DQ_MFMA(dsA, kkA);
            __builtin_amdgcn_sched_barrier(0);
            DQ_LOAD(dsA, kkA, v + 2);
            __builtin_amdgcn_sched_barrier(0);
            DQ_MFMA(dsB, kkB);
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    // Partials: register r of lane (n, hf) holds dQ[32 i + row(r, hf)][2n, 2n + 1].
    // Each wave parks its heavy-block partial in its LDS slot when it moves
    // on to the light block (no barrier there), and the blocks are added
    // over the 4 slots only at the end, in a fixed order: thread tid adds
    // float4s tid, tid + 256 of the 32 x 64 block.
    __shared__ __attribute__((aligned(16))) float red[4][32 * 64];
    auto park = [&]() {
#pragma unroll
        for (int r = 0; r < 16; ++r)
            *reinterpret_cast<float2 *>(&red[w][mfma_row(r, hf) * 64 + 2 * n]) = make_float2(a0[r], a1[r]);
    };
    auto sum_store = [&](int i) {
#pragma unroll
        for (int k = 0; k < 2; ++k)
        {
            const int e = tid + 256 * k, row = 32 * i + (e >> 4);
            float4 s = reinterpret_cast<const float4 *>(red[0])[e];
#pragma unroll
            for (int ww = 1; ww < 4; ++ww)
            {
                const float4 x = reinterpret_cast<const float4 *>(red[ww])[e];
                s.x += x.x;
                s.y += x.y;
                s.z += x.z;
                s.w += x.w;
            }
            if (row < T)
                store4_nt(gx + (long)row * 3 * C + 4 * (e & 15),
                          make_float4(s.x * scale, s.y * scale, s.z * scale, s.w * scale));
        }
    };

    DQ_LOAD(dsA, kkA, 0);
    __builtin_amdgcn_sched_barrier(0);
    run(0, 2 * na);
    park();
    if (two)
    {
        a0 = zero16();
        a1 = zero16();
        run(2 * na, 2 * nu);
    }
    __syncthreads();
    sum_store(qa);
    if (two)
    {
        __syncthreads();
        park();
        __syncthreads();
        sum_store(pr);
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

size_t bwd_d64_workspace_bytes(const Shape &s, size_t cap, int *bh_per_chunk)
{
    const long n_qb = (s.T + 31) / 32;
    const size_t per_bh = (size_t)(n_qb * (n_qb + 1) / 2) * 4096;
    const long BH = (long)s.B * s.H;
    if (per_bh > cap)
    {
        if (bh_per_chunk)
            *bh_per_chunk = 0;
        return per_bh;
    }
    long chunk = (long)(cap / per_bh);
    chunk = chunk > BH ? BH : chunk;
    if (bh_per_chunk)
        *bh_per_chunk = (int)chunk;
    return per_bh * (size_t)chunk;
}

hipError_t launch_bwd_rowdot_d64(float *D, const float *dy, const float *y, const Shape &s, hipStream_t st)
{
    const long n4 = (long)s.B * s.T * 16L * s.H;
    launch_timed(kKindRowdot, bwd_rowdot_d64_kernel, dim3((unsigned)((n4 + 255) / 256)), dim3(256), st, D, dy, y,
                 n4);
    return hipGetLastError();
}

int device_cu_count()
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

hipError_t launch_bwd_d64(float *grad_x, float *D, const float *lse, const float *dy, const float *y,
                          const float *qkv, float *ws, int bh_per_chunk, const Shape &s, hipStream_t st)
{
    // D rows inside the dK/dV kernel while few key groups recompute a block's
    // D (T <= 256: at most 4): one launch less, measured backward 70.9 ->
    // 68.2 us at B=16 T=256, 37.2 -> 35.9 us at B=1 T=256; at T = 512 the
    // two ways measure the same and at T = 4096 (64 key groups) the separate
    // D-row pass is as fast or faster, so longer rows keep it.
    const bool fuse_d = s.T <= 256;
    hipError_t e = hipSuccess;
    if (!fuse_d)
    {
        e = launch_bwd_rowdot_d64(D, dy, y, s, st);
        if (e != hipSuccess)
            return e;
    }
    const int n_qb = (s.T + 31) / 32;
    const int BH = s.B * s.H;
    const float scale = softmax_scale(64);
    for (int bh0 = 0; bh0 < BH; bh0 += bh_per_chunk)
    {
        const int cnt = BH - bh0 < bh_per_chunk ? BH - bh0 : bh_per_chunk;
        const dim3 g((unsigned)((long)((s.T + 63) / 64) * cnt));
        if (fuse_d)
            launch_timed(kKindDkdv, bwd_dkdv_d64_kernel<true>, g, dim3(256), st, grad_x, ws, lse, D, dy, y, qkv, s.T,
                         s.C, s.H, bh0, cnt, n_qb, scale * kLog2e, scale, device_cu_count());
        else
            launch_timed(kKindDkdv, bwd_dkdv_d64_kernel<false>, g, dim3(256), st, grad_x, ws, lse, D, dy, y, qkv,
                         s.T, s.C, s.H, bh0, cnt, n_qb, scale * kLog2e, scale, device_cu_count());
        const unsigned dq_blocks = (unsigned)((long)((n_qb + 1) / 2) * cnt);  // one workgroup per pair
        launch_timed(kKindDq, bwd_dq_d64_kernel, dim3(dq_blocks), dim3(256), st, grad_x, ws, qkv, s.T, s.C, s.H,
                     bh0, cnt, n_qb, scale);
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

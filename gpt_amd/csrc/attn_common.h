// Shared definitions for the gfx950 causal-attention kernels.
//
// Tensor layouts are the reference's (src/backend/backend_interface.h:161-184):
//   qkv [B, T, 3C] (Q | K | V, head h at column h*d of each third),
//   y [B, T, C], lse / D [B, T, H], grad_x [B, T, 3C].
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "attn_addr.h"

namespace gpt_attn {

typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
// Lazy online-softmax rescaling: probabilities are taken against a reference
// max that may lag the running max by up to this much (log2 units), so they
// stay <= 2^8 and fp32 sums of them cannot overflow for any T < 2^100.
constexpr float kLazyRescale = 8.f;

// LDS row stride (floats) for the 64-wide fp32 tiles of the 32x32x2 kernels:
// their row reads (one row per lane of a half-wave) measured free of bank
// conflicts at 64 + 4 words.
constexpr int kRowStride = 68;

// LDS layout of the 32 x 64 fp32 tiles of the 16x16x4 kernels. gfx950's LDS
// has 64 banks x 4 bytes and serves a ds_read_b128 in four phases of 16
// lanes: within each half-wave, first the lanes whose quad index
// (lane >> 2) & 7 has even parity, then those with odd parity (measured with
// SQ_LDS_BANK_CONFLICT on pairs of lanes reading the same bank). A phase is
// conflict-free when its 16 lanes hit 16 distinct 4-bank groups. Rows are 64
// words and the 16-byte column group cg of row `row` is stored at
// cg ^ tile_swz(row); both tile reads of these kernels, (row = lane % 16,
// cg = 4 (lane / 16) + c) and (row = 4 (lane / 16) + r, cg = lane % 16),
// and the staging writes (row = tid / 16, cg = tid % 16) are then
// conflict-free (measured: zero conflict cycles; the same reads at a stride of
// 68 words take two cycles per phase).
constexpr int kTileRow = 64;
__device__ __forceinline__ int tile_swz(int row) { return ((row & 3) << 2) | ((row >> 2) & 3); }
// word offset of column group cg (4 floats) of a row in a swizzled tile
__device__ __forceinline__ int tile_off(int row, int cg) { return row * kTileRow + 4 * (cg ^ tile_swz(row)); }

// v_mfma_f32_32x32x2_f32: D[32x32] += A[32x2] * B[2x32].
// Lane l supplies A[l%32][l/32] and B[l/32][l%32]; it holds accumulator
// element D[row(r, l/32)][l%32] in register r (see mfma_row).
__device__ __forceinline__ v16f mfma32(float a, float b, v16f c)
{
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

// v_mfma_f32_16x16x4_f32: D[16x16] += A[16x4] * B[4x16]. Lane l supplies
// A[l%16][l/16] and B[l/16][l%16]; register r of lane l holds
// D[4 * (l/16) + r][l%16] (checked on gfx950 with a one-hot probe).
__device__ __forceinline__ v4f mfma16(float a, float b, v4f c)
{
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ v4f zero4()
{
    v4f z;
    z[0] = z[1] = z[2] = z[3] = 0.f;
    return z;
}

// Row index of accumulator register r for a lane in half `hf` (= lane / 32).
__device__ __forceinline__ constexpr int mfma_row(int r, int hf)
{
    return 8 * (r >> 2) + 4 * hf + (r & 3);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float fast_log2(float x) { return __builtin_amdgcn_logf(x); }

// Value held by lane l ^ 32 (the other half of the wave64).
__device__ __forceinline__ float swap_halves(float x) { return __shfl_xor(x, 32, 64); }

// v_permlane32_swap with both operands = x: element 0 is x of lane l % 32
// (the lower half's value), element 1 is x of lane 32 + l % 32 (the upper
// half's value), in every lane. A VALU op, unlike the LDS bpermute that
// __shfl_xor(x, 32) becomes.
__device__ __forceinline__ float2 halves(float x)
{
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return make_float2(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// max / sum of x over lanes l and l ^ 32, the same bits in both lanes
// (lower-half operand first).
__device__ __forceinline__ float halves_max(float x)
{
    const float2 p = halves(x);
    return fmaxf(p.x, p.y);
}
__device__ __forceinline__ float halves_sum(float x)
{
    const float2 p = halves(x);
    return p.x + p.y;
}

// v_permlane16_swap with both operands = x: element 0 is x of lane l & ~16,
// element 1 is x of lane l | 16 (the two 16-lane rows of each 32-lane half),
// in both lanes of the pair (checked on gfx950).
__device__ __forceinline__ float2 rows16(float x)
{
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return make_float2(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// max / sum of x over lanes l and l ^ 16, the same bits in both lanes.
__device__ __forceinline__ float rows16_max(float x)
{
    const float2 p = rows16(x);
    return fmaxf(p.x, p.y);
}
__device__ __forceinline__ float rows16_sum(float x)
{
    const float2 p = rows16(x);
    return p.x + p.y;
}

// x of another lane of the same 16-lane DPP row (CTRL: a gfx9 DPP control,
// e.g. 0x140 row_mirror: lane 15 - i; 0x141 row_half_mirror: lane 7 - i within
// each 8-lane half; 0x4E quad_perm [2,3,0,1]: lane i ^ 2; 0xB1 quad_perm
// [1,0,3,2]: lane i ^ 1). A VALU op, unlike the LDS bpermute of __shfl_xor.
template <int CTRL> __device__ __forceinline__ float dpp_row(float x)
{
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, false));
}

// Sum of x over the 16 lanes of the DPP row, in every lane of the row (the
// lanes add in different orders, so they may differ in the last bits; each
// lane's result is the same from run to run). After the two mirrors lanes
// 0..3 hold the sums of {0,15,7,8}, {1,14,6,9}, {2,13,5,10}, {3,12,4,11}
// (lanes 4..7 the same groups in reverse, the upper half likewise), which
// the two quad permutations add up.
__device__ __forceinline__ float row16_sum(float x)
{
    x += dpp_row<0x140>(x);
    x += dpp_row<0x141>(x);
    x += dpp_row<0x4E>(x);
    x += dpp_row<0xB1>(x);
    return x;
}

// Compiler-level ordering point between one wave's LDS writes and its reads
// of other lanes' values (a wave's LDS instructions execute in issue order).
__device__ __forceinline__ void wave_lds_sync()
{
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Raw buffer resource over `bytes` bytes starting at `base` (stride 0, the
// gfx9 word-3 for untyped 32-bit data). A load whose VGPR offset lies at or
// past `bytes` returns zeros instead of touching memory, which is how the
// kernels read rows past T: no clamps, no branches.
// The base and size must be wave-uniform; they are passed through
// readfirstlane so that the descriptor stays in SGPRs even where the compiler
// has computed the address arithmetic in VGPRs (a descriptor it cannot prove
// uniform turns every load into a waterfall loop).
typedef __amdgpu_buffer_rsrc_t rsrc_t;
__device__ __forceinline__ rsrc_t make_rsrc(const void *base, uint32_t bytes)
{
    // (readfirstlane is int -> int; join_words zero-extends the low word)
    const uint64_t a = reinterpret_cast<uint64_t>(base);
    const uint64_t u = join_words(__builtin_amdgcn_readfirstlane((int)(uint32_t)(a >> 32)),
                                  __builtin_amdgcn_readfirstlane((int)(uint32_t)a));
    return __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void *>(u), (short)0,
                                             __builtin_amdgcn_readfirstlane((int)bytes), 0x00020000);
}
// Buffer offset used for a block that does not exist: past the end of every
// buffer range the kernels build (the host only takes the buffer-load kernels
// for tensors below 2^31 bytes per batch slice, and lane offsets inside a
// block stay far below 2^31), so such a load returns zeros and touches no
// memory. Lets software-pipelined loops issue the same loads every iteration.
constexpr uint32_t kNoBlock = 0x80000000u;

__device__ __forceinline__ float4 bload4(rsrc_t r, uint32_t off)
{
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0);
    return make_float4(__uint_as_float(v[0]), __uint_as_float(v[1]), __uint_as_float(v[2]), __uint_as_float(v[3]));
}
__device__ __forceinline__ float2 bload2(rsrc_t r, uint32_t off)
{
    const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, (int)off, 0, 0);
    return make_float2(__uint_as_float(v[0]), __uint_as_float(v[1]));
}
__device__ __forceinline__ float bload1(rsrc_t r, uint32_t off)
{
    return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, 0));
}

// Loads straight into LDS (buffer_load ... lds): lane l's 4 or 16 bytes land
// at lds + 4 l or lds + 16 l bytes (checked on gfx950; the global side may
// be any per-lane offset). `lds` must be wave-uniform. The loads count in
// vmcnt like any other; lds_dma_wait() waits for this wave's to land, and a
// workgroup barrier after it makes them visible to the other waves. Offsets
// past the buffer's range land as zeros, as for register loads.
__device__ __forceinline__ void dma16(rsrc_t r, float *lds, uint32_t voff, uint32_t soff)
{
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void *)lds, 16, (int)voff,
                                             (int)soff, 0, 0);
}
__device__ __forceinline__ void dma4(rsrc_t r, float *lds, uint32_t voff, uint32_t soff)
{
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void *)lds, 4, (int)voff,
                                             (int)soff, 0, 0);
}
// s_waitcnt vmcnt(N) (expcnt and lgkmcnt left at their maxima; N < 16). On
// gfx9 vector memory operations, loads and stores alike, retire in issue
// order, so vmcnt(N) waits for everything but the N most recent ones: a wave
// that issued N stores after its loads to LDS waits for those loads alone.
template <int N>
__device__ __forceinline__ void vm_wait()
{
    static_assert(N >= 0 && N < 16, "vmcnt field");
    __builtin_amdgcn_s_waitcnt(0x0F70 | N);
}
__device__ __forceinline__ void lds_dma_wait() { vm_wait<0>(); }

// Workgroup barrier that orders LDS only: it waits for this wave's LDS
// operations alone. On gfx950 outside thread-group split mode
// __syncthreads() compiles to the same code (its workgroup-scope fences need
// no vmcnt wait there, so neither waits for outstanding global stores); this
// form states the intent. Loads to LDS count in vmcnt and must be waited for
// (vm_wait) before it.
__device__ __forceinline__ void lds_barrier()
{
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// The same loads with a wave-uniform part of the offset in an SGPR (soffset).
// gfx950's range check applies to voffset + soffset + the immediate, so rows
// past the range still read as zeros, and block / row bases cost no VGPRs.
__device__ __forceinline__ float4 bload4s(rsrc_t r, uint32_t voff, uint32_t soff)
{
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, 0);
    return make_float4(__uint_as_float(v[0]), __uint_as_float(v[1]), __uint_as_float(v[2]), __uint_as_float(v[3]));
}
__device__ __forceinline__ float2 bload2s(rsrc_t r, uint32_t voff, uint32_t soff)
{
    const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, (int)voff, (int)soff, 0);
    return make_float2(__uint_as_float(v[0]), __uint_as_float(v[1]));
}
__device__ __forceinline__ float bload1s(rsrc_t r, uint32_t voff, uint32_t soff)
{
    return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, (int)voff, (int)soff, 0));
}

// 16-byte store with the non-temporal hint, for results no later work of the
// launch reads (the backward's dQ, dK, dV rows): they stream out instead of
// taking L2 / MALL lines from the Q, dO, O and K blocks the other key groups
// read again (C3 12-layer step 0.964 -> 0.929-0.937 ms, C2 -2.5 %, C4 -1 %;
// the forward's O, which the backward reads back, measured 10 % slower so).
__device__ __forceinline__ void store4_nt(float *p, float4 v)
{
    typedef float f4 __attribute__((ext_vector_type(4)));
    const f4 x = {v.x, v.y, v.z, v.w};
    __builtin_nontemporal_store(x, reinterpret_cast<f4 *>(p));
}

// 16-byte buffer store at device scope (sc1): written through the XCD's L2
// to memory. Callers arrange that one instruction covers whole rows (16 lanes
// x 16 bytes of one 256-byte row each): with 16-byte pieces scattered over
// many lines the write-throughs are partial and slow (C3 forward 27.7 us
// against 24.2 us for plain stores), with whole rows the launch ends without
// a writeback of dirty lines.
__device__ __forceinline__ void store4_sc1(rsrc_t r, uint32_t voff, float4 v)
{
    typedef unsigned u4 __attribute__((ext_vector_type(4)));
    const u4 x = {__float_as_uint(v.x), __float_as_uint(v.y), __float_as_uint(v.z), __float_as_uint(v.w)};
    __builtin_amdgcn_raw_buffer_store_b128(x, r, (int)voff, 0, 16);
}

// Index of the calling wave in its workgroup, as a value the compiler knows
// to be wave-uniform (so offsets derived from it can live in SGPRs).
// Compile-time index (of an LDS double buffer) passed to generic lambdas.
template <int N>
struct BufIdx
{
    static constexpr int value = N;
};

__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)); }

// Item of workgroup b in a grid of G workgroups, n_cu < G <= 2 n_cu, whose
// items come in classes of `per_class` items each, class 0 the heaviest.
// The dispatcher puts workgroups b and n_cu + b on the same CU (b < G - n_cu)
// and every other workgroup alone on its CU, and workgroup b on XCD b % 8.
// Within each XCD (items with index = b mod 8) the heaviest items get the
// single CUs and the rest are paired heaviest with lightest, so that the
// heaviest CU carries as little as the classes allow (B = 8, T = 256: 12 %
// less time for the forward and for the backward). Returns false where the
// shapes do not allow it (then the caller keeps its own order).
__device__ __forceinline__ bool paired_item(int b, int G, int n_cu, int per_class, int *cls, int *idx)
{
    if (n_cu <= 0 || n_cu % 8 != 0 || per_class % 8 != 0 || G <= n_cu || G > 2 * n_cu || G % per_class != 0)
        return false;
    const int m = n_cu / 8, g = G / 8, pairs = g - m, singles = 2 * m - g, pc = per_class / 8;
    int p, r;
    if (b < n_cu)
    {
        const int u = b / 8;
        r = b % 8;
        p = u >= pairs ? u - pairs : singles + u;  // single, or the heavy item of pair u
    }
    else
    {
        const int u = (b - n_cu) / 8;
        r = (b - n_cu) % 8;
        p = g - 1 - u;  // the light item of pair u
    }
    *cls = p / pc;
    *idx = 8 * (p % pc) + r;
    return true;
}

__device__ __forceinline__ v16f zero16()
{
    v16f z;
#pragma unroll
    for (int i = 0; i < 16; ++i)
        z[i] = 0.f;
    return z;
}

}  // namespace gpt_attn

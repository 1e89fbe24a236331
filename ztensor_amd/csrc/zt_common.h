// Shared device helpers for the gfx950 quantized GEMV kernels.
//
// Conventions used by every kernel in this library:
//  * A weight matrix has `rows` output rows and K input columns and is stored
//    row-major ([rows, K]); quantization blocks/groups run along K.
//  * Activations B are [K, N] (element (k, n) at B[k*N + n]) and the output
//    C is [rows, N] (element (r, n) at C[r*N + n]); N is the batch.  For
//    N == 1 both are plain vectors.  This is the C = dequant(A) * B
//    convention of the kernel-runner GEMMs this library stands in for.
//  * Launchers return a hipError_t as int (0 = success), allocate nothing
//    and launch asynchronously on the caller's stream.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#include "zt_hip.h"

#define ZT_EXPORT extern "C" __attribute__((visibility("default")))

namespace zt {

constexpr int kWave = 64;

// Workgroups of a 1-D grid of G go to the 8 XCDs in turn (workgroup b to XCD
// b mod 8).  This maps b to a logical index so that each XCD takes one
// contiguous range of logical indices (the first G mod 8 XCDs one more):
// neighbouring logical workgroups then share one XCD's L2.
__device__ __forceinline__ int xcd_contiguous(int b, int G) {
    const int x = b & 7, i = b >> 3, per = G >> 3, rem = G & 7;
    return x < rem ? x * (per + 1) + i : rem * (per + 1) + (x - rem) * per + i;
}

// fp16 bits -> fp32, exact widening (v_cvt_f32_f16; fp16 denormals are kept).
__device__ __forceinline__ float h2f(uint16_t h) {
    return __half2float(__ushort_as_half(h));
}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// A dequantized value as stored: fp32 as is, or fp16 bits rounded to
// nearest, ties to even (v_cvt_f16_f32 in the default rounding mode).
template <class OutT>
__device__ __forceinline__ OutT out_cvt(float v);
template <>
__device__ __forceinline__ float out_cvt<float>(float v) { return v; }
template <>
__device__ __forceinline__ uint16_t out_cvt<uint16_t>(float v) { return __half_as_ushort(__float2half_rn(v)); }

// 128-bit streaming load of weight data that is read exactly once: the
// nontemporal hint keeps it from evicting the reused activations.
__device__ __forceinline__ uint4 ld_stream(const uint4* p) {
    u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

// Cross-lane exchange steps of wave_reduce_rows.  For a pair (a, b) of
// per-lane values, pair_step<OFF> returns, in lanes whose bit OFF is clear,
// a + a(partner) and, in lanes whose bit OFF is set, b + b(partner), where
// the partner lane differs from the caller in bit OFF.
//  * OFF 32 / 16: v_permlane32_swap / v_permlane16_swap exchange the upper
//    half of `a` with the lower half of `b`, so a' + b' is exactly that sum
//    with no per-lane select;
//  * OFF 8 / 4 / 2 / 1: a DPP row_mirror / row_half_mirror / quad_perm move
//    (partners 15-l, 7-l, l^2, l^1 inside a 16-lane row; each flips bit OFF)
//    fused into the add, with two mask selects choosing what is kept and sent.
template <int OFF>
__device__ __forceinline__ float pair_step(float a, float b) {
    if constexpr (OFF == 32 || OFF == 16) {
        const uint32_t ua = __float_as_uint(a), ub = __float_as_uint(b);
        auto r = (OFF == 32) ? __builtin_amdgcn_permlane32_swap(ua, ub, false, false)
                             : __builtin_amdgcn_permlane16_swap(ua, ub, false, false);
        return __uint_as_float(r[0]) + __uint_as_float(r[1]);
    } else {
        constexpr uint64_t m = OFF == 8 ? 0xFF00FF00FF00FF00ull
                             : OFF == 4 ? 0xF0F0F0F0F0F0F0F0ull
                             : OFF == 2 ? 0xCCCCCCCCCCCCCCCCull : 0xAAAAAAAAAAAAAAAAull;
        constexpr int ctrl = OFF == 8 ? 0x140 : OFF == 4 ? 0x141 : OFF == 2 ? 0x4E : 0xB1;
        float keep, send;
        asm("v_cndmask_b32_e64 %0, %1, %2, %3" : "=v"(keep) : "v"(a), "v"(b), "s"(m));
        asm("v_cndmask_b32_e64 %0, %1, %2, %3" : "=v"(send) : "v"(b), "v"(a), "s"(m));
        return keep + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(send), ctrl, 0xF, 0xF, false));
    }
}

// One value: v + v(partner) in every lane.
template <int OFF>
__device__ __forceinline__ float single_step(float v) {
    if constexpr (OFF == 32 || OFF == 16) {
        return pair_step<OFF>(v, v);
    } else {
        constexpr int ctrl = OFF == 8 ? 0x140 : OFF == 4 ? 0x141 : OFF == 2 ? 0x4E : 0xB1;
        return v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), ctrl, 0xF, 0xF, false));
    }
}

template <int R, int OFF>
__device__ __forceinline__ void reduce_level(float (&v)[R]) {
    if constexpr (OFF >= 1) {
        constexpr int c = R * OFF / 32 > 1 ? R * OFF / 32 : 1;  // live values per lane at this level
        if constexpr (c > 1) {
#pragma unroll
            for (int i = 0; i < c / 2; i++) v[i] = pair_step<OFF>(v[i], v[c / 2 + i]);
        } else {
            v[0] = single_step<OFF>(v[0]);
        }
        reduce_level<R, OFF / 2>(v);
    }
}

// Sum R per-lane values across a wave64.  After the call, every lane l holds
// the full sum of value index row_of_lane<R>(l) in v[0].  The first log2(R)
// steps halve the number of live values per lane (each lane keeps one half
// and trades the other with its partner), so the reduction costs R-1 +
// log2(64/R) exchange-and-add steps instead of 6*R.
template <int R>
__device__ __forceinline__ void wave_reduce_rows(float (&v)[R]) {
    static_assert(R >= 1 && R <= 32 && (R & (R - 1)) == 0, "R must be a power of two <= 32");
    reduce_level<R, 32>(v);
}

// Which value index lane l holds after wave_reduce_rows<R>.
template <int R>
__device__ __forceinline__ int row_of_lane(int lane) {
    int r = 0, off = 32;
#pragma unroll
    for (int c = R; c > 1; c >>= 1, off >>= 1)
        if (lane & off) r += c / 2;
    return r;
}

// Lanes 0 .. 64/R-1 of each group hold duplicates; lane is the writer for
// its value index iff it is the lowest lane of its group.
template <int R>
__device__ __forceinline__ bool is_row_writer(int lane) {
    return (lane & (kWave / R - 1)) == 0;
}

// Cross-wave combine of per-wave row sums through LDS and the final store.
// red must hold nwaves*R floats.
template <int R>
__device__ __forceinline__ void block_reduce_store(float (&acc)[R], float* red, float* __restrict__ y,
                                                   long y_stride, int row0, int rows) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nwaves = blockDim.x >> 6;
    wave_reduce_rows<R>(acc);
    if (nwaves == 1) {
        if (is_row_writer<R>(lane)) {
            int r = row0 + row_of_lane<R>(lane);
            if (r < rows) y[(long)r * y_stride] = acc[0];
        }
        return;
    }
    if (is_row_writer<R>(lane)) red[wave * R + row_of_lane<R>(lane)] = acc[0];
    __syncthreads();
    if ((int)threadIdx.x < R) {
        float s = 0.0f;
        for (int w = 0; w < nwaves; w++) s += red[w * R + threadIdx.x];
        int r = row0 + threadIdx.x;
        if (r < rows) y[(long)r * y_stride] = s;
    }
}

__host__ __forceinline__ int ceil_div(long a, long b) { return (int)((a + b - 1) / b); }

// Rows per wave: the largest R in {1,2,4,8} that still gives at least
// `target` waves over the grid, so small matrices spread over all 256 CUs
// while big ones keep several 16-byte loads in flight per lane.
__host__ __forceinline__ int pick_rows_per_wave(long rows, int waves_per_group, long batch, long target) {
    int R = 8;
    while (R > 1 && ((rows + R - 1) / R) * waves_per_group * batch < target) R >>= 1;
    return R;
}

}  // namespace zt

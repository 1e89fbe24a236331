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

// fp16 bits -> fp32, exact widening (v_cvt_f32_f16; fp16 denormals are kept).
__device__ __forceinline__ float h2f(uint16_t h) {
    return __half2float(__ushort_as_half(h));
}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// 128-bit streaming load of weight data that is read exactly once: the
// nontemporal hint keeps it from evicting the reused activations.
__device__ __forceinline__ uint4 ld_stream(const uint4* p) {
    u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

// Sum R per-lane values across a wave64.  After the call, lane l holds the
// full sum of value index row_of_lane<R>(l) in v[0].  The first log2(R)
// exchange steps halve the number of live values per lane (each lane keeps
// one half and ships the other to its partner), so the whole reduction costs
// R-1 + log2(64/R) shuffles instead of 6*R.
template <int R>
__device__ __forceinline__ void wave_reduce_rows(float (&v)[R]) {
    const int lane = threadIdx.x & 63;
    int off = 32;
#pragma unroll
    for (int c = R; c > 1; c >>= 1, off >>= 1) {
        const bool upper = (lane & off) != 0;
#pragma unroll
        for (int i = 0; i < c / 2; i++) {
            float keep = upper ? v[c / 2 + i] : v[i];
            float send = upper ? v[i] : v[c / 2 + i];
            v[i] = keep + __shfl_xor(send, off, 64);
        }
    }
    for (; off >= 1; off >>= 1) v[0] += __shfl_xor(v[0], off, 64);
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

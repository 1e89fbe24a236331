// Ternary {-1, 0, +1} GEMV for gfx950.
//
// Weight format: 2 bits per weight, code 00 = -1, 01 = 0, 10 = +1, element
// j of a byte at bits 2*(j%4) (tensor/ternary_storage.go:5-62).  The device
// layout is the row-aligned one the GPU path uploads
// (compute/ternary_gemv_gpu.go:52-67): row r occupies bytes
// [r*bpr, (r+1)*bpr) with bpr = ceil(K/4); pad bits of a row's last byte
// are zero (code 00), so activations past K are treated as 0.
//
// Two kernels:
//  * f32 activations (the reference's TernaryGEMV / ternary_gemv_f32
//    contract, compute/ternary_gemv.go:12-64): each 2-bit code c is
//    converted with v_cvt_f32_ubyte and sum (c-1) x = sum c x - sum x;
//  * int8 activations with a per-tensor weight scale and a per-token
//    activation scale (BitNet decode): integer dot products with
//    v_dot4_i32_i8 on the codes, y = float(sum c q - sum q) * (w_scale *
//    x_scale).  The integer sum is exact, so the result is bit-identical to
//    the fp32 reference reduction (whose partial sums are exact integers).
//
// Work split: a lane owns CB consecutive bytes of a row (4*CB weights);
// CB = 16 when bpr % 16 == 0 (one 128-bit load), 4 when bpr % 4 == 0, else
// 1.  Its activations stay in registers while the wave walks R rows; waves of
// a workgroup split K and combine through LDS.  With K % 64 == 0 (every
// BitNet shape) both activation types take a fixed-step form of the same
// split (ternary_i8_steps_kernel, ternary_f32_steps_kernel) with every load
// issued first; f32 activations up to K = 16384 take the quad mapping
// instead (ternary_f32_quad_kernel: four lanes a 16-byte chunk, a dword of
// codes and 16 activations a lane).
#include "zt_common.h"

namespace zt {

template <int CB>
__device__ __forceinline__ void load_codes(const uint8_t* __restrict__ p, uint32_t (&w)[(CB + 3) / 4]) {
    if constexpr (CB == 16) {
        const uint4 v = ld_stream(reinterpret_cast<const uint4*>(p));
        w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
    } else if constexpr (CB == 4) {
        w[0] = __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(p));
    } else {
        w[0] = *p;
    }
}

// ----------------------------------------------------------- int8 x

template <int CB, int R>
__global__ void __launch_bounds__(512) ternary_i8_kernel(const uint8_t* __restrict__ W, const int8_t* __restrict__ xq,
                                                         const float* __restrict__ x_scale,
                                                         const float* __restrict__ w_scale, float* __restrict__ y,
                                                         int rows, int K, int bpr) {
    constexpr int ND = (CB + 3) / 4;  // weight dwords per lane
    __shared__ float red[8 * R];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nwaves = blockDim.x >> 6;
    const int nchunk = bpr / CB;
    const int row0 = blockIdx.x * R;
    const float scale = w_scale[0] * x_scale[0];  // issued first: its latency overlaps the weight stream
    long rbase[R];
#pragma unroll
    for (int r = 0; r < R; r++) rbase[r] = (long)min(row0 + r, rows - 1) * bpr;

    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.0f;

    for (int c = wave * kWave + lane; c < nchunk; c += nwaves * kWave) {
        uint32_t w[R][ND];
#pragma unroll
        for (int r = 0; r < R; r++) load_codes<CB>(W + rbase[r] + (long)c * CB, w[r]);
        // xd[i][t] holds activations 16i+4t .. 16i+4t+3 (zero past K);
        // xp[i][s] packs activations 16i+s, 16i+4+s, 16i+8+s, 16i+12+s: the
        // order in which (w >> 2s) & 0x03030303 lays out the codes of dword i.
        const int k0 = c * CB * 4;
        uint32_t xd[ND][4];
        if (k0 + 4 * CB <= K && (CB == 1 || ((uintptr_t)(xq + k0) & 15) == 0)) {
            if constexpr (CB == 16) {
#pragma unroll
                for (int i = 0; i < ND; i++) {
                    const uint4 v = *reinterpret_cast<const uint4*>(xq + k0 + 16 * i);
                    xd[i][0] = v.x; xd[i][1] = v.y; xd[i][2] = v.z; xd[i][3] = v.w;
                }
            } else if constexpr (CB == 4) {
                const uint4 v = *reinterpret_cast<const uint4*>(xq + k0);
                xd[0][0] = v.x; xd[0][1] = v.y; xd[0][2] = v.z; xd[0][3] = v.w;
            } else {
                xd[0][0] = (uint32_t)(uint8_t)xq[k0] | ((uint32_t)(uint8_t)xq[k0 + 1] << 8) |
                           ((uint32_t)(uint8_t)xq[k0 + 2] << 16) | ((uint32_t)(uint8_t)xq[k0 + 3] << 24);
                xd[0][1] = xd[0][2] = xd[0][3] = 0;
            }
        } else {
#pragma unroll
            for (int i = 0; i < ND; i++)
#pragma unroll
                for (int t = 0; t < 4; t++) {
                    uint32_t v = 0;
#pragma unroll
                    for (int b = 0; b < 4; b++) {
                        const int e = 16 * i + 4 * t + b, k = k0 + e;
                        if (e < 4 * CB && k < K) v |= (uint32_t)(uint8_t)xq[k] << (8 * b);
                    }
                    xd[i][t] = v;
                }
        }
        int xp[ND][4];
        int xsum = 0;
#pragma unroll
        for (int i = 0; i < ND; i++) {
            // 4x4 byte transpose with v_perm_b32.
            const uint32_t t0 = __builtin_amdgcn_perm(xd[i][1], xd[i][0], 0x05010400u);
            const uint32_t t1 = __builtin_amdgcn_perm(xd[i][3], xd[i][2], 0x05010400u);
            const uint32_t t2 = __builtin_amdgcn_perm(xd[i][1], xd[i][0], 0x07030602u);
            const uint32_t t3 = __builtin_amdgcn_perm(xd[i][3], xd[i][2], 0x07030602u);
            xp[i][0] = (int)__builtin_amdgcn_perm(t1, t0, 0x05040100u);
            xp[i][1] = (int)__builtin_amdgcn_perm(t1, t0, 0x07060302u);
            xp[i][2] = (int)__builtin_amdgcn_perm(t3, t2, 0x05040100u);
            xp[i][3] = (int)__builtin_amdgcn_perm(t3, t2, 0x07060302u);
#pragma unroll
            for (int s2 = 0; s2 < 4; s2++) xsum = __builtin_amdgcn_sdot4((int)xd[i][s2], 0x01010101, xsum, false);
        }
#pragma unroll
        for (int r = 0; r < R; r++) {
            int s32 = 0;
#pragma unroll
            for (int i = 0; i < ND; i++)
#pragma unroll
                for (int s = 0; s < 4; s++)
                    s32 = __builtin_amdgcn_sdot4((int)((w[r][i] >> (2 * s)) & 0x03030303u), xp[i][s], s32, false);
            acc[r] += (float)(s32 - xsum);  // |partial| <= K*127 < 2^24: exact in fp32
        }
    }
    // Every partial sum is an integer below 2^24, so the float reduction is exact.
    float tot[R];
#pragma unroll
    for (int r = 0; r < R; r++) tot[r] = acc[r];
    wave_reduce_rows<R>(tot);
    if (nwaves == 1) {
        if (is_row_writer<R>(lane)) {
            const int r = row0 + row_of_lane<R>(lane);
            if (r < rows) y[r] = tot[0] * scale;
        }
        return;
    }
    if (is_row_writer<R>(lane)) red[wave * R + row_of_lane<R>(lane)] = tot[0];
    __syncthreads();
    if ((int)threadIdx.x < R) {
        float s = 0.0f;
        for (int w2 = 0; w2 < nwaves; w2++) s += red[w2 * R + threadIdx.x];
        const int r = row0 + threadIdx.x;
        if (r < rows) y[r] = s * scale;
    }
}

// int8 x with K % 64 == 0 and K <= 65536, every lane one 16-byte chunk (64
// codes) of each of R rows: all loads of the wave (R code chunks, 64
// activation bytes, then the two scales) are issued before any arithmetic,
// as buffer loads whose wave-uniform row offsets are scalar offsets, and
// lanes past the last chunk read zeros through an out-of-range offset.  The
// loop kernel above waited for its scale loads (and the workgroup size)
// before its first weight load: a full memory round trip per wave.
template <int R>
__device__ __forceinline__ void ternary_i8_steps_body(const uint8_t* __restrict__ W, const int8_t* __restrict__ xq,
                                                      const float* __restrict__ x_scale,
                                                      const float* __restrict__ w_scale, float* __restrict__ y,
                                                      int rows, int bpr, int nw, int row0, float* red) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int c = wave * 64 + lane;  // 16-byte chunk of the row
    const uint32_t voff = c * 16 < bpr ? (uint32_t)c * 16u : 0x80000000u;
    const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc((void*)W, (short)0, 0x7fffffff, 0x00020000);
    const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc((void*)xq, (short)0, bpr * 4, 0x00020000);
    u32x4 w[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
        const uint32_t row = (uint32_t)min(row0 + r, rows - 1);
        w[r] = __builtin_amdgcn_raw_buffer_load_b128(rw, voff, row * (uint32_t)bpr, 2);  // nontemporal
    }
    u32x4 xv[4];
#pragma unroll
    for (int i = 0; i < 4; i++)
        xv[i] = __builtin_amdgcn_raw_buffer_load_b128(rx, voff == 0x80000000u ? voff : voff * 4u + 16u * i, 0, 0);
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void*)x_scale, (short)0, 4, 0x00020000);
    const __amdgpu_buffer_rsrc_t rt = __builtin_amdgcn_make_buffer_rsrc((void*)w_scale, (short)0, 4, 0x00020000);
    const float xs = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rs, 0u, 0, 0));
    const float wsc = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rt, 0u, 0, 0));
    int xp[4][4];
    int xsum = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t d0 = xv[i].x, d1 = xv[i].y, d2 = xv[i].z, d3 = xv[i].w;
        // 4x4 byte transpose: xp[i][s] packs activations 16i+s, 16i+4+s,
        // 16i+8+s, 16i+12+s, the order (w >> 2s) & 0x03030303 lays out the codes
        const uint32_t t0 = __builtin_amdgcn_perm(d1, d0, 0x05010400u);
        const uint32_t t1 = __builtin_amdgcn_perm(d3, d2, 0x05010400u);
        const uint32_t t2 = __builtin_amdgcn_perm(d1, d0, 0x07030602u);
        const uint32_t t3 = __builtin_amdgcn_perm(d3, d2, 0x07030602u);
        xp[i][0] = (int)__builtin_amdgcn_perm(t1, t0, 0x05040100u);
        xp[i][1] = (int)__builtin_amdgcn_perm(t1, t0, 0x07060302u);
        xp[i][2] = (int)__builtin_amdgcn_perm(t3, t2, 0x05040100u);
        xp[i][3] = (int)__builtin_amdgcn_perm(t3, t2, 0x07060302u);
        xsum = __builtin_amdgcn_sdot4((int)d0, 0x01010101, xsum, false);
        xsum = __builtin_amdgcn_sdot4((int)d1, 0x01010101, xsum, false);
        xsum = __builtin_amdgcn_sdot4((int)d2, 0x01010101, xsum, false);
        xsum = __builtin_amdgcn_sdot4((int)d3, 0x01010101, xsum, false);
    }
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
        const uint32_t wd[4] = {w[r].x, w[r].y, w[r].z, w[r].w};
        int s32 = 0;
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int s = 0; s < 4; s++)
                s32 = __builtin_amdgcn_sdot4((int)((wd[i] >> (2 * s)) & 0x03030303u), xp[i][s], s32, false);
        acc[r] = (float)(s32 - xsum);  // |partial| <= 64 * 127: exact
    }
    // every partial sum is an integer below 2^24, so the float reduction is exact
    wave_reduce_rows<R>(acc);
    const float scale = wsc * xs;
    if (nw == 1) {
        if (is_row_writer<R>(lane)) {
            const int r = row0 + row_of_lane<R>(lane);
            if (r < rows) y[r] = acc[0] * scale;
        }
        return;
    }
    if (is_row_writer<R>(lane)) red[wave * R + row_of_lane<R>(lane)] = acc[0];
    __syncthreads();
    if ((int)threadIdx.x < R) {
        float sm = 0.0f;
        for (int w2 = 0; w2 < nw; w2++) sm += red[w2 * R + threadIdx.x];
        const int r = row0 + threadIdx.x;
        if (r < rows) y[r] = sm * scale;
    }
}

template <int R>
__global__ void __launch_bounds__(1024) ternary_i8_steps_kernel(const uint8_t* __restrict__ W,
                                                                const int8_t* __restrict__ xq,
                                                                const float* __restrict__ x_scale,
                                                                const float* __restrict__ w_scale,
                                                                float* __restrict__ y, int rows, int bpr, int nw) {
    __shared__ float red[16 * R];
    ternary_i8_steps_body<R>(W, xq, x_scale, w_scale, y, rows, bpr, nw, blockIdx.x * R, red);
}

// Up to three ternary matrices that read the same int8 activation vector
// (a BitNet layer's q/k/v, or gate/up) in one launch: workgroups are
// numbered through the matrices in turn, and each finds its matrix from the
// row counts.  The activations, the three weight bases, the row counts and
// the row length come first in the arguments, inside the dwords gfx950
// preloads into SGPRs, so no wave waits on an argument load before its
// first weight load; scales and outputs follow.
template <int R>
__global__ void __launch_bounds__(1024) ternary_i8_group3_kernel(const int8_t* __restrict__ xq, const uint8_t* w0,
                                                                 const uint8_t* w1, const uint8_t* w2, int rows0,
                                                                 int rows1, int rows2, int bpr, int nw, int n,
                                                                 const float* __restrict__ x_scale,
                                                                 const float* ws0, const float* ws1,
                                                                 const float* ws2, float* y0, float* y1, float* y2) {
    __shared__ float red[16 * R];
    const int b = blockIdx.x;
    const int g1 = (rows0 + R - 1) / R, g2 = g1 + (rows1 + R - 1) / R;
    const int m = (b >= g1 ? 1 : 0) + (n > 2 && b >= g2 ? 1 : 0);
    const uint8_t* W = m == 0 ? w0 : m == 1 ? w1 : w2;
    const int rows = m == 0 ? rows0 : m == 1 ? rows1 : rows2;
    ternary_i8_steps_body<R>(W, xq, x_scale, m == 0 ? ws0 : m == 1 ? ws1 : ws2, m == 0 ? y0 : m == 1 ? y1 : y2, rows,
                             bpr, nw, (b - (m == 0 ? 0 : m == 1 ? g1 : g2)) * R, red);
}

// ----------------------------------------------------------- fp32 x

// fp32 x with K % 64 == 0 and K <= 65536: the fixed-step form of the int8
// kernel above (each lane one 16-byte chunk of R rows, every load issued
// before any arithmetic), with the 64 fp32 activations of the chunk as 16
// buffer loads shared by the R rows, and sum (c - 1) x = sum c x - sum x.
template <int R>
__global__ void __launch_bounds__(1024) ternary_f32_steps_kernel(const uint8_t* __restrict__ W,
                                                                 const float* __restrict__ x, float* __restrict__ y,
                                                                 int rows, int bpr, int nw) {
    __shared__ float red[16 * R];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int row0 = blockIdx.x * R;
    const int c = wave * 64 + lane;  // 16-byte chunk of the row: codes of elements 64c .. 64c+63
    const bool ok = c * 16 < bpr;
    const uint32_t voff = ok ? (uint32_t)c * 16u : 0x80000000u;
    const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc((void*)W, (short)0, 0x7fffffff, 0x00020000);
    const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc((void*)x, (short)0, bpr * 16, 0x00020000);
    u32x4 w[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
        const uint32_t row = (uint32_t)min(row0 + r, rows - 1);
        w[r] = __builtin_amdgcn_raw_buffer_load_b128(rw, voff, row * (uint32_t)bpr, 2);  // nontemporal
    }
    u32x4 xv[16];
#pragma unroll
    for (int i = 0; i < 16; i++)
        xv[i] = __builtin_amdgcn_raw_buffer_load_b128(rx, ok ? (uint32_t)c * 256u + 16u * i : 0x80000000u, 0, 0);
    float xs[64];
#pragma unroll
    for (int i = 0; i < 16; i++) {
        xs[4 * i] = __uint_as_float(xv[i].x);
        xs[4 * i + 1] = __uint_as_float(xv[i].y);
        xs[4 * i + 2] = __uint_as_float(xv[i].z);
        xs[4 * i + 3] = __uint_as_float(xv[i].w);
    }
    float xsum = 0.0f;
#pragma unroll
    for (int e = 0; e < 64; e += 4) xsum += (xs[e] + xs[e + 1]) + (xs[e + 2] + xs[e + 3]);
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
        const uint32_t wd[4] = {w[r].x, w[r].y, w[r].z, w[r].w};
        float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int s = 0; s < 4; s++) {
                // codes of elements 16i + 4j + s, j = 0..3, one per byte
                const uint32_t cds = (wd[i] >> (2 * s)) & 0x03030303u;
                s0 = fmaf((float)(cds & 0xffu), xs[16 * i + s], s0);
                s1 = fmaf((float)((cds >> 8) & 0xffu), xs[16 * i + 4 + s], s1);
                s0 = fmaf((float)((cds >> 16) & 0xffu), xs[16 * i + 8 + s], s0);
                s1 = fmaf((float)(cds >> 24), xs[16 * i + 12 + s], s1);
            }
        acc[r] = (s0 + s1) - xsum;
    }
    wave_reduce_rows<R>(acc);
    if (nw == 1) {
        if (is_row_writer<R>(lane)) {
            const int r = row0 + row_of_lane<R>(lane);
            if (r < rows) y[r] = acc[0];
        }
        return;
    }
    if (is_row_writer<R>(lane)) red[wave * R + row_of_lane<R>(lane)] = acc[0];
    __syncthreads();
    if ((int)threadIdx.x < R) {
        float sm = 0.0f;
        for (int w2 = 0; w2 < nw; w2++) sm += red[w2 * R + threadIdx.x];
        const int r = row0 + threadIdx.x;
        if (r < rows) y[r] = sm;
    }
}


// fp32 x on the quad mapping: four lanes a 16-byte chunk, lane 4c + q taking
// dword q (the codes of elements 64c + 16q .. +15) of R rows and those 16
// activations (four 16-byte loads), waves splitting the row's chunks 16 a
// wave.  A quarter of the per-lane work of the kernel above and four times the
// lanes, for rows whose K leaves that kernel's single wave mostly idle or
// short of parallelism.
template <int R>
__global__ void __launch_bounds__(1024) ternary_f32_quad_kernel(const uint8_t* __restrict__ W,
                                                                const float* __restrict__ x, float* __restrict__ y,
                                                                int rows, int bpr, int nw) {
    __shared__ float red[16 * R];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int row0 = blockIdx.x * R;
    const int e = wave * 64 + lane;  // dword of the row: codes of elements 16e .. 16e+15
    const bool ok = e * 4 < bpr;
    const uint32_t voff = ok ? (uint32_t)e * 4u : 0x80000000u;
    const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc((void*)W, (short)0, 0x7fffffff, 0x00020000);
    const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc((void*)x, (short)0, bpr * 16, 0x00020000);
    uint32_t w[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
        const uint32_t row = (uint32_t)min(row0 + r, rows - 1);
        w[r] = __builtin_amdgcn_raw_buffer_load_b32(rw, voff, row * (uint32_t)bpr, 2);  // nontemporal
    }
    u32x4 xv[4];
#pragma unroll
    for (int i = 0; i < 4; i++)
        xv[i] = __builtin_amdgcn_raw_buffer_load_b128(rx, ok ? (uint32_t)e * 64u + 16u * i : 0x80000000u, 0, 0);
    float xs[16];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        xs[4 * i] = __uint_as_float(xv[i].x);
        xs[4 * i + 1] = __uint_as_float(xv[i].y);
        xs[4 * i + 2] = __uint_as_float(xv[i].z);
        xs[4 * i + 3] = __uint_as_float(xv[i].w);
    }
    const float xsum = ((xs[0] + xs[1]) + (xs[2] + xs[3])) + ((xs[4] + xs[5]) + (xs[6] + xs[7])) +
                       (((xs[8] + xs[9]) + (xs[10] + xs[11])) + ((xs[12] + xs[13]) + (xs[14] + xs[15])));
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
        float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
        for (int s = 0; s < 4; s++) {
            // codes of elements 4j + s, j = 0..3, one per byte
            const uint32_t cds = (w[r] >> (2 * s)) & 0x03030303u;
            s0 = fmaf((float)(cds & 0xffu), xs[s], s0);
            s1 = fmaf((float)((cds >> 8) & 0xffu), xs[4 + s], s1);
            s0 = fmaf((float)((cds >> 16) & 0xffu), xs[8 + s], s0);
            s1 = fmaf((float)(cds >> 24), xs[12 + s], s1);
        }
        acc[r] = (s0 + s1) - xsum;
    }
    wave_reduce_rows<R>(acc);
    if (nw == 1) {
        if (is_row_writer<R>(lane)) {
            const int r = row0 + row_of_lane<R>(lane);
            if (r < rows) y[r] = acc[0];
        }
        return;
    }
    if (is_row_writer<R>(lane)) red[wave * R + row_of_lane<R>(lane)] = acc[0];
    __syncthreads();
    if ((int)threadIdx.x < R) {
        float sm = 0.0f;
        for (int w2 = 0; w2 < nw; w2++) sm += red[w2 * R + threadIdx.x];
        const int r = row0 + threadIdx.x;
        if (r < rows) y[r] = sm;
    }
}


template <int CB, int R>
__global__ void __launch_bounds__(512) ternary_f32_kernel(const uint8_t* __restrict__ W, const float* __restrict__ x,
                                                          float* __restrict__ y, int rows, int K, int bpr) {
    constexpr int ND = (CB + 3) / 4;
    __shared__ float red[8 * R];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nwaves = blockDim.x >> 6;
    const int nchunk = bpr / CB;
    const int row0 = blockIdx.x * R;
    long rbase[R];
#pragma unroll
    for (int r = 0; r < R; r++) rbase[r] = (long)min(row0 + r, rows - 1) * bpr;

    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.0f;

    for (int c = wave * kWave + lane; c < nchunk; c += nwaves * kWave) {
        uint32_t w[R][ND];
#pragma unroll
        for (int r = 0; r < R; r++) load_codes<CB>(W + rbase[r] + (long)c * CB, w[r]);
        const int k0 = c * CB * 4;
        float xv[ND][16];
        if (k0 + 4 * CB <= K && (((uintptr_t)(x + k0)) & 15) == 0) {
#pragma unroll
            for (int i = 0; i < ND; i++)
#pragma unroll
                for (int q = 0; q < (CB == 1 ? 1 : 4); q++) {
                    const float4 v = *reinterpret_cast<const float4*>(x + k0 + 16 * i + 4 * q);
                    xv[i][4 * q] = v.x; xv[i][4 * q + 1] = v.y; xv[i][4 * q + 2] = v.z; xv[i][4 * q + 3] = v.w;
                }
            if constexpr (CB == 1) {
#pragma unroll
                for (int e = 4; e < 16; e++) xv[0][e] = 0.0f;
            }
        } else {
#pragma unroll
            for (int i = 0; i < ND; i++)
#pragma unroll
                for (int e = 0; e < 16; e++) {
                    const int k = k0 + 16 * i + e;
                    xv[i][e] = (e < 4 * CB && k < K) ? x[k] : 0.0f;
                }
        }
        float xsum = 0.0f;
#pragma unroll
        for (int i = 0; i < ND; i++)
#pragma unroll
            for (int e = 0; e < 16; e++) xsum += xv[i][e];
#pragma unroll
        for (int r = 0; r < R; r++) {
            float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
            for (int i = 0; i < ND; i++)
#pragma unroll
                for (int s = 0; s < 4; s++) {
                    const uint32_t cds = (w[r][i] >> (2 * s)) & 0x03030303u;  // codes of elements 4j+s
#pragma unroll
                    for (int j = 0; j < 4; j += 2) {
                        s0 = fmaf((float)((cds >> (8 * j)) & 0xffu), xv[i][4 * j + s], s0);
                        s1 = fmaf((float)((cds >> (8 * j + 8)) & 0xffu), xv[i][4 * j + 4 + s], s1);
                    }
                }
            acc[r] += (s0 + s1) - xsum;
        }
    }
    block_reduce_store<R>(acc, red, y, 1, row0, rows);
}

template <int CB>
static void launch_ternary(bool i8, int R, dim3 g, dim3 b, hipStream_t st, const uint8_t* W, const void* x,
                           const float* xs, const float* ws, float* y, int rows, int K, int bpr) {
#define ZT_TERN_CASE(RR)                                                                                     \
    case RR:                                                                                                 \
        if (i8)                                                                                              \
            ternary_i8_kernel<CB, RR><<<g, b, 0, st>>>(W, (const int8_t*)x, xs, ws, y, rows, K, bpr);       \
        else                                                                                                 \
            ternary_f32_kernel<CB, RR><<<g, b, 0, st>>>(W, (const float*)x, y, rows, K, bpr);               \
        break;
    switch (R) {
        ZT_TERN_CASE(8)
        ZT_TERN_CASE(4)
        ZT_TERN_CASE(2)
        default:
        ZT_TERN_CASE(1)
    }
#undef ZT_TERN_CASE
}

static int ternary_gemv(bool i8, const void* Wv, const void* x, const float* xs, const float* ws, float* y, int M,
                        int K, hipStream_t st) {
    if (M < 0 || K < 0) return (int)hipErrorInvalidValue;
    if (M == 0) return (int)hipSuccess;
    if (Wv == nullptr || y == nullptr || (K > 0 && x == nullptr)) return (int)hipErrorInvalidValue;
    if (i8 && (xs == nullptr || ws == nullptr)) return (int)hipErrorInvalidValue;
    const uint8_t* W = static_cast<const uint8_t*>(Wv);
    const int bpr = (K + 3) / 4;
    if (!i8 && K % 64 == 0 && K <= 65536 && ((uintptr_t)W & 15) == 0 && ((uintptr_t)x & 15) == 0 &&
        (long)M * bpr < 0x7fffffffL) {
        const float* xf = static_cast<const float*>(x);
        if (K <= 16384) {
            // the quad mapping, 4 rows a wave (measured, us, against one lane a chunk of 64 codes,
            // with x staged in LDS for several row groups where that was faster: 2560 x 2560
            // 2.97 / 3.79, 6912 x 2560 3.85 / 4.75, 2560 x 6912 4.73 / 5.10; 2 / 8 rows a wave:
            // 3.25 / 3.23, 5.12 / 4.06, 6.16 / 4.95)
            const int nq = ceil_div(bpr / 4, 64);  // waves: 64 dwords of codes each
            int Rq = 4;
            while (Rq > 1 && (long)ceil_div(M, Rq) * nq < 512) Rq >>= 1;
            const dim3 g(ceil_div(M, Rq)), b(nq * kWave);
            switch (Rq) {
                case 4: ternary_f32_quad_kernel<4><<<g, b, 0, st>>>(W, xf, y, M, bpr, nq); break;
                case 2: ternary_f32_quad_kernel<2><<<g, b, 0, st>>>(W, xf, y, M, bpr, nq); break;
                default: ternary_f32_quad_kernel<1><<<g, b, 0, st>>>(W, xf, y, M, bpr, nq); break;
            }
            return (int)hipGetLastError();
        }
        // past K = 16384: one lane a chunk, 4 rows a wave (at the BitNet shapes R = 1 / 2 / 4 / 8
        // measured 5.33 / 3.87 / 3.77 / 3.77, 10.7 / 6.75 / 5.52 / 6.30 and 11.4 / 7.71 / 6.18 /
        // 7.74 us)
        const int nw = (K + 4095) / 4096;
        int R = 4;
        while (R > 1 && (long)ceil_div(M, R) * nw < 512) R >>= 1;
        const dim3 g(ceil_div(M, R)), b(nw * kWave);
        switch (R) {
            case 4: ternary_f32_steps_kernel<4><<<g, b, 0, st>>>(W, xf, y, M, bpr, nw); break;
            case 2: ternary_f32_steps_kernel<2><<<g, b, 0, st>>>(W, xf, y, M, bpr, nw); break;
            default: ternary_f32_steps_kernel<1><<<g, b, 0, st>>>(W, xf, y, M, bpr, nw); break;
        }
        return (int)hipGetLastError();
    }
    if (i8 && K % 64 == 0 && K <= 65536 && ((uintptr_t)W & 15) == 0 && ((uintptr_t)x & 15) == 0 &&
        (long)M * bpr < 0x7fffffffL) {
        const int nw = (K + 4095) / 4096;  // 16-byte chunks of 64 codes, 64 chunks a wave
        // 4 rows a wave unless that leaves fewer than 512 waves: at the BitNet
        // shapes 4 measured 5-20% faster than 1, 2 or 8
        int R = 4;
        while (R > 1 && (long)ceil_div(M, R) * nw < 512) R >>= 1;
        const dim3 g(ceil_div(M, R)), b(nw * kWave);
        const int8_t* xq = static_cast<const int8_t*>(x);
        switch (R) {
            case 4: ternary_i8_steps_kernel<4><<<g, b, 0, st>>>(W, xq, xs, ws, y, M, bpr, nw); break;
            case 2: ternary_i8_steps_kernel<2><<<g, b, 0, st>>>(W, xq, xs, ws, y, M, bpr, nw); break;
            default: ternary_i8_steps_kernel<1><<<g, b, 0, st>>>(W, xq, xs, ws, y, M, bpr, nw); break;
        }
        return (int)hipGetLastError();
    }
    int CB = 1;
    if (bpr % 16 == 0 && ((uintptr_t)W & 15) == 0) CB = 16;
    else if (bpr % 4 == 0 && ((uintptr_t)W & 3) == 0) CB = 4;
    const int nchunk = bpr / CB;
    const int nwaves = nchunk <= 64 ? 1 : (nchunk >= 8 * 64 ? 8 : ceil_div(nchunk, 64));
    const int R = pick_rows_per_wave(M, nwaves, 1, 2048);
    dim3 grid(ceil_div(M, R)), block(nwaves * kWave);
    if (CB == 16) launch_ternary<16>(i8, R, grid, block, st, W, x, xs, ws, y, M, K, bpr);
    else if (CB == 4) launch_ternary<4>(i8, R, grid, block, st, W, x, xs, ws, y, M, K, bpr);
    else launch_ternary<1>(i8, R, grid, block, st, W, x, xs, ws, y, M, K, bpr);
    return (int)hipGetLastError();
}

// Row-aligned codes -> fp32 {-1, 0, +1} (TernaryStorage.Slice semantics,
// tensor/ternary_storage.go:65-71, over the row-aligned layout).
__global__ void ternary_dequant_kernel(const uint8_t* __restrict__ W, float* __restrict__ out, int rows, int K,
                                       int bpr) {
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long)rows * K) return;
    const long r = i / K, j = i % K;
    const int code = (W[r * bpr + j / 4] >> (2 * (j % 4))) & 3;
    out[i] = (float)(code - 1);
}

}  // namespace zt

using namespace zt;

ZT_EXPORT int zt_ternary_gemv_f32(const void* W_ternary, const float* x, float* y, int M, int K,
                                  hipStream_t stream) {
    return ternary_gemv(false, W_ternary, x, nullptr, nullptr, y, M, K, stream);
}

ZT_EXPORT int zt_ternary_gemv_i8(const void* W_ternary, const int8_t* x_q, const float* x_scale,
                                 const float* w_scale, float* y, int M, int K, hipStream_t stream) {
    return ternary_gemv(true, W_ternary, x_q, x_scale, w_scale, y, M, K, stream);
}

ZT_EXPORT int zt_ternary_gemv_i8_group(const zt_ternary_gemv_desc* descs, int n, const int8_t* x_q,
                                       const float* x_scale, int K, hipStream_t stream) {
    if (descs == nullptr || n < 1 || n > ZT_GROUP_MAX || K < 0 || x_scale == nullptr ||
        (K > 0 && (x_q == nullptr || ((uintptr_t)x_q & 15))))
        return (int)hipErrorInvalidValue;
    const int bpr = (K + 3) / 4;
    long total = 0;
    for (int i = 0; i < n; i++) {
        const zt_ternary_gemv_desc& d = descs[i];
        if (d.rows < 0 || d.reserved != 0) return (int)hipErrorInvalidValue;
        if (d.rows > 0 && (d.W == nullptr || d.w_scale == nullptr || d.y == nullptr)) return (int)hipErrorInvalidValue;
        total += d.rows;
    }
    if (total == 0) return (int)hipSuccess;
    bool fused = n <= 3 && K > 0 && K % 64 == 0 && K <= 65536;
    for (int i = 0; i < n; i++)
        fused = fused && descs[i].rows > 0 && ((uintptr_t)descs[i].W & 15) == 0 && (long)descs[i].rows * bpr < 0x7fffffffL;
    if (!fused) {
        // shapes or counts outside the grouped kernel: one launch per matrix
        for (int i = 0; i < n; i++) {
            const zt_ternary_gemv_desc& d = descs[i];
            const int rc = d.rows == 0 ? 0 : ternary_gemv(true, d.W, x_q, x_scale, d.w_scale, d.y, d.rows, K, stream);
            if (rc != 0) return rc;
        }
        return (int)hipSuccess;
    }
    // the single-matrix configuration, rows per wave from the group's total rows
    const int nw = (K + 4095) / 4096;
    int R = 4;
    while (R > 1 && (long)ceil_div(total, R) * nw < 512) R >>= 1;
    const uint8_t* w[3] = {nullptr, nullptr, nullptr};
    const float* ws[3] = {nullptr, nullptr, nullptr};
    float* y[3] = {nullptr, nullptr, nullptr};
    int rw[3] = {0, 0, 0}, wgs = 0;
    for (int i = 0; i < n; i++) {
        w[i] = static_cast<const uint8_t*>(descs[i].W);
        ws[i] = descs[i].w_scale;
        y[i] = descs[i].y;
        rw[i] = descs[i].rows;
        wgs += ceil_div(rw[i], R);
    }
#define ZT_TG3(RR)                                                                                                  \
    ternary_i8_group3_kernel<RR><<<wgs, nw * kWave, 0, stream>>>(x_q, w[0], w[1], w[2], rw[0], rw[1], rw[2], bpr,  \
                                                                 nw, n, x_scale, ws[0], ws[1], ws[2], y[0], y[1],   \
                                                                 y[2])
    switch (R) {
        case 4: ZT_TG3(4); break;
        case 2: ZT_TG3(2); break;
        default: ZT_TG3(1); break;
    }
#undef ZT_TG3
    return (int)hipGetLastError();
}

ZT_EXPORT int zt_dequant_ternary_f32(const void* W_ternary, float* out, int M, int K, hipStream_t stream) {
    if (M < 0 || K < 0) return (int)hipErrorInvalidValue;
    const long n = (long)M * K;
    if (n == 0) return (int)hipSuccess;
    ternary_dequant_kernel<<<ceil_div(n, 256), 256, 0, stream>>>(static_cast<const uint8_t*>(W_ternary), out, M, K,
                                                                  (K + 3) / 4);
    return (int)hipGetLastError();
}

// Group-quantized int4 and plain int8 GEMMs with fp32 activations: the
// reference's gemm_int4_f32, gemm_int4_f32_rmul and gemm_int8_f32
// (internal/cuda/kernels/gemm_int4.cu:29-144, gemm_int8.cu:16-73; Go
// GemmInt4F32 / GemmInt4F32RMul / GemmInt8F32, gemm_quantized.go:24-89).
//
// Formats, as the reference defines them:
//  * int4: two signed values per byte, element 2b in the low nibble of byte
//    b, sign-extended to [-8, 7]; per-group fp32 scale and uint8 zero,
//    w = float32(v - zero) * scale.  gemm_int4_f32: A [M, K/2], groups of
//    group_size along K (scales, zeros [M, ceil(K / group_size)]).
//    gemm_int4_f32_rmul: W [in, out/2], groups along out (scales, zeros
//    [in, ceil(out / group_size)]), C[b, j] = sum_k X[b, k] w[k, j].
//  * int8: A [M, K] int8, C = float(A) B.
//
// Kernels:
//  * batches of 1-4 on aligned shapes: VALU kernels that stream the weights
//    once (for A B intq_steps_kernel at batch 1 up to K = 32768, else
//    intq_gemv_kernel, and intq_gemv_xlds_kernel for 2-4 columns; for X W
//    int4_rmul_v16_kernel, 16-byte
//    loads, for out % 32 == 0, group_size % 32 == 0 and in <= 8192, else
//    int4_rmul_valu_kernel for out % 16 == 0 and group_size % 16 == 0);
//  * batches of 4-64 columns of A B (N % 4 == 0; beyond 16 columns while
//    M N <= 2^19 for int4, 2^18 for int8) with K % 32 == 0 (int4:
//    group_size % 32 == 0) and K <= 32768: the row-block MFMA GEMM of
//    zt_rbmfma.h (formats INT4G and INT8), fp16 encodings of the unsigned
//    nibble or byte against hi/lo fp16 activations, the offset (8 + z or
//    128) times the activation sum taken off once per 32-element block;
//  * wider batches of A B with K % 32 == 0 (int4: group_size % 32 == 0) and
//    an even N: intq_bf16_kernel, bf16 MFMA on exact three-part activations;
//  * every other call: intq_mfma_kernel, an LDS-tiled fp32 MFMA GEMM
//    (v_mfma_f32_16x16x4f32) that dequantizes each weight on its way into
//    LDS exactly as the reference does (one fp32 multiply), so every product
//    is the reference's fp32 product and only the summation order differs.
#include <type_traits>

#include "zt_common.h"
#include "zt_mfma.h"
#include "zt_bf16gemm.h"
#include "zt_rbmfma.h"

namespace zt {

// The low 4 bits of v, sign-extended (gemm_int4.cu:20-27).
__device__ __forceinline__ int sext4(uint32_t v) { return ((int)(v << 28)) >> 28; }
// Byte i of v, sign-extended.
__device__ __forceinline__ int sext8(uint32_t v, int i) { return ((int)(v << (24 - 8 * i))) >> 24; }

// ------------------------------------------------------------ A B, batch 1-4
//
// C[M, N] = dequant(A) B for N = NB = 1.  A wave owns R rows; lane l of
// wave w takes 16-element chunks c = l + 64 (w + nwaves i) of K (int8: one
// 16-byte load a row; int4: one 8-byte load, within one group since
// group_size % 16 == 0) and the 16 N-wide activation rows of the chunk (4 NB
// contiguous 16-byte loads, shared by the R rows).  int4 sums (v - z) x over
// the chunk and applies the scale once: s * sum((v - z) x).  The waves of a
// workgroup then combine through LDS (block_reduce_store).
template <bool INT4, int R, int NB>
__global__ void __launch_bounds__(1024) intq_gemv_kernel(const uint8_t* __restrict__ A, const float* __restrict__ x,
                                                         float* __restrict__ y, const float* __restrict__ scales,
                                                         const uint8_t* __restrict__ zeros, int rows, int K, int gs,
                                                         int ng) {
    __shared__ float red[16 * R];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nwaves = blockDim.x >> 6;
    const int row0 = blockIdx.x * R;
    const int nchunks = K / 16;
    const long rowbytes = INT4 ? K / 2 : K;
    float acc[NB][R];
#pragma unroll
    for (int n = 0; n < NB; n++)
#pragma unroll
        for (int r = 0; r < R; r++) acc[n][r] = 0.0f;
    int rr[R];
#pragma unroll
    for (int r = 0; r < R; r++) rr[r] = min(row0 + r, rows - 1);
    for (int c = wave * 64 + lane; c < nchunks; c += nwaves * 64) {
        float xv[16 * NB];
        const float4* xp = reinterpret_cast<const float4*>(x + (long)c * 16 * NB);
#pragma unroll
        for (int q = 0; q < 4 * NB; q++) {
            const float4 t = xp[q];
            xv[4 * q] = t.x; xv[4 * q + 1] = t.y; xv[4 * q + 2] = t.z; xv[4 * q + 3] = t.w;
        }
        if constexpr (INT4) {
            uint2 w[R];
            float s[R];
            int z[R];
            const int g = c * 16 / gs;
#pragma unroll
            for (int r = 0; r < R; r++) {
                w[r] = *reinterpret_cast<const uint2*>(A + rr[r] * rowbytes + (long)c * 8);
                s[r] = scales[(long)rr[r] * ng + g];
                z[r] = zeros[(long)rr[r] * ng + g];
            }
#pragma unroll
            for (int r = 0; r < R; r++) {
                float ag[NB];
#pragma unroll
                for (int n = 0; n < NB; n++) ag[n] = 0.0f;
#pragma unroll
                for (int e = 0; e < 16; e++) {
                    const uint32_t d = e < 8 ? w[r].x : w[r].y;
                    const float v = (float)(sext4(d >> (4 * (e & 7))) - z[r]);
#pragma unroll
                    for (int n = 0; n < NB; n++) ag[n] = __builtin_fmaf(v, xv[e * NB + n], ag[n]);
                }
#pragma unroll
                for (int n = 0; n < NB; n++) acc[n][r] = __builtin_fmaf(s[r], ag[n], acc[n][r]);
            }
        } else {
            uint4 w[R];
#pragma unroll
            for (int r = 0; r < R; r++) w[r] = *reinterpret_cast<const uint4*>(A + rr[r] * rowbytes + (long)c * 16);
#pragma unroll
            for (int r = 0; r < R; r++) {
                const uint32_t d4[4] = {w[r].x, w[r].y, w[r].z, w[r].w};
#pragma unroll
                for (int e = 0; e < 16; e++) {
                    const float v = (float)sext8(d4[e >> 2], e & 3);
#pragma unroll
                    for (int n = 0; n < NB; n++) acc[n][r] = __builtin_fmaf(v, xv[e * NB + n], acc[n][r]);
                }
            }
        }
    }
#pragma unroll
    for (int n = 0; n < NB; n++) {
        if (n > 0) __syncthreads();  // red is reused by the next column
        block_reduce_store<R>(acc[n], red, y + n, NB, row0, rows);
    }
}

// Batch 1 in the fixed-step form of the Q4_0 GEMV: lane l of wave w takes
// the 16-element chunk c = (w S + t) 64 + l of step t, every load of the
// wave (R weight chunks, scales and zeros, 16 activations a step) issued
// before any arithmetic, as buffer loads whose wave-uniform row offsets are
// scalar offsets; lanes past the last chunk read zeros.  int4: with u = v + 8
// (nibble XOR 8) in [0, 15] as an fp16 subnormal u 2^-24 against x 2^24,
// each weight is one v_fma_mix, and sum (v - z) x = sum u x - (8 + z) sum x
// takes one FMA a chunk and row.  int8: u = q + 128 through v_cvt_f32_ubyte,
// sum q x = sum u x - 128 sum x.  Every product is exact; the sums carry sum
// u x's magnitude, about twice sum |(v - z) x| for int4 nibbles spread over
// [0, 15].
template <bool INT4, int S, int R>
__global__ void __launch_bounds__(1024) intq_steps_kernel(const uint8_t* __restrict__ A, const float* __restrict__ x,
                                                          float* __restrict__ y, const float* __restrict__ scales,
                                                          const uint8_t* __restrict__ zeros, int rows, int K, int gs,
                                                          int ng) {
    __shared__ float red[16 * R];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int row0 = blockIdx.x * R;
    const int nchunks = K / 16;
    const uint32_t rowbytes = INT4 ? (uint32_t)K / 2u : (uint32_t)K;
    constexpr int WB = INT4 ? 8 : 16;  // weight bytes a chunk
    const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc((void*)A, (short)0, 0x7fffffff, 0x00020000);
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void*)scales, (short)0, 0x7fffffff, 0x00020000);
    const __amdgpu_buffer_rsrc_t rz = __builtin_amdgcn_make_buffer_rsrc((void*)zeros, (short)0, 0x7fffffff, 0x00020000);
    const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc((void*)x, (short)0, K * 4, 0x00020000);
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
    u32x4 w[S][R];
    uint32_t sv[S][R], zv[S][R];
    u32x4 xv[S][4];
#pragma unroll
    for (int t = 0; t < S; t++) {
        const int c = (wave * S + t) * 64 + lane;
        const bool ok = c < nchunks;
#pragma unroll
        for (int r = 0; r < R; r++) {
            const uint32_t row = (uint32_t)min(row0 + r, rows - 1);
            const uint32_t wo = ok ? row * rowbytes + (uint32_t)c * WB : 0x80000000u;
            if constexpr (INT4) {
                const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(ra, wo, 0, 2);  // nontemporal
                w[t][r] = (u32x4){v.x, v.y, 0u, 0u};
            } else {
                w[t][r] = __builtin_amdgcn_raw_buffer_load_b128(ra, wo, 0, 2);
            }
        }
    }
#pragma unroll
    for (int t = 0; t < S; t++) {
        const int c = (wave * S + t) * 64 + lane;
        const bool ok = c < nchunks;
        if constexpr (INT4) {
            const int g = c * 16 / gs;
#pragma unroll
            for (int r = 0; r < R; r++) {
                const uint32_t row = (uint32_t)min(row0 + r, rows - 1);
                const uint32_t gi = row * (uint32_t)ng + (uint32_t)g;
                sv[t][r] = __builtin_amdgcn_raw_buffer_load_b32(rs, ok ? gi * 4u : 0x80000000u, 0, 0);
                zv[t][r] = __builtin_amdgcn_raw_buffer_load_b8(rz, ok ? gi : 0x80000000u, 0, 0);
            }
        }
#pragma unroll
        for (int i = 0; i < 4; i++)
            xv[t][i] = __builtin_amdgcn_raw_buffer_load_b128(rx, ok ? (uint32_t)c * 64u + 16u * i : 0x80000000u, 0, 0);
    }
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.0f;
#pragma unroll
    for (int t = 0; t < S; t++) {
        float xs[16];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            xs[4 * i] = __uint_as_float(xv[t][i].x);
            xs[4 * i + 1] = __uint_as_float(xv[t][i].y);
            xs[4 * i + 2] = __uint_as_float(xv[t][i].z);
            xs[4 * i + 3] = __uint_as_float(xv[t][i].w);
        }
        float xsum = 0.0f;
#pragma unroll
        for (int e = 0; e < 16; e += 4) xsum += (xs[e] + xs[e + 1]) + (xs[e + 2] + xs[e + 3]);
        if constexpr (INT4) {
            float xp[16];
#pragma unroll
            for (int e = 0; e < 16; e++) xp[e] = xs[e] * 16777216.0f;  // 2^24
#pragma unroll
            for (int r = 0; r < R; r++) {
                float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
                for (int h = 0; h < 2; h++) {
                    const uint32_t d = (h == 0 ? w[t][r].x : w[t][r].y) ^ 0x88888888u;  // u = v + 8
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        // nibbles e and e + 4 of the dword: elements 8h + e and 8h + e + 4
                        const half2v m = as_half2((d >> (4 * e)) & 0x000F000Fu);
                        s0 = __builtin_fmaf((float)m.x, xp[8 * h + e], s0);
                        s1 = __builtin_fmaf((float)m.y, xp[8 * h + e + 4], s1);
                    }
                }
                const float zf = (float)(8u + (zv[t][r] & 0xffu));
                acc[r] = __builtin_fmaf(__uint_as_float(sv[t][r]), __builtin_fmaf(-zf, xsum, s0 + s1), acc[r]);
            }
        } else {
#pragma unroll
            for (int r = 0; r < R; r++) {
                const uint32_t d4[4] = {w[t][r].x, w[t][r].y, w[t][r].z, w[t][r].w};
                float s0 = -128.0f * xsum, s1 = 0.0f;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const uint32_t u = d4[i] ^ 0x80808080u;  // q + 128
                    s0 = __builtin_fmaf((float)(u & 0xffu), xs[4 * i], s0);
                    s1 = __builtin_fmaf((float)((u >> 8) & 0xffu), xs[4 * i + 1], s1);
                    s0 = __builtin_fmaf((float)((u >> 16) & 0xffu), xs[4 * i + 2], s0);
                    s1 = __builtin_fmaf((float)(u >> 24), xs[4 * i + 3], s1);
                }
                acc[r] += s0 + s1;
            }
        }
    }
    block_reduce_store<R>(acc, red, y, 1, row0, rows);
}

template <bool INT4, int S>
static void launch_intq_steps(int R, dim3 g, dim3 b, hipStream_t st, const uint8_t* A, const float* x, float* y,
                              const float* s, const uint8_t* z, int M, int K, int gs, int ng) {
    switch (R) {
        case 8: intq_steps_kernel<INT4, S, 8><<<g, b, 0, st>>>(A, x, y, s, z, M, K, gs, ng); break;
        case 4: intq_steps_kernel<INT4, S, 4><<<g, b, 0, st>>>(A, x, y, s, z, M, K, gs, ng); break;
        case 2: intq_steps_kernel<INT4, S, 2><<<g, b, 0, st>>>(A, x, y, s, z, M, K, gs, ng); break;
        default: intq_steps_kernel<INT4, S, 1><<<g, b, 0, st>>>(A, x, y, s, z, M, K, gs, ng); break;
    }
}

// Batches of 2-4: the kernel above reads the activation chunk of every
// 16 elements once per R rows of a wave, 8 N / R times the weight bytes.
// Here a wave owns R = 2 or 4 rows over all of K and the 8 waves of a workgroup
// share the activations through LDS: chunks of 4096 elements (16 N KB) are
// staged once per workgroup, in the order the lanes read them (a lane's
// 16 N floats of step s as 4 N slots of 64 consecutive float4, so every
// ds_read_b128 is conflict-free), while the chunk's weight loads (4 steps of
// 1024 elements a row, all issued first) are in flight.  No cross-wave sum:
// each wave reduces its own rows across its lanes.
constexpr int kIqxKC = 4096;

template <bool INT4, int NB, int R>
__global__ void __launch_bounds__(512) intq_gemv_xlds_kernel(const uint8_t* __restrict__ A, const float* __restrict__ x,
                                                             float* __restrict__ y, const float* __restrict__ scales,
                                                             const uint8_t* __restrict__ zeros, int rows, int K, int gs,
                                                             int ng) {
    constexpr int S = kIqxKC / 1024, Q = 4 * NB;  // steps a chunk, float4 slots a step
    __shared__ float4 xs[S * Q * 64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int row0 = (blockIdx.x * 8 + wave) * R;
    const long rowbytes = INT4 ? K / 2 : K;
    int rr[R];
#pragma unroll
    for (int r = 0; r < R; r++) rr[r] = min(row0 + r, rows - 1);
    float acc[NB][R];
#pragma unroll
    for (int n = 0; n < NB; n++)
#pragma unroll
        for (int r = 0; r < R; r++) acc[n][r] = 0.0f;
    for (int kc0 = 0; kc0 < K; kc0 += kIqxKC) {
        const int kn = min(kIqxKC, K - kc0);
        typedef typename std::conditional<INT4, uint2, uint4>::type WT;
        WT w[S][R];
        float sc[S][R];
        int zr[S][R];
#pragma unroll
        for (int st = 0; st < S; st++) {
            const int e = 1024 * st + 16 * lane;  // first element of the lane's 16 in the chunk
            const bool ok = e < kn;
#pragma unroll
            for (int r = 0; r < R; r++) {
                const long off = rr[r] * rowbytes + (long)(ok ? kc0 + e : 0) / (INT4 ? 2 : 1);
                if constexpr (INT4) {
                    w[st][r] = ok ? *reinterpret_cast<const uint2*>(A + off) : make_uint2(0u, 0u);
                    const long gi = (long)rr[r] * ng + (ok ? kc0 + e : 0) / gs;
                    sc[st][r] = scales[gi];
                    zr[st][r] = zeros[gi];
                } else {
                    w[st][r] = ok ? *reinterpret_cast<const uint4*>(A + off) : make_uint4(0u, 0u, 0u, 0u);
                }
            }
        }
        if (kc0 > 0) __syncthreads();  // every wave is done with the previous chunk
        const float4* xg = reinterpret_cast<const float4*>(x + (long)kc0 * NB);
        for (int t = threadIdx.x; t < kn * NB / 4; t += 512) {
            const int st = t / (256 * NB), f = 4 * (t % (256 * NB));  // step, float index within the step
            const int ln = f / (16 * NB), q = (f % (16 * NB)) / 4;
            xs[(st * Q + q) * 64 + ln] = xg[t];
        }
        __syncthreads();
#pragma unroll
        for (int st = 0; st < S; st++) {
            if (1024 * st + 16 * lane >= kn) continue;
            float xv[16 * NB];
#pragma unroll
            for (int q = 0; q < Q; q++) {
                const float4 v = xs[(st * Q + q) * 64 + lane];
                xv[4 * q] = v.x; xv[4 * q + 1] = v.y; xv[4 * q + 2] = v.z; xv[4 * q + 3] = v.w;
            }
#pragma unroll
            for (int r = 0; r < R; r++) {
                if constexpr (INT4) {
                    float ag[NB];
#pragma unroll
                    for (int n = 0; n < NB; n++) ag[n] = 0.0f;
#pragma unroll
                    for (int e = 0; e < 16; e++) {
                        const uint32_t d = e < 8 ? w[st][r].x : w[st][r].y;
                        const float v = (float)(sext4(d >> (4 * (e & 7))) - zr[st][r]);
#pragma unroll
                        for (int n = 0; n < NB; n++) ag[n] = __builtin_fmaf(v, xv[e * NB + n], ag[n]);
                    }
#pragma unroll
                    for (int n = 0; n < NB; n++) acc[n][r] = __builtin_fmaf(sc[st][r], ag[n], acc[n][r]);
                } else {
                    const uint32_t d4[4] = {w[st][r].x, w[st][r].y, w[st][r].z, w[st][r].w};
#pragma unroll
                    for (int e = 0; e < 16; e++) {
                        const float v = (float)sext8(d4[e >> 2], e & 3);
#pragma unroll
                        for (int n = 0; n < NB; n++) acc[n][r] = __builtin_fmaf(v, xv[e * NB + n], acc[n][r]);
                    }
                }
            }
        }
    }
#pragma unroll
    for (int n = 0; n < NB; n++) {
        wave_reduce_rows<R>(acc[n]);
        if (is_row_writer<R>(lane)) {
            const int row = row0 + row_of_lane<R>(lane);
            if (row < rows) y[(long)row * NB + n] = acc[n][0];
        }
    }
}

template <bool INT4, int NB>
static void launch_intq_gemv_r(int R, dim3 g, dim3 b, hipStream_t st, const uint8_t* A, const float* x, float* y,
                               const float* s, const uint8_t* z, int M, int K, int gs, int ng) {
    switch (R) {
        case 8: intq_gemv_kernel<INT4, 8, NB><<<g, b, 0, st>>>(A, x, y, s, z, M, K, gs, ng); break;
        case 4: intq_gemv_kernel<INT4, 4, NB><<<g, b, 0, st>>>(A, x, y, s, z, M, K, gs, ng); break;
        case 2: intq_gemv_kernel<INT4, 2, NB><<<g, b, 0, st>>>(A, x, y, s, z, M, K, gs, ng); break;
        default: intq_gemv_kernel<INT4, 1, NB><<<g, b, 0, st>>>(A, x, y, s, z, M, K, gs, ng); break;
    }
}

template <bool INT4>
static void launch_intq_gemv(hipStream_t st, const uint8_t* A, const float* x, float* y, const float* s,
                             const uint8_t* z, int M, int K, int N, int gs, int ng) {
    if (N >= 2) {
        // 4 rows a wave from 8192 rows (>= 256 workgroups), else 2
        const bool r4 = M >= 8192;
        const dim3 g(ceil_div(M, r4 ? 32 : 16)), b(512);
        switch (N) {
            case 2:
                if (r4) intq_gemv_xlds_kernel<INT4, 2, 4><<<g, b, 0, st>>>(A, x, y, s, z, M, K, gs, ng);
                else intq_gemv_xlds_kernel<INT4, 2, 2><<<g, b, 0, st>>>(A, x, y, s, z, M, K, gs, ng);
                break;
            case 3:
                if (r4) intq_gemv_xlds_kernel<INT4, 3, 4><<<g, b, 0, st>>>(A, x, y, s, z, M, K, gs, ng);
                else intq_gemv_xlds_kernel<INT4, 3, 2><<<g, b, 0, st>>>(A, x, y, s, z, M, K, gs, ng);
                break;
            default:
                if (r4) intq_gemv_xlds_kernel<INT4, 4, 4><<<g, b, 0, st>>>(A, x, y, s, z, M, K, gs, ng);
                else intq_gemv_xlds_kernel<INT4, 4, 2><<<g, b, 0, st>>>(A, x, y, s, z, M, K, gs, ng);
                break;
        }
        return;
    }
    const int nchunks = K / 16;
    const long rowbytes = INT4 ? K / 2 : K;
    // the fixed-step form up to K = 32768 (us, loop kernel against fixed
    // steps: int4 4096 x 4096 5.10 / 4.47, 14336 x 4096 10.07 / 9.16; int8
    // 4096 x 4096 5.24 / 4.93, 4096 x 14336 12.08 / 11.71)
    if (nchunks <= 64 * 16 * 2 && (long)M * rowbytes < 0x7fffffffL && (long)M * ng * 4 < 0x7fffffffL) {
        const int S = nchunks <= 64 * 16 ? 1 : 2;
        const int nw = ceil_div(nchunks, 64 * S);
        const int R = pick_rows_per_wave(M, nw, 1, 2048);
        const dim3 g(ceil_div(M, R)), b(nw * kWave);
        if (S == 1) launch_intq_steps<INT4, 1>(R, g, b, st, A, x, y, s, z, M, K, gs, ng);
        else launch_intq_steps<INT4, 2>(R, g, b, st, A, x, y, s, z, M, K, gs, ng);
        return;
    }
    const int nw = max(1, min(16, ceil_div(nchunks, 64)));
    const int R = pick_rows_per_wave(M, nw, 1, 2048);
    launch_intq_gemv_r<INT4, 1>(R, dim3(ceil_div(M, R)), dim3(nw * kWave), st, A, x, y, s, z, M, K, gs, ng);
}

// ------------------------------------------------------------ X W, batch 1-4
//
// C[b, j] = sum_k X[b, k] w[k, j], batch NB in 1..4, out % 16 == 0 and
// group_size % 16 == 0.  A workgroup of 16 waves owns 16 LPR output
// columns: lane l owns columns 16 (l % LPR) .. +15 (one 8-byte load a row,
// all in one group) and row phase l / LPR, so a load instruction reads
// 64 / LPR rows x 8 LPR bytes; wave w takes the w-th sixteenth of K, and U
// rows a lane are loaded before any is used (at K = 4096 that is all of the
// lane's rows).  Per row
// the lane forms t = X[b, k] * scale and adds t * float(v - zero) for its 16
// columns (the reference rounds float(v - zero) * scale first, then
// multiplies by X: the two differ by one fp32 rounding per product).  The
// row phases are added by lane shuffles, the 16 waves through LDS in wave
// order.
template <int NB, int U, int LPR>
__global__ void __launch_bounds__(1024) int4_rmul_valu_kernel(const uint8_t* __restrict__ W,
                                                              const float* __restrict__ X, float* __restrict__ C,
                                                              const float* __restrict__ scales,
                                                              const uint8_t* __restrict__ zeros, int K, int Nout,
                                                              int gs, int ng) {
    constexpr int NPH = 64 / LPR;  // row phases
    __shared__ float red[16][LPR][16 * NB];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nwaves = blockDim.x >> 6;
    const int cl = lane % LPR, ph = lane / LPR;
    // neighbouring column blocks read the same weight, scale and zero lines:
    // keep them on one XCD (one L2)
    const int bx = xcd_contiguous(blockIdx.x, (Nout + 16 * LPR - 1) / (16 * LPR));
    const int col = bx * 16 * LPR + 16 * cl;  // first of the lane's 16 columns
    const bool colok = col < Nout;
    const int cc = colok ? col : 0;
    const int g = cc / gs;
    const long rowbytes = Nout / 2;
    const int kw = (K + nwaves - 1) / nwaves;
    const int kbeg = wave * kw, kend = min(K, kbeg + kw);
    float acc[NB][16];
#pragma unroll
    for (int b = 0; b < NB; b++)
#pragma unroll
        for (int j = 0; j < 16; j++) acc[b][j] = 0.0f;
    for (int k0 = kbeg + ph; k0 < kend; k0 += NPH * U) {
        uint2 w[U];
        float s[U], xv[U][NB];
        int z[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int k = k0 + NPH * u;
            const bool ok = colok && k < kend;
            const int kk = ok ? k : kbeg;
            w[u] = ok ? *reinterpret_cast<const uint2*>(W + (long)kk * rowbytes + cc / 2) : make_uint2(0u, 0u);
            s[u] = scales[(long)kk * ng + g];
            z[u] = zeros[(long)kk * ng + g];
#pragma unroll
            for (int b = 0; b < NB; b++) xv[u][b] = ok ? X[(long)b * K + kk] : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            float t[NB];
#pragma unroll
            for (int b = 0; b < NB; b++) t[b] = xv[u][b] * s[u];
#pragma unroll
            for (int j = 0; j < 16; j++) {
                const uint32_t d = j < 8 ? w[u].x : w[u].y;
                const float v = (float)(sext4(d >> (4 * (j & 7))) - z[u]);
#pragma unroll
                for (int b = 0; b < NB; b++) acc[b][j] = __builtin_fmaf(t[b], v, acc[b][j]);
            }
        }
    }
    // row phases (the lane bits above those of cl) into lanes 0 .. LPR-1
#pragma unroll
    for (int b = 0; b < NB; b++)
#pragma unroll
        for (int j = 0; j < 16; j++) {
            float v = acc[b][j];
#pragma unroll
            for (int m = LPR; m < 64; m <<= 1) v += __shfl_xor(v, m);
            acc[b][j] = v;
        }
    if (ph == 0) {
#pragma unroll
        for (int b = 0; b < NB; b++)
#pragma unroll
            for (int j = 0; j < 16; j++) red[wave][cl][16 * b + j] = acc[b][j];
    }
    __syncthreads();
    // outputs (b, column) over the workgroup's threads, the waves summed in order
    for (int t = threadIdx.x; t < 16 * LPR * NB; t += blockDim.x) {
        const int b = t / (16 * LPR), c = t % (16 * LPR);
        const int n = bx * 16 * LPR + c;
        if (n < Nout) {
            float sum = 0.0f;
            for (int w = 0; w < nwaves; w++) sum += red[w][c >> 4][16 * b + (c & 15)];
            C[(long)b * Nout + n] = sum;
        }
    }
}

template <int NB>
static void launch_int4_rmul_valu(hipStream_t st, const uint8_t* W, const float* X, float* C, const float* s,
                                  const uint8_t* z, int K, int Nout, int gs, int ng) {
    const int nw = max(1, min(16, K / 256));
    // 16 columns a workgroup (one lane a row, 64 row phases): 4096 x 4096
    // batch 1 21.1 us, against 25.6 with 32 columns and 28.0 with 64 (more
    // workgroups keep more rows in flight; neighbouring workgroups share
    // each row's 64-byte lines in L2); batch 4 28.8 against 31.3 us
    // (4 rows a lane per pass, 2 at batch 4 to stay within 128 VGPRs)
    int4_rmul_valu_kernel<NB, NB == 4 ? 2 : 4, 1><<<dim3(ceil_div(Nout, 16)), dim3(nw * kWave), 0, st>>>(
        W, X, C, s, z, K, Nout, gs, ng);
}

// X W, batch 1-4, out % 32 == 0 and group_size % 32 == 0: the same sum with
// 16-byte weight loads.  A lane owns 32 output columns (one 16-byte piece of
// a row, all in one group), the 64 lanes of a wave take K rows in turn, and
// a workgroup of NW waves owns 32 columns and all of K.  Per row the lane
// forms t = X[b, k] * scale and adds t * u for u = v + 8 in [0, 15]: the
// nibble enters v_fma_mix as an fp16 subnormal u 2^-24 against t 2^24, so
// the product is t u exactly and each weight costs one FMA and half a mask;
// sum t (8 + zero) goes to one more accumulator and comes off at the end:
// C = sum t u - sum t (8 + zero) = sum t (v - zero).  Against the reference
// (float(v - zero) * scale first, then times X, one sum) each product
// differs by one fp32 rounding, and the two sums carry sum t u's magnitude,
// about twice sum |t (v - zero)| for nibbles spread over [0, 15].  Each
// wave sums its 64 lanes by halving exchanges (wave_reduce_rows), and the
// workgroup adds the waves in wave order: the same bits every call.
template <int NB, int U, int NW>
__global__ void __launch_bounds__(NW * 64) int4_rmul_v16_kernel(const uint8_t* __restrict__ W,
                                                                const float* __restrict__ X, float* __restrict__ C,
                                                                const float* __restrict__ scales,
                                                                const uint8_t* __restrict__ zeros, int K, int Nout,
                                                                int gs, int ng) {
    __shared__ float red[NW][NB][33];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int bx = xcd_contiguous(blockIdx.x, Nout / 32);
    const int col = bx * 32, g = col / gs;
    const uint32_t rowbytes = (uint32_t)Nout / 2u;
    const __amdgpu_buffer_rsrc_t rw =
        __builtin_amdgcn_make_buffer_rsrc((void*)W, (short)0, (int)((uint32_t)K * rowbytes), 0x00020000);
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc((void*)scales, (short)0, K * ng * 4, 0x00020000);
    const __amdgpu_buffer_rsrc_t rz = __builtin_amdgcn_make_buffer_rsrc((void*)zeros, (short)0, K * ng, 0x00020000);
    const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc((void*)X, (short)0, NB * K * 4, 0x00020000);
    const int kw = (K + NW - 1) / NW;
    const int kbeg = wave * kw, kend = min(K, kbeg + kw);
    float acc[NB][32], ctr[NB];
#pragma unroll
    for (int b = 0; b < NB; b++) {
        ctr[b] = 0.0f;
#pragma unroll
        for (int j = 0; j < 32; j++) acc[b][j] = 0.0f;
    }
    for (int k0 = kbeg + lane; k0 < kend; k0 += 64 * U) {
        u32x4 w[U];
        float sv[U], xv[U][NB];
        uint32_t zv[U];
        // rows past the wave's range read zeros (out-of-range buffer offsets), so t = 0
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int k = k0 + 64 * u;
            const bool ok = k < kend;
            w[u] = __builtin_amdgcn_raw_buffer_load_b128(rw, ok ? (uint32_t)k * rowbytes + (uint32_t)col / 2u : 0x80000000u,
                                                         0, 2);  // nontemporal
            sv[u] = __uint_as_float(
                __builtin_amdgcn_raw_buffer_load_b32(rs, ok ? (uint32_t)(k * ng + g) * 4u : 0x80000000u, 0, 0));
            zv[u] = __builtin_amdgcn_raw_buffer_load_b8(rz, ok ? (uint32_t)(k * ng + g) : 0x80000000u, 0, 0);
#pragma unroll
            for (int b = 0; b < NB; b++)
                xv[u][b] = __uint_as_float(
                    __builtin_amdgcn_raw_buffer_load_b32(rx, ok ? (uint32_t)(b * K + k) * 4u : 0x80000000u, 0, 0));
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            float tp[NB];
#pragma unroll
            for (int b = 0; b < NB; b++) {
                const float t = xv[u][b] * sv[u];
                ctr[b] = __builtin_fmaf(t, (float)(8u + (zv[u] & 0xffu)), ctr[b]);
                tp[b] = t * 16777216.0f;  // 2^24
            }
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint32_t d = w[u][i] ^ 0x88888888u;  // u = v + 8 in every nibble
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    // nibbles e and e + 4 of the dword: elements 8i + e and 8i + e + 4
                    const half2v m = as_half2((d >> (4 * e)) & 0x000F000Fu);
#pragma unroll
                    for (int b = 0; b < NB; b++) {
                        acc[b][8 * i + e] = __builtin_fmaf((float)m.x, tp[b], acc[b][8 * i + e]);
                        acc[b][8 * i + e + 4] = __builtin_fmaf((float)m.y, tp[b], acc[b][8 * i + e + 4]);
                    }
                }
            }
        }
    }
#pragma unroll
    for (int b = 0; b < NB; b++) {
        wave_reduce_rows<32>(acc[b]);
        float c = ctr[b];
        c = single_step<32>(c);
        c = single_step<16>(c);
        c = single_step<8>(c);
        c = single_step<4>(c);
        c = single_step<2>(c);
        c = single_step<1>(c);
        if (is_row_writer<32>(lane)) red[wave][b][row_of_lane<32>(lane)] = acc[b][0];
        if (lane == 0) red[wave][b][32] = c;
    }
    __syncthreads();
    for (int t = threadIdx.x; t < 32 * NB; t += NW * 64) {
        const int b = t >> 5, j = t & 31;
        float sa = 0.0f, sc = 0.0f;
        for (int wv = 0; wv < NW; wv++) {
            sa += red[wv][b][j];
            sc += red[wv][b][32];
        }
        C[(long)b * Nout + col + j] = sa - sc;
    }
}

template <int NB>
static void launch_int4_rmul_v16(hipStream_t st, const uint8_t* W, const float* X, float* C, const float* s,
                                 const uint8_t* z, int K, int Nout, int gs, int ng) {
    constexpr int U = NB <= 2 ? 8 : 4;  // rows a lane loads before using any (within 256 VGPRs)
    int4_rmul_v16_kernel<NB, U, 8><<<dim3(Nout / 32), dim3(8 * kWave), 0, st>>>(W, X, C, s, z, K, Nout, gs, ng);
}

// ------------------------------------------------------------ fp32 MFMA GEMM
//
// C[M, N] = sum_k Aop(m, k) Bop(k, n) with
//   V = 0 (int8 A B):  Aop = float(A[m, k]),  Bop = B[k, n];
//   V = 1 (int4 A B):  Aop = float(v - z) * s of A[m, k] (groups along K),
//                      Bop = B[k, n];
//   V = 2 (X W):       Aop = X[m, k] (M = batch), Bop = float(v - z) * s of
//                      W[k, n] (groups along N).
// A workgroup of 4 waves owns a 64 x 64 tile of C; each wave a 32 x 32
// quarter, 2 x 2 tiles of v_mfma_f32_16x16x4f32 (lane l supplies A[l % 16]
// [l / 16] and B[l / 16][l % 16]; D lane l holds rows 4 (l / 16) .. +3 of
// column l % 16).  K advances 32 at a time through two LDS buffers, [k][m]
// and [k][n] with rows padded to 80 floats, so each lane group's reads hit
// distinct banks; the next K step's global loads are issued before the
// current step's MFMAs.  Every global load is a scalar element load
// coalesced across lanes, so no shape or alignment is required.
constexpr int kIqTM = 64, kIqTN = 64, kIqTK = 32, kIqLP = 80;

template <int V>
__global__ void __launch_bounds__(256) intq_mfma_kernel(const void* __restrict__ Ap, const void* __restrict__ Bp,
                                                        float* __restrict__ C, const float* __restrict__ scales,
                                                        const uint8_t* __restrict__ zeros, int M, int N, int K, int gs,
                                                        int ng) {
    __shared__ float As[2][kIqTK][kIqLP];
    __shared__ float Bs[2][kIqTK][kIqLP];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int m0 = blockIdx.y * kIqTM, n0 = blockIdx.x * kIqTN;
    float ra[8], rb[8];

    // the A operand of K step k0 into ra
    auto load_a = [&](int k0) {
        if constexpr (V == 0 || V == 1) {
            // thread: row m0 + tid / 4, K positions k0 + 8 (tid % 4) .. +7
            const int m = m0 + (tid >> 2), kb = k0 + 8 * (tid & 3);
            if constexpr (V == 0) {
                const int8_t* a = static_cast<const int8_t*>(Ap) + (long)min(m, M - 1) * K;
#pragma unroll
                for (int e = 0; e < 8; e++) ra[e] = (m < M && kb + e < K) ? (float)a[kb + e] : 0.0f;
            } else {
                const uint8_t* a = static_cast<const uint8_t*>(Ap) + (long)min(m, M - 1) * (K / 2);
                const long gbase = (long)min(m, M - 1) * ng;
                int g = min(kb, K - 1) / gs, rem = min(kb, K - 1) - g * gs;
                float s = scales[gbase + g];
                int z = zeros[gbase + g];
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    const int k = kb + e;
                    if (rem == gs) {
                        g++;
                        rem = 0;
                        if (k < K) {
                            s = scales[gbase + g];
                            z = zeros[gbase + g];
                        }
                    }
                    rem++;
                    float v = 0.0f;
                    if (m < M && k < K) {
                        const uint32_t byte = a[k >> 1];
                        v = (float)(sext4((k & 1) ? byte >> 4 : byte) - z) * s;
                    }
                    ra[e] = v;
                }
            }
        } else {
            // X rows: thread K position k0 + tid % 32, rows m0 + tid / 32 + 8 i
            const float* xr = static_cast<const float*>(Ap);
            const int k = k0 + (tid & 31);
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const int m = m0 + (tid >> 5) + 8 * i;
                ra[i] = (m < M && k < K) ? xr[(long)m * K + k] : 0.0f;
            }
        }
    };
    // the B operand of K step k0 into rb
    auto load_b = [&](int k0) {
        if constexpr (V == 0 || V == 1) {
            // thread: column n0 + tid % 64, K rows k0 + tid / 64 + 4 i
            const float* b = static_cast<const float*>(Bp);
            const int n = n0 + (tid & 63);
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const int k = k0 + (tid >> 6) + 4 * i;
                rb[i] = (n < N && k < K) ? b[(long)k * N + n] : 0.0f;
            }
        } else {
            // W row k0 + tid / 8, columns n0 + 8 (tid % 8) .. +7
            const int k = k0 + (tid >> 3), nb = n0 + 8 * (tid & 7);
            const uint8_t* w = static_cast<const uint8_t*>(Bp) + (long)min(k, K - 1) * (N / 2);
            const long gbase = (long)min(k, K - 1) * ng;
            int g = min(nb, N - 1) / gs, rem = min(nb, N - 1) - g * gs;
            float s = scales[gbase + g];
            int z = zeros[gbase + g];
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const int n = nb + e;
                if (rem == gs) {
                    g++;
                    rem = 0;
                    if (n < N) {
                        s = scales[gbase + g];
                        z = zeros[gbase + g];
                    }
                }
                rem++;
                float v = 0.0f;
                if (k < K && n < N) {
                    const uint32_t byte = w[n >> 1];
                    v = (float)(sext4((n & 1) ? byte >> 4 : byte) - z) * s;
                }
                rb[e] = v;
            }
        }
    };
    auto store = [&](int buf) {
        if constexpr (V == 0 || V == 1) {
            const int m = tid >> 2, kb = 8 * (tid & 3);
#pragma unroll
            for (int e = 0; e < 8; e++) As[buf][kb + e][m] = ra[e];
            const int n = tid & 63, kr = tid >> 6;
#pragma unroll
            for (int i = 0; i < 8; i++) Bs[buf][kr + 4 * i][n] = rb[i];
        } else {
            const int k = tid & 31, mr = tid >> 5;
#pragma unroll
            for (int i = 0; i < 8; i++) As[buf][k][mr + 8 * i] = ra[i];
            const int kr = tid >> 3, nb = 8 * (tid & 7);
#pragma unroll
            for (int e = 0; e < 8; e++) Bs[buf][kr][nb + e] = rb[e];
        }
    };

    const int wm = (wave & 1) * 32, wn = (wave >> 1) * 32;
    const int li = lane & 15, lk = lane >> 4;
    float4v acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) acc[i][j] = (float4v){0.f, 0.f, 0.f, 0.f};
    const int nsteps = (K + kIqTK - 1) / kIqTK;
    if (nsteps > 0) {
        load_a(0);
        load_b(0);
        store(0);
    }
    __syncthreads();
    for (int t = 0; t < nsteps; t++) {
        const int buf = t & 1;
        if (t + 1 < nsteps) {
            load_a((t + 1) * kIqTK);
            load_b((t + 1) * kIqTK);
        }
#pragma unroll
        for (int kk = 0; kk < kIqTK / 4; kk++) {
            const int kr = 4 * kk + lk;
            const float a0 = As[buf][kr][wm + li], a1 = As[buf][kr][wm + 16 + li];
            const float b0 = Bs[buf][kr][wn + li], b1 = Bs[buf][kr][wn + 16 + li];
            acc[0][0] = __builtin_amdgcn_mfma_f32_16x16x4f32(a0, b0, acc[0][0], 0, 0, 0);
            acc[0][1] = __builtin_amdgcn_mfma_f32_16x16x4f32(a0, b1, acc[0][1], 0, 0, 0);
            acc[1][0] = __builtin_amdgcn_mfma_f32_16x16x4f32(a1, b0, acc[1][0], 0, 0, 0);
            acc[1][1] = __builtin_amdgcn_mfma_f32_16x16x4f32(a1, b1, acc[1][1], 0, 0, 0);
        }
        // the other buffer was last read in step t - 1, before the barrier that ended it
        if (t + 1 < nsteps) store(buf ^ 1);
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int n = n0 + wn + 16 * j + li;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int m = m0 + wm + 16 * i + 4 * lk + r;
                if (m < M && n < N) C[(long)m * N + n] = acc[i][j][r];
            }
        }
}

// ------------------------------------------------------------ bf16 MFMA GEMM
//
// C[M, N] = dequant(A) B on bf16 MFMA (v_mfma_f32_16x16x32_bf16): every
// fp32 activation is split into three bf16 parts, x = b1 + b2 + b3 (b1 = x
// with its low 16 bits cleared, b2 the same of x - b1, b3 = x - b1 - b2,
// which has at most 8 significant bits), so each bf16 x bf16 product is
// exact and only the fp32 sums round.  The weights enter exactly too:
//   int8: float(q) has at most 8 significant bits, so it is a bf16 exactly,
//     and the result is exact up to the fp32 accumulation;
//   int4: 128 + (v ^ 8) as the bf16 0x4300 | u' (u' = nibble ^ 8 in 0..15),
//     with v - z = u' - (8 + z); an all-ones A operand gives Dx = sum_k x per
//     column and step, and each output takes s * (D - (136 + z) Dx), s and
//     z of its row and the step's group (group_size % 32 == 0).  D and
//     (136 + z) Dx are each about (136 + |v|) / |v - z| times the step's
//     result, so their fp32 roundings weigh that much more than in a sum of
//     dequantized products: measured per output against the exact product,
//     relative to sum |w x|, 3.8e-7 with z = 0 (the reference's fp32 loop:
//     2.2e-7), 1.6e-7 with z up to 15 and 3.9e-8 up to 255.
// A workgroup of 4 waves owns a 32 TI x 32 TI tile of C, each wave
// 16 TI x 16 TI (TI x TI MFMA tiles; TI = 4, or 2 when 128 x 128 tiles would
// leave fewer than 256 workgroups); K advances 32 a step.  Weight A operands come straight from
// global memory (lane 16 g + i: 8 consecutive K values of row i, one 8-byte
// int8 or 4-byte int4 load); the activation tile is split into its parts
// and staged in LDS as [part][column][32 K values in operand order], read
// with one ds_read_b128 a part, tile and step; the next step's loads are in
// flight during the current step's MFMAs.  int4 slot order within 8 K values
// is 0 4 1 5 2 6 3 7, the order the nibble masks 0x000F000F yield.
typedef __bf16 bf16x8v __attribute__((ext_vector_type(8)));
constexpr int kBfLP = 40;  // LDS row: 32 bf16 + 8 pad

__device__ __forceinline__ uint32_t hi16_pack(float a, float b) {
    // (bf16 bits of a) | (bf16 bits of b) << 16, both exact truncations
    return __builtin_amdgcn_perm(__float_as_uint(b), __float_as_uint(a), 0x07060302u);
}

// Weight formats of the bf16 MFMA GEMM (one 32-K step is one block or group
// of 32 elements):
//   I4: group-quantized int4 (A [M, K/2], fp32 scales and uint8 zeros [M, ng]);
//   I8: plain int8 (A [M, K]);
//   Q4_0: the separated Q4_0 upload's data region (16 bytes a block, element j
//     the low nibble of byte j and j + 16 the high) with fp16 scales [M, K/32];
//     the operand is 128 + u for the nibble u and the offset 136 (w = u - 8);
//   Q8_F32 / Q8_F16: separated Q8_0 (32 int8 a block), fp32 or fp16 scales;
//   Q8_RAW: the 36-byte blocks [fp32 scale][32 x int8].
enum class BfFmt { I4, I8, Q4_0, Q8_F32, Q8_F16, Q8_RAW };

template <BfFmt F, int TI, int PF>
__global__ void __launch_bounds__(256) bf16_gemm_kernel(const uint8_t* __restrict__ A, const float* __restrict__ B,
                                                        float* __restrict__ C, const void* __restrict__ scales,
                                                        const uint8_t* __restrict__ zeros, int M, int N, int K, int gs,
                                                        int ng) {
    constexpr bool INT4 = F == BfFmt::I4;                  // nibbles in the 0 4 1 5 2 6 3 7 slot order
    constexpr bool OFF = INT4 || F == BfFmt::Q4_0;          // an offset times sum x per step and row
    constexpr bool SCALED = F != BfFmt::I8;                 // a scale per step and row
    constexpr int TM = 32 * TI, TN = 32 * TI, CP = 16 * TI;  // tile, column pairs
    __shared__ __attribute__((aligned(16))) uint16_t Bs[2][3][TN][kBfLP];
    __shared__ float scs[2][TM], zzs[2][TM];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int li = lane & 15, lg = lane >> 4;
    int byi = blockIdx.y, bxi = blockIdx.x;
    const int m0 = byi * TM, n0 = bxi * TN;
    const int wm = (wave & 1) * 16 * TI, wn = (wave >> 1) * 16 * TI;
    const long rowbytes = (INT4 || F == BfFmt::Q4_0) ? K / 2 : F == BfFmt::Q8_RAW ? (long)(K / 32) * 36 : K;
    // this lane's A rows (one per row tile), clamped; rows past M load zeros
    int arow[TI];
    bool aok[TI];
#pragma unroll
    for (int i = 0; i < TI; i++) {
        const int m = m0 + wm + 16 * i + li;
        aok[i] = m < M;
        arow[i] = aok[i] ? m : 0;
    }
    // activation staging role: column pair cp, K octet ko (threads past 4 octets idle)
    const int cp = tid % CP, ko = tid / CP;
    const bool stager = TI == 4 || ko < 4;  // every thread stages with 128-column tiles
    const int bn = n0 + 2 * cp;
    const bool bok = stager && bn < N;

    // two register sets, step t in set t & 1.  PF = 2: step t + 2's loads are
    // issued during step t, so they have two steps of MFMAs to return (for
    // 64 x 64 tiles; with 128 x 128 tiles the second set's registers would
    // halve the waves a SIMD holds).  PF = 1: one set and a rolled loop, step
    // t + 1's loads issued during step t.
    uint2 araw8[2][TI];
    uint32_t araw4[2][TI];
    float2 braw[2][8];
    float sreg[2] = {0.0f, 0.0f}, zreg[2] = {0.0f, 0.0f};
    auto load_step = [&](auto parc, int k0) {
        constexpr int P = decltype(parc)::value;
#pragma unroll
        for (int i = 0; i < TI; i++) {
            if constexpr (INT4) {
                const long off = (long)arow[i] * rowbytes + (k0 + 8 * lg) / 2;
                araw4[P][i] = aok[i] ? *reinterpret_cast<const uint32_t*>(A + off) : 0x88888888u;  // u' = 0
            } else if constexpr (F == BfFmt::Q4_0) {
                // elements 8 lg .. 8 lg + 7 of block k0 / 32: the low (lg < 2) or high nibbles of bytes
                // 8 (lg & 1) .. +7
                const long off = (long)arow[i] * rowbytes + (k0 / 32) * 16 + 8 * (lg & 1);
                araw8[P][i] = aok[i] ? *reinterpret_cast<const uint2*>(A + off) : make_uint2(0u, 0u);
            } else if constexpr (F == BfFmt::Q8_RAW) {
                // 4-byte aligned only: two dword loads
                const long off = (long)arow[i] * rowbytes + (k0 / 32) * 36 + 4 + 8 * lg;
                araw8[P][i] = aok[i] ? make_uint2(*reinterpret_cast<const uint32_t*>(A + off),
                                                  *reinterpret_cast<const uint32_t*>(A + off + 4))
                                     : make_uint2(0u, 0u);
            } else {
                const long off = (long)arow[i] * rowbytes + k0 + 8 * lg;
                araw8[P][i] = aok[i] ? *reinterpret_cast<const uint2*>(A + off) : make_uint2(0u, 0u);
            }
        }
#pragma unroll
        for (int r = 0; r < 8; r++)
            braw[P][r] = bok ? *reinterpret_cast<const float2*>(B + (long)(k0 + 8 * ko + r) * N + bn) : make_float2(0.f, 0.f);
        if constexpr (SCALED) {
            if (tid < TM) {  // every step: each set holds its own step's scale (and offset)
                const int m = m0 + tid;
                const bool mok = m < M;
                const long mr = mok ? m : 0, bi = mr * (K / 32) + k0 / 32;
                if constexpr (INT4) {
                    const long gi = mr * ng + k0 / gs;
                    sreg[P] = mok ? static_cast<const float*>(scales)[gi] : 0.0f;
                    zreg[P] = 136.0f + (float)zeros[gi];
                } else if constexpr (F == BfFmt::Q4_0) {
                    sreg[P] = mok ? h2f(static_cast<const uint16_t*>(scales)[bi]) : 0.0f;
                    zreg[P] = 136.0f;
                } else if constexpr (F == BfFmt::Q8_F32) {
                    sreg[P] = mok ? static_cast<const float*>(scales)[bi] : 0.0f;
                } else if constexpr (F == BfFmt::Q8_F16) {
                    sreg[P] = mok ? h2f(static_cast<const uint16_t*>(scales)[bi]) : 0.0f;
                } else {  // Q8_RAW: the block's first 4 bytes
                    sreg[P] = mok ? *reinterpret_cast<const float*>(A + mr * rowbytes + (k0 / 32) * 36) : 0.0f;
                }
            }
        }
    };
    auto stage = [&](auto parc, int buf) {
        constexpr int P = decltype(parc)::value;
        // B parts: for each of the 2 columns, 8 K values in slot order
#pragma unroll
        for (int c = 0; c < 2 && stager; c++) {
            float v[8];
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const int r = INT4 ? ((j & 1) ? 4 + (j >> 1) : (j >> 1)) : j;  // slot j holds K offset r
                v[j] = c == 0 ? braw[P][r].x : braw[P][r].y;
            }
            uint32_t p1[4], p2[4], p3[4];
#pragma unroll
            for (int q = 0; q < 4; q++) {
                float a = v[2 * q], b = v[2 * q + 1];
                const float a1 = __uint_as_float(__float_as_uint(a) & 0xFFFF0000u);
                const float b1 = __uint_as_float(__float_as_uint(b) & 0xFFFF0000u);
                const float ar = a - a1, br = b - b1;
                const float a2 = __uint_as_float(__float_as_uint(ar) & 0xFFFF0000u);
                const float b2 = __uint_as_float(__float_as_uint(br) & 0xFFFF0000u);
                p1[q] = hi16_pack(a1, b1);
                p2[q] = hi16_pack(a2, b2);
                p3[q] = hi16_pack(ar - a2, br - b2);
            }
            const int n = 2 * cp + c;
            *reinterpret_cast<u32x4*>(&Bs[buf][0][n][8 * ko]) = (u32x4){p1[0], p1[1], p1[2], p1[3]};
            *reinterpret_cast<u32x4*>(&Bs[buf][1][n][8 * ko]) = (u32x4){p2[0], p2[1], p2[2], p2[3]};
            *reinterpret_cast<u32x4*>(&Bs[buf][2][n][8 * ko]) = (u32x4){p3[0], p3[1], p3[2], p3[3]};
        }
        if constexpr (SCALED) {
            if (tid < TM) {
                scs[buf][tid] = sreg[P];
                if constexpr (OFF) zzs[buf][tid] = zreg[P];
            }
        }
    };

    float4v acc[TI][TI];
#pragma unroll
    for (int i = 0; i < TI; i++)
#pragma unroll
        for (int j = 0; j < TI; j++) acc[i][j] = (float4v){0.f, 0.f, 0.f, 0.f};
    const int nsteps = K / 32;
    using P0 = std::integral_constant<int, 0>;
    using P1 = std::integral_constant<int, 1>;
    load_step(P0{}, 0);
    if (PF == 2 && nsteps > 1) load_step(P1{}, 32);
    stage(P0{}, 0);
    __syncthreads();
    // step t: Bs[t & 1] holds its activations, set t & 1 its weights; set
    // (t + 1) & 1 has step t + 1's loads in flight
    auto body = [&](auto parc, int t) {
        constexpr int P = decltype(parc)::value;
        using Q = std::integral_constant<int, PF == 2 ? 1 - P : P>;
        const int buf = t & 1;
        // decode this step's A operands, then reuse the set for step t + 2
        u32x4 av[TI];
#pragma unroll
        for (int i = 0; i < TI; i++) {
            if constexpr (INT4) {
                const uint32_t d = araw4[P][i] ^ 0x88888888u;
                av[i] = (u32x4){(d & 0x000F000Fu) | 0x43004300u, ((d >> 4) & 0x000F000Fu) | 0x43004300u,
                                ((d >> 8) & 0x000F000Fu) | 0x43004300u, ((d >> 12) & 0x000F000Fu) | 0x43004300u};
            } else if constexpr (F == BfFmt::Q4_0) {
                // elements in order, pairs (2h, 2h + 1) from bytes 2h, 2h + 1 moved to bytes 0 and 2, then
                // their low or high nibbles as the bf16 128 + u
                const uint32_t sh = 4u * (uint32_t)(lg >> 1);
                const uint32_t w2[2] = {araw8[P][i].x, araw8[P][i].y};
                uint32_t q[4];
#pragma unroll
                for (int h = 0; h < 4; h++) {
                    const uint32_t t2 = __builtin_amdgcn_perm(0u, w2[h >> 1], (h & 1) ? 0x0c030c02u : 0x0c010c00u);
                    q[h] = ((t2 >> sh) & 0x000F000Fu) | 0x43004300u;
                }
                av[i] = (u32x4){q[0], q[1], q[2], q[3]};
            } else {
                const uint32_t w2[2] = {araw8[P][i].x, araw8[P][i].y};
                uint32_t q[4];
#pragma unroll
                for (int h = 0; h < 4; h++) {
                    const uint32_t wd = w2[h >> 1];
                    const int b0 = 2 * (h & 1);
                    q[h] = hi16_pack((float)sext8(wd, b0), (float)sext8(wd, b0 + 1));
                }
                av[i] = (u32x4){q[0], q[1], q[2], q[3]};
            }
        }
        if constexpr (PF == 2) {
            if (t + 2 < nsteps) load_step(parc, 32 * (t + 2));
        } else {
            if (t + 1 < nsteps) load_step(Q{}, 32 * (t + 1));
        }
        float4v sc4[TI], zz4[TI];
        if constexpr (SCALED) {
#pragma unroll
            for (int i = 0; i < TI; i++) {
                sc4[i] = *reinterpret_cast<const float4v*>(&scs[buf][wm + 16 * i + 4 * lg]);
                if constexpr (OFF) zz4[i] = *reinterpret_cast<const float4v*>(&zzs[buf][wm + 16 * i + 4 * lg]);
            }
        }
#pragma unroll
        for (int j = 0; j < TI; j++) {
            const int n = wn + 16 * j + li;
            bf16x8v bp[3];
#pragma unroll
            for (int p = 0; p < 3; p++)
                bp[p] = __builtin_bit_cast(bf16x8v, *reinterpret_cast<const u32x4*>(&Bs[buf][p][n][8 * lg]));
            if constexpr (OFF) {
                const bf16x8v ones = __builtin_bit_cast(bf16x8v, (u32x4){0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u});
                float4v dx = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones, bp[0], (float4v){0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                dx = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones, bp[1], dx, 0, 0, 0);
                dx = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones, bp[2], dx, 0, 0, 0);
#pragma unroll
                for (int i = 0; i < TI; i++) {
                    const bf16x8v a = __builtin_bit_cast(bf16x8v, av[i]);
                    float4v d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bp[0], (float4v){0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                    d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bp[1], d, 0, 0, 0);
                    d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bp[2], d, 0, 0, 0);
#pragma unroll
                    for (int r = 0; r < 4; r++)
                        acc[i][j][r] = __builtin_fmaf(sc4[i][r], __builtin_fmaf(-zz4[i][r], dx[r], d[r]), acc[i][j][r]);
                }
            } else if constexpr (SCALED) {
#pragma unroll
                for (int i = 0; i < TI; i++) {
                    const bf16x8v a = __builtin_bit_cast(bf16x8v, av[i]);
                    float4v d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bp[0], (float4v){0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                    d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bp[1], d, 0, 0, 0);
                    d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bp[2], d, 0, 0, 0);
#pragma unroll
                    for (int r = 0; r < 4; r++) acc[i][j][r] = __builtin_fmaf(sc4[i][r], d[r], acc[i][j][r]);
                }
            } else {
#pragma unroll
                for (int i = 0; i < TI; i++) {
                    const bf16x8v a = __builtin_bit_cast(bf16x8v, av[i]);
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bp[0], acc[i][j], 0, 0, 0);
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bp[1], acc[i][j], 0, 0, 0);
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bp[2], acc[i][j], 0, 0, 0);
                }
            }
        }
        // the other buffer was last read in step t - 1, before the barrier that ended it
        if (t + 1 < nsteps) stage(Q{}, buf ^ 1);
        __syncthreads();
    };
    if constexpr (PF == 2) {
        for (int t = 0; t < nsteps; t += 2) {
            body(P0{}, t);
            if (t + 1 < nsteps) body(P1{}, t + 1);
        }
    } else {
        for (int t = 0; t < nsteps; t++) body(P0{}, t);
    }
#pragma unroll
    for (int i = 0; i < TI; i++)
#pragma unroll
        for (int j = 0; j < TI; j++) {
            const int n = n0 + wn + 16 * j + li;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int m = m0 + wm + 16 * i + 4 * lg + r;
                if (m < M && n < N) C[(long)m * N + n] = acc[i][j][r];
            }
        }
}

template <BfFmt F>
static void launch_bf16_gemm(hipStream_t st, const uint8_t* A, const float* B, float* C, const void* s,
                             const uint8_t* z, int M, int N, int K, int gs, int ng) {
    // 128 x 128 tiles while they give 256 workgroups, else 64 x 64, else 32 x 32 (one 16 x 16 tile a
    // wave) where fewer than 256 tiles of 64 remain, 192 for the formats with an offset, whose
    // all-ones MFMAs weigh most in the smallest tiles (us, 64 x 64 against 32 x 32: 4096 x 4096 at
    // 128 columns, 128 tiles of 64, int4 159.7 / 136.2, int8 106.7 / 94.0; 14336 x 4096 at 32 and 64
    // columns, 224 tiles of 64, Q8_0 133 / 100 and 136 / 126, Q4_0 at 64 columns 167 / 269)
    constexpr bool OFF = F == BfFmt::I4 || F == BfFmt::Q4_0;
    if ((long)ceil_div(M, 128) * ceil_div(N, 128) >= 256)
        bf16_gemm_kernel<F, 4, 1><<<dim3(ceil_div(N, 128), ceil_div(M, 128)), 256, 0, st>>>(A, B, C, s, z, M, N, K, gs, ng);
    else if ((long)ceil_div(M, 64) * ceil_div(N, 64) < (OFF ? 192 : 256))
        bf16_gemm_kernel<F, 1, 2><<<dim3(ceil_div(N, 32), ceil_div(M, 32)), 256, 0, st>>>(A, B, C, s, z, M, N, K, gs, ng);
    else
        bf16_gemm_kernel<F, 2, 2><<<dim3(ceil_div(N, 64), ceil_div(M, 64)), 256, 0, st>>>(A, B, C, s, z, M, N, K, gs, ng);
}

void bf16_gemm_q4_0(hipStream_t st, const uint8_t* data, const uint16_t* scales, const float* B, float* C, int M,
                    int N, int K) {
    launch_bf16_gemm<BfFmt::Q4_0>(st, data, B, C, scales, nullptr, M, N, K, 32, K / 32);
}

void bf16_gemm_q8_0(hipStream_t st, int layout, const uint8_t* data, const void* scales, const float* B, float* C,
                    int M, int N, int K) {
    if (layout == 0)
        launch_bf16_gemm<BfFmt::Q8_RAW>(st, data, B, C, nullptr, nullptr, M, N, K, 32, K / 32);
    else if (layout == 1)
        launch_bf16_gemm<BfFmt::Q8_F32>(st, data, B, C, scales, nullptr, M, N, K, 32, K / 32);
    else
        launch_bf16_gemm<BfFmt::Q8_F16>(st, data, B, C, scales, nullptr, M, N, K, 32, K / 32);
}

template <bool INT4>
static void launch_intq_bf16(hipStream_t st, const uint8_t* A, const float* B, float* C, const float* s,
                             const uint8_t* z, int M, int N, int K, int gs, int ng) {
    launch_bf16_gemm<INT4 ? BfFmt::I4 : BfFmt::I8>(st, A, B, C, s, z, M, N, K, gs, ng);
}

template <int V>
static void launch_intq_mfma(hipStream_t st, const void* A, const void* B, float* C, const float* s, const uint8_t* z,
                             int M, int N, int K, int gs, int ng) {
    const dim3 g(ceil_div(N, kIqTN), ceil_div(M, kIqTM));
    intq_mfma_kernel<V><<<g, 256, 0, st>>>(A, B, C, s, z, M, N, K, gs, ng);
}

}  // namespace zt

using namespace zt;

// Grid limits of the MFMA GEMM: blockIdx.y holds M / 64.
static bool intq_grid_ok(long M, long N) { return (M + kIqTM - 1) / kIqTM <= 65535 && (N + kIqTN - 1) / kIqTN < 0x7fffffffL; }

// Batches of 4-64 columns (N % 4 == 0) on the row-block MFMA GEMM: one
// launch per 4 or 8 columns, each streaming the weights once, so its time
// grows with M N while the bf16 tile GEMM's stays flat up to 128 columns.
// Measured (us, row-block / bf16): int4 4096 x 4096 batch 8 7.7 / 170,
// 64 72 / 172; 14336 x 4096 batch 32 91 / 176, 64 183 / 176; int8 4096 x
// 4096 batch 64 83 / 115, 14336 x 4096 batch 16 58 / 118, 32 139 / 118.  So
// up to 16 columns always, and to 64 while M N <= 2^19 (int4) or 2^18 (int8).
static bool intq_rb_ok(int N, int K, long M, long ng, const void* a, const void* B, bool int4) {
    return N >= 4 && (N <= 16 || (N <= 64 && M * N <= (int4 ? 1L << 19 : 1L << 18))) && K % 32 == 0 && ((uintptr_t)a & 15) == 0 && M * ng * 4 < 0x7fffffffL &&
           rbf_ok<RbFmt::INT8>(N, K / 32, M, B);
}

ZT_EXPORT int zt_gemm_int8_f32(const void* A, const float* B, float* C, int M, int K, int N, hipStream_t stream) {
    if (M < 0 || K < 0 || N < 0) return (int)hipErrorInvalidValue;
    if (M == 0 || N == 0) return (int)hipSuccess;
    if (A == nullptr || C == nullptr || (K > 0 && B == nullptr) || !intq_grid_ok(M, N)) return (int)hipErrorInvalidValue;
    const uint8_t* a = static_cast<const uint8_t*>(A);
    if (K > 0 && intq_rb_ok(N, K, M, 1, a, B, false))
        launch_rbf<RbFmt::INT8>(nullptr, a, B, C, M, K / 32, N, stream);
    else if (N <= 4 && K > 0 && K % 16 == 0 && ((uintptr_t)a & 15) == 0 && ((uintptr_t)B & 15) == 0)
        launch_intq_gemv<false>(stream, a, B, C, nullptr, nullptr, M, K, N, 1, 1);
    else if (K > 0 && K % 32 == 0 && N % 2 == 0 && ((uintptr_t)a & 7) == 0 && ((uintptr_t)B & 7) == 0)
        launch_intq_bf16<false>(stream, a, B, C, nullptr, nullptr, M, N, K, 1, 1);
    else
        launch_intq_mfma<0>(stream, A, B, C, nullptr, nullptr, M, N, K, 1, 1);
    return (int)hipGetLastError();
}

ZT_EXPORT int zt_gemm_int4_f32(const void* A, const float* B, float* C, const float* scales, const void* zeros, int M,
                               int K, int N, int group_size, hipStream_t stream) {
    if (K % 2 != 0 || group_size <= 0) return (int)hipErrorInvalidValue;  // gemm_int4.cu:64-69
    if (M < 0 || K < 0 || N < 0) return (int)hipErrorInvalidValue;
    if (M == 0 || N == 0) return (int)hipSuccess;
    if (A == nullptr || C == nullptr || !intq_grid_ok(M, N)) return (int)hipErrorInvalidValue;
    if (K > 0 && (B == nullptr || scales == nullptr || zeros == nullptr)) return (int)hipErrorInvalidValue;
    const int ng = K > 0 ? ceil_div(K, group_size) : 1;
    const uint8_t* a = static_cast<const uint8_t*>(A);
    const uint8_t* z = static_cast<const uint8_t*>(zeros);
    if (K > 0 && group_size % 32 == 0 && intq_rb_ok(N, K, M, ng, a, B, true) && ((uintptr_t)scales & 3) == 0)
        launch_rbf<RbFmt::INT4G>(scales, a, B, C, M, K / 32, N, stream, z, group_size / 32, ng);
    else if (N <= 4 && K > 0 && K % 16 == 0 && group_size % 16 == 0 && ((uintptr_t)a & 7) == 0 && ((uintptr_t)B & 15) == 0)
        launch_intq_gemv<true>(stream, a, B, C, scales, z, M, K, N, group_size, ng);
    else if (K > 0 && K % 32 == 0 && group_size % 32 == 0 && N % 2 == 0 && ((uintptr_t)a & 3) == 0 &&
             ((uintptr_t)B & 7) == 0)
        launch_intq_bf16<true>(stream, a, B, C, scales, z, M, N, K, group_size, ng);
    else
        launch_intq_mfma<1>(stream, A, B, C, scales, z, M, N, K, group_size, ng);
    return (int)hipGetLastError();
}

ZT_EXPORT int zt_gemm_int4_f32_rmul(const void* W, const float* B, float* C, const float* scales, const void* zeros,
                                    int batch, int in_features, int out_features, int group_size, hipStream_t stream) {
    if (out_features % 2 != 0 || group_size <= 0) return (int)hipErrorInvalidValue;  // gemm_int4.cu:122-127
    if (batch < 0 || in_features < 0 || out_features < 0) return (int)hipErrorInvalidValue;
    if (batch == 0 || out_features == 0) return (int)hipSuccess;
    if (C == nullptr || !intq_grid_ok(batch, out_features)) return (int)hipErrorInvalidValue;
    if (in_features > 0 && (W == nullptr || B == nullptr || scales == nullptr || zeros == nullptr))
        return (int)hipErrorInvalidValue;
    const int ng = ceil_div(out_features, group_size);
    const uint8_t* z = static_cast<const uint8_t*>(zeros);
    const uint8_t* w = static_cast<const uint8_t*>(W);
    // the 16-byte-load kernel up to K = 8192; beyond, its half as many
    // workgroups each walk too long a K (us, batch 1 / 4: in x out 4096 x 4096
    // 19.2 / 22.1 against 19.1 / 27.3, 4096 x 14336 41.1 / 45.5 against
    // 64.1 / 102.6, 14336 x 4096 68.8 / 68.5 against 53.2 / 57.4).  Past
    // batch 4 the same kernels run once per group of up to 4 rows of X: the
    // fp32 MFMA GEMM's out / 64 workgroups each walk all of K whatever the
    // batch (376 us at 4096 x 4096 for batches 8-32, 1310 at 4096 x 14336),
    // so groups of 4 win up to batch 64 on the 16-byte kernel (about 22 us a
    // group) and batch 16 on the 8-byte one (about 57 us a group at 14336 x 4096).
    const bool v16 = in_features > 0 && in_features <= 8192 && out_features % 32 == 0 && group_size % 32 == 0 &&
                     ((uintptr_t)w & 15) == 0 && (long)in_features * (out_features / 2) < 0x7fffffffL &&
                     (long)in_features * ng * 4 < 0x7fffffffL;
    const bool valu = in_features > 0 && out_features % 16 == 0 && group_size % 16 == 0 && ((uintptr_t)w & 7) == 0;
    if ((v16 && batch <= 64) || (valu && batch <= 16)) {
        for (int b0 = 0; b0 < batch; b0 += 4) {
            const float* xb = B + (long)b0 * in_features;
            float* cb = C + (long)b0 * out_features;
            const int nb = min(4, batch - b0);
            if (v16) {
                switch (nb) {
                    case 1: launch_int4_rmul_v16<1>(stream, w, xb, cb, scales, z, in_features, out_features, group_size, ng); break;
                    case 2: launch_int4_rmul_v16<2>(stream, w, xb, cb, scales, z, in_features, out_features, group_size, ng); break;
                    case 3: launch_int4_rmul_v16<3>(stream, w, xb, cb, scales, z, in_features, out_features, group_size, ng); break;
                    default: launch_int4_rmul_v16<4>(stream, w, xb, cb, scales, z, in_features, out_features, group_size, ng); break;
                }
            } else {
                switch (nb) {
                    case 1: launch_int4_rmul_valu<1>(stream, w, xb, cb, scales, z, in_features, out_features, group_size, ng); break;
                    case 2: launch_int4_rmul_valu<2>(stream, w, xb, cb, scales, z, in_features, out_features, group_size, ng); break;
                    case 3: launch_int4_rmul_valu<3>(stream, w, xb, cb, scales, z, in_features, out_features, group_size, ng); break;
                    default: launch_int4_rmul_valu<4>(stream, w, xb, cb, scales, z, in_features, out_features, group_size, ng); break;
                }
            }
        }
    } else {
        launch_intq_mfma<2>(stream, B, W, C, scales, z, batch, out_features, in_features, group_size, ng);
    }
    return (int)hipGetLastError();
}

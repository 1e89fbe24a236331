// Q8_0 GEMV / small-batch GEMM and dequantization for gfx950.
//
// Q8_0 here is the Q8Storage format: 32 int8 weights and one fp32 scale per
// block, w = float(q) * scale (tensor/quantized.go:278-363).  Its raw
// serialisation is 36-byte blocks [fp32 scale LE][32 x int8]
// (tensor/quantized.go:425-438), which leaves the int8 payload only 4-byte
// aligned.  Two device layouts are accepted:
//   * raw:       the 36-byte blocks as RawBytes() produces them (the layout
//                gemm_q8_f32 takes, internal/cuda/kernels/gemm_q8.cu:3-6);
//   * separated: [scales: nblk * 4 bytes][pad to 16 bytes][data: nblk * 32 bytes],
//                the Q8 counterpart of Q4's RawBytesGPU, built once at
//                upload (zt_q8_raw_to_gpu on the host or zt_q8_repack on the
//                device).  Every block's 32 bytes are two aligned 128-bit
//                loads, so a wave reads 2 KiB of a row contiguously.
//
// Batch 1 uses the quad mapping of zt_q4.hip (four lanes per block, see
// gemv_q8_quad_kernel); batches of 4, 8, 12, ... columns run the row-block
// MFMA GEMM of zt_rbmfma.h (rbf_kernel); other batches use lane <-> block
// column, R rows per wave with the 32 activations held in registers, one
// column per grid row, split-K across the waves of a workgroup.  Decode: q XOR 0x80 is q+128 as an unsigned byte,
// which v_cvt_f32_ubyte converts directly; sum (q+128) x - 128 sum x
// recovers the signed dot product.
#include "zt_bf16gemm.h"
#include "zt_common.h"
#include "zt_rbmfma.h"

namespace zt {

constexpr int kRaw36 = 0, kSep32 = 1, kSep16 = 2;

// Scale of block blk in a separated layout (fp16 scales widen exactly).
template <int L>
__device__ __forceinline__ float sep_scale(const uint8_t* base, long blk) {
    if constexpr (L == kSep16) return h2f(reinterpret_cast<const uint16_t*>(base)[blk]);
    else return reinterpret_cast<const float*>(base)[blk];
}

__device__ __forceinline__ float q8_dot_dwords(const uint32_t* d, const float (&xv)[32], float xsum) {
    float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const uint32_t u = d[i] ^ 0x80808080u;  // bytes q+128
#pragma unroll
        for (int j = 0; j < 4; j += 2) {
            s0 = fmaf((float)((u >> (8 * j)) & 0xffu), xv[4 * i + j], s0);
            s1 = fmaf((float)((u >> (8 * j + 8)) & 0xffu), xv[4 * i + j + 1], s1);
        }
    }
    return (s0 + s1) - 128.0f * xsum;
}

template <class XT, bool CONTIG>
__device__ __forceinline__ void load_x32f(const XT* __restrict__ x, long x_stride, int b, float (&xv)[32]) {
    if constexpr (CONTIG) {
        const float4* p = reinterpret_cast<const float4*>(x + (long)b * 32);
#pragma unroll
        for (int i = 0; i < 8; i++) {
            float4 t = p[i];
            xv[4 * i] = t.x; xv[4 * i + 1] = t.y; xv[4 * i + 2] = t.z; xv[4 * i + 3] = t.w;
        }
    } else {
#pragma unroll
        for (int i = 0; i < 32; i++) xv[i] = x[((long)b * 32 + i) * x_stride];
    }
}

// Layout L: kRaw36 = raw 36-byte blocks; kSep32 = separated, fp32 scales;
// kSep16 = separated, fp16 scales (GGUF Q8_0 after its upload repack).
template <int L, int R, bool CONTIG>
__global__ void __launch_bounds__(512) gemv_q8_kernel(const uint8_t* __restrict__ base, long data_offset,
                                                      const float* __restrict__ x, float* __restrict__ y,
                                                      long xy_stride, int rows, int kb) {
    __shared__ float red[8 * R];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nwaves = blockDim.x >> 6;
    x += blockIdx.y;
    y += blockIdx.y;
    const int row0 = blockIdx.x * R;
    long rbase[R];
#pragma unroll
    for (int r = 0; r < R; r++) rbase[r] = (long)min(row0 + r, rows - 1) * kb;
    const uint4* data = reinterpret_cast<const uint4*>(base + data_offset);

    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.0f;

    for (int b = wave * kWave + lane; b < kb; b += nwaves * kWave) {
        uint32_t d[R][8];
        float s[R];
#pragma unroll
        for (int r = 0; r < R; r++) {
            const long blk = rbase[r] + b;
            if constexpr (L != kRaw36) {
                const uint4 a = ld_stream(&data[2 * blk]);
                const uint4 c = ld_stream(&data[2 * blk + 1]);
                d[r][0] = a.x; d[r][1] = a.y; d[r][2] = a.z; d[r][3] = a.w;
                d[r][4] = c.x; d[r][5] = c.y; d[r][6] = c.z; d[r][7] = c.w;
                s[r] = sep_scale<L>(base, blk);
            } else {
                const uint32_t* p = reinterpret_cast<const uint32_t*>(base + blk * 36);
                s[r] = __uint_as_float(__builtin_nontemporal_load(p));
#pragma unroll
                for (int i = 0; i < 8; i++) d[r][i] = __builtin_nontemporal_load(p + 1 + i);
            }
        }
        float xv[32];
        load_x32f<float, CONTIG>(x, xy_stride, b, xv);
        float xsum = 0.0f;
#pragma unroll
        for (int i = 0; i < 32; i++) xsum += xv[i];
#pragma unroll
        for (int r = 0; r < R; r++) acc[r] = fmaf(s[r], q8_dot_dwords(d[r], xv, xsum), acc[r]);
    }
    block_reduce_store<R>(acc, red, y, xy_stride, row0, rows);
}

template <int L, bool CONTIG>
static void launch_q8(int R, dim3 g, dim3 b, hipStream_t st, const uint8_t* base, long off, const float* x,
                      float* y, long stride, int rows, int kb) {
    switch (R) {
        case 8: gemv_q8_kernel<L, 8, CONTIG><<<g, b, 0, st>>>(base, off, x, y, stride, rows, kb); break;
        case 4: gemv_q8_kernel<L, 4, CONTIG><<<g, b, 0, st>>>(base, off, x, y, stride, rows, kb); break;
        case 2: gemv_q8_kernel<L, 2, CONTIG><<<g, b, 0, st>>>(base, off, x, y, stride, rows, kb); break;
        default: gemv_q8_kernel<L, 1, CONTIG><<<g, b, 0, st>>>(base, off, x, y, stride, rows, kb); break;
    }
}

// Batch-1 GEMV: four lanes share one block.  Lane q of a quad takes bytes
// 8q .. 8q+7 of the block's 32 int8 weights (one 8-byte load in the
// separated layout; in the raw 36-byte blocks one 12-byte load of dwords
// 2q .. 2q+2, whose second and third are the lane's data and whose first is,
// in lane 0, the block's scale, broadcast over the quad) and the matching 8
// activations as two 16-byte loads, so a quad reads its block's 128 bytes of
// activations contiguously.  R rows per wave, split-K over the waves.
template <int L, int R>
__global__ void __launch_bounds__(512) gemv_q8_quad_kernel(const uint8_t* __restrict__ base, long data_offset,
                                                           const float* __restrict__ x, float* __restrict__ y,
                                                           int rows, int kb) {
    __shared__ float red[8 * R];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nwaves = blockDim.x >> 6;
    const int q = lane & 3;
    const int row0 = blockIdx.x * R;
    long rbase[R];
#pragma unroll
    for (int r = 0; r < R; r++) rbase[r] = (long)min(row0 + r, rows - 1) * kb;
    const uint2* data = reinterpret_cast<const uint2*>(base + data_offset);
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.0f;
    // raw blocks: one buffer resource a row (wave-uniform), so offsets within
    // a row fit 32 bits at any matrix size
    __amdgpu_buffer_rsrc_t rrow[L == kRaw36 ? R : 1];
    if constexpr (L == kRaw36) {
#pragma unroll
        for (int r = 0; r < R; r++)
            rrow[r] = __builtin_amdgcn_make_buffer_rsrc((void*)(base + rbase[r] * 36), (short)0, kb * 36, 0x00020000);
    }

    for (int b = wave * 16 + (lane >> 2); b < kb; b += nwaves * 16) {
        uint32_t d[R][2];
        float s[R];
#pragma unroll
        for (int r = 0; r < R; r++) {
            const long blk = rbase[r] + b;
            if constexpr (L != kRaw36) {
                typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
                const u32x2 v = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(&data[blk * 4 + q]));
                d[r][0] = v.x;
                d[r][1] = v.y;
                s[r] = sep_scale<L>(base, blk);
            } else {
                typedef uint32_t u32x3 __attribute__((ext_vector_type(3)));
                const u32x3 v = __builtin_amdgcn_raw_buffer_load_b96(rrow[r], (uint32_t)(b * 36 + 8 * q), 0, 2);
                d[r][0] = v.y;
                d[r][1] = v.z;
                // quad_perm [0, 0, 0, 0]: lane 0's first dword is the block's scale
                s[r] = __int_as_float(__builtin_amdgcn_update_dpp(0, (int)v.x, 0x00, 0xF, 0xF, false));
                (void)blk;
            }
        }
        const float4 xa = *reinterpret_cast<const float4*>(x + (long)b * 32 + 8 * q);
        const float4 xb = *reinterpret_cast<const float4*>(x + (long)b * 32 + 8 * q + 4);
        const float xv[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
        const float xsum = ((xa.x + xa.y) + (xa.z + xa.w)) + ((xb.x + xb.y) + (xb.z + xb.w));
#pragma unroll
        for (int r = 0; r < R; r++) {
            float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
            for (int i = 0; i < 2; i++) {
                const uint32_t u = d[r][i] ^ 0x80808080u;  // bytes q+128
                s0 = fmaf((float)(u & 0xffu), xv[4 * i], s0);
                s1 = fmaf((float)((u >> 8) & 0xffu), xv[4 * i + 1], s1);
                s0 = fmaf((float)((u >> 16) & 0xffu), xv[4 * i + 2], s0);
                s1 = fmaf((float)(u >> 24), xv[4 * i + 3], s1);
            }
            acc[r] = fmaf(s[r], (s0 + s1) - 128.0f * xsum, acc[r]);
        }
    }
    block_reduce_store<R>(acc, red, y, 1, row0, rows);
}

// The same quad mapping in the fixed-step form of the Q4_0 kernel: each wave
// does S steps of 16 blocks, every load issued before any arithmetic as
// buffer loads with the wave-uniform row offsets as scalar offsets; lanes
// past the last block read zeros.  On the raw 36-byte blocks (9 dwords: the
// fp32 scale, then 8 data dwords) lane q of a quad loads the 12 bytes at
// block offset 8q, dwords 2q .. 2q + 2: its data dwords 2q + 1, 2q + 2 are
// always the second and third, and lane 0's first is the block's scale,
// which a DPP quad broadcast hands to the other three.  One load instruction
// a block and row, where a separate scale load touched the same lines again.
template <int L, int S, int R>
__global__ void __launch_bounds__(1024) gemv_q8_steps_kernel(const uint8_t* __restrict__ base, long data_offset,
                                                             const float* __restrict__ x, float* __restrict__ y,
                                                             int rows, int kb) {
    __shared__ float red[16 * R];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int q = lane & 3;
    const int row0 = blockIdx.x * R;
    constexpr uint32_t SB = L == kSep16 ? 2u : 4u;  // bytes per scale
    const __amdgpu_buffer_rsrc_t rd =
        __builtin_amdgcn_make_buffer_rsrc((void*)(base + data_offset), (short)0, 0x7fffffff, 0x00020000);
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0, 0x7fffffff, 0x00020000);
    const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc((void*)x, (short)0, kb * 128, 0x00020000);
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
    typedef uint32_t u32x3 __attribute__((ext_vector_type(3)));
    u32x2 d[S][R];
    uint32_t sc[S][R];
    u32x4 xa[S], xb[S];
#pragma unroll
    for (int t = 0; t < S; t++) {
        const int b = (wave * S + t) * 16 + (lane >> 2);
        const bool ok = b < kb;
#pragma unroll
        for (int r = 0; r < R; r++) {
            const uint32_t row = (uint32_t)min(row0 + r, rows - 1);
            if constexpr (L == kRaw36) {
                const u32x3 v = __builtin_amdgcn_raw_buffer_load_b96(rs, ok ? (uint32_t)(b * 36 + q * 8) : 0x80000000u,
                                                                     row * (uint32_t)kb * 36u, 2);  // nontemporal
                d[t][r] = (u32x2){v.y, v.z};
                sc[t][r] = v.x;  // the scale in lane 0 of the quad
            } else
                d[t][r] = __builtin_amdgcn_raw_buffer_load_b64(rd, ok ? (uint32_t)(b * 32 + q * 8) : 0x80000000u,
                                                               row * (uint32_t)kb * 32u, 2);  // nontemporal
        }
    }
#pragma unroll
    for (int t = 0; t < S; t++) {
        const int b = (wave * S + t) * 16 + (lane >> 2);
        const bool ok = b < kb;
#pragma unroll
        for (int r = 0; r < R; r++) {
            const uint32_t row = (uint32_t)min(row0 + r, rows - 1);
            const uint32_t so = ok ? (uint32_t)b * SB : 0x80000000u;
            if constexpr (L == kRaw36)
                continue;
            else if constexpr (L == kSep16)
                sc[t][r] = __builtin_amdgcn_raw_buffer_load_b16(rs, so, row * (uint32_t)kb * SB, 0);
            else
                sc[t][r] = __builtin_amdgcn_raw_buffer_load_b32(rs, so, row * (uint32_t)kb * SB, 0);
        }
        const uint32_t xo = ok ? (uint32_t)(b * 128 + q * 32) : 0x80000000u;
        xa[t] = __builtin_amdgcn_raw_buffer_load_b128(rx, xo, 0, 0);
        xb[t] = __builtin_amdgcn_raw_buffer_load_b128(rx, xo + 16, 0, 0);
    }
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.0f;
#pragma unroll
    for (int t = 0; t < S; t++) {
        const float xv[8] = {__uint_as_float(xa[t].x), __uint_as_float(xa[t].y), __uint_as_float(xa[t].z),
                             __uint_as_float(xa[t].w), __uint_as_float(xb[t].x), __uint_as_float(xb[t].y),
                             __uint_as_float(xb[t].z), __uint_as_float(xb[t].w)};
        const float m128 = -128.0f * (((xv[0] + xv[1]) + (xv[2] + xv[3])) + ((xv[4] + xv[5]) + (xv[6] + xv[7])));
#pragma unroll
        for (int r = 0; r < R; r++) {
            float s0 = m128, s1 = 0.0f;
#pragma unroll
            for (int i = 0; i < 2; i++) {
                const uint32_t u = d[t][r][i] ^ 0x80808080u;  // bytes q+128
                s0 = fmaf((float)(u & 0xffu), xv[4 * i], s0);
                s1 = fmaf((float)((u >> 8) & 0xffu), xv[4 * i + 1], s1);
                s0 = fmaf((float)((u >> 16) & 0xffu), xv[4 * i + 2], s0);
                s1 = fmaf((float)(u >> 24), xv[4 * i + 3], s1);
            }
            const uint32_t sb = L == kRaw36 ? (uint32_t)__builtin_amdgcn_update_dpp(0, (int)sc[t][r], 0x00, 0xF, 0xF, false)
                                            : sc[t][r];  // raw: quad_perm [0, 0, 0, 0]
            const float scale = L == kSep16 ? h2f(sb & 0xffffu) : __uint_as_float(sb);
            acc[r] = fmaf(scale, s0 + s1, acc[r]);
        }
    }
    block_reduce_store<R>(acc, red, y, 1, row0, rows);
}

template <int L, int S>
static void launch_q8_steps(int R, dim3 g, dim3 b, hipStream_t st, const uint8_t* base, long off, const float* x,
                            float* y, int rows, int kb) {
    switch (R) {
        case 8: gemv_q8_steps_kernel<L, S, 8><<<g, b, 0, st>>>(base, off, x, y, rows, kb); break;
        case 4: gemv_q8_steps_kernel<L, S, 4><<<g, b, 0, st>>>(base, off, x, y, rows, kb); break;
        case 2: gemv_q8_steps_kernel<L, S, 2><<<g, b, 0, st>>>(base, off, x, y, rows, kb); break;
        default: gemv_q8_steps_kernel<L, S, 1><<<g, b, 0, st>>>(base, off, x, y, rows, kb); break;
    }
}

template <int L>
static void launch_q8_quad(int R, dim3 g, dim3 b, hipStream_t st, const uint8_t* base, long off, const float* x,
                           float* y, int rows, int kb) {
    switch (R) {
        case 8: gemv_q8_quad_kernel<L, 8><<<g, b, 0, st>>>(base, off, x, y, rows, kb); break;
        case 4: gemv_q8_quad_kernel<L, 4><<<g, b, 0, st>>>(base, off, x, y, rows, kb); break;
        case 2: gemv_q8_quad_kernel<L, 2><<<g, b, 0, st>>>(base, off, x, y, rows, kb); break;
        default: gemv_q8_quad_kernel<L, 1><<<g, b, 0, st>>>(base, off, x, y, rows, kb); break;
    }
}

template <int L>
static int gemm_q8(const void* A, const float* B, float* C, int M, int K, int N, long data_offset, hipStream_t st) {
    if (M < 0 || N < 0 || K < 0 || K % 32 != 0 || data_offset < 0 || N > 65535) return (int)hipErrorInvalidValue;
    if (M == 0 || N == 0) return (int)hipSuccess;
    if (A == nullptr || B == nullptr || C == nullptr) return (int)hipErrorInvalidValue;
    const uint8_t* base = static_cast<const uint8_t*>(A);
    if ((uintptr_t)base & 3) return (int)hipErrorInvalidValue;
    if (L != kRaw36 && ((uintptr_t)(base + data_offset) & 15)) return (int)hipErrorInvalidValue;
    if (N == 1 && ((uintptr_t)B & 15)) return (int)hipErrorInvalidValue;
    const int kb = K / 32;
    if (N == 1) {
        // fixed steps: S = 1 for K <= 4096, 2 (up to 16 waves) up to K = 8192;
        // the loop kernel beyond (at K = 14336 it measured 1-7% faster on
        // the separated layout)
        const bool steps_ok = kb <= 256;
        if ((long)M * kb * (L == kRaw36 ? 36 : 32) < 0x7fffffffL && data_offset < 0x7fffffffL && steps_ok) {
            const int S = kb <= 128 ? 1 : 2;
            int nws = ceil_div(kb, 16 * S);
            if (nws > 12) nws = 16;
            const int Rs = pick_rows_per_wave(M, nws, 1, 2048);
            const dim3 g(ceil_div(M, Rs)), blk(nws * kWave);
            if (S == 1)
                launch_q8_steps<L, 1>(Rs, g, blk, st, base, data_offset, B, C, M, kb);
            else
                launch_q8_steps<L, 2>(Rs, g, blk, st, base, data_offset, B, C, M, kb);
            return (int)hipGetLastError();
        }
        const int nw = min(8, ceil_div(kb, 16));
        const int R = pick_rows_per_wave(M, nw, 1, 2048);
        launch_q8_quad<L>(R, dim3(ceil_div(M, R)), dim3(nw * kWave), st, base, data_offset, B, C, M, kb);
        return (int)hipGetLastError();
    }
    // Wide batches (prefill widths): the bf16 MFMA tile GEMM of zt_intq.hip from 128 columns, from 32
    // at 8192 rows and more, from 64 past K = 8192 (us, separated layout, row-block against tile
    // GEMM, 4096 x 4096 / 14336 x 4096 / 4096 x 14336 rows x K: 32 columns 43 / 147 / 189 against
    // 88 / 100 / 310; 64 columns 86 / 292 / 380 against 90 / 126 / 312; 128 columns 173 / 589 / 760
    // against 99 / 161 / 344; 512 columns 695 / 2333 / 3039 against 154 / 256 / 520; the raw blocks
    // alike)
    const bool wide = N >= 128 || (N >= 32 && M >= 8192) || (N >= 64 && K > 8192);
    if (wide && N % 2 == 0 && ((uintptr_t)B & 7) == 0 && (long)ceil_div(M, 32) <= 65535) {
        bf16_gemm_q8_0(st, L, L == kRaw36 ? base : base + data_offset, base, B, C, M, N, K);
        return (int)hipGetLastError();
    }
    // N = 4, 8, 12, ...: the row-block MFMA GEMM, every weight read once per
    // group of 4 or 8 columns
    constexpr RbFmt RF = L == kRaw36 ? RbFmt::Q8_RAW : L == kSep32 ? RbFmt::Q8_SEP : RbFmt::Q8_SEP16;
    if (rbf_ok<RF>(N, kb, M, B) && data_offset < 0x7fffffffL) {
        launch_rbf<RF>(base, L == kRaw36 ? base : base + data_offset, B, C, M, kb, N, st);
        return (int)hipGetLastError();
    }
    const int nwaves = kb <= 64 ? 1 : (kb >= 8 * 64 ? 8 : ceil_div(kb, 64));
    const int R = pick_rows_per_wave(M, nwaves, N, 2048);
    dim3 grid(ceil_div(M, R), N), block(nwaves * kWave);
    launch_q8<L, false>(R, grid, block, st, base, data_offset, B, C, N, M, kb);
    return (int)hipGetLastError();
}

// ------------------------------------------------------------ dequantize

template <int L>
__global__ void dequant_q8_kernel(const uint8_t* __restrict__ base, long data_offset, float* __restrict__ out,
                                  long nelem) {
    const long blk = (long)blockIdx.x * blockDim.x + threadIdx.x;
    const long nblk = (nelem + 31) / 32;
    if (blk >= nblk) return;
    float scale;
    const uint8_t* q;
    if constexpr (L != kRaw36) {
        scale = sep_scale<L>(base, blk);
        q = base + data_offset + blk * 32;
    } else {
        scale = *reinterpret_cast<const float*>(base + blk * 36);
        q = base + blk * 36 + 4;
    }
    const long rem = nelem - blk * 32;
    const int n = rem >= 32 ? 32 : (int)rem;
    float* o = out + blk * 32;
    for (int j = 0; j < n; j++) o[j] = (float)(int8_t)q[j] * scale;
}

template <int L>
static int dequant_q8(const void* A, float* out, long nelem, long data_offset, hipStream_t st) {
    if (nelem < 0 || data_offset < 0) return (int)hipErrorInvalidValue;
    if (nelem == 0) return (int)hipSuccess;
    if ((uintptr_t)A & 3) return (int)hipErrorInvalidValue;
    const long nblk = (nelem + 31) / 32;
    dequant_q8_kernel<L><<<ceil_div(nblk, 256), 256, 0, st>>>(static_cast<const uint8_t*>(A), data_offset, out,
                                                                 nelem);
    return (int)hipGetLastError();
}

// Raw 36-byte blocks -> separated layout, one thread per block.
__global__ void q8_repack_kernel(const uint8_t* __restrict__ raw, uint8_t* __restrict__ out, long nblk,
                                 long data_offset) {
    const long blk = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (blk >= nblk) return;
    const uint32_t* src = reinterpret_cast<const uint32_t*>(raw + blk * 36);
    reinterpret_cast<uint32_t*>(out)[blk] = src[0];
    uint32_t* dst = reinterpret_cast<uint32_t*>(out + data_offset + blk * 32);
#pragma unroll
    for (int i = 0; i < 8; i++) dst[i] = src[1 + i];
}

}  // namespace zt

using namespace zt;

// Byte offset of the data region in the separated Q8_0 layout.
ZT_EXPORT long zt_q8_gpu_data_offset(long nblk) { return (nblk * 4 + 15) & ~15L; }

ZT_EXPORT long zt_q8_gpu_bytes(long nblk) { return zt_q8_gpu_data_offset(nblk) + nblk * 32; }

ZT_EXPORT int zt_gemm_q8_f32(const void* A_q8, const float* B, float* C, int M, int K, int N, hipStream_t stream) {
    return gemm_q8<kRaw36>(A_q8, B, C, M, K, N, 0, stream);
}

ZT_EXPORT int zt_gemm_q8sep_f32(const void* A_q8, const float* B, float* C, int M, int K, int N, long data_offset,
                                hipStream_t stream) {
    return gemm_q8<kSep32>(A_q8, B, C, M, K, N, data_offset, stream);
}

ZT_EXPORT int zt_dequant_q8_f32(const void* A_q8, float* out, long nelem, hipStream_t stream) {
    return dequant_q8<kRaw36>(A_q8, out, nelem, 0, stream);
}

ZT_EXPORT int zt_dequant_q8sep_f32(const void* A_q8, float* out, long nelem, long data_offset, hipStream_t stream) {
    return dequant_q8<kSep32>(A_q8, out, nelem, data_offset, stream);
}

ZT_EXPORT int zt_q8_repack(const void* raw, void* out, long nblk, hipStream_t stream) {
    if (nblk < 0 || ((uintptr_t)raw & 3) || ((uintptr_t)out & 15)) return (int)hipErrorInvalidValue;
    if (nblk == 0) return (int)hipSuccess;
    q8_repack_kernel<<<ceil_div(nblk, 256), 256, 0, stream>>>(static_cast<const uint8_t*>(raw),
                                                              static_cast<uint8_t*>(out), nblk,
                                                              zt_q8_gpu_data_offset(nblk));
    return (int)hipGetLastError();
}

// GGUF Q8_0 (tensor/mmap_storage.go:265-284: 34-byte blocks [fp16 d][32 x
// int8]) over its separated upload layout [fp16 d, nblk*2][pad 16][int8,
// nblk*32]: data_offset = zt_q8gguf_gpu_data_offset(nblk).
ZT_EXPORT int zt_gemm_q8gguf_f32(const void* A, const float* B, float* C, int M, int K, int N, long data_offset,
                                 hipStream_t stream) {
    return gemm_q8<kSep16>(A, B, C, M, K, N, data_offset, stream);
}

ZT_EXPORT int zt_dequant_q8gguf_f32(const void* A, float* out, long nelem, long data_offset, hipStream_t stream) {
    return dequant_q8<kSep16>(A, out, nelem, data_offset, stream);
}

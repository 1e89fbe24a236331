// Q4_0 and IQ4_NL GEMV / small-batch GEMM and dequantization for gfx950.
//
// Both formats use 32-weight blocks with one fp16 scale and 16 bytes of
// nibbles, uploaded in the separated layout
//     [scales: nblk * 2 bytes][pad to 16 bytes][data: nblk * 16 bytes]
// (tensor/quantized.go:158-198 RawBytesGPU / Q4GPUDataOffset).  Block i of
// the [rows, K] matrix is block (row * K/32 + kb).  They differ only in how
// a block decodes:
//   Q4_0   w[j] = (lo_j - 8) * d, w[j+16] = (hi_j - 8) * d   (byte j, GGML split order;
//          tensor/quantized.go:96-114)
//   IQ4_NL w[2i] = d * T[lo_i], w[2i+1] = d * T[hi_i]       (interleaved order, float table;
//          tensor/iq4_storage.go:28-46)
//
// Batch-1 GEMV design (HBM-bound; every weight byte is read once):
//  * four lanes share one 32-weight block: lane q of the quad loads dword q
//    of the block's 16 data bytes, so a wave covers 16 blocks per row and
//    its activation loads are 64 (Q4_0: two 16-byte halves) or 128
//    (IQ4_NL) contiguous bytes per block instead of a 128-byte stride per
//    lane, which is what keeps the load pipe streaming;
//  * each wave walks R rows with the same block columns, so the lane's 8
//    activations are loaded once and reused R times;
//  * the waves of a workgroup split K (split-K) and combine through LDS;
//  * Q4_0: a nibble masked into the low bits of an fp16 half is the
//    subnormal q * 2^-24 (exact), which v_fma_mix_f32 multiplies straight
//    into an fp32 accumulator: 5 integer ops + 8 FMAs per 8 weights with no
//    conversions; sum_j (q_j - 8) x_j = sum_j q_j x_j - 8 * sum_j x_j;
//  * IQ4_NL: a 256-entry LDS table maps a data byte to the fp32 codebook
//    values of its two nibbles, one ds_read_b64 per two weights;
//  * the block scale multiplies the block's partial sum once.
// Batched IQ4_NL calls with fp16 activations and N = 4, 8, 12 or 16 use the
// row-block MFMA GEMM further down (12 and 16 past 2048 rows the 16x16x32
// MFMA GEMM); other batched calls (N > 1, column-strided activations) use
// the block-per-lane kernel with one grid row per column.
#include "zt_bf16gemm.h"
#include "zt_rbmfma.h"

namespace zt {

enum class Fmt { Q4_0, IQ4NL };

// tensor/iq4_storage.go:28-33 IQ4NLTable.
__constant__ float kIQ4NLTable[16] = {
    -1.0f, -0.6961928f, -0.5250730f, -0.3947555f, -0.2831612f, -0.1790887f, -0.0805542f, 0.0f,
    0.0805542f, 0.1790887f, 0.2831612f, 0.3947555f, 0.5250730f, 0.6961928f, 1.0f, 1.3312578f};

// Codebook entry of data byte i (element pair: low nibble first) as two fp16
// pairs: .x = (T_hi[low], T_hi[high]), .y = (T_lo'[low], T_lo'[high]) with
// T_hi = fp16(T) and T_lo' = fp16(2^11 (T - T_hi)), so T = T_hi + 2^-11 T_lo'
// to within 2^-22 |T|.
__device__ __forceinline__ uint2 iq4_pair_entry(int i) {
    const float a = kIQ4NLTable[i & 15], b = kIQ4NLTable[i >> 4];
    const _Float16 ah = (_Float16)a, bh = (_Float16)b;
    const _Float16 al = (_Float16)((a - (float)ah) * 2048.0f), bl = (_Float16)((b - (float)bh) * 2048.0f);
    return make_uint2((uint32_t)__builtin_bit_cast(uint16_t, ah) | ((uint32_t)__builtin_bit_cast(uint16_t, bh) << 16),
                      (uint32_t)__builtin_bit_cast(uint16_t, al) | ((uint32_t)__builtin_bit_cast(uint16_t, bl) << 16));
}

// Table entry for a data byte i of the tiled MFMA kernel: (T_hi of the low
// nibble, T_hi of the high nibble, T_lo of the low, T_lo of the high) as
// fp16, with T_lo = fp16(T - T_hi) unscaled (subnormal for the smallest
// entries).  T_hi + T_lo is within 2^-22.3 |T| of every codebook value
// (exact for 0, +-1, +-0.6961928 and 1.3312578).
__device__ __forceinline__ uint2 iq4_quad_entry(int i) {
    const float a = kIQ4NLTable[i & 15], b = kIQ4NLTable[i >> 4];
    const _Float16 ah = (_Float16)a, bh = (_Float16)b;
    const _Float16 al = (_Float16)(a - (float)ah), bl = (_Float16)(b - (float)bh);
    return make_uint2((uint32_t)__builtin_bit_cast(uint16_t, ah) | ((uint32_t)__builtin_bit_cast(uint16_t, bh) << 16),
                      (uint32_t)__builtin_bit_cast(uint16_t, al) | ((uint32_t)__builtin_bit_cast(uint16_t, bl) << 16));
}

// The IQ4_NL codebook table of the fp32-activation row-block GEMM (rbf_kernel).
struct Iq4QuadTbl {
    __device__ static uint2 entry(int i) { return iq4_quad_entry(i); }
};

// Dot product of one data dword (8 codes, elements in order) with the fp16
// activation dwords xx[0..3]: hi and lo parts summed separately by
// v_dot2_f32_f16 and joined as hi + 2^-11 lo.
__device__ __forceinline__ float iq4_dot16(const uint2* tbl, uint32_t w, const uint32_t (&xx)[4]) {
    float v = 0.0f, vl = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const uint2 e = tbl[(w >> (8 * j)) & 0xffu];
        v = __builtin_amdgcn_fdot2(as_half2(e.x), as_half2(xx[j]), v, false);
        vl = __builtin_amdgcn_fdot2(as_half2(e.y), as_half2(xx[j]), vl, false);
    }
    return __builtin_fmaf(vl, 0x1p-11f, v);
}

template <class XT>
__device__ __forceinline__ float to_f32(XT v);
template <>
__device__ __forceinline__ float to_f32<float>(float v) { return v; }
template <>
__device__ __forceinline__ float to_f32<uint16_t>(uint16_t v) { return h2f(v); }

// Loads the 32 activations of block column b into registers.
template <class XT, bool CONTIG>
__device__ __forceinline__ void load_x32(const XT* __restrict__ x, long x_stride, int b, float (&xv)[32]) {
    if constexpr (CONTIG && sizeof(XT) == 4) {
        const float4* p = reinterpret_cast<const float4*>(x + (long)b * 32);
#pragma unroll
        for (int i = 0; i < 8; i++) {
            float4 t = p[i];
            xv[4 * i] = t.x; xv[4 * i + 1] = t.y; xv[4 * i + 2] = t.z; xv[4 * i + 3] = t.w;
        }
    } else if constexpr (CONTIG && sizeof(XT) == 2) {
        const uint4* p = reinterpret_cast<const uint4*>(x + (long)b * 32);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            uint4 t = p[i];
            uint32_t w[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
            for (int j = 0; j < 4; j++) {
                xv[8 * i + 2 * j] = h2f((uint16_t)(w[j] & 0xffff));
                xv[8 * i + 2 * j + 1] = h2f((uint16_t)(w[j] >> 16));
            }
        }
    } else {
#pragma unroll
        for (int i = 0; i < 32; i++) xv[i] = to_f32<XT>(x[((long)b * 32 + i) * x_stride]);
    }
}

// sum_j w_j x_j over one block, without the block scale.
template <Fmt F>
__device__ __forceinline__ float block_dot(const uint4 w, const float (&xv)[32], float xsum, const float2* tbl) {
    const uint32_t d[4] = {w.x, w.y, w.z, w.w};
    if constexpr (F == Fmt::Q4_0) {
        float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t lo = d[i] & 0x0f0f0f0fu;         // elements 4i .. 4i+3
            const uint32_t hi = (d[i] >> 4) & 0x0f0f0f0fu;  // elements 16+4i .. 16+4i+3
#pragma unroll
            for (int j = 0; j < 4; j++) {
                s0 = fmaf((float)((lo >> (8 * j)) & 0xffu), xv[4 * i + j], s0);
                s1 = fmaf((float)((hi >> (8 * j)) & 0xffu), xv[16 + 4 * i + j], s1);
            }
        }
        return (s0 + s1) - 8.0f * xsum;
    } else {
        float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; i++) {
#pragma unroll
            for (int j = 0; j < 4; j++) {  // byte j of dword i holds elements 8i+2j (low), 8i+2j+1 (high)
                const float2 t = tbl[(d[i] >> (8 * j)) & 0xffu];
                s0 = fmaf(t.x, xv[8 * i + 2 * j], s0);
                s1 = fmaf(t.y, xv[8 * i + 2 * j + 1], s1);
            }
        }
        return s0 + s1;
    }
}

// The 8 activations lane q of a quad needs for block b: Q4_0 elements
// 4q..4q+3 and 16+4q..16+4q+3 (GGML split order), IQ4_NL elements 8q..8q+7.
template <Fmt F, class XT>
__device__ __forceinline__ void load_x8(const XT* __restrict__ x, int b, int q, float (&xv)[8]) {
    if constexpr (sizeof(XT) == 4) {
        const float* p = reinterpret_cast<const float*>(x) + (long)b * 32;
        const float4 a = *reinterpret_cast<const float4*>(p + (F == Fmt::Q4_0 ? 4 * q : 8 * q));
        const float4 c = *reinterpret_cast<const float4*>(p + (F == Fmt::Q4_0 ? 16 + 4 * q : 8 * q + 4));
        xv[0] = a.x; xv[1] = a.y; xv[2] = a.z; xv[3] = a.w;
        xv[4] = c.x; xv[5] = c.y; xv[6] = c.z; xv[7] = c.w;
    } else {
        const uint16_t* p = reinterpret_cast<const uint16_t*>(x) + (long)b * 32;
        const uint2 a = *reinterpret_cast<const uint2*>(p + (F == Fmt::Q4_0 ? 4 * q : 8 * q));
        const uint2 c = *reinterpret_cast<const uint2*>(p + (F == Fmt::Q4_0 ? 16 + 4 * q : 8 * q + 4));
        xv[0] = h2f(a.x & 0xffff); xv[1] = h2f(a.x >> 16); xv[2] = h2f(a.y & 0xffff); xv[3] = h2f(a.y >> 16);
        xv[4] = h2f(c.x & 0xffff); xv[5] = h2f(c.x >> 16); xv[6] = h2f(c.y & 0xffff); xv[7] = h2f(c.y >> 16);
    }
}

// sum_j w_j x_j over the 8 weights of one data dword (without the block
// scale).  Q4_0: byte j of the dword holds element 4q+j (low nibble,
// activation xv[j]) and 16+4q+j (high nibble, xv[4+j]).  IQ4_NL: nibble m
// is element 8q+m (activation xv[m]).
template <Fmt F>
__device__ __forceinline__ float dword_dot(uint32_t d, const float (&xv)[8], float xsum, const float2* tbl) {
    if constexpr (F == Fmt::Q4_0) {
        const uint32_t d8 = d >> 8;
        const half2v m0 = as_half2(d & 0x000F000Fu);   // bytes 0,2 low nibbles  (q * 2^-24)
        const half2v m1 = as_half2(d & 0x00F000F0u);   // bytes 0,2 high nibbles (q * 2^-20)
        const half2v m2 = as_half2(d8 & 0x000F000Fu);  // bytes 1,3 low nibbles
        const half2v m3 = as_half2(d8 & 0x00F000F0u);  // bytes 1,3 high nibbles
        float sa = (float)m0.x * xv[0];
        float sb = (float)m1.x * xv[4];
        sa = __builtin_fmaf((float)m2.x, xv[1], sa);
        sb = __builtin_fmaf((float)m3.x, xv[5], sb);
        sa = __builtin_fmaf((float)m0.y, xv[2], sa);
        sb = __builtin_fmaf((float)m1.y, xv[6], sb);
        sa = __builtin_fmaf((float)m2.y, xv[3], sa);
        sb = __builtin_fmaf((float)m3.y, xv[7], sb);
        return __builtin_fmaf(sa, 16777216.0f, __builtin_fmaf(sb, 1048576.0f, -8.0f * xsum));
    } else {
        float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; j++) {  // byte j: elements 8q+2j (low nibble), 8q+2j+1 (high nibble)
            const float2 t = tbl[(d >> (8 * j)) & 0xffu];
            s0 = fmaf(t.x, xv[2 * j], s0);
            s1 = fmaf(t.y, xv[2 * j + 1], s1);
        }
        return s0 + s1;
    }
}

template <Fmt F, int R, class XT>
__global__ void __launch_bounds__(512) gemv_quad_kernel(const uint16_t* __restrict__ scales,
                                                        const uint32_t* __restrict__ data,
                                                        const XT* __restrict__ x, float* __restrict__ y,
                                                        int rows, int kb) {
    __shared__ float red[8 * R];
    __shared__ float2 tbl[256];  // IQ4_NL: byte value -> (T[low nibble], T[high nibble])
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nwaves = blockDim.x >> 6;
    const int q = lane & 3;
    if constexpr (F == Fmt::IQ4NL) {
        for (int i = threadIdx.x; i < 256; i += blockDim.x) tbl[i] = make_float2(kIQ4NLTable[i & 0xf], kIQ4NLTable[i >> 4]);
        __syncthreads();
    }
    const int row0 = blockIdx.x * R;
    long rbase[R];
#pragma unroll
    for (int r = 0; r < R; r++) rbase[r] = (long)min(row0 + r, rows - 1) * kb;
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.0f;

    for (int b = wave * 16 + (lane >> 2); b < kb; b += nwaves * 16) {
        uint32_t w[R];
        uint16_t s[R];
#pragma unroll
        for (int r = 0; r < R; r++) {
            w[r] = __builtin_nontemporal_load(&data[(rbase[r] + b) * 4 + q]);
            s[r] = scales[rbase[r] + b];
        }
        float xv[8];
        load_x8<F, XT>(x, b, q, xv);
        float xsum = 0.0f;
        if constexpr (F == Fmt::Q4_0) xsum = ((xv[0] + xv[1]) + (xv[2] + xv[3])) + ((xv[4] + xv[5]) + (xv[6] + xv[7]));
#pragma unroll
        for (int r = 0; r < R; r++) acc[r] = fmaf(h2f(s[r]), dword_dot<F>(w[r], xv, xsum, tbl), acc[r]);
    }
    block_reduce_store<R>(acc, red, y, 1, row0, rows);
}


// Q4_0 batch-1 GEMV where every wave does a fixed number S of 16-block
// steps per row (the quad mapping of gemv_quad_kernel), with every load of
// all S steps issued before any arithmetic.  Leaner per wave, which is what
// matters when waves are this short:
//  * buffer loads: the row offsets are wave-uniform and go in the scalar
//    offset, so no per-lane 64-bit address arithmetic; lanes past the last
//    block get an out-of-range offset and read zeros;
//  * the activations are pre-scaled once by 2^24 / 2^20, so each row is one
//    v_fma_mix chain started at -8*sum(x), and the fp16 block scale enters
//    v_fma_mix directly.
template <int S, int R, class XT = float>
__device__ __forceinline__ void q4_steps_body(const uint16_t* __restrict__ scales, const uint32_t* __restrict__ data,
                                              const XT* __restrict__ x, float* __restrict__ y, int rows, int kb,
                                              int row0, float* red) {
    constexpr bool H = sizeof(XT) == 2;  // fp16 activations: two 8-byte loads, widened exactly
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int q = lane & 3;
    const __amdgpu_buffer_rsrc_t rd = __builtin_amdgcn_make_buffer_rsrc((void*)data, (short)0, 0x7fffffff, 0x00020000);
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void*)scales, (short)0, 0x7fffffff, 0x00020000);
    const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc((void*)x, (short)0, kb * (H ? 64 : 128), 0x00020000);
    uint32_t w[S][R], s[S][R];
    u32x4 xa[S], xb[S];
#pragma unroll
    for (int t = 0; t < S; t++) {
        const int b = (wave * S + t) * 16 + (lane >> 2);
        const bool ok = b < kb;
        const uint32_t voff = ok ? (uint32_t)(b * 16 + q * 4) : 0x80000000u;
#pragma unroll
        for (int r = 0; r < R; r++) {
            const uint32_t row = (uint32_t)min(row0 + r, rows - 1);
            w[t][r] = __builtin_amdgcn_raw_buffer_load_b32(rd, voff, row * (uint32_t)kb * 16u, 2);  // nontemporal
        }
    }
#pragma unroll
    for (int t = 0; t < S; t++) {
        const int b = (wave * S + t) * 16 + (lane >> 2);
        const uint32_t soff = b < kb ? (uint32_t)(b * 2) : 0x80000000u;
#pragma unroll
        for (int r = 0; r < R; r++) {
            const uint32_t row = (uint32_t)min(row0 + r, rows - 1);
            s[t][r] = __builtin_amdgcn_raw_buffer_load_b16(rs, soff, row * (uint32_t)kb * 2u, 0);
        }
        if constexpr (H) {
            typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
            const uint32_t xo = b < kb ? (uint32_t)(b * 64 + q * 8) : 0x80000000u;
            const u32x2 a = __builtin_amdgcn_raw_buffer_load_b64(rx, xo, 0, 0);       // values 4q .. 4q+3
            const u32x2 c = __builtin_amdgcn_raw_buffer_load_b64(rx, xo + 32, 0, 0);  // values 16+4q ..
            xa[t] = (u32x4){a.x, a.y, 0u, 0u};
            xb[t] = (u32x4){c.x, c.y, 0u, 0u};
        } else {
            const uint32_t xo = b < kb ? (uint32_t)(b * 128 + q * 16) : 0x80000000u;
            xa[t] = __builtin_amdgcn_raw_buffer_load_b128(rx, xo, 0, 0);       // values 4q .. 4q+3
            xb[t] = __builtin_amdgcn_raw_buffer_load_b128(rx, xo + 64, 0, 0);  // values 16+4q ..
        }
    }
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.0f;
#pragma unroll
    for (int t = 0; t < S; t++) {
        float l0, l1, l2, l3, h0, h1, h2, h3;
        if constexpr (H) {
            l0 = h2f((uint16_t)xa[t].x); l1 = h2f((uint16_t)(xa[t].x >> 16));
            l2 = h2f((uint16_t)xa[t].y); l3 = h2f((uint16_t)(xa[t].y >> 16));
            h0 = h2f((uint16_t)xb[t].x); h1 = h2f((uint16_t)(xb[t].x >> 16));
            h2 = h2f((uint16_t)xb[t].y); h3 = h2f((uint16_t)(xb[t].y >> 16));
        } else {
            l0 = __uint_as_float(xa[t].x); l1 = __uint_as_float(xa[t].y); l2 = __uint_as_float(xa[t].z);
            l3 = __uint_as_float(xa[t].w);
            h0 = __uint_as_float(xb[t].x); h1 = __uint_as_float(xb[t].y); h2 = __uint_as_float(xb[t].z);
            h3 = __uint_as_float(xb[t].w);
        }
        const float c0 = -8.0f * (((l0 + l1) + (l2 + l3)) + ((h0 + h1) + (h2 + h3)));
        const float pl0 = l0 * 16777216.0f, pl1 = l1 * 16777216.0f, pl2 = l2 * 16777216.0f, pl3 = l3 * 16777216.0f;
        const float ph0 = h0 * 1048576.0f, ph1 = h1 * 1048576.0f, ph2 = h2 * 1048576.0f, ph3 = h3 * 1048576.0f;
#pragma unroll
        for (int r = 0; r < R; r++) {
            const uint32_t d = w[t][r], d8 = d >> 8;
            const half2v m0 = as_half2(d & 0x000F000Fu), m1 = as_half2(d & 0x00F000F0u);
            const half2v m2 = as_half2(d8 & 0x000F000Fu), m3 = as_half2(d8 & 0x00F000F0u);
            float v = __builtin_fmaf((float)m0.x, pl0, c0);
            v = __builtin_fmaf((float)m1.x, ph0, v);
            v = __builtin_fmaf((float)m2.x, pl1, v);
            v = __builtin_fmaf((float)m3.x, ph1, v);
            v = __builtin_fmaf((float)m0.y, pl2, v);
            v = __builtin_fmaf((float)m1.y, ph2, v);
            v = __builtin_fmaf((float)m2.y, pl3, v);
            v = __builtin_fmaf((float)m3.y, ph3, v);
            acc[r] = __builtin_fmaf((float)as_half2(s[t][r]).x, v, acc[r]);
        }
    }
    block_reduce_store<R>(acc, red, y, 1, row0, rows);
}

template <int S, int R, class XT = float>
__global__ void __launch_bounds__(1024) gemv_q4_steps_kernel(const uint16_t* __restrict__ scales,
                                                             const uint32_t* __restrict__ data,
                                                             const XT* __restrict__ x, float* __restrict__ y,
                                                             int rows, int kb) {
    __shared__ float red[16 * R];
    q4_steps_body<S, R, XT>(scales, data, x, y, rows, kb, blockIdx.x * R, red);
}

// NC fp32 activation columns of a batch at once (C[M, N] = A B, B[K, N]
// row-major), on the fixed-step form above: every weight dword and scale is
// loaded once for all NC columns, and each lane keeps R x NC sums.  The lane
// reads, for each of its 8 K positions (4q .. 4q+3 and 16+4q .. 16+4q+3 of
// its block), the NC consecutive floats of columns n0 .. n0+NC-1 of that B
// row (row stride ldx floats): one 16-byte load per 4 columns, or one 8-byte
// load for NC = 2.  Products are formed exactly as at batch 1 (fp16
// subnormal nibbles against activations pre-scaled by 2^24 / 2^20, a chain
// started at -8 sum(x) per column), so each column's sums are those of the
// batch-1 kernel.  The R x NC values are summed across the wave by the
// halving exchanges, across the waves through LDS in wave order, and stored
// once: no atomics, the same bits every call.
template <int NC>
__device__ __forceinline__ void q4n_load_row(__amdgpu_buffer_rsrc_t rx, uint32_t off, float (&v)[NC]) {
    if constexpr (NC == 2) {
        const uint2 d = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(rx, off, 0, 0));
        v[0] = __uint_as_float(d.x);
        v[1] = __uint_as_float(d.y);
    } else {
#pragma unroll
        for (int c = 0; c < NC / 4; c++) {
            const u32x4 d = __builtin_amdgcn_raw_buffer_load_b128(rx, off + 16u * c, 0, 0);
            v[4 * c] = __uint_as_float(d.x);
            v[4 * c + 1] = __uint_as_float(d.y);
            v[4 * c + 2] = __uint_as_float(d.z);
            v[4 * c + 3] = __uint_as_float(d.w);
        }
    }
}

template <int S, int R, int NC>
__global__ void __launch_bounds__(1024) gemv_q4n_steps_kernel(const uint16_t* __restrict__ scales,
                                                              const uint32_t* __restrict__ data,
                                                              const float* __restrict__ x, float* __restrict__ y,
                                                              int rows, int kb, int ldx, int n0) {
    constexpr int V = R * NC;
    __shared__ float red[16 * V];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nwaves = blockDim.x >> 6;
    const int q = lane & 3;
    const int row0 = blockIdx.x * R;
    const __amdgpu_buffer_rsrc_t rd = __builtin_amdgcn_make_buffer_rsrc((void*)data, (short)0, 0x7fffffff, 0x00020000);
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void*)scales, (short)0, 0x7fffffff, 0x00020000);
    const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc((void*)x, (short)0, kb * 128 * ldx, 0x00020000);
    uint32_t w[S][R], s[S][R];
#pragma unroll
    for (int t = 0; t < S; t++) {
        const int b = (wave * S + t) * 16 + (lane >> 2);
        const bool ok = b < kb;
        const uint32_t voff = ok ? (uint32_t)(b * 16 + q * 4) : 0x80000000u;
        const uint32_t soff = ok ? (uint32_t)(b * 2) : 0x80000000u;
#pragma unroll
        for (int r = 0; r < R; r++) {
            const uint32_t row = (uint32_t)min(row0 + r, rows - 1);
            w[t][r] = __builtin_amdgcn_raw_buffer_load_b32(rd, voff, row * (uint32_t)kb * 16u, 2);  // nontemporal
        }
#pragma unroll
        for (int r = 0; r < R; r++) {
            const uint32_t row = (uint32_t)min(row0 + r, rows - 1);
            s[t][r] = __builtin_amdgcn_raw_buffer_load_b16(rs, soff, row * (uint32_t)kb * 2u, 0);
        }
    }
    float acc[V];
#pragma unroll
    for (int i = 0; i < V; i++) acc[i] = 0.0f;
#pragma unroll
    for (int t = 0; t < S; t++) {
        const int b = (wave * S + t) * 16 + (lane >> 2);
        const bool ok = b < kb;
        // K rows 32b + 4q + i (low nibbles) and 32b + 16 + 4q + i (high nibbles)
        float xl[4][NC], xh[4][NC];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t kl = (uint32_t)(32 * b + 4 * q + i);
            q4n_load_row<NC>(rx, ok ? (kl * (uint32_t)ldx + (uint32_t)n0) * 4u : 0x80000000u, xl[i]);
            q4n_load_row<NC>(rx, ok ? ((kl + 16u) * (uint32_t)ldx + (uint32_t)n0) * 4u : 0x80000000u, xh[i]);
        }
        float c0[NC];
#pragma unroll
        for (int n = 0; n < NC; n++) {
            c0[n] = -8.0f * (((xl[0][n] + xl[1][n]) + (xl[2][n] + xl[3][n])) +
                             ((xh[0][n] + xh[1][n]) + (xh[2][n] + xh[3][n])));
#pragma unroll
            for (int i = 0; i < 4; i++) {
                xl[i][n] *= 16777216.0f;
                xh[i][n] *= 1048576.0f;
            }
        }
#pragma unroll
        for (int r = 0; r < R; r++) {
            const uint32_t d = w[t][r], d8 = d >> 8;
            const half2v m0 = as_half2(d & 0x000F000Fu), m1 = as_half2(d & 0x00F000F0u);
            const half2v m2 = as_half2(d8 & 0x000F000Fu), m3 = as_half2(d8 & 0x00F000F0u);
            const float sc = (float)as_half2(s[t][r]).x;
#pragma unroll
            for (int n = 0; n < NC; n++) {
                float v = __builtin_fmaf((float)m0.x, xl[0][n], c0[n]);
                v = __builtin_fmaf((float)m1.x, xh[0][n], v);
                v = __builtin_fmaf((float)m2.x, xl[1][n], v);
                v = __builtin_fmaf((float)m3.x, xh[1][n], v);
                v = __builtin_fmaf((float)m0.y, xl[2][n], v);
                v = __builtin_fmaf((float)m1.y, xh[2][n], v);
                v = __builtin_fmaf((float)m2.y, xl[3][n], v);
                v = __builtin_fmaf((float)m3.y, xh[3][n], v);
                acc[r * NC + n] = __builtin_fmaf(sc, v, acc[r * NC + n]);
            }
        }
    }
    wave_reduce_rows<V>(acc);
    if (is_row_writer<V>(lane)) red[wave * V + row_of_lane<V>(lane)] = acc[0];
    __syncthreads();
    if ((int)threadIdx.x < V) {
        float sum = 0.0f;
        for (int wv = 0; wv < nwaves; wv++) sum += red[wv * V + threadIdx.x];
        const int r = row0 + (int)threadIdx.x / NC;
        if (r < rows) y[(long)r * ldx + n0 + (int)threadIdx.x % NC] = sum;
    }
}

// Several Q4_0 matrices that read the same activation vector (q/k/v, or
// gate/up, of a decode layer) in one launch.  Workgroups [wg0[i], wg0[i+1])
// run matrix i with the fixed-step body above; the matrices keep their own
// separated uploads, so nothing is merged or re-laid out.  The descriptors
// travel in the kernel arguments.
// Up to three matrices in the standard RawBytesGPU layout (data offset
// Q4GPUDataOffset(rows * K/32)): everything a workgroup needs before its
// first weight load - the activations, K, the matrix bases and row counts
// - is in the first 13 argument dwords, which arrive preloaded in SGPRs; the
// matrix index and data offset are computed from them.  The output
// pointers come later, by ordinary argument loads that the weight loads
// hide.  (The general kernel below reads a 32-byte descriptor first: about
// 0.5 us more a launch.)
template <int S, int R>
__global__ void __launch_bounds__(1024) gemv_q4_group3_kernel(const float* __restrict__ x, int kb, int n,
                                                              const uint8_t* a0, const uint8_t* a1,
                                                              const uint8_t* a2, int rows0, int rows1, int rows2,
                                                              float* y0, float* y1, float* y2) {
    __shared__ float red[16 * R];
    const int b = blockIdx.x;
    const int w1 = (rows0 + R - 1) / R, w2 = w1 + (rows1 + R - 1) / R;
    const int m = (b >= w1 ? 1 : 0) + (n > 2 && b >= w2 ? 1 : 0);
    const uint8_t* a = m == 0 ? a0 : m == 1 ? a1 : a2;
    const int rows = m == 0 ? rows0 : m == 1 ? rows1 : rows2;
    float* y = m == 0 ? y0 : m == 1 ? y1 : y2;
    const long nblk = (long)rows * kb;
    const uint32_t* dt = reinterpret_cast<const uint32_t*>(a + ((nblk * 2 + 15) & ~15L));
    q4_steps_body<S, R>(reinterpret_cast<const uint16_t*>(a), dt, x, y, rows, kb,
                        (b - (m == 0 ? 0 : m == 1 ? w1 : w2)) * R, red);
}

// The kernel's x and kb arguments, then the workgroup starts and the count,
// arrive in preloaded SGPRs, so finding the matrix costs no memory access;
// its 32-byte descriptor is then one scalar load.
struct Q4GroupMat {
    const uint16_t* sc;
    const uint32_t* dt;
    float* y;
    int rows;
    int wg0;
};

struct Q4GroupArgs {
    int wg0[ZT_GROUP_MAX];  // first workgroup of matrix i (wg0[0] = 0); unused entries past n
    int n;
    int pad[3];
    Q4GroupMat mat[ZT_GROUP_MAX];
};

template <int S, int R>
__global__ void __launch_bounds__(1024) gemv_q4_group_kernel(const float* __restrict__ x, int kb,
                                                             const Q4GroupArgs g) {
    __shared__ float red[16 * R];
    const int b = blockIdx.x;
    int m = 0;
#pragma unroll
    for (int i = 1; i < ZT_GROUP_MAX; i++) m += (i < g.n && b >= g.wg0[i]) ? 1 : 0;
    const Q4GroupMat d = g.mat[m];
    q4_steps_body<S, R>(d.sc, d.dt, x, d.y, d.rows, kb, (b - d.wg0) * R, red);
}

// IQ4_NL batch-1 GEMV with fp16 activations.  The quad mapping of
// gemv_quad_kernel (lane q of a quad holds dword q of a block: elements
// 8q .. 8q+7, byte j = elements 8q+2j (low nibble) and 8q+2j+1 (high)),
// with a 2 KB LDS table from a data byte to two fp16 pairs (iq4_pair_entry):
// the codebook (tensor/iq4_storage.go:28-33) split as T = T_hi + 2^-11 T_lo',
// exact to 2^-22 |T|.  Each pair lines up with the activation dword
// (x[8q+2j], x[8q+2j+1]), so each byte is one ds_read_b64 and two
// v_dot2_f32_f16 into separate hi and lo sums (products exact in fp32, fp32
// sums), joined once per block before the scale.  The fp16-rounded table
// alone (one ds_read_b32 and one dot a byte, error up to 2^-11 per entry)
// measured no faster: 11.3 us against 10.1 us for the split at 18944 x 3584.
// Buffer loads take the wave-uniform row offsets as scalar offsets; lanes
// past the last block read zeros through out-of-range offsets.
template <int R>
__global__ void __launch_bounds__(1024) gemv_iq4nl_h16_kernel(const uint16_t* __restrict__ scales,
                                                              const uint32_t* __restrict__ data,
                                                              const uint16_t* __restrict__ x, float* __restrict__ y,
                                                              int rows, int kb) {
    __shared__ float red[16 * R];
    __shared__ uint2 tbl[256];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nwaves = blockDim.x >> 6;
    const int q = lane & 3;
    const int row0 = blockIdx.x * R;
    const __amdgpu_buffer_rsrc_t rd = __builtin_amdgcn_make_buffer_rsrc((void*)data, (short)0, 0x7fffffff, 0x00020000);
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void*)scales, (short)0, 0x7fffffff, 0x00020000);
    const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc((void*)x, (short)0, kb * 64, 0x00020000);
    for (int i = threadIdx.x; i < 256; i += blockDim.x) tbl[i] = iq4_pair_entry(i);
    __syncthreads();
    uint32_t rofs[R];
#pragma unroll
    for (int r = 0; r < R; r++) rofs[r] = (uint32_t)min(row0 + r, rows - 1) * (uint32_t)kb;
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.0f;
    for (int b0 = wave * 16; b0 < kb; b0 += nwaves * 16) {
        const int b = b0 + (lane >> 2);
        const bool ok = b < kb;
        const uint32_t voff = ok ? (uint32_t)(b * 16 + q * 4) : 0x80000000u;
        const uint32_t soff = ok ? (uint32_t)(b * 2) : 0x80000000u;
        uint32_t w[R], s[R];
#pragma unroll
        for (int r = 0; r < R; r++) w[r] = __builtin_amdgcn_raw_buffer_load_b32(rd, voff, rofs[r] * 16u, 2);  // nontemporal
#pragma unroll
        for (int r = 0; r < R; r++) s[r] = __builtin_amdgcn_raw_buffer_load_b16(rs, soff, rofs[r] * 2u, 0);
        const u32x4 xv = __builtin_amdgcn_raw_buffer_load_b128(rx, ok ? (uint32_t)(b * 64 + q * 16) : 0x80000000u, 0, 0);
        const uint32_t xx[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
        for (int r = 0; r < R; r++) acc[r] = __builtin_fmaf(h2f(s[r]), iq4_dot16(tbl, w[r], xx), acc[r]);
    }
    block_reduce_store<R>(acc, red, y, 1, row0, rows);
}

// The same computation with a fixed S steps of 16 blocks per wave for
// K <= 4096 (the form of gemv_q4_steps_kernel): every weight, scale and
// activation load of all steps is issued before the table is built and any
// product is formed, so a wave waits for one memory round trip where the
// loop above waits for one per iteration.  Two steps of 4 rows on 4 waves
// measured 15-17% faster than the loop at 14336-18944 x 3584.
template <int S, int R>
__global__ void __launch_bounds__(1024) gemv_iq4nl_h16_steps_kernel(const uint16_t* __restrict__ scales,
                                                                    const uint32_t* __restrict__ data,
                                                                    const uint16_t* __restrict__ x,
                                                                    float* __restrict__ y, int rows, int kb) {
    __shared__ float red[16 * R];
    __shared__ uint2 tbl[256];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int q = lane & 3;
    const int row0 = blockIdx.x * R;
    const __amdgpu_buffer_rsrc_t rd = __builtin_amdgcn_make_buffer_rsrc((void*)data, (short)0, 0x7fffffff, 0x00020000);
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void*)scales, (short)0, 0x7fffffff, 0x00020000);
    const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc((void*)x, (short)0, kb * 64, 0x00020000);
    uint32_t w[S][R], s[S][R];
    u32x4 xv[S];
#pragma unroll
    for (int t = 0; t < S; t++) {
        const int b = (wave * S + t) * 16 + (lane >> 2);
        const uint32_t voff = b < kb ? (uint32_t)(b * 16 + q * 4) : 0x80000000u;
#pragma unroll
        for (int r = 0; r < R; r++) {
            const uint32_t row = (uint32_t)min(row0 + r, rows - 1);
            w[t][r] = __builtin_amdgcn_raw_buffer_load_b32(rd, voff, row * (uint32_t)kb * 16u, 2);  // nontemporal
        }
    }
#pragma unroll
    for (int t = 0; t < S; t++) {
        const int b = (wave * S + t) * 16 + (lane >> 2);
        const uint32_t soff = b < kb ? (uint32_t)(b * 2) : 0x80000000u;
#pragma unroll
        for (int r = 0; r < R; r++) {
            const uint32_t row = (uint32_t)min(row0 + r, rows - 1);
            s[t][r] = __builtin_amdgcn_raw_buffer_load_b16(rs, soff, row * (uint32_t)kb * 2u, 0);
        }
        xv[t] = __builtin_amdgcn_raw_buffer_load_b128(rx, b < kb ? (uint32_t)(b * 64 + q * 16) : 0x80000000u, 0, 0);
    }
    for (int i = threadIdx.x; i < 256; i += blockDim.x) tbl[i] = iq4_pair_entry(i);
    // the table is visible to the workgroup; the loads stay in flight
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.0f;
#pragma unroll
    for (int t = 0; t < S; t++) {
        const uint32_t xx[4] = {xv[t].x, xv[t].y, xv[t].z, xv[t].w};
#pragma unroll
        for (int r = 0; r < R; r++) acc[r] = __builtin_fmaf(h2f(s[t][r]), iq4_dot16(tbl, w[t][r], xx), acc[r]);
    }
    block_reduce_store<R>(acc, red, y, 1, row0, rows);
}

// fp32 activations in the same fixed-step form: the lane's 8 activations
// (elements 8q .. 8q+7 of its block) are two 16-byte loads a step, and the
// 2 KB table maps a data byte to the fp32 pair (T[low], T[high]) of the
// reference's codebook, so each product is the reference's fp32 product:
// two FMAs a byte.
template <int S, int R>
__global__ void __launch_bounds__(1024) gemv_iq4nl_f32_steps_kernel(const uint16_t* __restrict__ scales,
                                                                    const uint32_t* __restrict__ data,
                                                                    const float* __restrict__ x,
                                                                    float* __restrict__ y, int rows, int kb) {
    __shared__ float red[16 * R];
    __shared__ float2 tbl[256];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int q = lane & 3;
    const int row0 = blockIdx.x * R;
    const __amdgpu_buffer_rsrc_t rd = __builtin_amdgcn_make_buffer_rsrc((void*)data, (short)0, 0x7fffffff, 0x00020000);
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void*)scales, (short)0, 0x7fffffff, 0x00020000);
    const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc((void*)x, (short)0, kb * 128, 0x00020000);
    uint32_t w[S][R], s[S][R];
    u32x4 xa[S], xb[S];
#pragma unroll
    for (int t = 0; t < S; t++) {
        const int b = (wave * S + t) * 16 + (lane >> 2);
        const uint32_t voff = b < kb ? (uint32_t)(b * 16 + q * 4) : 0x80000000u;
#pragma unroll
        for (int r = 0; r < R; r++) {
            const uint32_t row = (uint32_t)min(row0 + r, rows - 1);
            w[t][r] = __builtin_amdgcn_raw_buffer_load_b32(rd, voff, row * (uint32_t)kb * 16u, 2);  // nontemporal
        }
    }
#pragma unroll
    for (int t = 0; t < S; t++) {
        const int b = (wave * S + t) * 16 + (lane >> 2);
        const uint32_t soff = b < kb ? (uint32_t)(b * 2) : 0x80000000u;
#pragma unroll
        for (int r = 0; r < R; r++) {
            const uint32_t row = (uint32_t)min(row0 + r, rows - 1);
            s[t][r] = __builtin_amdgcn_raw_buffer_load_b16(rs, soff, row * (uint32_t)kb * 2u, 0);
        }
        const uint32_t xo = b < kb ? (uint32_t)(b * 128 + q * 32) : 0x80000000u;
        xa[t] = __builtin_amdgcn_raw_buffer_load_b128(rx, xo, 0, 0);
        xb[t] = __builtin_amdgcn_raw_buffer_load_b128(rx, xo + 16, 0, 0);
    }
    for (int i = threadIdx.x; i < 256; i += blockDim.x) tbl[i] = make_float2(kIQ4NLTable[i & 15], kIQ4NLTable[i >> 4]);
    // the table is visible to the workgroup; the loads stay in flight
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.0f;
#pragma unroll
    for (int t = 0; t < S; t++) {
        const float xv[8] = {__uint_as_float(xa[t].x), __uint_as_float(xa[t].y), __uint_as_float(xa[t].z),
                             __uint_as_float(xa[t].w), __uint_as_float(xb[t].x), __uint_as_float(xb[t].y),
                             __uint_as_float(xb[t].z), __uint_as_float(xb[t].w)};
#pragma unroll
        for (int r = 0; r < R; r++) {
            float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
            for (int j = 0; j < 4; j++) {  // byte j: elements 8q+2j (low nibble), 8q+2j+1 (high nibble)
                const float2 e = tbl[(w[t][r] >> (8 * j)) & 0xffu];
                s0 = __builtin_fmaf(e.x, xv[2 * j], s0);
                s1 = __builtin_fmaf(e.y, xv[2 * j + 1], s1);
            }
            acc[r] = __builtin_fmaf(h2f((uint16_t)s[t][r]), s0 + s1, acc[r]);
        }
    }
    block_reduce_store<R>(acc, red, y, 1, row0, rows);
}

// fp32 activations past K = 4096: the loop form of gemv_iq4nl_h16_kernel
// (buffer loads with wave-uniform row offsets as scalar offsets, a grid of
// about 8192 waves) with the fp32 pair table.
template <int R>
__global__ void __launch_bounds__(1024) gemv_iq4nl_f32_kernel(const uint16_t* __restrict__ scales,
                                                              const uint32_t* __restrict__ data,
                                                              const float* __restrict__ x, float* __restrict__ y,
                                                              int rows, int kb) {
    __shared__ float red[16 * R];
    __shared__ float2 tbl[256];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nwaves = blockDim.x >> 6;
    const int q = lane & 3;
    const int row0 = blockIdx.x * R;
    const __amdgpu_buffer_rsrc_t rd = __builtin_amdgcn_make_buffer_rsrc((void*)data, (short)0, 0x7fffffff, 0x00020000);
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void*)scales, (short)0, 0x7fffffff, 0x00020000);
    const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc((void*)x, (short)0, kb * 128, 0x00020000);
    for (int i = threadIdx.x; i < 256; i += blockDim.x) tbl[i] = make_float2(kIQ4NLTable[i & 15], kIQ4NLTable[i >> 4]);
    __syncthreads();
    uint32_t rofs[R];
#pragma unroll
    for (int r = 0; r < R; r++) rofs[r] = (uint32_t)min(row0 + r, rows - 1) * (uint32_t)kb;
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.0f;
    for (int b0 = wave * 16; b0 < kb; b0 += nwaves * 16) {
        const int b = b0 + (lane >> 2);
        const bool ok = b < kb;
        const uint32_t voff = ok ? (uint32_t)(b * 16 + q * 4) : 0x80000000u;
        const uint32_t soff = ok ? (uint32_t)(b * 2) : 0x80000000u;
        uint32_t w[R], sv[R];
#pragma unroll
        for (int r = 0; r < R; r++) w[r] = __builtin_amdgcn_raw_buffer_load_b32(rd, voff, rofs[r] * 16u, 2);  // nontemporal
#pragma unroll
        for (int r = 0; r < R; r++) sv[r] = __builtin_amdgcn_raw_buffer_load_b16(rs, soff, rofs[r] * 2u, 0);
        const uint32_t xo = ok ? (uint32_t)(b * 128 + q * 32) : 0x80000000u;
        const u32x4 xa = __builtin_amdgcn_raw_buffer_load_b128(rx, xo, 0, 0);
        const u32x4 xb = __builtin_amdgcn_raw_buffer_load_b128(rx, xo + 16, 0, 0);
        const float xv[8] = {__uint_as_float(xa.x), __uint_as_float(xa.y), __uint_as_float(xa.z), __uint_as_float(xa.w),
                             __uint_as_float(xb.x), __uint_as_float(xb.y), __uint_as_float(xb.z), __uint_as_float(xb.w)};
#pragma unroll
        for (int r = 0; r < R; r++) {
            float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const float2 e = tbl[(w[r] >> (8 * j)) & 0xffu];
                s0 = __builtin_fmaf(e.x, xv[2 * j], s0);
                s1 = __builtin_fmaf(e.y, xv[2 * j + 1], s1);
            }
            acc[r] = __builtin_fmaf(h2f((uint16_t)sv[r]), s0 + s1, acc[r]);
        }
    }
    block_reduce_store<R>(acc, red, y, 1, row0, rows);
}

template <int S>
static void launch_iq4nl_f32_steps(int R, dim3 grid, dim3 block, hipStream_t st, const uint16_t* sc,
                                   const uint32_t* dt, const float* x, float* y, int rows, int kb) {
    switch (R) {
        case 8: gemv_iq4nl_f32_steps_kernel<S, 8><<<grid, block, 0, st>>>(sc, dt, x, y, rows, kb); break;
        case 4: gemv_iq4nl_f32_steps_kernel<S, 4><<<grid, block, 0, st>>>(sc, dt, x, y, rows, kb); break;
        case 2: gemv_iq4nl_f32_steps_kernel<S, 2><<<grid, block, 0, st>>>(sc, dt, x, y, rows, kb); break;
        default: gemv_iq4nl_f32_steps_kernel<S, 1><<<grid, block, 0, st>>>(sc, dt, x, y, rows, kb); break;
    }
}

template <int S>
static void launch_iq4nl_h16_steps(int R, dim3 grid, dim3 block, hipStream_t st, const uint16_t* sc,
                                   const uint32_t* dt, const uint16_t* x, float* y, int rows, int kb) {
    switch (R) {
        case 8: gemv_iq4nl_h16_steps_kernel<S, 8><<<grid, block, 0, st>>>(sc, dt, x, y, rows, kb); break;
        case 4: gemv_iq4nl_h16_steps_kernel<S, 4><<<grid, block, 0, st>>>(sc, dt, x, y, rows, kb); break;
        case 2: gemv_iq4nl_h16_steps_kernel<S, 2><<<grid, block, 0, st>>>(sc, dt, x, y, rows, kb); break;
        default: gemv_iq4nl_h16_steps_kernel<S, 1><<<grid, block, 0, st>>>(sc, dt, x, y, rows, kb); break;
    }
}

static void launch_iq4nl_h16(int R, dim3 grid, dim3 block, hipStream_t st, const uint16_t* sc, const uint32_t* dt,
                             const uint16_t* x, float* y, int rows, int kb) {
    switch (R) {
        case 8: gemv_iq4nl_h16_kernel<8><<<grid, block, 0, st>>>(sc, dt, x, y, rows, kb); break;
        case 4: gemv_iq4nl_h16_kernel<4><<<grid, block, 0, st>>>(sc, dt, x, y, rows, kb); break;
        case 2: gemv_iq4nl_h16_kernel<2><<<grid, block, 0, st>>>(sc, dt, x, y, rows, kb); break;
        default: gemv_iq4nl_h16_kernel<1><<<grid, block, 0, st>>>(sc, dt, x, y, rows, kb); break;
    }
}

template <int S, class XT>
static void launch_q4_steps(int R, dim3 grid, dim3 block, hipStream_t st, const uint16_t* sc, const uint32_t* dt,
                            const XT* x, float* y, int rows, int kb) {
    switch (R) {
        case 8: gemv_q4_steps_kernel<S, 8, XT><<<grid, block, 0, st>>>(sc, dt, x, y, rows, kb); break;
        case 4: gemv_q4_steps_kernel<S, 4, XT><<<grid, block, 0, st>>>(sc, dt, x, y, rows, kb); break;
        case 2: gemv_q4_steps_kernel<S, 2, XT><<<grid, block, 0, st>>>(sc, dt, x, y, rows, kb); break;
        default: gemv_q4_steps_kernel<S, 1, XT><<<grid, block, 0, st>>>(sc, dt, x, y, rows, kb); break;
    }
}

template <Fmt F, class XT>
static void launch_quad(int R, dim3 grid, dim3 block, hipStream_t st, const uint16_t* sc, const uint32_t* dt,
                        const XT* x, float* y, int rows, int kb) {
    switch (R) {
        case 8: gemv_quad_kernel<F, 8, XT><<<grid, block, 0, st>>>(sc, dt, x, y, rows, kb); break;
        case 4: gemv_quad_kernel<F, 4, XT><<<grid, block, 0, st>>>(sc, dt, x, y, rows, kb); break;
        case 2: gemv_quad_kernel<F, 2, XT><<<grid, block, 0, st>>>(sc, dt, x, y, rows, kb); break;
        default: gemv_quad_kernel<F, 1, XT><<<grid, block, 0, st>>>(sc, dt, x, y, rows, kb); break;
    }
}

// ------------------------------------------------------------ IQ4_NL MFMA GEMM
//
// Batched IQ4_NL (fp16 activations, 4 <= N <= 16, N % 4 == 0, K % 128 == 0):
// the workgroup structure, X staging and transposing B reads of zt_mfma.h.
//  * For a 128-K unit, lane (i = lane%16, g = lane/16) loads the 16 data
//    bytes of block 4u+g of row i.  Two v_permlane32_swap and two
//    v_permlane16_swap transpose the four lanes' dwords so that register c
//    holds dword g of block 4u+c: MFMA step c then covers exactly one block
//    (lane group g supplies its elements 8g .. 8g+7), and the block's fp16
//    scale multiplies the step's result.
//  * The fp32 codebook value T[q] enters the MFMA as two exact fp16 parts,
//    T_hi = fp16(T) and T_lo = fp16(T - T_hi) (|T - T_hi - T_lo| <=
//    2^-22.3 |T|, T_lo subnormal for +-0.0805542), looked up together as
//    one dword from a 16-entry LDS table; two MFMAs per step accumulate
//    both parts.
__device__ __forceinline__ uint32_t pack_lo16(uint32_t a, uint32_t b) { return __builtin_amdgcn_perm(b, a, 0x05040100u); }
__device__ __forceinline__ uint32_t pack_hi16(uint32_t a, uint32_t b) { return __builtin_amdgcn_perm(b, a, 0x07060302u); }

__global__ void __launch_bounds__(512) iq4nl_mfma_kernel(const uint16_t* __restrict__ scales,
                                                         const uint4* __restrict__ data,
                                                         const uint16_t* __restrict__ x, float* __restrict__ y,
                                                         int rows, int K, int N) {
    constexpr int NT = kMfmaTiles;
    constexpr int BPC = kMfmaUC * 4;  // blocks per chunk
    extern __shared__ __attribute__((aligned(16))) char smem[];
    const int xbytes = mfma_xbytes(N);
    char* zero_area = smem + xbytes;
    uint32_t* tbl = reinterpret_cast<uint32_t*>(zero_area + 16);  // 16 x (T_hi | T_lo << 16)
    uint16_t* ss = reinterpret_cast<uint16_t*>(tbl + 16);         // [block in chunk][row]

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int li = lane & 15, lg = lane >> 4;
    const int row0 = blockIdx.x * kMfmaRows;
    const int nunits = K / 128, kb = K / 32;
    if (tid < 4) reinterpret_cast<uint32_t*>(zero_area)[tid] = 0u;
    if (tid < 16) {
        const float t = kIQ4NLTable[tid];
        const _Float16 hi = (_Float16)t;
        const _Float16 lo = (_Float16)(t - (float)hi);
        tbl[tid] = (uint32_t)__builtin_bit_cast(uint16_t, hi) | ((uint32_t)__builtin_bit_cast(uint16_t, lo) << 16);
    }

    float4v acc[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) acc[t] = (float4v){0.f, 0.f, 0.f, 0.f};
    long abase[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) abase[t] = (long)min(row0 + 16 * t + li, rows - 1) * kb;
    const MfmaBRole ro(li, N);

    const int ub = 0, ue = nunits;
    for (int c0 = ub; c0 < ue; c0 += kMfmaUC) {
        uint4 w[kMfmaUPW][NT];
#pragma unroll
        for (int u = 0; u < kMfmaUPW; u++) {
            const int unit = min(c0 + wave + kMfmaWaves * u, ue - 1);
#pragma unroll
            for (int t = 0; t < NT; t++) w[u][t] = ld_stream(&data[abase[t] + unit * 4 + lg]);
        }
        mfma_stage_x(smem, x, c0, ue * 128, N);
        for (int e = tid; e < BPC * kMfmaRows; e += blockDim.x) {
            const int bb = e / kMfmaRows, r = e % kMfmaRows;
            const int blk = c0 * 4 + bb;
            if (blk < kb) ss[e] = scales[(long)min(row0 + r, rows - 1) * kb + blk];
        }
        __syncthreads();
#pragma unroll
        for (int u = 0; u < kMfmaUPW; u++) {
            const int uu = wave + kMfmaWaves * u;
            if (c0 + uu < ue) {
                uint32_t r[NT][4];
#pragma unroll
                for (int t = 0; t < NT; t++) {
                    // 4x4 transpose across the lane groups: r[t][c] = dword g of block 4u+c.
                    auto p02 = __builtin_amdgcn_permlane32_swap(w[u][t].x, w[u][t].z, false, false);
                    auto p13 = __builtin_amdgcn_permlane32_swap(w[u][t].y, w[u][t].w, false, false);
                    auto q01 = __builtin_amdgcn_permlane16_swap(p02[0], p13[0], false, false);
                    auto q23 = __builtin_amdgcn_permlane16_swap(p02[1], p13[1], false, false);
                    r[t][0] = q01[0]; r[t][1] = q01[1]; r[t][2] = q23[0]; r[t][3] = q23[1];
                }
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    const half8v bv = mfma_b_operand(smem, ro, uu * 128 + 32 * c + 8 * lg, ro.jq, ro.jq + 4, N, xbytes);
#pragma unroll
                    for (int t = 0; t < NT; t++) {
                        uint32_t e[8];
#pragma unroll
                        for (int m = 0; m < 8; m++) e[m] = tbl[(r[t][c] >> (4 * m)) & 0xfu];
                        const uint32_t ah[4] = {pack_lo16(e[0], e[1]), pack_lo16(e[2], e[3]), pack_lo16(e[4], e[5]),
                                                pack_lo16(e[6], e[7])};
                        const uint32_t al[4] = {pack_hi16(e[0], e[1]), pack_hi16(e[2], e[3]), pack_hi16(e[4], e[5]),
                                                pack_hi16(e[6], e[7])};
                        float4v dd = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                            __builtin_bit_cast(half8v, (u32x4){ah[0], ah[1], ah[2], ah[3]}), bv,
                            (float4v){0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                        dd = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                            __builtin_bit_cast(half8v, (u32x4){al[0], al[1], al[2], al[3]}), bv, dd, 0, 0, 0);
                        const int rb0 = (uu * 4 + c) * kMfmaRows + 16 * t + 4 * lg;
                        const uint2 s4 = *reinterpret_cast<const uint2*>(ss + rb0);
                        acc[t][0] = fmaf(h2f(s4.x & 0xffff), dd[0], acc[t][0]);
                        acc[t][1] = fmaf(h2f(s4.x >> 16), dd[1], acc[t][1]);
                        acc[t][2] = fmaf(h2f(s4.y & 0xffff), dd[2], acc[t][2]);
                        acc[t][3] = fmaf(h2f(s4.y >> 16), dd[3], acc[t][3]);
                    }
                }
            }
        }
        __syncthreads();
    }
    mfma_reduce_store(acc, smem, y, row0, rows, N);
}

// ------------------------------------------------------------ IQ4_NL row-block GEMM
//
// Batches of N = 4, 8 (12, 16) with fp16 activations on the separated upload
// layout, in one launch: the row-block structure of zt_rbmfma.h
// (v_mfma_f32_4x4x4_16b_f16, lane = 32-element block of row j of a 4-row
// set, waves splitting K, activations staged per wave and read back
// transposed).  A block is one chunk, so it needs no regrouping.
//  * MFMA step u (0-15) covers data byte u of the lane's block, elements
//    2u and 2u+1: B = the byte's entry of a 2 KB LDS table,
//    (T_hi[lo], T_hi[hi], T_lo[lo], T_lo[hi]) (iq4_quad_entry), against
//    A = (x[2u], x[2u+1], x[2u], x[2u+1]), so the step's sum is
//    x0 (T_hi + T_lo)[lo] + x1 (T_hi + T_lo)[hi], the fp32 codebook to
//    within 2^-22 per entry, with every product exact;
//  * the block's sum then takes the block's fp16 scale: y += d D.
template <int NB, int R, int S>
__global__ void __launch_bounds__(NB > 2 && R > 1 ? 512 : 1024) iq4nl_rb_kernel(const uint16_t* __restrict__ scales,
                                                        const uint32_t* __restrict__ data,
                                                        const uint16_t* __restrict__ x, float* __restrict__ y,
                                                        int rows, int kb) {
    using Lay = RbLayout<NB>;
    constexpr int V = 4 * R * NB;
    extern __shared__ __attribute__((aligned(16))) char smem[];
    uint2* tbl = reinterpret_cast<uint2*>(smem);  // 256 entries, one per data byte
    char* regions = smem + 2048;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int blk = lane >> 2, j = lane & 3;
    char* xs = regions + wave * Lay::STEP;
    const int row0 = blockIdx.x * 4 * R;
    // rows past M read zeros: the buffers end at row M
    const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc((void*)data, (short)0, rows * kb * 16, 0x00020000);
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void*)scales, (short)0, rows * kb * 2, 0x00020000);
    const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc((void*)x, (short)0, kb * 64 * Lay::N, 0x00020000);
    const int step0 = wave * S;
    rb_stage_x<NB>(rx, xs, (uint32_t)step0 * Lay::STEP, lane);
    __builtin_amdgcn_sched_barrier(0);
    u32x4 w[S][R];
    uint32_t sc[S][R];
    const uint32_t brow = (uint32_t)(row0 + j) * (uint32_t)kb, bstep = 4u * (uint32_t)kb;
#pragma unroll
    for (int t = 0; t < S; t++) {
        const int c = (step0 + t) * 16 + blk;
        const bool ok = c < kb;
#pragma unroll
        for (int r = 0; r < R; r++) {
            const uint32_t b = brow + r * bstep + (uint32_t)c;
            w[t][r] = __builtin_amdgcn_raw_buffer_load_b128(rw, ok ? b * 16u : 0x80000000u, 0, 2);  // nontemporal
            sc[t][r] = __builtin_amdgcn_raw_buffer_load_b16(rs, ok ? b * 2u : 0x80000000u, 0, 0);
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    for (int i = threadIdx.x; i < 256; i += blockDim.x) tbl[i] = iq4_quad_entry(i);
    // the table is visible to the workgroup; the loads stay in flight
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    float acc[V];
#pragma unroll
    for (int i = 0; i < V; i++) acc[i] = 0.0f;
#pragma unroll
    for (int t = 0; t < S; t++) {
        if (t > 0) {
            // every read of the previous step's activations has returned before the
            // direct loads overwrite them
            __builtin_amdgcn_sched_barrier(0);
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            __builtin_amdgcn_sched_barrier(0);
            rb_stage_x<NB>(rx, xs, (uint32_t)(step0 + t) * Lay::STEP, lane);
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        } else {
            // the activations only: the 2 S R weight and scale loads after them may be outstanding
            asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * S * R) : "memory");
        }
        constexpr int RC = R < 4 / NB ? R : 4 / NB;
#pragma unroll
        for (int r0 = 0; r0 < R; r0 += RC) {
            float4v d[RC][NB];
#pragma unroll
            for (int r = 0; r < RC; r++)
#pragma unroll
                for (int js = 0; js < NB; js++) d[r][js] = (float4v){0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int u = 0; u < 16; u++) {
                half4v xa[NB];
#pragma unroll
                for (int js = 0; js < NB; js++) xa[js] = rb_tr_read(xs, rb_tr_offset_pair<NB>(lane, u, js));
#pragma unroll
                for (int r = 0; r < RC; r++) {
                    const u32x4& wv = w[t][r0 + r];
                    const uint32_t q = (u >> 2) == 0 ? wv.x : (u >> 2) == 1 ? wv.y : (u >> 2) == 2 ? wv.z : wv.w;
                    const int sh = 8 * (u & 3);
                    const uint32_t off = (sh == 0 ? q << 3 : q >> (sh - 3)) & 0x7F8u;  // byte * 8
                    const half4v bv = __builtin_bit_cast(half4v, *reinterpret_cast<const uint2*>(smem + off));
#pragma unroll
                    for (int js = 0; js < NB; js++)
                        d[r][js] = __builtin_amdgcn_mfma_f32_4x4x4f16(xa[js], bv, d[r][js], 0, 0, 0);
                }
            }
#pragma unroll
            for (int r = 0; r < RC; r++) {
                const float dv = h2f((uint16_t)sc[t][r0 + r]);
#pragma unroll
                for (int js = 0; js < NB; js++)
#pragma unroll
                    for (int v = 0; v < 4; v++) {
                        float& a = acc[((r0 + r) * NB + js) * 4 + v];
                        a = __builtin_fmaf(dv, d[r][js][v], a);
                    }
            }
        }
    }
    rb_finish<NB, R>(acc, regions, Lay::STEP, xs, y, row0, rows);
}

template <int NB, int R, int S>
static void launch_iq4nl_rb_t(dim3 g, int nw, hipStream_t st, const uint16_t* sc, const uint32_t* data,
                              const uint16_t* x, float* y, int rows, int kb) {
    const size_t lds = 2048 + (size_t)nw * RbLayout<NB>::STEP;
    if (lds > 65536) {  // past the default dynamic LDS limit (gfx950 has 160 KB a CU)
        static const bool raised = [] {
            return hipFuncSetAttribute(reinterpret_cast<const void*>(&iq4nl_rb_kernel<NB, R, S>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024) == hipSuccess;
        }();
        (void)raised;
    }
    iq4nl_rb_kernel<NB, R, S><<<g, nw * kWave, lds, st>>>(sc, data, x, y, rows, kb);
}

template <int NB>
static void launch_iq4nl_rb_n(int R, int S, dim3 g, int nw, hipStream_t st, const uint16_t* sc, const uint32_t* data,
                              const uint16_t* x, float* y, int rows, int kb) {
#define ZT_RB(RR, SS) \
    if (R == RR && S == SS) return launch_iq4nl_rb_t<NB, RR, SS>(g, nw, st, sc, data, x, y, rows, kb);
    ZT_RB(1, 1) ZT_RB(1, 2)
    if constexpr (NB <= 2) { ZT_RB(2, 1) ZT_RB(2, 2) ZT_RB(1, 4) ZT_RB(2, 4) ZT_RB(4, 1) }
    if constexpr (NB > 2) { ZT_RB(2, 1) ZT_RB(2, 2) ZT_RB(4, 1) ZT_RB(4, 2) }  // at most 8 waves: 512 threads
#undef ZT_RB
}

// Launch shape and eligibility: as the W4A16 row-block GEMM (steps of 16
// blocks, up to 16 waves splitting K, 8 for N >= 12), K <= 32768 (N >= 12:
// K <= 8192).
static bool iq4nl_rb_ok(int N, int kb, long M) {
    if (N < 4 || N > 16 || N % 4 != 0 || M * kb * 16 >= 0x7fffffffL) return false;
    return kb <= (N >= 12 ? 8 * 16 * 2 : 16 * 16 * 4);
}

static int launch_iq4nl_rb(const uint16_t* sc, const uint32_t* data, const uint16_t* x, float* y, int M, int kb, int N,
                           hipStream_t st) {
    const int steps = ceil_div(kb, 16), wmax = N >= 12 ? 8 : 16;
    const int S = steps <= wmax ? 1 : steps <= 2 * wmax ? 2 : 4;
    const int nw = ceil_div(steps, S);
    // R row sets a workgroup: up to 4 (2 past one step a wave) while about 200 or more workgroups
    // remain.  Measured at 3584 x 3584 (rows x K): batch 4 R = 1 / 2 / 4: 5.42 / 4.99 / 5.11 us, batch 8
    // 8.13 / 6.10 / 6.00; at 18944 x 3584, batch 8: 32.4 / 21.4 / 17.4 us (fewer activation bytes
    // staged per weight byte).  A sweep of 1-8 row sets x 1, 2 or 4 steps a wave (4 row sets past
    // one step and 8 under a 512-thread bound) at the Qwen2-7B shapes, batches 4 and 8, found
    // nothing more than 2% faster than this choice.  N >= 12 (at most 8 waves, the 512-thread
    // bound for more than one row set) takes up to 4: batch 16 at 3584 x 3584 19.3 / 12.0 / 8.0 us
    // with 1 / 2 / 4 row sets.
    const int rmax = N >= 12 ? 4 : S == 1 ? 4 : 2;
    int R = 1;
    while (R < rmax && ceil_div(M, 8 * R) >= 200) R *= 2;
    const dim3 g(ceil_div(M, 4 * R));
    switch (N) {
        case 4: launch_iq4nl_rb_n<1>(R, S, g, nw, st, sc, data, x, y, M, kb); break;
        case 8: launch_iq4nl_rb_n<2>(R, S, g, nw, st, sc, data, x, y, M, kb); break;
        case 12: launch_iq4nl_rb_n<3>(R, S, g, nw, st, sc, data, x, y, M, kb); break;
        default: launch_iq4nl_rb_n<4>(R, S, g, nw, st, sc, data, x, y, M, kb); break;
    }
    return (int)hipGetLastError();
}

static size_t iq4_mfma_lds_bytes(int N) {
    const size_t stage = (size_t)mfma_xbytes(N) + 16 + 16 * 4 + kMfmaUC * 4 * kMfmaRows * sizeof(uint16_t);
    return stage > mfma_reduce_bytes() ? stage : mfma_reduce_bytes();
}

template <Fmt F, int R, class XT, bool CONTIG>
__global__ void __launch_bounds__(512) gemv_blk18_kernel(const uint16_t* __restrict__ scales,
                                                         const uint4* __restrict__ data,
                                                         const XT* __restrict__ x, float* __restrict__ y,
                                                         long xy_stride, int rows, int kb) {
    __shared__ float red[8 * R];
    __shared__ float2 tbl[256];  // IQ4_NL: byte value -> (T[low nibble], T[high nibble])
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nwaves = blockDim.x >> 6;
    if constexpr (F == Fmt::IQ4NL) {
        for (int i = threadIdx.x; i < 256; i += blockDim.x) tbl[i] = make_float2(kIQ4NLTable[i & 0xf], kIQ4NLTable[i >> 4]);
        __syncthreads();
    }
    x += blockIdx.y;
    y += blockIdx.y;
    const int row0 = blockIdx.x * R;
    long rbase[R];
#pragma unroll
    for (int r = 0; r < R; r++) rbase[r] = (long)min(row0 + r, rows - 1) * kb;

    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.0f;

    for (int b = wave * kWave + lane; b < kb; b += nwaves * kWave) {
        uint4 w[R];
        uint16_t s[R];
#pragma unroll
        for (int r = 0; r < R; r++) {
            w[r] = ld_stream(&data[rbase[r] + b]);
            s[r] = scales[rbase[r] + b];
        }
        float xv[32];
        load_x32<XT, CONTIG>(x, xy_stride, b, xv);
        float xsum = 0.0f;
        if constexpr (F == Fmt::Q4_0) {
#pragma unroll
            for (int i = 0; i < 32; i++) xsum += xv[i];
        }
#pragma unroll
        for (int r = 0; r < R; r++) acc[r] = fmaf(h2f(s[r]), block_dot<F>(w[r], xv, xsum, tbl), acc[r]);
    }
    block_reduce_store<R>(acc, red, y, xy_stride, row0, rows);
}

template <Fmt F, class XT, bool CONTIG>
static void launch_gemv_r(int R, dim3 grid, dim3 block, hipStream_t st, const uint16_t* sc, const uint4* dt,
                          const XT* x, float* y, long stride, int rows, int kb) {
    switch (R) {
        case 8: gemv_blk18_kernel<F, 8, XT, CONTIG><<<grid, block, 0, st>>>(sc, dt, x, y, stride, rows, kb); break;
        case 4: gemv_blk18_kernel<F, 4, XT, CONTIG><<<grid, block, 0, st>>>(sc, dt, x, y, stride, rows, kb); break;
        case 2: gemv_blk18_kernel<F, 2, XT, CONTIG><<<grid, block, 0, st>>>(sc, dt, x, y, stride, rows, kb); break;
        default: gemv_blk18_kernel<F, 1, XT, CONTIG><<<grid, block, 0, st>>>(sc, dt, x, y, stride, rows, kb); break;
    }
}

template <int S, int NC>
static void launch_q4n_steps(int R, dim3 grid, dim3 block, hipStream_t st, const uint16_t* sc, const uint32_t* dt,
                             const float* x, float* y, int rows, int kb, int ldx, int n0) {
    switch (R) {
        case 8:
            if constexpr (NC <= 4) gemv_q4n_steps_kernel<S, 8, NC><<<grid, block, 0, st>>>(sc, dt, x, y, rows, kb, ldx, n0);
            break;
        case 4: gemv_q4n_steps_kernel<S, 4, NC><<<grid, block, 0, st>>>(sc, dt, x, y, rows, kb, ldx, n0); break;
        case 2: gemv_q4n_steps_kernel<S, 2, NC><<<grid, block, 0, st>>>(sc, dt, x, y, rows, kb, ldx, n0); break;
        default: gemv_q4n_steps_kernel<S, 1, NC><<<grid, block, 0, st>>>(sc, dt, x, y, rows, kb, ldx, n0); break;
    }
}

// Q4_0 with N > 1 fp32 columns on gemv_q4n_steps_kernel: column groups of 8
// (then 4) when B rows are 16-byte aligned, else groups of 2 when they are
// 8-byte aligned; each group is one launch that reads the weights once.
// Returns false (nothing launched) where the layout does not fit.
static bool launch_q4n(const uint16_t* sc, const uint32_t* dt, const float* B, float* C, int M, int kb, int N,
                       hipStream_t st) {
    if (N < 2 || kb > 512 || (long)M * kb * 16 >= 0x7fffffffL || (long)kb * 128 * N >= 0x7fffffffL) return false;
    const bool a16 = N % 4 == 0 && ((uintptr_t)B & 15) == 0;
    const bool a8 = N % 2 == 0 && ((uintptr_t)B & 7) == 0;
    if (!a16 && !a8) return false;
    const int S = kb <= 128 ? 1 : 2;
    int nw = ceil_div(kb, 16 * S);
    if (nw > 12) nw = 16;
    const dim3 block(nw * kWave);
    for (int n0 = 0; n0 < N;) {
        const int nc = a16 ? (N - n0 >= 8 ? 8 : 4) : 2;
        const int R = min(pick_rows_per_wave(M, nw, 1, 2048), 32 / nc);
        const dim3 grid(ceil_div(M, R));
        if (S == 1) {
            if (nc == 8) launch_q4n_steps<1, 8>(R, grid, block, st, sc, dt, B, C, M, kb, N, n0);
            else if (nc == 4) launch_q4n_steps<1, 4>(R, grid, block, st, sc, dt, B, C, M, kb, N, n0);
            else launch_q4n_steps<1, 2>(R, grid, block, st, sc, dt, B, C, M, kb, N, n0);
        } else {
            if (nc == 8) launch_q4n_steps<2, 8>(R, grid, block, st, sc, dt, B, C, M, kb, N, n0);
            else if (nc == 4) launch_q4n_steps<2, 4>(R, grid, block, st, sc, dt, B, C, M, kb, N, n0);
            else launch_q4n_steps<2, 2>(R, grid, block, st, sc, dt, B, C, M, kb, N, n0);
        }
        n0 += nc;
    }
    return true;
}

template <Fmt F, class XT>
static int gemm_blk18(const void* A, const XT* B, float* C, int M, int K, int N, int data_offset, hipStream_t st) {
    if (M < 0 || N < 0 || K < 0 || K % 32 != 0 || data_offset < 0 || N > 65535) return (int)hipErrorInvalidValue;
    if (M == 0 || N == 0) return (int)hipSuccess;
    if (A == nullptr || B == nullptr || C == nullptr) return (int)hipErrorInvalidValue;
    const uint8_t* base = static_cast<const uint8_t*>(A);
    const uint8_t* data = base + data_offset;
    if (((uintptr_t)base & 1) || ((uintptr_t)data & 15)) return (int)hipErrorInvalidValue;
    if (N == 1 && ((uintptr_t)B & 15)) return (int)hipErrorInvalidValue;
    const int kb = K / 32;
    const uint16_t* sc = reinterpret_cast<const uint16_t*>(base);
    if (N == 1) {
        const int nwaves = min(8, ceil_div(kb, 16));
        const int R = pick_rows_per_wave(M, nwaves, 1, 2048);
        if constexpr (F == Fmt::Q4_0) {
            // A fixed S steps per wave with all loads up front: S = 1 for K <= 4096,
            // S = 2 with up to 16 waves for K <= 16384 (measured best at K = 8192 and
            // 14336); longer rows loop.  Buffer offsets are 32-bit (data region < 2 GiB).
            // fp32 or fp16 activations (fp16: 3.96 / 7.75 us on the loop kernel against
            // 3.67 / 7.37 for fp32 at 4096 x 4096 / 14336 x 4096)
            const uint32_t* dt = reinterpret_cast<const uint32_t*>(data);
            if ((long)M * kb * 16 < 0x7fffffffL && kb <= 512) {
                const int S = kb <= 128 ? 1 : 2;
                int nw = ceil_div(kb, 16 * S);
                if (nw > 12) nw = 16;  // K = 14336: 16 waves measured 3% faster than 14
                const int Rs = pick_rows_per_wave(M, nw, 1, 2048);
                if (S == 1)
                    launch_q4_steps<1>(Rs, dim3(ceil_div(M, Rs)), dim3(nw * kWave), st, sc, dt, B, C, M, kb);
                else
                    launch_q4_steps<2>(Rs, dim3(ceil_div(M, Rs)), dim3(nw * kWave), st, sc, dt, B, C, M, kb);
                return (int)hipGetLastError();
            }
        }
        if constexpr (F == Fmt::IQ4NL && sizeof(XT) == 4) {
            // K <= 4096: the fixed-step form with the launch shape of the fp16 kernel below
            if ((long)M * kb * 16 < 0x7fffffffL && kb <= 128) {
                const int S = M >= 8192 ? 2 : 1;
                int nw = ceil_div(kb, 16 * S);
                if (nw > 4) nw = (nw + 3) & ~3;
                const int Rs = (long)ceil_div(M, 4) * nw >= 2048 ? 4 : pick_rows_per_wave(M, nw, 1, 2048);
                const dim3 g(ceil_div(M, Rs)), b(nw * kWave);
                const uint32_t* dt = reinterpret_cast<const uint32_t*>(data);
                const float* xf = reinterpret_cast<const float*>(B);
                if (S == 2)
                    launch_iq4nl_f32_steps<2>(Rs, g, b, st, sc, dt, xf, C, M, kb);
                else
                    launch_iq4nl_f32_steps<1>(Rs, g, b, st, sc, dt, xf, C, M, kb);
                return (int)hipGetLastError();
            }
            if ((long)M * kb * 16 < 0x7fffffffL) {
                const int Ri = pick_rows_per_wave(M, 16, 1, 2048);
                const int groups = ceil_div(M, Ri);
                const int nw = min(min(16, max(4, ceil_div(8192, groups))), ceil_div(kb, 16));
                const dim3 g(groups), b(nw * kWave);
                const uint32_t* dt = reinterpret_cast<const uint32_t*>(data);
                const float* xf = reinterpret_cast<const float*>(B);
                switch (Ri) {
                    case 8: gemv_iq4nl_f32_kernel<8><<<g, b, 0, st>>>(sc, dt, xf, C, M, kb); break;
                    case 4: gemv_iq4nl_f32_kernel<4><<<g, b, 0, st>>>(sc, dt, xf, C, M, kb); break;
                    case 2: gemv_iq4nl_f32_kernel<2><<<g, b, 0, st>>>(sc, dt, xf, C, M, kb); break;
                    default: gemv_iq4nl_f32_kernel<1><<<g, b, 0, st>>>(sc, dt, xf, C, M, kb); break;
                }
                return (int)hipGetLastError();
            }
        }
        if constexpr (F == Fmt::IQ4NL && sizeof(XT) == 2) {
            // Waves per workgroup chosen so the grid holds about 8192 waves
            // (4 .. 16, at most one per 16 blocks of a row).
            if ((long)M * kb * 16 < 0x7fffffffL && kb <= 128) {
                // K <= 4096: fixed steps, 2 steps on 4 waves for M >= 8192, else 1
                const int S = M >= 8192 ? 2 : 1;
                int nw = ceil_div(kb, 16 * S);
                if (nw > 4) nw = (nw + 3) & ~3;  // whole SIMD sets: 8 waves measured 3% faster than 7
                const int Rs = (long)ceil_div(M, 4) * nw >= 2048 ? 4 : pick_rows_per_wave(M, nw, 1, 2048);
                const dim3 g(ceil_div(M, Rs)), b(nw * kWave);
                const uint32_t* dt = reinterpret_cast<const uint32_t*>(data);
                const uint16_t* xh = reinterpret_cast<const uint16_t*>(B);
                if (S == 2)
                    launch_iq4nl_h16_steps<2>(Rs, g, b, st, sc, dt, xh, C, M, kb);
                else
                    launch_iq4nl_h16_steps<1>(Rs, g, b, st, sc, dt, xh, C, M, kb);
                return (int)hipGetLastError();
            }
            if ((long)M * kb * 16 < 0x7fffffffL) {
                const int Ri = pick_rows_per_wave(M, 16, 1, 2048);
                const int groups = ceil_div(M, Ri);
                const int nw = min(min(16, max(4, ceil_div(8192, groups))), ceil_div(kb, 16));
                launch_iq4nl_h16(Ri, dim3(groups), dim3(nw * kWave), st, sc, reinterpret_cast<const uint32_t*>(data),
                                 reinterpret_cast<const uint16_t*>(B), C, M, kb);
                return (int)hipGetLastError();
            }
        }
        launch_quad<F, XT>(R, dim3(ceil_div(M, R)), dim3(nwaves * kWave), st, sc,
                           reinterpret_cast<const uint32_t*>(data), B, C, M, kb);
        return (int)hipGetLastError();
    }
    if constexpr (F == Fmt::IQ4NL && sizeof(XT) == 4) {
        // fp32 activations, N % 4 == 0: the row-block GEMM, one launch a group of 4 or 8 columns
        if (rbf_ok<RbFmt::IQ4NL>(N, kb, M, B)) {
            launch_rbf<RbFmt::IQ4NL, Iq4QuadTbl>(sc, data, B, C, M, kb, N, st);
            return (int)hipGetLastError();
        }
    }
    if constexpr (F == Fmt::Q4_0 && sizeof(XT) == 4) {
        // 128 columns and more (prefill widths): the bf16 MFMA tile GEMM of zt_intq.hip, where the
        // row-block GEMM's launches of 8 columns each would re-run its per-column work (us, row-block
        // against tile GEMM, 4096 x 4096 / 14336 x 4096 / 4096 x 14336 rows x K: 64 columns 68.7 /
        // 160 / 360 against 106 / 269 / 402; 128 columns 136 / 321 / 715 against 127 / 185 / 465;
        // 512 columns 560 / 1283 / 2841 against 182 / 309 / 640)
        if (N >= 128 && N % 2 == 0 && ((uintptr_t)B & 7) == 0 && (long)ceil_div(M, 32) <= 65535) {
            bf16_gemm_q4_0(st, data, sc, reinterpret_cast<const float*>(B), C, M, N, K);
            return (int)hipGetLastError();
        }
        if (rbf_ok<RbFmt::Q4_0>(N, kb, M, B)) {
            launch_rbf<RbFmt::Q4_0>(sc, data, B, C, M, kb, N, st);
            return (int)hipGetLastError();
        }
        if (launch_q4n(sc, reinterpret_cast<const uint32_t*>(data), reinterpret_cast<const float*>(B), C, M, kb, N, st))
            return (int)hipGetLastError();
    }
    if constexpr (F == Fmt::IQ4NL && sizeof(XT) == 2) {
        // N = 4, 8 (12, 16 on up to 4096 rows; past that the 16x16x32 kernel below is as fast or
        // faster: 31.1 against 31.3 us at 18944 x 3584, batch 12): the row-block GEMM, one launch
        if (iq4nl_rb_ok(N, kb, M) && ((uintptr_t)B & 15) == 0 && (N <= 8 || M <= 4096))
            return launch_iq4nl_rb(sc, reinterpret_cast<const uint32_t*>(data), reinterpret_cast<const uint16_t*>(B),
                                   C, M, kb, N, st);
        if (mfma_shape_ok(N, K, B)) {
            // one workgroup per 32 rows over all of K: every output written once (no K split, no atomics)
            iq4nl_mfma_kernel<<<dim3(ceil_div(M, kMfmaRows)), kMfmaWaves * kWave, iq4_mfma_lds_bytes(N), st>>>(
                sc, reinterpret_cast<const uint4*>(data), reinterpret_cast<const uint16_t*>(B), C, M, K, N);
            return (int)hipGetLastError();
        }
    }
    const int nwaves = kb <= 64 ? 1 : (kb >= 8 * 64 ? 8 : ceil_div(kb, 64));
    const int R = pick_rows_per_wave(M, nwaves, N, 2048);
    dim3 grid(ceil_div(M, R), N), block(nwaves * kWave);
    launch_gemv_r<F, XT, false>(R, grid, block, st, sc, reinterpret_cast<const uint4*>(data), B, C, N, M, kb);
    return (int)hipGetLastError();
}

// ------------------------------------------------------------ dequantize

template <Fmt F, class OutT>
__global__ void dequant_blk18_kernel(const uint16_t* __restrict__ scales, const uint4* __restrict__ data,
                                     OutT* __restrict__ out, long nelem) {
    const long blk = (long)blockIdx.x * blockDim.x + threadIdx.x;
    const long nblk = (nelem + 31) / 32;
    if (blk >= nblk) return;
    const float d = h2f(scales[blk]);
    const uint4 w = data[blk];
    const uint32_t dw[4] = {w.x, w.y, w.z, w.w};
    float v[32];
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const uint32_t byte = (dw[i / 4] >> (8 * (i % 4))) & 0xffu;
        if constexpr (F == Fmt::Q4_0) {
            v[i] = (float)((int)(byte & 0x0f) - 8) * d;
            v[i + 16] = (float)((int)(byte >> 4) - 8) * d;
        } else {
            v[2 * i] = d * kIQ4NLTable[byte & 0x0f];
            v[2 * i + 1] = d * kIQ4NLTable[byte >> 4];
        }
    }
    OutT* o = out + blk * 32;
    const long rem = nelem - blk * 32;
    if (rem >= 32) {
#pragma unroll
        for (int i = 0; i < 32; i++) o[i] = out_cvt<OutT>(v[i]);
    } else {
        for (int i = 0; i < rem; i++) o[i] = out_cvt<OutT>(v[i]);
    }
}

template <Fmt F, class OutT = float>
static int dequant_blk18(const void* A, OutT* out, long nelem, int data_offset, hipStream_t st) {
    if (nelem < 0 || data_offset < 0) return (int)hipErrorInvalidValue;
    if (nelem == 0) return (int)hipSuccess;
    const uint8_t* base = static_cast<const uint8_t*>(A);
    if (((uintptr_t)base & 1) || ((uintptr_t)(base + data_offset) & 15)) return (int)hipErrorInvalidValue;
    const long nblk = (nelem + 31) / 32;
    dequant_blk18_kernel<F, OutT><<<ceil_div(nblk, 256), 256, 0, st>>>(
        reinterpret_cast<const uint16_t*>(base), reinterpret_cast<const uint4*>(base + data_offset), out, nelem);
    return (int)hipGetLastError();
}

}  // namespace zt

using namespace zt;

ZT_EXPORT int zt_gemm_q4_f32(const void* A_q4, const float* B, float* C, int M, int K, int N, int data_offset,
                             hipStream_t stream) {
    return gemm_blk18<Fmt::Q4_0, float>(A_q4, B, C, M, K, N, data_offset, stream);
}

ZT_EXPORT int zt_gemm_q4_group_f32(const zt_q4_gemv_desc* descs, int n, const float* x, int K,
                                   hipStream_t stream) {
    if (descs == nullptr || n < 1 || n > ZT_GROUP_MAX || K <= 0 || K % 32 != 0 || x == nullptr ||
        ((uintptr_t)x & 15))
        return (int)hipErrorInvalidValue;
    const int kb = K / 32;
    long total = 0;
    for (int i = 0; i < n; i++) {
        const zt_q4_gemv_desc& d = descs[i];
        const uint8_t* data = static_cast<const uint8_t*>(d.A) + d.data_offset;
        if (d.rows < 0 || d.reserved != 0) return (int)hipErrorInvalidValue;
        if (d.rows > 0 && (d.A == nullptr || d.y == nullptr || d.data_offset < 0 || ((uintptr_t)d.A & 1) ||
                           ((uintptr_t)data & 15)))
            return (int)hipErrorInvalidValue;
        total += d.rows;
    }
    if (total == 0) return (int)hipSuccess;
    bool fixed = kb <= 512;
    for (int i = 0; i < n; i++) fixed = fixed && (long)descs[i].rows * kb * 16 < 0x7fffffffL;
    if (!fixed) {
        // rows past the fixed-step kernel's reach: one launch per matrix
        for (int i = 0; i < n; i++) {
            const int rc = descs[i].rows == 0 ? 0
                         : zt_gemm_q4_f32(descs[i].A, x, descs[i].y, descs[i].rows, K, 1, (int)descs[i].data_offset,
                                          stream);
            if (rc != 0) return rc;
        }
        return (int)hipSuccess;
    }
    // the single-matrix launch configuration, rows per wave from the group's total rows
    const int S = kb <= 128 ? 1 : 2;
    int nw = ceil_div(kb, 16 * S);
    if (nw > 12) nw = 16;
    const int R = pick_rows_per_wave(total, nw, 1, 2048);
    bool std_layout = n <= 3;
    for (int i = 0; i < n; i++)
        std_layout = std_layout && descs[i].rows > 0 &&
                     descs[i].data_offset == ((2L * descs[i].rows * kb + 15) & ~15L);
    if (std_layout) {
        const uint8_t* a[3] = {nullptr, nullptr, nullptr};
        float* yv[3] = {nullptr, nullptr, nullptr};
        int rw[3] = {0, 0, 0};
        int wg3 = 0;
        for (int i = 0; i < n; i++) {
            a[i] = static_cast<const uint8_t*>(descs[i].A);
            yv[i] = descs[i].y;
            rw[i] = descs[i].rows;
            wg3 += ceil_div(descs[i].rows, R);
        }
        const dim3 grid3(wg3), block3(nw * kWave);
#define ZT_Q4G3(SS, RR) gemv_q4_group3_kernel<SS, RR><<<grid3, block3, 0, stream>>>(x, kb, n, a[0], a[1], a[2], \
                                                                                     rw[0], rw[1], rw[2], yv[0], \
                                                                                     yv[1], yv[2])
        if (S == 1) {
            switch (R) {
                case 8: ZT_Q4G3(1, 8); break;
                case 4: ZT_Q4G3(1, 4); break;
                case 2: ZT_Q4G3(1, 2); break;
                default: ZT_Q4G3(1, 1); break;
            }
        } else {
            switch (R) {
                case 8: ZT_Q4G3(2, 8); break;
                case 4: ZT_Q4G3(2, 4); break;
                case 2: ZT_Q4G3(2, 2); break;
                default: ZT_Q4G3(2, 1); break;
            }
        }
#undef ZT_Q4G3
        return (int)hipGetLastError();
    }
    Q4GroupArgs g{};
    int wg = 0;
    for (int i = 0; i < n; i++) {
        const uint8_t* base = static_cast<const uint8_t*>(descs[i].A);
        g.mat[i].sc = reinterpret_cast<const uint16_t*>(base);
        g.mat[i].dt = reinterpret_cast<const uint32_t*>(base + descs[i].data_offset);
        g.mat[i].y = descs[i].y;
        g.mat[i].rows = descs[i].rows;
        g.mat[i].wg0 = wg;
        g.wg0[i] = wg;
        wg += ceil_div(descs[i].rows, R);
    }
    g.n = n;
    const dim3 grid(wg), block(nw * kWave);
#define ZT_Q4G(SS, RR) gemv_q4_group_kernel<SS, RR><<<grid, block, 0, stream>>>(x, kb, g)
    if (S == 1) {
        switch (R) {
            case 8: ZT_Q4G(1, 8); break;
            case 4: ZT_Q4G(1, 4); break;
            case 2: ZT_Q4G(1, 2); break;
            default: ZT_Q4G(1, 1); break;
        }
    } else {
        switch (R) {
            case 8: ZT_Q4G(2, 8); break;
            case 4: ZT_Q4G(2, 4); break;
            case 2: ZT_Q4G(2, 2); break;
            default: ZT_Q4G(2, 1); break;
        }
    }
#undef ZT_Q4G
    return (int)hipGetLastError();
}

ZT_EXPORT int zt_gemm_q4_f16(const void* A_q4, const uint16_t* B, float* C, int M, int K, int N,
                             int data_offset, hipStream_t stream) {
    return gemm_blk18<Fmt::Q4_0, uint16_t>(A_q4, B, C, M, K, N, data_offset, stream);
}

ZT_EXPORT int zt_gemm_iq4nl_f32(const void* A_iq4, const float* B, float* C, int M, int K, int N,
                                int data_offset, hipStream_t stream) {
    return gemm_blk18<Fmt::IQ4NL, float>(A_iq4, B, C, M, K, N, data_offset, stream);
}

ZT_EXPORT int zt_gemm_iq4nl_f16(const void* A_iq4, const uint16_t* B, float* C, int M, int K, int N,
                                int data_offset, hipStream_t stream) {
    return gemm_blk18<Fmt::IQ4NL, uint16_t>(A_iq4, B, C, M, K, N, data_offset, stream);
}

ZT_EXPORT int zt_dequant_q4_f32(const void* A_q4, float* out, long nelem, int data_offset, hipStream_t stream) {
    return dequant_blk18<Fmt::Q4_0>(A_q4, out, nelem, data_offset, stream);
}

ZT_EXPORT int zt_dequant_q4_f16(const void* A_q4, uint16_t* out, long nelem, int data_offset, hipStream_t stream) {
    return dequant_blk18<Fmt::Q4_0, uint16_t>(A_q4, out, nelem, data_offset, stream);
}

ZT_EXPORT int zt_dequant_iq4nl_f32(const void* A_iq4, float* out, long nelem, int data_offset,
                                   hipStream_t stream) {
    return dequant_blk18<Fmt::IQ4NL>(A_iq4, out, nelem, data_offset, stream);
}

// ------------------------------------------------------------ IQ4_NL tiled layout
//
// An upload-time repack of the IQ4_NL separated layout for batched fp16
// activations (N in {4, 8, 12, 16}), the IQ4_NL counterpart of the tiled
// W4A16 layout.  For tile (rt, u) = rows 16 rt .. +16, blocks 4u .. 4u+3:
//   data: 1 KB at byte ((rt * K/128) + u) * 1024; the 16 bytes of lane
//     l = 16 g + i are dword g of blocks 4u, 4u+1, 4u+2, 4u+3 of row 16 rt + i
//     (elements 8g .. 8g+7 of each block, interleaved nibble order), so MFMA
//     step s takes component s of every lane and covers exactly block 4u+s;
//   scales: 128 bytes at ((rt * K/128) + u) * 128, fp16 [16 rows][4 blocks].
// Rows past M (to the next multiple of 16) are zero.

__global__ void iq4t_tile_kernel(const uint32_t* __restrict__ data, const uint16_t* __restrict__ scales,
                                 u32x4* __restrict__ wt, uint16_t* __restrict__ st, int rows, int nunits, long npieces) {
    const long p = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (p >= npieces) return;
    const int lane = (int)(p & 63), i = lane & 15, g = lane >> 4;
    const long tu = p >> 6;
    const int u = (int)(tu % nunits);
    const long row = (tu / nunits) * 16 + i;
    const long kb = (long)nunits * 4;
    u32x4 v = {0u, 0u, 0u, 0u};
    uint16_t sc = 0;
    if (row < rows) {
        const long b0 = row * kb + 4L * u;
        v = (u32x4){data[b0 * 4 + g], data[(b0 + 1) * 4 + g], data[(b0 + 2) * 4 + g], data[(b0 + 3) * 4 + g]};
        sc = scales[b0 + g];  // lane (i, g) also moves the scale of row i, block 4u + g
    }
    wt[p] = v;
    st[tu * 64 + i * 4 + g] = sc;
}

// Batched IQ4_NL on the tiled layout: the W4A16 tiled kernel's structure
// (4 waves x 32 rows a workgroup, UPW 128-K units, XCD-aware mapping, X and
// scales staged in LDS behind an LDS-only barrier while the 1 KB weight
// loads stream).  A operand: one ds_read_b64 per data byte from a 2 KB LDS
// table byte -> (hi pair, lo pair) (iq4_quad_entry, the codebook as T_hi +
// T_lo, within 2^-22.3 |T|).  The entries of two bytes are one A operand
// whose k slots hold Th Th Tl Tl Th Th Tl Tl of 4 elements, against a B
// operand with each activation pair twice, so the step's 8 elements of a
// lane take two chained MFMAs with no rescaling in between (an earlier form
// with a hi-part and a 2^-11-scaled lo-part MFMA needed a multiply per
// output and register moves to gather the parts: 17.0 -> 15.9 us at
// 18944 x 3584, batch 8).  Each step's result is scaled by its block's fp16
// scale in fp32.  The fp16-rounded table with one MFMA a step measured no
// faster than the split.
template <int UPW, int W, int N>
__global__ void __launch_bounds__(W * 64) iq4nlt_mfma_kernel(const uint4* __restrict__ wt,
                                                             const uint16_t* __restrict__ stl,
                                                             const uint16_t* __restrict__ x, int rows, int K, int nch,
                                                             int gx, int gy, float* __restrict__ y,
                                                             float* __restrict__ ws) {
    constexpr int KC = 128 * UPW;
    constexpr int RW = 32 * W;
    constexpr int XP = (KC * 2 * N / 16 + W * 64 - 1) / (W * 64);
    constexpr int SPC = RW / 16 * UPW * 128 / 16;  // 16-byte scale pieces of the workgroup
    constexpr int SP = (SPC + W * 64 - 1) / (W * 64);
    constexpr int XB = mfma_chunk_xbytes(KC, N);
    extern __shared__ __attribute__((aligned(16))) char smem[];
    char* zero_area = smem + XB;
    uint2* tbl = reinterpret_cast<uint2*>(zero_area + 16);         // 256 x (hi pair, lo pair)
    uint16_t* ssm = reinterpret_cast<uint16_t*>(tbl + 256);        // [tile in WG][unit][16 rows][4 blocks]
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int li = lane & 15, lg = lane >> 4;
    const int nunits = K / 128;
    int byi = blockIdx.y, bxi = blockIdx.x;
    // gx, gy: the grid's size, passed as arguments so they arrive in preloaded
    // SGPRs (gridDim is a kernel-argument load that every address waits for)
    if ((gx & 7) == 0) {
        const int id = blockIdx.x + gx * blockIdx.y, j = id >> 3;
        byi = j % gy;
        bxi = (id & 7) + 8 * (j / gy);
    }
    const int rw0 = bxi * RW, row0 = rw0 + 32 * wave;
    const int ntiles = (rows + 15) / 16;
    float4v acc[2];
    acc[0] = acc[1] = (float4v){0.f, 0.f, 0.f, 0.f};
    // this workgroup's K range: nch chunks of UPW units, one after another
    for (int ch = 0; ch < nch; ch++) {
    const int u0 = (byi * nch + ch) * UPW, u1 = min(nunits, u0 + UPW);
    if (u0 >= nunits) break;
    if (ch > 0) asm volatile("s_barrier" ::: "memory");  // every wave is done with the previous chunk's LDS
    const int npieces = (u1 - u0) * 128 * 2 * N / 16;
    const __amdgpu_buffer_rsrc_t rx =
        __builtin_amdgcn_make_buffer_rsrc((void*)(x + (long)u0 * 128 * N), (short)0, npieces * 16, 0x00020000);
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void*)stl, (short)0, 0x7fffffff, 0x00020000);
    u32x4 xr[XP];
#pragma unroll
    for (int i = 0; i < XP; i++)
        xr[i] = __builtin_amdgcn_raw_buffer_load_b128(rx, (uint32_t)(tid + i * W * 64) * 16u, 0, 0);
    // scales: piece e = (tile in WG) * UPW * 8 + unit * 8 + q (8 pieces of 16 bytes a tile-unit)
    u32x4 sr[SP];
#pragma unroll
    for (int i = 0; i < SP; i++) {
        const int e = tid + i * W * 64, tw = e / (UPW * 8), u = (e / 8) % UPW, q = e % 8;
        const int rt = rw0 / 16 + tw;
        const bool ok = e < SPC && rt < ntiles && u0 + u < u1;
        const uint32_t off = ok ? (uint32_t)(((rt * nunits + u0 + u) * 8 + q) * 16) : 0x80000000u;
        sr[i] = __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0);
    }
    uint4 w[UPW][2];
#pragma unroll
    for (int u = 0; u < UPW; u++) {
        const int unit = min(u0 + u, u1 - 1);
#pragma unroll
        for (int t = 0; t < 2; t++) {
            const int rt = min(row0 / 16 + t, ntiles - 1);
            w[u][t] = ld_stream(wt + ((long)rt * nunits + unit) * 64 + lane);
        }
    }
    if (tid < 4) reinterpret_cast<uint32_t*>(zero_area)[tid] = 0u;
    for (int i = tid; i < 256; i += W * 64) tbl[i] = iq4_quad_entry(i);
#pragma unroll
    for (int i = 0; i < XP; i++) {
        const int p = tid + i * W * 64;
        if (p < npieces) {
            const int off = p * 16;
            *reinterpret_cast<u32x4*>(smem + off + (off / (64 * N)) * (4 * N)) = xr[i];
        }
    }
#pragma unroll
    for (int i = 0; i < SP; i++) {
        const int e = tid + i * W * 64;
        if (e < SPC) *reinterpret_cast<u32x4*>(ssm + e * 8) = sr[i];
    }
    // LDS writes visible to the workgroup; the weight loads stay in flight.
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    // step s of unit u reads X rows 128u + 32s + 8lg + (li >> 2) (+ 4), whose
    // padded LDS offset is (8lg + (li >> 2)) 2N + (136u + 34s) 2N
    const int lbase = (8 * lg + (li >> 2)) * 2 * N + 8 * (li & 3);
#pragma unroll
    for (int u = 0; u < UPW; u++) {
        if (u0 + u < u1) {
#pragma unroll
            for (int s = 0; s < 4; s++) {
                const u32x4 bw = __builtin_bit_cast(u32x4, mfma_b_pair(smem, lbase + (136 * u + 34 * s) * 2 * N, 8 * N));
                // activation pairs (x0 x1), (x2 x3) each twice: k slots of the
                // A operand {entry(byte 0), entry(byte 1)} = Th0 Th1 Tl0 Tl1 Th2 Th3 Tl2 Tl3
                const half8v b1 = __builtin_bit_cast(half8v, (u32x4){bw[0], bw[0], bw[1], bw[1]});
                const half8v b2 = __builtin_bit_cast(half8v, (u32x4){bw[2], bw[2], bw[3], bw[3]});
#pragma unroll
                for (int t = 0; t < 2; t++) {
                    const uint32_t dw = s == 0 ? w[u][t].x : s == 1 ? w[u][t].y : s == 2 ? w[u][t].z : w[u][t].w;
                    const uint2 e0 = tbl[dw & 0xffu], e1 = tbl[(dw >> 8) & 0xffu], e2 = tbl[(dw >> 16) & 0xffu],
                                e3 = tbl[dw >> 24];
                    const u32x4 a1 = {e0.x, e0.y, e1.x, e1.y}, a2 = {e2.x, e2.y, e3.x, e3.y};
                    float4v d = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8v, a1), b1,
                                                                       (float4v){0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                    d = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8v, a2), b2, d, 0, 0, 0);
                    // scales of rows 4 lg + i of this tile, block 4u + s
                    const uint16_t* sp = ssm + ((2 * wave + t) * UPW + u) * 64 + 16 * lg + s;
#pragma unroll
                    for (int i = 0; i < 4; i++) acc[t][i] = fmaf(h2f(sp[4 * i]), d[i], acc[t][i]);
                }
            }
        }
    }
    }
    if (gy > 1) {
        // K split: partial tiles to the workspace, summed in split order by tiled_reduce_kernel
#pragma unroll
        for (int t = 0; t < 2; t++) {
            const int rt = row0 / 16 + t;
            if (rt < ntiles) tiled_store_partial(acc[t], ws, byi, ntiles, rt, lane, N);
        }
    } else if (li < N) {
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int row = row0 + 16 * t + 4 * lg + i;
                if (row < rows) y[(long)row * N + li] = acc[t][i];
            }
    }
}

template <int UPW, int N>
static void launch_iq4t(dim3 g, hipStream_t st, const uint4* wt, const uint16_t* sc, const uint16_t* x, float* y,
                        float* ws, int M, int K, int nch) {
    constexpr int W = 4;
    const size_t lds = (size_t)mfma_chunk_xbytes(128 * UPW, N) + 16 + 2048 + (size_t)2 * W * UPW * 64 * 2;
    iq4nlt_mfma_kernel<UPW, W, N><<<g, W * 64, lds, st>>>(wt, sc, x, M, K, nch, (int)g.x, (int)g.y, y, ws);
}

template <int N>
static void launch_iq4t_n(int upw, int nch, dim3 g, hipStream_t st, const uint4* wt, const uint16_t* sc,
                          const uint16_t* x, float* y, float* ws, int M, int K) {
    if (upw == 4)
        launch_iq4t<4, N>(g, st, wt, sc, x, y, ws, M, K, nch);
    else
        launch_iq4t<2, N>(g, st, wt, sc, x, y, ws, M, K, nch);
}

// Grid of the tiled IQ4_NL GEMM: 128 rows a workgroup and the largest K
// range, up to 4 units, that still gives >= 256 workgroups (8 units measured
// 8-13% slower at the Qwen2-7B shapes); K ranges split across blockIdx.y.
// When that leaves more than 8 splits and >= 256 workgroups remain with
// half as many, each workgroup walks 2 chunks in turn, so fewer partial tiles
// go through the workspace.
static dim3 iq4t_grid(int M, int K, int& upw, int& nch) {
    const int nunits = K / 128;
    const int gx = ceil_div(M, 128);
    upw = 4;
    while (upw > 2 && (long)gx * ceil_div(nunits, upw) < 256) upw >>= 1;
    // (2 chunks: 17.2 -> 16.0 us at 18944 x 3584, batch 8; 4 chunks measured 21 us)
    nch = (ceil_div(nunits, upw) > 8 && (long)gx * ceil_div(nunits, upw * 2) >= 256) ? 2 : 1;
    return dim3(gx, ceil_div(nunits, upw * nch));
}

ZT_EXPORT long zt_iq4nl_tiled_bytes(int M, int K) {
    if (M < 0 || K < 0 || K % 128 != 0) return -1;
    return (long)((M + 15) / 16) * 16 * (K / 2);
}

ZT_EXPORT long zt_iq4nl_tiled_scale_bytes(int M, int K) {
    if (M < 0 || K < 0 || K % 128 != 0) return -1;
    return (long)((M + 15) / 16) * 16 * (K / 32) * 2;
}

ZT_EXPORT int zt_iq4nl_tile(const void* A_iq4, int M, int K, int data_offset, void* W_tiled, void* S_tiled,
                            hipStream_t stream) {
    if (M < 0 || K < 0 || K % 128 != 0 || data_offset < 0) return (int)hipErrorInvalidValue;
    if (M == 0 || K == 0) return (int)hipSuccess;
    if (A_iq4 == nullptr || W_tiled == nullptr || S_tiled == nullptr) return (int)hipErrorInvalidValue;
    const uint8_t* base = static_cast<const uint8_t*>(A_iq4);
    if (((uintptr_t)base & 1) || ((uintptr_t)(base + data_offset) & 15) || ((uintptr_t)W_tiled & 15) ||
        ((uintptr_t)S_tiled & 15))
        return (int)hipErrorInvalidValue;
    const int nunits = K / 128;
    const long npieces = (long)((M + 15) / 16) * nunits * 64;
    iq4t_tile_kernel<<<ceil_div(npieces, 256), 256, 0, stream>>>(
        reinterpret_cast<const uint32_t*>(base + data_offset), reinterpret_cast<const uint16_t*>(base),
        static_cast<u32x4*>(W_tiled), static_cast<uint16_t*>(S_tiled), M, nunits, npieces);
    return (int)hipGetLastError();
}

ZT_EXPORT long zt_gemm_iq4nlt_workspace_bytes(int M, int K, int N) {
    if (M < 0 || K < 0 || K % 128 != 0 || (N != 4 && N != 8 && N != 12 && N != 16)) return -1;
    if (M == 0 || K == 0) return 0;
    int upw, nch;
    return tiled_ws_bytes(M, (int)iq4t_grid(M, K, upw, nch).y);
}

ZT_EXPORT int zt_gemm_iq4nlt_f16(const void* W_tiled, const void* S_tiled, const uint16_t* B, float* C, int M, int K,
                                 int N, void* workspace, long workspace_bytes, hipStream_t stream) {
    if (M < 0 || K < 0 || K % 128 != 0) return (int)hipErrorInvalidValue;
    if (N != 4 && N != 8 && N != 12 && N != 16) return (int)hipErrorInvalidValue;
    if (M == 0 || K == 0) return (int)hipSuccess;
    if (W_tiled == nullptr || S_tiled == nullptr || B == nullptr || C == nullptr) return (int)hipErrorInvalidValue;
    if (((uintptr_t)W_tiled & 15) || ((uintptr_t)S_tiled & 15) || ((uintptr_t)B & 15) || ((uintptr_t)C & 3))
        return (int)hipErrorInvalidValue;
    if ((long)((M + 15) / 16) * (K / 128) * 128 >= 0x7fffffffL) return (int)hipErrorInvalidValue;  // 32-bit scale offsets
    int upw, nch;
    const dim3 g = iq4t_grid(M, K, upw, nch);
    const long need = tiled_ws_bytes(M, (int)g.y);
    if (need > 0 && (workspace == nullptr || workspace_bytes < need || ((uintptr_t)workspace & 15)))
        return (int)hipErrorInvalidValue;
    const uint4* wt = static_cast<const uint4*>(W_tiled);
    const uint16_t* sc = static_cast<const uint16_t*>(S_tiled);
    float* ws = static_cast<float*>(workspace);
    switch (N) {
        case 4: launch_iq4t_n<4>(upw, nch, g, stream, wt, sc, B, C, ws, M, K); break;
        case 8: launch_iq4t_n<8>(upw, nch, g, stream, wt, sc, B, C, ws, M, K); break;
        case 12: launch_iq4t_n<12>(upw, nch, g, stream, wt, sc, B, C, ws, M, K); break;
        default: launch_iq4t_n<16>(upw, nch, g, stream, wt, sc, B, C, ws, M, K); break;
    }
    if (g.y > 1) tiled_reduce(workspace, C, M, N, (int)g.y, stream);
    return (int)hipGetLastError();
}

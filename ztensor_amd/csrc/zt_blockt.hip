// Small-batch GEMM on tiled upload layouts with MFMA, fp32 activations
// (N in {4, 8, 12, 16}), for gfx950: Q4_0, Q8_0 (and GGUF Q8_0), Q5_0
// (K % 128 == 0), and the K-quants Q4_K and Q5_K (K % 256 == 0).
//
// The reference computes these products with fp32 activations on its CPU
// engine (xblas.GemmF32Q4NT / GemmF32Q8NT, internal/xblas/gemm_quant.go:81-264)
// and with the per-row CUDA kernels gemm_q4_f32 / gemm_q8_f32
// (internal/cuda/kernels/gemm_q4.cu:117-201, gemm_q8.cu:121-182).  Here the
// batched product runs on v_mfma_f32_16x16x32_f16 instead:
//  * Weights are exact fp16 values of the normal range: a 4-bit value q
//    (Q4_0, Q4_K) becomes 2^14 + 2^10 q (the nibble moved to mantissa bits
//    6-9 under the exponent of 2^14: a shift and an and-or), a 5-bit value
//    (Q5_0, Q5_K) 2^15 + 2^10 q, a Q6_K value 2^15 + 2^9 q and a Q8_0 byte
//    2^15 + 2^7 (q + 128) (byte permutes and a shift-or).  Products with the
//    normalised activations are exact in fp32.  (These once entered as fp16
//    subnormals, q 2^-24; with activations spread in magnitude the gfx950
//    MFMAs sum such small products up to 1.5e-5 off, measured against fp64
//    products.)  The offset and the base are one more MFMA a step, every A
//    element -(base + off 2^10) (Q6_K 2^9, Q8_0 2^7), whose result is the C
//    input of the weight MFMAs of both tiles: each step's D is
//    2^10 sum((q - off) x), and one v_fma_mix per output takes the block's
//    fp16 scale straight from LDS.
//  * fp32 activations are split into two fp16 parts, x = hi + lo, after a
//    power-of-two normalisation per workgroup (max |x| of the workgroup's K
//    range maps into [2^14, 2^15)), so each activation is carried to about
//    2^-22 relative precision over the whole fp32 range; the normalisation
//    is undone exactly at the end.  For N <= 8 the hi parts sit in B columns
//    0..N-1 and the lo parts in columns 8..8+N-1 of the same MFMA, and the
//    two column halves are added once at the end; for N > 8 hi and lo are
//    two MFMAs into one accumulator.
//  * Each 16-row x 128-K tile is one contiguous block in MFMA lane order
//    (1 KB for Q4_0, 2 KB for Q8_0), so a wave's weight load is contiguous;
//    the workgroup structure (4 waves x 32 rows, UPW 128-K units, XCD-aware
//    K split, X and scales staged behind an LDS-only barrier while the
//    weights stream) follows the tiled W4A16 and IQ4_NL kernels.  K splits
//    store partial tiles to the caller's workspace and a second kernel sums
//    them in split order (tiled_reduce_kernel): fp32 atomics after a zero
//    fill measured 4.6 us of the 12.9 us at 14336 x 4096, batch 8.
//
// Tiled layouts (ntiles = ceil(M / 16), nunits = K / 128, tile-unit tu =
// rt * nunits + u; rows past M are zero):
//  * Q4_0 (zt_q4_tile): the IQ4_NL tiled layout applied to Q4_0's separated
//    layout, which has the same 18-byte block structure: data 1 KB at
//    tu * 1024, lane l = 16 g + i holds dword g of blocks 4u .. 4u+3 of row
//    16 rt + i; scales fp16 [16 rows][4 blocks] at tu * 128.
//  * Q8_0 (zt_q8_tile, zt_q8gguf_tile): data 2 KB at tu * 2048; half h
//    (1 KB) lane l = 16 g + i holds bytes 8g .. 8g+7 of block 4u + 2h, then
//    of block 4u + 2h + 1, of row 16 rt + i; scales fp32 [16 rows][4 blocks]
//    at tu * 256.
//  * Q5_0 (zt_q5_0_tile): the Q4_0 layout of its nibbles and scales, plus a
//    dword of fifth bits per lane at tu * 256 + 4 l (aux).
//  * Q4_K / Q5_K (zt_q4k_tile, zt_q5k_tile): each 32-value sub-block as a
//    Q4_0 block in the Q4_0 data layout; the 16-byte super-block headers
//    [tile][super-block][16 rows][16 B] (stl), decoded per workgroup into
//    (d * scale, dmin * min) pairs; Q5_K adds Q5_0's fifth-bit dwords (aux).
//    Each sub-block's min term uses the base MFMA (A all -2^14, Q5_K -2^15),
//    -2^14 sum(x) per step, which is also the C input of its weight MFMAs.
//  * Q6_K (zt_q6k_tile): the values 0..63 as bytes in the Q8_0 tile
//    positions, ordered so that lane group g holds values 4g .. 4g+3 of each
//    of a block's two 16-value groups; fp32 d * sc per group [16 rows]
//    [8 groups] at tu * 512.  Each group of a step is one 16x16x16 MFMA over
//    half of the A and B operands, with its own offset MFMA and scale (an
//    earlier form zeroed the other group's lane groups in two copies of B
//    for 16x16x32 MFMAs: 3.5-8% slower).
#include <algorithm>
#include <mutex>
#include <type_traits>

#include "zt_mfma.h"

namespace zt {

enum class BlkFmt { Q4_0, Q8_0, Q4_K, Q5_0, Q5_K, Q6_K };

// ST: the separated layout's scale type (float for Q8Storage, fp16 bits for
// GGUF Q8_0, widened exactly); the tiled scales are fp32 either way.
template <class ST>
__global__ void q8t_tile_kernel(const uint2* __restrict__ data, const ST* __restrict__ scales,
                                u32x4* __restrict__ wt, float* __restrict__ st, int rows, int nunits, long npieces) {
    const long p = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (p >= npieces) return;
    const int lane = (int)(p & 63), h = (int)((p >> 6) & 1), i = lane & 15, g = lane >> 4;
    const long tu = p >> 7;
    const int u = (int)(tu % nunits);
    const long row = (tu / nunits) * 16 + i;
    const long nb = (long)nunits * 4;  // blocks per row
    u32x4 v = {0u, 0u, 0u, 0u};
    if (row < rows) {
        const long b0 = row * nb + 4L * u + 2 * h;
        const uint2 a = data[b0 * 4 + g], b = data[(b0 + 1) * 4 + g];
        v = (u32x4){a.x, a.y, b.x, b.y};
    }
    wt[p] = v;
    if (h == 0) {
        float sv = 0.0f;
        if (row < rows) {
            if constexpr (sizeof(ST) == 2) sv = h2f(scales[row * nb + 4L * u + g]);
            else sv = scales[row * nb + 4L * u + g];
        }
        st[tu * 64 + i * 4 + g] = sv;
    }
}

// Q4_K tiled layout: the data in the Q4_0 tile format (each 32-value
// sub-block rewritten as the 16 bytes of a Q4_0 block: byte j holds values
// j and j+16), and the 16-byte super-block headers (fp16 d, fp16 dmin, 12
// bytes of 6-bit scales and mins) as [tile][super-block][16 rows][16 B].
// Q5_K (176-byte super-blocks: header, 128 bytes of nibbles as Q4_K, then
// 32 bytes of fifth bits, bit j of byte l for value l of sub-block j;
// tensor/quantized_kquant.go:509-549) tiles the same way, plus the fifth-bit dwords of the
// Q5_0 tiled layout in hq: bit k of byte s = the fifth bit of value
// 4g + (0, 2, 16, 18, 1, 3, 17, 19)[k] of block 4u+s.
template <bool Q5>
__global__ void q4kt_tile_kernel(const uint8_t* __restrict__ raw, u32x4* __restrict__ wt, u32x4* __restrict__ ht,
                                 uint32_t* __restrict__ hq, int rows, int nunits, long npieces) {
    constexpr int BB = Q5 ? 176 : 144;  // super-block bytes
    const long p = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (p >= npieces) return;
    const int lane = (int)(p & 63), i = lane & 15, g = lane >> 4;
    const long tu = p >> 6;
    const int u = (int)(tu % nunits);
    const long rt = tu / nunits;
    const long row = rt * 16 + i;
    const int nsb = nunits / 2;
    uint32_t v[4] = {0u, 0u, 0u, 0u}, fifth = 0u;
    if (row < rows) {
#pragma unroll
        for (int s = 0; s < 4; s++) {
            const int b = 4 * u + s, sb = b >> 3, j = b & 7, gq = j >> 1;
            if constexpr (Q5) {
                const uint8_t* qh = raw + (row * nsb + sb) * BB + 144;
                const int e[8] = {0, 2, 16, 18, 1, 3, 17, 19};
#pragma unroll
                for (int k = 0; k < 8; k++) fifth |= (uint32_t)((qh[4 * g + e[k]] >> j) & 1) << (8 * s + k);
            }
            const uint8_t* nib = raw + (row * nsb + sb) * BB + 16 + 32 * gq;
            const uint32_t a = *reinterpret_cast<const uint32_t*>(nib + 4 * g);
            const uint32_t c = *reinterpret_cast<const uint32_t*>(nib + 16 + 4 * g);
            v[s] = (j & 1) ? (((a >> 4) & 0x0F0F0F0Fu) | (c & 0xF0F0F0F0u))
                           : ((a & 0x0F0F0F0Fu) | ((c & 0x0F0F0F0Fu) << 4));
        }
    }
    wt[p] = (u32x4){v[0], v[1], v[2], v[3]};
    if constexpr (Q5) hq[p] = fifth;
    if ((u & 1) == 0 && g == 0) {  // header of (row, super-block u/2)
        u32x4 h = {0u, 0u, 0u, 0u};
        if (row < rows) h = *reinterpret_cast<const u32x4*>(raw + (row * nsb + u / 2) * BB);
        ht[(rt * nsb + u / 2) * 16 + i] = h;
    }
}

// Q5_0 tiled layout (from Q5_0Storage's RawBytesGPU: fp16 scales, uint32
// fifth-bit words, nibbles): the nibbles and scales exactly as the Q4_0 tiled
// layout, plus one dword per lane and tile-unit holding the fifth bits of
// the lane's 8 values in each of the 4 blocks (byte s = block 4u+s; bits
// 0..7 = values 4g, 4g+2, 4g+16, 4g+18, 4g+1, 4g+3, 4g+17, 4g+19, the order
// in which the kernel's masks take them).
__global__ void q5t_tile_kernel(const uint16_t* __restrict__ scales, const uint32_t* __restrict__ qh,
                                const uint32_t* __restrict__ qs, u32x4* __restrict__ wt, uint16_t* __restrict__ st,
                                uint32_t* __restrict__ ht, int rows, int nunits, long npieces) {
    const long p = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (p >= npieces) return;
    const int lane = (int)(p & 63), i = lane & 15, g = lane >> 4;
    const long tu = p >> 6;
    const int u = (int)(tu % nunits);
    const long row = (tu / nunits) * 16 + i;
    u32x4 v = {0u, 0u, 0u, 0u};
    uint32_t h = 0u;
    uint16_t sc = 0;
    if (row < rows) {
        const long b0 = row * (long)nunits * 4 + 4L * u;
        v = (u32x4){qs[b0 * 4 + g], qs[(b0 + 1) * 4 + g], qs[(b0 + 2) * 4 + g], qs[(b0 + 3) * 4 + g]};
        const int e[8] = {4 * g, 4 * g + 2, 4 * g + 16, 4 * g + 18, 4 * g + 1, 4 * g + 3, 4 * g + 17, 4 * g + 19};
#pragma unroll
        for (int s = 0; s < 4; s++) {
            const uint32_t w = qh[b0 + s];
#pragma unroll
            for (int k = 0; k < 8; k++) h |= ((w >> e[k]) & 1u) << (8 * s + k);
        }
        sc = scales[b0 + g];
    }
    wt[p] = v;
    ht[p] = h;
    st[tu * 64 + i * 4 + g] = sc;
}

// Q6_K tiled layout: the 6-bit values q (0..63) as bytes in the Q8_0 tile
// positions, lane group g taking values 4g .. 4g+3 and 16 + 4g .. 16 + 4g+3
// of each 32-value block (tensor/quantized_kquant.go:355-382: value 128h + 32j + l of a
// super-block takes its low 4 bits from ql[64h + 32(j&1) + l] (low nibble
// for j < 2, high for j >= 2) and its top 2 bits from qh[32h + l] >> 2j),
// and the fp32 products d * scale of every 16-value group as
// [tile-unit][16 rows][8 groups], the reference's first rounding.
__global__ void q6kt_tile_kernel(const uint8_t* __restrict__ raw, u32x4* __restrict__ wt, float* __restrict__ st,
                                 int rows, int nunits, long npieces) {
    const long p = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (p >= npieces) return;
    const int lane = (int)(p & 63), hh = (int)((p >> 6) & 1), i = lane & 15, g = lane >> 4;
    const long tu = p >> 7;
    const int u = (int)(tu % nunits);
    const long row = (tu / nunits) * 16 + i;
    const int nsb = nunits / 2;
    uint32_t v[4] = {0u, 0u, 0u, 0u};
    if (row < rows) {
#pragma unroll
        for (int bb = 0; bb < 2; bb++) {
            const int b = 4 * u + 2 * hh + bb;  // 32-value block of the row
#pragma unroll
            for (int k = 0; k < 8; k++) {
                // lane group g: values 4g .. 4g+3 of the block's first 16-value
                // group, then 4g .. 4g+3 of its second
                const int val = 32 * b + 16 * (k >> 2) + 4 * g + (k & 3), sb = val >> 8, vs = val & 255;
                const int h = vs >> 7, j = (vs >> 5) & 3, l = vs & 31;
                const uint8_t* blk = raw + ((long)row * nsb + sb) * 210;
                const int lo = (blk[64 * h + 32 * (j & 1) + l] >> (4 * (j >> 1))) & 15;
                const int hi = (blk[128 + 32 * h + l] >> (2 * j)) & 3;
                v[2 * bb + (k >> 2)] |= (uint32_t)(lo | (hi << 4)) << (8 * (k & 3));
            }
        }
    }
    wt[p] = (u32x4){v[0], v[1], v[2], v[3]};
    if (hh == 0 && g == 0) {
#pragma unroll
        for (int q = 0; q < 8; q++) {
            float sv = 0.0f;
            if (row < rows) {
                const int grp = 8 * u + q, sb = grp >> 4;  // 16 groups per super-block
                const uint8_t* blk = raw + ((long)row * nsb + sb) * 210;
                const float d = h2f((uint16_t)(blk[208] | (blk[209] << 8)));
                sv = d * (float)(int8_t)blk[192 + (grp & 15)];
            }
            st[(tu * 16 + i) * 8 + q] = sv;
        }
    }
}

// LDS row of chunk-relative activation row r (K index within the
// workgroup's range).  Within each 128-K unit, the 8 activations that lane
// group g of MFMA step s multiplies sit in rows 32 g + 8 s .. +7, in the
// order of the A operand's halves, so the two transposing reads of a step
// address 8 consecutive rows and the four lane groups are 32 rows apart.
template <BlkFmt F>
__device__ __forceinline__ int blkt_lds_row(int r) {
    const int u = r >> 7, b = (r >> 5) & 3, e = r & 31;
    int g, j;
    if constexpr (F == BlkFmt::Q6_K) {
        // lane group g: elements 4g .. 4g+3, then 16 + 4g .. 16 + 4g+3
        g = (e & 15) >> 2;
        j = ((e >> 4) << 2) + (e & 3);
    } else if constexpr (F != BlkFmt::Q8_0) {
        // A halves of lane group g: elements 4g, 4g+2, 4g+16, 4g+18, 4g+1, 4g+3, 4g+17, 4g+19
        const int i4 = e & 3;
        g = (e & 15) >> 2;
        j = (i4 & 1) * 4 + (i4 >> 1) + ((e >> 4) << 1);
    } else {
        g = e >> 3;  // elements 8g .. 8g+7 in order
        j = e & 7;
    }
    return (u << 7) + (g << 5) + (b << 3) + j;
}

template <BlkFmt F, int UPW, int N>
__global__ void __launch_bounds__(256) blkt_mfma_kernel(const uint4* __restrict__ wt, const void* __restrict__ stl,
                                                        const uint32_t* __restrict__ aux, const float* __restrict__ x,
                                                        int rows, int K, int gx, int gy, float* __restrict__ y,
                                                        float* __restrict__ ws) {
    constexpr int W = 4;
    constexpr int KC = 128 * UPW;
    constexpr int RW = 32 * W;
    constexpr int NPL = N <= 8 ? 1 : 2;                 // staged fp16 planes (hi/lo in columns, or two planes)
    constexpr int XPB = mfma_chunk_xbytes(KC, 16);      // one plane: 16 fp16 columns, 2 pad rows per 32
    constexpr int PPR = N / 4;                          // 16-byte pieces per fp32 activation row
    constexpr int XP = (KC * PPR + W * 64 - 1) / (W * 64);
    constexpr bool QK = F == BlkFmt::Q4_K || F == BlkFmt::Q5_K;  // super-block headers: (d*scale, dmin*min)
    constexpr bool Q5 = F == BlkFmt::Q5_0 || F == BlkFmt::Q5_K;  // fifth-bit dwords in aux
    constexpr bool Q6 = F == BlkFmt::Q6_K;  // byte values, one scale per 16: two half-steps
    constexpr int SB = F == BlkFmt::Q8_0 ? 4 : F == BlkFmt::Q6_K ? 8 : 2;  // scale bytes per (row, block)
    constexpr int PPT = 4 * SB;                         // 16-byte scale pieces per tile-unit
    // 16-byte scale pieces of the workgroup; Q4_K: one super-block header per row and super-block
    constexpr int SPC = QK ? (RW / 16) * (UPW / 2) * 16 : (RW / 16) * UPW * PPT;
    constexpr int SP = (SPC + W * 64 - 1) / (W * 64);
    constexpr int WL = (F == BlkFmt::Q8_0 || F == BlkFmt::Q6_K) ? 2 : 1;  // 16-byte weight loads per lane per tile-unit
    extern __shared__ __attribute__((aligned(16))) char smem[];
    float* wmax = reinterpret_cast<float*>(smem + NPL * XPB);  // per-wave max |x|
    char* ssm = smem + NPL * XPB + 16;                            // block scales
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
    const int u0 = byi * UPW, u1 = min(nunits, u0 + UPW);
    const int rw0 = bxi * RW, row0 = rw0 + 32 * wave;
    const int ntiles = (rows + 15) / 16;
    const int npieces = (u1 - u0) * 128 * PPR;
    const __amdgpu_buffer_rsrc_t rx =
        __builtin_amdgcn_make_buffer_rsrc((void*)(x + (long)u0 * 128 * N), (short)0, npieces * 16, 0x00020000);
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void*)stl, (short)0, 0x7fffffff, 0x00020000);
    u32x4 xr[XP];
#pragma unroll
    for (int i = 0; i < XP; i++)
        xr[i] = __builtin_amdgcn_raw_buffer_load_b128(rx, (uint32_t)(tid + i * W * 64) * 16u, 0, 0);
    u32x4 sr[SP];
#pragma unroll
    for (int i = 0; i < SP; i++) {
        const int e = tid + i * W * 64;
        uint32_t off;
        if constexpr (QK) {
            const int tw = e / (UPW / 2 * 16), sbl = (e / 16) % (UPW / 2), ri = e % 16;
            const int rt = rw0 / 16 + tw;
            const bool ok = e < SPC && rt < ntiles && u0 + 2 * sbl < u1;
            off = ok ? (uint32_t)(((rt * (nunits / 2) + u0 / 2 + sbl) * 16 + ri) * 16) : 0x80000000u;
        } else {
            const int tw = e / (UPW * PPT), u = (e / PPT) % UPW, q = e % PPT;
            const int rt = rw0 / 16 + tw;
            const bool ok = e < SPC && rt < ntiles && u0 + u < u1;
            off = ok ? (uint32_t)(((rt * nunits + u0 + u) * PPT + q) * 16) : 0x80000000u;
        }
        sr[i] = __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0);
    }
    uint4 w[UPW][2][WL];
#pragma unroll
    for (int u = 0; u < UPW; u++) {
        const int unit = min(u0 + u, u1 - 1);
#pragma unroll
        for (int t = 0; t < 2; t++) {
            const int rt = min(row0 / 16 + t, ntiles - 1);
#pragma unroll
            for (int h = 0; h < WL; h++) w[u][t][h] = ld_stream(wt + (((long)rt * nunits + unit) * WL + h) * 64 + lane);
        }
    }
    uint32_t qhw[Q5 ? UPW : 1][2];  // Q5_0, Q5_K: fifth bits of the lane's values, 4 blocks a dword
    if constexpr (Q5) {
#pragma unroll
        for (int u = 0; u < UPW; u++) {
            const int unit = min(u0 + u, u1 - 1);
#pragma unroll
            for (int t = 0; t < 2; t++) {
                const int rt = min(row0 / 16 + t, ntiles - 1);
                qhw[u][t] = __builtin_nontemporal_load(aux + ((long)rt * nunits + unit) * 64 + lane);
            }
        }
    }
    // workgroup max |x| -> power-of-two normalisation c = 2^sh
    float m = 0.0f;
#pragma unroll
    for (int i = 0; i < XP; i++)
#pragma unroll
        for (int c = 0; c < 4; c++) m = fmaxf(m, fabsf(__uint_as_float(xr[i][c])));
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
    if (lane == 0) wmax[wave] = m;
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    m = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
    int sh = 0;
    if (m > 0.0f && m <= 3.402823466e38f) {
        int e2;
        (void)frexpf(m, &e2);  // m = f 2^e2, f in [0.5, 1)
        sh = min(127, 15 - e2);
    }
    const float cs = ldexpf(1.0f, sh);
#pragma unroll
    for (int i = 0; i < XP; i++) {
        const int p = tid + i * W * 64;
        if (p < npieces) {
            const int r = p / PPR, c4 = (p % PPR) * 4;
            const float cr = cs;
            const int base = mfma_xrow(blkt_lds_row<F>(r), 16);
            uint32_t hv[2], lv[2];
#pragma unroll
            for (int c = 0; c < 4; c += 2) {
                const float v0 = __uint_as_float(xr[i][c]) * cr, v1 = __uint_as_float(xr[i][c + 1]) * cr;
                const _Float16 h0 = (_Float16)v0, h1 = (_Float16)v1;
                const _Float16 l0 = (_Float16)(v0 - (float)h0), l1 = (_Float16)(v1 - (float)h1);
                hv[c / 2] = (uint32_t)__builtin_bit_cast(uint16_t, h0) | ((uint32_t)__builtin_bit_cast(uint16_t, h1) << 16);
                lv[c / 2] = (uint32_t)__builtin_bit_cast(uint16_t, l0) | ((uint32_t)__builtin_bit_cast(uint16_t, l1) << 16);
            }
            const int lo_off = NPL == 1 ? 16 : XPB;
            if (N % 8 != 0 && c4 == N - 4) {
                // last piece of a row: it also zeroes the unused columns up to the
                // next multiple of 8, so every lane of a transposing read reads data
                *reinterpret_cast<uint4*>(smem + base + 2 * c4) = make_uint4(hv[0], hv[1], 0u, 0u);
                *reinterpret_cast<uint4*>(smem + lo_off + base + 2 * c4) = make_uint4(lv[0], lv[1], 0u, 0u);
            } else {
                *reinterpret_cast<uint2*>(smem + base + 2 * c4) = make_uint2(hv[0], hv[1]);
                *reinterpret_cast<uint2*>(smem + lo_off + base + 2 * c4) = make_uint2(lv[0], lv[1]);
            }
        }
    }
#pragma unroll
    for (int i = 0; i < SP; i++) {
        const int e = tid + i * W * 64;
        if constexpr (QK) {
            // header -> (d * scale, dmin * min) of the super-block's 8 sub-blocks
            // (tensor/quantized_kquant.go:34-79), fp32 products as the reference
            // forms them; stored [tile][unit][16 rows][4 blocks] as float2
            const int tw = e / (UPW / 2 * 16), sbl = (e / 16) % (UPW / 2), ri = e % 16;
            if (e < SPC && u0 + 2 * sbl < u1) {
                const u32x4 h = sr[i];
                const float d = h2f(h.x & 0xffffu), dmin = h2f(h.x >> 16);
                uint8_t b[12];
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    b[k] = (uint8_t)(h.y >> (8 * k));
                    b[4 + k] = (uint8_t)(h.z >> (8 * k));
                    b[8 + k] = (uint8_t)(h.w >> (8 * k));
                }
                float2* dst = reinterpret_cast<float2*>(ssm) + ((tw * UPW + 2 * sbl) * 16 + ri) * 4;
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    const int sc = j < 4 ? (b[j] & 63) : ((b[j + 4] & 0xF) | ((b[j - 4] >> 6) << 4));
                    const int mn = j < 4 ? (b[4 + j] & 63) : ((b[j + 4] >> 4) | ((b[j] >> 6) << 4));
                    dst[(j >> 2) * 64 + (j & 3)] = make_float2(d * (float)sc, dmin * (float)mn);
                }
            }
        } else {
            if (e < SPC) *reinterpret_cast<u32x4*>(ssm + e * 16) = sr[i];
        }
    }
    // LDS writes visible to the workgroup; the weight loads stay in flight.
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    // transposing-read address of this lane for unit u, step s: X row
    // 128u + 32 lg + 8s + jq (and + 4 for the second read), columns 4 qq ..
    // 4 qq + 3; mfma_xrow of that row is this lane base plus (136u + 8s) * 32.
    const int jq = li >> 2, qq = li & 3;
    const int lbase = (34 * lg + jq) * 32 + 8 * qq;
    // -(base + off 2^10) in every A element: one MFMA a step gives that times
    // sum(x), the C input of both tiles' weight MFMAs, so each step's D is
    // 2^10 sum((q - off) x) (Q6_K: 2^9, Q8_0: 2^7).
    // Q4_0: -(2^14 + 8 2^10) = -24576; Q5_0: -(2^15 + 16 2^10) = -49152;
    // Q4_K: -2^14 and Q5_K: -2^15 (no offset; the MFMA's result is also the
    // sub-block's min term); Q6_K: -(2^15 + 32 2^9); Q8_0: -(2^15 + 128 2^7).
    const _Float16 ol = __builtin_bit_cast(
        _Float16, (uint16_t)(F == BlkFmt::Q4_0 ? 0xF600u : F == BlkFmt::Q4_K ? 0xF400u : F == BlkFmt::Q5_K ? 0xF800u
                             : 0xFA00u));
    const half8v aoff = (half8v){ol, ol, ol, ol, ol, ol, ol, ol};
    // nibble (or 5-bit value) to mantissa: mask in a VGPR, exponent in an SGPR (v_and_or_b32)
    uint32_t nmask = Q5 ? 0x01E001E0u : 0x03C003C0u,
             nexp = (Q5 || Q6 || F == BlkFmt::Q8_0) ? 0x78007800u : 0x74007400u;
    asm volatile("" : "+v"(nmask), "+s"(nexp));
    float4v acc[2];
    acc[0] = acc[1] = (float4v){0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int u = 0; u < UPW; u++) {
        if (u0 + u < u1) {
            // the 4 block scales of rows 4 lg + i of each tile for this unit
            // (Q4_K: the (scale, min) pairs of the 4 blocks, two float4 a row)
            using SV = typename std::conditional<F == BlkFmt::Q4_0 || F == BlkFmt::Q5_0, uint2, float4>::type;
            constexpr int SVR = (QK || Q6) ? 2 : 1;
            SV sc[2][4][SVR];
#pragma unroll
            for (int t = 0; t < 2; t++)
#pragma unroll
                for (int i = 0; i < 4; i++)
#pragma unroll
                    for (int h = 0; h < SVR; h++)
                        sc[t][i][h] = reinterpret_cast<const SV*>(ssm)[(((2 * wave + t) * UPW + u) * 16 + 4 * lg + i) * SVR + h];
#pragma unroll
            for (int s = 0; s < 4; s++) {
                half8v bv[NPL];
#pragma unroll
                for (int pl = 0; pl < NPL; pl++) {
                    const int o = pl * XPB + (136 * u + 8 * s) * 32;
                    const short4v ba = tr_read_b64(smem, lbase + o), bb = tr_read_b64(smem, lbase + o + 128);
                    bv[pl] = __builtin_bit_cast(half8v, (short8v){ba[0], ba[1], ba[2], ba[3], bb[0], bb[1], bb[2], bb[3]});
                }
                if constexpr (Q6) {
                    // lane group g holds values 4g .. 4g+3 of each of the step's
                    // two 16-value groups (slots 0-3, then 4-7), so a 16x16x16
                    // MFMA over one half of A and B is exactly one group's sum
                    half4v bq[2][NPL];
#pragma unroll
                    for (int pl = 0; pl < NPL; pl++) {
                        const short8v b8 = __builtin_bit_cast(short8v, bv[pl]);
                        bq[0][pl] = __builtin_bit_cast(half4v, (short4v){b8[0], b8[1], b8[2], b8[3]});
                        bq[1][pl] = __builtin_bit_cast(half4v, (short4v){b8[4], b8[5], b8[6], b8[7]});
                    }
                    const half4v ao = (half4v){ol, ol, ol, ol};
                    float4v dq[2];
#pragma unroll
                    for (int hq = 0; hq < 2; hq++) {
                        dq[hq] = __builtin_amdgcn_mfma_f32_16x16x16f16(ao, bq[hq][0], (float4v){0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                        if constexpr (NPL == 2) dq[hq] = __builtin_amdgcn_mfma_f32_16x16x16f16(ao, bq[hq][1], dq[hq], 0, 0, 0);
                    }
#pragma unroll
                    for (int t = 0; t < 2; t++) {
                        const uint4 q = w[u][t][s >> 1];
                        const uint32_t da = (s & 1) ? q.z : q.x, db = (s & 1) ? q.w : q.y;
                        // values 0..63 to 2^15 + 2^9 q: byte permute, then v_lshl_or_b32
                        auto q6h = [&](uint32_t v) { return (v << 4) | nexp; };
                        const half4v aq[2] = {
                            __builtin_bit_cast(half4v, (uint2){q6h(__builtin_amdgcn_perm(da, da, 0x0C010C00u)),
                                                               q6h(__builtin_amdgcn_perm(da, da, 0x0C030C02u))}),
                            __builtin_bit_cast(half4v, (uint2){q6h(__builtin_amdgcn_perm(db, db, 0x0C010C00u)),
                                                               q6h(__builtin_amdgcn_perm(db, db, 0x0C030C02u))})};
                        float4v d[2];
#pragma unroll
                        for (int hq = 0; hq < 2; hq++) {
                            d[hq] = __builtin_amdgcn_mfma_f32_16x16x16f16(aq[hq], bq[hq][0], dq[hq], 0, 0, 0);
                            if constexpr (NPL == 2)
                                d[hq] = __builtin_amdgcn_mfma_f32_16x16x16f16(aq[hq], bq[hq][1], d[hq], 0, 0, 0);
                        }
#pragma unroll
                        for (int i = 0; i < 4; i++) {
                            const SV& pr = sc[t][i][s >> 1];  // groups 2s, 2s+1
                            const float s0 = (s & 1) ? pr.z : pr.x, s1 = (s & 1) ? pr.w : pr.y;
                            acc[t][i] = fmaf(s0, d[0][i], fmaf(s1, d[1][i], acc[t][i]));
                        }
                    }
                    continue;
                }
                float4v dn = __builtin_amdgcn_mfma_f32_16x16x32_f16(aoff, bv[0], (float4v){0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                if constexpr (NPL == 2) dn = __builtin_amdgcn_mfma_f32_16x16x32_f16(aoff, bv[1], dn, 0, 0, 0);
#pragma unroll
                for (int t = 0; t < 2; t++) {
                    u32x4 av;
                    if constexpr (F != BlkFmt::Q8_0) {
                        const uint4 q = w[u][t][0];
                        const uint32_t dw = s == 0 ? q.x : s == 1 ? q.y : s == 2 ? q.z : q.w;
                        // nibbles at bits 0-3, 4-7, 8-11, 12-15 of each half to mantissa bits 6-9
                        // (Q5: 5-8, the fifth bit then at 9)
                        if constexpr (Q5)
                            av = (u32x4){((dw << 5) & nmask) | nexp, ((dw << 1) & nmask) | nexp,
                                         ((dw >> 3) & nmask) | nexp, ((dw >> 7) & nmask) | nexp};
                        else
                            av = (u32x4){((dw << 6) & nmask) | nexp, ((dw << 2) & nmask) | nexp,
                                         ((dw >> 2) & nmask) | nexp, ((dw >> 6) & nmask) | nexp};
                        if constexpr (Q5) {
                            // fifth bits to bit 9 of each half (2^10 16 more); y = byte | byte << 15
                            // puts byte bits k and k+1 16 bits apart
                            const uint32_t xb = (qhw[u][t] >> (8 * s)) & 0xFFu, yb = xb | (xb << 15);
                            av[0] |= (yb << 9) & 0x02000200u;
                            av[1] |= (yb << 7) & 0x02000200u;
                            av[2] |= (yb << 5) & 0x02000200u;
                            av[3] |= (yb << 3) & 0x02000200u;
                        }
                    } else {
                        const uint4 q = w[u][t][s >> 1];
                        const uint32_t da = ((s & 1) ? q.z : q.x) ^ 0x80808080u;
                        const uint32_t db = ((s & 1) ? q.w : q.y) ^ 0x80808080u;
                        // bytes q + 128 to 2^15 + 2^7 (q + 128): byte permute, then v_lshl_or_b32
                        auto q8h = [&](uint32_t v) { return (v << 2) | nexp; };
                        av = (u32x4){q8h(__builtin_amdgcn_perm(da, da, 0x0C010C00u)),
                                     q8h(__builtin_amdgcn_perm(da, da, 0x0C030C02u)),
                                     q8h(__builtin_amdgcn_perm(db, db, 0x0C010C00u)),
                                     q8h(__builtin_amdgcn_perm(db, db, 0x0C030C02u))};
                    }
                    float4v d = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8v, av), bv[0], dn,
                                                                      0, 0, 0);
                    if constexpr (NPL == 2)
                        d = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8v, av), bv[1], d, 0, 0, 0);
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        if constexpr (QK) {
                            // D = 2^10 sum(q x) and dn = -2^14 sum(x) (Q5_K: -2^15):
                            // 2^10 (d sc sum(q x) - dmin mn sum(x)) = sv D + (mv 2^-4) dn
                            const SV& pr = sc[t][i][s >> 1];
                            const float sv = (s & 1) ? pr.z : pr.x, mv = (s & 1) ? pr.w : pr.y;
                            acc[t][i] = fmaf(sv, d[i], fmaf(mv * (F == BlkFmt::Q5_K ? 0.03125f : 0.0625f), dn[i],
                                                            acc[t][i]));
                        } else {
                            float sv;
                            if constexpr (F == BlkFmt::Q4_0 || F == BlkFmt::Q5_0) {  // fp16 scales
                                const uint32_t h2 = (s < 2) ? sc[t][i][0].x : sc[t][i][0].y;
                                sv = h2f((s & 1) ? (uint16_t)(h2 >> 16) : (uint16_t)(h2 & 0xffffu));
                            } else {
                                sv = s == 0 ? sc[t][i][0].x : s == 1 ? sc[t][i][0].y : s == 2 ? sc[t][i][0].z : sc[t][i][0].w;
                            }
                            acc[t][i] = fmaf(sv, d[i], acc[t][i]);
                        }
                    }
                }
            }
        }
    }
    // y = acc / (2^10 c) (Q6_K: 2^9 c; Q8_0: 2^7 c): the weight encoding's
    // factor and the activation normalisation undone in one exact
    // power-of-two scaling
#pragma unroll
    for (int t = 0; t < 2; t++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            float v = acc[t][i];
            if constexpr (NPL == 1) v += __shfl_xor(v, 8);  // hi columns n + lo columns 8 + n
            acc[t][i] = ldexpf(v, (F == BlkFmt::Q8_0 ? -7 : Q6 ? -9 : -10) - sh);
        }
    if (gy > 1) {
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

template <BlkFmt F, int UPW, int N>
static void launch_blkt(dim3 g, hipStream_t st, const uint4* wt, const void* sc, const uint32_t* aux, const float* x,
                        float* y, float* ws, int M, int K) {
    constexpr int NPL = N <= 8 ? 1 : 2;
    constexpr int SB = F == BlkFmt::Q8_0 ? 4 : (F == BlkFmt::Q4_K || F == BlkFmt::Q5_K || F == BlkFmt::Q6_K) ? 8 : 2;  // LDS bytes per (row, block)
    const size_t lds = (size_t)NPL * mfma_chunk_xbytes(128 * UPW, 16) + 16 + (size_t)8 * UPW * 64 * SB;
    blkt_mfma_kernel<F, UPW, N><<<g, 256, lds, st>>>(wt, sc, aux, x, M, K, (int)g.x, (int)g.y, y, ws);
}

template <BlkFmt F, int N>
static void launch_blkt_n(int upw, dim3 g, hipStream_t st, const uint4* wt, const void* sc, const uint32_t* aux,
                          const float* x, float* y, float* ws, int M, int K) {
    if (upw >= 4)
        launch_blkt<F, 4, N>(g, st, wt, sc, aux, x, y, ws, M, K);
    else
        launch_blkt<F, 2, N>(g, st, wt, sc, aux, x, y, ws, M, K);
}

// Grid of a tiled block GEMM: 128 rows by the largest K range per
// workgroup, up to 4 units, that still gives >= 256 (Q4_0) or >= 512 (Q8_0)
// workgroups; measured at the Llama-3-8B shapes, batches 8 and 16: 8 units
// were 3-14% slower for Q4_0 and 8-40% for Q8_0, and 8 waves a workgroup
// were slower at every unit count.
template <BlkFmt F>
static dim3 blkt_grid(int M, int K, int& upw) {
    const int nunits = K / 128, gx = ceil_div(M, 128);
    const long minwg = (F == BlkFmt::Q8_0 || F == BlkFmt::Q6_K) ? 512 : 256;
    upw = 4;
    while (upw > 2 && (long)gx * ceil_div(nunits, upw) < minwg) upw >>= 1;
    return dim3(gx, ceil_div(nunits, upw));
}

template <BlkFmt F>
static long blkt_ws_bytes(int M, int K, int N) {
    constexpr int KQ = (F == BlkFmt::Q4_K || F == BlkFmt::Q5_K || F == BlkFmt::Q6_K) ? 256 : 128;
    if (M < 0 || K < 0 || K % KQ != 0 || (N != 4 && N != 8 && N != 12 && N != 16)) return -1;
    if (M == 0 || K == 0) return 0;
    int upw;
    return tiled_ws_bytes(M, (int)blkt_grid<F>(M, K, upw).y);
}

template <BlkFmt F>
static int gemm_blkt(const void* W_tiled, const void* S_tiled, const float* B, float* C, int M, int K, int N,
                     void* ws, long ws_bytes, hipStream_t stream, const void* aux = nullptr, int force_upw = 0) {
    constexpr int KQ = (F == BlkFmt::Q4_K || F == BlkFmt::Q5_K || F == BlkFmt::Q6_K) ? 256 : 128;  // K-quants: whole super-blocks
    if (M < 0 || K < 0 || K % KQ != 0) return (int)hipErrorInvalidValue;
    if (N != 4 && N != 8 && N != 12 && N != 16) return (int)hipErrorInvalidValue;
    if (M == 0 || K == 0) return (int)hipSuccess;
    if (W_tiled == nullptr || S_tiled == nullptr || B == nullptr || C == nullptr) return (int)hipErrorInvalidValue;
    if (((uintptr_t)W_tiled & 15) || ((uintptr_t)S_tiled & 15) || ((uintptr_t)B & 15) || ((uintptr_t)C & 3))
        return (int)hipErrorInvalidValue;
    if ((F == BlkFmt::Q5_0 || F == BlkFmt::Q5_K) && (aux == nullptr || ((uintptr_t)aux & 15)))
        return (int)hipErrorInvalidValue;
    constexpr long SB = F == BlkFmt::Q8_0 ? 4 : F == BlkFmt::Q6_K ? 8 : 2;  // global scale bytes per (row, block); Q4_K: 16 per 8 blocks
    if ((long)((M + 15) / 16) * (K / 128) * 64 * SB >= 0x7fffffffL) return (int)hipErrorInvalidValue;  // 32-bit scale offsets
    int upw;
    dim3 g = blkt_grid<F>(M, K, upw);
    if (force_upw == 2 || force_upw == 4) {  // a row slice of a larger call: that call's K split
        upw = force_upw;
        g.y = ceil_div(K / 128, upw);
    }
    const long need = tiled_ws_bytes(M, (int)g.y);
    if (need > 0 && (ws == nullptr || ws_bytes < need || ((uintptr_t)ws & 15))) return (int)hipErrorInvalidValue;
    const uint4* wt = static_cast<const uint4*>(W_tiled);
    float* wsf = static_cast<float*>(ws);
    switch (N) {
        case 4: launch_blkt_n<F, 4>(upw, g, stream, wt, S_tiled, static_cast<const uint32_t*>(aux), B, C, wsf, M, K); break;
        case 8: launch_blkt_n<F, 8>(upw, g, stream, wt, S_tiled, static_cast<const uint32_t*>(aux), B, C, wsf, M, K); break;
        case 12: launch_blkt_n<F, 12>(upw, g, stream, wt, S_tiled, static_cast<const uint32_t*>(aux), B, C, wsf, M, K); break;
        default: launch_blkt_n<F, 16>(upw, g, stream, wt, S_tiled, static_cast<const uint32_t*>(aux), B, C, wsf, M, K); break;
    }
    if (g.y > 1) tiled_reduce(ws, C, M, N, (int)g.y, stream);
    return (int)hipGetLastError();
}

}  // namespace zt

using namespace zt;

// The IQ4_NL tile repack (zt_q4.hip) moves bytes and scales only, so it
// serves Q4_0's separated layout, which has the same 18-byte block shape.
extern "C" int zt_iq4nl_tile(const void* A_iq4, int M, int K, int data_offset, void* W_tiled, void* S_tiled,
                             hipStream_t stream);

ZT_EXPORT long zt_q4_tiled_bytes(int M, int K) {
    if (M < 0 || K < 0 || K % 128 != 0) return -1;
    return (long)((M + 15) / 16) * 16 * (K / 2);
}

ZT_EXPORT long zt_q4_tiled_scale_bytes(int M, int K) {
    if (M < 0 || K < 0 || K % 128 != 0) return -1;
    return (long)((M + 15) / 16) * 16 * (K / 32) * 2;
}

ZT_EXPORT int zt_q4_tile(const void* A_q4, int M, int K, int data_offset, void* W_tiled, void* S_tiled,
                         hipStream_t stream) {
    return zt_iq4nl_tile(A_q4, M, K, data_offset, W_tiled, S_tiled, stream);
}

ZT_EXPORT long zt_gemm_q4t_workspace_bytes(int M, int K, int N) { return blkt_ws_bytes<BlkFmt::Q4_0>(M, K, N); }

ZT_EXPORT int zt_gemm_q4t_f32(const void* W_tiled, const void* S_tiled, const float* B, float* C, int M, int K, int N,
                              void* workspace, long workspace_bytes, hipStream_t stream) {
    return gemm_blkt<BlkFmt::Q4_0>(W_tiled, S_tiled, B, C, M, K, N, workspace, workspace_bytes, stream);
}

// ---- allocation-free batched Q4_0: the K-split workspace in static device memory
//
// zt_gemm_q4t_f32_noalloc runs the kernels of zt_gemm_q4t_f32 with their
// workspace in `scratch`, a file-scope device array every GPU holds one copy
// of (at its own address) from the first call on it until the process ends.
// Host code never passes the array's name to a kernel: its device address is
// looked up once per device with hipGetSymbolAddress, with that device
// current, and kept in scratch_addr.  Calls on one GPU share the array, so
// calls that overlap on one GPU (different streams) race; on one stream they
// run in order.  Nothing in it needs clearing: every (split, tile) partial a
// call reads is written by the same call first.
static __device__ __align__(256) char scratch[ZT_NOALLOC_SCRATCH_BYTES];

constexpr int kScratchDevices = 64;
static std::mutex scratch_mu;
static void* scratch_addr[kScratchDevices];

// Device address of `scratch` on the current device, looked up on the first call.
static int scratch_on_current_device(void** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return (int)e;
    if (dev < 0 || dev >= kScratchDevices) return (int)hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(scratch_mu);
    if (scratch_addr[dev] == nullptr) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return (int)e;
        if (p == nullptr) return (int)hipErrorInvalidSymbol;
        scratch_addr[dev] = p;
    }
    *out = scratch_addr[dev];
    return (int)hipSuccess;
}

ZT_EXPORT int zt_gemm_q4t_f32_noalloc(const void* W_tiled, const void* S_tiled, const float* B, float* C, int M, int K,
                                      int N, hipStream_t stream) {
    const long need = blkt_ws_bytes<BlkFmt::Q4_0>(M, K, N);
    if (need < 0) return (int)hipErrorInvalidValue;
    if (need <= ZT_NOALLOC_SCRATCH_BYTES) {
        void* ws = nullptr;
        if (need > 0) {
            const int rc = scratch_on_current_device(&ws);
            if (rc != 0) return rc;
        }
        return gemm_blkt<BlkFmt::Q4_0>(W_tiled, S_tiled, B, C, M, K, N, ws, need, stream);
    }
    // Partials past the scratch: run the call as slices of whole 128-row
    // workgroup rows, each with the full call's K split, one after another on
    // the stream, so every output is the workspace entry point's to the bit.
    // A slice's tiles are contiguous in both tiled arrays (tile (rt, u) at
    // (rt * K/128 + u) * 1024 data bytes and * 128 scale bytes).
    int upw;
    const int splits = (int)blkt_grid<BlkFmt::Q4_0>(M, K, upw).y;
    const long per_group = tiled_ws_bytes(128, splits);  // 8 row tiles
    const long groups = ZT_NOALLOC_SCRATCH_BYTES / per_group;
    if (groups < 1) return (int)hipErrorOutOfMemory;
    if (W_tiled == nullptr || S_tiled == nullptr || B == nullptr || C == nullptr) return (int)hipErrorInvalidValue;
    void* ws = nullptr;
    const int rc0 = scratch_on_current_device(&ws);
    if (rc0 != 0) return rc0;
    const long slice = groups * 128, units = K / 128;
    for (long r0 = 0; r0 < M; r0 += slice) {
        const int rows = (int)std::min<long>(slice, M - r0);
        const long rt0 = r0 / 16;
        const int rc = gemm_blkt<BlkFmt::Q4_0>(static_cast<const uint8_t*>(W_tiled) + rt0 * units * 1024,
                                               static_cast<const uint8_t*>(S_tiled) + rt0 * units * 128, B,
                                               C + r0 * N, rows, K, N, ws, ZT_NOALLOC_SCRATCH_BYTES, stream, nullptr,
                                               upw);
        if (rc != 0) return rc;
    }
    return (int)hipSuccess;
}

ZT_EXPORT long zt_q8_tiled_bytes(int M, int K) {
    if (M < 0 || K < 0 || K % 128 != 0) return -1;
    return (long)((M + 15) / 16) * 16 * K;
}

ZT_EXPORT long zt_q8_tiled_scale_bytes(int M, int K) {
    if (M < 0 || K < 0 || K % 128 != 0) return -1;
    return (long)((M + 15) / 16) * 16 * (K / 32) * 4;
}

template <class ST>
static int q8_tile(const void* A_q8, int M, int K, long data_offset, void* W_tiled, void* S_tiled, hipStream_t stream) {
    if (M < 0 || K < 0 || K % 128 != 0 || data_offset < 0) return (int)hipErrorInvalidValue;
    if (M == 0 || K == 0) return (int)hipSuccess;
    if (A_q8 == nullptr || W_tiled == nullptr || S_tiled == nullptr) return (int)hipErrorInvalidValue;
    const uint8_t* base = static_cast<const uint8_t*>(A_q8);
    if (((uintptr_t)base & (sizeof(ST) - 1)) || ((uintptr_t)(base + data_offset) & 15) || ((uintptr_t)W_tiled & 15) ||
        ((uintptr_t)S_tiled & 15))
        return (int)hipErrorInvalidValue;
    const int nunits = K / 128;
    const long npieces = (long)((M + 15) / 16) * nunits * 128;
    q8t_tile_kernel<ST><<<ceil_div(npieces, 256), 256, 0, stream>>>(
        reinterpret_cast<const uint2*>(base + data_offset), reinterpret_cast<const ST*>(base),
        static_cast<u32x4*>(W_tiled), static_cast<float*>(S_tiled), M, nunits, npieces);
    return (int)hipGetLastError();
}

ZT_EXPORT int zt_q8_tile(const void* A_q8, int M, int K, long data_offset, void* W_tiled, void* S_tiled,
                         hipStream_t stream) {
    return q8_tile<float>(A_q8, M, K, data_offset, W_tiled, S_tiled, stream);
}

ZT_EXPORT int zt_q8gguf_tile(const void* A_q8, int M, int K, long data_offset, void* W_tiled, void* S_tiled,
                             hipStream_t stream) {
    return q8_tile<uint16_t>(A_q8, M, K, data_offset, W_tiled, S_tiled, stream);
}

ZT_EXPORT long zt_gemm_q8t_workspace_bytes(int M, int K, int N) { return blkt_ws_bytes<BlkFmt::Q8_0>(M, K, N); }

ZT_EXPORT int zt_gemm_q8t_f32(const void* W_tiled, const void* S_tiled, const float* B, float* C, int M, int K, int N,
                              void* workspace, long workspace_bytes, hipStream_t stream) {
    return gemm_blkt<BlkFmt::Q8_0>(W_tiled, S_tiled, B, C, M, K, N, workspace, workspace_bytes, stream);
}

ZT_EXPORT long zt_q4k_tiled_bytes(int M, int K) {
    if (M < 0 || K < 0 || K % 256 != 0) return -1;
    return (long)((M + 15) / 16) * 16 * (K / 2);
}

ZT_EXPORT long zt_q4k_tiled_header_bytes(int M, int K) {
    if (M < 0 || K < 0 || K % 256 != 0) return -1;
    return (long)((M + 15) / 16) * 16 * (K / 256) * 16;
}

ZT_EXPORT int zt_q4k_tile(const void* W_q4k, int M, int K, void* W_tiled, void* H_tiled, hipStream_t stream) {
    if (M < 0 || K < 0 || K % 256 != 0) return (int)hipErrorInvalidValue;
    if (M == 0 || K == 0) return (int)hipSuccess;
    if (W_q4k == nullptr || W_tiled == nullptr || H_tiled == nullptr) return (int)hipErrorInvalidValue;
    if (((uintptr_t)W_q4k & 15) || ((uintptr_t)W_tiled & 15) || ((uintptr_t)H_tiled & 15))
        return (int)hipErrorInvalidValue;
    const int nunits = K / 128;
    const long npieces = (long)((M + 15) / 16) * nunits * 64;
    q4kt_tile_kernel<false><<<ceil_div(npieces, 256), 256, 0, stream>>>(
        static_cast<const uint8_t*>(W_q4k), static_cast<u32x4*>(W_tiled), static_cast<u32x4*>(H_tiled), nullptr, M,
        nunits, npieces);
    return (int)hipGetLastError();
}

ZT_EXPORT long zt_gemm_q4kt_workspace_bytes(int M, int K, int N) { return blkt_ws_bytes<BlkFmt::Q4_K>(M, K, N); }

ZT_EXPORT int zt_gemm_q4kt_f32(const void* W_tiled, const void* H_tiled, const float* B, float* C, int M, int K, int N,
                               void* workspace, long workspace_bytes, hipStream_t stream) {
    return gemm_blkt<BlkFmt::Q4_K>(W_tiled, H_tiled, B, C, M, K, N, workspace, workspace_bytes, stream);
}

ZT_EXPORT long zt_q5_0_tiled_bytes(int M, int K) { return zt_q4_tiled_bytes(M, K); }

ZT_EXPORT long zt_q5_0_tiled_scale_bytes(int M, int K) { return zt_q4_tiled_scale_bytes(M, K); }

ZT_EXPORT long zt_q5_0_tiled_qh_bytes(int M, int K) {
    if (M < 0 || K < 0 || K % 128 != 0) return -1;
    return (long)((M + 15) / 16) * (K / 128) * 256;
}

ZT_EXPORT int zt_q5_0_tile(const void* A_q5, int M, int K, long qh_offset, long qs_offset, void* W_tiled,
                           void* S_tiled, void* H_tiled, hipStream_t stream) {
    if (M < 0 || K < 0 || K % 128 != 0 || qh_offset < 0 || qs_offset < 0) return (int)hipErrorInvalidValue;
    if (M == 0 || K == 0) return (int)hipSuccess;
    if (A_q5 == nullptr || W_tiled == nullptr || S_tiled == nullptr || H_tiled == nullptr)
        return (int)hipErrorInvalidValue;
    const uint8_t* base = static_cast<const uint8_t*>(A_q5);
    if (((uintptr_t)base & 1) || ((uintptr_t)(base + qh_offset) & 3) || ((uintptr_t)(base + qs_offset) & 15) ||
        ((uintptr_t)W_tiled & 15) || ((uintptr_t)S_tiled & 15) || ((uintptr_t)H_tiled & 15))
        return (int)hipErrorInvalidValue;
    const int nunits = K / 128;
    const long npieces = (long)((M + 15) / 16) * nunits * 64;
    q5t_tile_kernel<<<ceil_div(npieces, 256), 256, 0, stream>>>(
        reinterpret_cast<const uint16_t*>(base), reinterpret_cast<const uint32_t*>(base + qh_offset),
        reinterpret_cast<const uint32_t*>(base + qs_offset), static_cast<u32x4*>(W_tiled),
        static_cast<uint16_t*>(S_tiled), static_cast<uint32_t*>(H_tiled), M, nunits, npieces);
    return (int)hipGetLastError();
}

ZT_EXPORT long zt_gemm_q5_0t_workspace_bytes(int M, int K, int N) { return blkt_ws_bytes<BlkFmt::Q5_0>(M, K, N); }

ZT_EXPORT int zt_gemm_q5_0t_f32(const void* W_tiled, const void* S_tiled, const void* H_tiled, const float* B, float* C,
                                int M, int K, int N, void* workspace, long workspace_bytes, hipStream_t stream) {
    return gemm_blkt<BlkFmt::Q5_0>(W_tiled, S_tiled, B, C, M, K, N, workspace, workspace_bytes, stream, H_tiled);
}

ZT_EXPORT long zt_q5k_tiled_bytes(int M, int K) { return zt_q4k_tiled_bytes(M, K); }

ZT_EXPORT long zt_q5k_tiled_header_bytes(int M, int K) { return zt_q4k_tiled_header_bytes(M, K); }

ZT_EXPORT long zt_q5k_tiled_qh_bytes(int M, int K) {
    if (M < 0 || K < 0 || K % 256 != 0) return -1;
    return (long)((M + 15) / 16) * (K / 128) * 256;
}

ZT_EXPORT int zt_q5k_tile(const void* W_q5k, int M, int K, void* W_tiled, void* H_tiled, void* Q_tiled,
                          hipStream_t stream) {
    if (M < 0 || K < 0 || K % 256 != 0) return (int)hipErrorInvalidValue;
    if (M == 0 || K == 0) return (int)hipSuccess;
    if (W_q5k == nullptr || W_tiled == nullptr || H_tiled == nullptr || Q_tiled == nullptr)
        return (int)hipErrorInvalidValue;
    if (((uintptr_t)W_q5k & 15) || ((uintptr_t)W_tiled & 15) || ((uintptr_t)H_tiled & 15) || ((uintptr_t)Q_tiled & 15))
        return (int)hipErrorInvalidValue;
    const int nunits = K / 128;
    const long npieces = (long)((M + 15) / 16) * nunits * 64;
    q4kt_tile_kernel<true><<<ceil_div(npieces, 256), 256, 0, stream>>>(
        static_cast<const uint8_t*>(W_q5k), static_cast<u32x4*>(W_tiled), static_cast<u32x4*>(H_tiled),
        static_cast<uint32_t*>(Q_tiled), M, nunits, npieces);
    return (int)hipGetLastError();
}

ZT_EXPORT long zt_gemm_q5kt_workspace_bytes(int M, int K, int N) { return blkt_ws_bytes<BlkFmt::Q5_K>(M, K, N); }

ZT_EXPORT int zt_gemm_q5kt_f32(const void* W_tiled, const void* H_tiled, const void* Q_tiled, const float* B, float* C,
                               int M, int K, int N, void* workspace, long workspace_bytes, hipStream_t stream) {
    return gemm_blkt<BlkFmt::Q5_K>(W_tiled, H_tiled, B, C, M, K, N, workspace, workspace_bytes, stream, Q_tiled);
}

ZT_EXPORT long zt_q6k_tiled_bytes(int M, int K) {
    if (M < 0 || K < 0 || K % 256 != 0) return -1;
    return (long)((M + 15) / 16) * 16 * K;
}

ZT_EXPORT long zt_q6k_tiled_scale_bytes(int M, int K) {
    if (M < 0 || K < 0 || K % 256 != 0) return -1;
    return (long)((M + 15) / 16) * 16 * (K / 16) * 4;
}

ZT_EXPORT int zt_q6k_tile(const void* W_q6k, int M, int K, void* W_tiled, void* S_tiled, hipStream_t stream) {
    if (M < 0 || K < 0 || K % 256 != 0) return (int)hipErrorInvalidValue;
    if (M == 0 || K == 0) return (int)hipSuccess;
    if (W_q6k == nullptr || W_tiled == nullptr || S_tiled == nullptr) return (int)hipErrorInvalidValue;
    if (((uintptr_t)W_q6k & 1) || ((uintptr_t)W_tiled & 15) || ((uintptr_t)S_tiled & 15)) return (int)hipErrorInvalidValue;
    const int nunits = K / 128;
    const long npieces = (long)((M + 15) / 16) * nunits * 128;
    q6kt_tile_kernel<<<ceil_div(npieces, 256), 256, 0, stream>>>(static_cast<const uint8_t*>(W_q6k),
                                                                static_cast<u32x4*>(W_tiled), static_cast<float*>(S_tiled),
                                                                M, nunits, npieces);
    return (int)hipGetLastError();
}

ZT_EXPORT long zt_gemm_q6kt_workspace_bytes(int M, int K, int N) { return blkt_ws_bytes<BlkFmt::Q6_K>(M, K, N); }

ZT_EXPORT int zt_gemm_q6kt_f32(const void* W_tiled, const void* S_tiled, const float* B, float* C, int M, int K, int N,
                               void* workspace, long workspace_bytes, hipStream_t stream) {
    return gemm_blkt<BlkFmt::Q6_K>(W_tiled, S_tiled, B, C, M, K, N, workspace, workspace_bytes, stream);
}

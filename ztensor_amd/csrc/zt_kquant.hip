// K-quant (Q4_K, Q5_K, Q6_K) and Q5_0 batch-1 GEMV and dequantization for gfx950.
//
// Formats (value v of a 256-value super-block; each stored in the raw
// contiguous layout RawBytes() holds and the reference uploads as is,
// compute/gpu_engine.go:817-874):
//   Q4_K 144 B [fp16 d][fp16 dmin][12 B 6-bit scales/mins][128 B nibbles]:
//        group g = v/64 reads bytes 32g..32g+31; low nibble of byte l is
//        v = 64g+l (sub-block 2g), high nibble v = 64g+32+l (sub-block 2g+1);
//        w = (d*sc)*q - dmin*mn            (tensor/quantized_kquant.go:34-79)
//   Q5_K 176 B: Q4_K plus qh[32]: bit 2g / 2g+1 of qh[l] is the fifth bit of
//        the low / high nibble value                    (:509-549)
//   Q6_K 210 B [128 ql][64 qh][16 int8 scales][fp16 d]: value v uses scale
//        v/16; w = (d*sc)*(q-32)                        (:355-382)
//   Q5_0 22 B blocks of 32 [fp16 d][uint32 qh][16 B qs], uploaded in the
//        separated layout [d, nblk*2][pad 16][qh, nblk*4][pad 16][qs, nblk*16]
//        (tensor/quantized_q5_0.go:118-165); w = d*((nib | qh bit << 4) - 16).
//
// Batch-1 GEMV design (HBM-bound, every weight byte read once):
//  * K-quants: 16 lanes per super-block, each taking 8 bytes of the
//    low-bit array (16 weights), so a wave covers 4 super-blocks of R rows
//    per step and the waves of a workgroup split K;
//  * the nibbles (with the fifth / sixth bit OR-ed in by masks) are read as
//    fp16 subnormals q*2^-24 (low nibble) or q*2^-20 (high nibble, in place)
//    and v_fma_mix_f32 multiplies them into fp32 accumulators against
//    activations pre-scaled by 2^24 / 2^20, one chain per sub-block;
//  * the per-sub-block scale and min enter once per chain:
//    sum_v w_v x_v = d*(sc0*S0 + sc1*S1) - dmin*(mn0*X0 + mn1*X1)
//    (S = sum q x, X = sum x over the lane's values of that sub-block);
//  * Q6_K's 210-byte blocks are only 2-byte aligned: fields are read as
//    aligned dwords and joined with v_alignbit;
//  * Q5_0 uses the quad mapping of the Q4_0 kernel (four lanes per 32-value
//    block, one dword of nibbles each) with the qh bits spread into the
//    nibble bytes.
// The reference's CPU GEMVs apply each weight's dequantized value to x and
// sum in element order; the factored sums here reorder that fp32 sum, so
// GEMV results agree within rounding (the dequantizers are bit-exact).
#include "zt_mfma.h"

namespace zt {

// NW dwords at a 2-byte aligned address, from aligned dwords joined with
// v_alignbit.  The extra dword is read only when the address is misaligned:
// an aligned field ends at its last dword, and reading further could pass
// the end of the last block.
template <int NW>
__device__ __forceinline__ void ld_a2(const uint8_t* p, uint32_t (&out)[NW]) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(p);
    const uint32_t* q = reinterpret_cast<const uint32_t*>(a & ~(uintptr_t)3);
    const uint32_t s = (uint32_t)(a & 3) * 8u;
    uint32_t w[NW + 1];
#pragma unroll
    for (int i = 0; i < NW; i++) w[i] = __builtin_nontemporal_load(q + i);
    w[NW] = s ? __builtin_nontemporal_load(q + NW) : 0u;
#pragma unroll
    for (int i = 0; i < NW; i++) out[i] = __builtin_amdgcn_alignbit(w[i + 1], w[i], s);
}

// NW dwords at a 4*NW-byte aligned address.
template <int NW>
__device__ __forceinline__ void ld_vec(const uint8_t* p, uint32_t (&out)[NW]) {
    if constexpr (NW == 4) {
        const uint4 v = *reinterpret_cast<const uint4*>(p);
        out[0] = v.x; out[1] = v.y; out[2] = v.z; out[3] = v.w;
    } else {
        const uint2 v = *reinterpret_cast<const uint2*>(p);
        out[0] = v.x; out[1] = v.y;
    }
}

// Sum of the masked fp16 subnormals of NW dwords against pre-scaled
// activations.  m[j][0] / m[j][1] hold the values of bytes (0,2) / (1,3) of
// dword j in their two halves, i.e. values 4j+0, 4j+2 / 4j+1, 4j+3.
template <int NW>
__device__ __forceinline__ float chainw(const uint32_t (&m)[NW][2], const float (&xp)[4 * NW], float acc) {
#pragma unroll
    for (int j = 0; j < NW; j++) {
        const half2v a = as_half2(m[j][0]), b = as_half2(m[j][1]);
        acc = __builtin_fmaf((float)a.x, xp[4 * j + 0], acc);
        acc = __builtin_fmaf((float)b.x, xp[4 * j + 1], acc);
        acc = __builtin_fmaf((float)a.y, xp[4 * j + 2], acc);
        acc = __builtin_fmaf((float)b.y, xp[4 * j + 3], acc);
    }
    return acc;
}

// The lane's activations: 4*NW values at lo and 4*NW at hi (16-byte aligned),
// pre-scaled by 2^24 / 2^20 for the low / high nibble chains, plus their sums.
template <int NW>
struct KqX {
    float lo[4 * NW], hi[4 * NW];
    float slo, shi;
};

template <int NW>
__device__ __forceinline__ void kq_load_x(const float* __restrict__ x, long lo, long hi, bool valid, KqX<NW>& o) {
    float a[4 * NW], b[4 * NW];
#pragma unroll
    for (int i = 0; i < NW; i++) {
        float4 u = make_float4(0.f, 0.f, 0.f, 0.f), v = u;
        if (valid) {
            u = *reinterpret_cast<const float4*>(x + lo + 4 * i);
            v = *reinterpret_cast<const float4*>(x + hi + 4 * i);
        }
        a[4 * i] = u.x; a[4 * i + 1] = u.y; a[4 * i + 2] = u.z; a[4 * i + 3] = u.w;
        b[4 * i] = v.x; b[4 * i + 1] = v.y; b[4 * i + 2] = v.z; b[4 * i + 3] = v.w;
    }
    float sa = 0.0f, sb = 0.0f;
#pragma unroll
    for (int i = 0; i < 4 * NW; i++) {
        sa += a[i];
        sb += b[i];
        o.lo[i] = a[i] * 16777216.0f;
        o.hi[i] = b[i] * 1048576.0f;
    }
    o.slo = sa;
    o.shi = sb;
}

// Scale and min pairs (sub-blocks 2g, 2g+1) of a Q4_K/Q5_K header, as two
// bytes each (byte 0 = sub-block 2g).  hi_grp = g >= 2, sh = 16*(g&1).
__device__ __forceinline__ void kq_sc_mn(const uint4 h, bool hi_grp, uint32_t sh, uint32_t& scp, uint32_t& mnp) {
    const uint32_t A = h.y >> sh, B = h.z >> sh, C = h.w >> sh;
    const uint32_t s_lo = A & 0x3F3Fu, m_lo = B & 0x3F3Fu;
    const uint32_t s_hi = (C & 0x0F0Fu) | ((A >> 2) & 0x3030u);
    const uint32_t m_hi = ((C >> 4) & 0x0F0Fu) | ((B >> 2) & 0x3030u);
    scp = hi_grp ? s_hi : s_lo;
    mnp = hi_grp ? m_hi : m_lo;
}

// ------------------------------------------------------------ K-quant GEMV

template <int FMT>
struct KqFmt;
template <>
struct KqFmt<4> { static constexpr int bytes = 144; };
template <>
struct KqFmt<5> { static constexpr int bytes = 176; };
template <>
struct KqFmt<6> { static constexpr int bytes = 210; };

// NW = dwords of the low-bit array per lane (2 or 4): 128 / (4*NW) lanes
// share a super-block and a wave covers NW super-blocks per step.
template <int FMT, int NW, int R>
__global__ void __launch_bounds__(512) kq_gemv_kernel(const uint8_t* __restrict__ W, const float* __restrict__ x,
                                                      float* __restrict__ y, int rows, int nsb) {
    constexpr int BB = KqFmt<FMT>::bytes;
    constexpr int NB = 4 * NW;        // low-bit bytes per lane
    constexpr int LPS = 128 / NB;     // lanes per super-block
    constexpr int SPW = 64 / LPS;     // super-blocks per wave step
    __shared__ float red[8 * R];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nwaves = blockDim.x >> 6;
    const int slot = lane / LPS, t = lane % LPS;
    const int row0 = blockIdx.x * R;
    // Lane roles.  Q4_K/Q5_K: bytes t*NB .. of the 128 nibble bytes: group
    // g = t*NB/32, offset o = t*NB%32 -> values 64g+o+i (sub-block 2g) and
    // 64g+32+o+i (2g+1); Q5_K's fifth bits are qh bytes o .. o+NB-1.
    // Q6_K: half h = t*NB/64, w = t*NB%64: ql bytes 64h+w .. are values
    // vlo = 128h + 32*(w>=32) + w%32 + i (scale vlo/16, qh bits 0-1 / 2-3)
    // and vlo+64 (scale +4, qh bits 4-5 / 6-7); qh bytes 32h + w%32 ...
    const int byte0 = t * NB;
    const int g = byte0 >> 5, o = byte0 & 31;
    const int h6 = byte0 >> 6, w6 = byte0 & 63;
    const bool hi_grp = g >= 2;
    const uint32_t sh = 16u * (uint32_t)(g & 1);
    const int vlo = FMT == 6 ? 128 * h6 + 32 * (w6 >= 32) + (w6 & 31) : 64 * g + o;
    const int vhi = FMT == 6 ? vlo + 64 : vlo + 32;
    long rbase[R];
#pragma unroll
    for (int r = 0; r < R; r++) rbase[r] = (long)min(row0 + r, rows - 1) * nsb;
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.0f;

    for (int base = wave * SPW; base < nsb; base += nwaves * SPW) {
        const int sb = base + slot;
        const bool valid = sb < nsb;
        const int sbc = valid ? sb : nsb - 1;
        KqX<NW> xs;
        kq_load_x<NW>(x, (long)sbc * 256 + vlo, (long)sbc * 256 + vhi, valid, xs);
#pragma unroll
        for (int r = 0; r < R; r++) {
            const uint8_t* blk = W + (rbase[r] + sbc) * BB;
            uint32_t ml[NW][2], mh[NW][2];
            uint32_t qd[NW], hd[NW];
            if constexpr (FMT == 4 || FMT == 5) {
                const uint4 hdr = *reinterpret_cast<const uint4*>(blk);
                ld_vec<NW>(blk + 16 + byte0, qd);
                if constexpr (FMT == 5) ld_vec<NW>(blk + 144 + o, hd);
#pragma unroll
                for (int j = 0; j < NW; j++) {
                    const uint32_t d = qd[j], d8 = d >> 8;
                    uint32_t l0 = d & 0x000F000Fu, l2 = d8 & 0x000F000Fu, h0 = d & 0x00F000F0u, h2 = d8 & 0x00F000F0u;
                    if constexpr (FMT == 5) {
                        const uint32_t L = hd[j] >> (2 * g), H = hd[j] >> (2 * g + 1);
                        l0 |= (L << 4) & 0x00100010u;  // byte 0 / 2 fifth bit -> bit 4 / 20
                        l2 |= (L >> 4) & 0x00100010u;  // byte 1 / 3 -> bit 4 / 20
                        h0 |= (H << 8) & 0x01000100u;  // (q<<4) fifth bit -> bit 8 / 24
                        h2 |= H & 0x01000100u;
                    }
                    ml[j][0] = l0; ml[j][1] = l2; mh[j][0] = h0; mh[j][1] = h2;
                }
                const float S0 = chainw<NW>(ml, xs.lo, 0.0f);
                const float S1 = chainw<NW>(mh, xs.hi, 0.0f);
                uint32_t scp, mnp;
                kq_sc_mn(hdr, hi_grp, sh, scp, mnp);
                const float sc0 = (float)(scp & 0xFFu), sc1 = (float)((scp >> 8) & 0xFFu);  // v_cvt_f32_ubyte0/1
                const float mn0 = (float)(mnp & 0xFFu), mn1 = (float)((mnp >> 8) & 0xFFu);
                const float tq = __builtin_fmaf(sc1, S1, sc0 * S0);
                const float tm = __builtin_fmaf(mn1, xs.shi, mn0 * xs.slo);
                const half2v dd = as_half2(hdr.x);  // (d, dmin)
                acc[r] = __builtin_fmaf((float)dd.x, tq, acc[r]);
                acc[r] = __builtin_fmaf(-(float)dd.y, tm, acc[r]);
            } else {
                ld_a2<NW>(blk + byte0, qd);
                ld_a2<NW>(blk + 128 + 32 * h6 + (w6 & 31), hd);
                uint32_t scw[2];
                ld_a2<2>(blk + 192 + 8 * h6, scw);  // scales 8h .. 8h+7
                const uint32_t dw = *reinterpret_cast<const uint16_t*>(blk + 208);
                const uint32_t qsh = (w6 >= 32) ? 2u : 0u;  // lo uses qh bits 0-1 (2-3), hi bits 4-5 (6-7)
#pragma unroll
                for (int j = 0; j < NW; j++) {
                    const uint32_t d = qd[j], d8 = d >> 8;
                    const uint32_t L = hd[j] >> qsh, H = hd[j] >> (qsh + 4);
                    ml[j][0] = (d & 0x000F000Fu) | ((L << 4) & 0x00300030u);
                    ml[j][1] = (d8 & 0x000F000Fu) | ((L >> 4) & 0x00300030u);
                    mh[j][0] = (d & 0x00F000F0u) | ((H << 8) & 0x03000300u);
                    mh[j][1] = (d8 & 0x00F000F0u) | (H & 0x03000300u);
                }
                const float S0 = chainw<NW>(ml, xs.lo, -32.0f * xs.slo);
                const float S1 = chainw<NW>(mh, xs.hi, -32.0f * xs.shi);
                // scale index of vlo relative to 8h: 2*(w>=32) + (w%32)/16; of vhi that + 4
                const int si = 2 * (w6 >= 32) + ((w6 & 31) >> 4);
                const int sc0 = __builtin_amdgcn_sbfe((int)scw[0], 8 * si, 8);
                const int sc1 = __builtin_amdgcn_sbfe((int)scw[1], 8 * si, 8);
                const float tq = __builtin_fmaf((float)sc1, S1, (float)sc0 * S0);
                const half2v dd = as_half2(dw);
                acc[r] = __builtin_fmaf((float)dd.x, tq, acc[r]);
            }
        }
    }
    block_reduce_store<R>(acc, red, y, 1, row0, rows);
}

// Q4_K / Q5_K batch-1 GEMV with one fixed step of 4 super-blocks per wave
// (16 lanes x 8 bytes of the nibble array a super-block, the lane roles of
// kq_gemv_kernel with NW = 2), for K <= 64 super-blocks per wave group.
// Every load - nibbles, Q5_K fifth bits, the 16-byte headers and the
// activations - is issued before any arithmetic, as buffer loads whose
// wave-uniform row offset is the scalar offset; lanes past the last
// super-block read zeros through out-of-range offsets.
template <int FMT, int R>
__global__ void __launch_bounds__(1024) kq_steps_kernel(const uint8_t* __restrict__ W, const float* __restrict__ x,
                                                        float* __restrict__ y, int rows, int nsb) {
    constexpr int BB = KqFmt<FMT>::bytes;
    __shared__ float red[16 * R];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int slot = lane >> 4, t = lane & 15;
    const int byte0 = t * 8, g = byte0 >> 5, o = byte0 & 31;
    const bool hi_grp = g >= 2;
    const uint32_t sh = 16u * (uint32_t)(g & 1);
    const int vlo = 64 * g + o;
    const int row0 = blockIdx.x * R;
    const int sb = wave * 4 + slot;
    const bool ok = sb < nsb;
    const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc((void*)W, (short)0, 0x7fffffff, 0x00020000);
    const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc((void*)x, (short)0, nsb * 1024, 0x00020000);
    const uint32_t vq = ok ? (uint32_t)(sb * BB + 16 + byte0) : 0x80000000u;
    const uint32_t vqh = ok ? (uint32_t)(sb * BB + 144 + o) : 0x80000000u;
    const uint32_t vh = ok ? (uint32_t)(sb * BB) : 0x80000000u;
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
    uint32_t q0[R], q1[R], h0[R], h1[R];
    u32x4 hdr[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
        const uint32_t ro = (uint32_t)min(row0 + r, rows - 1) * (uint32_t)(nsb * BB);
        // one 8-byte load each (super-blocks of 144 / 176 bytes keep both fields 8-byte aligned)
        const u32x2 qv = __builtin_amdgcn_raw_buffer_load_b64(rw, vq, ro, 2);  // nontemporal
        q0[r] = qv.x;
        q1[r] = qv.y;
        if constexpr (FMT == 5) {
            const u32x2 hv = __builtin_amdgcn_raw_buffer_load_b64(rw, vqh, ro, 2);
            h0[r] = hv.x;
            h1[r] = hv.y;
        }
        hdr[r] = __builtin_amdgcn_raw_buffer_load_b128(rw, vh, ro, 0);
    }
    const uint32_t xo = ok ? (uint32_t)((sb * 256 + vlo) * 4) : 0x80000000u;
    const u32x4 xl0 = __builtin_amdgcn_raw_buffer_load_b128(rx, xo, 0, 0);
    const u32x4 xl1 = __builtin_amdgcn_raw_buffer_load_b128(rx, xo + 16, 0, 0);
    const u32x4 xh0 = __builtin_amdgcn_raw_buffer_load_b128(rx, xo + 128, 0, 0);
    const u32x4 xh1 = __builtin_amdgcn_raw_buffer_load_b128(rx, xo + 144, 0, 0);
    const uint32_t lw[8] = {xl0.x, xl0.y, xl0.z, xl0.w, xl1.x, xl1.y, xl1.z, xl1.w};
    const uint32_t hw[8] = {xh0.x, xh0.y, xh0.z, xh0.w, xh1.x, xh1.y, xh1.z, xh1.w};
    float lo[8], hi[8], slo = 0.f, shi = 0.f;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const float a = __uint_as_float(lw[i]), b = __uint_as_float(hw[i]);
        slo += a;
        shi += b;
        lo[i] = a * 16777216.0f;  // low-nibble chain: q * 2^-24
        hi[i] = b * 1048576.0f;   // high-nibble chain: q * 2^-20
    }
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
        const uint32_t dq[2] = {q0[r], q1[r]};
        float S0 = 0.f, S1 = 0.f;
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const uint32_t d = dq[j], d8 = d >> 8;
            uint32_t l0 = d & 0x000F000Fu, l2 = d8 & 0x000F000Fu, m0 = d & 0x00F000F0u, m2 = d8 & 0x00F000F0u;
            if constexpr (FMT == 5) {
                const uint32_t hq = j == 0 ? h0[r] : h1[r];
                const uint32_t L = hq >> (2 * g), H = hq >> (2 * g + 1);
                l0 |= (L << 4) & 0x00100010u;  // fifth bits of bytes 0 / 2 -> bit 4 / 20
                l2 |= (L >> 4) & 0x00100010u;  // bytes 1 / 3
                m0 |= (H << 8) & 0x01000100u;  // (q << 4) fifth bit -> bit 8 / 24
                m2 |= H & 0x01000100u;
            }
            const half2v a = as_half2(l0), b = as_half2(l2), c = as_half2(m0), e = as_half2(m2);
            S0 = __builtin_fmaf((float)a.x, lo[4 * j + 0], S0);
            S0 = __builtin_fmaf((float)b.x, lo[4 * j + 1], S0);
            S0 = __builtin_fmaf((float)a.y, lo[4 * j + 2], S0);
            S0 = __builtin_fmaf((float)b.y, lo[4 * j + 3], S0);
            S1 = __builtin_fmaf((float)c.x, hi[4 * j + 0], S1);
            S1 = __builtin_fmaf((float)e.x, hi[4 * j + 1], S1);
            S1 = __builtin_fmaf((float)c.y, hi[4 * j + 2], S1);
            S1 = __builtin_fmaf((float)e.y, hi[4 * j + 3], S1);
        }
        const uint4 h = make_uint4(hdr[r].x, hdr[r].y, hdr[r].z, hdr[r].w);
        uint32_t scp, mnp;
        kq_sc_mn(h, hi_grp, sh, scp, mnp);
        const float sc0 = (float)(scp & 0xFFu), sc1 = (float)((scp >> 8) & 0xFFu);
        const float mn0 = (float)(mnp & 0xFFu), mn1 = (float)((mnp >> 8) & 0xFFu);
        const float tq = __builtin_fmaf(sc1, S1, sc0 * S0);
        const float tm = __builtin_fmaf(mn1, shi, mn0 * slo);
        const half2v dd = as_half2(h.x);  // (d, dmin)
        acc[r] = __builtin_fmaf(-(float)dd.y, tm, (float)dd.x * tq);
    }
    block_reduce_store<R>(acc, red, y, 1, row0, rows);
}

template <int FMT>
static void launch_kq_steps(int R, dim3 grid, dim3 block, hipStream_t st, const uint8_t* W, const float* x, float* y,
                            int rows, int nsb) {
    switch (R) {
        case 16: kq_steps_kernel<FMT, 16><<<grid, block, 0, st>>>(W, x, y, rows, nsb); break;
        case 8: kq_steps_kernel<FMT, 8><<<grid, block, 0, st>>>(W, x, y, rows, nsb); break;
        case 4: kq_steps_kernel<FMT, 4><<<grid, block, 0, st>>>(W, x, y, rows, nsb); break;
        case 2: kq_steps_kernel<FMT, 2><<<grid, block, 0, st>>>(W, x, y, rows, nsb); break;
        default: kq_steps_kernel<FMT, 1><<<grid, block, 0, st>>>(W, x, y, rows, nsb); break;
    }
}

template <int FMT, int NW>
static void launch_kq(int R, dim3 grid, dim3 block, hipStream_t st, const uint8_t* W, const float* x, float* y,
                      int rows, int nsb) {
    switch (R) {
        case 8: kq_gemv_kernel<FMT, NW, 8><<<grid, block, 0, st>>>(W, x, y, rows, nsb); break;
        case 4: kq_gemv_kernel<FMT, NW, 4><<<grid, block, 0, st>>>(W, x, y, rows, nsb); break;
        case 2: kq_gemv_kernel<FMT, NW, 2><<<grid, block, 0, st>>>(W, x, y, rows, nsb); break;
        default: kq_gemv_kernel<FMT, NW, 1><<<grid, block, 0, st>>>(W, x, y, rows, nsb); break;
    }
}

template <int FMT>
static int gemv_kq(const void* W, const float* x, float* y, int M, int K, hipStream_t st) {
    if (M < 0 || K < 0 || K % 256 != 0) return (int)hipErrorInvalidValue;
    if (M == 0 || K == 0) {
        if (M > 0 && K == 0 && y) {  // empty sum
            mfma_zero(y, M, st);
            return (int)hipGetLastError();
        }
        return (int)hipSuccess;
    }
    if (W == nullptr || x == nullptr || y == nullptr) return (int)hipErrorInvalidValue;
    if (((uintptr_t)x & 15) || ((uintptr_t)W & (FMT == 6 ? 1 : 15))) return (int)hipErrorInvalidValue;
    const int nsb = K / 256;
    const uint8_t* w = static_cast<const uint8_t*>(W);
    if constexpr (FMT != 6) {
        // One fixed step per wave for K <= 16384 (32-bit buffer offsets) and
        // M >= 2048 (below, the loop kernel measured faster): 16 rows a wave
        // when more than 8 waves split K (measured best at K = 14336), else 8.
        if (nsb <= 64 && M >= 2048 && (long)M * nsb * KqFmt<FMT>::bytes < 0x7fffffffL) {
            const int nw = ceil_div(nsb, 4);
            const int Rs = nw > 8 && (long)ceil_div(M, 16) * nw >= 2048 ? 16 : pick_rows_per_wave(M, nw, 1, 2048);
            launch_kq_steps<FMT>(Rs, dim3(ceil_div(M, Rs)), dim3(nw * kWave), st, w, x, y, M, nsb);
            return (int)hipGetLastError();
        }
    }
    // 8 bytes of the low-bit array per lane (NW = 2): measured on the
    // Llama-3-8B shapes, 16 bytes per lane (NW = 4) was no faster for
    // Q4_K / Q5_K and 10-15% slower for Q6_K.
    const int nwaves = min(8, ceil_div(nsb, 4));
    const int R = pick_rows_per_wave(M, nwaves, 1, 2048);
    launch_kq<FMT, 2>(R, dim3(ceil_div(M, R)), dim3(nwaves * kWave), st, w, x, y, M, nsb);
    return (int)hipGetLastError();
}

// ------------------------------------------------------------ Q6_K split layout
//
// The raw 210-byte super-blocks are only 2-byte aligned, so the raw-layout
// GEMV reads every field as aligned dwords joined with v_alignbit.  The
// split layout (zt_q6k_split) regroups the same 210 bytes a super-block
// into four naturally aligned arrays over all M * nsb super-blocks t = row
// * nsb + sb: QL at 128 t, QH at 128 T + 64 t, SC at 192 T + 16 t and D at
// 208 T + 2 t (T = M * nsb).  Each lane's fields are then single 8-byte
// (ql, qh, scales) and 2-byte (d) buffer loads.

__global__ void q6k_split_kernel(const uint16_t* __restrict__ raw, uint16_t* __restrict__ out, long total) {
    const long t = (long)blockIdx.x * blockDim.x + threadIdx.x;  // super-block
    if (t >= total) return;
    const uint16_t* b = raw + t * 105;  // 210 bytes
#pragma unroll 8
    for (int i = 0; i < 64; i++) out[t * 64 + i] = b[i];                     // ql
#pragma unroll 8
    for (int i = 0; i < 32; i++) out[total * 64 + t * 32 + i] = b[64 + i];   // qh
#pragma unroll
    for (int i = 0; i < 8; i++) out[total * 96 + t * 8 + i] = b[96 + i];     // scales
    out[total * 104 + t] = b[104];                                           // d
}

// Q6_K batch-1 GEMV on the split layout: 16 lanes a super-block (8 ql bytes
// each, the lane roles of kq_gemv_kernel with NW = 2), 4 super-blocks a
// wave and step, the waves of a workgroup splitting K.  Every load of a
// step is issued before any arithmetic, as buffer loads whose wave-uniform
// row offsets are scalar offsets; lanes past the last super-block read
// zeros through out-of-range offsets.
template <int R>
__global__ void __launch_bounds__(1024) q6ks_gemv_kernel(const uint8_t* __restrict__ W, const float* __restrict__ x,
                                                         float* __restrict__ y, int rows, int nsb) {
    __shared__ float red[16 * R];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nwaves = blockDim.x >> 6;
    const int slot = lane >> 4, t = lane & 15;
    const int byte0 = t * 8, h6 = byte0 >> 6, w6 = byte0 & 63;
    // ql bytes 64 h + w .. +7: low nibbles are values vlo .. vlo+7, high
    // nibbles vlo+64 ..; qh bytes 32 h + w % 32 .. +7 hold their top two bits
    const int vlo = 128 * h6 + 32 * (w6 >= 32) + (w6 & 31), vhi = vlo + 64;
    const uint32_t qsh = (w6 >= 32) ? 2u : 0u;
    const int si = 2 * (w6 >= 32) + ((w6 & 31) >> 4);  // scale of vlo within 8 h .. 8 h + 7; vhi's is si + 4
    const int row0 = blockIdx.x * R;
    const uint32_t T = (uint32_t)rows * (uint32_t)nsb;
    const __amdgpu_buffer_rsrc_t rw =
        __builtin_amdgcn_make_buffer_rsrc((void*)W, (short)0, (int)(T * 210u), 0x00020000);
    const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc((void*)x, (short)0, nsb * 1024, 0x00020000);
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.0f;
    for (int sb0 = wave * 4; sb0 < nsb; sb0 += nwaves * 4) {
        const int sb = sb0 + slot;
        const bool ok = sb < nsb;
        const uint32_t vql = ok ? (uint32_t)(sb * 128 + byte0) : 0x80000000u;
        const uint32_t vqh = ok ? (uint32_t)(T * 128u + sb * 64 + 32 * h6 + (w6 & 31)) : 0x80000000u;
        const uint32_t vsc = ok ? (uint32_t)(T * 192u + sb * 16 + 8 * h6) : 0x80000000u;
        const uint32_t vd = ok ? (uint32_t)(T * 208u + sb * 2) : 0x80000000u;
        uint2 ql[R], qh[R], sc[R];
        uint32_t dd[R];
#pragma unroll
        for (int r = 0; r < R; r++) {
            const uint32_t rs = (uint32_t)min(row0 + r, rows - 1) * (uint32_t)nsb;
            ql[r] = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(rw, vql, rs * 128u, 2));
            qh[r] = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(rw, vqh, rs * 64u, 2));
            sc[r] = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(rw, vsc, rs * 16u, 0));
            dd[r] = __builtin_amdgcn_raw_buffer_load_b16(rw, vd, rs * 2u, 0);
        }
        const uint32_t xo = ok ? (uint32_t)((sb * 256 + vlo) * 4) : 0x80000000u;
        const u32x4 xl0 = __builtin_amdgcn_raw_buffer_load_b128(rx, xo, 0, 0);
        const u32x4 xl1 = __builtin_amdgcn_raw_buffer_load_b128(rx, xo + 16, 0, 0);
        const u32x4 xh0 = __builtin_amdgcn_raw_buffer_load_b128(rx, xo + 256, 0, 0);
        const u32x4 xh1 = __builtin_amdgcn_raw_buffer_load_b128(rx, xo + 272, 0, 0);
        const uint32_t lw[8] = {xl0.x, xl0.y, xl0.z, xl0.w, xl1.x, xl1.y, xl1.z, xl1.w};
        const uint32_t hw[8] = {xh0.x, xh0.y, xh0.z, xh0.w, xh1.x, xh1.y, xh1.z, xh1.w};
        float xlo[8], xhi[8], slo = 0.f, shi = 0.f;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const float a = __uint_as_float(lw[i]), b = __uint_as_float(hw[i]);
            slo += a;
            shi += b;
            xlo[i] = a * 16777216.0f;  // low-nibble chain: q * 2^-24
            xhi[i] = b * 1048576.0f;   // high-nibble chain: q * 2^-20
        }
#pragma unroll
        for (int r = 0; r < R; r++) {
            const uint32_t qd[2] = {ql[r].x, ql[r].y}, hd[2] = {qh[r].x, qh[r].y};
            uint32_t ml[2][2], mh[2][2];
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const uint32_t d = qd[j], d8 = d >> 8;
                const uint32_t L = hd[j] >> qsh, H = hd[j] >> (qsh + 4);
                ml[j][0] = (d & 0x000F000Fu) | ((L << 4) & 0x00300030u);
                ml[j][1] = (d8 & 0x000F000Fu) | ((L >> 4) & 0x00300030u);
                mh[j][0] = (d & 0x00F000F0u) | ((H << 8) & 0x03000300u);
                mh[j][1] = (d8 & 0x00F000F0u) | (H & 0x03000300u);
            }
            const float S0 = chainw<2>(ml, xlo, -32.0f * slo);
            const float S1 = chainw<2>(mh, xhi, -32.0f * shi);
            const int sc0 = __builtin_amdgcn_sbfe((int)sc[r].x, 8 * si, 8);
            const int sc1 = __builtin_amdgcn_sbfe((int)sc[r].y, 8 * si, 8);
            const float tq = __builtin_fmaf((float)sc1, S1, (float)sc0 * S0);
            acc[r] = __builtin_fmaf(h2f((uint16_t)dd[r]), tq, acc[r]);
        }
    }
    block_reduce_store<R>(acc, red, y, 1, row0, rows);
}

static void launch_q6ks(int R, dim3 grid, dim3 block, hipStream_t st, const uint8_t* W, const float* x, float* y,
                        int rows, int nsb) {
    switch (R) {
        case 8: q6ks_gemv_kernel<8><<<grid, block, 0, st>>>(W, x, y, rows, nsb); break;
        case 4: q6ks_gemv_kernel<4><<<grid, block, 0, st>>>(W, x, y, rows, nsb); break;
        case 2: q6ks_gemv_kernel<2><<<grid, block, 0, st>>>(W, x, y, rows, nsb); break;
        default: q6ks_gemv_kernel<1><<<grid, block, 0, st>>>(W, x, y, rows, nsb); break;
    }
}

// ------------------------------------------------------------ Q5_0 GEMV

// Spreads bits 0..3 of v into bit 0 of bytes 0..3 (distinct partial
// products of v * 0x00204081 land on distinct bits, so nothing carries).
__device__ __forceinline__ uint32_t spread4(uint32_t v) { return ((v & 0xFu) * 0x00204081u) & 0x01010101u; }

template <int R>
__global__ void __launch_bounds__(512) q5_0_gemv_kernel(const uint16_t* __restrict__ scales,
                                                        const uint32_t* __restrict__ qh,
                                                        const uint32_t* __restrict__ qs, const float* __restrict__ x,
                                                        float* __restrict__ y, int rows, int kb) {
    __shared__ float red[8 * R];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nwaves = blockDim.x >> 6;
    const int q = lane & 3;
    const int row0 = blockIdx.x * R;
    long rbase[R];
#pragma unroll
    for (int r = 0; r < R; r++) rbase[r] = (long)min(row0 + r, rows - 1) * kb;
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.0f;
    for (int b = wave * 16 + (lane >> 2); b < kb; b += nwaves * 16) {
        uint32_t w[R], hb[R];
        uint16_t s[R];
#pragma unroll
        for (int r = 0; r < R; r++) {
            w[r] = __builtin_nontemporal_load(&qs[(rbase[r] + b) * 4 + q]);
            hb[r] = qh[rbase[r] + b];
            s[r] = scales[rbase[r] + b];
        }
        // lane q: values 4q..4q+3 (low nibbles, qh bits 4q..) and 16+4q.. (high nibbles, qh bits 16+4q..)
        const float* p = x + (long)b * 32;
        const float4 a = *reinterpret_cast<const float4*>(p + 4 * q);
        const float4 c = *reinterpret_cast<const float4*>(p + 16 + 4 * q);
        const float xsum = ((a.x + a.y) + (a.z + a.w)) + ((c.x + c.y) + (c.z + c.w));
        const float xl[4] = {a.x * 16777216.0f, a.y * 16777216.0f, a.z * 16777216.0f, a.w * 16777216.0f};
        const float xh[4] = {c.x * 1048576.0f, c.y * 1048576.0f, c.z * 1048576.0f, c.w * 1048576.0f};
#pragma unroll
        for (int r = 0; r < R; r++) {
            const uint32_t d = w[r], d8 = d >> 8;
            const uint32_t el = spread4(hb[r] >> (4 * q)), eh = spread4(hb[r] >> (16 + 4 * q));
            const half2v m0 = as_half2((d & 0x000F000Fu) | ((el << 4) & 0x00100010u));
            const half2v m2 = as_half2((d8 & 0x000F000Fu) | ((el >> 4) & 0x00100010u));
            const half2v m1 = as_half2((d & 0x00F000F0u) | ((eh << 8) & 0x01000100u));
            const half2v m3 = as_half2((d8 & 0x00F000F0u) | (eh & 0x01000100u));
            float v = __builtin_fmaf((float)m0.x, xl[0], -16.0f * xsum);
            v = __builtin_fmaf((float)m1.x, xh[0], v);
            v = __builtin_fmaf((float)m2.x, xl[1], v);
            v = __builtin_fmaf((float)m3.x, xh[1], v);
            v = __builtin_fmaf((float)m0.y, xl[2], v);
            v = __builtin_fmaf((float)m1.y, xh[2], v);
            v = __builtin_fmaf((float)m2.y, xl[3], v);
            v = __builtin_fmaf((float)m3.y, xh[3], v);
            acc[r] = __builtin_fmaf(h2f(s[r]), v, acc[r]);
        }
    }
    block_reduce_store<R>(acc, red, y, 1, row0, rows);
}

// Q5_0 batch-1 GEMV in the fixed-step form of the Q4_0 kernel: each wave
// does S steps of 16 blocks (the quad mapping above), all loads issued
// before any arithmetic as buffer loads with the wave-uniform row offsets
// as scalar offsets; lanes past the last block read zeros.
template <int S, int R>
__global__ void __launch_bounds__(1024) q5_0_steps_kernel(const uint16_t* __restrict__ scales,
                                                          const uint32_t* __restrict__ qh,
                                                          const uint32_t* __restrict__ qs, const float* __restrict__ x,
                                                          float* __restrict__ y, int rows, int kb) {
    __shared__ float red[16 * R];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int q = lane & 3;
    const int row0 = blockIdx.x * R;
    const __amdgpu_buffer_rsrc_t rq = __builtin_amdgcn_make_buffer_rsrc((void*)qs, (short)0, 0x7fffffff, 0x00020000);
    const __amdgpu_buffer_rsrc_t rh = __builtin_amdgcn_make_buffer_rsrc((void*)qh, (short)0, 0x7fffffff, 0x00020000);
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void*)scales, (short)0, 0x7fffffff, 0x00020000);
    const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc((void*)x, (short)0, kb * 128, 0x00020000);
    uint32_t w[S][R], hb[S][R], sc[S][R];
    u32x4 xa[S], xc[S];
#pragma unroll
    for (int t = 0; t < S; t++) {
        const int b = (wave * S + t) * 16 + (lane >> 2);
        const bool ok = b < kb;
#pragma unroll
        for (int r = 0; r < R; r++) {
            const uint32_t row = (uint32_t)min(row0 + r, rows - 1);
            w[t][r] = __builtin_amdgcn_raw_buffer_load_b32(rq, ok ? (uint32_t)(b * 16 + q * 4) : 0x80000000u,
                                                           row * (uint32_t)kb * 16u, 2);  // nontemporal
        }
    }
#pragma unroll
    for (int t = 0; t < S; t++) {
        const int b = (wave * S + t) * 16 + (lane >> 2);
        const bool ok = b < kb;
#pragma unroll
        for (int r = 0; r < R; r++) {
            const uint32_t row = (uint32_t)min(row0 + r, rows - 1);
            const uint32_t blk4 = ok ? (uint32_t)(b * 4) : 0x80000000u, blk2 = ok ? (uint32_t)(b * 2) : 0x80000000u;
            hb[t][r] = __builtin_amdgcn_raw_buffer_load_b32(rh, blk4, row * (uint32_t)kb * 4u, 0);
            sc[t][r] = __builtin_amdgcn_raw_buffer_load_b16(rs, blk2, row * (uint32_t)kb * 2u, 0);
        }
        const uint32_t xo = ok ? (uint32_t)(b * 128 + q * 16) : 0x80000000u;
        xa[t] = __builtin_amdgcn_raw_buffer_load_b128(rx, xo, 0, 0);       // values 4q .. 4q+3
        xc[t] = __builtin_amdgcn_raw_buffer_load_b128(rx, xo + 64, 0, 0);  // values 16+4q ..
    }
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.0f;
#pragma unroll
    for (int t = 0; t < S; t++) {
        const float a0 = __uint_as_float(xa[t].x), a1 = __uint_as_float(xa[t].y), a2 = __uint_as_float(xa[t].z),
                    a3 = __uint_as_float(xa[t].w);
        const float c0 = __uint_as_float(xc[t].x), c1 = __uint_as_float(xc[t].y), c2 = __uint_as_float(xc[t].z),
                    c3 = __uint_as_float(xc[t].w);
        const float base = -16.0f * (((a0 + a1) + (a2 + a3)) + ((c0 + c1) + (c2 + c3)));
        const float xl[4] = {a0 * 16777216.0f, a1 * 16777216.0f, a2 * 16777216.0f, a3 * 16777216.0f};
        const float xh[4] = {c0 * 1048576.0f, c1 * 1048576.0f, c2 * 1048576.0f, c3 * 1048576.0f};
#pragma unroll
        for (int r = 0; r < R; r++) {
            const uint32_t d = w[t][r], d8 = d >> 8;
            const uint32_t el = spread4(hb[t][r] >> (4 * q)), eh = spread4(hb[t][r] >> (16 + 4 * q));
            const half2v m0 = as_half2((d & 0x000F000Fu) | ((el << 4) & 0x00100010u));
            const half2v m2 = as_half2((d8 & 0x000F000Fu) | ((el >> 4) & 0x00100010u));
            const half2v m1 = as_half2((d & 0x00F000F0u) | ((eh << 8) & 0x01000100u));
            const half2v m3 = as_half2((d8 & 0x00F000F0u) | (eh & 0x01000100u));
            float v = __builtin_fmaf((float)m0.x, xl[0], base);
            v = __builtin_fmaf((float)m1.x, xh[0], v);
            v = __builtin_fmaf((float)m2.x, xl[1], v);
            v = __builtin_fmaf((float)m3.x, xh[1], v);
            v = __builtin_fmaf((float)m0.y, xl[2], v);
            v = __builtin_fmaf((float)m1.y, xh[2], v);
            v = __builtin_fmaf((float)m2.y, xl[3], v);
            v = __builtin_fmaf((float)m3.y, xh[3], v);
            acc[r] = __builtin_fmaf((float)as_half2(sc[t][r]).x, v, acc[r]);
        }
    }
    block_reduce_store<R>(acc, red, y, 1, row0, rows);
}

template <int S>
static void launch_q5_0_steps(int R, dim3 grid, dim3 block, hipStream_t st, const uint16_t* sc, const uint32_t* qh,
                              const uint32_t* qs, const float* x, float* y, int rows, int kb) {
    switch (R) {
        case 8: q5_0_steps_kernel<S, 8><<<grid, block, 0, st>>>(sc, qh, qs, x, y, rows, kb); break;
        case 4: q5_0_steps_kernel<S, 4><<<grid, block, 0, st>>>(sc, qh, qs, x, y, rows, kb); break;
        case 2: q5_0_steps_kernel<S, 2><<<grid, block, 0, st>>>(sc, qh, qs, x, y, rows, kb); break;
        default: q5_0_steps_kernel<S, 1><<<grid, block, 0, st>>>(sc, qh, qs, x, y, rows, kb); break;
    }
}

static int gemv_q5_0(const void* W, const float* x, float* y, int M, int K, int qh_off, int qs_off, hipStream_t st) {
    if (M < 0 || K < 0 || K % 32 != 0 || qh_off < 0 || qs_off < 0) return (int)hipErrorInvalidValue;
    if (M == 0 || K == 0) {
        if (M > 0 && K == 0 && y) {
            mfma_zero(y, M, st);
            return (int)hipGetLastError();
        }
        return (int)hipSuccess;
    }
    if (W == nullptr || x == nullptr || y == nullptr) return (int)hipErrorInvalidValue;
    const uint8_t* base = static_cast<const uint8_t*>(W);
    if (((uintptr_t)base & 3) || ((uintptr_t)(base + qh_off) & 3) || ((uintptr_t)(base + qs_off) & 15) ||
        ((uintptr_t)x & 15))
        return (int)hipErrorInvalidValue;
    const int kb = K / 32;
    const uint16_t* sc = reinterpret_cast<const uint16_t*>(base);
    const uint32_t* qh = reinterpret_cast<const uint32_t*>(base + qh_off);
    if ((long)M * kb * 16 < 0x7fffffffL && kb <= 512) {
        // fixed steps, as for Q4_0: S = 1 for K <= 4096, else 2 with up to 16 waves
        const int S = kb <= 128 ? 1 : 2;
        const int nw = ceil_div(kb, 16 * S);
        const int Rs = pick_rows_per_wave(M, nw, 1, 2048);
        const uint32_t* qsp = reinterpret_cast<const uint32_t*>(base + qs_off);
        if (S == 1)
            launch_q5_0_steps<1>(Rs, dim3(ceil_div(M, Rs)), dim3(nw * kWave), st, sc, qh, qsp, x, y, M, kb);
        else
            launch_q5_0_steps<2>(Rs, dim3(ceil_div(M, Rs)), dim3(nw * kWave), st, sc, qh, qsp, x, y, M, kb);
        return (int)hipGetLastError();
    }
    const int nwaves = min(8, ceil_div(kb, 16));
    const int R = pick_rows_per_wave(M, nwaves, 1, 2048);
    const uint32_t* qs = reinterpret_cast<const uint32_t*>(base + qs_off);
    const dim3 grid(ceil_div(M, R)), block(nwaves * kWave);
    switch (R) {
        case 8: q5_0_gemv_kernel<8><<<grid, block, 0, st>>>(sc, qh, qs, x, y, M, kb); break;
        case 4: q5_0_gemv_kernel<4><<<grid, block, 0, st>>>(sc, qh, qs, x, y, M, kb); break;
        case 2: q5_0_gemv_kernel<2><<<grid, block, 0, st>>>(sc, qh, qs, x, y, M, kb); break;
        default: q5_0_gemv_kernel<1><<<grid, block, 0, st>>>(sc, qh, qs, x, y, M, kb); break;
    }
    return (int)hipGetLastError();
}

// ------------------------------------------------------------ dequantizers

// One thread per 32-value piece of a super-block (piece p = 0..7: values
// 32p .. 32p+31), each value computed with the reference's operations and
// rounding order, so the output is bit-identical to the CPU dequantizers.
template <int FMT>
__global__ void kq_dequant_kernel(const uint8_t* __restrict__ W, float* __restrict__ out, long npieces) {
    constexpr int BB = KqFmt<FMT>::bytes;
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= npieces) return;
    const long sbi = i >> 3;
    const int p = (int)(i & 7);
    const uint8_t* b = W + sbi * BB;
    float* o = out + i * 32;
    if constexpr (FMT == 4 || FMT == 5) {
        // piece p is sub-block p: group g = p/2, low nibbles (p even) or high (p odd)
        const int g = p >> 1, hi = p & 1;
        const float d = h2f((uint16_t)(b[0] | (b[1] << 8))), dmin = h2f((uint16_t)(b[2] | (b[3] << 8)));
        const uint8_t* sc = b + 4;
        uint32_t scale, mn;
        if (p < 4) {
            scale = sc[p] & 63;
            mn = sc[4 + p] & 63;
        } else {
            scale = (sc[8 + p - 4] & 0xF) | ((sc[p - 4] >> 6) << 4);
            mn = (sc[8 + p - 4] >> 4) | ((sc[4 + p - 4] >> 6) << 4);
        }
        const float s = d * (float)scale, m = dmin * (float)mn;
#pragma unroll 4
        for (int l = 0; l < 32; l++) {
            const uint8_t v = b[16 + 32 * g + l];
            uint32_t qv = hi ? (v >> 4) : (v & 0xF);
            if constexpr (FMT == 5) qv |= ((b[144 + l] >> (2 * g + hi)) & 1) << 4;
            o[l] = __fsub_rn(__fmul_rn(s, (float)qv), m);
        }
    } else {
        // piece p = half h = p/4, quarter j = p%4 (values 128h + 32j + l)
        const int h = p >> 2, j = p & 3;
        const float d = h2f((uint16_t)(b[208] | (b[209] << 8)));
        const uint8_t* ql = b + 64 * h + (j & 1) * 32;
        const uint8_t* qh = b + 128 + 32 * h;
        const int8_t* sc = reinterpret_cast<const int8_t*>(b + 192 + 8 * h);
#pragma unroll 4
        for (int l = 0; l < 32; l++) {
            const uint32_t nib = (j < 2) ? (ql[l] & 0xF) : (ql[l] >> 4);
            const uint32_t top = (qh[l] >> (2 * j)) & 3;
            const int q = (int)(nib | (top << 4)) - 32;
            o[l] = __fmul_rn(__fmul_rn(d, (float)sc[l / 16 + 2 * j]), (float)q);
        }
    }
}

template <int FMT>
static int dequant_kq(const void* W, float* out, int rows, int K, hipStream_t st) {
    if (rows < 0 || K < 0 || K % 256 != 0) return (int)hipErrorInvalidValue;
    if (rows == 0 || K == 0) return (int)hipSuccess;
    if (W == nullptr || out == nullptr) return (int)hipErrorInvalidValue;
    const long npieces = (long)rows * (K / 256) * 8;
    kq_dequant_kernel<FMT><<<ceil_div(npieces, 256), 256, 0, st>>>(static_cast<const uint8_t*>(W), out, npieces);
    return (int)hipGetLastError();
}

// Q5_0 over the raw 22-byte blocks (the layout dequant_q5_0_f32 reads,
// internal/cuda/kernels/dequant_q5_0.cu:18-67): one thread per block.
__global__ void q5_0_dequant_kernel(const uint8_t* __restrict__ raw, float* __restrict__ out, long nblk) {
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nblk) return;
    const uint8_t* b = raw + i * 22;
    const float d = h2f((uint16_t)(b[0] | (b[1] << 8)));
    const uint32_t qh = (uint32_t)b[2] | ((uint32_t)b[3] << 8) | ((uint32_t)b[4] << 16) | ((uint32_t)b[5] << 24);
    float* o = out + i * 32;
#pragma unroll 4
    for (int j = 0; j < 16; j++) {
        const uint8_t v = b[6 + j];
        const int x0 = (int)((v & 0xF) | (((qh >> j) & 1) << 4)) - 16;
        const int x1 = (int)((v >> 4) | (((qh >> (j + 16)) & 1) << 4)) - 16;
        o[j] = __fmul_rn(d, (float)x0);
        o[j + 16] = __fmul_rn(d, (float)x1);
    }
}

}  // namespace zt

using namespace zt;

ZT_EXPORT int zt_gemv_q4k_f32(const void* W, const float* x, float* y, int M, int K, hipStream_t stream) {
    return gemv_kq<4>(W, x, y, M, K, stream);
}
ZT_EXPORT int zt_gemv_q5k_f32(const void* W, const float* x, float* y, int M, int K, hipStream_t stream) {
    return gemv_kq<5>(W, x, y, M, K, stream);
}
ZT_EXPORT int zt_gemv_q6k_f32(const void* W, const float* x, float* y, int M, int K, hipStream_t stream) {
    return gemv_kq<6>(W, x, y, M, K, stream);
}
ZT_EXPORT long zt_q6k_split_bytes(int M, int K) {
    if (M < 0 || K < 0 || K % 256 != 0) return -1;
    return (long)M * (K / 256) * 210;
}

ZT_EXPORT int zt_q6k_split(const void* W_q6k, int M, int K, void* W_split, hipStream_t stream) {
    if (M < 0 || K < 0 || K % 256 != 0) return (int)hipErrorInvalidValue;
    if (M == 0 || K == 0) return (int)hipSuccess;
    if (W_q6k == nullptr || W_split == nullptr || ((uintptr_t)W_q6k & 1) || ((uintptr_t)W_split & 15))
        return (int)hipErrorInvalidValue;
    const long total = (long)M * (K / 256);
    q6k_split_kernel<<<ceil_div(total, 256), 256, 0, stream>>>(static_cast<const uint16_t*>(W_q6k),
                                                              static_cast<uint16_t*>(W_split), total);
    return (int)hipGetLastError();
}

ZT_EXPORT int zt_gemv_q6ks_f32(const void* W_split, const float* x, float* y, int M, int K, hipStream_t stream) {
    if (M < 0 || K < 0 || K % 256 != 0) return (int)hipErrorInvalidValue;
    if (M == 0 || K == 0) {
        if (M > 0 && K == 0 && y) {  // empty sum
            mfma_zero(y, M, stream);
            return (int)hipGetLastError();
        }
        return (int)hipSuccess;
    }
    if (W_split == nullptr || x == nullptr || y == nullptr || ((uintptr_t)W_split & 15) || ((uintptr_t)x & 15))
        return (int)hipErrorInvalidValue;
    const int nsb = K / 256;
    if ((long)M * nsb * 210 >= 0x7fffffffL || nsb > (1 << 20)) return (int)hipErrorInvalidValue;  // 32-bit buffer offsets
    // 4 super-blocks a wave and step, up to 16 waves splitting K (one step
    // each for K <= 16384), up to 8 rows a wave (16 spill registers at
    // 1024-thread workgroups)
    const int nw = min(16, ceil_div(nsb, 4));
    const int R = pick_rows_per_wave(M, nw, 1, 2048);
    launch_q6ks(R, dim3(ceil_div(M, R)), dim3(nw * kWave), stream, static_cast<const uint8_t*>(W_split), x, y, M, nsb);
    return (int)hipGetLastError();
}

ZT_EXPORT int zt_gemv_q5_0_f32(const void* W, const float* x, float* y, int M, int K, int qh_offset, int qs_offset,
                               hipStream_t stream) {
    return gemv_q5_0(W, x, y, M, K, qh_offset, qs_offset, stream);
}

ZT_EXPORT int zt_dequant_q4k_f32(const void* W, float* out, int rows, int K, hipStream_t stream) {
    return dequant_kq<4>(W, out, rows, K, stream);
}
ZT_EXPORT int zt_dequant_q5k_f32(const void* W, float* out, int rows, int K, hipStream_t stream) {
    return dequant_kq<5>(W, out, rows, K, stream);
}
ZT_EXPORT int zt_dequant_q6k_f32(const void* W, float* out, int rows, int K, hipStream_t stream) {
    return dequant_kq<6>(W, out, rows, K, stream);
}
ZT_EXPORT int zt_dequant_q5_0_f32(const void* W, float* out, int rows, int K, hipStream_t stream) {
    if (rows < 0 || K < 0 || K % 32 != 0) return (int)hipErrorInvalidValue;
    if (rows == 0 || K == 0) return (int)hipSuccess;
    if (W == nullptr || out == nullptr) return (int)hipErrorInvalidValue;
    const long nblk = (long)rows * (K / 32);
    q5_0_dequant_kernel<<<ceil_div(nblk, 256), 256, 0, stream>>>(static_cast<const uint8_t*>(W), out, nblk);
    return (int)hipGetLastError();
}

// Device dequantizers for the byte formats of the reference's Dequantizer
// registry (tensor/quant_registry.go:10-73, 231-240): the bytes a
// registered Dequantize(src []byte, dst []float32) takes, decoded on the
// GPU into fp32, bit for bit with the reference.
//
//  * "Q4_0": Q4Storage.RawBytes, 18-byte blocks [fp16 d][16 bytes], byte j
//    = element j (low nibble) and j+16 (high), w = float32(q - 8) * d
//    (tensor/quantized.go:96-114).
//  * "AWQ_4": the registry's wire format (tensor/quantized_awq.go:242-305):
//    a 12-byte header (numElements, groupSize, nGroups, uint32 LE), nGroups
//    (fp16 scale, fp16 zero) pairs, then every group's packed words, 8
//    nibbles per little-endian uint32, each group starting on a fresh word;
//    groups run over the flat element index, across row boundaries;
//    w = (float32(q) - zero) * scale (tensor/quantized_awq.go:118-136).
//  * "FP8_E4M3" / "FP8_E5M2": a 4-byte LE fp32 scale, then one byte per
//    element; w = decode(byte) * scale (tensor/quant_registry.go:190-229).
//    The decoders follow tensor/fp8_storage.go:229-250, 304-331: E4M3 has no
//    NaN or infinity (exponent 15 is an ordinary binade), E5M2 maps
//    exponent 31 to +-inf and NaN.
//  * "IQ3_S": 110-byte super-blocks of 256 values [fp16 d][64 qs][8 qh]
//    [32 sign bytes][4 scale bytes] (tensor/iq3_storage.go:12-95): value
//    32 i + 8 j + 4 h + k of the block (sub-block i, group j, half h) takes
//    qs byte 8 i + 2 j + h, whose 2-bit field k gives the magnitude
//    1 + 2 field (the reference's grid, tensor/iq3_grid.go:15-27, is that
//    formula for both values of the qh bit, so qh does not enter), the
//    sub-block scale d * (1 + 2 sc) with sc the low / high nibble of scale
//    byte i / 2, and sign bit k + 4 h of sign byte 4 i + j.
//    w = (d * (1 + 2 sc)) * magnitude, negated when the sign bit is set;
//    both products are exact in fp32.
//  * "W8A8": the 36-byte [fp32 scale][32 int8] groups of Q8_0, with the same
//    w = float32(q) * scale (tensor/quantized_w8a8.go:92-103, 285-316), so it
//    runs zt_dequant_q8_f32.
// "Q8_0", "Q4_K", "Q5_K", "Q6_K" and "Q5_0" are the raw blocks that
// zt_dequant_q8_f32, zt_dequant_q4k/q5k/q6k_f32 and zt_dequant_q5_0_f32
// already take.
//
// One thread per output element (Q4_0: per block; AWQ_4: per packed word),
// one fp32 rounding per element in the reference's order.
#include "zt_common.h"

namespace zt {

__global__ void dequant_q4raw_kernel(const uint8_t* __restrict__ src, float* __restrict__ out, long nelem, long nblk) {
    const long b = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nblk) return;
    const uint8_t* blk = src + b * 18;
    const uint16_t* h = reinterpret_cast<const uint16_t*>(blk);
    const float d = h2f(h[0]);
    const long o = b * 32;
#pragma unroll
    for (int w = 0; w < 8; w++) {  // 16 data bytes as 8 aligned halves
        const uint32_t v = h[1 + w];
#pragma unroll
        for (int k = 0; k < 2; k++) {
            const int j = 2 * w + k;
            const uint32_t byte = (v >> (8 * k)) & 0xffu;
            const float lo = (float)((int)(byte & 0xfu) - 8), hi = (float)((int)(byte >> 4) - 8);
            if (o + j < nelem) out[o + j] = lo * d;
            if (o + j + 16 < nelem) out[o + j + 16] = hi * d;
        }
    }
}

// One thread per packed word: word t of the data region is word w of group
// gi = t / wpg (wpg = ceil(group / 8) words a full group), elements
// gi * group + 8w .. +7 of the flat index.
__global__ void dequant_awq4_kernel(const uint8_t* __restrict__ wire, float* __restrict__ out, long nelem, int group,
                                    int ngroups, long nwords) {
    const long t = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= nwords) return;
    const int wpg = (group + 7) / 8;
    const long gi = t / wpg;
    const int w = (int)(t % wpg);
    const uint16_t* sz = reinterpret_cast<const uint16_t*>(wire + 12 + 4 * gi);
    const float scale = h2f(sz[0]), zero = h2f(sz[1]);
    const uint32_t word = reinterpret_cast<const uint32_t*>(wire + 12 + 4L * ngroups)[t];
    const long g0 = gi * group;
    const long gend = g0 + group < nelem ? g0 + group : nelem;
#pragma unroll
    for (int k = 0; k < 8; k++) {
        const long e = g0 + 8L * w + k;
        if (8 * w + k < group && e < gend) out[e] = ((float)((word >> (4 * k)) & 0xfu) - zero) * scale;
    }
}

__device__ __forceinline__ float decode_e4m3(uint32_t b) {
    const uint32_t sign = (b >> 7) & 1u, exp = (b >> 3) & 0xfu, mant = b & 7u;
    if (exp == 0) {  // zero and subnormals: mant/8 * 2^-6, exact
        const float v = (float)mant * 0.125f * 0.015625f;
        return sign ? -v : v;
    }
    return __uint_as_float((sign << 31) | ((exp + 120u) << 23) | (mant << 20));
}

__device__ __forceinline__ float decode_e5m2(uint32_t b) {
    const uint32_t sign = (b >> 7) & 1u, exp = (b >> 2) & 0x1fu, mant = b & 3u;
    if (exp == 0) {  // zero and subnormals: mant/4 * 2^-14, exact
        const float v = (float)mant * 0.25f * 6.103515625e-05f;
        return sign ? -v : v;
    }
    if (exp == 31) return mant == 0 ? __uint_as_float((sign << 31) | 0x7f800000u) : __uint_as_float(0x7fc00000u);
    return __uint_as_float((sign << 31) | ((exp + 112u) << 23) | (mant << 21));
}

template <bool E5M2>
__global__ void dequant_fp8_kernel(const uint8_t* __restrict__ wire, float* __restrict__ out, long nelem) {
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nelem) return;
    const float scale = *reinterpret_cast<const float*>(wire);
    const uint32_t b = wire[4 + i];
    out[i] = (E5M2 ? decode_e5m2(b) : decode_e4m3(b)) * scale;
}

// One thread per output element of the IQ3_S super-blocks.
__global__ void dequant_iq3s_kernel(const uint8_t* __restrict__ src, float* __restrict__ out, long nelem) {
    const long e = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= nelem) return;
    const uint8_t* blk = src + (e >> 8) * 110;
    const int v = (int)(e & 255), i = v >> 5, j = (v >> 3) & 3, h = (v >> 2) & 1, k = v & 3;
    const float d = h2f((uint16_t)(blk[0] | (blk[1] << 8)));
    const uint32_t sb = blk[106 + (i >> 1)];
    const uint32_t sc = (i & 1) ? (sb >> 4) : (sb & 15u);
    const float sub = d * (float)(1 + 2 * (int)sc);
    const uint32_t q = blk[2 + 8 * i + 2 * j + h];
    const float mag = (float)(1 + 2 * (int)((q >> (2 * k)) & 3u));
    const float w = sub * mag;
    out[e] = ((blk[74 + 4 * i + j] >> (k + 4 * h)) & 1u) ? -w : w;
}

}  // namespace zt

using namespace zt;

ZT_EXPORT int zt_dequant_q4raw_f32(const void* src, long src_bytes, float* out, long nelem, hipStream_t stream) {
    if (nelem < 0 || src_bytes < 0) return (int)hipErrorInvalidValue;
    if (nelem == 0) return (int)hipSuccess;
    const long nblk = (nelem + 31) / 32;
    if (src == nullptr || out == nullptr || src_bytes < nblk * 18 || ((uintptr_t)src & 1))
        return (int)hipErrorInvalidValue;
    dequant_q4raw_kernel<<<ceil_div(nblk, 256), 256, 0, stream>>>(static_cast<const uint8_t*>(src), out, nelem, nblk);
    return (int)hipGetLastError();
}

ZT_EXPORT int zt_dequant_awq4_f32(const void* wire, long wire_bytes, float* out, long nelem, int group_size,
                                  int ngroups, hipStream_t stream) {
    if (nelem < 0 || wire_bytes < 0) return (int)hipErrorInvalidValue;
    if (nelem == 0) return (int)hipSuccess;
    if (wire == nullptr || out == nullptr || group_size <= 0 || ((uintptr_t)wire & 3)) return (int)hipErrorInvalidValue;
    if ((long)ngroups != (nelem + group_size - 1) / group_size) return (int)hipErrorInvalidValue;
    const long wpg = (group_size + 7) / 8;
    const long last = nelem - (long)(ngroups - 1) * group_size;  // elements of the last group
    const long nwords = (long)(ngroups - 1) * wpg + (last + 7) / 8;
    if (wire_bytes < 12 + 4L * ngroups + 4 * nwords) return (int)hipErrorInvalidValue;
    dequant_awq4_kernel<<<ceil_div(nwords, 256), 256, 0, stream>>>(static_cast<const uint8_t*>(wire), out, nelem,
                                                                   group_size, ngroups, nwords);
    return (int)hipGetLastError();
}

ZT_EXPORT int zt_dequant_fp8_f32(const void* wire, long wire_bytes, float* out, long nelem, int e5m2,
                                 hipStream_t stream) {
    if (nelem < 0 || wire_bytes < 0 || (e5m2 != 0 && e5m2 != 1)) return (int)hipErrorInvalidValue;
    if (nelem == 0) return (int)hipSuccess;
    if (wire == nullptr || out == nullptr || wire_bytes < 4 + nelem || ((uintptr_t)wire & 3))
        return (int)hipErrorInvalidValue;
    const uint8_t* w = static_cast<const uint8_t*>(wire);
    if (e5m2)
        dequant_fp8_kernel<true><<<ceil_div(nelem, 256), 256, 0, stream>>>(w, out, nelem);
    else
        dequant_fp8_kernel<false><<<ceil_div(nelem, 256), 256, 0, stream>>>(w, out, nelem);
    return (int)hipGetLastError();
}

ZT_EXPORT int zt_dequant_iq3s_f32(const void* src, long src_bytes, float* out, long nelem, hipStream_t stream) {
    if (nelem < 0 || src_bytes < 0) return (int)hipErrorInvalidValue;
    if (nelem == 0) return (int)hipSuccess;
    const long nblk = (nelem + 255) / 256;
    if (src == nullptr || out == nullptr || src_bytes < nblk * 110) return (int)hipErrorInvalidValue;
    dequant_iq3s_kernel<<<ceil_div(nelem, 256), 256, 0, stream>>>(static_cast<const uint8_t*>(src), out, nelem);
    return (int)hipGetLastError();
}

// Host-side (CPU) half of libzt_hip.so: load-time layout conversions that
// turn the reference's serialised weight formats into the device layouts the
// kernels read.  They run once per weight at upload, like
// Q4Storage.RawBytesGPU (tensor/quantized.go:158-187) does for the CUDA
// engine, so no conversion happens inside a matmul call.
#include <string.h>

#include "zt_hip.h"

extern "C" {

int zt_abi_version(void) { return 102; }

// The header checks of the registry's AWQ_4 Dequantize
// (tensor/quantized_awq.go:245-297) and NewAWQStorageFromRaw's group count
// (:187-199), on the host copy of the wire bytes.
int zt_awq4_wire_header(const void* wire, long wire_bytes, long nelem, int* group_size, int* ngroups) {
    if (nelem < 0 || wire_bytes < 0 || group_size == nullptr || ngroups == nullptr) return 1;
    *group_size = 0;
    *ngroups = 0;
    if (nelem == 0) return 0;  // nothing to decode, the header is not read
    if (wire == nullptr || wire_bytes < 12) return 1;
    const unsigned char* b = static_cast<const unsigned char*>(wire);
    auto u32 = [b](int o) {
        return (unsigned long)b[o] | ((unsigned long)b[o + 1] << 8) | ((unsigned long)b[o + 2] << 16) |
               ((unsigned long)b[o + 3] << 24);
    };
    const long n = (long)u32(0), g = (long)(int)u32(4), ng = (long)(int)u32(8);
    if (n != nelem || g <= 0 || ng <= 0) return 1;
    if (ng != (n + g - 1) / g) return 1;
    if (wire_bytes < 12 + 4 * ng) return 1;
    const long last = n - (ng - 1) * g;
    const long words = (ng - 1) * ((g + 7) / 8) + (last + 7) / 8;
    if (wire_bytes - 12 - 4 * ng < 4 * words) return 1;
    *group_size = (int)g;
    *ngroups = (int)ng;
    return 0;
}

long zt_q4_gpu_data_offset(long nblk) { return (nblk * 2 + 15) & ~15L; }

long zt_q4_gpu_bytes(long nblk) { return zt_q4_gpu_data_offset(nblk) + nblk * 16; }

// tensor/quantized.go:168-187: scales first (LE fp16), zero padding to a
// 16-byte boundary, then every block's 16 nibble bytes.
void zt_q4_raw_to_gpu(const void* raw, long nblk, void* out) {
    const unsigned char* src = static_cast<const unsigned char*>(raw);
    unsigned char* dst = static_cast<unsigned char*>(out);
    const long doff = zt_q4_gpu_data_offset(nblk);
    memset(dst + nblk * 2, 0, (size_t)(doff - nblk * 2));
    for (long i = 0; i < nblk; i++) {
        dst[2 * i] = src[18 * i];
        dst[2 * i + 1] = src[18 * i + 1];
        memcpy(dst + doff + 16 * i, src + 18 * i + 2, 16);
    }
}

// IQ4_NL blocks have the same 18-byte shape (tensor/iq4_storage.go:12-23).
void zt_iq4nl_raw_to_gpu(const void* raw, long nblk, void* out) { zt_q4_raw_to_gpu(raw, nblk, out); }

// 36-byte Q8_0 blocks (tensor/quantized.go:425-438) -> [fp32 scales][pad][32-byte payloads].
void zt_q8_raw_to_gpu(const void* raw, long nblk, void* out) {
    const unsigned char* src = static_cast<const unsigned char*>(raw);
    unsigned char* dst = static_cast<unsigned char*>(out);
    const long doff = zt_q8_gpu_data_offset(nblk);
    memset(dst + nblk * 4, 0, (size_t)(doff - nblk * 4));
    for (long i = 0; i < nblk; i++) {
        memcpy(dst + 4 * i, src + 36 * i, 4);
        memcpy(dst + doff + 32 * i, src + 36 * i + 4, 32);
    }
}

// compute/ternary_gemv_gpu.go:55-67: element (i, j) of the flat 2-bit
// packing (bit offset 2*(i*K+j)) moves to byte i*ceil(K/4) + j/4, bits
// 2*(j%4); the pad bits of each row stay zero.
void zt_ternary_repack_rows(const void* raw, long M, long K, void* out) {
    const unsigned char* src = static_cast<const unsigned char*>(raw);
    unsigned char* dst = static_cast<unsigned char*>(out);
    const long bpr = (K + 3) / 4;
    memset(dst, 0, (size_t)(M * bpr));
    if (K % 4 == 0) {  // rows are already byte-aligned: a plain copy
        memcpy(dst, src, (size_t)(M * bpr));
        return;
    }
    for (long i = 0; i < M; i++)
        for (long j = 0; j < K; j++) {
            const long s = i * K + j;
            const unsigned bits = (src[s / 4] >> (2 * (s % 4))) & 3u;
            dst[i * bpr + j / 4] |= (unsigned char)(bits << (2 * (j % 4)));
        }
}

// tensor/quantized_q5_0.go:118-165 RawBytesGPU and its offsets: fp16 scales,
// zero padding to 16, the uint32 qh words, padding to 16, then every
// block's 16 nibble bytes.
long zt_q5_0_gpu_qh_offset(long nblk) { return (nblk * 2 + 15) & ~15L; }
long zt_q5_0_gpu_qs_offset(long nblk) { return zt_q5_0_gpu_qh_offset(nblk) + ((nblk * 4 + 15) & ~15L); }
long zt_q5_0_gpu_bytes(long nblk) { return zt_q5_0_gpu_qs_offset(nblk) + nblk * 16; }

void zt_q5_0_raw_to_gpu(const void* raw, long nblk, void* out) {
    const unsigned char* src = static_cast<const unsigned char*>(raw);
    unsigned char* dst = static_cast<unsigned char*>(out);
    const long qh = zt_q5_0_gpu_qh_offset(nblk), qs = zt_q5_0_gpu_qs_offset(nblk);
    memset(dst, 0, (size_t)qs);
    for (long i = 0; i < nblk; i++) {
        memcpy(dst + 2 * i, src + 22 * i, 2);
        memcpy(dst + qh + 4 * i, src + 22 * i + 2, 4);
        memcpy(dst + qs + 16 * i, src + 22 * i + 6, 16);
    }
}

// GGUF Q8_0 (34-byte blocks [fp16 d][32 x int8], tensor/mmap_storage.go:94-96,
// 265-284) -> [fp16 scales, nblk*2][pad to 16][int8 payloads, nblk*32]: every
// payload lands 16-byte aligned and the fp16 scales keep 34 bytes per block.
long zt_q8gguf_gpu_data_offset(long nblk) { return (nblk * 2 + 15) & ~15L; }
long zt_q8gguf_gpu_bytes(long nblk) { return zt_q8gguf_gpu_data_offset(nblk) + nblk * 32; }

void zt_q8gguf_raw_to_gpu(const void* raw, long nblk, void* out) {
    const unsigned char* src = static_cast<const unsigned char*>(raw);
    unsigned char* dst = static_cast<unsigned char*>(out);
    const long doff = zt_q8gguf_gpu_data_offset(nblk);
    memset(dst + nblk * 2, 0, (size_t)(doff - nblk * 2));
    for (long i = 0; i < nblk; i++) {
        memcpy(dst + 2 * i, src + 34 * i, 2);
        memcpy(dst + doff + 32 * i, src + 34 * i + 2, 32);
    }
}

}  // extern "C"

/*
 * zt_oracle.c -- CPU restatement of zerfoo/ztensor's quantized-weight
 * dequantizers and CPU GEMV/GEMM loops (the decode matmul path).
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the parity checker and the
 * CPU baseline of bench.py; it is never linked into, loaded by or called
 * from the product library (libzt_hip.so) or the ztensor_amd package.
 *
 * Every function follows one reference function; the citation is given as
 * path:line relative to the reference repository root.  Loop order, the
 * position of each rounding and the skip conditions are kept as the
 * reference has them, so results are bit-identical to the reference where
 * the reference's arithmetic is deterministic.  The file is compiled with
 * -ffp-contract=off because the reference is Go on amd64 (GOAMD64=v1), which
 * does not fuse x*y+z into an FMA in the scalar loops, while its AVX2 axpy
 * (gemm_simd_amd64.s) does use VFMADD231PS; orc_sgemm_simd reproduces that
 * by calling fmaf explicitly on the vector part and mul-then-add on the
 * scalar tail.
 *
 * Pinning (what checks each function besides restating it) is documented in
 * tests/test_oracle.py next to each test.
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define EXPORT __attribute__((visibility("default")))

/* ------------------------------------------------------------------ fp16 */

/* IEEE binary16 -> binary32 widening (exact).  Stands for
 * github.com/zerfoo/float16 v0.2.0 Float16.ToFloat32, which the reference
 * calls at tensor/quantized.go:99, tensor/iq4_storage.go:37,
 * tensor/quantized_gptq.go:136-137, tensor/fp16_storage.go:60. */
EXPORT float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t exp = (h >> 10) & 0x1f;
    uint32_t frac = h & 0x3ff;
    uint32_t bits;
    if (exp == 0) {
        if (frac == 0) {
            bits = sign;
        } else { /* subnormal: normalise */
            int e = -1;
            do { frac <<= 1; e++; } while ((frac & 0x400) == 0);
            frac &= 0x3ff;
            bits = sign | ((uint32_t)(127 - 15 - e) << 23) | (frac << 13);
        }
    } else if (exp == 31) {
        bits = sign | 0x7f800000u | (frac << 13);
    } else {
        bits = sign | ((exp - 15 + 127) << 23) | (frac << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* internal/xblas/q4dot.go:53-78 float16BitsToFloat32: same as IEEE for
 * finite values, but Inf/NaN map to 0 and subnormals are computed as
 * (frac/1024) * 2^-14 in two fp32 steps. */
EXPORT float orc_f16_bits_to_f32_xblas(uint16_t bits) {
    uint32_t sign = (bits >> 15) & 1;
    uint32_t exp = (bits >> 10) & 0x1f;
    uint32_t frac = bits & 0x3ff;
    if (exp == 0) {
        if (frac == 0) return 0.0f;
        float f = (float)frac / 1024.0f;
        f *= 1.0f / 16384.0f;
        return sign ? -f : f;
    }
    if (exp == 31) return 0.0f;
    uint32_t b32 = (sign << 31) | ((exp - 15 + 127) << 23) | (frac << 13);
    float f;
    memcpy(&f, &b32, 4);
    return f;
}

static inline uint16_t rd16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static inline uint32_t rd32(const uint8_t* p) {
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}

/* ------------------------------------------------------------------ Q4_0 */

/* tensor/quantized.go:96-114 Q4Storage.Dequantize over the RawBytes layout
 * (tensor/quantized.go:148-156): 18-byte blocks, fp16 scale LE then 16
 * bytes; low nibble -> element j, high nibble -> element j+16. */
EXPORT void orc_q4_dequant(const uint8_t* raw, int64_t nelem, float* dst) {
    int64_t nblk = (nelem + 31) / 32;
    for (int64_t bi = 0; bi < nblk; bi++) {
        const uint8_t* b = raw + bi * 18;
        float scale = orc_f16_to_f32(rd16(b));
        int64_t off = bi * 32;
        for (int j = 0; j < 16; j++) {
            uint8_t packed = b[2 + j];
            int q0 = (int)(packed & 0x0f) - 8;
            int q1 = (int)(packed >> 4) - 8;
            if (off + j < nelem) dst[off + j] = (float)q0 * scale;
            if (off + j + 16 < nelem) dst[off + j + 16] = (float)q1 * scale;
        }
    }
}

/* tensor/quantized.go:195-198 Q4GPUDataOffset. */
EXPORT int64_t orc_q4_gpu_data_offset(int64_t nblk) { return (nblk * 2 + 15) & ~(int64_t)15; }

/* tensor/quantized.go:168-187 RawBytesGPU: [scales nblk*2][pad to 16][data nblk*16]. */
EXPORT void orc_q4_raw_to_gpu(const uint8_t* raw, int64_t nblk, uint8_t* out) {
    int64_t doff = orc_q4_gpu_data_offset(nblk);
    memset(out, 0, (size_t)doff);
    for (int64_t i = 0; i < nblk; i++) {
        out[i * 2] = raw[i * 18];
        out[i * 2 + 1] = raw[i * 18 + 1];
        memcpy(out + doff + i * 16, raw + i * 18 + 2, 16);
    }
}

/* internal/xblas/q4dot.go:10-31 q4DotBlockScalar. */
EXPORT float orc_q4_dot_block(const uint8_t* packed, float scale, const float* x, int n) {
    if (n > 32) n = 32;
    float sum = 0.0f;
    for (int p = 0; p < 16; p++) {
        if (p >= n) break;
        uint8_t bv = packed[p];
        float lo = (float)((int)(bv & 0x0f) - 8);
        float hi = (float)((int)(bv >> 4) - 8);
        sum += lo * x[p];
        if (p + 16 < n) sum += hi * x[p + 16];
    }
    return sum * scale;
}

/* internal/xblas/q4dot.go:36-50 q4DotRowScalar (the amd64 q4DotRow,
 * internal/xblas/q4dot_generic.go:13-15). */
EXPORT float orc_q4_dot_row(const uint8_t* blocks, const float* x, int nblocks) {
    float total = 0.0f;
    for (int bi = 0; bi < nblocks; bi++) {
        const uint8_t* b = blocks + (int64_t)bi * 18;
        float scale = orc_f16_bits_to_f32_xblas(rd16(b));
        total += orc_q4_dot_block(b + 2, scale, x + (int64_t)bi * 32, 32);
    }
    return total;
}

/* ------------------------------------------------------- threading helper */

typedef void (*orc_range_fn)(void* ctx, int64_t j0, int64_t j1);
typedef struct { orc_range_fn fn; void* ctx; int64_t j0, j1; } orc_task;
static void* orc_task_run(void* p) {
    orc_task* t = (orc_task*)p;
    t->fn(t->ctx, t->j0, t->j1);
    return NULL;
}
/* Splits [0,n) into nthreads chunks of ceil(n/nthreads), the split of
 * gemmF32Q4NTParallel (internal/xblas/gemm_quant.go:122-157). */
static void orc_parallel_rows(int64_t n, int nthreads, orc_range_fn fn, void* ctx) {
    if (nthreads <= 1) { fn(ctx, 0, n); return; }
    int64_t chunk = (n + nthreads - 1) / nthreads;
    pthread_t th[256];
    orc_task tk[256];
    int nt = 0;
    for (int t = 0; t < nthreads && t < 256; t++) {
        int64_t j0 = (int64_t)t * chunk, j1 = j0 + chunk < n ? j0 + chunk : n;
        if (j0 >= n) break;
        tk[nt] = (orc_task){fn, ctx, j0, j1};
        pthread_create(&th[nt], NULL, orc_task_run, &tk[nt]);
        nt++;
    }
    for (int t = 0; t < nt; t++) pthread_join(th[t], NULL);
}

/* ----------------------------------------------------------- SgemmSimd */

/* internal/xblas/gemm_simd_amd64.s:8-75 sgemmAccRow: c[j] += a*b[j];
 * 16- then 8- then 4-wide VFMADD231PS blocks, scalar tail MULSS+ADDSS. */
static void orc_sgemm_acc_row(float* c, const float* b, float a, int64_t n) {
    int64_t j = 0;
    for (; j + 16 <= n; j += 16)
        for (int l = 0; l < 16; l++) c[j + l] = fmaf(a, b[j + l], c[j + l]);
    if (j + 8 <= n) { for (int l = 0; l < 8; l++) c[j + l] = fmaf(a, b[j + l], c[j + l]); j += 8; }
    if (j + 4 <= n) { for (int l = 0; l < 4; l++) c[j + l] = fmaf(a, b[j + l], c[j + l]); j += 4; }
    for (; j < n; j++) { float t = b[j] * a; c[j] = t + c[j]; }
}

/* internal/xblas/gemm_simd_amd64.go:19-37 SgemmSimd: C += A*B, K tiled by
 * 256, zero elements of A skipped.  The caller zeroes C (xblas.GemmF32 is
 * called on a fresh result tensor, compute/cpu_engine.go:1219-1237). */
EXPORT void orc_sgemm_simd(int64_t m, int64_t n, int64_t k, const float* a, const float* b, float* c) {
    if (m == 0 || n == 0 || k == 0) return;
    for (int64_t p0 = 0; p0 < k; p0 += 256) {
        int64_t p1 = p0 + 256 < k ? p0 + 256 : k;
        for (int64_t i = 0; i < m; i++) {
            float* crow = c + i * n;
            for (int64_t p = p0; p < p1; p++) {
                float av = a[i * k + p];
                if (av != 0.0f) orc_sgemm_acc_row(crow, b + p * n, av, n);
            }
        }
    }
}

/* ------------------------------------------------------ GemmF32Q4NT */

typedef struct { const float* a; const uint8_t* raw; float* c; int bpr; } q4nt_ctx;
static void q4nt_range(void* p, int64_t j0, int64_t j1) {
    q4nt_ctx* t = (q4nt_ctx*)p;
    for (int64_t j = j0; j < j1; j++)
        t->c[j] = orc_q4_dot_row(t->raw + j * t->bpr * 18, t->a, t->bpr);
}

/* internal/xblas/gemm_quant.go:81-157 GemmF32Q4NT: C[M,N] = A[M,K] * B^T,
 * B = Q4_0 [N,K] in RawBytes layout.  K%32 must be 0 (the reference's
 * k%32!=0 branch dequantizes and calls SgemmSimd; callers here use
 * orc_q4_dequant + orc_sgemm_simd for that).  For M=1 and N*K>=65536 the
 * reference splits N over min(NumCPU, N/4) workers; nthreads stands for
 * NumCPU.  Each output is one q4DotRow, so the split does not change bits. */
EXPORT void orc_gemm_f32_q4_nt(int64_t m, int64_t n, int64_t k, const float* a, const uint8_t* raw,
                               float* c, int nthreads) {
    int bpr = (int)(k / 32);
    if (m == 1 && n * k >= 256 * 256) {
        int nc = nthreads;
        if (nc > n / 4) nc = (int)(n / 4);
        if (nc > 1) {
            q4nt_ctx ctx = {a, raw, c, bpr};
            orc_parallel_rows(n, nc, q4nt_range, &ctx);
            return;
        }
    }
    for (int64_t i = 0; i < m; i++)
        for (int64_t j = 0; j < n; j++)
            c[i * n + j] = orc_q4_dot_row(raw + j * bpr * 18, a + i * k, bpr);
}

/* ------------------------------------------------------------------ Q8_0 */

/* tensor/quantized.go:344-355 Q8Storage.Dequantize over the RawBytes layout
 * (tensor/quantized.go:427-438): 36-byte blocks, fp32 scale LE + 32 int8. */
EXPORT void orc_q8_dequant(const uint8_t* raw, int64_t nelem, float* dst) {
    int64_t nblk = (nelem + 31) / 32;
    for (int64_t bi = 0; bi < nblk; bi++) {
        const uint8_t* b = raw + bi * 36;
        uint32_t sb = rd32(b);
        float scale;
        memcpy(&scale, &sb, 4);
        for (int j = 0; j < 32; j++) {
            int64_t idx = bi * 32 + j;
            if (idx >= nelem) break;
            dst[idx] = (float)(int8_t)b[4 + j] * scale;
        }
    }
}

typedef struct { const float* a; const uint8_t* raw; float* c; int bpr; } q8nt_ctx;
/* One output of GemmF32Q8NT: DequantizeBlock (tensor/quantized.go:358-363)
 * into a 32-float buffer, then sum += a*buf in element order
 * (internal/xblas/gemm_quant.go:193-203). */
static float q8_dot_row(const uint8_t* row, const float* a, int bpr) {
    float buf[32];
    float sum = 0.0f;
    for (int bi = 0; bi < bpr; bi++) {
        const uint8_t* b = row + (int64_t)bi * 36;
        uint32_t sb = rd32(b);
        float scale;
        memcpy(&scale, &sb, 4);
        for (int j = 0; j < 32; j++) buf[j] = (float)(int8_t)b[4 + j] * scale;
        const float* ab = a + (int64_t)bi * 32;
        for (int p = 0; p < 32; p++) sum += ab[p] * buf[p];
    }
    return sum;
}
static void q8nt_range(void* p, int64_t j0, int64_t j1) {
    q8nt_ctx* t = (q8nt_ctx*)p;
    for (int64_t j = j0; j < j1; j++) t->c[j] = q8_dot_row(t->raw + j * t->bpr * 36, t->a, t->bpr);
}

/* internal/xblas/gemm_quant.go:163-264 GemmF32Q8NT (+ gemmF32Q8NTParallel). */
EXPORT void orc_gemm_f32_q8_nt(int64_t m, int64_t n, int64_t k, const float* a, const uint8_t* raw,
                               float* c, int nthreads) {
    int bpr = (int)(k / 32);
    if (m == 1 && n * k >= 256 * 256) {
        int nc = nthreads;
        if (nc > n / 4) nc = (int)(n / 4);
        if (nc > 1) {
            q8nt_ctx ctx = {a, raw, c, bpr};
            orc_parallel_rows(n, nc, q8nt_range, &ctx);
            return;
        }
    }
    for (int64_t i = 0; i < m; i++)
        for (int64_t j = 0; j < n; j++) c[i * n + j] = q8_dot_row(raw + j * bpr * 36, a + i * k, bpr);
}

/* --------------------------------------------------------------- IQ4_NL */

/* tensor/iq4_storage.go:28-33 IQ4NLTable. */
static const float orc_iq4nl_table[16] = {
    -1.0f, -0.6961928f, -0.5250730f, -0.3947555f, -0.2831612f, -0.1790887f, -0.0805542f, 0.0f,
    0.0805542f, 0.1790887f, 0.2831612f, 0.3947555f, 0.5250730f, 0.6961928f, 1.0f, 1.3312578f};

EXPORT void orc_iq4nl_table_copy(float* dst) { memcpy(dst, orc_iq4nl_table, sizeof orc_iq4nl_table); }

/* tensor/iq4_storage.go:36-46 DequantizeIQ4NL (one block: dst[2i] = d*T[lo],
 * dst[2i+1] = d*T[hi]) and :75-89 IQ4NLStorage.Dequantize (partial last
 * block copied through a temporary). */
EXPORT void orc_iq4nl_dequant(const uint8_t* raw, int64_t nelem, float* dst) {
    int64_t nblk = (nelem + 31) / 32;
    for (int64_t bi = 0; bi < nblk; bi++) {
        const uint8_t* b = raw + bi * 18;
        float d = orc_f16_to_f32(rd16(b));
        float tmp[32];
        for (int i = 0; i < 16; i++) {
            uint8_t lo = b[2 + i] & 0x0f, hi = b[2 + i] >> 4;
            tmp[2 * i] = d * orc_iq4nl_table[lo];
            tmp[2 * i + 1] = d * orc_iq4nl_table[hi];
        }
        int64_t off = bi * 32, rem = nelem - off;
        memcpy(dst + off, tmp, sizeof(float) * (size_t)(rem >= 32 ? 32 : rem));
    }
}

/* ------------------------------------------------------------ GPTQ / AWQ */

/* tensor/quantized_gptq.go:134-163 GPTQStorage.Dequantize.  data is the
 * concatenation of every group's packed bytes (the layout that
 * NewGPTQStorageFromRaw, tensor/quantized_gptq.go:217-277, accepts); for
 * bits=4 element j of a group is the low nibble of byte j/2 when j is even
 * and the high nibble when odd. */
EXPORT void orc_gptq_dequant(const uint8_t* data, const uint16_t* scales, const uint16_t* zeros,
                             int64_t nelem, int64_t group, int bits, float* dst) {
    int64_t ngroups = (nelem + group - 1) / group;
    const uint8_t* g = data;
    for (int64_t gi = 0; gi < ngroups; gi++) {
        float scale = orc_f16_to_f32(scales[gi]);
        float zero = orc_f16_to_f32(zeros[gi]);
        int64_t off = gi * group, end = off + group < nelem ? off + group : nelem;
        int64_t count = end - off;
        if (bits == 4) {
            for (int64_t j = 0; j < count; j++) {
                int q = (j % 2 == 0) ? (g[j / 2] & 0x0f) : (g[j / 2] >> 4);
                dst[off + j] = ((float)q - zero) * scale;
            }
            g += (count + 1) / 2;
        } else {
            for (int64_t j = 0; j < count; j++) dst[off + j] = ((float)g[j] - zero) * scale;
            g += count;
        }
    }
}

/* tensor/quantized_awq.go:118-136 AWQStorage.Dequantize: 8 nibbles per
 * little-endian uint32, element j of a group at bits 4*(j%8) of word j/8. */
EXPORT void orc_awq_dequant(const uint32_t* words, const uint16_t* scales, const uint16_t* zeros,
                            int64_t nelem, int64_t group, float* dst) {
    int64_t ngroups = (nelem + group - 1) / group;
    const uint32_t* w = words;
    for (int64_t gi = 0; gi < ngroups; gi++) {
        float scale = orc_f16_to_f32(scales[gi]);
        float zero = orc_f16_to_f32(zeros[gi]);
        int64_t off = gi * group, end = off + group < nelem ? off + group : nelem;
        int64_t count = end - off;
        for (int64_t j = 0; j < count; j++) {
            int q = (int)((w[j / 8] >> ((j % 8) * 4)) & 0xf);
            dst[off + j] = ((float)q - zero) * scale;
        }
        w += (count + 7) / 8;
    }
}

/* tensor/quantized_awq.go:245-305 awqDequantizer.Dequantize (the registry's
 * "AWQ_4" wire format) with NewAWQStorageFromRaw's checks (:187-214):
 * header numElements, groupSize, nGroups (uint32 LE), nGroups (fp16 scale,
 * fp16 zero) pairs, then every group's packed words, each group starting on
 * a fresh word.  Returns 0, or 1 for short data, 2 for a numElements
 * mismatch, 3 for a bad groupSize / nGroups or a group count other than
 * ceil(n / groupSize).  n == 0 returns 0 without reading src. */
EXPORT int orc_awq4_wire_dequant(const uint8_t* src, int64_t src_len, float* dst, int64_t n) {
    if (n == 0) return 0;
    if (src_len < 12) return 1;
    uint32_t hdr[3];
    memcpy(hdr, src, 12);
    const int64_t num = (int64_t)hdr[0], group = (int64_t)(int32_t)hdr[1], ngroups = (int64_t)(int32_t)hdr[2];
    if (num != n) return 2;
    if (group <= 0 || ngroups <= 0) return 3;
    const int64_t meta = 12 + ngroups * 4;
    if (src_len < meta) return 1;
    int64_t total = 0;
    for (int64_t gi = 0; gi < ngroups; gi++) {
        int64_t count = group, remaining = num - gi * group;
        if (remaining < group) count = remaining;
        total += (count + 7) / 8;
    }
    if (src_len - meta < total * 4) return 1;
    if (ngroups != (num + group - 1) / group) return 3;
    uint16_t* scales = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)ngroups);
    uint16_t* zeros = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)ngroups);
    uint32_t* words = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)(total > 0 ? total : 1));
    for (int64_t gi = 0; gi < ngroups; gi++) {
        memcpy(&scales[gi], src + 12 + gi * 4, 2);
        memcpy(&zeros[gi], src + 12 + gi * 4 + 2, 2);
    }
    memcpy(words, src + meta, (size_t)total * 4);
    orc_awq_dequant(words, scales, zeros, num, group, dst);
    free(scales);
    free(zeros);
    free(words);
    return 0;
}

/* tensor/fp8_storage.go:229-250 decodeE4M3 (no NaN or infinity: exponent 15
 * is an ordinary binade) and :304-331 decodeE5M2, then the registry's
 * "FP8_E4M3" / "FP8_E5M2" Dequantize (tensor/quant_registry.go:190-229):
 * src = 4-byte LE fp32 scale, then one byte per element;
 * dst[i] = decode(src[4+i]) * scale.  Returns 1 for short data. */
static float orc_decode_e4m3(uint8_t b) {
    uint32_t sign = (b >> 7) & 1u, exp = (b >> 3) & 0xfu, mant = b & 7u;
    if (exp == 0 && mant == 0) return sign ? -0.0f : 0.0f;
    if (exp == 0) {
        float v = (float)mant / 8.0f * (float)pow(2.0, 1 - 7);
        return sign ? -v : v;
    }
    uint32_t bits = (sign << 31) | ((exp - 7 + 127) << 23) | (mant << 20);
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

static float orc_decode_e5m2(uint8_t b) {
    uint32_t sign = (b >> 7) & 1u, exp = (b >> 2) & 0x1fu, mant = b & 3u;
    if (exp == 0 && mant == 0) return sign ? -0.0f : 0.0f;
    if (exp == 31) {
        if (mant == 0) return sign ? -INFINITY : INFINITY;
        return NAN;
    }
    if (exp == 0) {
        float v = (float)mant / 4.0f * (float)pow(2.0, 1 - 15);
        return sign ? -v : v;
    }
    uint32_t bits = (sign << 31) | ((exp - 15 + 127) << 23) | (mant << 21);
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

EXPORT int orc_fp8_dequant(const uint8_t* src, int64_t src_len, float* dst, int64_t n, int e5m2) {
    if (src_len < 4 + n) return 1;
    float scale;
    memcpy(&scale, src, 4);
    for (int64_t i = 0; i < n; i++) dst[i] = (e5m2 ? orc_decode_e5m2(src[4 + i]) : orc_decode_e4m3(src[4 + i])) * scale;
    return 0;
}

/* tensor/iq3_storage.go:31-95 DequantizeIQ3S, one 110-byte super-block to
 * 256 values, in the reference's loop order: sub-block i (scale nibble of
 * byte 106 + i/2, multiplier d * (1 + 2 sc)), group j (qs bytes consumed in
 * pairs, one sign byte), grid entries from tensor/iq3_grid.go:17-27 (2-bit
 * field k of the 8 low index bits -> 1 + 2 field; the 9th bit, from qh,
 * selects an identical half of the table). */
static const uint8_t* orc_iq3s_grid(void) {
    static uint8_t grid[512][4];
    static int init = 0;
    if (!init) {
        for (int i = 0; i < 256; i++)
            for (int k = 0; k < 4; k++) grid[i][k] = grid[256 + i][k] = (uint8_t)(1 + 2 * ((i >> (2 * k)) & 3));
        init = 1;
    }
    return &grid[0][0];
}

static void orc_iq3s_block(const uint8_t* raw, float* dst) {
    const uint8_t* grid = orc_iq3s_grid();
    const float d = orc_f16_to_f32(rd16(raw));
    const uint8_t *qs = raw + 2, *qh = raw + 66, *signs = raw + 74, *scales = raw + 106;
    int qsi = 0, sgi = 0;
    for (int i = 0; i < 8; i++) {
        const uint8_t sc = (i % 2 == 0) ? (scales[i / 2] & 0x0F) : (scales[i / 2] >> 4);
        const float sub = d * (float)(1 + 2 * (int)sc);
        const uint8_t qhb = qh[i];
        for (int j = 0; j < 4; j++) {
            const int g1 = qs[qsi] | (((qhb >> (2 * j)) & 1) << 8);
            qsi++;
            const uint8_t sb = signs[sgi];
            sgi++;
            for (int k = 0; k < 4; k++) {
                float v = sub * (float)grid[4 * g1 + k];
                if (sb & (1 << k)) v = -v;
                dst[i * 32 + j * 8 + k] = v;
            }
            const int g2 = qs[qsi] | (((qhb >> (2 * j + 1)) & 1) << 8);
            qsi++;
            for (int k = 0; k < 4; k++) {
                float v = sub * (float)grid[4 * g2 + k];
                if (sb & (1 << (k + 4))) v = -v;
                dst[i * 32 + j * 8 + 4 + k] = v;
            }
        }
    }
}

/* IQ3SStorage.Dequantize (tensor/iq3_storage.go:113-128) behind the
 * registry's Dequantize (:169-179): status 1 when NewIQ3SStorageFromRaw
 * rejects the input (n <= 0, fewer than ceil(n/256) * 110 bytes); a partial
 * last block is decoded whole and its first values kept. */
EXPORT int orc_iq3s_dequant(const uint8_t* src, int64_t src_len, float* dst, int64_t n) {
    if (n <= 0) return 1;
    const int64_t nb = (n + 255) / 256;
    if (src_len < nb * 110) return 1;
    float tmp[256];
    for (int64_t b = 0; b < nb; b++) {
        orc_iq3s_block(src + b * 110, tmp);
        const int64_t rem = n - b * 256 < 256 ? n - b * 256 : 256;
        memcpy(dst + b * 256, tmp, (size_t)rem * sizeof(float));
    }
    return 0;
}

/* ----------------------------------------- dequant + SgemmSimd matmuls */

/* tensor/fp16_storage.go:53-63 Float16Storage.Slice. */
EXPORT void orc_f16_slice(const uint16_t* h, int64_t n, float* dst) {
    for (int64_t i = 0; i < n; i++) dst[i] = orc_f16_to_f32(h[i]);
}

/* compute/w4a16.go:71-105 MatMulW4A16 with the weights on the A side:
 * w4.Slice() (GPTQ dequant), fp16Act.Slice(), then eng.MatMul on float32,
 * which is xblas.GemmF32 -> SgemmSimd (compute/cpu_engine.go:1219-1237,
 * internal/xblas/gemm.go:12-14) into a zeroed result.
 * W is [M,K] (groups along K), X is fp16 [K,N], C is fp32 [M,N].
 * wtmp must hold M*K floats and xtmp K*N floats (the reference allocates
 * both on every call; the caller passes them so timing can include or
 * exclude allocation). */
EXPORT void orc_w4a16_matmul_gptq(const uint8_t* data, const uint16_t* scales, const uint16_t* zeros,
                                  const uint16_t* x16, float* c, int64_t m, int64_t k, int64_t n,
                                  int64_t group, float* wtmp, float* xtmp) {
    orc_gptq_dequant(data, scales, zeros, m * k, group, 4, wtmp);
    orc_f16_slice(x16, k * n, xtmp);
    memset(c, 0, sizeof(float) * (size_t)(m * n));
    orc_sgemm_simd(m, n, k, wtmp, xtmp, c);
}

/* IQ4_NL has no quantized GEMV in the reference: CPUEngine.MatMul falls
 * through to Data() (tensor/tensor.go:216-219) -> IQ4NLStorage.Slice
 * (tensor/iq4_storage.go:95) -> GemmF32 -> SgemmSimd
 * (compute/cpu_engine.go:1215-1245).  Activations arrive as fp16 and are
 * widened first (tensor/fp16_storage.go:53-63).  W [M,K], X [K,N], C [M,N]. */
EXPORT void orc_iq4nl_matmul(const uint8_t* raw, const uint16_t* x16, float* c, int64_t m, int64_t k,
                             int64_t n, float* wtmp, float* xtmp) {
    orc_iq4nl_dequant(raw, m * k, wtmp);
    orc_f16_slice(x16, k * n, xtmp);
    memset(c, 0, sizeof(float) * (size_t)(m * n));
    orc_sgemm_simd(m, n, k, wtmp, xtmp, c);
}

/* --------------------------------------------------------------- Ternary */

/* tensor/ternary_storage.go:39-47 TernaryStorage.Get: 2 bits per value,
 * element i at bits 2*(i%4) of byte i/4, value = code - 1. */
EXPORT int orc_ternary_get(const uint8_t* raw, int64_t i) {
    return (int)((raw[i / 4] >> ((i % 4) * 2)) & 3) - 1;
}

/* compute/ternary_gemv.go:68-77 ternaryLUT. */
static float orc_ternary_lut[256][4];
static int orc_ternary_lut_ready = 0;
static void orc_ternary_lut_init(void) {
    if (orc_ternary_lut_ready) return;
    for (int b = 0; b < 256; b++)
        for (int k = 0; k < 4; k++) orc_ternary_lut[b][k] = (float)((int8_t)((b >> (k * 2)) & 3) - 1);
    orc_ternary_lut_ready = 1;
}

/* compute/ternary_gemv.go:12-64 TernaryGEMV: weights packed flat across rows
 * (element i*cols+j), fp32 x, sequential fp32 sum per row; byte-aligned rows
 * use the 4-entry LUT per byte, the rest per-element extraction. */
EXPORT void orc_ternary_gemv(const uint8_t* raw, const float* x, int64_t rows, int64_t cols, float* y) {
    orc_ternary_lut_init();
    for (int64_t i = 0; i < rows; i++) {
        float sum = 0.0f;
        int64_t base = i * cols, j = 0;
        int64_t byteStart = base / 4;
        if (base % 4 == 0) {
            int64_t fullBytes = cols / 4;
            for (int64_t bi = 0; bi < fullBytes; bi++) {
                const float* l = orc_ternary_lut[raw[byteStart + bi]];
                sum += l[0] * x[j];
                sum += l[1] * x[j + 1];
                sum += l[2] * x[j + 2];
                sum += l[3] * x[j + 3];
                j += 4;
            }
        }
        for (; j < cols; j++) {
            int64_t idx = base + j;
            int bits = (raw[idx / 4] >> ((idx % 4) * 2)) & 3;
            if (bits == 0) sum -= x[j];
            else if (bits == 2) sum += x[j];
        }
        y[i] = sum;
    }
}

/* compute/ternary_gemv_gpu.go:55-67: repack flat-packed ternary weights into
 * one byte-aligned row of ceil(cols/4) bytes per output row (the layout the
 * GPU kernel reads).  out must be zeroed and hold rows*ceil(cols/4) bytes. */
EXPORT void orc_ternary_repack_rows(const uint8_t* raw, int64_t rows, int64_t cols, uint8_t* out) {
    int64_t bpr = (cols + 3) / 4;
    for (int64_t i = 0; i < rows; i++)
        for (int64_t j = 0; j < cols; j++) {
            int64_t s = i * cols + j;
            uint8_t bits = (raw[s / 4] >> ((s % 4) * 2)) & 3;
            out[i * bpr + j / 4] |= (uint8_t)(bits << ((j % 4) * 2));
        }
}

/* BitNet-style int8-activation ternary GEMV (the decode configuration of
 * this path).  The reference has no int8 activation path: TernaryGEMV takes
 * fp32 x (compute/ternary_gemv.go:12) and TernaryStorage has no scale
 * (tensor/ternary_storage.go:7-10).  The reduction is therefore defined as
 *   y = TernaryGEMV(W, float(q_x)) * (w_scale * x_scale)
 * in fp32, with the scale product rounded first.  Every partial sum is an
 * integer of magnitude <= cols*127 < 2^24, so the fp32 sums are exact and
 * the result is independent of summation order. */
EXPORT void orc_ternary_gemv_i8(const uint8_t* raw, const int8_t* qx, float x_scale, float w_scale,
                                int64_t rows, int64_t cols, float* y, float* xtmp) {
    for (int64_t j = 0; j < cols; j++) xtmp[j] = (float)qx[j];
    orc_ternary_gemv(raw, xtmp, rows, cols, y);
    float s = w_scale * x_scale;
    for (int64_t i = 0; i < rows; i++) y[i] = y[i] * s;
}

/* ------------------------------------------------------------- K-quants */

/* tensor/quantized_kquant.go:34-51 decodeQ4KScalesMins: the 6-bit scales and
 * mins of the eight 32-value sub-blocks, packed in bytes 4..15 of a Q4_K or
 * Q5_K super-block (Q5_K reuses it, :513). */
EXPORT void orc_kq_scales_mins(const uint8_t* blk, uint8_t* scales, uint8_t* mins) {
    const uint8_t* sc = blk + 4;
    for (int i = 0; i < 4; i++) {
        scales[i] = sc[i] & 63;
        mins[i] = sc[4 + i] & 63;
    }
    for (int i = 0; i < 4; i++) {
        scales[4 + i] = (uint8_t)((sc[8 + i] & 0xF) | ((sc[i] >> 6) << 4));
        mins[4 + i] = (uint8_t)((sc[8 + i] >> 4) | ((sc[4 + i] >> 6) << 4));
    }
}

/* tensor/quantized_kquant.go:54-79 DequantizeQ4K: one 144-byte super-block
 * [fp16 d][fp16 dmin][12 bytes scales/mins][128 bytes nibbles] -> 256 values.
 * Group g (64 values) reads bytes 32g..32g+31: low nibble of byte l ->
 * value 64g+l (sub-block 2g), high nibble -> 64g+32+l (sub-block 2g+1);
 * value = (d*sc)*q - dmin*mn, each product and the difference rounded. */
static void q4k_block(const uint8_t* b, float* dst) {
    float d = orc_f16_to_f32(rd16(b)), dmin = orc_f16_to_f32(rd16(b + 2));
    uint8_t scales[8], mins[8];
    orc_kq_scales_mins(b, scales, mins);
    const uint8_t* q = b + 16;
    for (int g = 0; g < 4; g++) {
        float sc0 = d * (float)scales[2 * g], mn0 = dmin * (float)mins[2 * g];
        float sc1 = d * (float)scales[2 * g + 1], mn1 = dmin * (float)mins[2 * g + 1];
        for (int l = 0; l < 32; l++) {
            uint8_t v = q[32 * g + l];
            dst[64 * g + l] = sc0 * (float)(v & 0xF) - mn0;
            dst[64 * g + l + 32] = sc1 * (float)(v >> 4) - mn1;
        }
    }
}

/* Partial last super-block through a 256-value temporary, as every
 * K-quant Dequantize does (tensor/quantized_kquant.go:263-277, 412-426,
 * 579-593). */
typedef void (*orc_kq_block_fn)(const uint8_t*, float*);
static void kq_dequant(orc_kq_block_fn fn, int bytes, const uint8_t* raw, int64_t nelem, float* dst) {
    int64_t nblk = (nelem + 255) / 256;
    for (int64_t bi = 0; bi < nblk; bi++) {
        int64_t off = bi * 256, rem = nelem - off;
        if (rem >= 256) {
            fn(raw + bi * bytes, dst + off);
        } else {
            float tmp[256];
            fn(raw + bi * bytes, tmp);
            memcpy(dst + off, tmp, sizeof(float) * (size_t)rem);
        }
    }
}

/* tensor/quantized_kquant.go:263-277 Q4KStorage.Dequantize. */
EXPORT void orc_q4k_dequant(const uint8_t* raw, int64_t nelem, float* dst) { kq_dequant(q4k_block, 144, raw, nelem, dst); }

/* tensor/quantized_kquant.go:355-382 DequantizeQ6K: one 210-byte super-block
 * [128 ql][64 qh][16 int8 scales][fp16 d].  Half h (128 values) uses ql
 * bytes 64h.., qh bytes 32h.. and scales 8h..; for l < 32 (is = l/16):
 *   q1 = (ql[l] & 15 | (qh[l] & 3) << 4) - 32           -> value l,      scale is
 *   q2 = (ql[32+l] & 15 | (qh[l] >> 2 & 3) << 4) - 32   -> value 32+l,   scale is+2
 *   q3 = (ql[l] >> 4 | (qh[l] >> 4 & 3) << 4) - 32      -> value 64+l,   scale is+4
 *   q4 = (ql[32+l] >> 4 | (qh[l] >> 6 & 3) << 4) - 32   -> value 96+l,   scale is+6
 * value = (d * scale) * q, two roundings left to right. */
static void q6k_block(const uint8_t* b, float* dst) {
    const uint8_t* ql = b;
    const uint8_t* qh = b + 128;
    const int8_t* sc = (const int8_t*)(b + 192);
    float d = orc_f16_to_f32(rd16(b + 208));
    for (int h = 0; h < 2; h++) {
        const uint8_t* l0 = ql + 64 * h;
        const uint8_t* h0 = qh + 32 * h;
        const int8_t* s0 = sc + 8 * h;
        float* o = dst + 128 * h;
        for (int l = 0; l < 32; l++) {
            int is = l / 16;
            int q1 = (int)(int8_t)((l0[l] & 0xF) | ((h0[l] & 3) << 4)) - 32;
            int q2 = (int)(int8_t)((l0[32 + l] & 0xF) | (((h0[l] >> 2) & 3) << 4)) - 32;
            int q3 = (int)(int8_t)((l0[l] >> 4) | (((h0[l] >> 4) & 3) << 4)) - 32;
            int q4 = (int)(int8_t)((l0[32 + l] >> 4) | (((h0[l] >> 6) & 3) << 4)) - 32;
            o[l] = d * (float)s0[is + 0] * (float)q1;
            o[32 + l] = d * (float)s0[is + 2] * (float)q2;
            o[64 + l] = d * (float)s0[is + 4] * (float)q3;
            o[96 + l] = d * (float)s0[is + 6] * (float)q4;
        }
    }
}

/* tensor/quantized_kquant.go:412-426 Q6KStorage.Dequantize. */
EXPORT void orc_q6k_dequant(const uint8_t* raw, int64_t nelem, float* dst) { kq_dequant(q6k_block, 210, raw, nelem, dst); }

/* tensor/quantized_kquant.go:509-549 DequantizeQ5K: one 176-byte super-block
 * [fp16 d][fp16 dmin][12 bytes scales/mins][128 ql][32 qh].  As Q4_K, plus
 * a fifth bit: for group g, bit 2g of qh[l] adds 16 to the low-nibble value
 * 64g+l and bit 2g+1 adds 16 to the high-nibble value 64g+32+l. */
static void q5k_block(const uint8_t* b, float* dst) {
    float d = orc_f16_to_f32(rd16(b)), dmin = orc_f16_to_f32(rd16(b + 2));
    uint8_t scales[8], mins[8];
    orc_kq_scales_mins(b, scales, mins);
    const uint8_t* ql = b + 16;
    const uint8_t* qh = b + 144;
    uint8_t u1 = 1, u2 = 2;
    for (int g = 0; g < 4; g++) {
        float sc0 = d * (float)scales[2 * g], mn0 = dmin * (float)mins[2 * g];
        float sc1 = d * (float)scales[2 * g + 1], mn1 = dmin * (float)mins[2 * g + 1];
        for (int l = 0; l < 32; l++) {
            uint8_t q = ql[32 * g + l], hb = qh[l];
            uint8_t hi0 = (hb & u1) ? 16 : 0, hi1 = (hb & u2) ? 16 : 0;
            dst[64 * g + l] = sc0 * (float)((q & 0xF) | hi0) - mn0;
            dst[64 * g + l + 32] = sc1 * (float)((q >> 4) | hi1) - mn1;
        }
        u1 = (uint8_t)(u1 << 2);
        u2 = (uint8_t)(u2 << 2);
    }
}

/* tensor/quantized_kquant.go:579-593 Q5KStorage.Dequantize. */
EXPORT void orc_q5k_dequant(const uint8_t* raw, int64_t nelem, float* dst) { kq_dequant(q5k_block, 176, raw, nelem, dst); }

/* One output of the K-quant GEMV-NTs: the row's super-blocks dequantized in
 * order and sum += a[p] * w[p] over all K values in element order.
 * GemmF32Q4KNT (internal/xblas/gemm_q4k.go:54-103) dequantizes per 32-value
 * sub-block with DequantizeSubBlock (tensor/quantized_kquant.go:82-106),
 * whose values equal DequantizeQ4K's (same d*sc, dmin*mn and formula);
 * GemmF32Q5KNT / GemmF32Q6KNT (internal/xblas/gemm_quant.go:273-317,
 * 384-428) dequantize whole super-blocks.  Either way the summation order is
 * p = 0 .. K-1 into one fp32 accumulator. */
typedef struct { const float* a; const uint8_t* raw; float* c; int64_t bpr; orc_kq_block_fn fn; int bytes; } kqnt_ctx;
static float kq_dot_row(const kqnt_ctx* t, const uint8_t* row) {
    float buf[256], sum = 0.0f;
    for (int64_t bi = 0; bi < t->bpr; bi++) {
        t->fn(row + bi * t->bytes, buf);
        const float* ab = t->a + bi * 256;
        for (int p = 0; p < 256; p++) sum += ab[p] * buf[p];
    }
    return sum;
}
static void kqnt_range(void* p, int64_t j0, int64_t j1) {
    kqnt_ctx* t = (kqnt_ctx*)p;
    for (int64_t j = j0; j < j1; j++) t->c[j] = kq_dot_row(t, t->raw + j * t->bpr * t->bytes);
}

/* fmt: 4 = Q4_K, 5 = Q5_K, 6 = Q6_K.  C[M,N] = A[M,K] * B^T, B = [N,K] in
 * contiguous super-blocks, K % 256 == 0 (the reference's other branch
 * dequantizes fully and calls SgemmSimd).  M = 1 with N*K >= 65536 splits N
 * over min(NumCPU, N/4) workers (gemm_q4k.go:72-79, gemm_quant.go:286-293,
 * 397-404); every output is computed whole by one worker, so the split does
 * not change any bit. */
EXPORT void orc_gemm_f32_kq_nt(int fmt, int64_t m, int64_t n, int64_t k, const float* a, const uint8_t* raw,
                               float* c, int nthreads) {
    kqnt_ctx ctx = {a, raw, c, k / 256, fmt == 4 ? q4k_block : fmt == 5 ? q5k_block : q6k_block,
                    fmt == 4 ? 144 : fmt == 5 ? 176 : 210};
    if (m == 1 && n * k >= 256 * 256) {
        int nc = nthreads;
        if (nc > n / 4) nc = (int)(n / 4);
        if (nc > 1) {
            orc_parallel_rows(n, nc, kqnt_range, &ctx);
            return;
        }
    }
    for (int64_t i = 0; i < m; i++) {
        ctx.a = a + i * k;
        ctx.c = c + i * n;
        kqnt_range(&ctx, 0, n);
    }
}

/* ------------------------------------------------------------------ Q5_0 */

/* tensor/quantized_q5_0.go:26-45 DequantizeQ5_0: 22-byte block [fp16 d]
 * [uint32 qh LE][16 bytes qs]; value j = d*((qs[j] & 15 | bit j of qh << 4) - 16),
 * value j+16 = d*((qs[j] >> 4 | bit j+16 of qh << 4) - 16).  :75-90
 * Q5_0Storage.Dequantize handles the partial last block. */
EXPORT void orc_q5_0_dequant(const uint8_t* raw, int64_t nelem, float* dst) {
    int64_t nblk = (nelem + 31) / 32;
    for (int64_t bi = 0; bi < nblk; bi++) {
        const uint8_t* b = raw + bi * 22;
        float d = orc_f16_to_f32(rd16(b));
        uint32_t qh = rd32(b + 2);
        float tmp[32];
        for (int j = 0; j < 16; j++) {
            uint8_t packed = b[6 + j];
            int x0 = (int)((packed & 0x0F) | (((qh >> j) & 1) << 4)) - 16;
            int x1 = (int)((packed >> 4) | (((qh >> (j + 16)) & 1) << 4)) - 16;
            tmp[j] = d * (float)x0;
            tmp[j + 16] = d * (float)x1;
        }
        int64_t off = bi * 32, rem = nelem - off;
        memcpy(dst + off, tmp, sizeof(float) * (size_t)(rem >= 32 ? 32 : rem));
    }
}

/* tensor/quantized_q5_0.go:151-165 Q5_0GPUQhOffset / Q5_0GPUQsOffset. */
EXPORT int64_t orc_q5_0_gpu_qh_offset(int64_t nblk) { return (nblk * 2 + 15) & ~(int64_t)15; }
EXPORT int64_t orc_q5_0_gpu_qs_offset(int64_t nblk) {
    return orc_q5_0_gpu_qh_offset(nblk) + ((nblk * 4 + 15) & ~(int64_t)15);
}

/* tensor/quantized_q5_0.go:118-147 RawBytesGPU: [fp16 d, nblk*2][pad 16]
 * [uint32 qh, nblk*4][pad 16][qs, nblk*16]. */
EXPORT void orc_q5_0_raw_to_gpu(const uint8_t* raw, int64_t nblk, uint8_t* out) {
    int64_t qh = orc_q5_0_gpu_qh_offset(nblk), qs = orc_q5_0_gpu_qs_offset(nblk);
    memset(out, 0, (size_t)qs);
    for (int64_t i = 0; i < nblk; i++) {
        memcpy(out + i * 2, raw + i * 22, 2);
        memcpy(out + qh + i * 4, raw + i * 22 + 2, 4);
        memcpy(out + qs + i * 16, raw + i * 22 + 6, 16);
    }
}

/* compute/cpu_engine.go:2450-2473, Q5_0 weights on the B side: dequantize
 * the [N,K] weights, transpose to [K,N], SgemmSimd into a zeroed C[M,N].
 * wtmp and ttmp each hold N*K floats. */
EXPORT void orc_gemm_f32_q5_0_nt(int64_t m, int64_t n, int64_t k, const float* a, const uint8_t* raw, float* c,
                                 float* wtmp, float* ttmp) {
    orc_q5_0_dequant(raw, n * k, wtmp);
    for (int64_t r = 0; r < n; r++)
        for (int64_t col = 0; col < k; col++) ttmp[col * n + r] = wtmp[r * k + col];
    memset(c, 0, sizeof(float) * (size_t)(m * n));
    orc_sgemm_simd(m, n, k, a, ttmp, c);
}

/* ------------------------------------------------------------ GGUF mmap */

/* tensor/mmap_storage.go:265-284 MmapStorage.dequantizeQ8_0: GGUF Q8_0,
 * 34-byte blocks [fp16 d][32 x int8], value = float32(int8) * d. */
EXPORT void orc_gguf_q8_0_dequant(const uint8_t* raw, int64_t nelem, float* dst) {
    int64_t nblk = (nelem + 31) / 32;
    for (int64_t bi = 0; bi < nblk; bi++) {
        const uint8_t* b = raw + bi * 34;
        float scale = orc_f16_to_f32(rd16(b));
        for (int j = 0; j < 32; j++) {
            int64_t idx = bi * 32 + j;
            if (idx >= nelem) break;
            dst[idx] = (float)(int8_t)b[2 + j] * scale;
        }
    }
}

/* internal/xblas/gemm_mmap.go:18-40 GemmF32MmapNT: C[M,N] = A[M,K] * B^T,
 * B an MmapStorage [N,K] of GGML type qtype (tensor/mmap_storage.go:18-30).
 * Q4_K / Q5_K / Q6_K stream super-blocks (gemm_mmap.go:56-195; the same
 * element-order sums as the storage GEMVs above); every other type is
 * dequantized whole (Slice, tensor/mmap_storage.go:127-134, 191-216) and
 * summed in element order.  Q4_0 (:239-263) dequantizes like Q4Storage,
 * Q5_0 (:368-400) like DequantizeQ5_0 (float32(q-16) * d).  wtmp holds N*K
 * floats for the dequantizing types. */
EXPORT int orc_gemm_f32_mmap_nt(int qtype, int64_t m, int64_t n, int64_t k, const float* a, const uint8_t* raw,
                                float* c, int nthreads, float* wtmp) {
    if (qtype == 12 || qtype == 13 || qtype == 14) {
        orc_gemm_f32_kq_nt(qtype == 12 ? 4 : qtype == 13 ? 5 : 6, m, n, k, a, raw, c, nthreads);
        return 0;
    }
    if (qtype == 2) orc_q4_dequant(raw, n * k, wtmp);
    else if (qtype == 8) orc_gguf_q8_0_dequant(raw, n * k, wtmp);
    else if (qtype == 6) orc_q5_0_dequant(raw, n * k, wtmp);
    else return -1;
    for (int64_t i = 0; i < m; i++)
        for (int64_t j = 0; j < n; j++) {
            float sum = 0.0f;
            for (int64_t p = 0; p < k; p++) sum += a[i * k + p] * wtmp[j * k + p];
            c[i * n + j] = sum;
        }
    return 0;
}

/* ------------------------------------------------ int4 / int8 GEMMs (a18) */

/* internal/cuda/kernels/gemm_int4.cu:20-27 extract_int4: element idx of a
 * packed row, even idx in the low nibble, sign-extended from 4 bits. */
static int orc_int4_at(const uint8_t* packed, int64_t idx) {
    uint8_t byte = packed[idx >> 1];
    int val = (idx & 1) ? (byte >> 4) : (byte & 0x0F);
    if (val >= 8) val -= 16;
    return val;
}

typedef struct {
    const uint8_t* a; const float* b; float* c; const float* scales; const uint8_t* zeros;
    int64_t m, k, n, gs;
} int4_ctx;

/* gemm_int4.cu:29-56 gemm_int4_kernel, one output (row, col) at a time:
 * dequant = (float)(v - zero) * scale, acc += dequant * B[k, col] in k order.
 * nvcc contracts the accumulation into an FMA (its default -fmad=true), so
 * the restatement calls fmaf. */
static void int4_rows(void* p, int64_t r0, int64_t r1) {
    const int4_ctx* x = (const int4_ctx*)p;
    int64_t ng = (x->k + x->gs - 1) / x->gs;
    for (int64_t row = r0; row < r1; row++)
        for (int64_t col = 0; col < x->n; col++) {
            float acc = 0.0f;
            for (int64_t kk = 0; kk < x->k; kk++) {
                int64_t g = kk / x->gs;
                float scale = x->scales[row * ng + g];
                int zero = (int)x->zeros[row * ng + g];
                int v = orc_int4_at(x->a + row * (x->k / 2), kk);
                float dequant = (float)(v - zero) * scale;
                acc = fmaf(dequant, x->b[kk * x->n + col], acc);
            }
            x->c[row * x->n + col] = acc;
        }
}

/* gemm_int4.cu:58-81 gemm_int4_f32: returns 1 (InvalidValue) for an odd K
 * or group_size <= 0, as the launcher does, else 0. */
EXPORT int orc_gemm_int4_f32(const uint8_t* a, const float* b, float* c, const float* scales, const uint8_t* zeros,
                             int64_t m, int64_t k, int64_t n, int64_t gs, int nthreads) {
    if (k % 2 != 0 || gs <= 0) return 1;
    int4_ctx ctx = {a, b, c, scales, zeros, m, k, n, gs};
    orc_parallel_rows(m, nthreads, int4_rows, &ctx);
    return 0;
}

/* gemm_int4.cu:89-115 gemm_int4_rmul_kernel: C[b, j] = sum_k B[b, k] *
 * dequant(W[k, j]), W [in, out/2] packed along out, scales / zeros
 * [in, ceil(out/gs)] with groups along out; acc += B * dequant (FMA). */
static void int4_rmul_rows(void* p, int64_t r0, int64_t r1) {
    const int4_ctx* x = (const int4_ctx*)p; /* m = batch, k = in, n = out */
    int64_t ng = (x->n + x->gs - 1) / x->gs;
    for (int64_t row = r0; row < r1; row++)
        for (int64_t col = 0; col < x->n; col++) {
            float acc = 0.0f;
            int64_t g = col / x->gs;
            for (int64_t kk = 0; kk < x->k; kk++) {
                float scale = x->scales[kk * ng + g];
                int zero = (int)x->zeros[kk * ng + g];
                int v = orc_int4_at(x->a + kk * (x->n / 2), col);
                float dequant = (float)(v - zero) * scale;
                acc = fmaf(x->b[row * x->k + kk], dequant, acc);
            }
            x->c[row * x->n + col] = acc;
        }
}

/* gemm_int4.cu:117-144 gemm_int4_f32_rmul: 1 for an odd out_features or
 * group_size <= 0, else 0. */
EXPORT int orc_gemm_int4_f32_rmul(const uint8_t* w, const float* x, float* c, const float* scales,
                                  const uint8_t* zeros, int64_t batch, int64_t in, int64_t out, int64_t gs,
                                  int nthreads) {
    if (out % 2 != 0 || gs <= 0) return 1;
    int4_ctx ctx = {w, x, c, scales, zeros, batch, in, out, gs};
    orc_parallel_rows(batch, nthreads, int4_rmul_rows, &ctx);
    return 0;
}

typedef struct { const int8_t* a; const float* b; float* c; int64_t m, k, n; } int8_ctx;

/* gemm_int8.cu:16-56 gemm_int8_kernel: acc += float(A[row, k]) * B[k, col]
 * over 32-wide K tiles in k order (zero-padded past K), one FMA each. */
static void int8_rows(void* p, int64_t r0, int64_t r1) {
    const int8_ctx* x = (const int8_ctx*)p;
    for (int64_t row = r0; row < r1; row++)
        for (int64_t col = 0; col < x->n; col++) {
            float acc = 0.0f;
            for (int64_t kk = 0; kk < x->k; kk++) acc = fmaf((float)x->a[row * x->k + kk], x->b[kk * x->n + col], acc);
            x->c[row * x->n + col] = acc;
        }
}

/* gemm_int8.cu:58-73 gemm_int8_f32. */
EXPORT void orc_gemm_int8_f32(const int8_t* a, const float* b, float* c, int64_t m, int64_t k, int64_t n,
                              int nthreads) {
    int8_ctx ctx = {a, b, c, m, k, n};
    orc_parallel_rows(m, nthreads, int8_rows, &ctx);
}

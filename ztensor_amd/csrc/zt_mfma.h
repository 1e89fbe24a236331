// Shared pieces of the small-batch MFMA GEMMs (W4A16, IQ4_NL) for gfx950.
//
// Common structure (C[rows, N] = W[rows, K] x X[K, N], 4 <= N <= 16, N % 4 == 0,
// K % 128 == 0, X fp16 row-major with N columns):
//  * a workgroup of kMfmaWaves waves owns kMfmaRows rows (two 16-row MFMA
//    tiles) and walks K in chunks of kMfmaKC;
//  * each chunk's X rows are copied (16 bytes a lane, coalesced) into LDS
//    with two padding rows after every 32, which puts the four 16-lane
//    groups of a transposing read on distinct banks;
//  * the B operand of v_mfma_f32_16x16x32_f16 (32 K x 16 columns) is read
//    with two ds_read_b64_tr_b16: within each 16-lane group, lane 4a + b
//    addresses X row r(a) and columns 4b .. 4b+3, and the read hands lane n
//    the four values X[r(0..3)][n]; columns >= N address a zero word;
//  * the waves' partial output tiles are summed through LDS at the end and
//    every output is stored once: a workgroup covers all of K, so the
//    result is the same on every run.
#pragma once

#include "zt_common.h"

namespace zt {

typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef _Float16 half8v __attribute__((ext_vector_type(8)));
typedef _Float16 half4v __attribute__((ext_vector_type(4)));
typedef short short4v __attribute__((ext_vector_type(4)));
typedef short short8v __attribute__((ext_vector_type(8)));
typedef float float4v __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) short4v lds_short4v;
typedef __attribute__((address_space(3))) char lds_char;

// A dword viewed as two fp16 halves (x = bits 0-15).
__device__ __forceinline__ half2v as_half2(uint32_t u) { return __builtin_bit_cast(half2v, u); }

constexpr int kMfmaRows = 32;                         // rows per workgroup (two 16-row tiles)
constexpr int kMfmaTiles = kMfmaRows / 16;
constexpr int kMfmaWaves = 8;                         // waves per workgroup
constexpr int kMfmaUPW = 2;                           // 128-K units per wave per chunk
constexpr int kMfmaKC = 128 * kMfmaWaves * kMfmaUPW;  // K per chunk
constexpr int kMfmaUC = kMfmaKC / 128;                // units per chunk

__device__ __forceinline__ short4v tr_read_b64(char* lds, int byte_off) {
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4v*)((lds_char*)lds + byte_off));
}

// Bytes of one staged X chunk: kMfmaKC rows of 2N bytes plus 2 pad rows per 32.
__host__ __device__ __forceinline__ int mfma_xbytes(int N) { return (kMfmaKC + kMfmaKC / 16) * 2 * N; }

// Bytes of a staged X chunk of KC rows (row stride 2N bytes, two pad rows per 32).
__host__ __device__ constexpr int mfma_chunk_xbytes(int KC, int N) { return (KC + KC / 16) * 2 * N; }

// LDS byte offset of chunk-relative X row k (row stride 2N, 2 pad rows per 32).
__device__ __forceinline__ int mfma_xrow(int k, int N) { return (k + 2 * (k >> 5)) * 2 * N; }

// Copies X rows [c0*128, min(c0*128 + kMfmaKC, kend)) into the padded LDS chunk.
__device__ __forceinline__ void mfma_stage_x(char* smem, const uint16_t* __restrict__ x, int c0, int kend, int N) {
    const int npieces = min(kMfmaKC, kend - c0 * 128) * 2 * N / 16;
    const uint4* xg = reinterpret_cast<const uint4*>(x + (long)c0 * 128 * N);
    for (int p = threadIdx.x; p < npieces; p += blockDim.x) {
        const uint4 v = xg[p];
        const int off = p * 16;  // a 16-byte piece never straddles a 32-row segment (64N bytes)
        *reinterpret_cast<uint4*>(smem + off + (off / (64 * N)) * (4 * N)) = v;
    }
}

// Per-lane roles of the transposing reads (li = lane % 16).
struct MfmaBRole {
    int jq, qq;
    bool colok;
    __device__ __forceinline__ MfmaBRole(int li, int N) : jq(li >> 2), qq(li & 3), colok(4 * (li & 3) < N) {}
};

// B operand for the 8 chunk-relative X rows k0 + ord[0..7] (ord given as the
// two row-offset quadruples of the two reads), column li.
__device__ __forceinline__ half8v mfma_b_operand(char* smem, const MfmaBRole& ro, int k0, int offa, int offb, int N,
                                                 int zero_off) {
    const int ra = k0 + offa, rb = k0 + offb;
    const int adda = ro.colok ? mfma_xrow(ra, N) + 8 * ro.qq : zero_off;
    const int addb = ro.colok ? mfma_xrow(rb, N) + 8 * ro.qq : zero_off;
    const short4v ba = tr_read_b64(smem, adda), bb = tr_read_b64(smem, addb);
    return __builtin_bit_cast(half8v, (short8v){ba[0], ba[1], ba[2], ba[3], bb[0], bb[1], bb[2], bb[3]});
}

// B operand from two transposing reads at LDS byte offsets a and a + db.
// The tiled kernels pass a = (lane part) + (compile-time part): every row a
// step reads lies in one 32-row segment of the padded chunk, so the pad term
// of mfma_xrow is a per-unit constant and the whole offset folds into the
// instructions' immediate field.  Columns >= N read neighbouring LDS bytes;
// they only reach D columns >= N, which are never stored.
__device__ __forceinline__ half8v mfma_b_pair(char* smem, int a, int db) {
    const short4v ba = tr_read_b64(smem, a), bb = tr_read_b64(smem, a + db);
    return __builtin_bit_cast(half8v, (short8v){ba[0], ba[1], ba[2], ba[3], bb[0], bb[1], bb[2], bb[3]});
}

// Sums the waves' partial tiles and stores C rows row0 .. row0+31, columns < N.
// acc[t][i] of lane l holds row 16t + 4*(l/16) + i, column l%16 (the MFMA
// D layout).  Uses smem as scratch; the caller has passed a barrier after
// its last read of the staged chunk.
__device__ __forceinline__ void mfma_reduce_store(float4v (&acc)[kMfmaTiles], char* smem, float* __restrict__ y,
                                                  int row0, int rows, int N) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    float* red = reinterpret_cast<float*>(smem);
#pragma unroll
    for (int t = 0; t < kMfmaTiles; t++)
#pragma unroll
        for (int i = 0; i < 4; i++) red[((wave * kMfmaTiles + t) * 4 + i) * 64 + lane] = acc[t][i];
    __syncthreads();
    for (int o = tid; o < kMfmaTiles * 256; o += blockDim.x) {
        const int t = o >> 8, r = (o >> 4) & 15, n = o & 15;
        const int ln = (r >> 2) * 16 + n, i = r & 3;
        float sum = 0.f;
#pragma unroll
        for (int wv = 0; wv < kMfmaWaves; wv++) sum += red[((wv * kMfmaTiles + t) * 4 + i) * 64 + ln];
        const int row = row0 + 16 * t + r;
        if (n < N && row < rows) y[(long)row * N + n] = sum;
    }
}

// ---- split-K through a workspace (tiled kernels)
//
// A K-split workgroup of a tiled kernel stores each of its partial 16-row
// output tiles in MFMA D lane order, one 16-byte store per lane, at
// ws + ((split * ntiles + rt) * 64 + lane) * 4 floats.  tiled_reduce_kernel
// then sums the splits of every tile in split order and writes C once: no
// zero fill, no atomics, and the same result on every run.  The workspace
// holds splits * ntiles KB.  Partials are stored and loaded nontemporally:
// they are read once, by the next kernel (with ordinary stores the GEMM
// measured 10-15% slower at the Llama-3-8B shapes, batch 16).

__device__ __forceinline__ void tiled_store_partial(const float4v& v, float* __restrict__ ws, int split, int ntiles,
                                                    int rt, int lane, int N) {
    if ((lane & 15) < N) __builtin_nontemporal_store(v, reinterpret_cast<float4v*>(ws + (((long)split * ntiles + rt) * 64 + lane) * 4));
}

static __global__ void __launch_bounds__(64) tiled_reduce_kernel(const float* __restrict__ ws, float* __restrict__ y,
                                                                 int rows, int N, int ntiles, int splits) {
    // thread = one output of a lane with column < N: (tile, lane 16g + i, element e),
    // consecutive threads on consecutive floats of the partial tiles
    const long q = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (q >= (long)ntiles * 16 * N) return;
    const long rt = q / (16 * N);
    const int r = (int)(q % (16 * N)), lg = r / (4 * N), li = (r / 4) % N, e = r % 4;
    const long p = (rt * 64 + 16 * lg + li) * 4 + e, stride = (long)ntiles * 256;
    // up to 32 splits' loads in flight before the adds, summed in split order
    float s = 0.0f;
    for (int k0 = 0; k0 < splits; k0 += 32) {
        float v[32];
#pragma unroll
        for (int j = 0; j < 32; j++) v[j] = k0 + j < splits ? __builtin_nontemporal_load(ws + (k0 + j) * stride + p) : 0.0f;
#pragma unroll
        for (int j = 0; j < 32; j++) s += v[j];
    }
    const long row = rt * 16 + 4 * lg + e;
    if (row < rows) y[row * N + li] = s;
}

__host__ __forceinline__ long tiled_ws_bytes(int rows, int splits) {
    return splits > 1 ? (long)splits * ((rows + 15) / 16) * 1024 : 0;
}

__host__ __forceinline__ void tiled_reduce(const void* ws, float* y, int rows, int N, int splits, hipStream_t st) {
    const int ntiles = (rows + 15) / 16;
    tiled_reduce_kernel<<<(int)(((long)ntiles * 16 * N + 63) / 64), 64, 0, st>>>(
        static_cast<const float*>(ws), y, rows, N, ntiles, splits);
}

static __global__ void mfma_zero_kernel(float* __restrict__ y, long n) {
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) y[i] = 0.0f;
}

static __global__ void mfma_zero4_kernel(float4* __restrict__ y, long n4) {
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n4) y[i] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
}

// Zeroes C before a split-K launch on the same stream (16-byte stores when
// C is 16-byte aligned and a multiple of 4 floats).
__host__ __forceinline__ void mfma_zero(float* y, long n, hipStream_t st) {
    if (((uintptr_t)y & 15) == 0 && n % 4 == 0)
        mfma_zero4_kernel<<<(int)((n / 4 + 255) / 256), 256, 0, st>>>(reinterpret_cast<float4*>(y), n / 4);
    else
        mfma_zero_kernel<<<(int)((n + 255) / 256), 256, 0, st>>>(y, n);
}

__host__ __forceinline__ size_t mfma_reduce_bytes() { return (size_t)kMfmaWaves * kMfmaTiles * 4 * 64 * sizeof(float); }

// Host-side eligibility of a call for the MFMA path.
__host__ __forceinline__ bool mfma_shape_ok(int N, int K, const void* x) {
    return N >= 4 && N <= 16 && N % 4 == 0 && K % 128 == 0 && ((uintptr_t)x & 15) == 0;
}

}  // namespace zt

// W4A16 GEMV / small-batch GEMM for gfx950: 4-bit group-quantized weights
// (GPTQ / AWQ) times fp16 activations, fp32 accumulation and fp32 output
// (the result type of compute.MatMulW4A16, compute/w4a16.go:64-119).
//
// Weight layout ([rows, K], groups of `group` consecutive weights along K):
//   packed: rows*K/2 bytes, element j at the low nibble of byte j/2 when j is
//           even and the high nibble when odd.  This is GPTQStorage's packing
//           (tensor/quantized_gptq.go:110-116, 145-155) with all groups
//           concatenated (NewGPTQStorageFromRaw, :217-277), and byte for byte
//           the same as AWQStorage's little-endian uint32 words with 8
//           nibbles each (tensor/quantized_awq.go:97-105, 118-136).
//   scales, zeros: fp16, one per group, [rows, K/group].  zeros may be
//           NULL, meaning the symmetric zero-point 8.
// Dequantization: w = (float(q) - zero) * scale (quantized_gptq.go:154).
//
// GEMV (VALU): lane <-> 32 consecutive weights (16 bytes, one 128-bit load),
// R rows per wave with the lane's activations held in registers, split-K
// over the waves of a workgroup.  Inside a chunk (one group, since group is
// a multiple of 32):
//     sum_j (q_j - z) x_j * s = s * (sum_j q_j x_j - z * sum_j x_j)
// q_j becomes an exact fp16 by OR-ing the nibble into the mantissa of 1024.0
// (0x6400 | q == 1024 + q) and subtracting 1024 with one packed fp16 add for
// two weights; v_dot2_f32_f16 then multiplies two exact fp16 products and
// accumulates them in fp32.  Nibble pairs are taken as (w >> 4t) &
// 0x000F000F, which pairs element e with e+4 inside each dword; the
// activations are pre-permuted into the same pairs once per lane.
//
// Small-batch GEMM (N = 4, 8, 12, 16): the row-block GEMM on
// v_mfma_f32_4x4x4_16b_f16, and for N = 12 and 16 past 2048 rows
// v_mfma_f32_16x16x32_f16 (see the sections below).
#include "zt_rbmfma.h"

namespace zt {


__device__ __forceinline__ half2v as_h2(uint32_t u) { return __builtin_bit_cast(half2v, u); }

// Two nibbles (bits 0-3 and 16-19 of v after the mask) -> exact fp16 pair.
__device__ __forceinline__ half2v nib_pair(uint32_t v) {
    const half2v biased = as_h2((v & 0x000F000Fu) | 0x64006400u);  // 1024 + q
    return biased - (half2v){(_Float16)1024.0f, (_Float16)1024.0f};
}

// fp16 activations of one 32-weight chunk, permuted into the nibble-pair
// order: xp[i][t] = (x[8i+t], x[8i+t+4]).
__device__ __forceinline__ void permute_x(const uint32_t (&xr)[16], uint32_t (&xp)[4][4]) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t X0 = xr[4 * i], X1 = xr[4 * i + 1], X2 = xr[4 * i + 2], X3 = xr[4 * i + 3];
        xp[i][0] = __builtin_amdgcn_perm(X2, X0, 0x05040100u);  // (x0, x4)
        xp[i][1] = __builtin_amdgcn_perm(X2, X0, 0x07060302u);  // (x1, x5)
        xp[i][2] = __builtin_amdgcn_perm(X3, X1, 0x05040100u);  // (x2, x6)
        xp[i][3] = __builtin_amdgcn_perm(X3, X1, 0x07060302u);  // (x3, x7)
    }
}

template <int R, bool CONTIG>
__global__ void __launch_bounds__(512) w4a16_gemv_kernel(const uint4* __restrict__ packed,
                                                         const uint16_t* __restrict__ scales,
                                                         const uint16_t* __restrict__ zeros,
                                                         const uint16_t* __restrict__ x, float* __restrict__ y,
                                                         long xy_stride, int rows, int nchunk, int chunks_per_group) {
    __shared__ float red[8 * R];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nwaves = blockDim.x >> 6;
    x += blockIdx.y;
    y += blockIdx.y;
    const int ngroups = nchunk / chunks_per_group;
    const int row0 = blockIdx.x * R;
    int rr[R];
#pragma unroll
    for (int r = 0; r < R; r++) rr[r] = min(row0 + r, rows - 1);

    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.0f;

    for (int c = wave * kWave + lane; c < nchunk; c += nwaves * kWave) {
        const int g = c / chunks_per_group;
        uint4 w[R];
        uint16_t s[R], z[R];
#pragma unroll
        for (int r = 0; r < R; r++) {
            w[r] = ld_stream(&packed[(long)rr[r] * nchunk + c]);
            s[r] = scales[(long)rr[r] * ngroups + g];
            z[r] = zeros ? zeros[(long)rr[r] * ngroups + g] : (uint16_t)0x4800;  // fp16 8.0
        }
        uint32_t xr[16];
        if constexpr (CONTIG) {
            const uint4* p = reinterpret_cast<const uint4*>(x + (long)c * 32);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint4 t = p[i];
                xr[4 * i] = t.x; xr[4 * i + 1] = t.y; xr[4 * i + 2] = t.z; xr[4 * i + 3] = t.w;
            }
        } else {
#pragma unroll
            for (int i = 0; i < 16; i++)
                xr[i] = (uint32_t)x[((long)c * 32 + 2 * i) * xy_stride] |
                        ((uint32_t)x[((long)c * 32 + 2 * i + 1) * xy_stride] << 16);
        }
        uint32_t xp[4][4];
        permute_x(xr, xp);
        float xsum = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; i++) xsum = __builtin_amdgcn_fdot2(as_h2(xr[i]), as_h2(0x3c003c00u), xsum, false);
#pragma unroll
        for (int r = 0; r < R; r++) {
            const uint32_t d[4] = {w[r].x, w[r].y, w[r].z, w[r].w};
            float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                s0 = __builtin_amdgcn_fdot2(nib_pair(d[i]), as_h2(xp[i][0]), s0, false);
                s1 = __builtin_amdgcn_fdot2(nib_pair(d[i] >> 4), as_h2(xp[i][1]), s1, false);
                s0 = __builtin_amdgcn_fdot2(nib_pair(d[i] >> 8), as_h2(xp[i][2]), s0, false);
                s1 = __builtin_amdgcn_fdot2(nib_pair(d[i] >> 12), as_h2(xp[i][3]), s1, false);
            }
            acc[r] = fmaf(h2f(s[r]), (s0 + s1) - h2f(z[r]) * xsum, acc[r]);
        }
    }
    block_reduce_store<R>(acc, red, y, xy_stride, row0, rows);
}

template <bool CONTIG>
static void launch_w4a16_gemv(int R, dim3 g, dim3 b, hipStream_t st, const uint4* w, const uint16_t* s,
                              const uint16_t* z, const uint16_t* x, float* y, long stride, int rows, int nchunk,
                              int cpg) {
    switch (R) {
        case 8: w4a16_gemv_kernel<8, CONTIG><<<g, b, 0, st>>>(w, s, z, x, y, stride, rows, nchunk, cpg); break;
        case 4: w4a16_gemv_kernel<4, CONTIG><<<g, b, 0, st>>>(w, s, z, x, y, stride, rows, nchunk, cpg); break;
        case 2: w4a16_gemv_kernel<2, CONTIG><<<g, b, 0, st>>>(w, s, z, x, y, stride, rows, nchunk, cpg); break;
        default: w4a16_gemv_kernel<1, CONTIG><<<g, b, 0, st>>>(w, s, z, x, y, stride, rows, nchunk, cpg); break;
    }
}

// Batch-1 GEMV: four lanes share one 32-weight chunk.  Lane q of a quad
// loads dword q of the chunk (weights 8q .. 8q+7; nibble m of the dword is
// weight 8q+m) and the 8 matching fp16 activations as one 16-byte load, so a
// wave reads 256 contiguous weight bytes per row and 16 contiguous chunks of
// activations.  A nibble masked into an fp16 half is the subnormal q * 2^-24
// (or q * 2^-20 for the upper nibble of a byte); v_fma_mix_f32 multiplies it
// by the fp16 activation into an fp32 accumulator exactly.  Per chunk and row:
// y += s * (2^24 sum_lo + 2^20 sum_hi - z * sum x).  The workgroup's scale
// and zero pairs are staged in LDS once (one dword per row and group), so a
// step issues one global load per row.
template <int R>
__global__ void __launch_bounds__(512) w4a16_quad_kernel(const uint32_t* __restrict__ packed,
                                                         const uint16_t* __restrict__ scales,
                                                         const uint16_t* __restrict__ zeros,
                                                         const uint16_t* __restrict__ x, float* __restrict__ y,
                                                         int rows, int nchunk, int chunks_per_group) {
    __shared__ float red[8 * R];
    extern __shared__ uint32_t sz[];  // [group][R]: scale | zero << 16
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nwaves = blockDim.x >> 6;
    const int q = lane & 3;
    const int ngroups = nchunk / chunks_per_group;
    const int row0 = blockIdx.x * R;
    int rr[R];
#pragma unroll
    for (int r = 0; r < R; r++) rr[r] = min(row0 + r, rows - 1);
    for (int e = threadIdx.x; e < R * ngroups; e += blockDim.x) {
        const int r = e / ngroups, g = e - r * ngroups;  // row-major walk: coalesced global reads
        const long gi = (long)min(row0 + r, rows - 1) * ngroups + g;
        sz[g * R + r] = (uint32_t)scales[gi] | ((uint32_t)(zeros ? zeros[gi] : (uint16_t)0x4800) << 16);  // zero 8.0
    }
    __syncthreads();
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.0f;

    for (int c = wave * 16 + (lane >> 2); c < nchunk; c += nwaves * 16) {
        const int g = c / chunks_per_group;
        uint32_t w[R];
#pragma unroll
        for (int r = 0; r < R; r++) w[r] = __builtin_nontemporal_load(&packed[((long)rr[r] * nchunk + c) * 4 + q]);
        const uint4 xv = *reinterpret_cast<const uint4*>(x + (long)c * 32 + 8 * q);
        const half2v x01 = as_h2(xv.x), x23 = as_h2(xv.y), x45 = as_h2(xv.z), x67 = as_h2(xv.w);
        float xsum = __builtin_amdgcn_fdot2(x01, as_h2(0x3c003c00u), 0.0f, false);
        xsum = __builtin_amdgcn_fdot2(x23, as_h2(0x3c003c00u), xsum, false);
        xsum = __builtin_amdgcn_fdot2(x45, as_h2(0x3c003c00u), xsum, false);
        xsum = __builtin_amdgcn_fdot2(x67, as_h2(0x3c003c00u), xsum, false);
#pragma unroll
        for (int r = 0; r < R; r++) {
            const uint32_t d = w[r], d8 = d >> 8;
            const half2v m0 = as_h2(d & 0x000F000Fu);   // weights 0, 4  (q * 2^-24)
            const half2v m1 = as_h2(d & 0x00F000F0u);   // weights 1, 5  (q * 2^-20)
            const half2v m2 = as_h2(d8 & 0x000F000Fu);  // weights 2, 6
            const half2v m3 = as_h2(d8 & 0x00F000F0u);  // weights 3, 7
            float sa = (float)m0.x * (float)x01.x;
            float sb = (float)m1.x * (float)x01.y;
            sa = __builtin_fmaf((float)m0.y, (float)x45.x, sa);
            sb = __builtin_fmaf((float)m1.y, (float)x45.y, sb);
            sa = __builtin_fmaf((float)m2.x, (float)x23.x, sa);
            sb = __builtin_fmaf((float)m3.x, (float)x23.y, sb);
            sa = __builtin_fmaf((float)m2.y, (float)x67.x, sa);
            sb = __builtin_fmaf((float)m3.y, (float)x67.y, sb);
            const uint32_t szr = sz[g * R + r];
            const float t = __builtin_fmaf(sa, 16777216.0f, __builtin_fmaf(sb, 1048576.0f, -h2f(szr >> 16) * xsum));
            acc[r] = fmaf(h2f(szr & 0xffff), t, acc[r]);
        }
    }
    block_reduce_store<R>(acc, red, y, 1, row0, rows);
}

template <int R>
static void launch_w4a16_quad_r(dim3 g, dim3 b, hipStream_t st, const uint32_t* w, const uint16_t* s,
                                const uint16_t* z, const uint16_t* x, float* y, int rows, int nchunk, int cpg) {
    const size_t lds = (size_t)R * (nchunk / cpg) * sizeof(uint32_t);
    w4a16_quad_kernel<R><<<g, b, lds, st>>>(w, s, z, x, y, rows, nchunk, cpg);
}

static void launch_w4a16_quad(int R, dim3 g, dim3 b, hipStream_t st, const uint32_t* w, const uint16_t* s,
                              const uint16_t* z, const uint16_t* x, float* y, int rows, int nchunk, int cpg) {
    switch (R) {
        case 8: launch_w4a16_quad_r<8>(g, b, st, w, s, z, x, y, rows, nchunk, cpg); break;
        case 4: launch_w4a16_quad_r<4>(g, b, st, w, s, z, x, y, rows, nchunk, cpg); break;
        case 2: launch_w4a16_quad_r<2>(g, b, st, w, s, z, x, y, rows, nchunk, cpg); break;
        default: launch_w4a16_quad_r<1>(g, b, st, w, s, z, x, y, rows, nchunk, cpg); break;
    }
}


// Batch-1 W4A16 with a fixed S steps of 16 chunks per wave (the quad
// mapping of w4a16_quad_kernel) for K <= 16384 (SZ = false) or K <= 32768
// (SZ = true).  Every load of all S steps - weights, the rows' (scale, zero)
// pairs of each step's group and the activations - is issued before any
// arithmetic, so a wave waits for one memory round trip.  Buffer loads take
// the wave-uniform row offsets as scalar offsets; lanes past the last chunk
// read zeros through out-of-range offsets.
//  * SZ = false: scales and zeros are the stored fp16 arrays, two 2-byte
//    loads per row and step (zeros == NULL: no records, zero-point 8);
//  * SZ = true: szr holds one dword per (row, group), scale | zero << 16,
//    row-major (zt_w4a16_pack_szr): one load per row and step.  At
//    28672 x 8192 this measured 23.4 us against 27.6 us for the two loads.
//  The arguments fit the 14 kernel-argument dwords gfx950 preloads into
//  SGPRs (meta = szr for SZ, else the scales), and the group of chunk c is
//  int((c + 0.5) * (1 / chunks_per_group)) in fp32, exact for every c <= 1024
//  and up to 4096 chunks a group (checked exhaustively: the 0.5 margin dwarfs
//  the product's rounding), so no wave waits on an argument load or an
//  integer division before its scale loads.
template <int S, int R, bool SZ>
__device__ __forceinline__ void w4a16_steps_body(const uint32_t* __restrict__ packed, const void* __restrict__ meta,
                                                 const uint16_t* __restrict__ zeros, const uint16_t* __restrict__ x,
                                                 float* __restrict__ y, int rows, int nchunk, int ngroups,
                                                 float inv_cpg, int row0, float* red) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int q = lane & 3;
    const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc((void*)packed, (short)0, 0x7fffffff, 0x00020000);
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void*)meta, (short)0, 0x7fffffff, 0x00020000);
    const __amdgpu_buffer_rsrc_t rz = __builtin_amdgcn_make_buffer_rsrc((void*)zeros, (short)0, zeros ? 0x7fffffff : 0,
                                                                        0x00020000);
    const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc((void*)x, (short)0, nchunk * 64, 0x00020000);
    uint32_t w[S][R], sc[S][R], zr[S][R];
    u32x4 xv[S];
#pragma unroll
    for (int t = 0; t < S; t++) {
        const int c = (wave * S + t) * 16 + (lane >> 2);
        const bool ok = c < nchunk;
        const uint32_t voff = ok ? (uint32_t)(c * 16 + q * 4) : 0x80000000u;
#pragma unroll
        for (int r = 0; r < R; r++) {
            const uint32_t row = (uint32_t)min(row0 + r, rows - 1);
            w[t][r] = __builtin_amdgcn_raw_buffer_load_b32(rw, voff, row * (uint32_t)nchunk * 16u, 2);  // nontemporal
        }
        xv[t] = __builtin_amdgcn_raw_buffer_load_b128(rx, ok ? (uint32_t)(c * 64 + q * 16) : 0x80000000u, 0, 0);
    }
#pragma unroll
    for (int t = 0; t < S; t++) {
        const int c = (wave * S + t) * 16 + (lane >> 2);
        const uint32_t g = (uint32_t)(((float)c + 0.5f) * inv_cpg);
#pragma unroll
        for (int r = 0; r < R; r++) {
            const uint32_t rowg = (uint32_t)min(row0 + r, rows - 1) * (uint32_t)ngroups;
            if (SZ) {
                sc[t][r] = __builtin_amdgcn_raw_buffer_load_b32(rs, c < nchunk ? g * 4u : 0x80000000u, rowg * 4u, 0);
            } else {
                const uint32_t goff = c < nchunk ? g * 2u : 0x80000000u;
                sc[t][r] = __builtin_amdgcn_raw_buffer_load_b16(rs, goff, rowg * 2u, 0);
                // no zeros array: the buffer has no records and reads 0; zero-point 8 is applied below
                zr[t][r] = __builtin_amdgcn_raw_buffer_load_b16(rz, goff, rowg * 2u, 0);
            }
        }
    }
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.0f;
#pragma unroll
    for (int t = 0; t < S; t++) {
        const half2v x01 = as_h2(xv[t].x), x23 = as_h2(xv[t].y), x45 = as_h2(xv[t].z), x67 = as_h2(xv[t].w);
        float xsum = __builtin_amdgcn_fdot2(x01, as_h2(0x3c003c00u), 0.0f, false);
        xsum = __builtin_amdgcn_fdot2(x23, as_h2(0x3c003c00u), xsum, false);
        xsum = __builtin_amdgcn_fdot2(x45, as_h2(0x3c003c00u), xsum, false);
        xsum = __builtin_amdgcn_fdot2(x67, as_h2(0x3c003c00u), xsum, false);
#pragma unroll
        for (int r = 0; r < R; r++) {
            const uint32_t d = w[t][r], d8 = d >> 8;
            const half2v m0 = as_h2(d & 0x000F000Fu);   // weights 0, 4  (q * 2^-24)
            const half2v m1 = as_h2(d & 0x00F000F0u);   // weights 1, 5  (q * 2^-20)
            const half2v m2 = as_h2(d8 & 0x000F000Fu);  // weights 2, 6
            const half2v m3 = as_h2(d8 & 0x00F000F0u);  // weights 3, 7
            float sa = (float)m0.x * (float)x01.x;
            float sb = (float)m1.x * (float)x01.y;
            sa = __builtin_fmaf((float)m0.y, (float)x45.x, sa);
            sb = __builtin_fmaf((float)m1.y, (float)x45.y, sb);
            sa = __builtin_fmaf((float)m2.x, (float)x23.x, sa);
            sb = __builtin_fmaf((float)m3.x, (float)x23.y, sb);
            sa = __builtin_fmaf((float)m2.y, (float)x67.x, sa);
            sb = __builtin_fmaf((float)m3.y, (float)x67.y, sb);
            const half2v szh = as_h2(sc[t][r]);
            const float z = SZ ? (float)szh.y : zeros ? (float)as_h2(zr[t][r]).x : 8.0f;
            const float tq = __builtin_fmaf(sa, 16777216.0f, __builtin_fmaf(sb, 1048576.0f, -z * xsum));
            acc[r] = __builtin_fmaf((float)szh.x, tq, acc[r]);
        }
    }
    block_reduce_store<R>(acc, red, y, 1, row0, rows);
}

template <int S, int R, bool SZ>
__global__ void __launch_bounds__(1024) w4a16_steps_kernel(const uint32_t* __restrict__ packed,
                                                           const void* __restrict__ meta,
                                                           const uint16_t* __restrict__ zeros,
                                                           const uint16_t* __restrict__ x, float* __restrict__ y,
                                                           int rows, int nchunk, int ngroups, float inv_cpg) {
    __shared__ float red[16 * R];
    w4a16_steps_body<S, R, SZ>(packed, meta, zeros, x, y, rows, nchunk, ngroups, inv_cpg, blockIdx.x * R, red);
}

// Several W4A16 matrices on packed (scale, zero) dwords that read the same
// activation vector (q/k/v, or gate/up, of a decode layer) in one launch:
// workgroups [wg0[i], wg0[i+1]) run matrix i with the body above, so each
// output is the single-matrix kernel's to the bit (the same steps and waves
// for one K, and a reduction tree that does not depend on the row count).
// The activation pointer, the step counts and the table of first workgroups
// arrive in preloaded argument SGPRs; a workgroup's matrix descriptor is one
// scalar load.
struct W4GroupMat {
    const uint32_t* w;
    const uint32_t* szr;
    float* y;
    int rows;
    int wg0;
};

struct W4GroupArgs {
    int wg0[ZT_GROUP_MAX];  // first workgroup of matrix i (wg0[0] = 0); entries past n hold the grid size
    int n;
    int pad[3];
    W4GroupMat mat[ZT_GROUP_MAX];
};

template <int S, int R>
__global__ void __launch_bounds__(1024) w4a16sz_group_kernel(const uint16_t* __restrict__ x, int nchunk, int ngroups,
                                                             float inv_cpg, const W4GroupArgs g) {
    __shared__ float red[16 * R];
    const int b = blockIdx.x;
    // entries past the last matrix hold the grid size, which no workgroup id reaches,
    // so the lookup needs only the table (argument dwords 6-13, preloaded)
    int m = 0;
#pragma unroll
    for (int i = 1; i < ZT_GROUP_MAX; i++) m += b >= g.wg0[i] ? 1 : 0;
    const W4GroupMat d = g.mat[m];
    w4a16_steps_body<S, R, true>(d.w, d.szr, nullptr, x, d.y, d.rows, nchunk, ngroups, inv_cpg, (b - d.wg0) * R, red);
}

template <int S>
static void launch_w4a16sz_group(int R, dim3 g, dim3 b, hipStream_t st, const uint16_t* x, int nchunk, int ngroups,
                                 float inv, const W4GroupArgs& a) {
    switch (R) {
        case 8: w4a16sz_group_kernel<S, 8><<<g, b, 0, st>>>(x, nchunk, ngroups, inv, a); break;
        case 4: w4a16sz_group_kernel<S, 4><<<g, b, 0, st>>>(x, nchunk, ngroups, inv, a); break;
        case 2: w4a16sz_group_kernel<S, 2><<<g, b, 0, st>>>(x, nchunk, ngroups, inv, a); break;
        default: w4a16sz_group_kernel<S, 1><<<g, b, 0, st>>>(x, nchunk, ngroups, inv, a); break;
    }
}

template <int S, bool SZ>
static void launch_w4a16_steps(int R, dim3 g, dim3 b, hipStream_t st, const uint32_t* w, const uint16_t* s,
                               const uint16_t* z, const uint32_t* szr, const uint16_t* x, float* y, int rows,
                               int nchunk, int cpg) {
    const void* meta = SZ ? static_cast<const void*>(szr) : static_cast<const void*>(s);
    const int ngroups = nchunk / cpg;
    const float inv = 1.0f / (float)cpg;
    switch (R) {
        case 8: w4a16_steps_kernel<S, 8, SZ><<<g, b, 0, st>>>(w, meta, z, x, y, rows, nchunk, ngroups, inv); break;
        case 4: w4a16_steps_kernel<S, 4, SZ><<<g, b, 0, st>>>(w, meta, z, x, y, rows, nchunk, ngroups, inv); break;
        case 2: w4a16_steps_kernel<S, 2, SZ><<<g, b, 0, st>>>(w, meta, z, x, y, rows, nchunk, ngroups, inv); break;
        default: w4a16_steps_kernel<S, 1, SZ><<<g, b, 0, st>>>(w, meta, z, x, y, rows, nchunk, ngroups, inv); break;
    }
}

// Rows per wave of the batch-1 steps kernel.
static int w4a16_steps_rows(int M, int nw) {
    // about 4096 waves, but at least 4 rows a wave where 2048 waves allow it: 8 rows from 4096 rows at
    // K = 4096 (3.98 against 4.16 us with 4 rows at 4096 x 4096 on packed scales; 24.4 against 27.0 us at
    // 28672 x 8192 rows x K), 4 rows at 1024 x 8192 (3.18 us, against 3.37 with 2 and 3.85 with 8)
    return max(pick_rows_per_wave(M, nw, 1, 4096), min(4, pick_rows_per_wave(M, nw, 1, 2048)));
}

// Packs (scale, zero) into one dword per (row, group), row-major.
__global__ void w4_szr_kernel(const uint16_t* __restrict__ scales, const uint16_t* __restrict__ zeros,
                              uint32_t* __restrict__ szr, long n) {
    const long e = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= n) return;
    const uint16_t z = zeros ? zeros[e] : (uint16_t)0x4800;  // fp16 8.0
    szr[e] = (uint32_t)scales[e] | ((uint32_t)z << 16);
}

// ------------------------------------------------------------ row-block GEMM
//
// Batches of N = 4 or 8 on the row-major layout in one launch
// (v_mfma_f32_4x4x4_16b_f16; lane roles, activation staging and the
// reductions: zt_rbmfma.h).  A workgroup of nw waves owns 4R rows (R sets
// of 4) over all of K; wave w takes steps w S .. w S + S - 1 (16 chunks of
// 32 K each).  Every weight and (scale, zero) load of the wave's S steps is
// issued up front, right after the first step's activation loads.
//  * B operand of step s (0-7) of a lane's 16-byte chunk: the nibble pairs
//    (e_m, e_m+4) of dword s/2, m = 2(s%2) and 2(s%2) + 1, K order
//    8(s/2) + 2(s%2) + {0, 4, 1, 5}, each moved to mantissa bits 6-9 of
//    the fp16 0x7400 = 2^14: b = 2^14 + 2^10 q exactly (a shift and an
//    and-or a dword).  The MFMA products x b are exact in fp32.  (fp16
//    subnormal weights, q 2^-24, would be one op cheaper, but products of
//    that size come out of the gfx950 MFMAs about 100 ulp low on average,
//    measured against fp64 sums; normal-range operands come out within
//    0.2 ulp.)
//  * a chunk lies in one group (group % 32 == 0), so its 8 MFMAs start from
//    zero.  With X = sum(x b) and X1 = sum(x 2^14) (8 MFMAs with B = 2^14,
//    per chunk and column), sum((q - z) x) s = (s 2^-10) X - (s (16 + z)
//    2^-14) X1: two FMAs per output and chunk, exact for any fp16 zero.
//  * the activation block of a step is read back as 8 A operands per n-set
//    (ds_read_b64_tr_b16), which every row set of the step shares.
// B operand of one MFMA step from a weight dword q: nibbles m and m + 1
// (m = 2 odd) of each half moved to mantissa bits 6-9 under the exponent of
// 2^14, two VALU ops a dword: a shift and v_and_or_b32, which the caller
// enables by holding the mask in a VGPR and the exponent in an SGPR (two
// literal constants do not fit one VOP3 instruction).
__device__ __forceinline__ half4v rb_w4_operand(uint32_t q, int odd, uint32_t mask, uint32_t expo) {
    const uint32_t lo = odd ? q >> 2 : q << 6, hi = odd ? q >> 6 : q << 2;
    return __builtin_bit_cast(half4v, (uint2){(lo & mask) | expo, (hi & mask) | expo});
}

// SZ: meta is the packed (scale | zero << 16) dwords of zt_w4a16_pack_szr;
// else meta is the fp16 scales and zeros the fp16 zeros (NULL: 8).
// Threads a workgroup may have: 4 row sets of 8 columns at two or four steps
// a wave run at most 8 waves (the launch shape keeps them there), so 512
// threads leave them up to 256 VGPRs (the 1024-thread bound spills the
// two-step form); everything else may take 16 waves.
constexpr int w4rb_bound(int NB, int R, int S) { return (NB == 2 && R == 4 && S >= 2) || (NB > 2 && R > 1) ? 512 : 1024; }

template <int NB, int R, int S, bool SZ>
__global__ void __launch_bounds__(w4rb_bound(NB, R, S)) w4a16_rb_kernel(const uint32_t* __restrict__ packed,
                                                        const void* __restrict__ meta,
                                                        const uint16_t* __restrict__ zeros,
                                                        const uint16_t* __restrict__ x, float* __restrict__ y,
                                                        int rows, int nchunk, int ngroups, float inv_cpg) {
    using Lay = RbLayout<NB>;
    constexpr int N = Lay::N, V = 4 * R * NB;
    extern __shared__ __attribute__((aligned(16))) char smem[];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    const int blk = lane >> 2, j = lane & 3;
    char* xs = smem + wave * Lay::STEP;
    const int row0 = blockIdx.x * 4 * R;
    // rows past M read zeros: the buffers end at row M
    const __amdgpu_buffer_rsrc_t rw =
        __builtin_amdgcn_make_buffer_rsrc((void*)packed, (short)0, rows * nchunk * 16, 0x00020000);
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc((void*)meta, (short)0, rows * ngroups * (SZ ? 4 : 2), 0x00020000);
    const __amdgpu_buffer_rsrc_t rz =
        __builtin_amdgcn_make_buffer_rsrc((void*)zeros, (short)0, zeros ? rows * ngroups * 2 : 0, 0x00020000);
    const __amdgpu_buffer_rsrc_t rx =
        __builtin_amdgcn_make_buffer_rsrc((void*)x, (short)0, nchunk * 64 * N, 0x00020000);
    const int step0 = wave * S;
    rb_stage_x<NB>(rx, xs, (uint32_t)step0 * Lay::STEP, lane);
    __builtin_amdgcn_sched_barrier(0);
    u32x4 w[S][R];
    uint32_t sc[S][R], zr[S][R];
    const uint32_t wrow = (uint32_t)(row0 + j) * (uint32_t)nchunk * 16u, wstep = 4u * (uint32_t)nchunk * 16u;
    const uint32_t srow = (uint32_t)(row0 + j) * (uint32_t)ngroups * (SZ ? 4u : 2u),
                   sstep = 4u * (uint32_t)ngroups * (SZ ? 4u : 2u);
#pragma unroll
    for (int t = 0; t < S; t++) {
        const int c = (step0 + t) * 16 + blk;
        const bool ok = c < nchunk;
        const uint32_t g = (uint32_t)(((float)c + 0.5f) * inv_cpg);
        const uint32_t wo = ok ? wrow + (uint32_t)c * 16u : 0x80000000u;
        const uint32_t so = ok ? srow + g * (SZ ? 4u : 2u) : 0x80000000u;
#pragma unroll
        for (int r = 0; r < R; r++) {
            w[t][r] = __builtin_amdgcn_raw_buffer_load_b128(rw, wo + r * wstep, 0, 2);  // nontemporal
            if (SZ) {
                sc[t][r] = __builtin_amdgcn_raw_buffer_load_b32(rs, so + r * sstep, 0, 0);
            } else {
                sc[t][r] = __builtin_amdgcn_raw_buffer_load_b16(rs, so + r * sstep, 0, 0);
                zr[t][r] = __builtin_amdgcn_raw_buffer_load_b16(rz, so + r * sstep, 0, 0);
            }
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    float acc[V];
#pragma unroll
    for (int i = 0; i < V; i++) acc[i] = 0.0f;
    const half4v ones = (half4v){16384, 16384, 16384, 16384};  // 2^14
    uint32_t bmask = 0x03C003C0u, bexp = 0x74007400u;
    asm volatile("" : "+v"(bmask), "+s"(bexp));  // the mask in a VGPR, the exponent in an SGPR
#pragma unroll
    for (int t = 0; t < S; t++) {
        if (t > 0) {
            // every read of the previous step's activations has returned before the
            // direct loads overwrite them (the compiler would otherwise sink some reads
            // past the loads, which it does not see as writes to the same LDS)
            __builtin_amdgcn_sched_barrier(0);
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            __builtin_amdgcn_sched_barrier(0);
            rb_stage_x<NB>(rx, xs, (uint32_t)(step0 + t) * Lay::STEP, lane);
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        } else {
            // wait for the activations only: the S R weight and S R (2 S R) scale loads issued after them may
            // still be outstanding
            asm volatile("s_waitcnt vmcnt(%0)" ::"n"(SZ ? 2 * S * R : 3 * S * R) : "memory");
        }
        half4v xa[NB][8];
        float4v dx[NB];
#pragma unroll
        for (int js = 0; js < NB; js++) {
            dx[js] = (float4v){0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int s = 0; s < 8; s++) xa[js][s] = rb_tr_read(xs, rb_tr_offset<NB>(lane, s, js));
#pragma unroll
            for (int s = 0; s < 8; s++) dx[js] = __builtin_amdgcn_mfma_f32_4x4x4f16(xa[js][s], ones, dx[js], 0, 0, 0);
        }
        // MFMA step outer, row set inner, in batches of RC row sets: the RC x NB
        // accumulation chains of a batch interleave
        constexpr int RC = R < 4 / NB ? R : 4 / NB;
#pragma unroll
        for (int r0 = 0; r0 < R; r0 += RC) {
            float4v d[RC][NB];
#pragma unroll
            for (int r = 0; r < RC; r++)
#pragma unroll
                for (int js = 0; js < NB; js++) d[r][js] = (float4v){0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int s = 0; s < 8; s++) {
#pragma unroll
                for (int r = 0; r < RC; r++) {
                    const u32x4& wv = w[t][r0 + r];
                    const uint32_t q = (s >> 1) == 0 ? wv.x : (s >> 1) == 1 ? wv.y : (s >> 1) == 2 ? wv.z : wv.w;
                    const half4v bv = rb_w4_operand(q, s & 1, bmask, bexp);
#pragma unroll
                    for (int js = 0; js < NB; js++)
                        d[r][js] = __builtin_amdgcn_mfma_f32_4x4x4f16(xa[js][s], bv, d[r][js], 0, 0, 0);
                }
            }
#pragma unroll
            for (int r = 0; r < RC; r++) {
                const half2v szh = as_h2(sc[t][r0 + r]);
                const float sv = (float)szh.x;
                const float zv = SZ ? (float)szh.y : zeros ? (float)as_h2(zr[t][r0 + r]).x : 8.0f;
                const float sa = sv * 0x1p-10f, sz = sv * (16.0f + zv) * 0x1p-14f;
#pragma unroll
                for (int js = 0; js < NB; js++)
#pragma unroll
                    for (int v = 0; v < 4; v++) {
                        float& a = acc[((r0 + r) * NB + js) * 4 + v];
                        a = __builtin_fmaf(sa, d[r][js][v], __builtin_fmaf(-sz, dx[js][v], a));
                    }
            }
        }
    }
    // waves split K: each wave leaves its sums in its own LDS region, then the
    // workgroup adds them in wave order
    rb_finish<NB, R>(acc, smem, Lay::STEP, xs, y, row0, rows);
}

template <int NB, int R, int S, bool SZ>
static void launch_w4a16_rb_t(dim3 g, int nw, hipStream_t st, const uint32_t* w, const void* meta,
                              const uint16_t* z, const uint16_t* x, float* y, int rows, int nchunk, int cpg) {
    const size_t lds = (size_t)nw * RbLayout<NB>::STEP;
    if (lds > 65536) {  // past the default dynamic LDS limit (gfx950 has 160 KB a CU)
        static const bool raised = [] {
            return hipFuncSetAttribute(reinterpret_cast<const void*>(&w4a16_rb_kernel<NB, R, S, SZ>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024) == hipSuccess;
        }();
        (void)raised;
    }
    w4a16_rb_kernel<NB, R, S, SZ><<<g, nw * kWave, lds, st>>>(w, meta, z, x, y, rows, nchunk, nchunk / cpg,
                                                               1.0f / (float)cpg);
}

template <int NB, bool SZ>
static void launch_w4a16_rb_n(int R, int S, dim3 g, int nw, hipStream_t st, const uint32_t* w, const void* meta,
                              const uint16_t* z, const uint16_t* x, float* y, int rows, int nchunk, int cpg) {
#define ZT_RB(RR, SS) \
    if (R == RR && S == SS) return launch_w4a16_rb_t<NB, RR, SS, SZ>(g, nw, st, w, meta, z, x, y, rows, nchunk, cpg);
    if constexpr (NB <= 2) {
        ZT_RB(1, 1) ZT_RB(2, 1) ZT_RB(4, 1)
        ZT_RB(1, 2) ZT_RB(2, 2) ZT_RB(4, 2)
        ZT_RB(1, 4) ZT_RB(2, 4)
    }
    if constexpr (NB == 2) {
        ZT_RB(4, 4)
    } else if constexpr (NB > 2) {
        ZT_RB(1, 1) ZT_RB(1, 2) ZT_RB(2, 1) ZT_RB(2, 2) ZT_RB(4, 1) ZT_RB(4, 2)
    }
#undef ZT_RB
}

// Launch shape of the row-block GEMM: S steps a wave and up to 16 waves
// splitting K (8 for N >= 8: 8-column activation blocks take 8 KB of LDS a
// wave, so 8 waves let two or more workgroups share a CU; N >= 12 also caps
// VGPRs), and R row sets a workgroup (up to 4) doubled while about 256
// workgroups remain.  Measured on the packed-scale
// kernel (us, default against the former >= 512 workgroups and 16 waves at
// N = 8): batch 8 4096 x 14336 (rows x K) 12.18 against 15.20, 28672 x
// 8192 37.97 against 42.83, 8192 x 8192 13.16 against 13.68, 4096 x 4096
// 4.92 against 5.45; batch 4 4096 x 14336 9.97 against 10.38, 4096 x 4096
// 4.38 against 4.31.  8 row sets were slower wherever the grid allows them.
static void w4a16_rb_shape(int M, int N, int nchunk, int& R, int& S, int& nw) {
    const int steps = ceil_div(nchunk, 16), wmax = N >= 8 ? 8 : 16;
    S = steps <= wmax ? 1 : steps <= 2 * wmax ? 2 : 4;
    nw = ceil_div(steps, S);
    // four steps a wave on more than 8 waves (N = 8: K > 16384) keeps 2 row
    // sets: 4 need the 512-thread bound.  N >= 12 runs at most 8 waves, so its
    // 2 and 4 row sets take the 512-thread bound too (us, batch 16, 1 / 2 / 4
    // row sets: 4096 x 4096 12.9 / 8.4 / 6.4, 14336 x 4096 42.1 / 26.0 / 20.6,
    // 28672 x 8192 123.7 / 84.9 / 63.4)
    const int rmax = (S == 4 && (nw > 8 || N == 4)) ? 2 : 4;
    R = 1;
    while (R < rmax && ceil_div(M, 8 * R) >= 256) R *= 2;
    // few rows (one row set a workgroup) and K of 16 steps or more: two steps a
    // wave on half the waves (1024 x 8192, batch 4 / 8: 3.56 / 4.06 us against
    // 3.73 / 4.74 at one step on 16 waves)
    if (R == 1 && S == 1 && steps >= 16 && N <= 8) {
        S = 2;
        nw = ceil_div(steps, 2);
    }
}

// Shapes the row-block GEMM takes: N % 4 == 0 up to 16, K <= 32768 (N >= 12:
// K <= 8192, two steps of 8 waves), 32-bit buffer offsets.
static bool w4a16_rb_ok(int N, int nchunk, long M) {
    if (N < 4 || N > 16 || N % 4 != 0 || M * nchunk * 16 >= 0x7fffffffL) return false;
    return nchunk <= (N >= 12 ? 8 * 16 * 2 : 16 * 16 * 4);
}

template <bool SZ>
static int launch_w4a16_rb(const uint32_t* w, const void* meta, const uint16_t* z, const uint16_t* x, float* y,
                           int M, int K, int N, int group_size, hipStream_t st) {
    const int nchunk = K / 32;
    int R, S, nw;
    w4a16_rb_shape(M, N, nchunk, R, S, nw);
    const dim3 g(ceil_div(M, 4 * R));
    switch (N) {
        case 4: launch_w4a16_rb_n<1, SZ>(R, S, g, nw, st, w, meta, z, x, y, M, nchunk, group_size / 32); break;
        case 8: launch_w4a16_rb_n<2, SZ>(R, S, g, nw, st, w, meta, z, x, y, M, nchunk, group_size / 32); break;
        case 12: launch_w4a16_rb_n<3, SZ>(R, S, g, nw, st, w, meta, z, x, y, M, nchunk, group_size / 32); break;
        default: launch_w4a16_rb_n<4, SZ>(R, S, g, nw, st, w, meta, z, x, y, M, nchunk, group_size / 32); break;
    }
    return (int)hipGetLastError();
}

// ------------------------------------------------------------ MFMA GEMM
//
// C[rows, N] = W[rows, K] x X[K, N] for 4 <= N <= 16, N % 4 == 0, K and the
// group size multiples of 128 (workgroup structure, X staging and the
// transposing B reads: zt_mfma.h).
//  * Wave w of the workgroup takes the 128-K units w and w+8 of each chunk.
//    For a unit, lane (i = lane%16, g = lane/16) loads 16 bytes of row i:
//    the 32 weights 32g .. 32g+31 of the unit.  Dword s of that load feeds
//    MFMA step s: its nibble pairs (m, m+4) become exact fp16 with
//    (0x6400 | q) - 1024, ordered [e0,e4,e1,e5,e2,e6,e3,e7], and the B
//    reads take X rows k0 + {0,4,1,5} and k0 + {2,6,3,7} to match.
//  * A third MFMA per step with an all-ones A gives sum_k x[k][n] for the
//    unit, so y += s * (sum_k q x - z * sum_k x) is exact for any fp16 zero
//    (one scale and zero per unit since the group size is a multiple of 128).
__device__ __forceinline__ half8v w4_a_operand(uint32_t d) {
    half8v a;
#pragma unroll
    for (int m = 0; m < 4; m++) {
        const half2v h = nib_pair(d >> (4 * m));  // (e_m, e_{m+4}), exact
        a[2 * m] = h.x;
        a[2 * m + 1] = h.y;
    }
    return a;
}

__global__ void __launch_bounds__(512) w4a16_mfma_kernel(const uint8_t* __restrict__ packed,
                                                         const uint16_t* __restrict__ scales,
                                                         const uint16_t* __restrict__ zeros,
                                                         const uint16_t* __restrict__ x, float* __restrict__ y,
                                                         int rows, int K, int N, int gs) {
    constexpr int NT = kMfmaTiles;
    extern __shared__ __attribute__((aligned(16))) char smem[];
    const int xbytes = mfma_xbytes(N);
    char* zero_area = smem + xbytes;
    uint16_t* ss = reinterpret_cast<uint16_t*>(zero_area + 16);
    uint16_t* zs = ss + kMfmaUC * kMfmaRows;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int li = lane & 15, lg = lane >> 4;
    const int row0 = blockIdx.x * kMfmaRows;
    const int nunits = K / 128;
    const int ngroups = K / gs;
    const long rowbytes = K / 2;
    if (tid < 4) reinterpret_cast<uint32_t*>(zero_area)[tid] = 0u;

    float4v acc[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) acc[t] = (float4v){0.f, 0.f, 0.f, 0.f};
    int arow[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) arow[t] = min(row0 + 16 * t + li, rows - 1);
    const MfmaBRole ro(li, N);
    const int offa = (ro.jq == 0) ? 0 : (ro.jq == 1) ? 4 : (ro.jq == 2) ? 1 : 5;  // rows {0,4,1,5}
    const int offb = offa + 2;                                                      // rows {2,6,3,7}
    const half8v ones = (half8v){1, 1, 1, 1, 1, 1, 1, 1};

    const int ub = 0, ue = nunits;
    // Weights of the next chunk are loaded while the current chunk computes.
    uint4 wn[kMfmaUPW][NT];
    auto load_w = [&](int c0) {
#pragma unroll
        for (int u = 0; u < kMfmaUPW; u++) {
            const int unit = min(c0 + wave + kMfmaWaves * u, ue - 1);
#pragma unroll
            for (int t = 0; t < NT; t++)
                wn[u][t] =
                    ld_stream(reinterpret_cast<const uint4*>(packed + (long)arow[t] * rowbytes + unit * 64 + 16 * lg));
        }
    };
    if (ub < ue) load_w(ub);
    for (int c0 = ub; c0 < ue; c0 += kMfmaUC) {
        uint4 w[kMfmaUPW][NT];
#pragma unroll
        for (int u = 0; u < kMfmaUPW; u++)
#pragma unroll
            for (int t = 0; t < NT; t++) w[u][t] = wn[u][t];
        mfma_stage_x(smem, x, c0, ue * 128, N);
        for (int e = tid; e < kMfmaUC * kMfmaRows; e += blockDim.x) {
            const int uu = e / kMfmaRows, r = e % kMfmaRows;
            if (c0 + uu < ue) {
                const long gi = (long)min(row0 + r, rows - 1) * ngroups + ((c0 + uu) * 128) / gs;
                ss[e] = scales[gi];
                zs[e] = zeros ? zeros[gi] : (uint16_t)0x4800;  // fp16 8.0
            }
        }
        __syncthreads();
        if (c0 + kMfmaUC < ue) load_w(c0 + kMfmaUC);
#pragma unroll
        for (int u = 0; u < kMfmaUPW; u++) {
            const int uu = wave + kMfmaWaves * u;
            if (c0 + uu < ue) {
                float4v d[NT], dn = (float4v){0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int t = 0; t < NT; t++) d[t] = (float4v){0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int s = 0; s < 4; s++) {
                    const half8v bv = mfma_b_operand(smem, ro, uu * 128 + 32 * lg + 8 * s, offa, offb, N, xbytes);
#pragma unroll
                    for (int t = 0; t < NT; t++) {
                        const uint32_t dw = s == 0 ? w[u][t].x : s == 1 ? w[u][t].y : s == 2 ? w[u][t].z : w[u][t].w;
                        d[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(w4_a_operand(dw), bv, d[t], 0, 0, 0);
                    }
                    dn = __builtin_amdgcn_mfma_f32_16x16x32_f16(ones, bv, dn, 0, 0, 0);
                }
#pragma unroll
                for (int t = 0; t < NT; t++) {
                    const int rb0 = uu * kMfmaRows + 16 * t + 4 * lg;
                    const uint2 s4 = *reinterpret_cast<const uint2*>(ss + rb0);
                    const uint2 z4 = *reinterpret_cast<const uint2*>(zs + rb0);
                    const uint16_t sv[4] = {(uint16_t)(s4.x & 0xffff), (uint16_t)(s4.x >> 16),
                                            (uint16_t)(s4.y & 0xffff), (uint16_t)(s4.y >> 16)};
                    const uint16_t zv[4] = {(uint16_t)(z4.x & 0xffff), (uint16_t)(z4.x >> 16),
                                            (uint16_t)(z4.y & 0xffff), (uint16_t)(z4.y >> 16)};
#pragma unroll
                    for (int i = 0; i < 4; i++)
                        acc[t][i] = fmaf(h2f(sv[i]), fmaf(-h2f(zv[i]), dn[i], d[t][i]), acc[t][i]);
                }
            }
        }
        __syncthreads();
    }
    mfma_reduce_store(acc, smem, y, row0, rows, N);
}

static size_t w4_mfma_lds_bytes(int N) {
    const size_t stage = (size_t)mfma_xbytes(N) + 16 + 2 * kMfmaUC * kMfmaRows * sizeof(uint16_t);
    return stage > mfma_reduce_bytes() ? stage : mfma_reduce_bytes();
}

// ------------------------------------------------------------ dequantize

// One thread per 32-weight chunk; bit-exact with GPTQStorage.Dequantize.
// OutT = uint16_t writes the fp32 value rounded to fp16 (round to nearest,
// ties to even: v_cvt_f16_f32 in the default mode), DequantW4ToFP16's
// Slice-then-FromFloat32 (compute/w4a16.go:170-175).
template <class OutT>
__global__ void w4_dequant_kernel(const uint4* __restrict__ packed, const uint16_t* __restrict__ scales,
                                  const uint16_t* __restrict__ zeros, OutT* __restrict__ out, long nchunk,
                                  int chunks_per_group) {
    const long c = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= nchunk) return;
    const long g = c / chunks_per_group;
    const float s = h2f(scales[g]);
    const float z = zeros ? h2f(zeros[g]) : 8.0f;
    const uint4 w = packed[c];
    const uint32_t d[4] = {w.x, w.y, w.z, w.w};
    OutT* o = out + c * 32;
#pragma unroll
    for (int i = 0; i < 32; i++) {
        const int q = (int)((d[i / 8] >> (4 * (i % 8))) & 0xfu);
        o[i] = out_cvt<OutT>(((float)q - z) * s);
    }
}

}  // namespace zt

using namespace zt;

ZT_EXPORT int zt_gemm_w4a16_f32(const void* W_packed, const uint16_t* scales, const uint16_t* zeros,
                                const uint16_t* B, float* C, int M, int K, int N, int group_size,
                                hipStream_t stream) {
    if (M < 0 || N < 0 || K < 0 || group_size <= 0 || group_size % 32 != 0 || K % group_size != 0 || N > 65535)
        return (int)hipErrorInvalidValue;
    if (M == 0 || N == 0) return (int)hipSuccess;
    if (C == nullptr) return (int)hipErrorInvalidValue;
    if (K == 0) {  // empty sums
        mfma_zero(C, (long)M * N, stream);
        return (int)hipGetLastError();
    }
    if (W_packed == nullptr || scales == nullptr || B == nullptr) return (int)hipErrorInvalidValue;
    if (((uintptr_t)W_packed & 15) || ((uintptr_t)scales & 1) || ((uintptr_t)zeros & 1))
        return (int)hipErrorInvalidValue;
    if (N == 1 && ((uintptr_t)B & 15)) return (int)hipErrorInvalidValue;
    // N = 4, 8 (and 12, 16 on up to 4096 rows, where the 32-row workgroups below would leave most
    // CUs idle: 4.3 against 9.7 us at 1024 x 4096, batch 16, and 6.4 against 9.9 at 4096 x 4096;
    // past that the 16x16x32 kernel is faster, 15.2 against 20.6 us at 14336 x 4096)
    if (w4a16_rb_ok(N, K / 32, M) && ((uintptr_t)B & 15) == 0 && (N <= 8 || M <= 4096))
        return launch_w4a16_rb<false>(static_cast<const uint32_t*>(W_packed), scales, zeros, B, C, M, K, N,
                                      group_size, stream);
    if (mfma_shape_ok(N, K, B) && group_size % 128 == 0) {
        // N = 12 or 16: one workgroup per 32 rows over all of K, so every output is written once
        // (no K split, no atomics)
        w4a16_mfma_kernel<<<dim3(ceil_div(M, kMfmaRows)), kMfmaWaves * kWave, w4_mfma_lds_bytes(N), stream>>>(
            static_cast<const uint8_t*>(W_packed), scales, zeros, B, C, M, K, N, group_size);
        return (int)hipGetLastError();
    }
    const int nchunk = K / 32;
    if (N == 1) {
        if ((long)M * nchunk * 16 < 0x7fffffffL && nchunk <= 512) {
            // fixed steps: S = 1 for K <= 4096, else 2 with up to 16 waves
            const int S = nchunk <= 128 ? 1 : 2;
            int nw = ceil_div(nchunk, 16 * S);
            if (nw > 12) nw = 16;  // whole SIMD sets: 14 waves measured slower than 16
            const int R = w4a16_steps_rows(M, nw);
            const dim3 g(ceil_div(M, R)), b(nw * kWave);
            const uint32_t* w = static_cast<const uint32_t*>(W_packed);
            if (S == 1)
                launch_w4a16_steps<1, false>(R, g, b, stream, w, scales, zeros, nullptr, B, C, M, nchunk,
                                             group_size / 32);
            else
                launch_w4a16_steps<2, false>(R, g, b, stream, w, scales, zeros, nullptr, B, C, M, nchunk,
                                             group_size / 32);
            return (int)hipGetLastError();
        }
        const int nw = min(8, ceil_div(nchunk, 16));
        const int R = pick_rows_per_wave(M, nw, 1, 2048);
        launch_w4a16_quad(R, dim3(ceil_div(M, R)), dim3(nw * kWave), stream, static_cast<const uint32_t*>(W_packed),
                          scales, zeros, B, C, M, nchunk, group_size / 32);
        return (int)hipGetLastError();
    }
    const int nwaves = nchunk <= 64 ? 1 : (nchunk >= 8 * 64 ? 8 : ceil_div(nchunk, 64));
    const int R = pick_rows_per_wave(M, nwaves, N, 2048);
    dim3 grid(ceil_div(M, R), N), block(nwaves * kWave);
    launch_w4a16_gemv<false>(R, grid, block, stream, static_cast<const uint4*>(W_packed), scales, zeros, B, C, N, M,
                             nchunk, group_size / 32);
    return (int)hipGetLastError();
}

ZT_EXPORT int zt_w4a16_pack_szr(const uint16_t* scales, const uint16_t* zeros, int M, int K, int group_size,
                                uint32_t* szr, hipStream_t stream) {
    if (M < 0 || K < 0 || group_size <= 0 || group_size % 32 != 0 || K % group_size != 0)
        return (int)hipErrorInvalidValue;
    if (M == 0 || K == 0) return (int)hipSuccess;
    if (scales == nullptr || szr == nullptr) return (int)hipErrorInvalidValue;
    if (((uintptr_t)scales & 1) || ((uintptr_t)zeros & 1) || ((uintptr_t)szr & 3)) return (int)hipErrorInvalidValue;
    const long n = (long)M * (K / group_size);
    w4_szr_kernel<<<ceil_div(n, 256), 256, 0, stream>>>(scales, zeros, szr, n);
    return (int)hipGetLastError();
}

// Steps a wave and waves of the batch-1 kernel on packed scales, for K / 32 chunks.
static void w4a16sz_steps_shape(int nchunk, int& S, int& nw) {
    S = nchunk <= 128 ? 1 : nchunk <= 256 ? 2 : 4;
    nw = ceil_div(nchunk, 16 * S);
    // whole SIMD sets: 14 waves measured 3% (K = 14336) to 30% (K = 28672) slower than 16
    if (nw > 12)
        nw = 16;
    else if (S == 4)
        nw = (nw + 3) & ~3;
}

ZT_EXPORT int zt_gemv_w4a16sz_f32(const void* W_packed, const uint32_t* szr, const uint16_t* x, float* y, int M,
                                  int K, int group_size, hipStream_t stream) {
    if (M < 0 || K < 0 || group_size <= 0 || group_size % 32 != 0 || K % group_size != 0)
        return (int)hipErrorInvalidValue;
    if (M == 0) return (int)hipSuccess;
    if (y == nullptr) return (int)hipErrorInvalidValue;
    if (K == 0) {  // empty sums (a fill kernel, not a memset node, so the call can be graph-captured)
        mfma_zero(y, M, stream);
        return (int)hipGetLastError();
    }
    if (W_packed == nullptr || szr == nullptr || x == nullptr) return (int)hipErrorInvalidValue;
    if (((uintptr_t)W_packed & 15) || ((uintptr_t)szr & 3) || ((uintptr_t)x & 15)) return (int)hipErrorInvalidValue;
    const int nchunk = K / 32;
    // 32-bit buffer offsets; at most 16 waves of 4 steps
    if ((long)M * nchunk * 16 >= 0x7fffffffL || nchunk > 1024) return (int)hipErrorInvalidValue;
    int S, nw;
    w4a16sz_steps_shape(nchunk, S, nw);
    const int R = w4a16_steps_rows(M, nw);
    const dim3 g(ceil_div(M, R)), b(nw * kWave);
    const uint32_t* w = static_cast<const uint32_t*>(W_packed);
    const int cpg = group_size / 32;
    if (S == 1)
        launch_w4a16_steps<1, true>(R, g, b, stream, w, nullptr, nullptr, szr, x, y, M, nchunk, cpg);
    else if (S == 2)
        launch_w4a16_steps<2, true>(R, g, b, stream, w, nullptr, nullptr, szr, x, y, M, nchunk, cpg);
    else
        launch_w4a16_steps<4, true>(R, g, b, stream, w, nullptr, nullptr, szr, x, y, M, nchunk, cpg);
    return (int)hipGetLastError();
}

ZT_EXPORT int zt_gemv_w4a16sz_group_f32(const zt_w4a16_gemv_desc* descs, int n, const uint16_t* x, int K,
                                        int group_size, hipStream_t stream) {
    if (descs == nullptr || n < 1 || n > ZT_GROUP_MAX || K < 0 || group_size <= 0 || group_size % 32 != 0 ||
        K % group_size != 0)
        return (int)hipErrorInvalidValue;
    long total = 0;
    bool fits = true;
    const int nchunk = K / 32;
    for (int i = 0; i < n; i++) {
        const zt_w4a16_gemv_desc& d = descs[i];
        if (d.rows < 0 || d.reserved != 0) return (int)hipErrorInvalidValue;
        if (d.rows == 0) continue;
        if (d.y == nullptr) return (int)hipErrorInvalidValue;
        if (K > 0 && (d.W == nullptr || d.szr == nullptr || ((uintptr_t)d.W & 15) || ((uintptr_t)d.szr & 3)))
            return (int)hipErrorInvalidValue;
        total += d.rows;
        fits = fits && (long)d.rows * nchunk * 16 < 0x7fffffffL;
    }
    if (total == 0) return (int)hipSuccess;
    if (K > 0 && (x == nullptr || ((uintptr_t)x & 15))) return (int)hipErrorInvalidValue;
    if (K == 0 || !fits || nchunk > 1024) {
        // empty sums, or shapes past the kernel's 32-bit offsets: one call per matrix
        for (int i = 0; i < n; i++) {
            const zt_w4a16_gemv_desc& d = descs[i];
            if (d.rows == 0) continue;
            const int rc = zt_gemv_w4a16sz_f32(d.W, d.szr, x, d.y, d.rows, K, group_size, stream);
            if (rc != 0) return rc;
        }
        return (int)hipSuccess;
    }
    int S, nw;
    w4a16sz_steps_shape(nchunk, S, nw);
    // rows a wave from the group's total rows, as for one matrix of that many rows
    const int R = w4a16_steps_rows((int)min(total, 0x7fffffffL), nw);
    W4GroupArgs a{};
    int wg = 0, m = 0;
    for (int i = 0; i < n; i++) {
        const zt_w4a16_gemv_desc& d = descs[i];
        if (d.rows == 0) continue;
        a.wg0[m] = wg;
        a.mat[m] = W4GroupMat{static_cast<const uint32_t*>(d.W), d.szr, d.y, d.rows, wg};
        wg += ceil_div(d.rows, R);
        m++;
    }
    a.n = m;
    for (int i = m; i < ZT_GROUP_MAX; i++) a.wg0[i] = wg;
    const int cpg = group_size / 32;
    const dim3 g(wg), b(nw * kWave);
    const float inv = 1.0f / (float)cpg;
    if (S == 1)
        launch_w4a16sz_group<1>(R, g, b, stream, x, nchunk, nchunk / cpg, inv, a);
    else if (S == 2)
        launch_w4a16sz_group<2>(R, g, b, stream, x, nchunk, nchunk / cpg, inv, a);
    else
        launch_w4a16sz_group<4>(R, g, b, stream, x, nchunk, nchunk / cpg, inv, a);
    return (int)hipGetLastError();
}

ZT_EXPORT int zt_gemm_w4a16sz_f32(const void* W_packed, const uint32_t* szr, const uint16_t* B, float* C, int M,
                                  int K, int N, int group_size, hipStream_t stream) {
    if (N == 1) return zt_gemv_w4a16sz_f32(W_packed, szr, B, C, M, K, group_size, stream);
    if (M < 0 || K < 0 || group_size <= 0 || group_size % 32 != 0 || K % group_size != 0 || N < 4 || N > 16 ||
        N % 4 != 0)
        return (int)hipErrorInvalidValue;
    if (M == 0) return (int)hipSuccess;
    if (C == nullptr) return (int)hipErrorInvalidValue;
    if (K == 0) {  // empty sums
        mfma_zero(C, (long)M * N, stream);
        return (int)hipGetLastError();
    }
    if (W_packed == nullptr || szr == nullptr || B == nullptr) return (int)hipErrorInvalidValue;
    if (((uintptr_t)W_packed & 15) || ((uintptr_t)szr & 3) || ((uintptr_t)B & 15)) return (int)hipErrorInvalidValue;
    if (!w4a16_rb_ok(N, K / 32, M)) return (int)hipErrorInvalidValue;
    return launch_w4a16_rb<true>(static_cast<const uint32_t*>(W_packed), szr, nullptr, B, C, M, K, N, group_size,
                                 stream);
}

template <class OutT>
static int dequant_w4(const void* W_packed, const uint16_t* scales, const uint16_t* zeros, OutT* out, long nelem,
                      int group_size, hipStream_t stream) {
    if (nelem < 0 || group_size <= 0 || group_size % 32 != 0 || nelem % group_size != 0)
        return (int)hipErrorInvalidValue;
    if (nelem == 0) return (int)hipSuccess;
    if (W_packed == nullptr || scales == nullptr || out == nullptr || ((uintptr_t)W_packed & 15))
        return (int)hipErrorInvalidValue;
    const long nchunk = nelem / 32;
    w4_dequant_kernel<OutT><<<ceil_div(nchunk, 256), 256, 0, stream>>>(static_cast<const uint4*>(W_packed), scales,
                                                                        zeros, out, nchunk, group_size / 32);
    return (int)hipGetLastError();
}

ZT_EXPORT int zt_dequant_w4_f32(const void* W_packed, const uint16_t* scales, const uint16_t* zeros, float* out,
                                long nelem, int group_size, hipStream_t stream) {
    return dequant_w4<float>(W_packed, scales, zeros, out, nelem, group_size, stream);
}

ZT_EXPORT int zt_dequant_w4_f16(const void* W_packed, const uint16_t* scales, const uint16_t* zeros, uint16_t* out,
                                long nelem, int group_size, hipStream_t stream) {
    return dequant_w4<uint16_t>(W_packed, scales, zeros, out, nelem, group_size, stream);
}

// ------------------------------------------------------------ tiled layout
//
// An upload-time repack of the W4A16 weights for the small-batch MFMA GEMM.
// The row-major packed layout puts the 16 rows of an MFMA tile 0.5 K bytes
// apart, so a load instruction in the A-operand lane order (lane = row) reads
// 16 rows x 64 bytes; the tiled layout stores each 16-row x 128-K tile as one
// contiguous 1 KB block in exactly that lane order:
//   tile (rt, u) at byte ((rt * K/128) + u) * 1024; lane l = 16 g + i holds the
//   16 packed bytes of row 16 rt + i, K range 128 u + 32 g .. +32 (the same
//   bytes, in the same nibble order, as the row-major layout);
// rows past M (to the next multiple of 16) are zero.  The group scale and
// zero of (row, group) are packed as one dword, fp16 scale in the low half
// and fp16 zero in the high half (8.0 without a zeros array), laid out
// [group][row] so that a tile's 16 rows are 64 contiguous bytes.  A wave's
// weight load is then one contiguous 1 KB block.

__global__ void w4t_tile_kernel(const uint4* __restrict__ packed, uint4* __restrict__ tiled, int rows, int nunits,
                                long npieces) {
    const long p = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (p >= npieces) return;
    const int lane = (int)(p & 63);
    const long tu = p >> 6;
    const int u = (int)(tu % nunits);
    const long rt = tu / nunits;
    const long row = rt * 16 + (lane & 15);
    uint4 v = make_uint4(0u, 0u, 0u, 0u);
    if (row < rows) v = packed[(row * nunits + u) * 4 + (lane >> 4)];
    tiled[p] = v;
}

__global__ void w4t_sz_kernel(const uint16_t* __restrict__ scales, const uint16_t* __restrict__ zeros,
                              uint32_t* __restrict__ sz, int rows, int ngroups) {
    const long e = (long)blockIdx.x * blockDim.x + threadIdx.x;  // e = group * rows + row
    if (e >= (long)rows * ngroups) return;
    const long g = e / rows, r = e % rows;
    const uint16_t s = scales[r * ngroups + g];
    const uint16_t z = zeros ? zeros[r * ngroups + g] : (uint16_t)0x4800;  // fp16 8.0
    sz[e] = (uint32_t)s | ((uint32_t)z << 16);
}

// Small-batch W4A16 GEMM on the tiled layout (N in {4, 8, 12, 16}, K % 128 == 0,
// group size % 128 == 0).  A workgroup of W waves owns 32 W rows (two 16-row
// tiles a wave) and a K range of UPW 128-K units; K ranges are split across
// workgroups (blockIdx.y), each split stores its partial tiles to the
// caller's workspace and tiled_reduce_kernel sums them in split order.
//  * The X chunk and the workgroup's (scale, zero) dwords are loaded first
//    (coalesced buffer loads), the weights next (each tile one contiguous
//    1 KB load), and X / scales are written to LDS while the weights stream;
//    the barrier waits for LDS only, so each unit computes as soon as its own
//    weights arrive.
//  * A operand: the nibble pairs (e_m, e_m+4) of a dword moved to mantissa
//    bits 6-9 under the exponent of 2^14 (a shift and an and-or a dword):
//    a = 2^14 + 2^10 q exactly, and the MFMA products a x are exact in fp32.
//    (fp16 subnormal weights q 2^-24 with unscaled activations give products
//    that the gfx950 MFMAs sum about 100 ulp low.)  With D = sum(a x) and X1
//    = sum(2^14 x) from an MFMA whose A is all 2^14,
//    y += (s 2^-10) D - (s (16 + z) 2^-14) X1, both factors formed once per
//    (row, unit) in fp32.
//  * Workgroups are mapped XCD-aware: workgroup id mod 8 selects the XCD,
//    and every K range of a row block runs on one XCD, whose L2 then holds
//    the row block's scale lines.
template <int UPW, int W, int N>
__global__ void __launch_bounds__(W * 64) w4a16t_mfma_kernel(const uint4* __restrict__ wt,
                                                             const uint32_t* __restrict__ szp,
                                                             const uint16_t* __restrict__ x, int rows, int K, int gs,
                                                             int nch, int gx, int gy, float* __restrict__ y,
                                                             float* __restrict__ ws) {
    constexpr int KC = 128 * UPW;
    constexpr int RW = 32 * W;
    constexpr int XP = (KC * 2 * N / 16 + W * 64 - 1) / (W * 64);
    constexpr int SP = (UPW * RW + W * 64 - 1) / (W * 64);
    constexpr int XB = mfma_chunk_xbytes(KC, N);
    extern __shared__ __attribute__((aligned(16))) char smem[];
    char* zero_area = smem + XB;
    float2* szs = reinterpret_cast<float2*>(zero_area + 16);
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
    const half8v ones = (half8v){16384, 16384, 16384, 16384, 16384, 16384, 16384, 16384};  // 2^14
    uint32_t bmask = 0x03C003C0u, bexp = 0x74007400u;
    asm volatile("" : "+v"(bmask), "+s"(bexp));  // v_and_or_b32: mask in a VGPR, exponent in an SGPR
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
    const __amdgpu_buffer_rsrc_t rsz = __builtin_amdgcn_make_buffer_rsrc((void*)szp, (short)0, 0x7fffffff, 0x00020000);
    // N = 16: a wave's 64 pieces of 16 bytes are one padded 32-row segment
    // (64 N bytes), so they go to LDS directly (buffer_load ... lds, the
    // lanes' bytes at consecutive 16-byte slots from the segment's base):
    // no registers held and no LDS writes for the activations
    constexpr bool XDMA = N == 16;
    u32x4 xr[XDMA ? 1 : XP];
#pragma unroll
    for (int i = 0; i < XP; i++) {
        if constexpr (XDMA) {
            const int c = wave + i * W;  // segment of this wave's pieces
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rx, (__attribute__((address_space(3))) void*)(smem + c * 68 * N), 16,
                (uint32_t)(tid + i * W * 64) * 16u, 0, 0, 0);
        } else {
            xr[i] = __builtin_amdgcn_raw_buffer_load_b128(rx, (uint32_t)(tid + i * W * 64) * 16u, 0, 0);
        }
    }
    uint32_t sr[SP];
#pragma unroll
    for (int i = 0; i < SP; i++) {
        const int e = tid + i * W * 64, u = e / RW, r = e % RW;
        const bool ok = e < UPW * RW && u0 + u < u1;
        const uint32_t off = ok ? (uint32_t)(((u0 + u) * 128 / gs) * rows + min(rw0 + r, rows - 1)) * 4u : 0x80000000u;
        sr[i] = __builtin_amdgcn_raw_buffer_load_b32(rsz, off, 0, 0);
    }
    // the weight loads stay behind the activation loads in issue order, so
    // the barrier below can wait for the activations alone (vmcnt counts in
    // issue order)
    if constexpr (XDMA) __builtin_amdgcn_sched_barrier(0);
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
    if constexpr (XDMA) __builtin_amdgcn_sched_barrier(0);
    if (tid < 4) reinterpret_cast<uint32_t*>(zero_area)[tid] = 0u;
#pragma unroll
    for (int i = 0; i < XP; i++) {
        const int p = tid + i * W * 64;
        if (!XDMA && p < npieces) {
            const int off = p * 16;
            *reinterpret_cast<u32x4*>(smem + off + (off / (64 * N)) * (4 * N)) = xr[i];
        }
    }
#pragma unroll
    for (int i = 0; i < SP; i++) {
        const int e = tid + i * W * 64;
        if (e < UPW * RW && u0 + e / RW < u1) {
            const float sc = h2f(sr[i] & 0xffff), zz = h2f(sr[i] >> 16);
            szs[e] = make_float2(sc * 0x1p-10f, sc * (16.0f + zz) * 0x1p-14f);
        }
    }
    // LDS writes visible to the workgroup; the weight loads stay in flight.
    // With direct activation loads, each wave first waits for its own: at
    // most the 2 UPW weight loads issued after them may be outstanding.
    if constexpr (XDMA)
        asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(2 * UPW) : "memory");
    else
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    const int jq = li >> 2;
    const int offa = (jq == 0) ? 0 : (jq == 1) ? 4 : (jq == 2) ? 1 : 5;  // rows {0,4,1,5}, then + 2: {2,6,3,7}
    // step s of unit u reads X rows 128u + 32lg + 8s + offa (+ 2), whose
    // padded LDS offset is (34lg + offa) 2N + (136u + 8s) 2N
    const int lbase = (34 * lg + offa) * 2 * N + 8 * (li & 3);
#pragma unroll
    for (int u = 0; u < UPW; u++) {
        if (u0 + u < u1) {
            float4v d[2], dn = (float4v){0.f, 0.f, 0.f, 0.f};
            d[0] = d[1] = (float4v){0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int s = 0; s < 4; s++) {
                const half8v bv = mfma_b_pair(smem, lbase + (136 * u + 8 * s) * 2 * N, 4 * N);
#pragma unroll
                for (int t = 0; t < 2; t++) {
                    const uint32_t dw = s == 0 ? w[u][t].x : s == 1 ? w[u][t].y : s == 2 ? w[u][t].z : w[u][t].w;
                    const u32x4 av = {((dw << 6) & bmask) | bexp, ((dw << 2) & bmask) | bexp,
                                      ((dw >> 2) & bmask) | bexp, ((dw >> 6) & bmask) | bexp};
                    d[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8v, av), bv, d[t], 0, 0, 0);
                }
                dn = __builtin_amdgcn_mfma_f32_16x16x32_f16(ones, bv, dn, 0, 0, 0);
            }
#pragma unroll
            for (int t = 0; t < 2; t++) {
                const float* q = reinterpret_cast<const float*>(szs + u * RW + 32 * wave + 16 * t + 4 * lg);
                const float4 qa = *reinterpret_cast<const float4*>(q), qb = *reinterpret_cast<const float4*>(q + 4);
                const float sv[4] = {qa.x, qa.z, qb.x, qb.z}, zv[4] = {qa.y, qa.w, qb.y, qb.w};
#pragma unroll
                for (int i = 0; i < 4; i++) acc[t][i] = fmaf(sv[i], d[t][i], fmaf(-zv[i], dn[i], acc[t][i]));
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
static void launch_w4t(dim3 g, hipStream_t st, const uint4* wt, const uint32_t* sz, const uint16_t* x, float* y,
                       float* ws, int M, int K, int gs, int nch) {
    constexpr int W = 4;
    const size_t lds = (size_t)mfma_chunk_xbytes(128 * UPW, N) + 16 + 8 * UPW * 32 * W;
    w4a16t_mfma_kernel<UPW, W, N><<<g, W * 64, lds, st>>>(wt, sz, x, M, K, gs, nch, (int)g.x, (int)g.y, y, ws);
}

template <int N>
static void launch_w4t_n(int upw, int nch, dim3 g, hipStream_t st, const uint4* wt, const uint32_t* sz,
                         const uint16_t* x, float* y, float* ws, int M, int K, int gs) {
    if (upw == 8)
        launch_w4t<8, N>(g, st, wt, sz, x, y, ws, M, K, gs, nch);
    else if (upw == 4)
        launch_w4t<4, N>(g, st, wt, sz, x, y, ws, M, K, gs, nch);
    else
        launch_w4t<2, N>(g, st, wt, sz, x, y, ws, M, K, gs, nch);
}

// Grid of the tiled W4A16 GEMM: 128 rows a workgroup, and a K range of 8, 4
// or 2 units (the rule below).  K ranges are split
// across blockIdx.y; when that leaves more than 8 splits, each workgroup
// walks nch chunks of upw units in turn, as long as >= 256 workgroups
// remain, so fewer partial tiles go through the workspace.
static dim3 w4t_grid(int M, int K, int& upw, int& nch) {
    const int nunits = K / 128;
    const int gx = ceil_div(M, 128);
    // 8 units a workgroup only while that still gives >= 1024 workgroups: 4
    // units measured faster below that (batch 8, us, 8 units against 4:
    // 8192 x 8192 12.35 / 11.13, 14336 x 4096 12.82 / 11.36, 4096 x 14336
    // rows x K 11.48 / 10.87); then down to 2 while < 256 workgroups (4096 x
    // 4096 keeps 4: 6.84 against 7.45 us with 2)
    upw = (long)gx * ceil_div(nunits, 8) >= 1024 ? 8 : 4;
    while (upw > 2 && (long)gx * ceil_div(nunits, upw) < 256) upw >>= 1;
    // (28672 x 8192, batch 16: 33.2 us with 28 splits, 31.6 with 2 chunks, 30.2 with 4)
    nch = 1;
    while (ceil_div(nunits, upw * nch) > 8 && (long)gx * ceil_div(nunits, upw * nch * 2) >= 256) nch *= 2;
    return dim3(gx, ceil_div(nunits, upw * nch));
}

ZT_EXPORT long zt_w4a16_tiled_bytes(int M, int K) {
    if (M < 0 || K < 0 || K % 128 != 0) return -1;
    return (long)((M + 15) / 16) * 16 * (K / 2);
}

ZT_EXPORT long zt_w4a16_sz_bytes(int M, int K, int group_size) {
    if (M < 0 || K < 0 || group_size <= 0 || K % group_size != 0) return -1;
    return (long)M * (K / group_size) * 4;
}

ZT_EXPORT int zt_w4a16_tile(const void* W_packed, const uint16_t* scales, const uint16_t* zeros, int M, int K,
                            int group_size, void* W_tiled, uint32_t* sz, hipStream_t stream) {
    if (M < 0 || K < 0 || K % 128 != 0 || group_size <= 0 || group_size % 32 != 0 || K % group_size != 0)
        return (int)hipErrorInvalidValue;
    if (M == 0 || K == 0) return (int)hipSuccess;
    if (W_packed == nullptr || scales == nullptr || W_tiled == nullptr || sz == nullptr) return (int)hipErrorInvalidValue;
    if (((uintptr_t)W_packed & 15) || ((uintptr_t)W_tiled & 15) || ((uintptr_t)scales & 1) || ((uintptr_t)zeros & 1) ||
        ((uintptr_t)sz & 3))
        return (int)hipErrorInvalidValue;
    const int nunits = K / 128, ngroups = K / group_size;
    const long npieces = (long)((M + 15) / 16) * nunits * 64;
    w4t_tile_kernel<<<ceil_div(npieces, 256), 256, 0, stream>>>(static_cast<const uint4*>(W_packed),
                                                               static_cast<uint4*>(W_tiled), M, nunits, npieces);
    w4t_sz_kernel<<<ceil_div((long)M * ngroups, 256), 256, 0, stream>>>(scales, zeros, sz, M, ngroups);
    return (int)hipGetLastError();
}

ZT_EXPORT long zt_gemm_w4a16t_workspace_bytes(int M, int K, int N) {
    if (M < 0 || K < 0 || K % 128 != 0 || (N != 4 && N != 8 && N != 12 && N != 16)) return -1;
    if (M == 0 || K == 0) return 0;
    int upw, nch;
    return tiled_ws_bytes(M, (int)w4t_grid(M, K, upw, nch).y);
}

ZT_EXPORT int zt_gemm_w4a16t_f32(const void* W_tiled, const uint32_t* sz, const uint16_t* B, float* C, int M, int K,
                                 int N, int group_size, void* workspace, long workspace_bytes, hipStream_t stream) {
    if (M < 0 || K < 0 || K % 128 != 0 || group_size <= 0 || group_size % 128 != 0 || K % group_size != 0)
        return (int)hipErrorInvalidValue;
    if (N != 4 && N != 8 && N != 12 && N != 16) return (int)hipErrorInvalidValue;
    if (M == 0 || K == 0) return (int)hipSuccess;
    if (W_tiled == nullptr || sz == nullptr || B == nullptr || C == nullptr) return (int)hipErrorInvalidValue;
    if (((uintptr_t)W_tiled & 15) || ((uintptr_t)sz & 3) || ((uintptr_t)B & 15) || ((uintptr_t)C & 3))
        return (int)hipErrorInvalidValue;
    if ((long)M * (K / group_size) >= (1L << 29)) return (int)hipErrorInvalidValue;  // 32-bit sz offsets
    int upw, nch;
    const dim3 g = w4t_grid(M, K, upw, nch);
    const long need = tiled_ws_bytes(M, (int)g.y);
    if (need > 0 && (workspace == nullptr || workspace_bytes < need || ((uintptr_t)workspace & 15)))
        return (int)hipErrorInvalidValue;
    const uint4* wt = static_cast<const uint4*>(W_tiled);
    float* ws = static_cast<float*>(workspace);
    switch (N) {
        case 4: launch_w4t_n<4>(upw, nch, g, stream, wt, sz, B, C, ws, M, K, group_size); break;
        case 8: launch_w4t_n<8>(upw, nch, g, stream, wt, sz, B, C, ws, M, K, group_size); break;
        case 12: launch_w4t_n<12>(upw, nch, g, stream, wt, sz, B, C, ws, M, K, group_size); break;
        default: launch_w4t_n<16>(upw, nch, g, stream, wt, sz, B, C, ws, M, K, group_size); break;
    }
    if (g.y > 1) tiled_reduce(workspace, C, M, N, (int)g.y, stream);
    return (int)hipGetLastError();
}

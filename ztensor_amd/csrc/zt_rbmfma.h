// Row-block small-batch GEMMs on v_mfma_f32_4x4x4_16b_f16 (gfx950).
//
// C[rows, N] = W[rows, K] x X[K, N] for N = 4 NB (NB = 1 to 4), with the
// weights in their row-major upload layout and one launch per call: no K
// split across workgroups, no workspace and no second kernel.
//
// Work of one wave and step (16 chunks of 32 K values, 512 K):
//  * lane l belongs to MFMA block b = l >> 2, which takes chunk b of the
//    step, and supplies row j = l & 3 of a 4-row set as the B operand
//    (B column j).  One 16-byte weight load a lane therefore reads 4 rows x
//    256 contiguous bytes per instruction, the batch-1 access pattern;
//  * the A operand (rows of A = the 4 activation columns of an n-set) comes
//    from the step's activations, staged in the wave's own LDS region by
//    direct buffer-to-LDS loads and read back with ds_read_b64_tr_b16:
//    within a 16-lane group, output lane 4q + i, element e is half i of
//    the 8-byte row addressed by lane 4e + q.  So block q of the group gets
//    X[k][4js + i] at the four K positions its lanes 4e + q address;
//  * D lane 4b + j, register v is then sum_k X[k][4js + v] * W[row j][k]:
//    each lane holds all 4 columns of an n-set for its own row, so the
//    row's group scale applies per lane.
// Blocks (chunks) are summed across the wave by lane exchanges at the end,
// and the waves of a workgroup, which split K, through LDS.
//
// LDS layout of a step (per wave, 1 KB x N): chunk c (32 K) holds 4N
// pieces of 16 bytes (N = 4: piece p = K rows 2p, 2p+1; N = 8: piece p = K
// row p), stored at piece (p + sig(c)) mod 4N.  With sig = {0, 1, 4, 5}
// (N = 4) or {0, 2, 8, 10} (N = 8) for c mod 4, the 16 rows a transposing
// read addresses (4 blocks x K offsets {0, 4, 1, 5} + const) fall on 16
// distinct 8-byte bank slots.  The rotation is a permutation inside a
// chunk, so each load instruction still writes 1 KB of consecutive LDS and
// reads 1 KB of consecutive global memory.
#pragma once

#include "zt_mfma.h"

namespace zt {

template <int NB>
struct RbLayout {
    static constexpr int N = 4 * NB;
    static constexpr int PPC = 4 * N;          // 16-byte pieces per 32-K chunk
    static constexpr int STEP = 1024 * N;      // bytes of one step's activations
    // N = 4 and 8: the conflict-free rotations above; N = 12 and 16 (only for
    // callers without a tiled layout) rotate by 2 (c mod 4) pieces
    __device__ static __forceinline__ int sig(int c) {
        return NB == 1 ? ((c & 1) | ((c & 2) << 1)) : NB == 2 ? (((c & 1) << 1) | ((c & 2) << 2)) : 2 * (c & 3);
    }
};

// The same step layout for K orders whose MFMA steps read the K offsets
// {0, 2, 1, 3} + const (a step takes bytes (0, 2) and then (1, 3) of a
// dword: Q8_0's bytes, or the low or high nibbles of Q4_0's).  The rotations
// {0, 4, 8, 12} (N = 8) and {0, 1, 8, 9} (N = 16) put the 16 rows of a
// transposing read on 16 distinct 8-byte bank slots: slot 2((k + sig) mod 16)
// + (js & 1) for N = 8 and 2((2k + js/2 + sig) mod 16) + (js & 1) for N = 16.
template <int NB>
struct RbO4Layout {
    static_assert(NB == 2 || NB == 4, "offset-{0,2,1,3} layout: N = 8 or 16");
    static constexpr int N = 4 * NB;
    static constexpr int PPC = 4 * N;
    static constexpr int STEP = 1024 * N;
    __device__ static __forceinline__ int sig(int c) { return NB == 2 ? 4 * (c & 3) : ((c & 1) | ((c & 2) << 2)); }
};

// LDS byte offset of the transposing read of the MFMA step whose K
// positions are kbase + {0, 2, 1, 3}, n-set js, in that layout.
template <int NB>
__device__ __forceinline__ int rb_o4_tr_offset_at(int lane, int k, int js) {
    using Lay = RbO4Layout<NB>;
    const int c = 4 * (lane >> 4) + (lane & 3);
    const int b = 2 * Lay::N * k + 8 * js;
    const int p = (b / 16 + Lay::sig(c)) % Lay::PPC;
    return (c * Lay::PPC + p) * 16 + (b & 8);
}

template <int NB>
__device__ __forceinline__ int rb_o4_tr_offset(int lane, int kbase, int js) {
    const int e = (lane >> 2) & 3;
    return rb_o4_tr_offset_at<NB>(lane, kbase + (((e & 1) << 1) | (e >> 1)), js);  // {0, 2, 1, 3}
}

// The natural-order reads of IQ4_NL's MFMA step v: K positions 4v + {0, 1,
// 2, 3}, the same 16 rows as the offset-{0,2,1,3} reads of that step, so
// again on 16 distinct bank slots.
template <int NB>
__device__ __forceinline__ int rb_o4_tr_offset_nat(int lane, int kbase, int js) {
    return rb_o4_tr_offset_at<NB>(lane, kbase + ((lane >> 2) & 3), js);
}

// Issues the direct loads of one step's activations (global bytes
// [gstep, gstep + STEP) of x) into the wave's LDS region `xs`.  Lanes past
// the end of x read zeros (out-of-range buffer offsets).
template <int NB>
__device__ __forceinline__ void rb_stage_x(__amdgpu_buffer_rsrc_t rx, char* xs, uint32_t gstep, int lane) {
    using Lay = RbLayout<NB>;
#pragma unroll
    for (int i = 0; i < Lay::N; i++) {
        const int P = 64 * i + lane, c = P / Lay::PPC, pr = P % Lay::PPC;
        const int p = (pr + Lay::PPC - Lay::sig(c)) % Lay::PPC;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (__attribute__((address_space(3))) void*)(xs + 1024 * i), 16,
                                                 gstep + (uint32_t)((c * Lay::PPC + p) * 16), 0, 0, 0);
    }
}

// LDS byte offset of the transposing read of MFMA step s (K positions
// 8(s/2) + 2(s%2) + {0, 4, 1, 5}) and n-set js, for this lane's role: the
// 8 bytes of X[k][4js .. 4js+3] sit at chunk byte 2Nk + 8js, in piece
// (2Nk + 8js) / 16 before the rotation (a piece never splits them).
template <int NB>
__device__ __forceinline__ int rb_tr_offset(int lane, int s, int js) {
    using Lay = RbLayout<NB>;
    const int e = (lane >> 2) & 3, q = lane & 3, c = 4 * (lane >> 4) + q;
    const int ko = (e & 1) * 4 + (e >> 1);  // {0, 4, 1, 5}
    const int k = 8 * (s >> 1) + 2 * (s & 1) + ko;
    const int b = 2 * Lay::N * k + 8 * js;
    const int p = (b / 16 + Lay::sig(c)) % Lay::PPC;
    return (c * Lay::PPC + p) * 16 + (b & 8);
}

// The same for the element pairs of IQ4_NL's interleaved nibbles: MFMA
// step u reads K positions 2u + {0, 1, 0, 1} (each pair twice).
template <int NB>
__device__ __forceinline__ int rb_tr_offset_pair(int lane, int u, int js) {
    using Lay = RbLayout<NB>;
    const int e = (lane >> 2) & 3, q = lane & 3, c = 4 * (lane >> 4) + q;
    const int k = 2 * u + (e & 1);
    const int b = 2 * Lay::N * k + 8 * js;
    const int p = (b / 16 + Lay::sig(c)) % Lay::PPC;
    return (c * Lay::PPC + p) * 16 + (b & 8);
}

__device__ __forceinline__ half4v rb_tr_read(char* xs, int off) {
    return __builtin_bit_cast(half4v, tr_read_b64(xs, off));
}

// Sum over the 16 blocks of a wave (lane bits 2-5) of V values per lane
// (V a multiple of 4).
// Bits 5 and 4 are halving steps (each lane keeps one half of its values
// and trades the other with its partner; v_permlane32_swap /
// v_permlane16_swap), bits 3 and 2 plain adds of DPP row_ror:8 and
// row_ror:4 partners, which keep the row j = lane & 3.  Afterwards v[0 ..
// V/4 - 1] of lane l hold the full sums of value indices
// rb_value_index<V>(l, i); lanes with bits 2-3 clear are the writers.
template <int V, int OFF>
__device__ __forceinline__ void rb_halve(float (&v)[V]) {
    if constexpr (OFF >= 16) {
        constexpr int c = V * OFF / 32;  // live values at this level
        if constexpr (c >= 2) {
#pragma unroll
            for (int i = 0; i < c / 2; i++) v[i] = pair_step<OFF>(v[i], v[c / 2 + i]);
        }
        rb_halve<V, OFF / 2>(v);
    }
}

template <int V>
__device__ __forceinline__ void rb_block_reduce(float (&v)[V]) {
    static_assert(V >= 4 && V % 4 == 0, "V must be a multiple of 4");
    rb_halve<V, 32>(v);
#pragma unroll
    for (int i = 0; i < V / 4; i++) {
        float t = v[i] + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v[i]), 0x128, 0xF, 0xF, false));
        v[i] = t + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(t), 0x124, 0xF, 0xF, false));
    }
}

template <int V>
__device__ __forceinline__ int rb_value_index(int lane, int i) {
    return i + ((lane & 32) ? V / 2 : 0) + ((lane & 16) ? V / 4 : 0);
}

// End of a row-block GEMM: sums the wave's 16 blocks (lane exchanges), leaves
// the wave's sums in its own LDS region `own`, and, after a barrier, adds the
// waves' sums in wave order (wave w's region at regions + w * region_bytes)
// and stores C rows row0 .. row0 + 4R - 1.  acc[(r NB + js) 4 + v] holds row
// row0 + 4r + (lane & 3), column 4js + v; C row m, column n is at
// y[m ldy + n0 + n] (ldy = N, n0 = 0 when the launch covers all of C's columns).
template <int NB, int R>
__device__ __forceinline__ void rb_finish(float (&acc)[4 * R * NB], const char* regions, int region_bytes, char* own,
                                          float* __restrict__ y, int row0, int rows, int ldy = 4 * NB, int n0 = 0) {
    constexpr int N = 4 * NB, V = 4 * R * NB;
    const int lane = threadIdx.x & 63, j = lane & 3, nw = blockDim.x >> 6;
    rb_block_reduce<V>(acc);
    float* red = reinterpret_cast<float*>(own);
    if ((lane & 12) == 0) {
#pragma unroll
        for (int i = 0; i < V / 4; i++) red[rb_value_index<V>(lane, i) * 4 + j] = acc[i];
    }
    __syncthreads();
    for (int o = threadIdx.x; o < 4 * V; o += blockDim.x) {
        // o walks C[row0 .., :] contiguously: o = (row - row0) * N + n
        const int rl = o / N, n = o % N;
        const int r = rl >> 2, jj = rl & 3, js = n >> 2, v = n & 3;
        const int idx = ((r * NB + js) * 4 + v) * 4 + jj;
        float sum = 0.0f;
        for (int wv = 0; wv < nw; wv++) sum += reinterpret_cast<const float*>(regions + wv * region_bytes)[idx];
        if (row0 + rl < rows) y[(long)(row0 + rl) * ldy + n0 + n] = sum;
    }
}

// ------------------------------------------------------------ fp32-activation row-block GEMMs
//
// Q4_0 and Q8_0 blocks (32 weights, one scale) with groups of 4 or 8 fp32
// activation columns (columns n0 .. n0 + 4NB - 1 of B[K, ldx]), one launch a
// group: the row-block structure above (v_mfma_f32_4x4x4_16b_f16, lane =
// block of row j of a 4-row set, waves splitting K, activations staged per
// wave and read back transposed, no K split across workgroups).  fp32
// activations cannot be MFMA operands as they are, so each wave step
//  * loads its 512 x 4NB activations into VGPRs (16-byte loads), takes the
//    step's max |x| over the wave and a power of two c with c max|x| in
//    [2^14, 2^15), and splits every c x into fp16 hi = fp16(c x) and
//    lo = fp16(c x - hi): hi + lo equals c x to 2^-22 |c x| wherever lo is a
//    normal fp16 (|x| >= 2^-17 max|x|), and to 2^-25 absolute below that;
//    c is undone exactly (a power of two) when the step's sums are taken;
//  * writes hi and lo as 8NB fp16 columns (hi n-sets 0 .. NB-1, lo n-sets
//    NB .. 2NB-1) in the offset-{0,2,1,3} layout.
// B operand of MFMA step s (0-7): four weights of the lane's block as
// normal-range fp16, whose products with hi and lo are exact in fp32 and
// sum without the low bias that subnormal operands get:
//  * Q4_0: the low (s even) or high nibbles of bytes (0, 2) and (1, 3) of
//    dword s/2 (K positions 4(s/2) + 16(s%2) + {0, 2, 1, 3}) as
//    2^14 + 2^10 q;
//  * Q8_0: bytes (0, 2) and (1, 3) of dword s (K positions 4s + {0, 2, 1,
//    3}) as 2^15 + 2^7 u, u = q + 128 (q XOR 0x80);
//  * IQ4_NL: 8 steps a block, step v on elements 4v .. 4v+3 (data bytes
//    2v and 2v+1, low nibble first) in natural K order; a 2 KB LDS table
//    gives each byte (T_hi[low], T_hi[high], T_lo[low], T_lo[high]), the
//    fp32 codebook as fp16 hi + lo (within 2^-22 per entry), so the two
//    entries' first dwords are the step's T_hi operand and their second
//    dwords its T_lo operand.  Three MFMAs a step, x_hi T_hi + x_lo T_hi +
//    x_hi T_lo, leave out x_lo T_lo, at most 2^-22 |x T| a product; no
//    offset, so no X chain, and y += d D / c.
// Per block, n-set and step: D = sum (hi + lo) b (hi and lo MFMAs into one
// chain) and X = sum (hi + lo) 2^14 (B = 2^14, shared by the row sets), so
// sum(q x) c = 2^-10 (D - 1.5 X) for Q4_0 (q - 8) and 2^-7 (D - 3 X) for
// Q8_0, and the block's scale d takes it: y += d 2^-e (D/c - o X/c).  Every
// output is summed in wave and then wave order and stored once (rb_finish).
// INT4G: group-quantized int4 (element 2b in the low nibble of byte b,
// signed, fp32 scale and uint8 zero a group of 32 g elements); INT8: plain
// int8 rows without scales.
enum class RbFmt { Q4_0, Q8_RAW, Q8_SEP, Q8_SEP16, IQ4NL, INT4G, INT8 };

template <RbFmt F>
struct RbFmtInfo {
    static constexpr bool IQ = F == RbFmt::IQ4NL;                                // codebook table, no offset
    static constexpr bool ZP = F == RbFmt::INT4G, NOSC = F == RbFmt::INT8;       // group zero; no scale
    static constexpr bool Q4 = F == RbFmt::Q4_0 || IQ || ZP, RAW = F == RbFmt::Q8_RAW;  // 16-byte blocks
    static constexpr int WD = Q4 ? 4 : 8;                                        // weight dwords a block
    static constexpr int WL = Q4 ? 1 : 2;                                       // weight loads a block (not RAW)
    static constexpr int LPB = RAW ? 3 : NOSC ? WL : ZP ? WL + 2 : WL + 1;        // loads a block, scale included
    static constexpr int BB = Q4 ? 16 : RAW ? 36 : 32;                           // data bytes a block
    static constexpr int SBY = RAW ? 36 : ZP ? 4 : (Q4 || F == RbFmt::Q8_SEP16) ? 2 : 4;  // scale stride
    static constexpr int TBL = IQ ? 2048 : 0;                                    // LDS table bytes
};

// No codebook: the block formats whose values the B operand encodes directly.
struct RbNoTable {
    __device__ static uint2 entry(int) { return make_uint2(0u, 0u); }
};

template <int NB>
__device__ __forceinline__ void rbf_load_x(__amdgpu_buffer_rsrc_t rx, u32x4 (&xr)[8 * NB], int step, int ldx, int n0,
                                           int lane) {
#pragma unroll
    for (int i = 0; i < 8 * NB; i++) {
        const int k = step * 512 + (NB == 1 ? 64 * i + lane : 32 * i + (lane >> 1));
        const int col = n0 + (NB == 1 ? 0 : 4 * (lane & 1));
        xr[i] = __builtin_amdgcn_raw_buffer_load_b128(rx, (uint32_t)(k * ldx + col) * 4u, 0, 0);
    }
}

// LDS position of element e of a 32-element chunk.  The Q4_0 steps read
// positions 4 d + {0, 2, 1, 3} (low nibbles of dword d) and 16 + the same
// (high nibbles); INT4G keeps element 8 d + 2 i in the low nibble of byte
// i of dword d and 8 d + 2 i + 1 in its high nibble, so its activations are
// stored at position 16 (e & 1) + 4 (e >> 3) + ((e >> 1) & 3).
template <bool ZP>
__device__ __forceinline__ int rbf_kpos(int e) {
    return ZP ? 16 * (e & 1) + 4 * (e >> 3) + ((e >> 1) & 3) : e;
}

// scales: fp16 or fp32 scales (Q8_RAW: the 36-byte blocks); data: 16- or
// 32-byte blocks (Q8_RAW: the 36-byte blocks again).
// Threads a workgroup may have.  8-column groups run at most 8 waves (their
// 16 KB of LDS a wave allow no more than 8 waves a CU anyway), so 512
// threads cost no occupancy and leave up to 256 VGPRs a lane; 4 row sets at
// four steps a wave (16-byte blocks, K <= 20480) run at most 10 waves and
// need about 170 VGPRs.
constexpr int rbf_bound(int NB, int R, int S) { return NB == 2 ? 512 : R == 4 && S == 4 ? 640 : 1024; }

template <RbFmt F, int NB, int R, int S, class Tbl = RbNoTable>
__global__ void __launch_bounds__(rbf_bound(NB, R, S)) rbf_kernel(const uint8_t* __restrict__ scales, const uint8_t* __restrict__ data,
                                                   const float* __restrict__ x, float* __restrict__ y, int rows,
                                                   int kb, int ldx, int n0, const uint8_t* __restrict__ zeros, int gsc,
                                                   int ng) {
    using Info = RbFmtInfo<F>;
    using Lay = RbO4Layout<2 * NB>;
    constexpr int V = 4 * R * NB;
    extern __shared__ __attribute__((aligned(16))) char smem[];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int blk = lane >> 2, j = lane & 3;
    char* regions = smem + Info::TBL;  // IQ4_NL: the codebook table first
    char* xs = regions + wave * Lay::STEP;
    const int row0 = blockIdx.x * 4 * R;
    // rows past M and K read zeros: the buffers end at row M and at K
    const __amdgpu_buffer_rsrc_t rw =
        __builtin_amdgcn_make_buffer_rsrc((void*)data, (short)0, rows * kb * Info::BB, 0x00020000);
    // INT4G: scales and zeros [rows, ng], group g of a row covering blocks gsc g .. gsc (g + 1) - 1
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        (void*)scales, (short)0, Info::ZP ? rows * ng * 4 : rows * kb * Info::SBY, 0x00020000);
    const __amdgpu_buffer_rsrc_t rz = __builtin_amdgcn_make_buffer_rsrc((void*)zeros, (short)0, rows * ng, 0x00020000);
    const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc((void*)x, (short)0, kb * 128 * ldx, 0x00020000);
    const int step0 = wave * S;
    u32x4 xr[8 * NB];
    rbf_load_x<NB>(rx, xr, step0, ldx, n0, lane);
    __builtin_amdgcn_sched_barrier(0);
    uint32_t w[S][R][Info::WD], sc[S][R], zp[S][R];
    const uint32_t brow = (uint32_t)(row0 + j) * (uint32_t)kb, bstep = 4u * (uint32_t)kb;
#pragma unroll
    for (int t = 0; t < S; t++) {
        const int c = (step0 + t) * 16 + blk;
        const bool ok = c < kb;
        const int gq = Info::ZP ? c / gsc : 0;
#pragma unroll
        for (int r = 0; r < R; r++) {
            const uint32_t b = brow + r * bstep + (uint32_t)c;
            const uint32_t wo = ok ? b * (uint32_t)Info::BB : 0x80000000u;
            if constexpr (Info::RAW) {
                // the block's 9 dwords as three 12-byte loads: the scale, then the 8 data dwords
                typedef uint32_t u32x3 __attribute__((ext_vector_type(3)));
                const u32x3 v0 = __builtin_amdgcn_raw_buffer_load_b96(rw, wo, 0, 2);
                const u32x3 v1 = __builtin_amdgcn_raw_buffer_load_b96(rw, wo + 12, 0, 2);
                const u32x3 v2 = __builtin_amdgcn_raw_buffer_load_b96(rw, wo + 24, 0, 2);
                sc[t][r] = v0.x;
                w[t][r][0] = v0.y; w[t][r][1] = v0.z;
                w[t][r][2] = v1.x; w[t][r][3] = v1.y; w[t][r][4] = v1.z;
                w[t][r][5] = v2.x; w[t][r][6] = v2.y; w[t][r][7] = v2.z;
            } else {
#pragma unroll
                for (int i = 0; i < Info::WL; i++) {
                    const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rw, wo + 16 * i, 0, 2);  // nontemporal
                    w[t][r][4 * i] = v.x;
                    w[t][r][4 * i + 1] = v.y;
                    w[t][r][4 * i + 2] = v.z;
                    w[t][r][4 * i + 3] = v.w;
                }
            }
            if constexpr (Info::NOSC) {
                sc[t][r] = 0x3f800000u;  // 1.0f
            } else if constexpr (Info::ZP) {
                const uint32_t gi = (uint32_t)(row0 + j + 4 * r) * (uint32_t)ng + (uint32_t)gq;
                sc[t][r] = __builtin_amdgcn_raw_buffer_load_b32(rs, ok ? 4u * gi : 0x80000000u, 0, 0);
                zp[t][r] = __builtin_amdgcn_raw_buffer_load_b8(rz, ok ? gi : 0x80000000u, 0, 0);
            } else if constexpr (!Info::RAW) {
                const uint32_t so = ok ? b * (uint32_t)Info::SBY : 0x80000000u;
                sc[t][r] = Info::SBY == 2 ? __builtin_amdgcn_raw_buffer_load_b16(rs, so, 0, 0)
                                          : __builtin_amdgcn_raw_buffer_load_b32(rs, so, 0, 0);
            }
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (Info::IQ) {
        uint2* tbl = reinterpret_cast<uint2*>(smem);
        for (int i = threadIdx.x; i < 256; i += blockDim.x) tbl[i] = Tbl::entry(i);
        // the table is visible to the workgroup; the loads stay in flight
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    }
    float acc[V];
#pragma unroll
    for (int i = 0; i < V; i++) acc[i] = 0.0f;
    const half4v ones = (half4v){16384, 16384, 16384, 16384};  // 2^14
    uint32_t bmask = Info::Q4 ? 0x03C003C0u : 0x03FC03FCu, bexp = Info::Q4 ? 0x74007400u : 0x78007800u;
    asm volatile("" : "+v"(bmask), "+s"(bexp));  // the mask in a VGPR, the exponent in an SGPR (v_and_or_b32)
    constexpr float kSm = Info::IQ ? 1.0f : Info::Q4 ? 0x1p-10f : 0x1p-7f, kOff = Info::Q4 ? 1.5f : 3.0f;
#pragma unroll
    for (int t = 0; t < S; t++) {
        if (t > 0) {
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this step's activations, issued a step ahead
        } else {
            // the activations only: the weight and scale loads after them may be outstanding
            asm volatile("s_waitcnt vmcnt(%0)" ::"n"(S * R * Info::LPB) : "memory");
        }
        // the step's normalisation c = 2^sh
        float m = 0.0f;
#pragma unroll
        for (int i = 0; i < 8 * NB; i++)
#pragma unroll
            for (int e = 0; e < 4; e++) m = fmaxf(m, fabsf(__uint_as_float(xr[i][e])));
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
        int sh = 0;
        if (m > 0.0f && m <= 3.402823466e38f) {
            int e2;
            (void)frexpf(m, &e2);  // m = f 2^e2, f in [0.5, 1)
            sh = min(127, 15 - e2);
        }
        const float cs = ldexpf(1.0f, sh), ic = ldexpf(1.0f, -sh);
        // the previous step's transposing reads precede these writes in the
        // wave's LDS order; the scheduler must not move either across
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < 8 * NB; i++) {
            uint32_t hv[2], lv[2];
#pragma unroll
            for (int e = 0; e < 4; e += 2) {
                const float v0 = __uint_as_float(xr[i][e]) * cs, v1 = __uint_as_float(xr[i][e + 1]) * cs;
                const _Float16 h0 = (_Float16)v0, h1 = (_Float16)v1;
                const _Float16 l0 = (_Float16)(v0 - (float)h0), l1 = (_Float16)(v1 - (float)h1);
                hv[e / 2] = (uint32_t)__builtin_bit_cast(uint16_t, h0) | ((uint32_t)__builtin_bit_cast(uint16_t, h1) << 16);
                lv[e / 2] = (uint32_t)__builtin_bit_cast(uint16_t, l0) | ((uint32_t)__builtin_bit_cast(uint16_t, l1) << 16);
            }
            if constexpr (NB == 1) {
                // K row k: one 16-byte piece (hi columns, then lo columns)
                const int k = 64 * i + lane, c = k >> 5, p = (rbf_kpos<Info::ZP>(k & 31) + Lay::sig(c)) & 31;
                *reinterpret_cast<uint4*>(xs + (c * 32 + p) * 16) = make_uint4(hv[0], hv[1], lv[0], lv[1]);
            } else {
                // K row k: pieces 2k (hi) and 2k + 1 (lo), this lane's 4 columns at byte 8 (lane & 1)
                const int k = 32 * i + (lane >> 1), c = k >> 5, hf = 8 * (lane & 1), kp = rbf_kpos<Info::ZP>(k & 31);
                const int ph = (2 * kp + Lay::sig(c)) & 63, pl = (2 * kp + 1 + Lay::sig(c)) & 63;
                *reinterpret_cast<uint2*>(xs + (c * 64 + ph) * 16 + hf) = make_uint2(hv[0], hv[1]);
                *reinterpret_cast<uint2*>(xs + (c * 64 + pl) * 16 + hf) = make_uint2(lv[0], lv[1]);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        // the registers are free again: the next step's activations load
        // while this step's MFMAs run
        if (t + 1 < S) rbf_load_x<NB>(rx, xr, step0 + t + 1, ldx, n0, lane);
        float4v d[R][NB], dx[NB];
#pragma unroll
        for (int js = 0; js < NB; js++) {
            dx[js] = (float4v){0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int r = 0; r < R; r++) d[r][js] = (float4v){0.f, 0.f, 0.f, 0.f};
        }
        if constexpr (Info::IQ) {
#pragma unroll
            for (int v = 0; v < 8; v++) {
                half4v xa[2 * NB];
#pragma unroll
                for (int js = 0; js < 2 * NB; js++) xa[js] = rb_tr_read(xs, rb_o4_tr_offset_nat<2 * NB>(lane, 4 * v, js));
                half4v bh[R], bl[R];
#pragma unroll
                for (int r = 0; r < R; r++) {
                    const uint32_t q = w[t][r][v >> 1] >> (16 * (v & 1));  // bytes 2v, 2v + 1 in bits 0-15
                    const uint2 e0 = *reinterpret_cast<const uint2*>(smem + ((q << 3) & 0x7F8u));
                    const uint2 e1 = *reinterpret_cast<const uint2*>(smem + ((q >> 5) & 0x7F8u));
                    bh[r] = __builtin_bit_cast(half4v, make_uint2(e0.x, e1.x));  // T_hi of elements 4v .. 4v+3
                    bl[r] = __builtin_bit_cast(half4v, make_uint2(e0.y, e1.y));  // T_lo
                }
                // x_hi T_hi, x_lo T_hi, x_hi T_lo: consecutive MFMAs of one chain are R NB apart
#pragma unroll
                for (int tm = 0; tm < 3; tm++)
#pragma unroll
                    for (int r = 0; r < R; r++)
#pragma unroll
                        for (int js = 0; js < NB; js++)
                            d[r][js] = __builtin_amdgcn_mfma_f32_4x4x4f16(xa[(tm == 1 ? NB : 0) + js],
                                                                         tm == 2 ? bl[r] : bh[r], d[r][js], 0, 0, 0);
            }
        } else {
#pragma unroll
            for (int s = 0; s < 8; s++) {
                const int kbase = Info::Q4 ? 4 * (s >> 1) + 16 * (s & 1) : 4 * s;
                half4v xa[2 * NB];
#pragma unroll
                for (int js = 0; js < 2 * NB; js++) xa[js] = rb_tr_read(xs, rb_o4_tr_offset<2 * NB>(lane, kbase, js));
                half4v bv[R];
#pragma unroll
                for (int r = 0; r < R; r++) {
                    uint32_t a, b;
                    if constexpr (Info::Q4) {
                        const uint32_t q = w[t][r][s >> 1] ^ (Info::ZP ? 0x88888888u : 0u);  // INT4G: u = v + 8
                        a = (s & 1) ? q << 2 : q << 6;  // bytes 0, 2: low or high nibbles
                        b = (s & 1) ? q >> 6 : q >> 2;  // bytes 1, 3
                    } else {
                        const uint32_t u = w[t][r][s] ^ 0x80808080u;  // q + 128
                        a = u << 2;                                  // bytes 0, 2
                        b = u >> 6;                                  // bytes 1, 3
                    }
                    bv[r] = __builtin_bit_cast(half4v, (uint2){(a & bmask) | bexp, (b & bmask) | bexp});
                }
                // hi parts, then lo parts: consecutive MFMAs of one chain are R NB + NB apart
#pragma unroll
                for (int hl = 0; hl < 2; hl++) {
#pragma unroll
                    for (int js = 0; js < NB; js++)
                        dx[js] = __builtin_amdgcn_mfma_f32_4x4x4f16(xa[hl * NB + js], ones, dx[js], 0, 0, 0);
#pragma unroll
                    for (int r = 0; r < R; r++)
#pragma unroll
                        for (int js = 0; js < NB; js++)
                            d[r][js] = __builtin_amdgcn_mfma_f32_4x4x4f16(xa[hl * NB + js], bv[r], d[r][js], 0, 0, 0);
                }
            }
        }  // Q4_0 / Q8_0 steps
#pragma unroll
        for (int r = 0; r < R; r++) {
            const float dv = (Info::SBY == 2 ? h2f((uint16_t)sc[t][r]) : __uint_as_float(sc[t][r])) * kSm;
            // INT4G: w = (u - 8 - z) s, so the offset is (16 + 8 + z) / 16 where Q4_0's is 24 / 16
            const float ko = Info::ZP ? __builtin_fmaf((float)(zp[t][r] & 0xffu), 0.0625f, kOff) : kOff;
#pragma unroll
            for (int js = 0; js < NB; js++)
#pragma unroll
                for (int v = 0; v < 4; v++) {
                    float& a = acc[(r * NB + js) * 4 + v];
                    if constexpr (Info::IQ)
                        a = __builtin_fmaf(dv, d[r][js][v] * ic, a);
                    else
                        a = __builtin_fmaf(dv, __builtin_fmaf(d[r][js][v], ic, -ko * dx[js][v] * ic), a);
                }
        }
    }
    // waves split K: each wave leaves its sums in its own LDS region, then the
    // workgroup adds them in wave order
    rb_finish<NB, R>(acc, regions, Lay::STEP, xs, y, row0, rows, ldx, n0);
}

template <RbFmt F, int NB, int R, int S, class Tbl>
static void launch_rbf_t(dim3 g, int nw, hipStream_t st, const uint8_t* sc, const uint8_t* data, const float* x,
                         float* y, int rows, int kb, int ldx, int n0, const uint8_t* zs, int gsc, int ng) {
    const size_t lds = RbFmtInfo<F>::TBL + (size_t)nw * RbO4Layout<2 * NB>::STEP;
    if (lds > 65536) {  // past the default dynamic LDS limit (gfx950 has 160 KB a CU)
        static const bool raised = [] {
            return hipFuncSetAttribute(reinterpret_cast<const void*>(&rbf_kernel<F, NB, R, S, Tbl>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024) == hipSuccess;
        }();
        (void)raised;
    }
    rbf_kernel<F, NB, R, S, Tbl><<<g, nw * kWave, lds, st>>>(sc, data, x, y, rows, kb, ldx, n0, zs, gsc, ng);
}

template <RbFmt F, int NB, class Tbl>
static void launch_rbf_n(int R, int S, dim3 g, int nw, hipStream_t st, const uint8_t* sc, const uint8_t* data,
                         const float* x, float* y, int rows, int kb, int ldx, int n0, const uint8_t* zs, int gsc,
                         int ng) {
#define ZT_RB(RR, SS)                                                                                    \
    if (R == RR && S == SS)                                                                              \
        return launch_rbf_t<F, NB, RR, SS, Tbl>(g, nw, st, sc, data, x, y, rows, kb, ldx, n0, zs, gsc, ng);
    ZT_RB(1, 1) ZT_RB(2, 1) ZT_RB(4, 1) ZT_RB(1, 2) ZT_RB(2, 2) ZT_RB(1, 4) ZT_RB(2, 4)
    if constexpr (RbFmtInfo<F>::Q4) { ZT_RB(8, 1) ZT_RB(4, 2) }
    if constexpr (RbFmtInfo<F>::Q4 && !RbFmtInfo<F>::ZP && NB == 1) { ZT_RB(4, 4) }
#undef ZT_RB
}

// Shapes the fp32-activation row-block GEMM takes: N % 4 == 0, 16-byte
// aligned activation rows, K <= 32768, 32-bit buffer offsets.
template <RbFmt F>
static bool rbf_ok(int N, int kb, long M, const void* B) {
    return N >= 4 && N % 4 == 0 && ((uintptr_t)B & 15) == 0 && kb <= 16 * 16 * 4 &&
           M * kb * RbFmtInfo<F>::BB < 0x7fffffffL && (long)(kb + 16) * 128 * N < 0x7fffffffL;
}

// One launch per column group: K in steps of 16 blocks over up to 16 waves
// (8 for 8-column groups, whose hi/lo activations take 16 KB of LDS a wave),
// 1, 2 or 4 steps a wave, and row sets doubled while about 200 workgroups
// remain: up to 8 for the 16-byte blocks (Q4_0, IQ4_NL) at one step a wave,
// 4 at two, and at four when that takes no more than 10 waves (K <= 20480),
// else 2; 2 for Q8_0's 32-byte blocks past one step (beyond that the kernel
// spills registers).  Columns go in groups of 8 up to K = 8192 (16-byte
// blocks) or 16384 (Q8_0), else of 4.  Measured (us, batch 4 / 8): Q4_0
// 14336 x 4096 10.8 / 17.8 with 8 row sets against 12.6 / 24.1 with 4;
// IQ4_NL 3584 x 18944 24.1 / 48.9 with 4 row sets at four steps against
// 32.2 / 65.7 with 2 (that launch's 10 waves and 82 KB of LDS hold one
// workgroup a CU, so halving the workgroups halves the rounds); at 4096 x
// 14336 two 4-column launches beat one 8-column launch at four steps a wave
// (29.8 against 31.6), for Q8_0 the 8-column launch wins (38.5 against 55.0).
template <RbFmt F, class Tbl = RbNoTable>
static void launch_rbf(const void* scales, const void* data, const void* B, float* C, int M, int kb, int N,
                       hipStream_t st, const void* zeros = nullptr, int gsc = 1, int ng = 0) {
    const uint8_t* zs = static_cast<const uint8_t*>(zeros);
    const uint8_t* sc = static_cast<const uint8_t*>(scales);
    const uint8_t* dt = static_cast<const uint8_t*>(data);
    const float* x = static_cast<const float*>(B);
    constexpr bool Q4 = RbFmtInfo<F>::Q4;  // 16-byte blocks: Q4_0 and IQ4_NL
    for (int n0 = 0; n0 < N;) {
        const int nc = (N - n0 >= 8 && kb <= (Q4 ? 8 * 16 * 2 : 8 * 16 * 4)) ? 8 : 4;
        const int steps = ceil_div(kb, 16), wmax = nc == 8 ? 8 : 16;
        const int S = steps <= wmax ? 1 : steps <= 2 * wmax ? 2 : 4;
        const int nw = ceil_div(steps, S);
        // (INT4G's zero bytes push 4 row sets at four steps past the 640-thread budget)
        const int rmax = S == 4 ? (Q4 && !RbFmtInfo<F>::ZP && nc == 4 && nw <= 10 ? 4 : 2) : (S == 2 && !Q4) ? 2 : (S == 1 && Q4) ? 8 : 4;
        int R = 1;
        while (R < rmax && ceil_div(M, 8 * R) >= 200) R *= 2;
        const dim3 g(ceil_div(M, 4 * R));
        if (nc == 8) launch_rbf_n<F, 2, Tbl>(R, S, g, nw, st, sc, dt, x, C, M, kb, N, n0, zs, gsc, ng);
        else launch_rbf_n<F, 1, Tbl>(R, S, g, nw, st, sc, dt, x, C, M, kb, N, n0, zs, gsc, ng);
        n0 += nc;
    }
}

}  // namespace zt

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

// The same step layout for K-orders whose MFMA steps read K offsets
// {0, 2, 1, 3} + const (Q4_0's nibble order: a step takes the low nibbles
// of bytes 0 and 2, then of bytes 1 and 3, of one dword).  The rotations
// {0, 4, 8, 12} (N = 8) and {0, 1, 8, 9} (N = 16) put the 16 rows of a
// transposing read on 16 distinct 8-byte bank slots: slot 2((k + sig) mod 16)
// + (js & 1) for N = 8 and 2((2k + js/2 + sig) mod 16) + (js & 1) for N = 16.
template <int NB>
struct RbQ4Layout {
    static_assert(NB == 2 || NB == 4, "Q4_0-order layout: N = 8 or 16");
    static constexpr int N = 4 * NB;
    static constexpr int PPC = 4 * N;
    static constexpr int STEP = 1024 * N;
    __device__ static __forceinline__ int sig(int c) { return NB == 2 ? 4 * (c & 3) : ((c & 1) | ((c & 2) << 2)); }
};

// LDS byte offset of the transposing read of MFMA step s (K positions
// 4(s/2) + 16(s%2) + {0, 2, 1, 3}) and n-set js in the Q4_0-order layout.
template <int NB>
__device__ __forceinline__ int rb_q4_tr_offset(int lane, int s, int js) {
    using Lay = RbQ4Layout<NB>;
    const int e = (lane >> 2) & 3, q = lane & 3, c = 4 * (lane >> 4) + q;
    const int ko = ((e & 1) << 1) | (e >> 1);  // {0, 2, 1, 3}
    const int k = 4 * (s >> 1) + 16 * (s & 1) + ko;
    const int b = 2 * Lay::N * k + 8 * js;
    const int p = (b / 16 + Lay::sig(c)) % Lay::PPC;
    return (c * Lay::PPC + p) * 16 + (b & 8);
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

}  // namespace zt

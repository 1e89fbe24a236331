// The bf16 MFMA tile GEMM of zt_intq.hip (bf16_gemm_kernel) on Q4_0 and
// Q8_0 block weights, for the wide batches of their batched entry points.
// Activations are split into three exact bf16 parts and the block values
// enter as exact bf16, so every product is exact; each 32-element block's
// sums take the block's scale (and Q4_0's offset 8) once.  C[M, N] = W B
// with B [K, N] row-major, N even, B 8-byte aligned, K % 32 == 0.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace zt {

// data: the separated upload's data region (16 bytes a block); scales: its fp16 scales.
void bf16_gemm_q4_0(hipStream_t st, const uint8_t* data, const uint16_t* scales, const float* B, float* C, int M,
                    int N, int K);

// Q8_0: layout 0 the raw 36-byte blocks (data = the blocks, scales unused),
// 1 separated with fp32 scales, 2 separated with fp16 scales (GGUF).
void bf16_gemm_q8_0(hipStream_t st, int layout, const uint8_t* data, const void* scales, const float* B, float* C,
                    int M, int N, int K);

}  // namespace zt

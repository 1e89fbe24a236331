/*
 * zt_hip.h -- C ABI of libzt_hip.so, the MI355X (gfx950) quantized-weight
 * GEMV / small-batch GEMM library for ztensor's decode matmul path.
 *
 * Every entry point takes plain pointers and integers (floats only by device
 * pointer), allocates nothing, launches asynchronously on `stream` and
 * returns a hipError_t as int: 0 on success, 1 (hipErrorInvalidValue) for a
 * shape, alignment or null-pointer violation (nothing is launched then), or
 * the launch error.  This is the contract of the reference's CUDA launchers
 * (internal/cuda/kernels/gemm_q4.cu:163-201) and of the purego layer that
 * calls them (internal/cuda/kernels/gemm_q4_purego.go:15-28: integer /
 * pointer arguments only, nonzero -> Go error -> CPU fallback).
 *
 * Matrix convention (the one GemmQ4F32 / GemmQ8F32 use,
 * internal/gpuapi/kernels.go:45-48,79-81): C[M,N] = dequant(A)[M,K] * B[K,N],
 * A is the weight with M output rows and blocks/groups along K, B is the
 * activation with element (k,n) at B[k*N+n], C is fp32 with element (m,n) at
 * C[m*N+n].  N is the batch (1 for decode GEMV).
 *
 * Device layouts (built once at upload, see the zt_*_raw_to_gpu helpers):
 *   Q4_0 / IQ4_NL: [scales nblk*2 B][pad to 16][data nblk*16 B]
 *                  (tensor/quantized.go:158-198 RawBytesGPU)
 *   Q8_0 raw:      36-byte blocks [fp32 scale][32 x int8] (tensor/quantized.go:425-438)
 *   Q8_0 sep:      [scales nblk*4 B][pad to 16][data nblk*32 B]
 *   GGUF Q8_0:     [fp16 scales nblk*2 B][pad to 16][data nblk*32 B]
 *   W4 (GPTQ/AWQ): packed nibbles [M, K/2] + fp16 scales/zeros [M, K/group]
 *                  (tensor/quantized_gptq.go:217-277, tensor/quantized_awq.go:23-39)
 *   Ternary:       row-aligned 2-bit codes [M, ceil(K/4)]
 *                  (compute/ternary_gemv_gpu.go:52-67)
 *   Q4_K/Q5_K/Q6_K: the raw contiguous super-blocks (144/176/210 bytes per
 *                  256 values) RawBytes() holds, uploaded unchanged as the
 *                  reference does (compute/gpu_engine.go:817-874)
 *   Q5_0:          [fp16 d nblk*2][pad 16][uint32 qh nblk*4][pad 16][qs nblk*16]
 *                  (tensor/quantized_q5_0.go:118-165 RawBytesGPU)
 */
#ifndef ZT_HIP_H
#define ZT_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* zt_stream_t; /* == hipStream_t; NULL = default stream */

/* ---- library ---------------------------------------------------------- */

/* ABI version of this header (major*100 + minor). */
int zt_abi_version(void);

/* ---- Q4_0 -------------------------------------------------------------- */

/* Replaces gemm_q4_f32 (internal/cuda/kernels/gemm_q4.cu:163-201) behind
 * KernelRunner.GemmQ4F32 (internal/gpuapi/kernels.go:45-48), whose ROCm
 * implementation is a "not implemented" stub
 * (internal/gpuapi/rocm_kernels.go:109-111).  A_q4 is the RawBytesGPU
 * layout, data_offset = Q4GPUDataOffset(M*K/32) (tensor/quantized.go:195-198).
 * K % 32 != 0 -> InvalidValue (gemm_q4.cu:169-171).  fp32 activations.
 * B is [K, N] row-major.  N == 1 needs B 16-byte aligned.  Batches (N > 1)
 * run one launch per group of 8 or 4 columns when N % 4 == 0 and B is
 * 16-byte aligned (an MFMA GEMM that reads every weight once a group, no
 * workspace, the same bits every call), groups of 2 for other even N with B
 * 8-byte aligned, else one launch per column. */
int zt_gemm_q4_f32(const void* A_q4, const float* B, float* C, int M, int K, int N, int data_offset,
                   zt_stream_t stream);

/* Q4_0 weights x fp16 activations (the Q4Storage case of
 * compute.detectW4A16, compute/w4a16.go:50-54), fp32 output. */
int zt_gemm_q4_f16(const void* A_q4, const uint16_t* B, float* C, int M, int K, int N, int data_offset,
                   zt_stream_t stream);

/* Device dequantizer, bit-exact with Q4Storage.Dequantize
 * (tensor/quantized.go:96-114) over the RawBytesGPU layout. */
int zt_dequant_q4_f32(const void* A_q4, float* out, long nelem, int data_offset, zt_stream_t stream);

/* Grouped Q4_0 GEMV: up to ZT_GROUP_MAX matrices that read the same fp32
 * activation vector x[K] (a decode layer's q/k/v, or gate/up), batch 1, in
 * one launch.  Each descriptor names one matrix in its own RawBytesGPU
 * upload (A, data_offset as for zt_gemm_q4_f32), its row count and its
 * output y[rows]; the storages are neither merged nor re-laid out.  Matrix
 * i gets the result of zt_gemm_q4_f32(A_i, x, y_i, rows_i, K, 1, ...) up to
 * the fp32 summation order (bit for bit when both launches use the same
 * rows per wave, which the group picks from its total row count).
 * `descs` is a host array read during the call (the
 * descriptors travel in the kernel arguments, so nothing is allocated or
 * copied to the device).  A descriptor with rows == 0 is skipped (its
 * pointers are not read).  n outside 1..ZT_GROUP_MAX, any bad descriptor,
 * K % 32 != 0 or a misaligned x -> InvalidValue.
 * The reference's answer to the same launch cost is merging the storages
 * (MergeQ4Storage, tensor/quantized.go:224-242), which this entry point
 * makes unnecessary; its CPU engine runs one GemmF32Q4NT per matrix
 * (internal/xblas/gemm_quant.go:81-157). */
#define ZT_GROUP_MAX 8
typedef struct zt_q4_gemv_desc {
    const void* A;    /* RawBytesGPU buffer */
    long data_offset; /* Q4GPUDataOffset(rows*K/32) */
    float* y;         /* rows fp32 outputs */
    int rows;
    int reserved;     /* 0 */
} zt_q4_gemv_desc;
int zt_gemm_q4_group_f32(const zt_q4_gemv_desc* descs, int n, const float* x, int K, zt_stream_t stream);

/* Host: RawBytes (18-byte blocks, tensor/quantized.go:146-156) ->
 * RawBytesGPU (tensor/quantized.go:158-187).  out holds
 * zt_q4_gpu_bytes(nblk) bytes. */
long zt_q4_gpu_data_offset(long nblk); /* tensor/quantized.go:195-198 */
long zt_q4_gpu_bytes(long nblk);
void zt_q4_raw_to_gpu(const void* raw, long nblk, void* out);

/* ---- IQ4_NL ------------------------------------------------------------ */

/* IQ4_NL GEMV/GEMM.  The reference has no IQ4_NL kernel or upload path
 * (IQ4NLStorage is only dequantized, tensor/iq4_storage.go:74-95, and
 * CPUEngine.MatMul falls back to Data() + SGEMM); the device layout is the
 * Q4_0 RawBytesGPU layout applied to IQ4_NL's 18-byte blocks
 * (tensor/iq4_storage.go:12-23).  Decode follows DequantizeIQ4NL
 * (tensor/iq4_storage.go:36-46): interleaved nibbles, float IQ4NLTable.
 * fp32 activations, B [K, N] row-major.  Batches (N > 1) run one launch per
 * group of 8 or 4 columns when N % 4 == 0 and B is 16-byte aligned (an MFMA
 * GEMM that reads every weight once a group, no workspace, the same bits
 * every call; activations and codebook both enter it as fp16 hi + lo parts,
 * within about 2^-22 of their fp32 values), else one launch per column. */
int zt_gemm_iq4nl_f32(const void* A_iq4, const float* B, float* C, int M, int K, int N, int data_offset,
                      zt_stream_t stream);
/* fp16 activations: batches of 4 and 8 (12 and 16 up to 2048 rows) with B
 * 16-byte aligned run one launch with no workspace (the row-block MFMA GEMM),
 * 12 and 16 past 2048 rows a 16x16x32 MFMA GEMM, one workgroup per 32 rows
 * over all of K; both store every output once. */
int zt_gemm_iq4nl_f16(const void* A_iq4, const uint16_t* B, float* C, int M, int K, int N, int data_offset,
                      zt_stream_t stream);
/* Bit-exact with IQ4NLStorage.Dequantize (tensor/iq4_storage.go:75-89). */
int zt_dequant_iq4nl_f32(const void* A_iq4, float* out, long nelem, int data_offset, zt_stream_t stream);
/* Host: IQ4NLStorage.RawBytes (tensor/iq4_storage.go:104) -> separated layout. */
void zt_iq4nl_raw_to_gpu(const void* raw, long nblk, void* out);
/* Tiled upload layout for batched fp16 activations on the same IQ4_NL
 * matmul (the engine's CPU fallback, compute/cpu_engine.go:1215-1245); the
 * reference has no GPU IQ4_NL kernel.  Built once from the separated layout:
 *   W_tiled: tile (rt, u) = rows 16 rt .. +16, blocks 4u .. 4u+3, 1 KB at
 *   ((rt * K/128) + u) * 1024; 16-byte piece l = 16 g + i holds dword g of
 *   blocks 4u .. 4u+3 of row 16 rt + i (zt_iq4nl_tiled_bytes bytes);
 *   S_tiled: fp16 block scales, 128 bytes a tile at ((rt * K/128) + u) * 128,
 *   [16 rows][4 blocks] (zt_iq4nl_tiled_scale_bytes bytes);
 * rows past M, to the next multiple of 16, are zero.  K % 128 == 0, the
 * separated layout's base 2-byte and data 16-byte aligned, W_tiled and
 * S_tiled 16-byte aligned, else InvalidValue. */
long zt_iq4nl_tiled_bytes(int M, int K);
long zt_iq4nl_tiled_scale_bytes(int M, int K);
int zt_iq4nl_tile(const void* A_iq4, int M, int K, int data_offset, void* W_tiled, void* S_tiled, zt_stream_t stream);
/* C[M, N] = dequant(W) B on the tiled layout, B fp16 [K, N] 16-byte
 * aligned, N in {4, 8, 12, 16}, K % 128 == 0, else InvalidValue.  The
 * codebook enters the MFMAs as two fp16 parts whose sum is within
 * 2^-22.3 of each entry (relative), so the products match the reference's
 * fp32 table to that bound and only fp32 summation order differs.  When K is split across workgroups, each split stores its
 * partial tiles to `workspace` (16-byte aligned, at least
 * zt_gemm_iq4nlt_workspace_bytes(M, K, N) bytes, 0 when K is not split)
 * and a second kernel sums them in split order: C is the same on every
 * run.  A missing or short workspace when one is needed -> InvalidValue. */
long zt_gemm_iq4nlt_workspace_bytes(int M, int K, int N);
int zt_gemm_iq4nlt_f16(const void* W_tiled, const void* S_tiled, const uint16_t* B, float* C, int M, int K, int N,
                       void* workspace, long workspace_bytes, zt_stream_t stream);

/* ---- Dequantizer registry formats ---------------------------------------- */

/* Device twins of the reference's registered Dequantizers
 * (tensor/quant_registry.go:10-73, 231-240; GetQuantType(name).Dequantize(
 * src, dst)): src holds the same bytes the registered Dequantize takes, in
 * device memory; out receives nelem fp32 values, bit-exact with the
 * reference's.  Names and entry points:
 *   "Q4_0"     zt_dequant_q4raw_f32  (Q4Storage.RawBytes, 18-byte blocks;
 *                                     tensor/quantized.go:96-114)
 *   "Q8_0"     zt_dequant_q8_f32     (36-byte blocks, above)
 *   "Q4_K" / "Q5_K" / "Q6_K" / "Q5_0"
 *              zt_dequant_q4k/q5k/q6k/q5_0_f32 (raw blocks, below)
 *   "AWQ_4"    zt_awq4_wire_header on the host copy, then zt_dequant_awq4_f32
 *              (tensor/quantized_awq.go:242-308)
 *   "FP8_E4M3" / "FP8_E5M2"
 *              zt_dequant_fp8_f32 (4-byte LE fp32 scale, then one byte per
 *              element; tensor/quant_registry.go:190-229, decoders
 *              tensor/fp8_storage.go:229-250, 304-331)
 *   "IQ3_S"    zt_dequant_iq3s_f32 (110-byte super-blocks of 256 values;
 *              tensor/iq3_storage.go:12-95, 98-128, 169-186; the grid of
 *              tensor/iq3_grid.go:15-27).  The reference's Dequantize
 *              rejects nelem == 0 (NewIQ3SStorageFromRaw); the host binding
 *              raises there, the entry point treats it as a no-op.
 *   "W8A8"     zt_dequant_q8_f32 (the Q8_0 36-byte groups;
 *              tensor/quantized_w8a8.go:285-322)
 * A source shorter than the format needs, a misaligned source (2 bytes for
 * Q4_0, 4 for AWQ_4 and FP8) or a null pointer -> InvalidValue, as the
 * reference's errShortData (tensor/quant_registry.go:242-245).  nelem == 0
 * is a no-op success. */
int zt_dequant_q4raw_f32(const void* src, long src_bytes, float* out, long nelem, zt_stream_t stream);
/* Host: checks the AWQ_4 wire header against nelem as the reference's
 * Dequantize and NewAWQStorageFromRaw do (numElements == nelem, groupSize > 0,
 * nGroups == ceil(nelem / groupSize), enough bytes for the (scale, zero)
 * pairs and every group's packed words) and returns groupSize and nGroups;
 * InvalidValue otherwise. */
int zt_awq4_wire_header(const void* wire, long wire_bytes, long nelem, int* group_size, int* ngroups);
int zt_dequant_awq4_f32(const void* wire, long wire_bytes, float* out, long nelem, int group_size, int ngroups,
                        zt_stream_t stream);
/* e5m2: 0 = FP8_E4M3 (no NaN or infinity: exponent 15 is an ordinary
 * binade, as the reference decodes it), 1 = FP8_E5M2. */
int zt_dequant_fp8_f32(const void* wire, long wire_bytes, float* out, long nelem, int e5m2, zt_stream_t stream);
int zt_dequant_iq3s_f32(const void* src, long src_bytes, float* out, long nelem, zt_stream_t stream);

/* ---- Q8_0 -------------------------------------------------------------- */

/* Replaces gemm_q8_f32 (internal/cuda/kernels/gemm_q8.cu:156-182) behind
 * KernelRunner.GemmQ8F32 (internal/gpuapi/kernels.go:79-81; ROCm stub
 * internal/gpuapi/rocm_kernels.go:133-135).  A_q8 is Q8Storage.RawBytes()
 * (36-byte blocks, fp32 scale), 4-byte aligned.  B is [K, N] row-major.
 * Batches with N % 4 == 0 and B 16-byte aligned run one MFMA launch per
 * group of 8 or 4 columns (every weight read once a group, no workspace);
 * other N one launch per column.  The same holds for zt_gemm_q8sep_f32 and
 * zt_gemm_q8gguf_f32. */
int zt_gemm_q8_f32(const void* A_q8, const float* B, float* C, int M, int K, int N, zt_stream_t stream);

/* Same product over the separated Q8_0 layout (aligned 32-byte payloads;
 * the Q8 counterpart of Q4's RawBytesGPU).  data_offset =
 * zt_q8_gpu_data_offset(M*K/32). */
int zt_gemm_q8sep_f32(const void* A_q8, const float* B, float* C, int M, int K, int N, long data_offset,
                      zt_stream_t stream);
/* Bit-exact with Q8Storage.Dequantize (tensor/quantized.go:344-355). */
int zt_dequant_q8_f32(const void* A_q8, float* out, long nelem, zt_stream_t stream);
int zt_dequant_q8sep_f32(const void* A_q8, float* out, long nelem, long data_offset, zt_stream_t stream);
/* Raw 36-byte blocks -> separated layout, on the device (raw 4-byte
 * aligned, out 16-byte aligned and zt_q8_gpu_bytes(nblk) long) or host. */
int zt_q8_repack(const void* raw, void* out, long nblk, zt_stream_t stream);
long zt_q8_gpu_data_offset(long nblk);
long zt_q8_gpu_bytes(long nblk);
void zt_q8_raw_to_gpu(const void* raw, long nblk, void* out);

/* GGUF Q8_0: the 34-byte [fp16 d][32 x int8] blocks of an mmap'd GGUF tensor
 * (MmapStorage, tensor/mmap_storage.go:94-96, 265-284).  The reference's GPU
 * engine hands these bytes to the 36-byte gemm_q8_f32
 * (compute/gpu_engine.go:2865-2870), which misreads them; here they are
 * repacked once at upload into [fp16 d, nblk*2][pad 16][int8, nblk*32]
 * (zt_q8gguf_raw_to_gpu; data_offset = zt_q8gguf_gpu_data_offset(nblk)) and
 * multiplied with the Q8_0 kernels.  Dequantization is bit-exact with
 * MmapStorage.dequantizeQ8_0. */
int zt_gemm_q8gguf_f32(const void* A, const float* B, float* C, int M, int K, int N, long data_offset,
                       zt_stream_t stream);
int zt_dequant_q8gguf_f32(const void* A, float* out, long nelem, long data_offset, zt_stream_t stream);
long zt_q8gguf_gpu_data_offset(long nblk);
long zt_q8gguf_gpu_bytes(long nblk);
void zt_q8gguf_raw_to_gpu(const void* raw, long nblk, void* out);

/* ---- W4A16 (GPTQ / AWQ 4-bit, fp16 activations) ----------------------- */

/* Backs W4A16MatMuler.MatMulW4A16 (compute/w4a16.go:137-143), which no
 * reference engine implements; the CPU fallback it replaces is
 * MatMulW4A16 (compute/w4a16.go:71-119: dequantize + fp32 GEMM, fp32
 * result).  W_packed: [M, K/2] nibbles (GPTQ bits=4 / AWQ byte order),
 * 16-byte aligned; scales, zeros: fp16 [M, K/group_size] (zeros NULL ->
 * zero-point 8); B: fp16 [K, N]; C: fp32 [M, N].  group_size % 32 == 0 and
 * K % group_size == 0, else InvalidValue. */
int zt_gemm_w4a16_f32(const void* W_packed, const uint16_t* scales, const uint16_t* zeros, const uint16_t* B,
                      float* C, int M, int K, int N, int group_size, zt_stream_t stream);
/* Batch-1 form of the same MatMulW4A16 (compute/w4a16.go:137-143) on a
 * packed (scale, zero) array built once at upload: szr is uint32
 * [M][K/group_size], fp16 scale in the low half and fp16 zero (8.0 when
 * zeros is NULL) in the high half (zt_w4a16_sz_bytes bytes), built by
 * zt_w4a16_pack_szr from the zt_gemm_w4a16_f32 scales and zeros.  One
 * load per row and group instead of two; y[M] = dequant(W) x, the result of
 * zt_gemm_w4a16_f32 with N = 1.  group_size % 32 == 0, K % group_size == 0,
 * K <= 32768, M * K / 2 < 2^31, W_packed and x 16-byte aligned, else
 * InvalidValue.  K == 0 writes zeros. */
int zt_w4a16_pack_szr(const uint16_t* scales, const uint16_t* zeros, int M, int K, int group_size, uint32_t* szr,
                      zt_stream_t stream);
int zt_gemv_w4a16sz_f32(const void* W_packed, const uint32_t* szr, const uint16_t* x, float* y, int M, int K,
                        int group_size, zt_stream_t stream);
/* Batches of the same MatMulW4A16 (compute/w4a16.go:137-143) on the packed
 * (scale, zero) dwords and the row-major weights as uploaded: B fp16 [K, N],
 * C fp32 [M, N].  N == 1 is zt_gemv_w4a16sz_f32; N = 4, 8, 12 or 16 runs
 * one launch with no workspace and the same result on every call.  Same
 * conditions as zt_gemv_w4a16sz_f32 plus B 16-byte aligned, K <= 32768
 * (N = 12, 16: K <= 8192); other N -> InvalidValue. */
int zt_gemm_w4a16sz_f32(const void* W_packed, const uint32_t* szr, const uint16_t* B, float* C, int M, int K, int N,
                        int group_size, zt_stream_t stream);
/* Grouped batch-1 W4A16: up to ZT_GROUP_MAX matrices on packed (scale,
 * zero) dwords that read the same fp16 activation vector x[K] (a decode
 * layer's q/k/v, or gate/up: MatMulW4A16 per projection, compute/
 * w4a16.go:137-143), one launch.  No reference counterpart: the reference
 * has no grouped or merged W4A16 matmul (MergeQ4Storage,
 * tensor/quantized.go:224-242, covers Q4_0 only).  Each y_i is
 * zt_gemv_w4a16sz_f32 on matrix i, bit for bit.  All matrices share K and
 * group_size; rows == 0 entries are skipped (their pointers are not read).
 * n outside 1..ZT_GROUP_MAX, a bad descriptor, a misaligned x or a bad
 * group size -> InvalidValue.  Allocates nothing. */
typedef struct zt_w4a16_gemv_desc {
    const void* W;        /* packed nibbles [rows, K/2], 16-byte aligned */
    const uint32_t* szr;  /* zt_w4a16_pack_szr dwords [rows][K/group_size] */
    float* y;             /* rows fp32 outputs */
    int rows;
    int reserved;         /* 0 */
} zt_w4a16_gemv_desc;
int zt_gemv_w4a16sz_group_f32(const zt_w4a16_gemv_desc* descs, int n, const uint16_t* x, int K, int group_size,
                              zt_stream_t stream);
/* Bit-exact with GPTQStorage.Dequantize (tensor/quantized_gptq.go:134-163)
 * and AWQStorage.Dequantize (tensor/quantized_awq.go:118-136). */
int zt_dequant_w4_f32(const void* W_packed, const uint16_t* scales, const uint16_t* zeros, float* out, long nelem,
                      int group_size, zt_stream_t stream);
/* DequantW4ToFP16 (compute/w4a16.go:170-175: Slice, then
 * NewFloat16StorageFromF32) on the device, "fp16 weights for HGEMM": the
 * fp32 values of zt_dequant_w4_f32 / zt_dequant_q4_f32, each rounded to
 * fp16 to nearest, ties to even (fp16 bits out).  Values beyond the fp16
 * range become +-inf.  The reference's fp32 -> fp16 rounding lives in
 * github.com/zerfoo/float16 v0.2.0, which no reference test pins; IEEE
 * round-to-nearest-even is assumed. */
int zt_dequant_w4_f16(const void* W_packed, const uint16_t* scales, const uint16_t* zeros, uint16_t* out, long nelem,
                      int group_size, zt_stream_t stream);
int zt_dequant_q4_f16(const void* A_q4, uint16_t* out, long nelem, int data_offset, zt_stream_t stream);

/* Tiled upload layout for the small-batch path of the same MatMulW4A16
 * (compute/w4a16.go:137-143).  The reference uploads W4A16 weights as
 * they are stored; this layout is built once at upload, like the separated
 * Q8_0 layout, and serves N in {4, 8, 12, 16}:
 *   W_tiled: each 16-row x 128-K tile is 1 KB, tile (rt, u) at byte
 *   (rt * K/128 + u) * 1024; 16-byte piece l = 16 g + i holds row 16 rt + i,
 *   K 128 u + 32 g .. +32, the same bytes as in W_packed; rows past M, to
 *   the next multiple of 16, are zero (zt_w4a16_tiled_bytes bytes);
 *   sz: uint32 [K/group_size][M], fp16 scale in the low half and fp16 zero
 *   (8.0 when zeros is NULL) in the high half (zt_w4a16_sz_bytes bytes).
 * zt_w4a16_tile builds both on the device from the zt_gemm_w4a16_f32
 * operands: K % 128 == 0, group_size % 32 == 0, K % group_size == 0,
 * W_packed and W_tiled 16-byte aligned, else InvalidValue.  The size
 * helpers return -1 for shapes the layout does not take. */
long zt_w4a16_tiled_bytes(int M, int K);
long zt_w4a16_sz_bytes(int M, int K, int group_size);
int zt_w4a16_tile(const void* W_packed, const uint16_t* scales, const uint16_t* zeros, int M, int K, int group_size,
                  void* W_tiled, uint32_t* sz, zt_stream_t stream);
/* C[M, N] = dequant(W) B on the tiled layout, the result of
 * zt_gemm_w4a16_f32 within the fp32 tolerance: N in {4, 8, 12, 16},
 * K % 128 == 0, group_size % 128 == 0, B fp16 [K, N] 16-byte aligned,
 * M * K/group_size < 2^29, else InvalidValue.  When K is split across
 * workgroups, the splits store partial tiles to `workspace` (16-byte
 * aligned, at least zt_gemm_w4a16t_workspace_bytes(M, K, N) bytes; 0 when
 * K is not split) and a second kernel sums them in split order, so C is
 * the same on every run.  A missing or short workspace when one is needed
 * -> InvalidValue. */
long zt_gemm_w4a16t_workspace_bytes(int M, int K, int N);
int zt_gemm_w4a16t_f32(const void* W_tiled, const uint32_t* sz, const uint16_t* B, float* C, int M, int K, int N,
                       int group_size, void* workspace, long workspace_bytes, zt_stream_t stream);

/* ---- Batched Q4_0 / Q8_0 on tiled layouts (MFMA) ------------------------- */

/* The batched products behind KernelRunner.GemmQ4F32 / GemmQ8F32
 * (internal/gpuapi/kernels.go:45-48, 79-81; CUDA gemm_q4_f32 / gemm_q8_f32,
 * internal/cuda/kernels/gemm_q4.cu:163-201, gemm_q8.cu:156-182) for batches
 * of 4, 8, 12 or 16 fp32 activation columns, on upload-time tiled layouts:
 *   Q4_0: zt_q4_tile builds the IQ4_NL tiled layout (above) from Q4_0's
 *   separated layout (RawBytesGPU, tensor/quantized.go:168-198), which has
 *   the same 18-byte block shape: W_tiled zt_q4_tiled_bytes, S_tiled (fp16
 *   scales) zt_q4_tiled_scale_bytes;
 *   Q8_0: zt_q8_tile builds it from the separated Q8_0 layout (data_offset =
 *   zt_q8_gpu_data_offset): tile (rt, u) = rows 16 rt .. +16, blocks
 *   4u .. 4u+3, 2 KB at ((rt * K/128) + u) * 2048; in half h (1 KB) piece
 *   l = 16 g + i holds bytes 8g .. 8g+7 of block 4u+2h, then of block
 *   4u+2h+1, of row 16 rt + i; S_tiled fp32 scales, 256 bytes a tile
 *   [16 rows][4 blocks].  Rows past M, to the next multiple of 16, are zero.
 * K % 128 == 0, W_tiled / S_tiled / B 16-byte aligned, N in {4, 8, 12, 16},
 * else InvalidValue.  Activations are split into two fp16 parts after a
 * power-of-two normalisation (about 2^-22 relative precision each).  When
 * K is split across workgroups the partial tiles go to the caller's
 * workspace (16-byte aligned, at least zt_gemm_q{4,8}t_workspace_bytes(M,
 * K, N) bytes, which is 0 when K is not split; a smaller or NULL workspace
 * then gives InvalidValue) and a second kernel sums them in a fixed order,
 * so C is the same on every run.  The workspace is scratch: calls that
 * overlap in time need their own. */
long zt_q4_tiled_bytes(int M, int K);
long zt_q4_tiled_scale_bytes(int M, int K);
int zt_q4_tile(const void* A_q4, int M, int K, int data_offset, void* W_tiled, void* S_tiled, zt_stream_t stream);
long zt_gemm_q4t_workspace_bytes(int M, int K, int N);
int zt_gemm_q4t_f32(const void* W_tiled, const void* S_tiled, const float* B, float* C, int M, int K, int N,
                    void* workspace, long workspace_bytes, zt_stream_t stream);

/* zt_gemm_q4t_f32 without a workspace argument and without allocating:
 * no counterpart in the reference.  It is for callers that cannot call
 * hipMalloc (code under HIP graph capture, serving loops, harnesses that
 * forbid allocation).  The K-split partials go to a static device array of
 * ZT_NOALLOC_SCRATCH_BYTES that every GPU holds one copy of from the first
 * call on it until the process ends; C is bit-identical to
 * zt_gemm_q4t_f32's.  A call whose partials exceed the array
 * (zt_gemm_q4t_workspace_bytes(M, K, N) > ZT_NOALLOC_SCRATCH_BYTES, e.g. the
 * 28672 x 8192 matrices of Llama-3-70B) runs as slices of whole 128-row
 * groups, one after another on the stream, each with the whole call's K
 * split, so C is still bit-identical; only a call whose single 128-row slice
 * needs more (K > 2^19 at 128 or more rows) returns hipErrorOutOfMemory (2)
 * without launching.  Other argument errors return InvalidValue as
 * zt_gemm_q4t_f32 does.  Calls on one GPU share the array: calls that
 * overlap on one GPU (on different streams) race, calls on one stream do
 * not.  The current device must be the stream's device. */
#define ZT_NOALLOC_SCRATCH_BYTES (8L << 20)
int zt_gemm_q4t_f32_noalloc(const void* W_tiled, const void* S_tiled, const float* B, float* C, int M, int K, int N,
                            zt_stream_t stream);
long zt_q8_tiled_bytes(int M, int K);
long zt_q8_tiled_scale_bytes(int M, int K);
int zt_q8_tile(const void* A_q8, int M, int K, long data_offset, void* W_tiled, void* S_tiled, zt_stream_t stream);
/* The same tiled Q8_0 layout built from the GGUF Q8_0 separated layout
 * (fp16 scales, zt_q8gguf_raw_to_gpu, data_offset = zt_q8gguf_gpu_data_offset):
 * the scales are widened to fp32 exactly, so zt_gemm_q8t_f32 runs GGUF Q8_0
 * batches (MmapStorage, tensor/mmap_storage.go:94-96). */
int zt_q8gguf_tile(const void* A_q8, int M, int K, long data_offset, void* W_tiled, void* S_tiled, zt_stream_t stream);
long zt_gemm_q8t_workspace_bytes(int M, int K, int N);
int zt_gemm_q8t_f32(const void* W_tiled, const void* S_tiled, const float* B, float* C, int M, int K, int N,
                    void* workspace, long workspace_bytes, zt_stream_t stream);

/* Batched Q4_K on the same MFMA kernel: the raw super-blocks
 * (Q4KStorage.RawBytes, tensor/quantized_kquant.go:34-79, 144 bytes per 256
 * values, the layout UploadWeights places on the device,
 * compute/gpu_engine.go:817-836) are repacked by zt_q4k_tile into the Q4_0
 * tiled data layout (each 32-value sub-block as a 16-byte Q4_0 block) plus
 * the 16-byte super-block headers as [tile][super-block][16 rows][16 B]
 * (zt_q4k_tiled_bytes / zt_q4k_tiled_header_bytes).  zt_gemm_q4kt_f32 takes
 * both with fp32 B [K, N], N in {4, 8, 12, 16}, K % 256 == 0, and the
 * split-K workspace of zt_gemm_q4kt_workspace_bytes; each sub-block adds
 * (d*scale) * sum(q x) - (dmin*min) * sum(x) with the reference's fp32
 * products d*scale and dmin*min.  16-byte alignment as above, else
 * InvalidValue.  Replaces the reference's dequantize-then-SGEMM for
 * batched Q4_K (compute/gpu_engine.go:2240-2255). */
long zt_q4k_tiled_bytes(int M, int K);
long zt_q4k_tiled_header_bytes(int M, int K);
int zt_q4k_tile(const void* W_q4k, int M, int K, void* W_tiled, void* H_tiled, zt_stream_t stream);
long zt_gemm_q4kt_workspace_bytes(int M, int K, int N);
int zt_gemm_q4kt_f32(const void* W_tiled, const void* H_tiled, const float* B, float* C, int M, int K, int N,
                     void* workspace, long workspace_bytes, zt_stream_t stream);

/* Batched Q5_K: the Q4_K tiled layout (data, headers) of the 176-byte
 * super-blocks plus the fifth-bit dwords of the Q5_0 tiled layout
 * (zt_q5k_tiled_qh_bytes), built by zt_q5k_tile; zt_gemm_q5kt_f32 as
 * zt_gemm_q4kt_f32 with Q_tiled after H_tiled (11 arguments). */
long zt_q5k_tiled_bytes(int M, int K);
long zt_q5k_tiled_header_bytes(int M, int K);
long zt_q5k_tiled_qh_bytes(int M, int K);
int zt_q5k_tile(const void* W_q5k, int M, int K, void* W_tiled, void* H_tiled, void* Q_tiled, zt_stream_t stream);
long zt_gemm_q5kt_workspace_bytes(int M, int K, int N);
int zt_gemm_q5kt_f32(const void* W_tiled, const void* H_tiled, const void* Q_tiled, const float* B, float* C, int M,
                     int K, int N, void* workspace, long workspace_bytes, zt_stream_t stream);

/* Batched Q6_K on the same MFMA kernel.  zt_q6k_tile reads Q6KStorage's
 * 210-byte super-blocks (tensor/quantized_kquant.go:335-382: ql, qh, int8
 * scales, fp16 d) and writes the 6-bit values as bytes in the Q8_0 tile
 * positions (zt_q6k_tiled_bytes; piece 16 g + i of a tile-unit half holds,
 * for each of its two blocks, values 4g .. 4g+3 and 16 + 4g .. 16 + 4g+3
 * of row i) and the fp32 products d * sc of every
 * 16-value group, [tile-unit][16 rows][8 groups] (zt_q6k_tiled_scale_bytes).
 * zt_gemm_q6kt_f32: C[M, N] = W * B for N in {4, 8, 12, 16}, K % 256 == 0,
 * workspace as zt_gemm_q4t_f32.  Replaces the reference's
 * dequantize-then-SGEMM for batched Q6_K (compute/gpu_engine.go:2240-2255). */
long zt_q6k_tiled_bytes(int M, int K);
long zt_q6k_tiled_scale_bytes(int M, int K);
int zt_q6k_tile(const void* W_q6k, int M, int K, void* W_tiled, void* S_tiled, zt_stream_t stream);
long zt_gemm_q6kt_workspace_bytes(int M, int K, int N);
int zt_gemm_q6kt_f32(const void* W_tiled, const void* S_tiled, const float* B, float* C, int M, int K, int N,
                     void* workspace, long workspace_bytes, zt_stream_t stream);

/* Batched Q5_0 on the same MFMA kernel.  zt_q5_0_tile takes Q5_0Storage's
 * RawBytesGPU (tensor/quantized_q5_0.go:118-165; offsets zt_q5_0_gpu_qh_offset
 * / zt_q5_0_gpu_qs_offset) and writes the nibbles and fp16 scales in the
 * Q4_0 tiled layout (zt_q5_0_tiled_bytes, zt_q5_0_tiled_scale_bytes) plus
 * one dword of fifth bits per lane and tile-unit (zt_q5_0_tiled_qh_bytes;
 * byte s = block 4u+s, bits = values 4g, 4g+2, 4g+16, 4g+18, 4g+1, 4g+3,
 * 4g+17, 4g+19 of lane 16g+i's row).  zt_gemm_q5_0t_f32: fp32 B [K, N],
 * N in {4, 8, 12, 16}, K % 128 == 0, workspace as for Q4_0; each block adds
 * d * sum((q5 - 16) x).  Replaces the per-column GEMV of batched Q5_0. */
long zt_q5_0_tiled_bytes(int M, int K);
long zt_q5_0_tiled_scale_bytes(int M, int K);
long zt_q5_0_tiled_qh_bytes(int M, int K);
int zt_q5_0_tile(const void* A_q5, int M, int K, long qh_offset, long qs_offset, void* W_tiled, void* S_tiled,
                 void* H_tiled, zt_stream_t stream);
long zt_gemm_q5_0t_workspace_bytes(int M, int K, int N);
int zt_gemm_q5_0t_f32(const void* W_tiled, const void* S_tiled, const void* H_tiled, const float* B, float* C, int M,
                      int K, int N, void* workspace, long workspace_bytes, zt_stream_t stream);

/* ---- Ternary ----------------------------------------------------------- */

/* Replaces ternary_gemv_f32 (internal/cuda/kernels/ternary_gemv.cu:85-99),
 * the device half of TernaryGEMVGPU (compute/ternary_gemv_gpu.go:18-91):
 * y[M] = W[M,K] x[K], W row-aligned 2-bit codes, fp32 x and y. */
int zt_ternary_gemv_f32(const void* W_ternary, const float* x, float* y, int M, int K, zt_stream_t stream);

/* BitNet decode variant: int8 activations with a per-token fp32 scale and
 * one per-tensor fp32 weight scale, both by device pointer:
 *   y = float(sum_j w_j q_j) * (w_scale * x_scale).
 * No reference counterpart (TernaryGEMV takes fp32 x, TernaryStorage has no
 * scale: compute/ternary_gemv.go:12, tensor/ternary_storage.go:7-10); the
 * result equals TernaryGEMV(W, float(q)) * (w_scale * x_scale) bit for bit. */
int zt_ternary_gemv_i8(const void* W_ternary, const int8_t* x_q, const float* x_scale, const float* w_scale,
                       float* y, int M, int K, zt_stream_t stream);
/* Grouped BitNet GEMV: up to ZT_GROUP_MAX ternary matrices that read the
 * same int8 activations x_q[K] and x_scale (a layer's q/k/v, or gate/up)
 * in one launch (up to 3 matrices with K % 64 == 0 and K <= 65536 and
 * 16-byte aligned rows, else one launch per matrix).  No reference
 * counterpart (TernaryGEMV, compute/ternary_gemv.go:12, takes one matrix):
 * matrix i gets zt_ternary_gemv_i8(W_i, x_q, x_scale, w_scale_i, y_i,
 * rows_i, K) bit for bit (exact integer sums times the same scale product).
 * `descs` is a host array read during the call; rows == 0 skips a matrix.
 * n outside 1..ZT_GROUP_MAX, a bad descriptor or a misaligned x_q ->
 * InvalidValue. */
typedef struct zt_ternary_gemv_desc {
    const void* W;         /* row-aligned 2-bit codes, rows x ceil(K/4) bytes */
    const float* w_scale;  /* device pointer, one fp32 */
    float* y;              /* rows fp32 outputs */
    int rows;
    int reserved;          /* 0 */
} zt_ternary_gemv_desc;
int zt_ternary_gemv_i8_group(const zt_ternary_gemv_desc* descs, int n, const int8_t* x_q, const float* x_scale, int K,
                             zt_stream_t stream);
/* Codes -> fp32 {-1,0,+1} (TernaryStorage.Get, tensor/ternary_storage.go:39-47). */
int zt_dequant_ternary_f32(const void* W_ternary, float* out, int M, int K, zt_stream_t stream);
/* Host: flat TernaryStorage.RawBytes (tensor/ternary_storage.go:91-92) ->
 * row-aligned layout, the repack of compute/ternary_gemv_gpu.go:55-67.
 * out holds M*ceil(K/4) bytes. */
void zt_ternary_repack_rows(const void* raw, long M, long K, void* out);

/* ---- K-quants (Q4_K, Q5_K, Q6_K) and Q5_0 ------------------------------- */

/* Batch-1 GEMV y[M] = dequant(W)[M,K] x[K], fp32 x and y, W the raw
 * super-blocks [M, K/256] as uploaded by GPUEngine.UploadWeights
 * (compute/gpu_engine.go:817-874).  They replace gemv_q4k_f32 /
 * gemv_q5k_f32 / gemv_q6k_f32 (internal/cuda/kernels/gemv_q4k.cu:146-160,
 * gemv_q5k.cu:160-170, gemv_q6k.cu:135-145) behind KernelRunner.GemvQ4KF32 /
 * GemvQ5KF32 / GemvQ6KF32 (internal/gpuapi/kernels.go:50-63), whose ROCm
 * implementations return "not implemented"
 * (internal/gpuapi/rocm_kernels.go:113-123).  K % 256 != 0 -> InvalidValue,
 * as the reference launchers.  W: 16-byte aligned (Q6_K: 2-byte), x 16-byte. */
int zt_gemv_q4k_f32(const void* W, const float* x, float* y, int M, int K, zt_stream_t stream);
int zt_gemv_q5k_f32(const void* W, const float* x, float* y, int M, int K, zt_stream_t stream);
int zt_gemv_q6k_f32(const void* W, const float* x, float* y, int M, int K, zt_stream_t stream);

/* Q6_K split layout for the batch-1 GEMV (the same GemvQ6KF32 product over
 * a load-time regrouping; the reference reads the raw 210-byte
 * super-blocks, which are only 2-byte aligned).  zt_q6k_split writes the
 * raw super-blocks' bytes (W_q6k 2-byte aligned) as four naturally aligned
 * arrays over the T = M * K/256 super-blocks t = row * K/256 + sb: ql at
 * 128 t, qh at 128 T + 64 t, int8 scales at 192 T + 16 t, fp16 d at
 * 208 T + 2 t (zt_q6k_split_bytes = 210 T bytes; W_split 16-byte aligned).
 * zt_gemv_q6ks_f32 is zt_gemv_q6k_f32 on that layout (x 16-byte aligned,
 * K % 256 == 0, 210 T < 2^31, else InvalidValue). */
long zt_q6k_split_bytes(int M, int K);
int zt_q6k_split(const void* W_q6k, int M, int K, void* W_split, zt_stream_t stream);
int zt_gemv_q6ks_f32(const void* W_split, const float* x, float* y, int M, int K, zt_stream_t stream);

/* Replaces gemv_q5_0_f32 (internal/cuda/kernels/gemv_q5_0.cu:108-125) behind
 * KernelRunner.GemvQ5_0F32 (internal/gpuapi/kernels.go:65-69; ROCm stub
 * internal/gpuapi/rocm_kernels.go:125-127).  W is the RawBytesGPU layout,
 * qh_offset / qs_offset = Q5_0GPUQhOffset / Q5_0GPUQsOffset(M*K/32)
 * (tensor/quantized_q5_0.go:151-165).  K % 32 != 0 -> InvalidValue. */
int zt_gemv_q5_0_f32(const void* W, const float* x, float* y, int M, int K, int qh_offset, int qs_offset,
                     zt_stream_t stream);

/* Device dequantizers, bit-exact with Q4KStorage / Q5KStorage / Q6KStorage
 * .Dequantize (tensor/quantized_kquant.go:263-277, 579-593, 412-426); they
 * replace dequant_q4k_f32 etc. behind KernelRunner.DequantQ4KF32 /
 * DequantQ5KF32 / DequantQ6KF32 (internal/gpuapi/kernels.go:71-76).  W is
 * [rows, K] raw super-blocks, out rows*K floats, K % 256 == 0. */
int zt_dequant_q4k_f32(const void* W, float* out, int rows, int K, zt_stream_t stream);
int zt_dequant_q5k_f32(const void* W, float* out, int rows, int K, zt_stream_t stream);
int zt_dequant_q6k_f32(const void* W, float* out, int rows, int K, zt_stream_t stream);
/* Bit-exact with Q5_0Storage.Dequantize (tensor/quantized_q5_0.go:26-45,
 * 75-90) over the raw 22-byte blocks, the layout dequant_q5_0_f32 reads
 * (internal/cuda/kernels/dequant_q5_0.cu:18-67; KernelRunner.DequantQ5_0F32,
 * internal/gpuapi/kernels.go:77).  K % 32 == 0. */
int zt_dequant_q5_0_f32(const void* W, float* out, int rows, int K, zt_stream_t stream);

/* Host: Q5_0Storage.RawBytes (22-byte blocks) -> RawBytesGPU
 * (tensor/quantized_q5_0.go:118-147); offsets as Q5_0GPUQhOffset /
 * Q5_0GPUQsOffset (:151-165); out holds zt_q5_0_gpu_bytes(nblk) bytes. */
long zt_q5_0_gpu_qh_offset(long nblk);
long zt_q5_0_gpu_qs_offset(long nblk);
long zt_q5_0_gpu_bytes(long nblk);
void zt_q5_0_raw_to_gpu(const void* raw, long nblk, void* out);

/* ---- int4 / int8 GEMMs with fp32 activations -------------------------- */

/* The reference's group-quantized int4 and plain int8 GEMMs
 * (internal/cuda/kernels/gemm_int4.h, gemm_int8.h; gemm_int4.cu:29-144,
 * gemm_int8.cu:16-73; Go GemmInt4F32 / GemmInt4F32RMul / GemmInt8F32,
 * gemm_quantized.go:24-89), same argument order.  int4 values are signed
 * [-8, 7], two a byte, the even element in the low nibble; a weight is
 * float32(v - zero) * scale with fp32 scales and uint8 zeros per group.
 *   zt_gemm_int4_f32: C[M, N] = dequant(A) B, A [M, K/2] packed, B [K, N]
 *     fp32, scales / zeros [M, ceil(K / group_size)] (groups along K).
 *   zt_gemm_int4_f32_rmul: C[batch, out] = B dequant(W), W [in, out/2]
 *     packed along out, B [batch, in] fp32, scales / zeros
 *     [in, ceil(out / group_size)] (groups along out).
 *   zt_gemm_int8_f32: C[M, N] = float(A) B, A [M, K] int8.
 * Errors as the reference's launchers: an odd K (rmul: odd out_features) or
 * group_size <= 0 -> InvalidValue (1); also negative sizes or NULL buffers.
 * An empty M, N (batch, out) is a no-op; K = 0 writes zeros.  Any shape and
 * alignment is accepted; batches of 1-4 on K % 16 == 0 (int4 also
 * group_size % 16 == 0, A 8-byte and B 16-byte aligned; int8 A and B
 * 16-byte aligned) take the streaming GEMV kernels, everything else an fp32
 * MFMA GEMM.  Results equal the reference's within fp32 summation order. */
int zt_gemm_int4_f32(const void* A, const float* B, float* C, const float* scales, const void* zeros, int M, int K,
                     int N, int group_size, zt_stream_t stream);
int zt_gemm_int4_f32_rmul(const void* W, const float* B, float* C, const float* scales, const void* zeros, int batch,
                          int in_features, int out_features, int group_size, zt_stream_t stream);
int zt_gemm_int8_f32(const void* A, const float* B, float* C, int M, int K, int N, zt_stream_t stream);

/* ---- measurement ------------------------------------------------------- */

/* No counterpart in the reference: a plain streaming read of nbytes at p
 * (16-byte aligned; a trailing partial 16 bytes is not read), 16 bytes a lane
 * with nontemporal loads, no arithmetic.  Its time is the ceiling a GEMV
 * over the same bytes is compared with (the benchmark's `ceiling`).  sink
 * (4 bytes of device memory) is written only if the data xor-reduces to a
 * fixed key, which keeps the loads live. */
int zt_bench_stream_read(const void* p, long nbytes, void* sink, zt_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* ZT_HIP_H */

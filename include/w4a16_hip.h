/*
 * w4a16_hip.h -- C ABI of the MI355X (gfx950) W4A16 linear-layer library.
 *
 * FP16 activations [M, K] times packed INT4 weights [N, K/2] (two's complement
 * nibbles, even k in the low nibble) with one FP16 scale per `group_size`
 * weights along K, giving FP16 output [M, N]:
 *
 *     out[m][n] = fp16_rn( sum_k fp32(x[m][k]) * code[n][k] * fp32(scale[n][k / group_size]) )
 *
 * All pointers are device pointers; nothing here allocates, synchronises or
 * keeps state between calls, so every entry point is safe inside HIP graph
 * capture. Work is enqueued on `stream` (a hipStream_t; NULL = legacy stream).
 *
 * Return value: W4A16_OK (0) or one of the W4A16_ERR_* codes below;
 * w4a16_last_error() returns the message of the most recent failure on the
 * calling thread.
 */
#ifndef W4A16_HIP_H
#define W4A16_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define W4A16_OK 0
#define W4A16_ERR_GROUP_SIZE 1       /* group_size <= 0, odd, or not a multiple of 32 (dequantize) */
#define W4A16_ERR_SHAPE 2            /* inconsistent M/N/K/scale shapes */
#define W4A16_ERR_ALIGNMENT 3        /* pointer alignment the entry point requires is not met */
#define W4A16_ERR_NULL 4             /* NULL pointer with non-empty work */
#define W4A16_ERR_CONFIG 5           /* bad environment selector or tuning argument */
#define W4A16_ERR_LAUNCH 6           /* HIP reported an error at launch */
#define W4A16_ERR_TOO_LARGE 7        /* a dimension exceeds what the kernels index */

/* Kernel families, as reported by w4a16_plan_linear / accepted by w4a16_linear_f16_tuned. */
#define W4A16_KERNEL_NONE 0          /* M*N == 0: nothing launched */
#define W4A16_KERNEL_VALU 1          /* VALU dot2 GEMV, activations staged in LDS (M <= 8) */
#define W4A16_KERNEL_MFMA 2          /* fp16 MFMA 16x16x32 tiles, M zero-padded to 16 (M <= 8) */
#define W4A16_KERNEL_GENERIC 3       /* any M, any even group_size, any alignment */
#define W4A16_KERNEL_DIAG 4          /* M = 1 on fp16 MFMA, group dots on the 16x16 diagonal */
#define W4A16_KERNEL_VALU_OFFSET 5   /* VALU kernel, decode without f16 fix-ups, per-chunk offset correction */
#define W4A16_KERNEL_ONESHOT 6       /* VALU GEMV, every weight of a wavefront's rows requested at once (M <= 4) */
#define W4A16_KERNEL_MFMA_ONESHOT 7  /* fp16 MFMA, loads up front, activations staged in LDS (M <= 16, K <= 8192) */
#define W4A16_KERNEL_MFMA_PAIR 8     /* fp16 MFMA on 8 rows x 2 groups, loads up front (2 <= M <= 8, staged M*K in LDS) */
#define W4A16_KERNEL_STREAM 9        /* VALU GEMV, resident workgroups streaming rows along K (M = 1, K <= 32768) */
#define W4A16_KERNEL_GEMM 10         /* fp16 MFMA GEMM on weights decoded in registers (M > 16, prompts) */
#define W4A16_KERNEL_PAIR_STREAM 11  /* paired MFMA, resident workgroups streaming 8-row blocks (2 <= M <= 8) */
#define W4A16_KERNEL_GEMM_LDS 12     /* GEMM with the activation block staged in LDS per round of groups (large M) */
#define W4A16_KERNEL_PAIR_SPLIT 13   /* PAIR_STREAM over K slices, fp32 partials in a workspace + reduce (2 <= M <= 8) */
#define W4A16_KERNEL_GEMM32 14       /* GEMM_LDS on 32x32x16 MFMA tiles (large M, rows of up to 4096 weights) */
#define W4A16_KERNEL_PAIR_RING 15    /* fp16 MFMA on 8 rows x 2 groups, a ring of loads in flight per wavefront (M <= 16) */

/*
 * Fused W4A16 linear layer.
 * Replaces int4_linear_cuda (reference csrc/int4_linear_kernel.cu:641-802),
 * registered as torch op w4a16::linear (reference csrc/int4_linear.cpp:16-28).
 * activations: fp16 [M, K] row-major; packed_weights: uint8 [N, K/2];
 * scales: fp16 [N, K/group_size]; output: fp16 [M, N].
 * group_size == 128 with 16-byte aligned activations and weights and M <= 8
 * takes the tuned kernels and M > 8 the W4A16 GEMM (operands below 4 GiB;
 * its LDS-staged forms from M = 64; M = 9..16 on rows longer than 4096
 * weights the paired kernel with 16 row slots where its plan keeps at most 2
 * wavefronts on weight blocks, and N >= 8192 with rows of up to 2048 the
 * one-shot MFMA kernel; W4A16_DECODE = mfma_oneshot or mfma_pair selects
 * those kernels for M = 9..16); anything else takes the generic
 * kernel (the reference routes every M > 8 to its naive kernel).
 * Environment, read at every call, with the reference's semantics
 * (csrc/int4_linear_kernel.cu:459-491, :713-749):
 *   W4A16_DECODE = v1|v2|v3 selects an M = 1 variant on the tuned path
 *   (v1: looped VALU kernel, v2: diagonal MFMA kernel, v3: offset-decode
 *   VALU kernel, each one row per wavefront); v4, auto, unset and any
 *   value not listed here are the default routing. This build's family
 *   names oneshot|valu|valu_offset|mfma|mfma_oneshot|mfma_pair|stream|
 *   pair_stream select a kernel family for M <= 8 (and mfma_oneshot /
 *   mfma_pair for M = 9..16).
 *   W4A16_ROWS_PER_WARP = 1|2|4 sets output rows per wavefront at M = 1
 *   (the default routing then runs the looped VALU kernel with that many
 *   rows); it is read only at M = 1 on the tuned path and not under
 *   v1..v3, and there any other value is W4A16_ERR_CONFIG.
 */
int w4a16_linear_f16(const void* activations, const uint8_t* packed_weights,
                     const void* scales, void* output, int64_t M, int64_t N,
                     int64_t K, int64_t group_size, void* stream);

/*
 * Bytes of workspace w4a16_linear_ws_f16 uses for these sizes with group
 * size 128 and 16-byte aligned activations and weights under the default
 * routing (0: none). No reference counterpart (the reference's kernels keep
 * no partial sums).
 */
int64_t w4a16_linear_workspace_bytes(int64_t M, int64_t N, int64_t K, int64_t group_size);

/*
 * w4a16_linear_f16 with a caller workspace (device memory, 16-byte aligned,
 * contents ignored; workspace_bytes >= w4a16_linear_workspace_bytes): with
 * it, M = 3..8 layers with K > 16384 and N >= 8192 take
 * W4A16_KERNEL_PAIR_SPLIT, the streaming paired kernel over K slices, and
 * M = 12..16 layers of K = 5632 (N <= 4096), 8192 or 14336 (N <= 8192) and
 * M = 3..8 layers of K = 28672 (N = 4096..8192) and M = 5..8 layers of
 * K = 8192 with N >= 16384 the paired ring kernel over K slices; the fp32
 * partial sums are added in slice
 * order by a second launch. workspace == NULL routes exactly as w4a16_linear_f16;
 * a smaller non-NULL workspace is W4A16_ERR_CONFIG. The torch op
 * w4a16::linear (reference csrc/int4_linear.cpp:16-28) calls this entry
 * point with a workspace from the caching allocator.
 */
int w4a16_linear_ws_f16(const void* activations, const uint8_t* packed_weights,
                        const void* scales, void* output, int64_t M, int64_t N,
                        int64_t K, int64_t group_size, void* workspace,
                        int64_t workspace_bytes, void* stream);

/* Bytes of device scratch w4a16_linear_noalloc_f16 holds per GPU (8 MiB). */
#define W4A16_NOALLOC_SCRATCH_BYTES (8LL << 20)

/*
 * w4a16_linear_ws_f16's routing (split-K kernel included) with no allocation
 * of any kind: the split-K partial sums go to a device array of
 * W4A16_NOALLOC_SCRATCH_BYTES that the library carries (one per GPU, held
 * until the process ends), so the call makes no hipMalloc, hipFree or
 * allocating library call. No counterpart in the reference (its kernels
 * keep no partial sums): it is for callers that cannot allocate, such as
 * code under HIP graph capture, tight serving loops or harnesses that
 * forbid allocation. Results are bit-identical to w4a16_linear_ws_f16 with
 * a caller workspace, except for a layer whose split-K partials would need
 * more than the scratch (slices * M * N * 4 bytes): it takes the route of
 * w4a16_linear_f16 (no workspace, no split-K), bit-identical to that entry
 * point instead. Every call on
 * one GPU shares that GPU's scratch: calls that overlap on one GPU (two
 * streams, two threads) race and must be serialised by the caller. The
 * first call on a device that needs the scratch looks up its address
 * (hipGetSymbolAddress); make that call outside graph capture.
 */
int w4a16_linear_noalloc_f16(const void* activations, const uint8_t* packed_weights,
                             const void* scales, void* output, int64_t M, int64_t N,
                             int64_t K, int64_t group_size, void* stream);

/*
 * Dequantize packed INT4 weights to fp16 [N, K]: out = fp16_rn(code * scale),
 * bit-identical to reference w4a16/reference.py:6-46 followed by .to(float16).
 * Replaces int4_dequantize_cuda (reference csrc/int4_linear_kernel.cu:805-867),
 * registered as torch op w4a16::dequantize (reference csrc/int4_linear.cpp:20-23).
 * Requires group_size a positive multiple of 32 and 16-byte aligned weights,
 * as the reference does.
 */
int w4a16_dequantize_f16(const uint8_t* packed_weights, const void* scales,
                         void* output, int64_t N, int64_t K, int64_t group_size,
                         void* stream);

/*
 * Shape validator shared by the torch op and host-only tests. Arguments are
 * the sizes the three tensors carry. Returns W4A16_OK or an error code whose
 * w4a16_last_error() text matches the reference's TORCH_CHECK messages
 * (reference csrc/int4_linear_kernel.cu:671-691).
 */
int w4a16_check_linear_shapes(int64_t act_rows, int64_t act_cols,
                              int64_t packed_rows, int64_t packed_cols,
                              int64_t scale_rows, int64_t scale_cols,
                              int64_t group_size);

/* Same for dequantize (reference csrc/int4_linear_kernel.cu:826-841). */
int w4a16_check_dequantize_shapes(int64_t packed_rows, int64_t packed_cols,
                                  int64_t scale_rows, int64_t scale_cols,
                                  int64_t group_size, uint64_t packed_address);

/*
 * Which kernel and launch shape w4a16_linear_f16 would use for these
 * arguments (reads the same environment selectors). Pointers are used only
 * for their alignment. No reference counterpart: it exposes the dispatcher's
 * choice (reference csrc/int4_linear_kernel.cu:706-798) to tests and benches.
 */
int w4a16_plan_linear(const void* activations, const uint8_t* packed_weights,
                      int64_t M, int64_t N, int64_t K, int64_t group_size,
                      int* kernel, int* rows, int* splits, int* unroll,
                      int* max_blocks);

/* The same for w4a16_linear_ws_f16 with a workspace (the split-K routes). */
int w4a16_plan_linear_ws(const void* activations, const uint8_t* packed_weights,
                         int64_t M, int64_t N, int64_t K, int64_t group_size,
                         int* kernel, int* rows, int* splits, int* unroll,
                         int* max_blocks);

/*
 * w4a16_linear_f16 with an explicit kernel family and launch shape, for
 * tuning sweeps.
 *   W4A16_KERNEL_VALU: rows = output rows per wavefront task (1|2|4),
 *     splits = wavefronts per workgroup (1..4), unroll = chunks in flight per
 *     row (1|2|4|8; 8 needs rows <= 2), max_blocks = grid cap (0 = none).
 *   W4A16_KERNEL_MFMA: rows = 16-row blocks per wavefront (1|2|4),
 *     splits = wavefronts splitting K (1..8), unroll = groups in flight (1|2|4).
 *   W4A16_KERNEL_VALU_OFFSET (M = 1 only): as W4A16_KERNEL_VALU.
 *   W4A16_KERNEL_DIAG (M = 1 only): rows = output rows per wavefront task
 *     (1|2|4), splits = wavefronts per workgroup (1..4), unroll = 1 KiB spans
 *     in flight per row (1|2|4; 4 needs rows <= 2), max_blocks = grid cap.
 *   W4A16_KERNEL_ONESHOT (M <= 4): rows = output rows per wavefront (1|2; 4
 *     at M = 1 with splits 4 and unroll <= 8),
 *     splits = wavefronts per workgroup (4|8), unroll = 1 KiB loads per row
 *     per lane (0 = the smallest that covers K; else >= ceil(K / 2048) and
 *     one of 1..8, 10, 12, 14, 16), max_blocks ignored.
 *   W4A16_KERNEL_MFMA_ONESHOT (K <= 8192, M*K*2 + K/2 + 16 KiB of LDS):
 *     rows = 16-row blocks per workgroup (1|2), splits = wavefronts
 *     splitting K (4|8), unroll = groups per wavefront (0 = ceil(K / 128 /
 *     splits); else enough to cover K: 1..8, 10, 12, 14, 16 with 4 splits,
 *     1..8 with 8), max_blocks ignored.
 *   W4A16_KERNEL_MFMA_PAIR (2 <= M <= 16, K <= 32768; M > 8 runs in one
 *     launch with 16 row slots where that shape is instantiated and fits in
 *     LDS, else as two launches over rows [0, ceil(M/2)) and the rest, each
 *     choosing its own staging chunk, rows ignored): splits = wavefronts
 *     splitting the K / 256 group pairs (2|4|8), max_blocks = 8-row-block
 *     wavefronts per workgroup (1|2|4|8, splits * max_blocks <= 16), unroll =
 *     group pairs per wavefront (0 = ceil(K / 256 / splits); else with
 *     splits * unroll >= ceil(K / 256)), rows = group pairs of activations
 *     staged in LDS at a time (0 = automatic; splits * unroll = whole rows:
 *     unroll 1..8; 8 = double-buffered chunks: splits 4 with max_blocks
 *     1|2|4 and unroll 7|8, or splits 8 with max_blocks 1|2 and unroll
 *     3..8|10|12|14|16);
 *     staged activations, biases and reduction within 160 KiB of LDS.
 *   W4A16_KERNEL_STREAM (M = 1, K <= 32768): rows = output rows per
 *     wavefront task (1|2|4 with unroll 2|3|4, 8 with unroll 2), splits =
 *     wavefronts per workgroup (4|8), unroll = 1 KiB loads per row in flight
 *     (the ring runs on into the next rows when a row has fewer steps),
 *     max_blocks = grid (0 = the workgroups resident on the device at once).
 *   W4A16_KERNEL_PAIR_RING (1 <= M <= 16, K a multiple of 256, scales
 *     4-byte aligned): splits = wavefronts splitting K, rows = wavefronts
 *     on 8-row blocks per workgroup, unroll = group pairs in flight per
 *     wavefront, max_blocks = K slices (0 or 1 = none; 2..16 store fp32
 *     partial sums in a workspace of max_blocks * M * N * 4 bytes, then a
 *     reduce launch adds them in slice order); with P = ceil(K / 256 /
 *     slices) pairs per slice, (splits, rows, ceil(P / splits), unroll) at
 *     M = 1 one of (1,3,8,8) (1,3,8,7) (1,3,8,6) (1,8,8,4) (2,2,8,8)
 *     (2,2,8,7) (1,8,16,6) (4,1,6,6) (2,4,16,4) (2,4,16,6) (1,7,32,6)
 *     (2,2,28,10) (2,4,56,6); at M = 2..4 (4,1,2,2)
 *     (1,4,8,6) (1,4,8,7) (2,2,8,4) (2,2,8,6) (1,8,16,6) (8,1,3,3) (2,4,16,4)
 *     (4,2,14,6); at
 *     M = 5..8 (4,1,2,2) (1,4,8,6) (4,2,4,4) (1,8,16,6) (2,4,16,4) (2,4,16,5) (11,1,2,2); at M =
 *     9..16 (exact decode: the dequantized fp16 weights in the B operand)
 *     (8,1,1,1) (4,2,2,2) (2,4,4,4) (1,4,8,4), and with K slices (1,8,3,3)
 *     (1,8,14,4) (1,8,16,4); at M = 2..4 with K slices (1,8,28,4); at M =
 *     5..8 with K slices (1,8,14,2) (1,8,16,3) (1,4,7,2), whose wavefronts
 *     each take two 8-row blocks (a workgroup covers 16 * rows rows).
 *   W4A16_KERNEL_PAIR_STREAM (2 <= M <= 8, whole rows of activations in
 *     LDS): rows = wavefronts per workgroup (0 = the fewest that cover N / 8
 *     row blocks with the workgroups resident at once; else 1..16), unroll =
 *     group pairs in flight per wavefront (2|3|4|6), max_blocks = grid cap
 *     (0 = none), splits ignored.
 *   W4A16_KERNEL_PAIR_SPLIT (2 <= M <= 8, K <= 65536, needs a workspace of
 *     splits * M * N * 4 bytes): splits = K slices (2..16, every slice
 *     non-empty, M K / splits activations in LDS), rows = wavefronts per
 *     workgroup (0 = automatic; else 1..16), unroll = group pairs in flight
 *     (2|3|4|6), max_blocks = workgroups per slice cap (0 = none).
 *   W4A16_KERNEL_GEMM (any M; every operand below 4 GiB): rows = 16-row
 *     activation tiles per wavefront (1|2|4), max_blocks = 16-row weight
 *     tiles per wavefront (1|2|4), splits = wavefronts splitting K (2|4|8;
 *     not 8 with rows = max_blocks = 4), unroll ignored.
 *   W4A16_KERNEL_GEMM_LDS (any M; every operand below 4 GiB): rows = 16-row
 *     activation tiles per wavefront (2|4), max_blocks = 16-row weight tiles
 *     per wavefront (2|4), unroll = wavefronts sharing each staged round on
 *     different weight tiles (2|4), splits = wavefronts splitting K (1|2|4;
 *     4 needs unroll 2 and rows * max_blocks < 16, or rows * max_blocks < 8).
 *   W4A16_KERNEL_GEMM32 (any M; every operand below 4 GiB): as
 *     W4A16_KERNEL_GEMM_LDS with 32-row tiles; (rows, max_blocks, unroll,
 *     splits) one of (4, 2, 4, 1), (4, 1, 4, 1), (2, 1, 4, 2), (2, 2, 2, 2),
 *     (2, 2, 4, 1), (4, 1, 2, 2), (2, 1, 2, 4), (2, 1, 1, 4).
 *   W4A16_KERNEL_GENERIC: other arguments ignored.
 * The VALU and MFMA families need group_size 128, M <= 8 (16 for
 * W4A16_KERNEL_MFMA_ONESHOT, 2..16 for W4A16_KERNEL_MFMA_PAIR) and 16-byte
 * aligned activations and weights. workspace / workspace_bytes: as for
 * w4a16_linear_ws_f16 (only W4A16_KERNEL_PAIR_SPLIT and W4A16_KERNEL_PAIR_RING
 * with K slices use them; NULL / 0 otherwise). No reference counterpart (the reference's W4A16_DECODE /
 * W4A16_ROWS_PER_WARP selectors play this role).
 */
int w4a16_linear_f16_tuned(const void* activations, const uint8_t* packed_weights,
                           const void* scales, void* output, int64_t M, int64_t N,
                           int64_t K, int64_t group_size, void* stream,
                           int kernel, int rows, int splits, int unroll, int max_blocks,
                           void* workspace, int64_t workspace_bytes);

/* Message of the last failure on this thread ("" if none). */
const char* w4a16_last_error(void);

/* Library version string. */
const char* w4a16_version(void);

#ifdef __cplusplus
}
#endif

#endif /* W4A16_HIP_H */

// gfx950 kernels of the W4A16 linear layer.
//
// Shared layout facts (all kernels):
//   x       fp16 [M, K] row-major (activations)
//   w       uint8 [N, K/2] row-major, nibble i of a 32-bit word = weight i
//   scales  fp16 [N, K/G]
//   out     fp16 [M, N]
// A "chunk" is 16 bytes of one weight row = 32 weights; with G = 128 a group
// is 4 chunks = 64 bytes.
#pragma once

#include "w4a16_device.h"

namespace w4a16 {

// ---------------------------------------------------------------------------
// VALU GEMV (M = 1..8 activation rows, template), G = 128.
//
// Work unit ("task"): R consecutive output rows, handled by one wavefront over
// the whole of K. Lane l takes chunks l, l + 64, l + 128, ... of each of the
// R rows, U chunks per row per step, so every load instruction reads 1 KiB of
// contiguous weights. Each 16-byte chunk is decoded once (unpack8) and dotted
// with the M activation rows by v_dot2_f32_f16 (fp16 products, fp32 sums);
// the chunk dot is scaled by its group's fp32 scale (the reference's kernel
// scales per-chunk partials the same way, csrc/int4_linear_kernel.cu:390).
// The row sum is a DPP wavefront reduction; lane 0 stores it.
//
// A workgroup of W wavefronts stages the activations once in LDS, permuted to
// the unpack8 pair order and unit-major (unit q of chunk c of activation row m
// at xs[(m*4 + q) * C + c]: lanes reading consecutive chunks hit consecutive
// 16-byte slots), then each wavefront walks its (task, step) sequence --
// tasks blockIdx.x*W + wave, + gridDim.x*W -- with two register buffers: the
// loads of the next step are in flight while the current step computes. The
// first step's loads are issued before the activation staging. Task and row
// indices are wavefront-uniform (scalar registers), so each load is a scalar
// row base plus a per-lane 32-bit offset. Rows past N re-read row N-1 and are
// not stored.
// ---------------------------------------------------------------------------
// Copy the M activation rows into LDS, permuted to the unpack8 pair order,
// unit-major: unit q (8 halves) of chunk c of row m goes to xs[(m*4 + q)*C + c].
// Loads are issued in batches of 8 per thread before any is waited on, so the
// whole copy costs about one L2 round trip instead of one per unit.
// With SUMS, also store per chunk the fp32 sums of its even-k and odd-k
// activations (float2 at sums[m*C + c]) for the offset decode.
template <int M, bool SUMS>
__device__ __forceinline__ void stage_activations(const f16* __restrict__ x, u32x4* xs, float2* sums, int K,
                                                  int C) {
    constexpr int kBatch = 8;
    const int units_per_row = K >> 3;
    const int total = M * units_per_row;
    const int T = blockDim.x;
    for (int base = threadIdx.x; base < total; base += kBatch * T) {
        u32x4 a[kBatch];
#pragma unroll
        for (int j = 0; j < kBatch; ++j) {
            const int i = base + j * T;
            if (i < total) a[j] = *reinterpret_cast<const u32x4*>(x + (size_t)i * 8);
        }
#pragma unroll
        for (int j = 0; j < kBatch; ++j) {
            const int i = base + j * T;
            const int m = M == 1 ? 0 : i / units_per_row;
            const int u = i - m * units_per_row;
            if (i < total) xs[(m * 4 + (u & 3)) * C + (u >> 2)] = permute8(a[j]);
            if (SUMS) {
                // even k = low halves, odd k = high halves of the 4 words
                const f16x2 one = {(f16)1.0f, (f16)1.0f};
                float ev = 0.0f, od = 0.0f;
                if (i < total) {
                    const f16x2 w0 = as_f16x2(a[j].x), w1 = as_f16x2(a[j].y), w2 = as_f16x2(a[j].z),
                                w3 = as_f16x2(a[j].w);
                    ev = ((float)w0.x + (float)w1.x) + ((float)w2.x + (float)w3.x);
                    od = ((float)w0.y + (float)w1.y) + ((float)w2.y + (float)w3.y);
                }
                (void)one;
                // the 4 units of a chunk sit in 4 consecutive lanes (T is a multiple of 64, base % 4 == tid % 4)
                ev += dpp<0xB1>(ev);
                od += dpp<0xB1>(od);
                ev += dpp<0x4E>(ev);
                od += dpp<0x4E>(od);
                if (i < total && (u & 3) == 0) sums[m * C + (u >> 2)] = make_float2(ev, od);
            }
        }
    }
}

template <int M, int R, int U>
struct ValuStep {
    u32x4 w[U][R];
    f16 s[U][R];
};

template <int M, int R, int U>
__device__ __forceinline__ void valu_load(ValuStep<M, R, U>& b, const uint8_t* __restrict__ w,
                                          const f16* __restrict__ scales, int task, int step, int lane,
                                          int N, int C, int G, uint32_t row_bytes) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int n = min(task * R + r, N - 1);
        const uint8_t* wrow = w + (size_t)n * row_bytes;                 // wavefront-uniform
        const uint8_t* srow = reinterpret_cast<const uint8_t*>(scales + (size_t)n * G);
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int c = (step * U + u) * 64 + lane;
            if (c < C) {
                // unsigned 32-bit per-lane byte offsets: scalar base + vector offset addressing
                const uint32_t c32 = (uint32_t)c;
                b.w[u][r] = load_stream(reinterpret_cast<const u32x4*>(wrow + c32 * 16u));
                b.s[u][r] = *reinterpret_cast<const f16*>(srow + (c32 >> 2) * 2u);
            }
        }
    }
}


// One step of U chunks per row. Exact path: unpack8 (codes exact in f16),
// dot2 into one fp32 sum per chunk. Offset path (OFFSET): dot2 of the
// un-fixed values into an even-k sum E = sum x (1024 + v) and an odd-k sum
// O = sum x (1024 + 16 v); with v = s + 8 the chunk dot is
//   E - 1032 * Sx_even + (O - 1152 * Sx_odd) / 16,
// where Sx_even / Sx_odd are the chunk's activation sums staged in LDS.
template <int M, int R, int U, bool OFFSET>
__device__ __forceinline__ void valu_compute(const ValuStep<M, R, U>& b, const u32x4* xs, const float2* sums,
                                             float (&acc)[R][M], int step, int lane, int C) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int c = (step * U + u) * 64 + lane;
        if (c < C) {
            float d[R][M], e[R][M];
#pragma unroll
            for (int r = 0; r < R; ++r)
#pragma unroll
                for (int m = 0; m < M; ++m) d[r][m] = e[r][m] = 0.0f;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                u32x4 xa[M];
#pragma unroll
                for (int m = 0; m < M; ++m) xa[m] = xs[(m * 4 + q) * C + c];
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    const Codes8 cw = OFFSET ? unpack8_offset(b.w[u][r][q]) : unpack8(b.w[u][r][q]);
#pragma unroll
                    for (int m = 0; m < M; ++m) {
                        if (OFFSET) {
                            d[r][m] = __builtin_amdgcn_fdot2(as_f16x2(xa[m].x), cw.p[0], d[r][m], false);
                            e[r][m] = __builtin_amdgcn_fdot2(as_f16x2(xa[m].y), cw.p[1], e[r][m], false);
                            d[r][m] = __builtin_amdgcn_fdot2(as_f16x2(xa[m].z), cw.p[2], d[r][m], false);
                            e[r][m] = __builtin_amdgcn_fdot2(as_f16x2(xa[m].w), cw.p[3], e[r][m], false);
                        } else {
                            d[r][m] = __builtin_amdgcn_fdot2(as_f16x2(xa[m].x), cw.p[0], d[r][m], false);
                            d[r][m] = __builtin_amdgcn_fdot2(as_f16x2(xa[m].y), cw.p[1], d[r][m], false);
                            d[r][m] = __builtin_amdgcn_fdot2(as_f16x2(xa[m].z), cw.p[2], d[r][m], false);
                            d[r][m] = __builtin_amdgcn_fdot2(as_f16x2(xa[m].w), cw.p[3], d[r][m], false);
                        }
                    }
                }
            }
            float2 sx[M];
            if (OFFSET) {
#pragma unroll
                for (int m = 0; m < M; ++m) sx[m] = sums[m * C + c];
            }
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const float s = (float)b.s[u][r];
#pragma unroll
                for (int m = 0; m < M; ++m) {
                    float dot = d[r][m];
                    if (OFFSET) {
                        dot = __builtin_fmaf(-1032.0f, sx[m].x, dot);
                        const float odd = __builtin_fmaf(-1152.0f, sx[m].y, e[r][m]);
                        dot = __builtin_fmaf(odd, 0.0625f, dot);
                    }
                    acc[r][m] = __builtin_fmaf(dot, s, acc[r][m]);
                }
            }
        }
    }
}

template <int M, int R>
__device__ __forceinline__ void valu_finish(float (&acc)[R][M], f16* __restrict__ out, int task, int lane, int N) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
#pragma unroll
        for (int m = 0; m < M; ++m) {
            const float v = wave_sum(acc[r][m]);
            acc[r][m] = 0.0f;
            if (lane == 0 && task * R + r < N) out[(size_t)m * N + task * R + r] = (f16)v;
        }
    }
}

template <int M, int R, int U, bool OFFSET>
__global__ void __launch_bounds__(256)
gemv_valu(const f16* __restrict__ x, const uint8_t* __restrict__ w,
          const f16* __restrict__ scales, f16* __restrict__ out, int N, int K, int num_tasks) {
    extern __shared__ __align__(16) uint8_t smem[];
    u32x4* xs = reinterpret_cast<u32x4*>(smem);
    float2* sums = reinterpret_cast<float2*>(smem + (size_t)M * K * 2);   // OFFSET only

    const int W = blockDim.x >> 6;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int C = K >> 5;   // 16-byte chunks per row
    const int G = K >> 7;   // groups per row
    const int steps = (C + 64 * U - 1) / (64 * U);
    const uint32_t row_bytes = (uint32_t)(K >> 1);

    const int task0 = blockIdx.x * W + wave;
    const int task_stride = gridDim.x * W;
    const int my_tasks = task0 < num_tasks ? (num_tasks - 1 - task0) / task_stride + 1 : 0;
    const int units = my_tasks * steps;

    ValuStep<M, R, U> buf0, buf1;
    // (task, step) of the unit in buf0; buf1 holds the one after it
    int task = task0, step = 0;
    // The first two units' weights are requested before the activation
    // staging, so the staging latency overlaps the weight stream.
    int task1 = task, step1 = step + 1;
    if (step1 == steps) { step1 = 0; task1 += task_stride; }
    if (units > 0) valu_load(buf0, w, scales, task, step, lane, N, C, G, row_bytes);
    if (units > 1) valu_load(buf1, w, scales, task1, step1, lane, N, C, G, row_bytes);

    stage_activations<M, OFFSET>(x, xs, sums, K, C);
    __syncthreads();

    float acc[R][M];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int m = 0; m < M; ++m) acc[r][m] = 0.0f;

    for (int u = 0; u < units; u += 2) {
        // buf0 holds unit u = (task, step), buf1 unit u+1 = (task1, step1)
        valu_compute<M, R, U, OFFSET>(buf0, xs, sums, acc, step, lane, C);
        if (step == steps - 1) valu_finish(acc, out, task, lane, N);
        if (u + 1 >= units) break;
        // unit u+2 -> buf0
        task = task1;
        step = step1 + 1;
        if (step == steps) { step = 0; task += task_stride; }
        if (u + 2 < units) valu_load(buf0, w, scales, task, step, lane, N, C, G, row_bytes);
        valu_compute<M, R, U, OFFSET>(buf1, xs, sums, acc, step1, lane, C);
        if (step1 == steps - 1) valu_finish(acc, out, task1, lane, N);
        // unit u+3 -> buf1
        task1 = task;
        step1 = step + 1;
        if (step1 == steps) { step1 = 0; task1 += task_stride; }
        if (u + 3 < units) valu_load(buf1, w, scales, task1, step1, lane, N, C, G, row_bytes);
    }
}

// ---------------------------------------------------------------------------
// One-shot VALU GEMV (M = 1..4 activation rows, template), G = 128.
//
// Every wavefront owns R output rows and requests ALL of their weights at
// once: a row is L = ceil(C / 64) loads of 1 KiB (lane l takes chunks l,
// l + 64, ...; lanes past C re-read the row's last chunk and drop it), so a
// wavefront has R * L loads in flight and the whole matrix is requested
// within the first few hundred cycles of the launch. There is no loop and no
// second round of tasks: the grid has ceil(N / R) wavefronts.
//
// Order of requests, which matters because a wavefront's loads return in
// issue order: first the workgroup's share of the activations (contiguous
// 16-byte units, so they come back first), then the scales, then the
// weights. The activations are permuted to the unpack8 pair order and
// written to LDS unit-major (unit q of chunk c of row m at
// xs[(m*4 + q) * C + c], conflict-free for lanes reading consecutive
// chunks); after one barrier each wavefront consumes its weights in the
// order they arrive.
//
// Offset decode (unpack8_offset: one v_bitop3 per pair, no f16 fix-ups):
// even-k codes arrive as 1024 + v and odd-k codes as 1024 + 16 v, v = s + 8.
// The staged activations carry the odd-k halves pre-scaled by 1/16 (exact
// for normal fp16), so each product is x s plus an offset 1032 x (even k)
// or 72 x (odd k). Staging also stores, per chunk c of activation row m,
// bias[m][c] = -(1032 sum_even x + 1152 sum_odd x/16) in fp32 (one quad of
// lanes per chunk, DPP quad sum), and every chunk dot starts its
// v_dot2_f32_f16 chain from that bias, so the chunk sum is sum x s up to
// fp32 rounding of sums of magnitude ~1032 |x| (relative error ~1e-3 or
// less on the outputs). Then the fp32 scale per chunk and a DPP row sum.
//
// Fused decode-step variants (M = 1 only; the plain op passes an empty
// GemvFusion and NORM = PAIRED = false):
//   NORM (norm_weight): the activation row is RMS-normalised while it is staged,
//     y = fp16((fp32(x) * rsqrt(mean(x^2) + eps)) * fp32(norm_weight)),
//     the fp32 operation order of an RMSNorm that returns fp16;
//   RESID (residual): out[n] = fp16(fp32(residual[n]) + fp32(fp16(dot))), the fp16
//     "x + linear(a)" of a residual stream (residual may alias out: each
//     row is read and written by the same lane);
//   PAIRED (R = 2): wavefront i owns rows i and i + N/2 of a [gate; up]
//     weight pair and stores out[i] = fp16(silu(g) * u) with g, u, silu(g)
//     each rounded to fp16 first, as fp16 tensors would be;
//   ARGMAX: the rows' fp16 logits (stored when out != nullptr) feed a greedy
//     argmax over all N rows in the kernel's tail (argmax_tail);
//   ROPE (R = 2, the q|k|v projection of a decode step, head_dim 64): the
//     first rope_pairs = (H + KV) * 32 wavefronts own rows 64 h + d and
//     64 h + d + 32 of q or k head h (d < 32), the rest own v rows 2 i and
//     2 i + 1; the epilogue rounds both rows to fp16, rotates q / k pairs by
//     the angle fp32(position) * inv_freq[d] (fp32 sincosf, as the separate
//     rotary step), stores the rotated rows and, when 0 <= position <
//     max_seq, writes k and v into cache slot `position`.
// ---------------------------------------------------------------------------

struct GemvFusion {
    const f16* norm_weight;   // nullptr: no RMSNorm prologue
    float eps;
    const f16* residual;      // nullptr: no residual add
    // greedy argmax epilogue (ARGMAX; see argmax_tail)
    uint32_t* counters;       // arrival counters, zero on entry and on return
    uint64_t* partials;       // one (logit, index) key per workgroup
    int64_t* token;
    int64_t* position;        // nullptr: not advanced
    const f16* table;         // nullptr: no embedding gather
    int64_t vocab;
    int hidden;
    f16* emb_out;
    // rotary + KV append epilogue (ROPE; position above)
    const float* inv_freq;    // [32]
    f16* k_cache;             // [KV][max_seq][64]
    f16* v_cache;
    int rope_heads;           // H (query heads)
    int rope_pairs;           // (H + KV) * 32
    int max_seq;
};

// Order-preserving key of an fp16 logit at index n: larger logit first,
// then smaller index (torch.argmax's first maximum); -0 counts as +0 and any
// NaN as the largest value, as torch.argmax treats them.
__device__ __forceinline__ uint64_t argmax_key(float v, int n) {
    v = v + 0.0f;
    const uint32_t b = __builtin_bit_cast(uint32_t, v);
    const uint32_t ord = v != v ? 0xFFFFFFFFu : ((b & 0x80000000u) ? ~b : (b | 0x80000000u));
    return ((uint64_t)ord << 32) | (uint64_t)(0xFFFFFFFFu - (uint32_t)n);
}

// Greedy argmax over all workgroups' rows in the GEMV's tail: each workgroup
// publishes its best key, and the last workgroup to arrive (two-level
// counters: one per slot blockIdx % 8, which spreads the arrivals over eight
// cache lines, then one over the slots; device-scope atomics and fences)
// reduces the keys, writes the token, advances the position, gathers the
// token's embedding row and returns the counters to zero for the next call.
// Two calls sharing counters must not overlap.
template <int R, int W>
__device__ __forceinline__ void argmax_tail(const float (&rowsum)[R], int row0, int N, const GemvFusion& fz,
                                            int wave, int lane) {
    __shared__ uint64_t wbest[W];
    __shared__ int last;
    __shared__ int64_t chosen;
    uint64_t best = 0;   // below every key
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const uint64_t key = argmax_key((float)(f16)rowsum[r], row0 + r);
        if (row0 + r < N && key > best) best = key;
    }
    if (lane == 0) wbest[wave] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint64_t b = wbest[0];
#pragma unroll
        for (int w = 1; w < W; ++w) b = wbest[w] > b ? wbest[w] : b;
        __hip_atomic_store(&fz.partials[blockIdx.x], b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __threadfence();
        const unsigned x = blockIdx.x & 7u;
        const unsigned in_slot = (gridDim.x + 7u - x) / 8u;
        const unsigned slots = gridDim.x < 8u ? gridDim.x : 8u;
        int is_last = 0;
        if (atomicAdd(&fz.counters[32u * (1u + x)], 1u) == in_slot - 1u) {
            __threadfence();
            is_last = atomicAdd(&fz.counters[0], 1u) == slots - 1u;
        }
        last = is_last;
    }
    __syncthreads();
    if (!last) return;
    __threadfence();
    uint64_t b = 0;
    for (int i = threadIdx.x; i < (int)gridDim.x; i += 64 * W) {
        const uint64_t v = __hip_atomic_load(&fz.partials[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        b = v > b ? v : b;
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const uint64_t o = (uint64_t)__shfl_xor((unsigned long long)b, off);
        b = o > b ? o : b;
    }
    if (lane == 0) wbest[wave] = b;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint64_t k = wbest[0];
#pragma unroll
        for (int w = 1; w < W; ++w) k = wbest[w] > k ? wbest[w] : k;
        const int64_t t = (int64_t)(0xFFFFFFFFu - (uint32_t)(k & 0xFFFFFFFFu));
        fz.token[0] = t;
        chosen = t;
        if (fz.position != nullptr) fz.position[0] += 1;
        __hip_atomic_store(&fz.counters[0], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
        for (int s = 0; s < 8; ++s)
            __hip_atomic_store(&fz.counters[32 * (1 + s)], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (fz.emb_out == nullptr) return;
    __syncthreads();
    const int64_t t = chosen;
    for (int i = threadIdx.x; i < fz.hidden; i += 64 * W)
        fz.emb_out[i] = (t >= 0 && t < fz.vocab) ? fz.table[t * fz.hidden + i] : (f16)0.0f;
}

template <int M, int R, int L, int W, bool NORM, bool PAIRED, bool ARGMAX = false, bool ROPE = false,
          bool RESID = false>
__global__ void __launch_bounds__(64 * W)
gemv_oneshot(const f16* __restrict__ x, const uint8_t* __restrict__ w,
             const f16* __restrict__ scales, f16* out, int N, int K, GemvFusion fz) {
    static_assert(!PAIRED || (M == 1 && R == 2), "paired rows are an M = 1, R = 2 layout");
    static_assert(!ROPE || (M == 1 && R == 2 && !PAIRED && !ARGMAX), "rotary rows are an M = 1, R = 2 layout");
    static_assert(!RESID || (M == 1 && !PAIRED && !ARGMAX && !ROPE), "the residual add is a plain-row M = 1 epilogue");
    static_assert(!ARGMAX || (M == 1 && !PAIRED), "the argmax epilogue is an M = 1 plain-row layout");
    static_assert(!NORM || M == 1, "the RMSNorm prologue normalises one activation row");
    extern __shared__ __align__(16) uint8_t smem[];
    u32x4* xs = reinterpret_cast<u32x4*>(smem);
    const int C = K >> 5;
    const int G = K >> 7;
    float* cbias = reinterpret_cast<float*>(smem + (size_t)M * K * 2);   // [M][C], after xs
    const uint32_t row_bytes = (uint32_t)(K >> 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int task = blockIdx.x * W + wave;
    // row r of this wavefront, and the number of valid tasks
    const int half = N >> 1;
    const bool rot = ROPE && task < fz.rope_pairs;   // a q / k rotary pair (else v rows)
    const int row0 = PAIRED ? task : ROPE ? (rot ? (task >> 5) * 64 + (task & 31) : 2 * task) : task * R;
    const int row_step = PAIRED ? half : (ROPE && rot) ? 32 : 1;
    const bool valid = (PAIRED || ROPE) ? task < half : row0 < N;

    // 1. activations: units i = m * 4C + u, u = 4c + q. Up to kFirst units
    // per thread are requested ahead of the weights; any rest (large M * K)
    // is copied after them. Every request is unconditional (indices past
    // the end are clamped to the last element and their data is dropped):
    // branches around loads would make the compiler wait for all
    // outstanding loads at each join.
    constexpr int T = 64 * W;
    constexpr int kPer = (M * 4 * 64 * L + T - 1) / T;
    constexpr int kFirst = kPer < 8 ? kPer : 8;
    const int units = M * 4 * C;
    const int units_per_row = 4 * C;
    static_assert(!NORM || kPer == kFirst, "the RMSNorm prologue holds the whole row in registers");
    // the rotary epilogue's position and frequency, requested first
    int64_t rope_pos = 0;
    float rope_freq = 0.0f;
    if constexpr (ROPE) {
        rope_pos = fz.position[0];
        rope_freq = fz.inv_freq[task & 31];
    }
    u32x4 a[kFirst];
    u32x4 nw[NORM ? kFirst : 1];
#pragma unroll
    for (int p = 0; p < kFirst; ++p) {
        const int i = min((int)threadIdx.x + p * T, units - 1);
        a[p] = *reinterpret_cast<const u32x4*>(x + (size_t)i * 8);
    }
    if (NORM) {
#pragma unroll
        for (int p = 0; p < kFirst; ++p) {
            const int i = min((int)threadIdx.x + p * T, units - 1);
            nw[p] = *reinterpret_cast<const u32x4*>(fz.norm_weight + (size_t)i * 8);
        }
    }

    // 2. scales and weights of this wavefront's rows (rows past N re-read
    // N-1 and are not stored; chunks past C re-read chunk C-1 and are not used)
    uint32_t sv[R][L];   // fp16 bits, one per register (no packing, no early wait)
    u32x4 wv[R][L];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int n = min(row0 + r * row_step, N - 1);
        const uint16_t* srow = reinterpret_cast<const uint16_t*>(scales) + (size_t)n * G;
#pragma unroll
        for (int j = 0; j < L; ++j) {
            const int c = min(j * 64 + lane, C - 1);
            sv[r][j] = srow[c >> 2];
        }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int n = min(row0 + r * row_step, N - 1);
        const uint8_t* wrow = w + (size_t)n * row_bytes;   // wavefront-uniform
#pragma unroll
        for (int j = 0; j < L; ++j) {
            const uint32_t c = (uint32_t)min(j * 64 + lane, C - 1);
            wv[r][j] = load_stream(reinterpret_cast<const u32x4*>(wrow + c * 16u));
        }
    }
    // the rows' residual values (RESID), requested with the weights so the
    // epilogue does not wait a round trip for them (residual[n] is read and
    // rewritten by this lane only)
    f16 resv[R];
    if constexpr (RESID) {
#pragma unroll
        for (int r = 0; r < R; ++r) resv[r] = fz.residual[min(row0 + r, N - 1)];
    }
    // keep every request above ahead of the first wait below
    __builtin_amdgcn_sched_barrier(0);

    // 3. activations into LDS (RMS-normalised first when asked), with the
    // per-chunk offset bias
    if (NORM) {
        float* partial = cbias + M * C;   // W floats after the biases
        float ss = 0.0f;
#pragma unroll
        for (int p = 0; p < kFirst; ++p) {
            const int i = threadIdx.x + p * T;
            if (i < units) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const f16x2 h = as_f16x2(a[p][e]);
                    ss = __builtin_fmaf((float)h.x, (float)h.x, ss);
                    ss = __builtin_fmaf((float)h.y, (float)h.y, ss);
                }
            }
        }
        ss = wave_sum(ss);
        if (lane == 0) partial[wave] = ss;
        __syncthreads();
        float total = 0.0f;
#pragma unroll
        for (int v = 0; v < W; ++v) total += partial[v];
        const float inv = 1.0f / __builtin_sqrtf(total / (float)K + fz.eps);
#pragma unroll
        for (int p = 0; p < kFirst; ++p) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const f16x2 h = as_f16x2(a[p][e]);
                const f16x2 g = as_f16x2(nw[NORM ? p : 0][e]);
                const f16x2 y = {(f16)(((float)h.x * inv) * (float)g.x), (f16)(((float)h.y * inv) * (float)g.y)};
                a[p][e] = as_u32(y);
            }
        }
    }
    // unit i = (m, chunk c, quarter q) with q = i % 4: the four lanes of a
    // DPP quad hold one chunk (T and 4C are multiples of 4), so the quad sum
    // is that chunk's bias and every quad is wholly inside or past `units`
#pragma unroll
    for (int p = 0; p < kFirst; ++p) {
        const int i = threadIdx.x + p * T;
        float bias;
        const u32x4 v = stage_offset(a[p], bias);
        if (i < units) {
            const int m = M == 1 ? 0 : i / units_per_row;
            const int u = i - m * units_per_row;
            xs[(m * 4 + (u & 3)) * C + (u >> 2)] = v;
            if ((u & 3) == 0) cbias[m * C + (u >> 2)] = bias;
        }
    }
    if (kPer > kFirst) {
        for (int i = threadIdx.x + kFirst * T; i < units; i += T) {
            const int m = M == 1 ? 0 : i / units_per_row;
            const int u = i - m * units_per_row;
            float bias;
            const u32x4 v = stage_offset(*reinterpret_cast<const u32x4*>(x + (size_t)i * 8), bias);
            xs[(m * 4 + (u & 3)) * C + (u >> 2)] = v;
            if ((u & 3) == 0) cbias[m * C + (u >> 2)] = bias;
        }
    }
    __syncthreads();
    if (!valid && !ARGMAX) return;   // the argmax tail needs every wavefront at its barriers
    // the rotation's cos / sin, while the weights are still arriving
    float rope_cos = 1.0f, rope_sin = 0.0f;
    if constexpr (ROPE) {
        if (rot) sincosf((float)rope_pos * rope_freq, &rope_sin, &rope_cos);
    }

    // 4. dot products, row by row in arrival order. Straight-line code (no
    // branch per chunk, so each chunk waits only for its own load): lanes
    // past C compute on the clamped chunk and select 0.
    float rowsum[R][M];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        float acc[M];
#pragma unroll
        for (int m = 0; m < M; ++m) acc[m] = 0.0f;
#pragma unroll
        for (int j = 0; j < L; ++j) {
            const int c = j * 64 + lane;
            const int cc = min(c, C - 1);
            float d[M];
#pragma unroll
            for (int m = 0; m < M; ++m) d[m] = cbias[m * C + cc];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const Codes8 cw = unpack8_offset(wv[r][j][q]);
#pragma unroll
                for (int m = 0; m < M; ++m) {
                    const u32x4 xv = xs[(m * 4 + q) * C + cc];
                    d[m] = __builtin_amdgcn_fdot2(as_f16x2(xv.x), cw.p[0], d[m], false);
                    d[m] = __builtin_amdgcn_fdot2(as_f16x2(xv.y), cw.p[1], d[m], false);
                    d[m] = __builtin_amdgcn_fdot2(as_f16x2(xv.z), cw.p[2], d[m], false);
                    d[m] = __builtin_amdgcn_fdot2(as_f16x2(xv.w), cw.p[3], d[m], false);
                }
            }
            const float s = (float)__builtin_bit_cast(f16, (uint16_t)sv[r][j]);
#pragma unroll
            for (int m = 0; m < M; ++m) acc[m] = __builtin_fmaf(c < C ? d[m] : 0.0f, s, acc[m]);
        }
#pragma unroll
        for (int m = 0; m < M; ++m) {
            rowsum[r][m] = wave_sum(acc[m]);
            if (!PAIRED && !ROPE && lane == 0 && row0 + r < N && (!ARGMAX || out != nullptr)) {
                const int n = row0 + r;
                f16 v = (f16)rowsum[r][m];
                if constexpr (RESID) v = (f16)((float)resv[r] + (float)v);
                out[(size_t)m * N + n] = v;
            }
        }
    }
    if constexpr (ROPE) {
        if (lane == 0) {
            const f16 a0 = (f16)rowsum[0][0], a1 = (f16)rowsum[1][0];
            f16 y0 = a0, y1 = a1;
            if (rot) {
                y0 = (f16)((float)a0 * rope_cos - (float)a1 * rope_sin);
                y1 = (f16)((float)a1 * rope_cos + (float)a0 * rope_sin);
            }
            const int n1 = row0 + row_step;
            out[row0] = y0;
            out[n1] = y1;
            if (rope_pos >= 0 && rope_pos < fz.max_seq) {
                const size_t p = (size_t)rope_pos;
                if (!rot) {   // v rows 2i, 2i+1 of the v block
                    const int vi = row0 - 2 * fz.rope_pairs;
                    f16* vc = fz.v_cache + ((size_t)(vi >> 6) * fz.max_seq + p) * 64 + (vi & 63);
                    vc[0] = y0;
                    vc[1] = y1;
                } else if ((row0 >> 6) >= fz.rope_heads) {   // a k head
                    f16* kc = fz.k_cache + ((size_t)((row0 >> 6) - fz.rope_heads) * fz.max_seq + p) * 64 + (row0 & 63);
                    kc[0] = y0;
                    kc[32] = y1;
                }
            }
        }
    }
    if (PAIRED && lane == 0) {
        const float g = (float)(f16)rowsum[0][0];
        const float u = (float)(f16)rowsum[R - 1][0];
        const float act = (float)(f16)(g / (1.0f + expf(-g)));
        out[task] = (f16)(act * u);
    }
    if constexpr (ARGMAX) {
        float rs[R];
#pragma unroll
        for (int r = 0; r < R; ++r) rs[r] = rowsum[r][0];
        argmax_tail<R, W>(rs, row0, N, fz, wave, lane);
    }
}

// ---------------------------------------------------------------------------
// M = 1 GEMV on the matrix cores ("diagonal MFMA"), G = 128.
//
// A wavefront reads a row in 1 KiB spans (64 lanes x 16 bytes = 64 chunks =
// 16 groups) like the VALU kernel, but lane l = 16q + j takes chunk 4j + q of
// the span, so the four lanes j, 16+j, 32+j, 48+j hold the four chunks of
// group j. With B = the lane's decoded codes (column j = l%16, k-block q)
// and A = the matching activations (row i = l%16, same k-block), the four
// v_mfma_f32_16x16x32_f16 of one span (one per 32-bit word of the chunk)
// leave D[j][j] = the dot product of group j: the diagonal holds the span's
// 16 group dots (off-diagonal entries are unused). D[i][j] sits in lane
// 16(i/4) + j, register i%4, so the diagonal is lane l's register l%4 when
// (l%16)/4 == l/16.
//
// Decode without fix-ups: every nibble is placed one position up in the
// mantissa of binary16 1024 (unpack8_x16), giving 1024 + 16 v exactly with
// v = s + 8. Then sum x (1024 + 16 v) = 16 sum x s + 1152 sum x, and the
// second term is removed by starting each row's MFMA chain from
// -1152 sum x, computed once per span by four MFMAs against the constant
// B = -1152 (exact in binary16) and shared by the R rows. D = 16 * dot then
// takes the lane's group scale and a final exact 1/16. Products are exact
// in fp32 and the sums accumulate in fp32; the offset costs at most the
// rounding of an fp32 sum of magnitude ~1152 |sum x| per group.
//
// Activations are staged once per workgroup in LDS with chunk c of span s at
// slot s*64 + 16(c%4) + (c%64)/4 (unit-major, zero padded to whole spans),
// so lane l reads slot s*64 + l: conflict-free and already in A layout.
// Task/step/double-buffer structure as in the VALU kernel.
// ---------------------------------------------------------------------------
template <int R, int U>
struct DiagStep {
    u32x4 w[U][R];
    f16 s[U][R];
};

__device__ __forceinline__ int diag_chunk(int lane) { return 4 * (lane & 15) + (lane >> 4); }

// All eight nibbles of a word as 1024 + 16 v (v = nibble ^ 8), pair order
// (0,4) (1,5) (2,6) (3,7) as in unpack8: 3 shifts + 4 v_bitop3, no f16 math.
__device__ __forceinline__ u32x4 unpack8_x16(uint32_t word) {
    u32x4 o;
    o.x = __builtin_amdgcn_bitop3_b32(word << 4, 0x00F000F0u, 0x64806480u, 0x6A);
    o.y = __builtin_amdgcn_bitop3_b32(word, 0x00F000F0u, 0x64806480u, 0x6A);
    o.z = __builtin_amdgcn_bitop3_b32(word >> 4, 0x00F000F0u, 0x64806480u, 0x6A);
    o.w = __builtin_amdgcn_bitop3_b32(word >> 8, 0x00F000F0u, 0x64806480u, 0x6A);
    return o;
}

template <int R, int U>
__device__ __forceinline__ void diag_load(DiagStep<R, U>& b, const uint8_t* __restrict__ w,
                                          const f16* __restrict__ scales, int task, int step, int lane,
                                          int N, int C, int G, uint32_t row_bytes) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int n = min(task * R + r, N - 1);
        const uint8_t* wrow = w + (size_t)n * row_bytes;
        const uint8_t* srow = reinterpret_cast<const uint8_t*>(scales + (size_t)n * G);
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int span = step * U + u;
            const int c = span * 64 + diag_chunk(lane);
            if (c < C) {
                const uint32_t c32 = (uint32_t)c;
                b.w[u][r] = load_stream(reinterpret_cast<const u32x4*>(wrow + c32 * 16u));
                b.s[u][r] = *reinterpret_cast<const f16*>(srow + (c32 >> 2) * 2u);
            } else {
                b.w[u][r] = (u32x4){0x88888888u, 0x88888888u, 0x88888888u, 0x88888888u};   // all codes 0
                b.s[u][r] = (f16)0.0f;
            }
        }
    }
}

template <int R, int U>
__device__ __forceinline__ void diag_compute(const DiagStep<R, U>& b, const u32x4* xs, f32x4 (&acc)[R],
                                             int step, int lane, int spans) {
    const f16x8 neg_offset = {(f16)-1152.0f, (f16)-1152.0f, (f16)-1152.0f, (f16)-1152.0f,
                              (f16)-1152.0f, (f16)-1152.0f, (f16)-1152.0f, (f16)-1152.0f};
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int span = step * U + u;
        if (span < spans) {
            f16x8 a[4];
#pragma unroll
            for (int t = 0; t < 4; ++t) a[t] = __builtin_bit_cast(f16x8, xs[(t * spans + span) * 64 + lane]);
            // -1152 * (sum of each group's activations) on the diagonal
            f32x4 base = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int t = 0; t < 4; ++t) base = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[t], neg_offset, base, 0, 0, 0);
#pragma unroll
            for (int r = 0; r < R; ++r) {
                f16x8 bt[4];
#pragma unroll
                for (int t = 0; t < 4; ++t) bt[t] = __builtin_bit_cast(f16x8, unpack8_x16(b.w[u][r][t]));
                f32x4 d = base;
#pragma unroll
                for (int t = 0; t < 4; ++t) d = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[t], bt[t], d, 0, 0, 0);
                const float s = (float)b.s[u][r];
                acc[r] = d * s + acc[r];
            }
        }
    }
}

template <int R>
__device__ __forceinline__ void diag_finish(f32x4 (&acc)[R], f16* __restrict__ out, int task, int lane, int N) {
    const bool on_diag = ((lane & 15) >> 2) == (lane >> 4);
    const int e = lane & 3;
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const float d = e == 0 ? acc[r][0] : e == 1 ? acc[r][1] : e == 2 ? acc[r][2] : acc[r][3];
        const float v = wave_sum(on_diag ? d : 0.0f) * 0.0625f;   // D carried 16 x the dot
        acc[r] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
        if (lane == 0 && task * R + r < N) out[task * R + r] = (f16)v;
    }
}

// Activations into LDS in the diagonal-MFMA A layout (see above); padding
// beyond K is zero, so padded chunks contribute nothing.
__device__ __forceinline__ void stage_activations_diag(const f16* __restrict__ x, u32x4* xs, int K, int spans) {
    constexpr int kBatch = 8;
    const int units = K >> 3;            // real 16-byte units
    const int total = spans * 64 * 4;    // padded
    const int T = blockDim.x;
    for (int base = threadIdx.x; base < total; base += kBatch * T) {
        u32x4 a[kBatch];
#pragma unroll
        for (int j = 0; j < kBatch; ++j) {
            const int i = base + j * T;
            a[j] = (u32x4){0u, 0u, 0u, 0u};
            if (i < units) a[j] = *reinterpret_cast<const u32x4*>(x + (size_t)i * 8);
        }
#pragma unroll
        for (int j = 0; j < kBatch; ++j) {
            const int i = base + j * T;
            if (i < total) {
                const int c = i >> 2, t = i & 3;
                const int span = c >> 6, cl = c & 63;
                xs[(t * spans + span) * 64 + 16 * (cl & 3) + (cl >> 2)] = permute8(a[j]);
            }
        }
    }
}

template <int R, int U>
__global__ void __launch_bounds__(256)
gemv_diag(const f16* __restrict__ x, const uint8_t* __restrict__ w,
          const f16* __restrict__ scales, f16* __restrict__ out, int N, int K, int num_tasks) {
    extern __shared__ __align__(16) uint8_t smem[];
    u32x4* xs = reinterpret_cast<u32x4*>(smem);

    const int W = blockDim.x >> 6;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int C = K >> 5;
    const int G = K >> 7;
    const int spans = (C + 63) >> 6;
    const int steps = (spans + U - 1) / U;
    const uint32_t row_bytes = (uint32_t)(K >> 1);

    const int task0 = blockIdx.x * W + wave;
    const int task_stride = gridDim.x * W;
    const int my_tasks = task0 < num_tasks ? (num_tasks - 1 - task0) / task_stride + 1 : 0;
    const int units = my_tasks * steps;

    DiagStep<R, U> buf0, buf1;
    int task = task0, step = 0;
    if (units > 0) diag_load(buf0, w, scales, task, step, lane, N, C, G, row_bytes);
    stage_activations_diag(x, xs, K, spans);
    __syncthreads();

    f32x4 acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};

    for (int u = 0; u < units; u += 2) {
        int task1 = task, step1 = step + 1;
        if (step1 == steps) { step1 = 0; task1 += task_stride; }
        if (u + 1 < units) diag_load(buf1, w, scales, task1, step1, lane, N, C, G, row_bytes);
        diag_compute(buf0, xs, acc, step, lane, spans);
        if (step == steps - 1) diag_finish(acc, out, task, lane, N);
        if (u + 1 >= units) break;
        task = task1;
        step = step1 + 1;
        if (step == steps) { step = 0; task += task_stride; }
        if (u + 2 < units) diag_load(buf0, w, scales, task, step, lane, N, C, G, row_bytes);
        diag_compute(buf1, xs, acc, step1, lane, spans);
        if (step1 == steps - 1) diag_finish(acc, out, task1, lane, N);
    }
}

// ---------------------------------------------------------------------------
// MFMA kernel (runtime M = 1..8, zero-padded to 16), G = 128.
//
// v_mfma_f32_16x16x32_f16: A is 16x32 (rows i = activation rows), B is 32x16
// (columns j = output rows n), D is 16x16 fp32. Lane l supplies
// A[l%16][8(l/16) + 0..7] and B[8(l/16) + 0..7][l%16] and receives
// D[4(l/16) + 0..3][l%16].
// Lane l of a wavefront owns output row n = n_block + l%16 and loads the
// 16-byte chunk l/16 of that row's current 128-weight group: one load per
// lane covers a whole group for 16 rows. Word t (0..3) of every lane feeds
// MFMA t, so the group takes four MFMAs; A for MFMA t is activation row
// l%16 at the same 8 k positions, permuted to the unpack8 pair order (k order
// inside one MFMA does not matter as long as A and B agree). The group's
// 16x16 product is scaled by the per-lane (= per-column n) fp32 scale and
// accumulated in fp32.
// Wavefront = RB blocks of 16 rows sharing the A fragments; workgroup = S
// wavefronts splitting the groups of K (wave w takes groups w, w+S, ..., U
// of them in flight per step, so the S wavefronts of a workgroup read
// adjacent 64-byte pieces of each row at the same time), reduced through LDS
// at the end. Activation rows m >= M and rows past N
// follow the same path with zero A / clamped rows and are not stored.
// ---------------------------------------------------------------------------
template <int RB, int U>
__global__ void __launch_bounds__(512)
gemv_mfma(const f16* __restrict__ x, const uint8_t* __restrict__ w,
          const f16* __restrict__ scales, f16* __restrict__ out, int M, int N, int K) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int S = blockDim.x >> 6;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int col = lane & 15;      // n within a 16-row block; also activation row for A
    const int kq = lane >> 4;       // which 32-weight quarter of a group
    const int G = K >> 7;
    const int n_base = blockIdx.x * (16 * RB);

    const uint8_t* wrow[RB];
    const f16* srow[RB];
#pragma unroll
    for (int b = 0; b < RB; ++b) {
        const int n = min(n_base + b * 16 + col, N - 1);
        wrow[b] = w + (size_t)n * (size_t)(K >> 1) + kq * 16;
        srow[b] = scales + (size_t)n * G;
    }
    const bool has_act = col < M;
    const f16* xrow = x + (size_t)(has_act ? col : 0) * K + kq * 32;

    f32x4 acc[RB];
#pragma unroll
    for (int b = 0; b < RB; ++b) acc[b] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};

    for (int g0 = wave; g0 < G; g0 += U * S) {
        u32x4 wv[U][RB];
        f16 sv[U][RB];
        u32x4 xa[U][4];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int g = g0 + u * S;
            if (g < G) {
#pragma unroll
                for (int b = 0; b < RB; ++b) {
                    wv[u][b] = load_stream(reinterpret_cast<const u32x4*>(wrow[b] + (size_t)g * 64));
                    sv[u][b] = srow[b][g];
                }
                const u32x4* xp = reinterpret_cast<const u32x4*>(xrow + (size_t)g * 128);
#pragma unroll
                for (int t = 0; t < 4; ++t)
                    xa[u][t] = has_act ? xp[t] : (u32x4){0u, 0u, 0u, 0u};
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int g = g0 + u * S;
            if (g < G) {
                f16x8 a[4];
#pragma unroll
                for (int t = 0; t < 4; ++t) a[t] = __builtin_bit_cast(f16x8, permute8(xa[u][t]));
#pragma unroll
                for (int b = 0; b < RB; ++b) {
                    f32x4 d = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                    for (int t = 0; t < 4; ++t) {
                        const Codes8 cw = unpack8(wv[u][b][t]);
                        const f16x8 bt = __builtin_bit_cast(
                            f16x8, (u32x4){as_u32(cw.p[0]), as_u32(cw.p[1]), as_u32(cw.p[2]), as_u32(cw.p[3])});
                        d = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[t], bt, d, 0, 0, 0);
                    }
                    const float s = (float)sv[u][b];
                    acc[b] = d * s + acc[b];
                }
            }
        }
    }

    // Cross-wavefront reduction of the RB 16x16 tiles.
    f32x4* red = reinterpret_cast<f32x4*>(smem);
    if (S > 1) {
#pragma unroll
        for (int b = 0; b < RB; ++b) red[(wave * RB + b) * 64 + lane] = acc[b];
        __syncthreads();
        if (wave != 0) return;
#pragma unroll
        for (int b = 0; b < RB; ++b) {
            f32x4 v = red[b * 64 + lane];
            for (int s = 1; s < S; ++s) v += red[(s * RB + b) * 64 + lane];
            acc[b] = v;
        }
    }
    // D[i][j]: i = 4 kq + e (activation row), j = col (output row in block).
#pragma unroll
    for (int b = 0; b < RB; ++b) {
        const int n = n_base + b * 16 + col;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int m = kq * 4 + e;
            if (m < M && n < N) out[(size_t)m * N + n] = (f16)acc[b][e];
        }
    }
}

// ---------------------------------------------------------------------------
// One-shot MFMA kernel for small batches (runtime M = 1..16, one MFMA tile
// of activation rows), G = 128.
//
// Workgroup = SK x SN wavefronts: SN blocks of 16 output rows, each block's
// groups split over SK wavefronts (wavefront kw takes groups kw, kw + SK, ...,
// GPW of them, so at any step the SK wavefronts read adjacent 64-byte pieces
// of each row). MFMA layout as in gemv_mfma: lane l = 16 q + c supplies row
// n0 + c's chunk q of a group as B (word t -> MFMA t) and activation row c's
// matching 8 k values as A; D[4 q + e][c] lands in lane l, register e.
//
// Differences from gemv_mfma, each measured on the small-batch benchmark shapes:
//   * every weight and scale load of a wavefront is issued up front
//     (straight-line, clamped addresses), after the workgroup's activation
//     units, which return first;
//   * the activations are staged once per workgroup in LDS in A order
//     (unit (g, t, q) of row m at xs[((g*4 + t)*4 + q)*M + m]), and each
//     group's four A fragments are read one group ahead of its MFMAs;
//   * offset decode: B holds the codes without f16 fix-ups (1024 + v for
//     pos-0 nibbles, 1024 + 16 v for pos-1 nibbles, v = s + 8) and A the
//     activations with pos-1 halves pre-scaled by 1/16 (exact unless
//     subnormal), so the dot carries 1032 * sum(x pos-0) + 72 * sum(x pos-1)
//     on top of sum x*s. That bias depends only on the activations: it is
//     computed while staging (base[g][m], fp32) and each group's MFMA chain
//     starts from -base instead of 0. Products are exact; the sums are fp32
//     with a larger magnitude than sum x*s alone (the precision of the
//     offset decode, within the 1e-2 (1 + |ref|) bar with ~10x margin);
//   * the D rows of activation rows >= M read duplicated rows and are never
//     stored, so no lane selects zeros.
// Partial sums of the SK wavefronts are reduced through LDS.
// ---------------------------------------------------------------------------
template <int SK, int SN, int GPW>
__global__ void __launch_bounds__(64 * SK * SN)
gemv_mfma_oneshot(const f16* __restrict__ x, const uint8_t* __restrict__ w, const f16* __restrict__ scales,
                  f16* __restrict__ out, int M, int N, int K) {
    constexpr int S = SK * SN;
    constexpr int T = 64 * S;
    constexpr int kFirst = 8;
    extern __shared__ __align__(16) uint8_t smem[];
    const int G = K >> 7;
    u32x4* xs = reinterpret_cast<u32x4*>(smem);                               // M*K*2 bytes
    float* base = reinterpret_cast<float*>(smem + (size_t)M * K * 2);          // [G][16] fp32
    f32x4* red = reinterpret_cast<f32x4*>(smem + (size_t)M * K * 2 + (size_t)G * 64);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int col = lane & 15, q = lane >> 4;
    const int kw = wave % SK, nb = wave / SK;
    const int n0 = (blockIdx.x * SN + nb) * 16;
    const int n = min(n0 + col, N - 1);
    const uint32_t row_bytes = (uint32_t)(K >> 1);

    // 1. activation units (8 halves): i = m * K/8 + uk
    const int upr = K >> 3;
    const int units = M * upr;
    u32x4 a[kFirst];
#pragma unroll
    for (int p = 0; p < kFirst; ++p) {
        const int i = min((int)threadIdx.x + p * T, units - 1);
        a[p] = *reinterpret_cast<const u32x4*>(x + (size_t)i * 8);
    }
    // 2. scales and weights: groups kw + SK j (clamped; j past G is dropped)
    const uint16_t* srow = reinterpret_cast<const uint16_t*>(scales) + (size_t)n * G;
    const uint8_t* wrow = w + (size_t)n * row_bytes + q * 16;
    uint32_t sv[GPW];
    u32x4 wv[GPW];
#pragma unroll
    for (int j = 0; j < GPW; ++j) sv[j] = srow[min(kw + SK * j, G - 1)];
#pragma unroll
    for (int j = 0; j < GPW; ++j)
        wv[j] = load_stream(reinterpret_cast<const u32x4*>(wrow + (uint32_t)min(kw + SK * j, G - 1) * 64u));
    __builtin_amdgcn_sched_barrier(0);

    // 3. stage A fragments and the per-(group, row) bias
    const f16x2 sixteenth = {(f16)0.0625f, (f16)0.0625f};
    const f16x2 b0 = {(f16)1032.0f, (f16)1032.0f};
    const f16x2 b1 = {(f16)1152.0f, (f16)1152.0f};
    auto put = [&](int i, u32x4 v, bool valid) {
        const int m = i / upr;
        const int uk = i - m * upr;
        const int g = uk >> 4, qq = (uk >> 2) & 3, t = uk & 3;
        u32x4 pv = permute8(v);
        pv.y = as_u32(as_f16x2(pv.y) * sixteenth);
        pv.w = as_u32(as_f16x2(pv.w) * sixteenth);
        float c = 0.0f;
        c = __builtin_amdgcn_fdot2(as_f16x2(pv.x), b0, c, false);
        c = __builtin_amdgcn_fdot2(as_f16x2(pv.y), b1, c, false);
        c = __builtin_amdgcn_fdot2(as_f16x2(pv.z), b0, c, false);
        c = __builtin_amdgcn_fdot2(as_f16x2(pv.w), b1, c, false);
        // the 16 units of (m, g) sit in 16 consecutive lanes (a DPP row):
        // after the mirrors every lane of the row holds the row sum
        c += dpp<0xB1>(c);
        c += dpp<0x4E>(c);
        c += dpp<0x141>(c);
        c += dpp<0x140>(c);
        if (valid) {
            xs[((g * 4 + t) * 4 + qq) * M + m] = pv;
            if ((uk & 15) == 0) base[g * 16 + m] = -c;
        }
    };
#pragma unroll
    for (int p = 0; p < kFirst; ++p) {
        const int i = threadIdx.x + p * T;
        put(min(i, units - 1), a[p], i < units);
    }
    // rest of a large M*K (requested after the weights): whole rows of lanes
    for (int i0 = threadIdx.x + kFirst * T; i0 < ((units + T - 1) / T) * T; i0 += T) {
        const int i = min(i0, units - 1);
        put(i, *reinterpret_cast<const u32x4*>(x + (size_t)i * 8), i0 < units);
    }
    __syncthreads();

    // 4. groups: fragments of group j+1 read while group j runs on the MFMAs
    const int arow = col % M;
    auto fetch = [&](u32x4 (&av)[4], f32x4& bv, int j) {
        const int g = min(kw + SK * j, G - 1);
#pragma unroll
        for (int t = 0; t < 4; ++t) av[t] = xs[((g * 4 + t) * 4 + q) * M + arow];
        bv = *reinterpret_cast<const f32x4*>(base + g * 16 + 4 * q);
    };
    f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    u32x4 A0[4], A1[4];
    f32x4 B0, B1;
    fetch(A0, B0, 0);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < GPW; ++j) {
        u32x4 (&cur)[4] = (j & 1) ? A1 : A0;
        u32x4 (&nxt)[4] = (j & 1) ? A0 : A1;
        f32x4& cb = (j & 1) ? B1 : B0;
        f32x4& nbv = (j & 1) ? B0 : B1;
        if (j + 1 < GPW) fetch(nxt, nbv, j + 1);
        __builtin_amdgcn_sched_barrier(0);
        f32x4 d = cb;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const Codes8 cw = unpack8_offset(wv[j][t]);
            const f16x8 bt = __builtin_bit_cast(
                f16x8, (u32x4){as_u32(cw.p[0]), as_u32(cw.p[1]), as_u32(cw.p[2]), as_u32(cw.p[3])});
            d = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, cur[t]), bt, d, 0, 0, 0);
        }
        const float sc = (kw + SK * j) < G ? (float)__builtin_bit_cast(f16, (uint16_t)sv[j]) : 0.0f;
        acc = d * sc + acc;
    }

    // 5. reduce the SK partial tiles of this row block, store rows m < M
    if (SK > 1) {
        red[wave * 64 + lane] = acc;
        __syncthreads();
        if (kw != 0) return;
#pragma unroll
        for (int s2 = 1; s2 < SK; ++s2) acc += red[(wave + s2) * 64 + lane];
    }
    const int nn = n0 + col;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int m = q * 4 + e;
        if (m < M && nn < N) out[(size_t)m * N + nn] = (f16)acc[e];
    }
}

// ---------------------------------------------------------------------------
// Generic kernel: any M, any even G with K % G == 0, any pointer alignment
// (fp16 data needs only its natural 2-byte alignment). One wavefront per
// output row; lanes stride over the packed bytes; activation rows in tiles of
// 8. Each weight is dequantized exactly in fp32 (code * scale, as reference
// w4a16/reference.py:38-46 does) before the fp32 multiply-add.
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(256)
linear_generic(const f16* __restrict__ x, const uint8_t* __restrict__ w,
               const f16* __restrict__ scales, f16* __restrict__ out,
               int M, int N, int K, int G) {
    const int lane = threadIdx.x & 63;
    const int n = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (n >= N) return;  // wavefront-uniform; this kernel has no barriers
    const int KB = K >> 1;
    const int groups = K / G;
    const uint8_t* wrow = w + (size_t)n * KB;
    const f16* srow = scales + (size_t)n * groups;
    for (int m0 = 0; m0 < M; m0 += 8) {
        float acc[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[i] = 0.0f;
        for (int j = lane; j < KB; j += 64) {
            const uint32_t byte = wrow[j];
            const int lo = (int)((byte & 0xFu) ^ 8u) - 8;
            const int hi = (int)((byte >> 4) ^ 8u) - 8;
            const float s = (float)srow[(2 * j) / G];
            const float wl = (float)lo * s;
            const float wh = (float)hi * s;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                if (m0 + i < M) {
                    const f16* xr = x + (size_t)(m0 + i) * K + 2 * j;
                    acc[i] = __builtin_fmaf((float)xr[0], wl, acc[i]);
                    acc[i] = __builtin_fmaf((float)xr[1], wh, acc[i]);
                }
            }
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float v = wave_sum(acc[i]);
            if (lane == 0 && m0 + i < M) out[(size_t)(m0 + i) * N + n] = (f16)v;
        }
    }
}

// ---------------------------------------------------------------------------
// Dequantize: out[n][k] = fp16_rn(code * scale). The packed codes are read
// as 32-bit words (8 weights each, inside one group since G % 32 == 0): a
// wavefront takes 256 consecutive words, lane l words q 64 + l (q < 4), so
// every load instruction reads 256 contiguous bytes and every store writes
// 1 KiB. Codes are exact in f16, and an IEEE binary16 multiply of exact
// operands rounds the exact product once (round to nearest even, subnormals
// kept), which is the value of reference w4a16/reference.py:38-46 followed by
// .to(torch.float16).
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(256)
dequantize_kernel(const uint8_t* __restrict__ w, const f16* __restrict__ scales,
                  f16* __restrict__ out, int64_t words, int words_per_row,
                  int words_per_group, int groups_per_row) {
    const int lane = threadIdx.x & 63;
    const int64_t base = ((int64_t)blockIdx.x * 256 + (threadIdx.x & ~63)) * 4;   // the wavefront's first word
    const uint32_t* wp = reinterpret_cast<const uint32_t*>(w);
    uint32_t d[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int64_t j = base + 64 * q + lane;
        d[q] = j < words ? __builtin_nontemporal_load(wp + j) : 0u;
    }
    // row and word-in-row of word base + lane, then steps of 64 words
    int64_t n = (base + lane) / words_per_row;
    int c = (int)(base + lane - n * words_per_row);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int64_t j = base + 64 * q + lane;
        if (j < words) {
            const f16 s = scales[n * groups_per_row + c / words_per_group];
            const f16x2 ss = {s, s};
            const uint32_t u = d[q] ^ 0x88888888u;
            u32x4 v;
            v.x = as_u32(unpack_byte_pair<0>(u) * ss);
            v.y = as_u32(unpack_byte_pair<1>(u) * ss);
            v.z = as_u32(unpack_byte_pair<2>(u) * ss);
            v.w = as_u32(unpack_byte_pair<3>(u) * ss);
            reinterpret_cast<u32x4*>(out)[j] = v;
        }
        c += 64;
        while (c >= words_per_row) {   // 64 words may cross several short rows
            c -= words_per_row;
            ++n;
        }
    }
}

}  // namespace w4a16

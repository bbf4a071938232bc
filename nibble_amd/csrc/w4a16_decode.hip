// Decode-step kernels around the W4A16 GEMV (include/w4a16_decode.h): the
// per-layer attention of one new token (rotary embedding, KV-cache append,
// softmax(q k^T / sqrt(d)) v over the filled slots), greedy argmax with the
// position advance, and the embedding gather. Together with the fused GEMV
// entry point (w4a16_gemv_fused_f16, in w4a16_hip.hip) they run one Llama
// decode step as 5 launches per layer. Nothing here allocates or
// synchronises; positions and tokens live in device memory, so a whole step
// can be captured once in a HIP graph and replayed.
#include "w4a16_decode.h"
#include "w4a16_hip.h"

#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>

#include "w4a16_device.h"

namespace w4a16 {

// ---------------------------------------------------------------------------
// Attention of one new token, one wavefront per query head (head_dim 64).
//
// Inputs: qkv = [q (H x 64) | k (KV x 64) | v (KV x 64)] fp16 from the fused
// QKV projection; caches [KV, S, 64] fp16; cos / sin [S, 32] fp32 tables;
// position p (device int64).
//   1. rotary embedding, half-split convention (x1 = x[:32], x2 = x[32:]):
//      out[d] = x1*c - x2*s for d < 32, x2*c + x1*s for d >= 32, computed in
//      fp32 and rounded to fp16 (the q and k the cache holds); the first
//      query head of each KV group writes k and v to slot p, and every head
//      uses its own copy of slot p (never the cache line another workgroup
//      is writing);
//   2. slots 0..p in chunks of 64: lane t holds slot c0 + t's key row (8
//      16-byte loads, all requested before any is used) and its score
//      q.k / 8 in fp32; the chunk's value rows go to LDS (coalesced 16-byte
//      loads); an online softmax (running max, rescaled sum and output)
//      folds the chunk in, and lane d accumulates sum_t prob_t v_t[d];
//   3. out[d] = acc / sum, rounded to fp16.
// Slots past p are masked (weight exactly 0, as exp(-inf) is). A position
// outside [0, S) writes NaN to the head's output and touches no cache slot.
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(64)
decode_attention(const f16* __restrict__ qkv, f16* __restrict__ k_cache, f16* __restrict__ v_cache,
                 const float* __restrict__ cos_table, const float* __restrict__ sin_table,
                 const int64_t* __restrict__ position, f16* __restrict__ out, int num_heads, int num_kv, int S) {
    constexpr int D = 64;
    __shared__ float qs[D];
    __shared__ float probs[64];
    __shared__ __align__(16) f16 vt[64 * D];   // value rows of the current chunk

    const int hq = blockIdx.x;
    const int lane = threadIdx.x;
    const int group = num_heads / num_kv;
    const int hk = hq / group;
    const int64_t p64 = position[0];
    if (p64 < 0 || p64 >= S) {
        out[(size_t)hq * D + lane] = (f16)__builtin_nanf("");
        return;
    }
    const int p = (int)p64;
    const f16* kc = k_cache + (size_t)hk * S * D;
    const f16* vc = v_cache + (size_t)hk * S * D;

    // first chunk's cache rows, requested before the rotary work
    auto load_k = [&](u32x4 (&kr)[8], int t) {
        const u32x4* row = reinterpret_cast<const u32x4*>(kc + (size_t)min(t, S - 1) * D);
#pragma unroll
        for (int e = 0; e < 8; ++e) kr[e] = row[e];
    };
    auto load_v = [&](u32x4 (&vr)[8], int c0) {
        // lane l: rows c0 + l/8 + 8 i, 16-byte column block l % 8
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int t = min(c0 + (lane >> 3) + 8 * i, S - 1);
            vr[i] = reinterpret_cast<const u32x4*>(vc + (size_t)t * D)[lane & 7];
        }
    };
    u32x4 kr[8], vr[8];
    load_k(kr, lane);
    load_v(vr, 0);

    const float c = cos_table[(size_t)p * (D / 2) + (lane & 31)];
    const float s = sin_table[(size_t)p * (D / 2) + (lane & 31)];
    const f16* q = qkv + (size_t)hq * D;
    const f16* k = qkv + (size_t)num_heads * D + (size_t)hk * D;
    const f16* v = qkv + (size_t)(num_heads + num_kv) * D + (size_t)hk * D;
    const float qa = (float)q[lane], qb = (float)q[lane ^ 32];
    const float ka = (float)k[lane], kb = (float)k[lane ^ 32];
    const float qr = lane < 32 ? qa * c - qb * s : qa * c + qb * s;
    const float kro = lane < 32 ? ka * c - kb * s : ka * c + kb * s;
    const f16 q16 = (f16)qr, k16 = (f16)kro, v16 = v[lane];
    qs[lane] = (float)q16;
    if (hq % group == 0) {
        k_cache[((size_t)hk * S + p) * D + lane] = k16;
        v_cache[((size_t)hk * S + p) * D + lane] = v16;
    }
    // slot p's key row for the lane that scores it: gathered from the lanes
    __shared__ __align__(16) f16 knew[D];
    knew[lane] = k16;
    __syncthreads();

    float run_max = -__builtin_inff(), run_sum = 0.0f, acc = 0.0f;
    for (int c0 = 0; c0 <= p; c0 += 64) {
        const int t = c0 + lane;
        // this chunk's value rows into LDS (slot p patched with the new v)
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int row = (lane >> 3) + 8 * i;
            reinterpret_cast<u32x4*>(vt + row * D)[lane & 7] = vr[i];
        }
        // score of slot t
        float dot = 0.0f;
        if (t == p) {
#pragma unroll
            for (int e = 0; e < D; ++e) dot = __builtin_fmaf(qs[e], (float)knew[e], dot);
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) {
#pragma unroll
                for (int w2 = 0; w2 < 4; ++w2) {
                    const f16x2 h = as_f16x2(kr[e][w2]);
                    dot = __builtin_fmaf(qs[e * 8 + 2 * w2], (float)h.x, dot);
                    dot = __builtin_fmaf(qs[e * 8 + 2 * w2 + 1], (float)h.y, dot);
                }
            }
        }
        const float score = t <= p ? dot / 8.0f : -__builtin_inff();
        // next chunk's rows requested before this chunk's reductions
        if (c0 + 64 <= p) {
            load_k(kr, t + 64);
            load_v(vr, c0 + 64);
        }
        float cmax = score;
        for (int off = 32; off >= 1; off >>= 1) cmax = fmaxf(cmax, __shfl_xor(cmax, off));
        const float new_max = fmaxf(run_max, cmax);
        const float pr = t <= p ? expf(score - new_max) : 0.0f;
        float psum = pr;
        for (int off = 32; off >= 1; off >>= 1) psum += __shfl_xor(psum, off);
        const float rescale = expf(run_max - new_max);   // 0 on the first chunk
        probs[lane] = pr;
        __syncthreads();
        if (p - c0 < 64) vt[(p - c0) * D + lane] = v16;   // slot p from registers, not the cache
        __syncthreads();
        float part = 0.0f;
        const int rows = min(64, p - c0 + 1);
        for (int r = 0; r < rows; ++r) part = __builtin_fmaf(probs[r], (float)vt[r * D + lane], part);
        acc = acc * rescale + part;
        run_sum = run_sum * rescale + psum;
        run_max = new_max;
        __syncthreads();
    }
    out[(size_t)hq * D + lane] = (f16)(acc / run_sum);
}

// ---------------------------------------------------------------------------
// Greedy argmax over fp16 logits (first index of the maximum, as
// torch.argmax), one workgroup of 1024 threads reading 16-byte vectors when
// the logits are 16-byte aligned; writes the token and, when given, advances
// the position by one and gathers the token's embedding row into `emb_out`
// (the next decode step's input), so the step needs no separate gather.
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(1024)
argmax_kernel(const f16* __restrict__ logits, int n, int64_t* __restrict__ token, int64_t* __restrict__ position,
              const f16* __restrict__ table, int64_t vocab, int hidden, f16* __restrict__ emb_out) {
    __shared__ float best_v[16];
    __shared__ int best_i[16];
    __shared__ int64_t chosen;
    float bv = -__builtin_inff();
    int bi = n;   // sentinel: larger than any index
    const bool vec = (reinterpret_cast<uintptr_t>(logits) & 15u) == 0;
    const int nv = vec ? n >> 3 : 0;
    constexpr int kBatch = 4;   // vectors requested per thread before any is compared
    for (int j0 = threadIdx.x; j0 < nv; j0 += kBatch * blockDim.x) {
        u32x4 u[kBatch];
#pragma unroll
        for (int b = 0; b < kBatch; ++b) {
            const int j = min(j0 + b * (int)blockDim.x, nv - 1);
            u[b] = reinterpret_cast<const u32x4*>(logits)[j];
        }
#pragma unroll
        for (int b = 0; b < kBatch; ++b) {
            const int j = j0 + b * (int)blockDim.x;
            if (j >= nv) break;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const f16x2 h = as_f16x2(u[b][e]);
                const int i = 8 * j + 2 * e;
                const float a = (float)h.x, c = (float)h.y;
                if (a > bv || (a == bv && i < bi)) { bv = a; bi = i; }
                if (c > bv || (c == bv && i + 1 < bi)) { bv = c; bi = i + 1; }
            }
        }
    }
    for (int i = 8 * nv + threadIdx.x; i < n; i += blockDim.x) {
        const float v = (float)logits[i];
        if (v > bv || (v == bv && i < bi)) { bv = v; bi = i; }
    }
    for (int off = 32; off >= 1; off >>= 1) {
        const float ov = __shfl_xor(bv, off);
        const int oi = __shfl_xor(bi, off);
        if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
    }
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) { best_v[wave] = bv; best_i[wave] = bi; }
    __syncthreads();
    if (threadIdx.x == 0) {
        const int waves = blockDim.x >> 6;
        for (int w = 1; w < waves; ++w)
            if (best_v[w] > bv || (best_v[w] == bv && best_i[w] < bi)) { bv = best_v[w]; bi = best_i[w]; }
        const int64_t t = bi < n ? bi : 0;
        token[0] = t;
        chosen = t;
        if (position != nullptr) position[0] += 1;
    }
    if (emb_out == nullptr) return;
    __syncthreads();
    const int64_t t = chosen;
    const f16* row = table + t * hidden;
    for (int i = threadIdx.x; i < hidden; i += blockDim.x) emb_out[i] = t < vocab ? row[i] : (f16)0.0f;
}

// out[i] = table[token, i]; an out-of-range token gives zeros.
__global__ void __launch_bounds__(256)
embedding_kernel(const f16* __restrict__ table, int64_t vocab, int hidden, const int64_t* __restrict__ token,
                 f16* __restrict__ out) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= hidden) return;
    const int64_t t = token[0];
    out[i] = (t >= 0 && t < vocab) ? table[t * hidden + i] : (f16)0.0f;
}

}  // namespace w4a16

namespace w4a16_internal {
void set_last_error(const std::string& message);   // w4a16_hip.hip: the message w4a16_last_error() returns
}

namespace {

int fail(int code, const char* message) {
    w4a16_internal::set_last_error(message);
    return code;
}

int check_launch() {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        w4a16_internal::set_last_error(std::string("kernel launch failed: ") + hipGetErrorString(e));
        return W4A16_ERR_LAUNCH;
    }
    return W4A16_OK;
}

bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

}  // namespace

extern "C" {

int w4a16_decode_attention_f16(const void* qkv, void* k_cache, void* v_cache, const float* cos_table,
                               const float* sin_table, const int64_t* position, void* output, int64_t num_heads,
                               int64_t num_kv_heads, int64_t head_dim, int64_t max_seq_len, void* stream) {
    if (!qkv || !k_cache || !v_cache || !cos_table || !sin_table || !position || !output)
        return fail(W4A16_ERR_NULL, "attention: every pointer must be non-NULL");
    if (head_dim != 64) return fail(W4A16_ERR_CONFIG, "attention: head_dim must be 64");
    if (num_heads <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads != 0 || num_heads > 65535)
        return fail(W4A16_ERR_SHAPE, "attention: num_heads must be a positive multiple of num_kv_heads");
    if (max_seq_len <= 0 || max_seq_len > 16384)
        return fail(W4A16_ERR_SHAPE, "attention: max_seq_len must be in 1..16384");
    if (!aligned(k_cache, 16) || !aligned(v_cache, 16) || !aligned(qkv, 2) || !aligned(output, 2))
        return fail(W4A16_ERR_ALIGNMENT, "attention: caches must be 16-byte aligned, fp16 buffers 2-byte aligned");
    hipLaunchKernelGGL(w4a16::decode_attention, dim3((unsigned)num_heads), dim3(64), 0,
                       static_cast<hipStream_t>(stream), static_cast<const w4a16::f16*>(qkv),
                       static_cast<w4a16::f16*>(k_cache), static_cast<w4a16::f16*>(v_cache), cos_table, sin_table,
                       position, static_cast<w4a16::f16*>(output), (int)num_heads, (int)num_kv_heads,
                       (int)max_seq_len);
    return check_launch();
}

int w4a16_argmax_f16(const void* logits, int64_t n, int64_t* token, int64_t* position, void* stream) {
    return w4a16_argmax_embed_f16(logits, n, token, position, nullptr, 0, 0, nullptr, stream);
}

int w4a16_argmax_embed_f16(const void* logits, int64_t n, int64_t* token, int64_t* position, const void* table,
                           int64_t vocab, int64_t hidden, void* output, void* stream) {
    if (!logits || !token) return fail(W4A16_ERR_NULL, "argmax: logits and token must be non-NULL");
    if (n <= 0 || n > INT32_MAX - 1024) return fail(W4A16_ERR_SHAPE, "argmax: n must be in 1..2^31-1025");
    if ((table == nullptr) != (output == nullptr))
        return fail(W4A16_ERR_NULL, "argmax: table and output must both be given or both be NULL");
    if (table && (vocab < n || hidden <= 0 || hidden > INT32_MAX / 2))
        return fail(W4A16_ERR_SHAPE, "argmax: the embedding table needs vocab >= n and a positive hidden size");
    hipLaunchKernelGGL(w4a16::argmax_kernel, dim3(1), dim3(1024), 0, static_cast<hipStream_t>(stream),
                       static_cast<const w4a16::f16*>(logits), (int)n, token, position,
                       static_cast<const w4a16::f16*>(table), vocab, (int)hidden, static_cast<w4a16::f16*>(output));
    return check_launch();
}

int w4a16_embedding_f16(const void* table, int64_t vocab, int64_t hidden, const int64_t* token, void* output,
                        void* stream) {
    if (!table || !token || !output) return fail(W4A16_ERR_NULL, "embedding: every pointer must be non-NULL");
    if (vocab <= 0 || hidden <= 0 || hidden > INT32_MAX / 2)
        return fail(W4A16_ERR_SHAPE, "embedding: vocab and hidden must be positive");
    const int blocks = (int)((hidden + 255) / 256);
    hipLaunchKernelGGL(w4a16::embedding_kernel, dim3(blocks), dim3(256), 0, static_cast<hipStream_t>(stream),
                       static_cast<const w4a16::f16*>(table), vocab, (int)hidden, token,
                       static_cast<w4a16::f16*>(output));
    return check_launch();
}

}  // extern "C"

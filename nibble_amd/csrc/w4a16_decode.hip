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
// position p (device int64). Lane d:
//   1. rotary embedding, half-split convention (x1 = x[:32], x2 = x[32:]):
//      out[d] = x1*c - x2*s for d < 32, x2*c + x1*s for d >= 32, computed
//      in fp32 and rounded to fp16 (the q and k the cache holds);
//   2. the first query head of each KV group writes k and v to slot p;
//      every head uses its own registers for slot p, so no head reads a
//      slot another workgroup is writing;
//   3. scores s <= p: lanes over slots, fp32 dot / 8 (= sqrt(64)); slots
//      past p are masked out (weight exactly 0, as exp(-inf) is);
//   4. fp32 softmax (max-subtracted), then out[d] = sum_s prob_s v_s[d],
//      rounded to fp16.
// A position outside [0, S) writes NaN to the head's output and touches no
// cache slot.
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(64)
decode_attention(const f16* __restrict__ qkv, f16* __restrict__ k_cache, f16* __restrict__ v_cache,
                 const float* __restrict__ cos_table, const float* __restrict__ sin_table,
                 const int64_t* __restrict__ position, f16* __restrict__ out, int num_heads, int num_kv, int S) {
    constexpr int D = 64;
    extern __shared__ float shm[];   // [64] q, [64] k_new, [64] v_new, [S] scores
    float* qs = shm;
    float* ks = shm + D;
    float* vs = shm + 2 * D;
    float* prob = shm + 3 * D;

    const int hq = blockIdx.x;
    const int d = threadIdx.x;
    const int group = num_heads / num_kv;
    const int hk = hq / group;
    const int64_t p64 = position[0];
    if (p64 < 0 || p64 >= S) {
        out[(size_t)hq * D + d] = (f16)__builtin_nanf("");
        return;
    }
    const int p = (int)p64;

    const float c = cos_table[(size_t)p * (D / 2) + (d & 31)];
    const float s = sin_table[(size_t)p * (D / 2) + (d & 31)];
    const f16* q = qkv + (size_t)hq * D;
    const f16* k = qkv + (size_t)num_heads * D + (size_t)hk * D;
    const f16* v = qkv + (size_t)(num_heads + num_kv) * D + (size_t)hk * D;
    const float qa = (float)q[d], qb = (float)q[d ^ 32];
    const float ka = (float)k[d], kb = (float)k[d ^ 32];
    const float qr = d < 32 ? qa * c - qb * s : qa * c + qb * s;
    const float kr = d < 32 ? ka * c - kb * s : ka * c + kb * s;
    const f16 q16 = (f16)qr, k16 = (f16)kr, v16 = v[d];
    qs[d] = (float)q16;
    ks[d] = (float)k16;
    vs[d] = (float)v16;
    if (hq % group == 0) {
        k_cache[((size_t)hk * S + p) * D + d] = k16;
        v_cache[((size_t)hk * S + p) * D + d] = v16;
    }
    __syncthreads();

    // scores, lanes over slots
    const f16* kc = k_cache + (size_t)hk * S * D;
    float mx = -__builtin_inff();
    for (int t = d; t <= p; t += 64) {
        float dot = 0.0f;
        if (t == p) {
#pragma unroll 8
            for (int e = 0; e < D; ++e) dot = __builtin_fmaf(qs[e], ks[e], dot);
        } else {
            const u32x4* row = reinterpret_cast<const u32x4*>(kc + (size_t)t * D);
#pragma unroll
            for (int e8 = 0; e8 < D / 8; ++e8) {
                const u32x4 kv8 = row[e8];
#pragma unroll
                for (int w = 0; w < 4; ++w) {
                    const f16x2 h = as_f16x2(kv8[w]);
                    dot = __builtin_fmaf(qs[e8 * 8 + 2 * w], (float)h.x, dot);
                    dot = __builtin_fmaf(qs[e8 * 8 + 2 * w + 1], (float)h.y, dot);
                }
            }
        }
        const float score = dot / 8.0f;
        prob[t] = score;
        mx = fmaxf(mx, score);
    }
    // wavefront max and sum (every lane active)
    for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
    float sum = 0.0f;
    for (int t = d; t <= p; t += 64) {
        const float e = expf(prob[t] - mx);
        prob[t] = e;
        sum += e;
    }
    for (int off = 32; off >= 1; off >>= 1) sum += __shfl_xor(sum, off);
    __syncthreads();

    // out[d] = sum_t prob_t v_t[d] / sum
    const f16* vc = v_cache + (size_t)hk * S * D;
    float acc = 0.0f;
    for (int t = 0; t < p; ++t) acc = __builtin_fmaf(prob[t], (float)vc[(size_t)t * D + d], acc);
    acc = __builtin_fmaf(prob[p], vs[d], acc);
    out[(size_t)hq * D + d] = (f16)(acc / sum);
}

// ---------------------------------------------------------------------------
// Greedy argmax over fp16 logits (first index of the maximum, as
// torch.argmax), one workgroup of 1024 threads; writes the token and, when
// given, advances the position by one.
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(1024)
argmax_kernel(const f16* __restrict__ logits, int n, int64_t* __restrict__ token, int64_t* __restrict__ position) {
    __shared__ float best_v[16];
    __shared__ int best_i[16];
    float bv = -__builtin_inff();
    int bi = n;   // sentinel: larger than any index
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
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
        token[0] = bi < n ? bi : 0;
        if (position != nullptr) position[0] += 1;
    }
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
    const int lds = (int)(3 * 64 + max_seq_len) * 4;
    hipLaunchKernelGGL(w4a16::decode_attention, dim3((unsigned)num_heads), dim3(64), lds,
                       static_cast<hipStream_t>(stream), static_cast<const w4a16::f16*>(qkv),
                       static_cast<w4a16::f16*>(k_cache), static_cast<w4a16::f16*>(v_cache), cos_table, sin_table,
                       position, static_cast<w4a16::f16*>(output), (int)num_heads, (int)num_kv_heads,
                       (int)max_seq_len);
    return check_launch();
}

int w4a16_argmax_f16(const void* logits, int64_t n, int64_t* token, int64_t* position, void* stream) {
    if (!logits || !token) return fail(W4A16_ERR_NULL, "argmax: logits and token must be non-NULL");
    if (n <= 0 || n > INT32_MAX - 1024) return fail(W4A16_ERR_SHAPE, "argmax: n must be in 1..2^31-1025");
    hipLaunchKernelGGL(w4a16::argmax_kernel, dim3(1), dim3(1024), 0, static_cast<hipStream_t>(stream),
                       static_cast<const w4a16::f16*>(logits), (int)n, token, position);
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

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
#include <utility>
#include <type_traits>

#include "w4a16_attn_device.h"
#include "w4a16_device.h"

namespace w4a16 {

// ---------------------------------------------------------------------------
// Attention of one new token, one workgroup of WA wavefronts per query head
// (head_dim 64).
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
//   2. slots 0..p in chunks of 64, wavefront w taking chunks w, w + WA, ...:
//      lane t holds slot c0 + t's key row (8 16-byte loads, requested before
//      any is used) and its score q.k / 8 in fp32; the chunk's value rows go
//      to the wavefront's LDS tile (coalesced 16-byte loads, rows past p
//      zeroed); an online softmax (running max, rescaled sum and output; DPP
//      reductions) folds the chunk in, and lane d accumulates
//      sum_t prob_t v_t[d]. The next chunk's rows are requested before the
//      current chunk's reductions;
//   3. the WA partial states (max m_w, sum l_w, output o_w) combine as
//      out[d] = sum_w o_w[d] e^(m_w - M) / sum_w l_w e^(m_w - M), rounded to
//      fp16 (a wavefront with no chunk has l_w = 0 and drops out).
// Slots past p get weight exactly 0. A position outside [0, S) writes NaN
// to the head's output and touches no cache slot. Every load that does not
// depend on the position (cache rows of each wavefront's first chunk, q, k,
// v) is requested before the position arrives.
// ---------------------------------------------------------------------------
// SPLIT: workgroup (hq, s) of gridDim.y attends a share of the slots 0 .. p
// (64-slot aligned, the shares in slot order) and writes its unnormalised
// state to partial[hq][s] = {max, sum, acc[64]} for decode_attention_merge;
// only share 0 appends the new k / v rows.
template <int WA, bool SPLIT>
__global__ void __launch_bounds__(64 * WA)
decode_attention(const f16* __restrict__ qkv, f16* __restrict__ k_cache, f16* __restrict__ v_cache,
                 const float* __restrict__ cos_table, const float* __restrict__ sin_table,
                 const int64_t* __restrict__ position, f16* __restrict__ out, int num_heads, int num_kv, int S,
                 float* __restrict__ partial) {
    static_assert(!SPLIT || WA > 1, "the split form merges its wavefronts through LDS");
    constexpr int D = 64;
    __shared__ __align__(16) float qs_all[WA][D];
    __shared__ __align__(16) f16 knew_all[WA][D];
    __shared__ __align__(16) f16 vnew_all[WA][D];
    __shared__ __align__(16) float probs[WA][64];
    __shared__ __align__(16) f16 vt[WA][64 * D];
    __shared__ float wmax[WA], wsum[WA];
    __shared__ float wacc[WA][D];

    const int64_t p64 = position[0];
    __builtin_amdgcn_sched_barrier(0);
    const int hq = blockIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int group = num_heads / num_kv;
    const int hk = hq / group;
    const f16* kc = k_cache + (size_t)hk * S * D;
    const f16* vc = v_cache + (size_t)hk * S * D;

    auto load_k = [&](u32x4 (&kr)[8], int c0) {
        const u32x4* row = reinterpret_cast<const u32x4*>(kc + (size_t)min(c0 + lane, S - 1) * D);
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
    int c0 = 64 * wave;
    int end = 0;   // slots c0 .. end - 1 (set below for the unsplit form)
    if constexpr (SPLIT) {
        const int pe = (p64 >= 0 && p64 < S) ? (int)p64 : 0;
        // at least 3 chunks per share: shorter contexts use fewer shares
        const int per = max(((pe + (int)gridDim.y) / (int)gridDim.y + 63) & ~63, 192);
        const int lo = min((int)blockIdx.y * per, pe + 1);
        c0 += lo;
        end = min(lo + per, pe + 1);
    }
    load_k(kr, c0);
    load_v(vr, c0);
    const f16* q = qkv + (size_t)hq * D;
    const f16* k = qkv + (size_t)num_heads * D + (size_t)hk * D;
    const f16* v = qkv + (size_t)(num_heads + num_kv) * D + (size_t)hk * D;
    const f16 qa16 = q[lane], qb16 = q[lane ^ 32], ka16 = k[lane], kb16 = k[lane ^ 32];
    const f16 v16 = v[lane];
    __builtin_amdgcn_sched_barrier(0);

    const bool valid = p64 >= 0 && p64 < S;
    const int p = valid ? (int)p64 : 0;
    const float c = cos_table[(size_t)p * (D / 2) + (lane & 31)];
    const float s = sin_table[(size_t)p * (D / 2) + (lane & 31)];
    const float qa = (float)qa16, qb = (float)qb16, ka = (float)ka16, kb = (float)kb16;
    const float qr = lane < 32 ? qa * c - qb * s : qa * c + qb * s;
    const float kro = lane < 32 ? ka * c - kb * s : ka * c + kb * s;
    const f16 q16 = (f16)qr, k16 = (f16)kro;
    // every wavefront keeps its own copy (no branch the loads above could sink into)
    float* qs = qs_all[wave];
    f16* knew = knew_all[wave];
    f16* vnew = vnew_all[wave];
    qs[lane] = (float)q16;
    knew[lane] = k16;
    vnew[lane] = v16;
    if (valid && wave == 0 && hq % group == 0 && (!SPLIT || blockIdx.y == 0)) {
        k_cache[((size_t)hk * S + p) * D + lane] = k16;
        v_cache[((size_t)hk * S + p) * D + lane] = v16;
    }
    wave_lds_sync();
    if (!valid) {   // (the split form's merge writes the NaN rows)
        if (!SPLIT && wave == 0) out[(size_t)hq * D + lane] = (f16)__builtin_nanf("");
        return;
    }
    if constexpr (!SPLIT) end = p + 1;

    float run_max = -__builtin_inff(), run_sum = 0.0f, acc = 0.0f;
    f16* my_vt = vt[wave];
    float* my_probs = probs[wave];
    for (; c0 < end; c0 += 64 * WA) {
        const int t = c0 + lane;
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
        const float score = t < end ? dot * 0.125f : -__builtin_inff();
        // value rows of the chunk to LDS: rows past p zeroed, slot p from vnew
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int row = (lane >> 3) + 8 * i;
            const int slot = c0 + row;
            u32x4 val = vr[i];
            if (slot == p) val = reinterpret_cast<const u32x4*>(vnew)[lane & 7];
            if (slot >= end) val = (u32x4){0u, 0u, 0u, 0u};
            reinterpret_cast<u32x4*>(my_vt + row * D)[lane & 7] = val;
        }
        // next chunk's rows requested before this chunk's reductions
        const int next = c0 + 64 * WA;
        if (next < end) {
            load_k(kr, next);
            load_v(vr, next);
        }
        const float cmax = wave_max(score);
        const float new_max = fmaxf(run_max, cmax);
        const float pr = t < end ? expf(score - new_max) : 0.0f;
        const float psum = wave_sum(pr);
        const float rescale = expf(run_max - new_max);   // 0 on the first chunk
        my_probs[lane] = pr;
        wave_lds_sync();
        float part = 0.0f;
#pragma unroll
        for (int r4 = 0; r4 < 16; ++r4) {
            const f32x4 pp = reinterpret_cast<const f32x4*>(my_probs)[r4];
            part = __builtin_fmaf(pp.x, (float)my_vt[(4 * r4 + 0) * D + lane], part);
            part = __builtin_fmaf(pp.y, (float)my_vt[(4 * r4 + 1) * D + lane], part);
            part = __builtin_fmaf(pp.z, (float)my_vt[(4 * r4 + 2) * D + lane], part);
            part = __builtin_fmaf(pp.w, (float)my_vt[(4 * r4 + 3) * D + lane], part);
        }
        wave_lds_sync();
        acc = acc * rescale + part;
        run_sum = run_sum * rescale + psum;
        run_max = new_max;
    }
    if constexpr (WA == 1) {
        out[(size_t)hq * D + lane] = (f16)(acc / run_sum);
        return;
    }
    if (lane == 0) {
        wmax[wave] = run_max;
        wsum[wave] = run_sum;
    }
    wacc[wave][lane] = acc;
    __syncthreads();
    if (wave != 0) return;
    float m = wmax[0];
#pragma unroll
    for (int w = 1; w < WA; ++w) m = fmaxf(m, wmax[w]);
    float num = 0.0f, den = 0.0f;
#pragma unroll
    for (int w = 0; w < WA; ++w) {
        const float f = wsum[w] > 0.0f ? expf(wmax[w] - m) : 0.0f;
        num = __builtin_fmaf(wacc[w][lane], f, num);
        den = __builtin_fmaf(wsum[w], f, den);
    }
    if constexpr (SPLIT) {
        // a share past p (no slots) leaves max -inf and sum 0
        float* pp = partial + ((size_t)hq * gridDim.y + blockIdx.y) * (D + 2);
        if (lane == 0) {
            pp[0] = m;
            pp[1] = den;
        }
        pp[2 + lane] = num;
    } else {
        out[(size_t)hq * D + lane] = (f16)(num / den);
    }
}

// The split form's states of head blockIdx.x merged: out = sum_s acc_s e^(m_s - m)
// / sum_s sum_s e^(m_s - m), m the largest share maximum (shares with no slots
// skipped); NaN rows for a position outside [0, S).
__global__ void __launch_bounds__(64)
decode_attention_merge(const float* __restrict__ partial, const int64_t* __restrict__ position,
                       f16* __restrict__ out, int splits, int S) {
    constexpr int D = 64;
    const int hq = blockIdx.x, lane = threadIdx.x;
    const int64_t p64 = position[0];
    // every share's values requested together (the workspace is read in
    // bounds whatever the position; an invalid one only selects NaN at the end)
    const float* pp = partial + (size_t)hq * splits * (D + 2);
    float m = -__builtin_inff();
#pragma unroll 8
    for (int s = 0; s < splits; ++s) m = fmaxf(m, pp[(size_t)s * (D + 2)]);
    float num = 0.0f, den = 0.0f;
#pragma unroll 8
    for (int s = 0; s < splits; ++s) {
        const float* ps = pp + (size_t)s * (D + 2);
        const float l = ps[1], a = ps[2 + lane];
        const float f = l > 0.0f ? expf(ps[0] - m) : 0.0f;
        num = __builtin_fmaf(a, f, num);
        den = __builtin_fmaf(l, f, den);
    }
    const bool valid = p64 >= 0 && p64 < S;
    out[(size_t)hq * D + lane] = valid ? (f16)(num / den) : (f16)__builtin_nanf("");
}

// ---------------------------------------------------------------------------
// Greedy argmax over fp16 logits (first index of the maximum, as
// torch.argmax: any NaN counts as the largest value, so the first NaN wins,
// and -0 equals +0), one workgroup of 1024 threads
// reading 16-byte vectors when the logits are 16-byte aligned; writes the
// token (and, when given, the same to token_copy, a slot of a token
// history) and, when given, advances the position by one and gathers the
// token's embedding row into `emb_out` (the next decode step's input), so the
// step needs no separate gather. Two passes: the maximum (IEEE 754-2019
// maximum, which propagates NaN: v_pk_maximum3_f16 over each thread's
// vectors, v_maximum3_f32 across the workgroup), and the first index that
// holds it (the first NaN when the maximum is NaN), searched only by the
// threads whose own maximum it is (from the registers of the first round,
// re-read past it). The position is read at
// launch and the last steps (the winners' reduction, the token, the gather)
// run in wavefront 0 alone.
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(1024)
argmax_kernel(const f16* __restrict__ logits, int n, int64_t* __restrict__ token, int64_t* __restrict__ position,
              const f16* __restrict__ table, int64_t vocab, int hidden, f16* __restrict__ emb_out,
              int64_t* __restrict__ token_copy) {
    constexpr int T = 1024;
    __shared__ float wave_max[T / 64];
    __shared__ int wave_first[T / 64];
    // the position is requested first, so its round trip overlaps the logits'
    const int64_t pos0 = (position != nullptr && threadIdx.x == 0) ? position[0] : 0;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const bool vec = (reinterpret_cast<uintptr_t>(logits) & 15u) == 0;
    const int nv = vec ? n >> 3 : 0;
    constexpr int kBatch = 4;   // vectors requested per thread before any is compared
    const f16 ninf = __builtin_bit_cast(f16, (uint16_t)0xFC00u);
    f16x2 m2 = {ninf, ninf};
    u32x4 u[kBatch];   // after the loop: the last round's vectors (the only round when nv <= kBatch T)
    for (int j0 = tid; j0 < nv; j0 += kBatch * T) {
#pragma unroll
        for (int b = 0; b < kBatch; ++b) u[b] = reinterpret_cast<const u32x4*>(logits)[min(j0 + b * T, nv - 1)];
#pragma unroll
        for (int b = 0; b < kBatch; ++b)
            if (j0 + b * T < nv)
#pragma unroll
                for (int e = 0; e < 4; ++e) m2 = __builtin_elementwise_maximum(m2, as_f16x2(u[b][e]));
    }
    for (int i = 8 * nv + tid; i < n; i += T) m2.x = __builtin_elementwise_maximum(m2.x, logits[i]);
    const float mine = __builtin_elementwise_maximum((float)m2.x, (float)m2.y);
    float gm = mine;
    for (int off = 32; off >= 1; off >>= 1) gm = __builtin_elementwise_maximum(gm, __shfl_xor(gm, off));
    if (lane == 0) wave_max[wave] = gm;
    __syncthreads();
#pragma unroll
    for (int w = 0; w < T / 64; ++w) gm = __builtin_elementwise_maximum(gm, wave_max[w]);
    const bool any_nan = gm != gm;

    // the first index holding the target among this thread's elements, in
    // index order (rounds, vectors of a round, elements of a vector, then the
    // tail): gm, or the first NaN when any logit is one (a compact loop of its
    // own, re-reading the thread's logits: the common path keeps its code
    // size); every logit -inf gives token 0
    int first = n;
    if (__builtin_expect(any_nan, false)) {
        if (mine != mine) {
#pragma unroll 1
            for (int j = tid; j < nv && first == n; j += T) {
                const u32x4 v = reinterpret_cast<const u32x4*>(logits)[j];
#pragma unroll 1
                for (int e = 0; e < 8; ++e)
                    if (((v[e >> 1] >> (16 * (e & 1))) & 0x7fffu) > 0x7c00u) {
                        first = 8 * j + e;
                        break;
                    }
            }
#pragma unroll 1
            for (int i = 8 * nv + tid; i < n && first == n; i += T)
                if ((__builtin_bit_cast(uint16_t, logits[i]) & 0x7fffu) > 0x7c00u) first = i;
        }
    } else if (mine == gm && gm != -__builtin_inff()) {
        const bool one_round = nv <= kBatch * T;
        for (int j0 = tid; j0 < nv; j0 += kBatch * T) {
            if (!one_round)
#pragma unroll
                for (int b = 0; b < kBatch; ++b) u[b] = reinterpret_cast<const u32x4*>(logits)[min(j0 + b * T, nv - 1)];
#pragma unroll
            for (int b = 0; b < kBatch; ++b) {
                const int j = j0 + b * T;
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const f16x2 h = as_f16x2(u[b][e >> 1]);
                    if (j < nv && (float)((e & 1) ? h.y : h.x) == gm) first = min(first, 8 * j + e);
                }
            }
            if (first < n) break;
        }
        for (int i = 8 * nv + tid; i < n && first == n; i += T)
            if ((float)logits[i] == gm) first = i;
    }
    for (int off = 32; off >= 1; off >>= 1) first = min(first, __shfl_xor(first, off));
    if (lane == 0) wave_first[wave] = first;
    __syncthreads();
    if (wave != 0) return;
    // wavefront 0: the smallest of the 16 wavefronts' first indices, the
    // token, the position, the gather
    first = lane < T / 64 ? wave_first[lane] : n;
    for (int off = 8; off >= 1; off >>= 1) first = min(first, __shfl_xor(first, off));
    first = __shfl(first, 0);
    const int64_t t = first < n ? first : 0;
    if (lane == 0) {
        token[0] = t;
        if (token_copy != nullptr) token_copy[0] = t;
        if (position != nullptr) position[0] = pos0 + 1;
    }
    if (emb_out == nullptr) return;
    const f16* row = table + t * hidden;
    const bool in_range = t < vocab;
    if ((hidden & 7) == 0 && ((reinterpret_cast<uintptr_t>(row) | reinterpret_cast<uintptr_t>(emb_out)) & 15u) == 0) {
        const int nvec = hidden >> 3;
        for (int i0 = lane; i0 < nvec; i0 += 4 * 64) {
            u32x4 v[4];
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                const int i = min(i0 + 64 * b, nvec - 1);
                v[b] = in_range ? reinterpret_cast<const u32x4*>(row)[i] : (u32x4){0u, 0u, 0u, 0u};
            }
#pragma unroll
            for (int b = 0; b < 4; ++b)
                if (i0 + 64 * b < nvec) reinterpret_cast<u32x4*>(emb_out)[i0 + 64 * b] = v[b];
        }
    } else {
        for (int i = lane; i < hidden; i += 64) emb_out[i] = in_range ? row[i] : (f16)0.0f;
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


// ---------------------------------------------------------------------------
// Attention of one new token fused with the o projection and the residual
// add, for positions p < 64 (one chunk of cache slots), head_dim 64.
//
// Grid: ceil(N / (R * W)) workgroups of W wavefronts, N = hidden size, W =
// KV, or 2 KV with HV (the cached form): wavefronts KV .. 2 KV - 1 then only
// load the V rows of KV head w - KV into the V tile (a workgroup barrier
// before O^T), so each CU's 64 KB of cache rows are requested by twice the
// wavefronts (the per-CU request rate, not the bytes, bounds this staging).
// Every workgroup recomputes the whole attention output (all H = KV * group
// query heads over slots 0..p) from the caches, keeps it in LDS as the o
// GEMV's activation row (unit-major: 16-byte unit q of 32-weight chunk c at
// slot q C + c, natural order) and then runs the GEMV for its R * W output
// rows (every wavefront, helpers included) with the exact decode (unpack8
// against permute8 of the unit), so no staging pass follows the attention;
// the o weights and the rows' residual values are requested at launch, so
// they stream in while the attention runs. Wavefront g < KV handles KV head
// g and its `group` query heads (group <= 16) on the matrix cores:
//   S^T = K Q^T (v_mfma_f32_16x16x32_f16; A = cache rows, lane (q4, j) holds
//     slot 16 mt + j, dims 32 s + 8 q4 .. +8; B = rotated q of head j), so
//     lane (q4, j) receives head j's scores for slots 16 mt + 4 q4 + e;
//   softmax per head over its 64 slots (masked past p; the four lanes of a
//     head combine through two cross-row exchanges), scale 1/8;
//   O^T = V^T P^T: B = P^T straight from the score registers (virtual slot
//     32 s + 8 q4 + i is slot 16 (2 s + i / 4) + 4 q4 + i % 4, the order the
//     lane already holds), A = V^T read from a row-major V tile in LDS (each
//     lane stores its cache row, slots past p zeroed so that no stale value
//     meets a zero weight) with ds_read_b64_tr_b16: within each 16-lane
//     group, lane i receives half i % 4 of the 8 bytes addressed by lanes
//     4k + i / 4 (k = 0..3), so lanes 4k + m pointing at slot s0 + k, dims
//     d0 + 4m give lane i the four slots s0..s0+3 of dim d0 + i.
// Rotary embedding (half-split, as decode_attention) uses cos / sin of
// p * inv_freq[i] computed in the kernel (fp32 product, sincosf), so no load
// waits on the position; q and the new k are rotated in fp32 and rounded to
// fp16; slot p's k and v come from qkv (registers / LDS), never from the
// cache line that workgroup 0 writes (the append) in the same launch.
// Output rows: resid[n] = fp16(fp32(resid[n]) + fp32(fp16(dot))). A position
// outside [0, min(S, 64)) makes every attention value NaN (so the residual
// stream turns NaN) and touches no cache slot.
// ---------------------------------------------------------------------------
constexpr int kAttnOSlots = 64;
constexpr int kVStride = 72;   // V tile row stride in halves (144 bytes: conflict-free 16-byte stores)

template <int KV, int R, int L, bool CACHED, bool HV = false>
__global__ void __launch_bounds__(64 * KV * (HV ? 2 : 1))
attn_o_kernel(const f16* __restrict__ qkv, f16* __restrict__ k_cache, f16* __restrict__ v_cache,
              const float* __restrict__ inv_freq, const int64_t* __restrict__ position,
              const uint8_t* __restrict__ w, const f16* __restrict__ scales, f16* resid, int group, int S,
              int N) {
    static_assert(!HV || CACHED, "V helper wavefronts serve the cached form (slot p already in the caches)");
    constexpr int D = 64;
    constexpr int NW = KV * (HV ? 2 : 1);   // wavefronts per workgroup
    const int64_t p64 = position[0];
    const float freq = CACHED ? 0.0f : inv_freq[threadIdx.x & 31];
    __builtin_amdgcn_sched_barrier(0);
    extern __shared__ __align__(16) uint8_t smem[];
    const int H = KV * group;
    const int K = H * D;                 // o projection input width
    const int C = K >> 5, G = K >> 7;
    f16* vt_all = reinterpret_cast<f16*>(smem);                        // [KV][64 slots][kVStride]
    u32x4* xs = reinterpret_cast<u32x4*>(vt_all + KV * kAttnOSlots * kVStride);   // [4][C] attention units
    float* trig_all = reinterpret_cast<float*>(xs + 4 * C);             // [KV][64]: cos | sin

    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int q4 = lane >> 4, j = lane & 15;
    // HV: wavefronts KV .. 2 KV - 1 load the V rows of KV head wave - KV into
    // the V tile while wavefronts 0 .. KV - 1 load K and q and attend
    const bool helper = HV && wave >= KV;
    const int g = HV ? (wave & (KV - 1)) : wave;
    const f16* kc = k_cache + (size_t)g * S * D;
    const f16* vc = v_cache + (size_t)g * S * D;
    const int hq = g * group + min(j, group - 1);

    // 1. every load that does not need the position
    u32x4 ka[4][2] = {};
    if (!helper) {
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
            const int row = min(16 * mt + j, S - 1);
#pragma unroll
            for (int s = 0; s < 2; ++s)
                ka[mt][s] = *reinterpret_cast<const u32x4*>(kc + (size_t)row * D + 32 * s + 8 * q4);
        }
    }
    u32x4 vr[8] = {};
    if (!HV || helper) {
        const int row = min(lane, S - 1);
#pragma unroll
        for (int e = 0; e < 8; ++e) vr[e] = reinterpret_cast<const u32x4*>(vc + (size_t)row * D)[e];
    }
    u32x4 qb[2] = {}, kn[2];
    if (!helper) {
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            qb[s] = *reinterpret_cast<const u32x4*>(qkv + (size_t)hq * D + 32 * s + 8 * q4);
            if (!CACHED) kn[s] = *reinterpret_cast<const u32x4*>(qkv + (size_t)(H + g) * D + 32 * s + 8 * q4);
        }
    }
    const f16 vn = CACHED ? (f16)0.0f : qkv[(size_t)(H + KV + g) * D + lane];
    // o weights and scales of this wavefront's R rows (one-shot layout)
    const int row0 = (blockIdx.x * NW + wave) * R;
    const uint32_t row_bytes = (uint32_t)(K >> 1);
    uint32_t sv[R][L];
    u32x4 wv[R][L];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int n = min(row0 + r, N - 1);
        const uint16_t* srow = reinterpret_cast<const uint16_t*>(scales) + (size_t)n * G;
#pragma unroll
        for (int l = 0; l < L; ++l) sv[r][l] = srow[min(l * 64 + lane, C - 1) >> 2];
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int n = min(row0 + r, N - 1);
        const uint8_t* wrow = w + (size_t)n * row_bytes;
#pragma unroll
        for (int l = 0; l < L; ++l) {
            const uint32_t c = (uint32_t)min(l * 64 + lane, C - 1);
            wv[r][l] = load_stream(reinterpret_cast<const u32x4*>(wrow + c * 16u));
        }
    }
    // the rows' residual values (each is read and rewritten by this lane 0 only)
    f16 res[R];
#pragma unroll
    for (int r = 0; r < R; ++r) res[r] = resid[min(row0 + r, N - 1)];
    __builtin_amdgcn_sched_barrier(0);

    const bool valid = p64 >= 0 && p64 < S && p64 < kAttnOSlots;
    const int p = valid ? (int)p64 : 0;

    u32x4 qr[2];
    if constexpr (CACHED) {
        // q arrives rotated and slot p is already in the caches
        qr[0] = qb[0];
        qr[1] = qb[1];
    } else {
        // 2. cos / sin of p * inv_freq, one frequency per lane (two copies)
        float* trig = trig_all + wave * 64;
        {
            float sn, cs;
            sincosf((float)p * freq, &sn, &cs);
            trig[lane] = lane < 32 ? cs : sn;
        }
        wave_lds_sync();
        // rotate q (B operand) and the new k: dims 8 q4 + i (s = 0) pair with 32 + 8 q4 + i (s = 1)
        u32x4 kr[2];
#pragma unroll
        for (int h = 0; h < 4; ++h) {
            const float c0 = trig[8 * q4 + 2 * h], c1 = trig[8 * q4 + 2 * h + 1];
            const float s0 = trig[32 + 8 * q4 + 2 * h], s1 = trig[32 + 8 * q4 + 2 * h + 1];
            const f16x2 qa = as_f16x2(qb[0][h]), qz = as_f16x2(qb[1][h]);
            const f16x2 ka2 = as_f16x2(kn[0][h]), kz = as_f16x2(kn[1][h]);
            const f16x2 qlo = {(f16)((float)qa.x * c0 - (float)qz.x * s0), (f16)((float)qa.y * c1 - (float)qz.y * s1)};
            const f16x2 qhi = {(f16)((float)qz.x * c0 + (float)qa.x * s0), (f16)((float)qz.y * c1 + (float)qa.y * s1)};
            const f16x2 klo = {(f16)((float)ka2.x * c0 - (float)kz.x * s0), (f16)((float)ka2.y * c1 - (float)kz.y * s1)};
            const f16x2 khi = {(f16)((float)kz.x * c0 + (float)ka2.x * s0), (f16)((float)kz.y * c1 + (float)ka2.y * s1)};
            qr[0][h] = as_u32(qlo);
            qr[1][h] = as_u32(qhi);
            kr[0][h] = as_u32(klo);
            kr[1][h] = as_u32(khi);
        }
        // slot p's key row is the new k (never the cache line being written)
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
            const bool is_p = 16 * mt + j == p;
#pragma unroll
            for (int s = 0; s < 2; ++s) ka[mt][s] = is_p ? kr[s] : ka[mt][s];
        }
        // the append: workgroup 0 writes slot p of this KV head
        if (blockIdx.x == 0 && valid) {
            if (j == 0) {
#pragma unroll
                for (int s = 0; s < 2; ++s)
                    *reinterpret_cast<u32x4*>(k_cache + ((size_t)g * S + p) * D + 32 * s + 8 * q4) = kr[s];
            }
            v_cache[((size_t)g * S + p) * D + lane] = vn;
        }
    }

    // 3. V tile into LDS, row-major: lane l stores slot l (zero past p), then
    // slot p from qkv
    f16* vt = vt_all + g * kAttnOSlots * kVStride;
    if (!HV || helper) {
        const bool live = lane <= p;
        u32x4* row = reinterpret_cast<u32x4*>(vt + lane * kVStride);
#pragma unroll
        for (int e = 0; e < 8; ++e) row[e] = live ? vr[e] : (u32x4){0u, 0u, 0u, 0u};
        if (!CACHED) {
            wave_lds_sync();
            vt[p * kVStride + lane] = vn;
        }
    }

    // 4. S^T = K Q^T, softmax over the head's 64 slots
    f32x4 st[4];
    float sum = 0.0f;
    u32x4 pb[2];   // P^T as the B operand of the two k-steps
    if (!helper) {
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
        st[mt] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int s = 0; s < 2; ++s)
            st[mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, ka[mt][s]),
                                                            __builtin_bit_cast(f16x8, qr[s]), st[mt], 0, 0, 0);
    }
    float mx = -__builtin_inff();
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int slot = 16 * mt + 4 * q4 + e;
            st[mt][e] = slot <= p ? st[mt][e] * 0.125f : -__builtin_inff();
            mx = fmaxf(mx, st[mt][e]);
        }
    mx = row_pair_max(mx);
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
        float pe[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int slot = 16 * mt + 4 * q4 + e;
            pe[e] = slot <= p ? __expf(st[mt][e] - mx) : 0.0f;
            sum += pe[e];
        }
        const f16x2 a = {(f16)pe[0], (f16)pe[1]}, b = {(f16)pe[2], (f16)pe[3]};
        pb[mt >> 1][2 * (mt & 1)] = as_u32(a);
        pb[mt >> 1][2 * (mt & 1) + 1] = as_u32(b);
    }
    sum = row_pair_sum(sum);
    }
    // the V tile complete (HV: written by the helper wavefronts)
    if constexpr (HV) __syncthreads();
    else wave_lds_sync();

    // 5. O^T = V^T P^T; lane (q4, j) receives head j, dims 16 md + 4 q4 + e
    if (!helper) {
    const float inv_sum = valid ? 1.0f / sum : __builtin_nanf("");
    const int tk = j >> 2, tm = j & 3;   // this lane's row / 4-dim block in the transposing read
#pragma unroll
    for (int md = 0; md < 4; ++md) {
        f32x4 o = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            const f16* src = vt + (32 * s + 4 * q4 + tk) * kVStride + 16 * md + 4 * tm;
            const uint2 lo = lds_read_tr16(src);
            const uint2 hi = lds_read_tr16(src + 16 * kVStride);
            const u32x4 a = {lo.x, lo.y, hi.x, hi.y};
            o = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, pb[s]), o,
                                                       0, 0, 0);
        }
        if (j < group) {
            const f16x2 a = {(f16)(o[0] * inv_sum), (f16)(o[1] * inv_sum)};
            const f16x2 b = {(f16)(o[2] * inv_sum), (f16)(o[3] * inv_sum)};
            // dims k .. k+3 of the row: chunk k / 32, unit (k / 8) % 4, halves k % 8 ..
            const int k = (g * group + j) * D + 16 * md + 4 * q4;
            uint8_t* dst = reinterpret_cast<uint8_t*>(xs + ((k >> 3) & 3) * C + (k >> 5)) + (k & 7) * 2;
            *reinterpret_cast<uint2*>(dst) = make_uint2(as_u32(a), as_u32(b));
        }
    }
    }
    __syncthreads();

    // 6. o rows: exact decode against the permuted attention units, then the
    // residual add
    u32x4 xp[L][4];
#pragma unroll
    for (int l = 0; l < L; ++l)
#pragma unroll
        for (int qq = 0; qq < 4; ++qq) xp[l][qq] = permute8(xs[qq * C + min(l * 64 + lane, C - 1)]);
#pragma unroll
    for (int r = 0; r < R; ++r) {
        float acc = 0.0f;
#pragma unroll
        for (int l = 0; l < L; ++l) {
            const int c = l * 64 + lane;
            float d = 0.0f;
#pragma unroll
            for (int qq = 0; qq < 4; ++qq) {
                const Codes8 cw = unpack8(wv[r][l][qq]);
                d = __builtin_amdgcn_fdot2(as_f16x2(xp[l][qq].x), cw.p[0], d, false);
                d = __builtin_amdgcn_fdot2(as_f16x2(xp[l][qq].y), cw.p[1], d, false);
                d = __builtin_amdgcn_fdot2(as_f16x2(xp[l][qq].z), cw.p[2], d, false);
                d = __builtin_amdgcn_fdot2(as_f16x2(xp[l][qq].w), cw.p[3], d, false);
            }
            const float sc = (float)__builtin_bit_cast(f16, (uint16_t)sv[r][l]);
            acc = __builtin_fmaf(c < C ? d : 0.0f, sc, acc);
        }
        const float v = wave_sum(acc);
        const int n = row0 + r;
        if (lane == 0 && n < N) resid[n] = (f16)((float)res[r] + (float)(f16)v);
    }
}


// ---------------------------------------------------------------------------
// Prefill: the element-wise work around the W4A16 projections of a T-token
// prompt, each as one launch.
// ---------------------------------------------------------------------------

// out[r] = fp16((fp32(x[r]) * inv) * fp32(w)), inv = 1 / sqrt(mean(x[r]^2) +
// eps) in fp32: the decode step's RMSNorm, one workgroup per row.
__global__ void __launch_bounds__(256)
rmsnorm_rows_kernel(const f16* __restrict__ x, const f16* __restrict__ w, float eps, f16* __restrict__ out,
                    int hidden) {
    __shared__ float partial[4];
    const f16* xr = x + (size_t)blockIdx.x * hidden;
    f16* orow = out + (size_t)blockIdx.x * hidden;
    float ss = 0.0f;
    for (int i = threadIdx.x; i < hidden; i += 256) {
        const float v = (float)xr[i];
        ss = __builtin_fmaf(v, v, ss);
    }
    ss = wave_sum(ss);
    if ((threadIdx.x & 63) == 0) partial[threadIdx.x >> 6] = ss;
    __syncthreads();
    const float total = (partial[0] + partial[1]) + (partial[2] + partial[3]);
    const float inv = 1.0f / __builtin_sqrtf(total / (float)hidden + eps);
    for (int i = threadIdx.x; i < hidden; i += 256) orow[i] = (f16)(((float)xr[i] * inv) * (float)w[i]);
}

// Residual add + RMSNorm of rows of at most kAddNormMax elements, one
// workgroup per row: s = fp16(fp32(x[r]) + fp32(delta[r])) (the rounding of
// an fp16 tensor add) is written to x_out[r], and out[r] = fp16((fp32(s) *
// inv) * fp32(w)) with inv = 1 / sqrt(mean(s^2) + eps). Every load of a
// thread is issued before its first store (x_out may be x, so a store
// would otherwise order the loads after it), and the row stays in registers
// between the two passes.
constexpr int kAddNormPer = 32;                  // elements per thread
constexpr int kAddNormMax = 256 * kAddNormPer;   // 8192

__global__ void __launch_bounds__(256)
add_rmsnorm_rows_kernel(const f16* x, const f16* __restrict__ delta, const f16* __restrict__ w, float eps,
                        f16* x_out, f16* __restrict__ out, int hidden) {
    __shared__ float partial[4];
    const size_t row = (size_t)blockIdx.x * hidden;
    f16 xa[kAddNormPer], da[kAddNormPer];
#pragma unroll
    for (int j = 0; j < kAddNormPer; ++j) {
        const int i = min((int)threadIdx.x + 256 * j, hidden - 1);
        xa[j] = x[row + i];
        da[j] = delta[row + i];
    }
    float v[kAddNormPer];
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < kAddNormPer; ++j) {
        const int i = threadIdx.x + 256 * j;
        const f16 sum = (f16)((float)xa[j] + (float)da[j]);
        const float sv = i < hidden ? (float)sum : 0.0f;
        if (i < hidden) x_out[row + i] = sum;
        v[j] = sv;
        ss = __builtin_fmaf(sv, sv, ss);
    }
    ss = wave_sum(ss);
    if ((threadIdx.x & 63) == 0) partial[threadIdx.x >> 6] = ss;
    __syncthreads();
    const float total = (partial[0] + partial[1]) + (partial[2] + partial[3]);
    const float inv = 1.0f / __builtin_sqrtf(total / (float)hidden + eps);
#pragma unroll
    for (int j = 0; j < kAddNormPer; ++j) {
        const int i = threadIdx.x + 256 * j;
        if (i < hidden) out[row + i] = (f16)((v[j] * inv) * (float)w[i]);
    }
}

// The same two launches on 16-byte units (rows a multiple of 8 elements, at
// most kAddNormMax, every buffer 16-byte aligned): thread t holds units t,
// t + 256, ... of its row, all requested before any store. ADD = false is
// the plain RMSNorm (x_out, delta unused).
constexpr int kNormUnits = kAddNormMax / 8 / 256;   // 16-byte units per thread (4)

template <bool ADD>
__global__ void __launch_bounds__(256)
norm_rows_vec_kernel(const f16* x, const f16* __restrict__ delta, const f16* __restrict__ w, float eps,
                     f16* x_out, f16* __restrict__ out, int hidden) {
    __shared__ float partial[4];
    const size_t row = (size_t)blockIdx.x * hidden;
    const int units = hidden >> 3;
    u32x4 xv[kNormUnits], dv[kNormUnits], wv[kNormUnits];
#pragma unroll
    for (int u = 0; u < kNormUnits; ++u) {
        const int i = min((int)threadIdx.x + 256 * u, units - 1);
        xv[u] = *reinterpret_cast<const u32x4*>(x + row + (size_t)i * 8);
        if (ADD) dv[u] = *reinterpret_cast<const u32x4*>(delta + row + (size_t)i * 8);
        wv[u] = *reinterpret_cast<const u32x4*>(w + (size_t)i * 8);
    }
    float ss = 0.0f;
#pragma unroll
    for (int u = 0; u < kNormUnits; ++u) {
        const int i = threadIdx.x + 256 * u;
        if (ADD) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const f16x2 a = as_f16x2(xv[u][e]), b = as_f16x2(dv[u][e]);
                const f16x2 sum = {(f16)((float)a.x + (float)b.x), (f16)((float)a.y + (float)b.y)};
                xv[u][e] = as_u32(sum);
            }
            if (i < units) store_through(reinterpret_cast<u32x4*>(x_out + row + (size_t)i * 8), xv[u]);
        }
        if (i < units) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const f16x2 a = as_f16x2(xv[u][e]);
                ss = __builtin_fmaf((float)a.x, (float)a.x, ss);
                ss = __builtin_fmaf((float)a.y, (float)a.y, ss);
            }
        }
    }
    ss = wave_sum(ss);
    if ((threadIdx.x & 63) == 0) partial[threadIdx.x >> 6] = ss;
    __syncthreads();
    const float total = (partial[0] + partial[1]) + (partial[2] + partial[3]);
    const float inv = 1.0f / __builtin_sqrtf(total / (float)hidden + eps);
#pragma unroll
    for (int u = 0; u < kNormUnits; ++u) {
        const int i = threadIdx.x + 256 * u;
        if (i < units) {
            u32x4 o;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const f16x2 a = as_f16x2(xv[u][e]), g = as_f16x2(wv[u][e]);
                const f16x2 y = {(f16)(((float)a.x * inv) * (float)g.x), (f16)(((float)a.y * inv) * (float)g.y)};
                o[e] = as_u32(y);
            }
            store_through(reinterpret_cast<u32x4*>(out + row + (size_t)i * 8), o);
        }
    }
}

// A prompt's embedding rows and their RMSNorm in one launch (the vectorised
// layout of norm_rows_vec_kernel): row r is table[tokens[r]] (zeros for a
// token outside [0, vocab)), written to x_out[r] as the residual stream, and
// out[r] = its RMSNorm with the arithmetic of norm_rows_vec_kernel<false>, so
// both equal the gather followed by that kernel, bit for bit. position (may
// be NULL) <- rows: the decode position after the prompt.
__global__ void __launch_bounds__(256)
embed_norm_rows_kernel(const f16* __restrict__ table, int64_t vocab, const int64_t* __restrict__ tokens,
                       const f16* __restrict__ w, float eps, f16* __restrict__ x_out, f16* __restrict__ out,
                       int hidden, int64_t* __restrict__ position) {
    __shared__ float partial[4];
    const int64_t t = tokens[blockIdx.x];
    const bool in_range = t >= 0 && t < vocab;
    const f16* src = table + (in_range ? t : 0) * (int64_t)hidden;
    const size_t row = (size_t)blockIdx.x * hidden;
    const int units = hidden >> 3;
    u32x4 xv[kNormUnits], wv[kNormUnits];
#pragma unroll
    for (int u = 0; u < kNormUnits; ++u) {
        const int i = min((int)threadIdx.x + 256 * u, units - 1);
        xv[u] = in_range ? *reinterpret_cast<const u32x4*>(src + (size_t)i * 8) : (u32x4){0u, 0u, 0u, 0u};
        wv[u] = *reinterpret_cast<const u32x4*>(w + (size_t)i * 8);
    }
    if (position != nullptr && blockIdx.x == 0 && threadIdx.x == 0) position[0] = (int64_t)gridDim.x;
    float ss = 0.0f;
#pragma unroll
    for (int u = 0; u < kNormUnits; ++u) {
        const int i = threadIdx.x + 256 * u;
        if (i < units) {
            store_through(reinterpret_cast<u32x4*>(x_out + row + (size_t)i * 8), xv[u]);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const f16x2 a = as_f16x2(xv[u][e]);
                ss = __builtin_fmaf((float)a.x, (float)a.x, ss);
                ss = __builtin_fmaf((float)a.y, (float)a.y, ss);
            }
        }
    }
    ss = wave_sum(ss);
    if ((threadIdx.x & 63) == 0) partial[threadIdx.x >> 6] = ss;
    __syncthreads();
    const float total = (partial[0] + partial[1]) + (partial[2] + partial[3]);
    const float inv = 1.0f / __builtin_sqrtf(total / (float)hidden + eps);
#pragma unroll
    for (int u = 0; u < kNormUnits; ++u) {
        const int i = threadIdx.x + 256 * u;
        if (i < units) {
            u32x4 o;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const f16x2 a = as_f16x2(xv[u][e]), g = as_f16x2(wv[u][e]);
                const f16x2 y = {(f16)(((float)a.x * inv) * (float)g.x), (f16)(((float)a.y * inv) * (float)g.y)};
                o[e] = as_u32(y);
            }
            store_through(reinterpret_cast<u32x4*>(out + row + (size_t)i * 8), o);
        }
    }
}

// out[r, i] = fp16(fp16(silu(g)) * u), g = gate_up[r, i], u = gate_up[r, inter + i]:
// the roundings of torch's silu(g) * u on fp16 tensors.
__device__ __forceinline__ f16 silu_mul_one(f16 gh, f16 uh) {
    const float g = (float)gh;
    const f16 sg = (f16)(g / (1.0f + __expf(-g)));
    return (f16)((float)sg * (float)uh);
}

__global__ void __launch_bounds__(256)
silu_mul_kernel(const f16* __restrict__ gate_up, f16* __restrict__ out, int rows, int inter) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (int64_t)rows * inter) return;
    const int64_t r = i / inter, c = i - r * inter;
    out[i] = silu_mul_one(gate_up[r * 2 * inter + c], gate_up[r * 2 * inter + inter + c]);
}

// The same on 16-byte units (inter a multiple of 8, buffers 16-byte aligned):
// thread i takes elements 8 i .. 8 i + 7 of the output.
__global__ void __launch_bounds__(256)
silu_mul_vec_kernel(const f16* __restrict__ gate_up, f16* __restrict__ out, int rows, int inter) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int units = inter >> 3;
    if (i >= (int64_t)rows * units) return;
    const int64_t r = i / units, c = (i - r * units) * 8;
    const u32x4 gv = *reinterpret_cast<const u32x4*>(gate_up + r * 2 * inter + c);
    const u32x4 uv = *reinterpret_cast<const u32x4*>(gate_up + r * 2 * inter + inter + c);
    u32x4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const f16x2 g = as_f16x2(gv[e]), u = as_f16x2(uv[e]);
        const f16x2 y = {silu_mul_one(g.x, u.x), silu_mul_one(g.y, u.y)};
        o[e] = as_u32(y);
    }
    *reinterpret_cast<u32x4*>(out + r * inter + c) = o;
}

// Prefill attention of T new tokens at cache slots start .. start + T - 1, in
// two launches (one for short prompts, below). prefill_rope_append_kernel:
// the rotary embedding of the new k rows (fp32, rounded to fp16) and the v
// rows, written to the caches, one thread per (token, kv head, dim). prefill_attention_kernel: workgroup (hq,
// b) of 4 wavefronts takes query head hq and the 4 queries t = 4 b .. 4 b +
// 3, one per wavefront (num_heads * ceil(T / 4) workgroups); it stages the k
// and v rows of the slots its last query sees from the caches (16-byte
// loads) and the rotary q of its queries, and computes softmax(q k^T / 8) v
// in fp32 with an online softmax over 64-slot chunks; query t sees slots 0 ..
// start + t. qkv rows (stride (num_heads + 2 num_kv) * 64) hold [q | k | v]
// as the decode step's; output [T, num_heads * 64] fp16. LDS: q [4][64]
// fp32, k and v [slots][kRow] fp16 (rows padded to 72 halves, so a wavefront
// reading 64 rows spreads over the banks). The rotary k is computed once per
// (token, kv head), not once per workgroup that sees it. Up to
// kPrefillOneLaunch tokens the attention launch does the append itself
// (FUSED): each workgroup computes the rotary k of the new slots it sees, and
// the workgroups of the group's first query head write their own 4 tokens'
// rows to the caches; at those lengths the recomputation costs less than a
// second launch.
constexpr int kPrefillRow = 72;
constexpr int kPrefillOneLaunch = 16;
constexpr int kPrefillMaxSlots = 256;   // start + tokens: 73 KiB of LDS at 256 slots
constexpr int kPrefillBlock = 256;      // slots per streamed block past kPrefillMaxSlots
constexpr int kPrefillThreads = 512;    // matrix-core prefill attention: 8 wavefronts per workgroup
constexpr int kPrefillMergeBytes = 4 * 18 * 64 * 4;   // its merge of the two wavefronts per column block
constexpr int kPrefillQueries = 4;      // queries per workgroup, one per wavefront

__global__ void __launch_bounds__(256)
prefill_rope_append_kernel(const f16* __restrict__ qkv, f16* __restrict__ k_cache, f16* __restrict__ v_cache,
                           const float* __restrict__ cos_table, const float* __restrict__ sin_table, int start,
                           int T, int num_heads, int num_kv, int S) {
    constexpr int D = 64;
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (int64_t)T * num_kv * D) return;
    const int d = (int)(i % D);
    const int hk = (int)((i / D) % num_kv);
    const int t = (int)(i / ((int64_t)D * num_kv));
    const int slot = start + t;
    const f16* row = qkv + (size_t)t * (num_heads + 2 * num_kv) * D;
    const f16* k = row + (size_t)num_heads * D + (size_t)hk * D;
    const f16* v = row + (size_t)(num_heads + num_kv) * D + (size_t)hk * D;
    const float c = cos_table[(size_t)slot * (D / 2) + (d & 31)];
    const float sn = sin_table[(size_t)slot * (D / 2) + (d & 31)];
    const float k1 = (float)k[d & 31], k2 = (float)k[(d & 31) + 32];
    k_cache[((size_t)hk * S + slot) * D + d] = (f16)(d < 32 ? k1 * c - k2 * sn : k2 * c + k1 * sn);
    v_cache[((size_t)hk * S + slot) * D + d] = v[d];
}

template <bool FUSED>
__global__ void __launch_bounds__(256)
prefill_attention_kernel(const f16* __restrict__ qkv, f16* __restrict__ k_cache, f16* __restrict__ v_cache,
                         const float* __restrict__ cos_table, const float* __restrict__ sin_table, int start, int T,
                         f16* __restrict__ out, int num_heads, int num_kv, int S) {
    constexpr int D = 64;
    constexpr int QB = kPrefillQueries;
    extern __shared__ __align__(16) uint8_t smem[];
    const int t0 = blockIdx.y * QB;
    const int tq = min(QB, T - t0);          // queries of this workgroup
    const int NK = start + t0 + tq;          // slots its last query sees
    float* qs = reinterpret_cast<float*>(smem);                            // [QB][64]
    f16* ks = reinterpret_cast<f16*>(smem + (size_t)QB * D * 4);         // [NK][kPrefillRow]
    f16* vs = ks + (size_t)NK * kPrefillRow;                               // [NK][kPrefillRow]
    __shared__ __align__(16) float probs[4][64];
    const int hq = blockIdx.x;
    const int group = num_heads / num_kv;
    const int hk = hq / group;
    const int row_stride = (num_heads + 2 * num_kv) * D;

    // the visible slots' k and v rows from the caches (16 bytes per thread
    // and step): all of them, or (FUSED) those below start
    const int cached = FUSED ? start : NK;
    for (int i = threadIdx.x; i < cached * 8; i += 256) {
        const int srow = i >> 3, c = i & 7;
        const size_t g = ((size_t)hk * S + srow) * D;
        reinterpret_cast<u32x4*>(ks + srow * kPrefillRow)[c] = reinterpret_cast<const u32x4*>(k_cache + g)[c];
        reinterpret_cast<u32x4*>(vs + srow * kPrefillRow)[c] = reinterpret_cast<const u32x4*>(v_cache + g)[c];
    }
    if (FUSED) {
        // the new slots it sees: rotary k and v; the group's first query head
        // appends the rows of its own tokens t0 .. t0 + tq - 1
        const bool writer = hq % group == 0;
        for (int i = threadIdx.x; i < (t0 + tq) * D; i += 256) {
            const int t = i / D, d = i - t * D;
            const int slot = start + t;
            const f16* row = qkv + (size_t)t * row_stride;
            const float c = cos_table[(size_t)slot * (D / 2) + (d & 31)];
            const float sn = sin_table[(size_t)slot * (D / 2) + (d & 31)];
            const f16* k = row + (size_t)num_heads * D + (size_t)hk * D;
            const f16* v = row + (size_t)(num_heads + num_kv) * D + (size_t)hk * D;
            const float k1 = (float)k[d & 31], k2 = (float)k[(d & 31) + 32];
            const f16 kr = (f16)(d < 32 ? k1 * c - k2 * sn : k2 * c + k1 * sn);
            const f16 vv = v[d];
            ks[slot * kPrefillRow + d] = kr;
            vs[slot * kPrefillRow + d] = vv;
            if (writer && t >= t0) {
                k_cache[((size_t)hk * S + slot) * D + d] = kr;
                v_cache[((size_t)hk * S + slot) * D + d] = vv;
            }
        }
    }
    // rotary q of this workgroup's queries
    for (int i = threadIdx.x; i < tq * D; i += 256) {
        const int tl = i / D, d = i - tl * D;
        const int slot = start + t0 + tl;
        const f16* q = qkv + (size_t)(t0 + tl) * row_stride + (size_t)hq * D;
        const float c = cos_table[(size_t)slot * (D / 2) + (d & 31)];
        const float sn = sin_table[(size_t)slot * (D / 2) + (d & 31)];
        const float q1 = (float)q[d & 31], q2 = (float)q[(d & 31) + 32];
        qs[tl * D + d] = (float)(f16)(d < 32 ? q1 * c - q2 * sn : q2 * c + q1 * sn);
    }
    __syncthreads();

    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    float* my_probs = probs[wave];
    if (wave < tq) {
        const int t = t0 + wave;
        const int last = start + t;   // highest visible slot
        const float* qrow = qs + wave * D;
        float run_max = -__builtin_inff(), run_sum = 0.0f, acc = 0.0f;
        for (int c0 = 0; c0 <= last; c0 += 64) {
            const int slot = c0 + lane;
            float dot = 0.0f;
            if (slot <= last) {
                const u32x4* krow = reinterpret_cast<const u32x4*>(ks + slot * kPrefillRow);
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const u32x4 kk = krow[e];
#pragma unroll
                    for (int w2 = 0; w2 < 4; ++w2) {
                        const f16x2 h = as_f16x2(kk[w2]);
                        dot = __builtin_fmaf(qrow[e * 8 + 2 * w2], (float)h.x, dot);
                        dot = __builtin_fmaf(qrow[e * 8 + 2 * w2 + 1], (float)h.y, dot);
                    }
                }
            }
            const float score = slot <= last ? dot * 0.125f : -__builtin_inff();
            const float new_max = fmaxf(run_max, wave_max(score));
            const float pr = slot <= last ? __expf(score - new_max) : 0.0f;
            const float psum = wave_sum(pr);
            const float rescale = __expf(run_max - new_max);   // 0 on the first chunk
            my_probs[lane] = pr;
            wave_lds_sync();
            float part = 0.0f;
            const int n = min(64, last + 1 - c0);
            for (int r = 0; r < n; ++r) part = __builtin_fmaf(my_probs[r], (float)vs[(c0 + r) * kPrefillRow + lane], part);
            wave_lds_sync();
            acc = acc * rescale + part;
            run_sum = run_sum * rescale + psum;
            run_max = new_max;
        }
        out[(size_t)t * num_heads * D + (size_t)hq * D + lane] = (f16)(acc / run_sum);
    }
}


// Prefill attention on the matrix cores, for any prompt length, when the
// query heads per KV head, group, are a power of two up to 64 and qkv and the
// rotary tables are 16-byte aligned. The launcher runs the FUSED form: slots
// below start come from the caches, the new tokens' rotary k and v rows are
// computed from qkv by every workgroup that sees them and appended to the
// caches by the workgroup that owns the token (FUSED = false reads every slot
// from the caches, for callers that appended them beforehand).
// Workgroup (hk, y) of 8 wavefronts takes KV head hk and the 64 / group tokens
// t = b 64 / group .., b = gridDim.y - 1 - y (the workgroups with the most
// slots to attend dispatched first), of all its group query heads: 64 query
// columns, column c = token offset * group + head offset, wavefronts w and
// w + 4 owning columns 16 w .. 16 w + 15. It stages the k and v rows of every
// slot its last token sees once (shared by the 64 columns, where the one-query
// kernel above restages them per head and per 4 queries); wavefront w walks
// the even chunks of 32 slots and w + 4 the odd ones, each with an online
// softmax, and w merges the two states at the end:
//   S^T = K Q^T (v_mfma_f32_16x16x32_f16; A = k rows from LDS, lane (q4, j)
//     holds slot 16 mt + j, dims 32 s + 8 q4 .. +8; B = the rotary q of column
//     j, rounded to fp16), so lane (q4, j) receives column j's scores for
//     slots c0 + 16 mt + 4 q4 + e, scaled by 1/8 and masked past the column's
//     last slot (start + its token);
//   the column's running maximum and sum across the four lanes that hold it
//     by v_permlane16_swap / v_permlane32_swap;
//   O^T += V^T P^T with P^T (fp16) straight from the score registers and V^T
//     from the row-major LDS tile through ds_read_b64_tr_b16 (the lane mapping
//     of attn_o_kernel), the accumulator rescaled by exp(old max - new max).
// fp32 scores, softmax and accumulation; the probabilities enter the MFMA as
// fp16. LDS: k and v [NK rounded up to 32][kPrefillRow] fp16, rows past NK
// zero.
// ---------------------------------------------------------------------------
template <bool FUSED>
__global__ void __launch_bounds__(kPrefillThreads)
prefill_attention_mfma_kernel(const f16* __restrict__ qkv, f16* __restrict__ k_cache,
                              f16* __restrict__ v_cache, const float* __restrict__ cos_table,
                              const float* __restrict__ sin_table, int start, int T, f16* __restrict__ out,
                              int num_heads, int num_kv, int S, int glog) {
    constexpr int D = 64;
    constexpr int KR = kPrefillRow;
    constexpr int NT = kPrefillThreads;
    extern __shared__ __align__(16) uint8_t smem[];
    const int group = 1 << glog;
    const int tpw = 64 >> glog;   // tokens per workgroup
    const int hk = blockIdx.x;
    // the last tokens (most slots to attend) in the first workgroups dispatched
    const int t0 = (gridDim.y - 1 - blockIdx.y) * tpw;
    const int NK = start + min(t0 + tpw, T);   // slots the workgroup's last token sees
    const int NKP = (NK + 31) & ~31;
    // LDS rows: every slot the workgroup sees (FUSED), or one block of up to
    // kPrefillBlock slots at a time, streamed from the caches (FUSED = false)
    const int LR = FUSED ? NKP : min(NKP, kPrefillBlock);
    f16* ks = reinterpret_cast<f16*>(smem);   // [LR][KR]
    f16* vs = ks + (size_t)LR * KR;           // [LR][KR]
    const int row_stride = (num_heads + 2 * num_kv) * D;
    // wavefronts w and w + 4 own columns 16 w .. 16 w + 15: w the even
    // 32-slot chunks, w + 4 the odd ones (half = 0 / 1)
    const int wave = __builtin_amdgcn_readfirstlane((threadIdx.x >> 6) & 3);
    const int half = __builtin_amdgcn_readfirstlane(threadIdx.x >> 8);
    const int lane = threadIdx.x & 63;
    const int q4 = lane >> 4, j = lane & 15;

    // 1. this lane's query column (requested first) and the k / v rows
    const int col = 16 * wave + j;
    const int tq = t0 + (col >> glog);
    const int tqc = min(tq, T - 1);
    const int hq = hk * group + (col & (group - 1));
    const f16* qrow = qkv + (size_t)tqc * row_stride + (size_t)hq * D;
    const u32x4 qa = *reinterpret_cast<const u32x4*>(qrow + 8 * q4);
    const u32x4 qz = *reinterpret_cast<const u32x4*>(qrow + 32 + 8 * q4);
    float cs[8], sn[8];
    {
        const size_t ti = (size_t)(start + tqc) * (D / 2) + 8 * q4;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            cs[i] = cos_table[ti + i];
            sn[i] = sin_table[ti + i];
        }
    }
    // cache rows r0 .. r0 + n - 1 into LDS rows 0 .. n - 1, rows n .. np - 1
    // zero (16-byte units; loads clamped into the rows being copied)
    const u32x4* kc = reinterpret_cast<const u32x4*>(k_cache + (size_t)hk * S * D);
    const u32x4* vc = reinterpret_cast<const u32x4*>(v_cache + (size_t)hk * S * D);
    auto stage_rows = [&](int r0, int n, int np) {
        const int units = n * 8, punits = np * 8;
        for (int i0 = threadIdx.x; i0 < punits; i0 += 8 * NT) {
            u32x4 kb[8], vb[8];
#pragma unroll
            for (int b = 0; b < 8; ++b) {
                const int i = r0 * 8 + max(min(i0 + NT * b, units - 1), 0);
                kb[b] = kc[i];
                vb[b] = vc[i];
            }
#pragma unroll
            for (int b = 0; b < 8; ++b) {
                const int i = i0 + NT * b;
                if (i < punits) {
                    const bool live = i < units;
                    const int r = i >> 3, e = i & 7;
                    reinterpret_cast<u32x4*>(ks + (size_t)r * KR)[e] = live ? kb[b] : (u32x4){0u, 0u, 0u, 0u};
                    reinterpret_cast<u32x4*>(vs + (size_t)r * KR)[e] = live ? vb[b] : (u32x4){0u, 0u, 0u, 0u};
                }
            }
        }
    };
    if constexpr (FUSED) {
        stage_rows(0, start, start);   // the slots below start
        // the new rows this workgroup sees (tokens 0 .. nn - 1) from qkv: v
        // as is, k rotated at its slot (fp32, rounded to fp16, as
        // prefill_rope_append_kernel); the workgroup's own tokens t0 .. nn - 1
        // are appended to the caches; rows NK .. NKP - 1 zero
        const int nn = NK - start;
        const f16* kq = qkv + (size_t)num_heads * D + (size_t)hk * D;
        const f16* vq = qkv + (size_t)(num_heads + num_kv) * D + (size_t)hk * D;
        for (int i0 = threadIdx.x; i0 < nn * 8; i0 += 4 * NT) {
            u32x4 vb[4];
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                const int i = min(i0 + NT * b, nn * 8 - 1);
                vb[b] = *reinterpret_cast<const u32x4*>(vq + (size_t)(i >> 3) * row_stride + 8 * (i & 7));
            }
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                const int i = i0 + NT * b;
                if (i < nn * 8) {
                    const int r = i >> 3, e = i & 7;
                    reinterpret_cast<u32x4*>(vs + (size_t)(start + r) * KR)[e] = vb[b];
                    if (r >= t0)
                        reinterpret_cast<u32x4*>(v_cache + ((size_t)hk * S + start + r) * D)[e] = vb[b];
                }
            }
        }
        for (int i0 = threadIdx.x; i0 < nn * 4; i0 += 2 * NT) {
            u32x4 ka[2], kz[2];
            f32x4 cv[2][2], sv[2][2];
#pragma unroll
            for (int b = 0; b < 2; ++b) {
                const int i = min(i0 + NT * b, nn * 4 - 1);
                const int r = i >> 2, db = i & 3;
                const f16* kr = kq + (size_t)r * row_stride + 8 * db;
                ka[b] = *reinterpret_cast<const u32x4*>(kr);
                kz[b] = *reinterpret_cast<const u32x4*>(kr + 32);
                const size_t ti = (size_t)(start + r) * (D / 2) + 8 * db;
                cv[b][0] = *reinterpret_cast<const f32x4*>(cos_table + ti);
                cv[b][1] = *reinterpret_cast<const f32x4*>(cos_table + ti + 4);
                sv[b][0] = *reinterpret_cast<const f32x4*>(sin_table + ti);
                sv[b][1] = *reinterpret_cast<const f32x4*>(sin_table + ti + 4);
            }
#pragma unroll
            for (int b = 0; b < 2; ++b) {
                const int i = i0 + NT * b;
                if (i < nn * 4) {
                    const int r = i >> 2, db = i & 3;
                    float c8[8], s8[8];
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        c8[e] = cv[b][e >> 2][e & 3];
                        s8[e] = sv[b][e >> 2][e & 3];
                    }
                    u32x4 lo, hi;
                    rope8(ka[b], kz[b], c8, s8, 1.0f, lo, hi);
                    f16* krow = ks + (size_t)(start + r) * KR;
                    reinterpret_cast<u32x4*>(krow)[db] = lo;
                    reinterpret_cast<u32x4*>(krow)[4 + db] = hi;
                    if (r >= t0) {
                        u32x4* dst = reinterpret_cast<u32x4*>(k_cache + ((size_t)hk * S + start + r) * D);
                        dst[db] = lo;
                        dst[4 + db] = hi;
                    }
                }
            }
        }
        for (int i = threadIdx.x; i < (NKP - NK) * 8; i += NT) {
            const int r = NK + (i >> 3), e = i & 7;
            reinterpret_cast<u32x4*>(ks + (size_t)r * KR)[e] = (u32x4){0u, 0u, 0u, 0u};
            reinterpret_cast<u32x4*>(vs + (size_t)r * KR)[e] = (u32x4){0u, 0u, 0u, 0u};
        }
    }
    // the rotary q (B operand): dims 8 q4 + i (s = 0) pair with 32 + 8 q4 + i
    // (s = 1), times the score scale 1/8 (a power of two: the fp16 rounding of
    // the scaled value is the scaled rounding)
    u32x4 qb[2];
    rope8(qa, qz, cs, sn, 0.125f, qb[0], qb[1]);
    __syncthreads();
    // a wavefront none of whose columns is a token only stages and takes part
    // in the barriers
    const bool active = t0 + ((16 * wave) >> glog) < T;

    // 2. chunks of 32 slots up to the wavefront's last visible slot
    const int last = start + tqc;
    const int lastw = active ? start + min(t0 + ((16 * wave + 15) >> glog), T - 1) : -1;
    const int tk = j >> 2, tm = j & 3;   // this lane's row / 4-dim block in the transposing read
    float run_max = -__builtin_inff(), run_sum = 0.0f;
    f32x4 o[4];
#pragma unroll
    for (int md = 0; md < 4; ++md) o[md] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
    // the smallest last slot among the wavefront's columns: chunks wholly at or
    // below it need no mask
    const int firstlast = start + min(t0 + ((16 * wave) >> glog), T - 1);
    constexpr float kLog2e = 1.4426950408889634f;
    // one chunk: LDS rows c0 .. c0 + 31 holding slots base .. base + 31
    auto chunk = [&](int c0, int base, auto masked) {
        constexpr bool MASK = decltype(masked)::value;
        f32x4 st[2];
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
            st[mt] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
            const f16* krow = ks + (size_t)(c0 + 16 * mt + j) * KR + 8 * q4;
#pragma unroll
            for (int s2 = 0; s2 < 2; ++s2)
                st[mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                    __builtin_bit_cast(f16x8, *reinterpret_cast<const u32x4*>(krow + 32 * s2)),
                    __builtin_bit_cast(f16x8, qb[s2]), st[mt], 0, 0, 0);
        }
        float mx = run_max;
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                if constexpr (MASK) {
                    const int slot = base + 16 * mt + 4 * q4 + e;
                    st[mt][e] = slot <= last ? st[mt][e] : -__builtin_inff();
                }
                mx = fmaxf(mx, st[mt][e]);
            }
        mx = row_pair_max(mx);
        // -inf while no slot of the column has been seen (odd chunks only);
        // exp(x - m) as 2^(x log2 e - m log2 e), masked scores giving 2^-inf = 0
        const float mbl = (mx == -__builtin_inff() ? 0.0f : mx) * kLog2e;
        const float rescale = __builtin_amdgcn_exp2f(run_max * kLog2e - mbl);   // 0 on the column's first chunk
        float psum = 0.0f;
        float pe[2][4];
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                pe[mt][e] = __builtin_amdgcn_exp2f(__builtin_fmaf(st[mt][e], kLog2e, -mbl));
                psum += pe[mt][e];
            }
        const f16x2 p00 = {(f16)pe[0][0], (f16)pe[0][1]}, p01 = {(f16)pe[0][2], (f16)pe[0][3]};
        const f16x2 p10 = {(f16)pe[1][0], (f16)pe[1][1]}, p11 = {(f16)pe[1][2], (f16)pe[1][3]};
        const u32x4 pb = {as_u32(p00), as_u32(p01), as_u32(p10), as_u32(p11)};
        psum = row_pair_sum(psum);
        run_sum = run_sum * rescale + psum;
        run_max = mx;
#pragma unroll
        for (int md = 0; md < 4; ++md) {
            const f16* src = vs + (size_t)(c0 + 4 * q4 + tk) * KR + 16 * md + 4 * tm;
            const uint2 lo = lds_read_tr16(src);
            const uint2 hi = lds_read_tr16(src + 16 * KR);
            const u32x4 a = {lo.x, lo.y, hi.x, hi.y};
            o[md] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, pb),
                                                           o[md] * rescale, 0, 0, 0);
        }
    };
    // LDS rows 0 .. rows - 1 hold slots b0 .. b0 + rows - 1
    auto attend = [&](int b0, int rows) {
        for (int c0 = 32 * half; c0 < rows && b0 + c0 <= lastw; c0 += 64) {
            if (b0 + c0 + 31 <= firstlast)
                chunk(c0, b0 + c0, std::false_type{});
            else
                chunk(c0, b0 + c0, std::true_type{});
        }
    };
    if constexpr (FUSED) {
        attend(0, NKP);
    } else {
        // blocks of kPrefillBlock slots: every wavefront stages, the active
        // ones attend; the softmax state carries over from block to block
        for (int b0 = 0; b0 < NK; b0 += kPrefillBlock) {
            const int nb = min(kPrefillBlock, NK - b0), nbp = (nb + 31) & ~31;
            if (b0 > 0) __syncthreads();   // every wavefront done with the previous block
            stage_rows(b0, nb, nbp);
            __syncthreads();
            attend(b0, nbp);
        }
    }

    // 3. the odd-chunk wavefront's state merged into the even one's through
    // LDS (the k / v rows are no longer read): [wave][18 values][64 lanes];
    // with one chunk of slots (NKP = 32, the same for the whole workgroup)
    // the odd-chunk wavefronts attended nothing and there is nothing to merge
    if (NKP == 32) {
        if (half == 1 || !active || tq >= T) return;
    } else {
        __syncthreads();
        float* xs = reinterpret_cast<float*>(smem) + (size_t)wave * 18 * 64 + lane;
        if (half == 1) {
            xs[0] = run_max;
            xs[64] = run_sum;
#pragma unroll
            for (int md = 0; md < 4; ++md)
#pragma unroll
                for (int e = 0; e < 4; ++e) xs[(2 + 4 * md + e) * 64] = o[md][e];
        }
        __syncthreads();
        if (half == 1 || !active || tq >= T) return;
        // run_max is finite here: the even chunks start at slot 0
        const float m1 = xs[0];
        const float m = fmaxf(run_max, m1);
        const float a0 = __builtin_amdgcn_exp2f((run_max - m) * kLog2e), a1 = __builtin_amdgcn_exp2f((m1 - m) * kLog2e);
        run_sum = run_sum * a0 + xs[64] * a1;
#pragma unroll
        for (int md = 0; md < 4; ++md)
#pragma unroll
            for (int e = 0; e < 4; ++e) o[md][e] = o[md][e] * a0 + xs[(2 + 4 * md + e) * 64] * a1;
    }

    // 4. lane (q4, j) holds column j's dims 16 md + 4 q4 .. + 3
    const float inv = 1.0f / run_sum;
    f16* orow = out + (size_t)tq * num_heads * D + (size_t)hq * D;
    const bool vec = (reinterpret_cast<uintptr_t>(out) & 7u) == 0;
#pragma unroll
    for (int md = 0; md < 4; ++md) {
        const f16x2 a = {(f16)(o[md][0] * inv), (f16)(o[md][1] * inv)};
        const f16x2 b = {(f16)(o[md][2] * inv), (f16)(o[md][3] * inv)};
        f16* dst = orow + 16 * md + 4 * q4;
        if (vec) {
            *reinterpret_cast<uint2*>(dst) = make_uint2(as_u32(a), as_u32(b));
        } else {
            dst[0] = a.x;
            dst[1] = a.y;
            dst[2] = b.x;
            dst[3] = b.y;
        }
    }
}

// The K slices of a split-K linear layer, added and rounded, then the
// residual add + RMSNorm of norm_rows_vec_kernel<true>, one workgroup per
// row of at most 2048 elements (one 8-element unit per thread): d =
// fp16(part[0] + part[1] + .. + part[S - 1]) in slice order in fp32 (the
// arithmetic of pair_split_reduce), s = fp16(fp32(x) + fp32(d)) to x_out, and
// out = fp16((fp32(s) * inv) * fp32(w)) with inv = 1 / sqrt(mean(s^2) + eps),
// the squares summed per thread, per wavefront by DPP and over the four
// wavefronts as (0 + 1) + (2 + 3) (those of norm_rows_vec_kernel): the
// outputs equal the reduce launch followed by that kernel, bit for bit.
template <int S>
__global__ void __launch_bounds__(256)
split_add_rmsnorm_kernel(const float* __restrict__ part, const f16* x, const f16* __restrict__ w, float eps,
                         f16* x_out, f16* __restrict__ out, int rows, int hidden) {
    __shared__ float partial[4];
    const size_t row = (size_t)blockIdx.x * hidden;
    const size_t mn = (size_t)rows * hidden;
    const int units = hidden >> 3;
    const int i = min((int)threadIdx.x, units - 1);
    const u32x4 xv = *reinterpret_cast<const u32x4*>(x + row + (size_t)i * 8);
    const u32x4 wv = *reinterpret_cast<const u32x4*>(w + (size_t)i * 8);
    f32x4 pv[S][2];
#pragma unroll
    for (int sl = 0; sl < S; ++sl)
#pragma unroll
        for (int h = 0; h < 2; ++h)
            pv[sl][h] = *reinterpret_cast<const f32x4*>(part + sl * mn + row + (size_t)i * 8 + 4 * h);
    u32x4 sv;
    float ss = 0.0f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        float d[2];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            float acc = pv[0][e >> 1][2 * (e & 1) + j];
#pragma unroll
            for (int sl = 1; sl < S; ++sl) acc += pv[sl][e >> 1][2 * (e & 1) + j];
            d[j] = (float)(f16)acc;
        }
        const f16x2 a = as_f16x2(xv[e]);
        const f16x2 sum = {(f16)((float)a.x + d[0]), (f16)((float)a.y + d[1])};
        sv[e] = as_u32(sum);
    }
    if ((int)threadIdx.x < units) {
        store_through(reinterpret_cast<u32x4*>(x_out + row + (size_t)threadIdx.x * 8), sv);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const f16x2 a = as_f16x2(sv[e]);
            ss = __builtin_fmaf((float)a.x, (float)a.x, ss);
            ss = __builtin_fmaf((float)a.y, (float)a.y, ss);
        }
    }
    ss = wave_sum(ss);
    if ((threadIdx.x & 63) == 0) partial[threadIdx.x >> 6] = ss;
    __syncthreads();
    const float total = (partial[0] + partial[1]) + (partial[2] + partial[3]);
    const float inv = 1.0f / __builtin_sqrtf(total / (float)hidden + eps);
    if ((int)threadIdx.x < units) {
        u32x4 o;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const f16x2 a = as_f16x2(sv[e]), g = as_f16x2(wv[e]);
            const f16x2 y = {(f16)(((float)a.x * inv) * (float)g.x), (f16)(((float)a.y * inv) * (float)g.y)};
            o[e] = as_u32(y);
        }
        store_through(reinterpret_cast<u32x4*>(out + row + (size_t)threadIdx.x * 8), o);
    }
}

}  // namespace w4a16

namespace w4a16_internal {
void set_last_error(const std::string& message);   // w4a16_hip.hip: the message w4a16_last_error() returns

using SplitNormKern = void (*)(const float*, const w4a16::f16*, const w4a16::f16*, float, w4a16::f16*, w4a16::f16*,
                               int, int);
template <int... S>
SplitNormKern split_norm_table(int slices, std::integer_sequence<int, S...>) {
    static constexpr SplitNormKern table[] = {w4a16::split_add_rmsnorm_kernel<S + 2>...};
    return table[slices - 2];
}

// split_add_rmsnorm_kernel over `rows` rows of `hidden` (8 | hidden <= 2048,
// every buffer 16-byte aligned; the caller checks), slices 2..16.
int launch_split_add_rmsnorm(int slices, const float* part, const w4a16::f16* x, const w4a16::f16* w, float eps,
                             w4a16::f16* x_out, w4a16::f16* out, int rows, int hidden, hipStream_t stream) {
    if (slices < 2 || slices > 16 || hidden <= 0 || hidden > 2048 || hidden % 8 != 0) {
        set_last_error("split-K reduce + RMSNorm: 2..16 slices, rows of 8..2048 elements (a multiple of 8)");
        return W4A16_ERR_CONFIG;
    }
    hipLaunchKernelGGL(split_norm_table(slices, std::make_integer_sequence<int, 15>{}), dim3((unsigned)rows),
                       dim3(256), 0, stream, part, x, w, eps, x_out, out, rows, hidden);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_last_error(std::string("kernel launch failed: ") + hipGetErrorString(e));
        return W4A16_ERR_LAUNCH;
    }
    return W4A16_OK;
}
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

namespace {

// Shape checks and launch shared by the two attention + o entry points.
template <bool CACHED>
int launch_attention_o(const void* qkv, void* k_cache, void* v_cache, const float* inv_freq, const int64_t* position,
                       const uint8_t* o_packed, const void* o_scales, void* residual, int64_t num_heads,
                       int64_t num_kv_heads, int64_t head_dim, int64_t max_seq_len, int64_t hidden,
                       int64_t group_size, void* stream) {
    using namespace w4a16;
    if (!qkv || !k_cache || !v_cache || (!CACHED && !inv_freq) || !position || !o_packed || !o_scales || !residual)
        return fail(W4A16_ERR_NULL, "attention_o: every pointer must be non-NULL");
    if (head_dim != 64) return fail(W4A16_ERR_CONFIG, "attention_o: head_dim must be 64");
    if (group_size != 128) return fail(W4A16_ERR_CONFIG, "attention_o: group_size must be 128");
    if (num_kv_heads != 1 && num_kv_heads != 2 && num_kv_heads != 4 && num_kv_heads != 8)
        return fail(W4A16_ERR_CONFIG, "attention_o: num_kv_heads must be 1, 2, 4 or 8");
    if (num_heads <= 0 || num_heads % num_kv_heads != 0 || num_heads / num_kv_heads > 16 || num_heads * 64 > 4096)
        return fail(W4A16_ERR_SHAPE,
                    "attention_o: num_heads must be a multiple of num_kv_heads, at most 16 per KV head and 64 in all");
    if (max_seq_len <= 0 || max_seq_len > 16384)
        return fail(W4A16_ERR_SHAPE, "attention_o: max_seq_len must be in 1..16384");
    if (hidden <= 0 || hidden > INT32_MAX / 2) return fail(W4A16_ERR_SHAPE, "attention_o: hidden must be positive");
    if (!aligned(qkv, 16) || !aligned(k_cache, 16) || !aligned(v_cache, 16) || !aligned(o_packed, 16) ||
        !aligned(o_scales, 2) || !aligned(residual, 2) || (!CACHED && !aligned(inv_freq, 4)))
        return fail(W4A16_ERR_ALIGNMENT, "attention_o: qkv, caches and o_packed must be 16-byte aligned");
    const int KV = (int)num_kv_heads, group = (int)(num_heads / num_kv_heads);
    const int K = (int)num_heads * 64;
    const int L = (K / 32 + 63) / 64;   // 1 KiB loads per o row: 1 or 2
    // the cached form: 2 KV wavefronts (V rows loaded by helper wavefronts),
    // one o row each; the rotating form: KV wavefronts of 2 o rows. Graph
    // timing, 1.1B model (KV = 4, positions 16..47): 4.92-4.94 us against
    // 5.10 for the cached form on KV wavefronts of 2 rows (decode 2775 ->
    // 2809 tok/s on one box)
    constexpr int R = CACHED ? 1 : 2;   // o rows per wavefront
    constexpr bool HV = CACHED;
    void (*kern)(const f16*, f16*, f16*, const float*, const int64_t*, const uint8_t*, const f16*, f16*, int, int,
                 int) = nullptr;
    switch (KV) {
        case 1: kern = L == 1 ? attn_o_kernel<1, R, 1, CACHED, HV> : attn_o_kernel<1, R, 2, CACHED, HV>; break;
        case 2: kern = L == 1 ? attn_o_kernel<2, R, 1, CACHED, HV> : attn_o_kernel<2, R, 2, CACHED, HV>; break;
        case 4: kern = L == 1 ? attn_o_kernel<4, R, 1, CACHED, HV> : attn_o_kernel<4, R, 2, CACHED, HV>; break;
        default: kern = L == 1 ? attn_o_kernel<8, R, 1, CACHED, HV> : attn_o_kernel<8, R, 2, CACHED, HV>; break;
    }
    const int nw = HV ? 2 * KV : KV, rpw = R;
    const int lds = KV * kAttnOSlots * kVStride * 2 + K * 2 + KV * 64 * 4;
    if (lds > 64 * 1024) {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, lds);
        if (e != hipSuccess) return fail(W4A16_ERR_LAUNCH, "attention_o: LDS request refused");
    }
    const int rows_per_block = rpw * nw;
    const int blocks = (int)((hidden + rows_per_block - 1) / rows_per_block);
    hipLaunchKernelGGL(kern, dim3(blocks), dim3(64 * nw), lds, static_cast<hipStream_t>(stream),
                       static_cast<const f16*>(qkv), static_cast<f16*>(k_cache), static_cast<f16*>(v_cache), inv_freq,
                       position, o_packed, static_cast<const f16*>(o_scales), static_cast<f16*>(residual), group,
                       (int)max_seq_len, (int)hidden);
    return check_launch();
}

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
    // wavefronts per head: one chunk of 64 slots each at a time; short caches
    // keep one wavefront (a second would only re-read the same chunk)
    const int WA = max_seq_len <= 64 ? 1 : max_seq_len <= 256 ? 4 : 8;
    void (*kern)(const w4a16::f16*, w4a16::f16*, w4a16::f16*, const float*, const float*, const int64_t*,
                 w4a16::f16*, int, int, int, float*) = WA == 1   ? w4a16::decode_attention<1, false>
                                                       : WA == 4 ? w4a16::decode_attention<4, false>
                                                                 : w4a16::decode_attention<8, false>;
    hipLaunchKernelGGL(kern, dim3((unsigned)num_heads), dim3(64 * WA), 0, static_cast<hipStream_t>(stream),
                       static_cast<const w4a16::f16*>(qkv), static_cast<w4a16::f16*>(k_cache),
                       static_cast<w4a16::f16*>(v_cache), cos_table, sin_table, position,
                       static_cast<w4a16::f16*>(output), (int)num_heads, (int)num_kv_heads, (int)max_seq_len,
                       nullptr);
    return check_launch();
}

int w4a16_decode_attention_split_f16(const void* qkv, void* k_cache, void* v_cache, const float* cos_table,
                                     const float* sin_table, const int64_t* position, void* output,
                                     int64_t num_heads, int64_t num_kv_heads, int64_t head_dim,
                                     int64_t max_seq_len, int64_t splits, void* workspace,
                                     int64_t workspace_bytes, void* stream) {
    if (!qkv || !k_cache || !v_cache || !cos_table || !sin_table || !position || !output || !workspace)
        return fail(W4A16_ERR_NULL, "split attention: every pointer must be non-NULL");
    if (head_dim != 64) return fail(W4A16_ERR_CONFIG, "split attention: head_dim must be 64");
    if (num_heads <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads != 0 || num_heads > 65535)
        return fail(W4A16_ERR_SHAPE, "split attention: num_heads must be a positive multiple of num_kv_heads");
    if (max_seq_len <= 0 || max_seq_len > 16384)
        return fail(W4A16_ERR_SHAPE, "split attention: max_seq_len must be in 1..16384");
    if (splits < 1 || splits > 64) return fail(W4A16_ERR_CONFIG, "split attention: splits must be in 1..64");
    if (workspace_bytes < num_heads * splits * 66 * 4)
        return fail(W4A16_ERR_TOO_LARGE, "split attention: workspace below num_heads * splits * 264 bytes");
    if (!aligned(k_cache, 16) || !aligned(v_cache, 16) || !aligned(qkv, 2) || !aligned(output, 2) ||
        !aligned(workspace, 4))
        return fail(W4A16_ERR_ALIGNMENT,
                    "split attention: caches 16-byte aligned, fp16 buffers 2-byte, workspace 4-byte aligned");
    hipStream_t st = static_cast<hipStream_t>(stream);
    const auto skern = w4a16::decode_attention<4, true>;
    hipLaunchKernelGGL(skern, dim3((unsigned)num_heads, (unsigned)splits), dim3(256), 0,
                       st, static_cast<const w4a16::f16*>(qkv), static_cast<w4a16::f16*>(k_cache),
                       static_cast<w4a16::f16*>(v_cache), cos_table, sin_table, position,
                       static_cast<w4a16::f16*>(output), (int)num_heads, (int)num_kv_heads, (int)max_seq_len,
                       static_cast<float*>(workspace));
    const int rc = check_launch();
    if (rc != W4A16_OK) return rc;
    hipLaunchKernelGGL(w4a16::decode_attention_merge, dim3((unsigned)num_heads), dim3(64), 0, st,
                       static_cast<const float*>(workspace), position, static_cast<w4a16::f16*>(output), (int)splits,
                       (int)max_seq_len);
    return check_launch();
}

int w4a16_attention_o_f16(const void* qkv, void* k_cache, void* v_cache, const float* inv_freq,
                          const int64_t* position, const uint8_t* o_packed, const void* o_scales, void* residual,
                          int64_t num_heads, int64_t num_kv_heads, int64_t head_dim, int64_t max_seq_len,
                          int64_t hidden, int64_t group_size, void* stream) {
    return launch_attention_o<false>(qkv, k_cache, v_cache, inv_freq, position, o_packed, o_scales, residual,
                                     num_heads, num_kv_heads, head_dim, max_seq_len, hidden, group_size, stream);
}

int w4a16_attention_o_cached_f16(const void* qkv, const void* k_cache, const void* v_cache, const int64_t* position,
                                 const uint8_t* o_packed, const void* o_scales, void* residual, int64_t num_heads,
                                 int64_t num_kv_heads, int64_t head_dim, int64_t max_seq_len, int64_t hidden,
                                 int64_t group_size, void* stream) {
    return launch_attention_o<true>(qkv, const_cast<void*>(k_cache), const_cast<void*>(v_cache), nullptr, position,
                                    o_packed, o_scales, residual, num_heads, num_kv_heads, head_dim, max_seq_len,
                                    hidden, group_size, stream);
}

int w4a16_argmax_f16(const void* logits, int64_t n, int64_t* token, int64_t* position, void* stream) {
    return w4a16_argmax_embed_f16(logits, n, token, position, nullptr, 0, 0, nullptr, nullptr, stream);
}

int w4a16_argmax_embed_f16(const void* logits, int64_t n, int64_t* token, int64_t* position, const void* table,
                           int64_t vocab, int64_t hidden, void* output, int64_t* token_copy, void* stream) {
    if (!logits || !token) return fail(W4A16_ERR_NULL, "argmax: logits and token must be non-NULL");
    if (n <= 0 || n > INT32_MAX - 1024) return fail(W4A16_ERR_SHAPE, "argmax: n must be in 1..2^31-1025");
    if ((table == nullptr) != (output == nullptr))
        return fail(W4A16_ERR_NULL, "argmax: table and output must both be given or both be NULL");
    if (table && (vocab < n || hidden <= 0 || hidden > INT32_MAX / 2))
        return fail(W4A16_ERR_SHAPE, "argmax: the embedding table needs vocab >= n and a positive hidden size");
    hipLaunchKernelGGL(w4a16::argmax_kernel, dim3(1), dim3(1024), 0, static_cast<hipStream_t>(stream),
                       static_cast<const w4a16::f16*>(logits), (int)n, token, position,
                       static_cast<const w4a16::f16*>(table), vocab, (int)hidden, static_cast<w4a16::f16*>(output),
                       token_copy);
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

int w4a16_rmsnorm_f16(const void* x, const void* weight, float eps, void* output, int64_t rows, int64_t hidden,
                      void* stream) {
    if (rows == 0) return W4A16_OK;
    if (!x || !weight || !output) return fail(W4A16_ERR_NULL, "rmsnorm: every pointer must be non-NULL");
    if (rows < 0 || rows > INT32_MAX || hidden <= 0 || hidden > INT32_MAX)
        return fail(W4A16_ERR_SHAPE, "rmsnorm: rows must be non-negative and hidden positive");
    if (!(eps >= 0.0f)) return fail(W4A16_ERR_CONFIG, "rmsnorm: eps must be non-negative");
    if (!aligned(x, 2) || !aligned(weight, 2) || !aligned(output, 2))
        return fail(W4A16_ERR_ALIGNMENT, "rmsnorm: fp16 buffers must be 2-byte aligned");
    using w4a16::f16;
    if (hidden % 8 == 0 && hidden <= w4a16::kAddNormMax && aligned(x, 16) && aligned(weight, 16) &&
        aligned(output, 16)) {
        hipLaunchKernelGGL(w4a16::norm_rows_vec_kernel<false>, dim3((unsigned)rows), dim3(256), 0,
                           static_cast<hipStream_t>(stream), static_cast<const f16*>(x), nullptr,
                           static_cast<const f16*>(weight), eps, nullptr, static_cast<f16*>(output), (int)hidden);
        return check_launch();
    }
    hipLaunchKernelGGL(w4a16::rmsnorm_rows_kernel, dim3((unsigned)rows), dim3(256), 0,
                       static_cast<hipStream_t>(stream), static_cast<const f16*>(x), static_cast<const f16*>(weight),
                       eps, static_cast<f16*>(output), (int)hidden);
    return check_launch();
}

int w4a16_embed_rmsnorm_f16(const void* table, int64_t vocab, int64_t hidden, const int64_t* tokens, int64_t rows,
                            const void* weight, float eps, void* x_out, void* output, int64_t* position,
                            void* stream) {
    if (rows == 0) return W4A16_OK;
    if (!table || !tokens || !weight || !x_out || !output)
        return fail(W4A16_ERR_NULL, "embed + rmsnorm: table, tokens, weight, x_out and output must be non-NULL");
    if (rows < 0 || rows > INT32_MAX || vocab <= 0)
        return fail(W4A16_ERR_SHAPE, "embed + rmsnorm: rows must be non-negative and vocab positive");
    if (hidden <= 0 || hidden % 8 != 0 || hidden > w4a16::kAddNormMax)
        return fail(W4A16_ERR_SHAPE, "embed + rmsnorm: hidden must be a positive multiple of 8 up to 8192");
    if (!(eps >= 0.0f)) return fail(W4A16_ERR_CONFIG, "embed + rmsnorm: eps must be non-negative");
    if (!aligned(table, 16) || !aligned(weight, 16) || !aligned(x_out, 16) || !aligned(output, 16) ||
        !aligned(tokens, 8) || (position != nullptr && !aligned(position, 8)))
        return fail(W4A16_ERR_ALIGNMENT, "embed + rmsnorm: fp16 buffers must be 16-byte aligned, tokens and "
                                         "position 8-byte aligned");
    using w4a16::f16;
    hipLaunchKernelGGL(w4a16::embed_norm_rows_kernel, dim3((unsigned)rows), dim3(256), 0,
                       static_cast<hipStream_t>(stream), static_cast<const f16*>(table), vocab, tokens,
                       static_cast<const f16*>(weight), eps, static_cast<f16*>(x_out), static_cast<f16*>(output),
                       (int)hidden, position);
    return check_launch();
}

int w4a16_add_rmsnorm_f16(const void* x, const void* delta, const void* weight, float eps, void* x_out,
                          void* output, int64_t rows, int64_t hidden, void* stream) {
    if (rows == 0) return W4A16_OK;
    if (!x || !delta || !weight || !x_out || !output)
        return fail(W4A16_ERR_NULL, "add_rmsnorm: every pointer must be non-NULL");
    if (rows < 0 || rows > INT32_MAX || hidden <= 0 || hidden > w4a16::kAddNormMax)
        return fail(W4A16_ERR_SHAPE, "add_rmsnorm: rows must be non-negative and 0 < hidden <= 8192");
    if (!(eps >= 0.0f)) return fail(W4A16_ERR_CONFIG, "add_rmsnorm: eps must be non-negative");
    if (!aligned(x, 2) || !aligned(delta, 2) || !aligned(weight, 2) || !aligned(x_out, 2) || !aligned(output, 2))
        return fail(W4A16_ERR_ALIGNMENT, "add_rmsnorm: fp16 buffers must be 2-byte aligned");
    using w4a16::f16;
    if (hidden % 8 == 0 && aligned(x, 16) && aligned(delta, 16) && aligned(weight, 16) && aligned(x_out, 16) &&
        aligned(output, 16)) {
        hipLaunchKernelGGL(w4a16::norm_rows_vec_kernel<true>, dim3((unsigned)rows), dim3(256), 0,
                           static_cast<hipStream_t>(stream), static_cast<const f16*>(x), static_cast<const f16*>(delta),
                           static_cast<const f16*>(weight), eps, static_cast<f16*>(x_out), static_cast<f16*>(output),
                           (int)hidden);
        return check_launch();
    }
    hipLaunchKernelGGL(w4a16::add_rmsnorm_rows_kernel, dim3((unsigned)rows), dim3(256), 0,
                       static_cast<hipStream_t>(stream), static_cast<const f16*>(x), static_cast<const f16*>(delta),
                       static_cast<const f16*>(weight), eps, static_cast<f16*>(x_out), static_cast<f16*>(output),
                       (int)hidden);
    return check_launch();
}

int w4a16_silu_mul_f16(const void* gate_up, void* output, int64_t rows, int64_t inter, void* stream) {
    if (rows == 0) return W4A16_OK;
    if (!gate_up || !output) return fail(W4A16_ERR_NULL, "silu_mul: every pointer must be non-NULL");
    if (rows < 0 || inter <= 0 || rows * inter > (int64_t)INT32_MAX * 128)
        return fail(W4A16_ERR_SHAPE, "silu_mul: rows must be non-negative and inter positive");
    if (!aligned(gate_up, 2) || !aligned(output, 2))
        return fail(W4A16_ERR_ALIGNMENT, "silu_mul: fp16 buffers must be 2-byte aligned");
    if (inter % 8 == 0 && aligned(gate_up, 16) && aligned(output, 16)) {
        const int64_t vblocks = (rows * (inter / 8) + 255) / 256;
        hipLaunchKernelGGL(w4a16::silu_mul_vec_kernel, dim3((unsigned)vblocks), dim3(256), 0,
                           static_cast<hipStream_t>(stream), static_cast<const w4a16::f16*>(gate_up),
                           static_cast<w4a16::f16*>(output), (int)rows, (int)inter);
        return check_launch();
    }
    const int64_t blocks = (rows * inter + 255) / 256;
    hipLaunchKernelGGL(w4a16::silu_mul_kernel, dim3((unsigned)blocks), dim3(256), 0,
                       static_cast<hipStream_t>(stream), static_cast<const w4a16::f16*>(gate_up),
                       static_cast<w4a16::f16*>(output), (int)rows, (int)inter);
    return check_launch();
}

int w4a16_prefill_attention_f16(const void* qkv, void* k_cache, void* v_cache, const float* cos_table,
                                const float* sin_table, int64_t start, int64_t tokens, void* output,
                                int64_t num_heads, int64_t num_kv_heads, int64_t head_dim, int64_t max_seq_len,
                                void* stream) {
    if (tokens == 0) return W4A16_OK;
    if (!qkv || !k_cache || !v_cache || !cos_table || !sin_table || !output)
        return fail(W4A16_ERR_NULL, "prefill attention: every pointer must be non-NULL");
    if (head_dim != 64) return fail(W4A16_ERR_CONFIG, "prefill attention: head_dim must be 64");
    if (num_heads <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads != 0 || num_heads > 65535)
        return fail(W4A16_ERR_SHAPE, "prefill attention: num_heads must be a positive multiple of num_kv_heads");
    if (tokens < 0 || start < 0 || start + tokens > max_seq_len || max_seq_len > INT32_MAX / 64)
        return fail(W4A16_ERR_SHAPE, "prefill attention: needs 0 <= tokens and start + tokens <= max_seq_len");
    if (!aligned(k_cache, 16) || !aligned(v_cache, 16) || !aligned(qkv, 2) || !aligned(output, 2))
        return fail(W4A16_ERR_ALIGNMENT, "prefill attention: caches must be 16-byte aligned, qkv and output 2-byte");
    const int nk = (int)(start + tokens);   // slots the last query block sees
    const size_t lds = (size_t)w4a16::kPrefillQueries * 64 * 4 + (size_t)2 * nk * w4a16::kPrefillRow * 2;
    const bool fused = tokens <= w4a16::kPrefillOneLaunch;
    const int64_t group = num_heads / num_kv_heads;
    int glog = 0;
    while ((int64_t)1 << glog < group) ++glog;
    const bool mfma = ((int64_t)1 << glog) == group && group <= 64 && aligned(qkv, 16) && aligned(cos_table, 16) &&
                      aligned(sin_table, 16);
    if (nk > w4a16::kPrefillMaxSlots) {
        // past the slots LDS holds at once: the new rows appended by a launch
        // of their own, then the matrix-core kernel streaming the caches
        // through LDS in blocks of kPrefillBlock slots
        if (!mfma)
            return fail(W4A16_ERR_SHAPE, "prefill attention past 256 slots needs query heads per KV head a power of "
                                         "two up to 64 and 16-byte aligned qkv and rotary tables");
        if ((tokens + (64 >> glog) - 1) / (64 >> glog) > 65535)
            return fail(W4A16_ERR_SHAPE, "prefill attention: tokens / (64 / query heads per KV head) above 65535");
        const int64_t appends = tokens * num_kv_heads * 64;
        hipLaunchKernelGGL(w4a16::prefill_rope_append_kernel, dim3((unsigned)((appends + 255) / 256)), dim3(256), 0,
                           static_cast<hipStream_t>(stream), static_cast<const w4a16::f16*>(qkv),
                           static_cast<w4a16::f16*>(k_cache), static_cast<w4a16::f16*>(v_cache), cos_table, sin_table,
                           (int)start, (int)tokens, (int)num_heads, (int)num_kv_heads, (int)max_seq_len);
        int rc = check_launch();
        if (rc != W4A16_OK) return rc;
        const auto skern = w4a16::prefill_attention_mfma_kernel<false>;
        const size_t slds = std::max((size_t)2 * w4a16::kPrefillBlock * w4a16::kPrefillRow * 2,
                                     (size_t)w4a16::kPrefillMergeBytes);
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(skern),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, (int)slds);
        if (e != hipSuccess) return fail(W4A16_ERR_LAUNCH, "prefill attention: LDS request refused");
        const int tpw = 64 >> glog;
        hipLaunchKernelGGL(skern, dim3((unsigned)num_kv_heads, (unsigned)((tokens + tpw - 1) / tpw)),
                           dim3(w4a16::kPrefillThreads), slds,
                           static_cast<hipStream_t>(stream), static_cast<const w4a16::f16*>(qkv),
                           static_cast<w4a16::f16*>(k_cache), static_cast<w4a16::f16*>(v_cache), cos_table,
                           sin_table, (int)start, (int)tokens, static_cast<w4a16::f16*>(output), (int)num_heads,
                           (int)num_kv_heads, (int)max_seq_len, glog);
        return check_launch();
    }
    if (mfma) {
        const auto mkern = w4a16::prefill_attention_mfma_kernel<true>;
        const void* mk = reinterpret_cast<const void*>(mkern);
        const size_t mlds = std::max((size_t)2 * ((nk + 31) & ~31) * w4a16::kPrefillRow * 2,
                                     (size_t)w4a16::kPrefillMergeBytes);
        if (mlds > 64 * 1024) {
            const hipError_t e = hipFuncSetAttribute(mk, hipFuncAttributeMaxDynamicSharedMemorySize, (int)mlds);
            if (e != hipSuccess) return fail(W4A16_ERR_LAUNCH, "prefill attention: LDS request refused");
        }
        const int tpw = 64 >> glog;
        hipLaunchKernelGGL(mkern, dim3((unsigned)num_kv_heads, (unsigned)((tokens + tpw - 1) / tpw)),
                           dim3(w4a16::kPrefillThreads), mlds, static_cast<hipStream_t>(stream), static_cast<const w4a16::f16*>(qkv),
                           static_cast<w4a16::f16*>(k_cache), static_cast<w4a16::f16*>(v_cache), cos_table,
                           sin_table, (int)start, (int)tokens, static_cast<w4a16::f16*>(output), (int)num_heads,
                           (int)num_kv_heads, (int)max_seq_len, glog);
        return check_launch();
    }
    const auto attend = fused ? w4a16::prefill_attention_kernel<true> : w4a16::prefill_attention_kernel<false>;
    const void* kern = reinterpret_cast<const void*>(attend);
    if (lds > 64 * 1024) {
        const hipError_t e = hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return fail(W4A16_ERR_LAUNCH, "prefill attention: LDS request refused");
    }
    const unsigned blocks = (unsigned)((tokens + w4a16::kPrefillQueries - 1) / w4a16::kPrefillQueries);
    if (!fused) {
        const int64_t appends = tokens * num_kv_heads * 64;
        hipLaunchKernelGGL(w4a16::prefill_rope_append_kernel, dim3((unsigned)((appends + 255) / 256)), dim3(256), 0,
                           static_cast<hipStream_t>(stream), static_cast<const w4a16::f16*>(qkv),
                           static_cast<w4a16::f16*>(k_cache), static_cast<w4a16::f16*>(v_cache), cos_table, sin_table,
                           (int)start, (int)tokens, (int)num_heads, (int)num_kv_heads, (int)max_seq_len);
        const int rc = check_launch();
        if (rc != W4A16_OK) return rc;
    }
    hipLaunchKernelGGL(attend, dim3((unsigned)num_heads, blocks), dim3(256), lds, static_cast<hipStream_t>(stream),
                       static_cast<const w4a16::f16*>(qkv), static_cast<w4a16::f16*>(k_cache),
                       static_cast<w4a16::f16*>(v_cache), cos_table, sin_table, (int)start, (int)tokens,
                       static_cast<w4a16::f16*>(output), (int)num_heads, (int)num_kv_heads, (int)max_seq_len);
    return check_launch();
}

}  // extern "C"

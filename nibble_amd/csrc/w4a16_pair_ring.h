// Small-batch GEMV (M = 1..8) on the matrix cores in the paired layout, with
// a ring of weight loads in flight per wavefront, for gfx950. Kept apart
// from w4a16_kernels.h so its instantiations build in their own
// translation unit.
#pragma once

#include "w4a16_attn_device.h"
#include "w4a16_device.h"

namespace w4a16 {

// ---------------------------------------------------------------------------
// Paired-layout ring GEMV, G = 128, G even, runtime M <= MS (MS = 1, 4 or 8
// row slots).
//
// Operand layout of v_mfma_f32_16x16x32_f16 (lane l = 16 q + c): lane l
// supplies A row c, k = 8q .. 8q + 7 and B column c, k = 8q .. 8q + 7, and
// receives D rows 4q .. 4q + 3 of column c. Column c of B is weight row
// c & 7 of an 8-row block, group 2p + (c >> 3) of group pair p: the lane
// loads bytes 16q .. 16q + 15 of that group, so one load instruction reads
// 8 rows x 128 contiguous bytes, and its four 32-bit words are the B
// operands of the pair's four MFMAs (word t: k = 32q + 8t .. + 7 of the
// group). A row c holds activation row c & 7 (M = 1: row 0 in every A row)
// of the group of half c >> 3, so D[i][c] is a wanted product when i and c
// lie in the same half: D rows 0..7 x columns 0..7 (lanes 0..7 and 16..23,
// group 2p) and D rows 8..15 x columns 8..15 (lanes 40..47 and 56..63,
// group 2p + 1). The halves of an output are added at the end (lane l + 40
// onto lane l); the cross-half blocks are dropped. The MFMA count per byte of
// weights does not depend on M.
//
// Offset decode: B holds the codes without fix-ups (even k as 1024 + v, odd
// k as 1024 + 16 v with v = s + 8, one shift and four v_bitop3 per word); A
// holds the activations permuted to the same pair order with the odd-k
// halves scaled by 1/16 (exact for normal fp16), so the chain's sum is
// sum(x s) + 1032 sum(x_even) + 1152 sum(x_odd / 16). The activation term is
// computed once per (group, activation row) while staging and each chain
// starts from its negative, loaded into the accumulator straight from LDS.
// The group scale then multiplies the chain's result in fp32 FMAs (one at M =
// 1, four otherwise). VALU work per 8 rows x 128 weights: 20 decode
// instructions and 1 or 4 FMAs.
//
// Workgroup = SK x SN wavefronts; wavefront (kw, nb) owns RB blocks of 8 rows
// and pairs kw PPW .. kw PPW + PPW - 1. Order of requests: the workgroup's
// activation units, its scale words, then the wavefront's first D pairs of
// weights (a wavefront's loads return in issue order). Staging writes the
// permuted units, the per-(group, row) bias and the workgroup's scales as
// fp32 split by half (s[row][h][p] = scale of group 2p + h), one barrier,
// then pair j is decoded as its load arrives, pair j + D is requested into
// the registers it freed, and pair j goes through the MFMAs. Requesting every
// pair up front (D = PPW) measured slower: the memory pipeline accepts
// requests at its own pace, so a wavefront that issues all of them sits at
// the issue of its later loads while its first pairs have long arrived, the
// staging and every multiply wait until the last request is out (about
// 3.5 us into a 4096 x 14336 call, from in-kernel timestamps) and the
// arithmetic then runs as a burst after the stream (7.05 against 6.34 us at
// that shape and M = 1). Pairs past K (SK PPW > G/2) re-read the last pair
// with zero activations, zero bias and zero scale. SK > 1: the K slices'
// partial sums are added in slice order through LDS.
//
// Staged activations: unit (m, g, u) (row m, k = 128 g + 8 u .. + 7) at byte
// m RS + 272 g + 16 u. The group stride of 272 bytes and a row stride RS
// = 32 mod 256 put the 16 units one A-fragment read takes from a DPP row of
// lanes (8 rows x 2 groups) on distinct 16-byte bank slots; staging writes
// 16 consecutive units per DPP row.
// ---------------------------------------------------------------------------
__host__ __device__ constexpr int pair_ring_group_bytes() { return 272; }

__host__ __device__ constexpr int64_t pair_ring_row_bytes(int SK, int PPW, int MS = 8) {
    // 2 SK PPW groups of 272 bytes, padded to 32 mod 256 (16 mod 256 with 16
    // row slots, whose A-fragment reads take 16 rows of one group)
    return ((int64_t)2 * SK * PPW * 272 + (MS == 16 ? 240 : 224) + 255) / 256 * 256 - (MS == 16 ? 240 : 224);
}

__host__ __device__ constexpr int64_t pair_ring_lds_bytes(int MS, int SK, int SN, int RB, int PPW) {
    return (MS == 1 ? (int64_t)2 * SK * PPW * 272 : MS * pair_ring_row_bytes(SK, PPW, MS))   // staged units
           + (MS == 16 ? 0 : (int64_t)2 * SK * PPW * (MS == 1 ? 1 : 8) * 4)                 // per-(group, row) bias
           + (int64_t)8 * RB * SN * 2 * SK * PPW * 4                                         // fp32 scales
           + (SK > 1 ? (int64_t)SN * RB * SK * (MS == 1 ? 8 : MS == 16 ? 128 : 64) * 4 : 0) // K-slice partials
           + (MS == 1 ? (int64_t)SK * SN * 4 : 0);                                           // RMSNorm partials
}

// The outputs of every form, and the fp32 K-slice partial sums of the
// 16-row-slot forms, go out through store_through (w4a16_device.h). Graph
// timing at M = 1: 2048 x 5632 3.21-3.28 -> 3.16-3.18 us, 5632 x 2048 3.17 ->
// 3.14, 4096 x 14336 6.44-6.48 -> 6.43-6.44 (non-temporal stores instead: +0.5
// us on the first two); 5632 x 2048 at M = 16 with 8 K slices 7.34 -> 7.14.
// The partial sums at M <= 8 keep ordinary stores (28672 x 8192 at M = 8, 2 MB
// of partials beside the weight stream: 24.95 against 25.9 us written
// through).

// LDS of the ATTN prologue beyond the GEMV's: the slice's attention output
// in natural order [16 rows][256] fp16, then one V tile [32 slots][72] fp16
// per attending wavefront (rows padded to 144 bytes, as the prompt attention
// kernel's).
__host__ __device__ constexpr int64_t pair_ring_attn_lds_bytes() { return 16 * 256 * 2 + 4 * 32 * 72 * 2; }

// Fused work around the GEMV: an RMSNorm of the activation row while it is
// staged (norm_weight, M = 1), a residual add in the epilogue (residual, M =
// 1), and the prompt attention that produces the activations (ATTN: qkv ..
// max_seq).
struct RingFusion {
    const f16* norm_weight;   // null: no RMSNorm
    float eps;
    const f16* residual;      // null: no residual add
    const f16* qkv;           // [T][(H + 2 num_kv) 64]: q heads, k heads, v heads
    f16* k_cache;             // [num_kv][max_seq][64]
    f16* v_cache;
    const float* cos_table;   // [max_seq][32]
    const float* sin_table;
    int start;                // the prompt's first cache slot
    int group;                // query heads per KV head
    int num_kv;
    int max_seq;
};

// The ATTN prologue of one wavefront (see gemv_pair_ring): query head hq's
// causal attention over the prompt's T tokens at slots fz.start ..
// fz.start + T - 1 (at most slot 31), row t < T of the output written to
// out[256 t .. 256 t + 63] (fp16); vt is the wavefront's V tile [32][72].
// append: this wavefront writes the new k / v rows of its KV head to the
// caches (the caller picks one per KV head). Every lane must be active.
__device__ __forceinline__ void attend_slice(const RingFusion& fz, int T, int K, int hq, bool append, int lane,
                                             f16* out, f16* vt) {
    constexpr int VR = 72;
    constexpr float kLog2e = 1.4426950408889634f;
    const int H = K >> 6;
    const int start = fz.start, nk = start + T;
    const int kv = hq / fz.group;
    const size_t rs = (size_t)(H + 2 * fz.num_kv) * 64;   // qkv row stride
    const f16* kq = fz.qkv + (size_t)(H + kv) * 64;
    const f16* vq = fz.qkv + (size_t)(H + fz.num_kv + kv) * 64;
    f16* kc = fz.k_cache + (size_t)kv * fz.max_seq * 64;
    f16* vc = fz.v_cache + (size_t)kv * fz.max_seq * 64;
    const int j = lane & 15, q4 = lane >> 4;
    const u32x4 zero = {0u, 0u, 0u, 0u};

    // 1. loads: query column j (token min(j, T - 1)), key rows 16 mt + j
    // (dims 8 q4 .. + 7 and 32 + 8 q4 .. + 7), V units lane + 64 b (slot i
    // >> 3, dims 8 (i & 7) ..), slots below start from the caches and the
    // new ones from qkv, then the rotary values of the query's and the keys'
    // slots
    const int tq = min(j, T - 1);
    const f16* qrow = fz.qkv + (size_t)tq * rs + (size_t)hq * 64;
    const u32x4 qa = *reinterpret_cast<const u32x4*>(qrow + 8 * q4);
    const u32x4 qz = *reinterpret_cast<const u32x4*>(qrow + 32 + 8 * q4);
    u32x4 kl[2], kh[2];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
        const int r = 16 * mt + j;
        const f16* src = r < start ? kc + (size_t)r * 64 : kq + (size_t)min(max(r - start, 0), T - 1) * rs;
        kl[mt] = *reinterpret_cast<const u32x4*>(src + 8 * q4);
        kh[mt] = *reinterpret_cast<const u32x4*>(src + 32 + 8 * q4);
    }
    u32x4 vv[4];
#pragma unroll
    for (int b = 0; b < 4; ++b) {
        const int i = lane + 64 * b, r = i >> 3;
        const f16* src = r < start ? vc + (size_t)r * 64 : vq + (size_t)min(max(r - start, 0), T - 1) * rs;
        vv[b] = *reinterpret_cast<const u32x4*>(src + 8 * (i & 7));
    }
    auto trig = [&](int pos, float (&c)[8], float (&sn)[8]) {
        const size_t ti = (size_t)pos * 32 + 8 * q4;
        const f32x4 c0 = *reinterpret_cast<const f32x4*>(fz.cos_table + ti);
        const f32x4 c1 = *reinterpret_cast<const f32x4*>(fz.cos_table + ti + 4);
        const f32x4 s0 = *reinterpret_cast<const f32x4*>(fz.sin_table + ti);
        const f32x4 s1 = *reinterpret_cast<const f32x4*>(fz.sin_table + ti + 4);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            c[e] = c0[e];
            c[4 + e] = c1[e];
            sn[e] = s0[e];
            sn[4 + e] = s1[e];
        }
    };
    float qc[8], qs[8], kcs[2][8], ksn[2][8];
    trig(start + tq, qc, qs);
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) trig(min(16 * mt + j, nk - 1), kcs[mt], ksn[mt]);

    // 2. the rotary q (B operand, times 1/8) and the key rows (A operand):
    // cached rows as they are, new rows rotated at their slot, rows past the
    // prompt zero; then the append
    u32x4 qb[2];
    rope8(qa, qz, qc, qs, 0.125f, qb[0], qb[1]);
    u32x4 ka[2][2];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
        const int r = 16 * mt + j;
        u32x4 lo, hi;
        rope8(kl[mt], kh[mt], kcs[mt], ksn[mt], 1.0f, lo, hi);
        ka[mt][0] = r < start ? kl[mt] : r < nk ? lo : zero;
        ka[mt][1] = r < start ? kh[mt] : r < nk ? hi : zero;
    }
    if (append) {
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
            const int r = 16 * mt + j;
            if (r >= start && r < nk) {
                *reinterpret_cast<u32x4*>(kc + (size_t)r * 64 + 8 * q4) = ka[mt][0];
                *reinterpret_cast<u32x4*>(kc + (size_t)r * 64 + 32 + 8 * q4) = ka[mt][1];
            }
        }
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const int i = lane + 64 * b, r = i >> 3;
            if (r >= start && r < nk) *reinterpret_cast<u32x4*>(vc + (size_t)r * 64 + 8 * (i & 7)) = vv[b];
        }
    }

    // 3. the V tile, slot rows (zero past the prompt)
#pragma unroll
    for (int b = 0; b < 4; ++b) {
        const int i = lane + 64 * b, r = i >> 3;
        *reinterpret_cast<u32x4*>(vt + r * VR + 8 * (i & 7)) = r < nk ? vv[b] : zero;
    }
    wave_lds_sync();

    // 4. S^T = K Q^T: lane (q4, j) holds column j's scores of slots 16 mt +
    // 4 q4 + e, masked past the column's slot; softmax over the 32 slots
    f32x4 st[2];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
        st[mt] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2)
            st[mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, ka[mt][s2]),
                                                            __builtin_bit_cast(f16x8, qb[s2]), st[mt], 0, 0, 0);
    }
    const int last = start + tq;
    float mx = -__builtin_inff();
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int slot = 16 * mt + 4 * q4 + e;
            st[mt][e] = slot <= last ? st[mt][e] : -__builtin_inff();
            mx = fmaxf(mx, st[mt][e]);
        }
    mx = row_pair_max(mx);
    const float mbl = mx * kLog2e;   // finite: slot 0 is visible to every column
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

    // 5. O^T = V^T P^T (V^T through the transposing LDS read): lane (q4, j)
    // receives token j's dims 16 md + 4 q4 .. + 3
    const float inv = 1.0f / psum;
    const int tk = j >> 2, tm = j & 3;
#pragma unroll
    for (int md = 0; md < 4; ++md) {
        const f16* src = vt + (4 * q4 + tk) * VR + 16 * md + 4 * tm;
        const uint2 lo = lds_read_tr16(src);
        const uint2 hi = lds_read_tr16(src + 16 * VR);
        const u32x4 av = {lo.x, lo.y, hi.x, hi.y};
        const f32x4 o = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, av),
                                                               __builtin_bit_cast(f16x8, pb),
                                                               (f32x4){0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
        if (j < T) {
            const f16x2 a = {(f16)(o[0] * inv), (f16)(o[1] * inv)};
            const f16x2 b = {(f16)(o[2] * inv), (f16)(o[3] * inv)};
            *reinterpret_cast<uint2*>(out + j * 256 + 16 * md + 4 * q4) = make_uint2(as_u32(a), as_u32(b));
        }
    }
}

// SPLIT (narrow layers of long rows): the K / 256 pairs are cut into S
// slices of SK PPW pairs; workgroup b takes slice b mod S of rows (b / S) R
// .., stages only that slice's activations, and stores fp32 partial sums to
// part[slice][m][n] instead of fp16 outputs (pair_split_reduce adds the
// slices in slice order). Every CU then stages M K / S activations instead
// of M K, which on such layers outweighs the CU's weights.
//
// MS = 16 (M = 9..16, a short prompt): the dequantized weights in B, exact
// codes times the group scale rounded to fp16 once (as w4a16_dequantize_f16
// writes them), the activations staged unscaled and no bias, summed in the
// MFMA's fp32 accumulators across pairs: the reference's prefill (dequantize,
// fp16 GEMM with fp32 accumulation) up to summation order. A rows are the 16
// activation rows of one group, so each pair runs two MFMAs per word against
// the same B (group 2p in A for B columns 0..7, group 2p + 1 for columns
// 8..15) and a lane keeps both; the halves of an output sit in lanes l and
// l + 8. The staged row stride is 16 mod 256 so the 16 rows of a fragment
// read fall on distinct bank slots.
//
// SILU (MS = 16 or 1, RB = 2): N is the intermediate width, the weights hold
// 2 N rows (gate rows, then up rows); block 0 of a wavefront is gate rows n
// .. n + 7 and block 1 the up rows N + n .., and the output is
// fp16(fp16(silu(fp16(g))) * fp16(u)), the roundings of silu(gate) * up on
// fp16 tensors.
//
// NORM (MS = 1): the staged row is y = fp16((fp32(x) * rsqrt(mean(x^2) + eps))
// * fp32(norm_weight)), the fp32 operation order of an RMSNorm that returns
// fp16 (the squares summed per thread, per wavefront by DPP, then the
// wavefronts in order; one more barrier). RESID (MS = 1): out[n] =
// fp16(fp32(residual[n]) + fp32(fp16(dot))), a residual stream's x +
// linear(a); residual may alias out (each row is read and written by the
// same lane, the read requested with the first weights).
//
// ATTN (MS = 16, SPLIT, one pair per slice, SK = 1, SN >= 4): x is not read;
// the activations are the causal attention of a prompt's M tokens at cache
// slots start .. start + M - 1 (start + M <= 32, head_dim 64, K = 64 H for
// H query heads), the o projection's input. Slice sl holds query heads 4 sl
// .. 4 sl + 3; wavefront w < 4 attends head 4 sl + w for every token (MFMA
// column j = token j) and writes its output rows to LDS, the other
// wavefronts wait at the barrier, and staging reads the units from there.
// The arithmetic is prefill_attention_mfma_kernel's for one chunk of 32
// slots (rotary q scaled by 1/8 and k in fp32 rounded to fp16, S^T = K Q^T
// and O^T = V^T P^T on the matrix cores, the softmax's max and sum across
// the column's four lanes, exp as exp2 of the log2 e scaled score, P in
// fp16); the compiler may round a rotary value to fp16 in one step (fused
// multiply-add with an fp16 result) in one kernel and through fp32 in the
// other, so a rotary q or k can differ from that kernel's by one fp16 unit.
// Slots below start come from the caches; the new tokens' k (rotated at
// their slots) and v come from qkv, and the first query head of each KV
// head in row block 0 appends them to the caches.
template <int MS, int SK, int SN, int RB, int PPW, int D, bool SPLIT = false, bool SILU = false, bool NORM = false,
          bool RESID = false, bool ATTN = false>
__global__ void __launch_bounds__(64 * SK * SN)
gemv_pair_ring(const f16* __restrict__ x, const uint8_t* __restrict__ w, const f16* __restrict__ scales,
               f16* out, int M, int N, int K, float* __restrict__ part, int S, RingFusion fz) {
    static_assert(MS == 1 || MS == 4 || MS == 8 || MS == 16, "1, 4, 8 or 16 activation row slots");
    static_assert(D >= 1 && D <= PPW, "ring depth 1 .. PPW");
    static_assert(!SILU || ((MS == 16 || MS == 1) && RB == 2 && !SPLIT),
                  "the SiLU form pairs a gate block and its up block");
    static_assert(!NORM || (MS == 1 && !SPLIT), "the RMSNorm prologue normalises one whole activation row");
    static_assert(!RESID || (MS == 1 && !SPLIT && !SILU), "the residual epilogue adds to one output row");
    static_assert(!ATTN || (MS == 16 && SPLIT && SK == 1 && PPW == 1 && SN >= 4 && !SILU),
                  "the attention prologue fills one pair (four heads) per K slice");
    constexpr bool W16 = MS == 16;            // exact decode, two MFMAs per word
    constexpr int W = SK * SN;
    constexpr int T = 64 * W;
    constexpr int PS = SK * PPW;              // pairs staged
    constexpr int GS = 2 * PS;                // groups staged
    constexpr int US = GS * 16;               // activation units staged per row
    constexpr int XU = (MS * US + T - 1) / T; // staging units per thread
    constexpr int RO = SILU ? 1 : RB;         // output blocks of 8 rows per wavefront
    constexpr int R = 8 * RO * SN;            // output rows per workgroup
    constexpr int SR = 8 * RB * SN;           // weight rows per workgroup
    constexpr int SD = SR * PS;               // scale words (pairs) per workgroup
    constexpr int SU = (SD + T - 1) / T;      // scale words per thread
    constexpr int RS = MS == 1 ? 0 : (int)pair_ring_row_bytes(SK, PPW, MS);
    constexpr int XB = MS == 1 ? GS * 272 : MS * RS;
    constexpr int BS = MS == 1 ? 1 : 8;       // bias slots per group
    constexpr int NB = W16 ? 0 : GS * BS;     // bias words
    extern __shared__ __align__(16) uint8_t smem[];
    float* bias = reinterpret_cast<float*>(smem + XB);   // [GS][BS]
    float* sc = bias + NB;                                 // [SR][2][PS]
    float* red = sc + SR * 2 * PS;                         // [SN RB][SK][8, 64 or 128]
    float* np = red + (SK > 1 ? SN * RB * SK * (MS == 1 ? 8 : MS == 16 ? 128 : 64) : 0);   // [W] (MS = 1)
    // ATTN: the slice's attention rows [16][256] fp16, then the V tiles
    f16* xa = reinterpret_cast<f16*>(smem + (pair_ring_lds_bytes(MS, SK, SN, RB, PPW) + 15) / 16 * 16);

    const int G = K >> 7;
    const int P = G >> 1;
    const int units = K >> 3;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int col = lane & 15, q = lane >> 4;
    const int brow = col & 7, h = col >> 3;
    const int kw = wave % SK, nb = wave / SK;
    const int sl = SPLIT ? (int)blockIdx.x % S : 0;   // K slice
    const int n0 = (SPLIT ? (int)blockIdx.x / S : (int)blockIdx.x) * R;
    const int nw = n0 + nb * RO * 8;                  // first output row of the wavefront
    const int pb = sl * PS;                           // first pair of the slice
    const uint32_t row_bytes = (uint32_t)(K >> 1);
    // weight row of block b, row r (clamped to the layer)
    auto wrow = [&](int base, int b, int r) {
        if constexpr (SILU) return (b ? N : 0) + min(base + r, N - 1);
        else return min(base + 8 * b + r, N - 1);
    };

    // 1. requests: activation units (clamped; units past K or M are not
    // staged), the workgroup's scale words, then the wavefront's first D
    // pairs of weights
    u32x4 a[XU];
    if constexpr (!ATTN) {
#pragma unroll
        for (int u = 0; u < XU; ++u) {
            const int i = threadIdx.x + u * T;
            const int m = MS == 1 ? 0 : min(i / US, M - 1);
            const int uu = min(pb * 32 + (MS == 1 ? i : i % US), units - 1);
            a[u] = *reinterpret_cast<const u32x4*>(x + (size_t)m * K + (size_t)uu * 8);
        }
    }
    u32x4 gw[NORM ? XU : 1];
    if constexpr (NORM) {
#pragma unroll
        for (int u = 0; u < XU; ++u) {
            const int uu = min(pb * 32 + (int)threadIdx.x + u * T, units - 1);
            gw[u] = *reinterpret_cast<const u32x4*>(fz.norm_weight + (size_t)uu * 8);
        }
    }
    const uint32_t* s32 = reinterpret_cast<const uint32_t*>(scales);
    uint32_t sw[SU];
#pragma unroll
    for (int u = 0; u < SU; ++u) {
        const int d = threadIdx.x + u * T;
        const int r = d / PS, p = d - r * PS;   // staged row r = (wavefront, block, row)
        const int blk = r >> 3;
        const int n = wrow(n0 + (blk / RB) * RO * 8, blk % RB, r & 7);
        sw[u] = s32[(size_t)n * P + min(pb + p, P - 1)];
    }
    // weights of pair j go to ring slot j % D
    u32x4 wv[D][RB];
    auto issue = [&](int j) {
        const uint32_t pg = (uint32_t)min(pb + kw * PPW + j, P - 1);
#pragma unroll
        for (int b = 0; b < RB; ++b) {
            const int n = wrow(nw, b, brow);
            wv[j % D][b] = load_stream(reinterpret_cast<const u32x4*>(w + (size_t)n * row_bytes + pg * 128u +
                                                                     (uint32_t)(h * 64 + q * 16)));
        }
    };
#pragma unroll
    for (int j = 0; j < D; ++j) issue(j);
    // the residual values of this lane's output rows (lanes 0..7)
    f16 resv[RB];
    if constexpr (RESID) {
#pragma unroll
        for (int b = 0; b < RB; ++b) resv[b] = fz.residual[min(nw + 8 * b + (lane & 7), N - 1)];
    }
    __builtin_amdgcn_sched_barrier(0);

    if constexpr (NORM) {
        // mean of squares of the row (units past K are not staged)
        float ss = 0.0f;
#pragma unroll
        for (int u = 0; u < XU; ++u) {
            const int i = threadIdx.x + u * T;
            if (i < US && pb * 32 + i < units) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const f16x2 p = as_f16x2(a[u][e]);
                    ss = __builtin_fmaf((float)p.x, (float)p.x, ss);
                    ss = __builtin_fmaf((float)p.y, (float)p.y, ss);
                }
            }
        }
        ss = wave_sum(ss);
        if (lane == 0) np[wave] = ss;
        __syncthreads();
        float total = 0.0f;
#pragma unroll
        for (int v = 0; v < W; ++v) total += np[v];
        const float inv = 1.0f / __builtin_sqrtf(total / (float)K + fz.eps);
#pragma unroll
        for (int u = 0; u < XU; ++u) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const f16x2 p = as_f16x2(a[u][e]), g = as_f16x2(gw[u][e]);
                const f16x2 y = {(f16)(((float)p.x * inv) * (float)g.x), (f16)(((float)p.y * inv) * (float)g.y)};
                a[u][e] = as_u32(y);
            }
        }
    }

    if constexpr (ATTN) {
        // the first query head of each KV head in row block 0 appends
        const int hq = 4 * sl + wave;
        if (wave < 4)
            attend_slice(fz, M, K, hq, blockIdx.x < (unsigned)S && hq % fz.group == 0, lane, xa + wave * 64,
                         xa + 16 * 256 + wave * 32 * 72);
        __syncthreads();
#pragma unroll
        for (int u = 0; u < XU; ++u) {
            const int i = threadIdx.x + u * T;
            const int m = min(i / US, M - 1);
            a[u] = *reinterpret_cast<const u32x4*>(xa + m * 256 + (i % US) * 8);
        }
    }

    // 2. staging: unit i = m US + uu covers x[m][8 uu .. 8 uu + 7] (group
    // uu / 16); the 16 units of a (row, group) sit in one DPP row, whose sum
    // is that row's bias for the group (offset decode only)
    const f16x2 sixteenth = {(f16)0.0625f, (f16)0.0625f};
    const f16x2 c_even = {(f16)1032.0f, (f16)1032.0f};
    const f16x2 c_odd = {(f16)1152.0f, (f16)1152.0f};
#pragma unroll
    for (int u = 0; u < XU; ++u) {
        const int i = threadIdx.x + u * T;
        const int m = MS == 1 ? 0 : i / US;
        const int uu = MS == 1 ? i : i % US;
        u32x4 v = permute8(a[u]);
        if constexpr (!W16) {
            v.y = as_u32(as_f16x2(v.y) * sixteenth);
            v.w = as_u32(as_f16x2(v.w) * sixteenth);
        }
        if (pb * 32 + uu >= units) v = (u32x4){0u, 0u, 0u, 0u};
        float cs = 0.0f;
        if constexpr (!W16) {
            cs = __builtin_amdgcn_fdot2(as_f16x2(v.x), c_even, 0.0f, false);
            cs = __builtin_amdgcn_fdot2(as_f16x2(v.y), c_odd, cs, false);
            cs = __builtin_amdgcn_fdot2(as_f16x2(v.z), c_even, cs, false);
            cs = __builtin_amdgcn_fdot2(as_f16x2(v.w), c_odd, cs, false);
            cs += dpp<0xB1>(cs);
            cs += dpp<0x4E>(cs);
            cs += dpp<0x141>(cs);
            cs += dpp<0x140>(cs);
        }
        if ((MS == 1 ? i < US : m < M) && i < MS * US) {
            const int g = uu >> 4;
            *reinterpret_cast<u32x4*>(smem + (MS == 1 ? 0 : m * RS) + g * 272 + (uu & 15) * 16) = v;
            if (!W16 && (uu & 15) == 0) bias[g * BS + (MS == 1 ? 0 : m)] = -cs;
        }
    }
#pragma unroll
    for (int u = 0; u < SU; ++u) {
        const int d = threadIdx.x + u * T;
        const int r = d / PS, p = d - r * PS;
        if (d < SD) {
            const bool ok = pb + p < P;
            const f16x2 sv = as_f16x2(sw[u]);
            sc[(2 * r) * PS + p] = ok ? (float)sv.x : 0.0f;
            sc[(2 * r + 1) * PS + p] = ok ? (float)sv.y : 0.0f;
        }
    }
    __syncthreads();

    // 3. pairs in arrival order; A fragments of pair j + 1 read during pair j.
    // MS <= 8: A row c = activation row c & 7 (clamped to M - 1) of group
    // 2p + h; D rows 4q .. 4q + 3 = activation rows 4 (q & 1) .. + 3 of group
    // 2p + (q >> 1). MS = 16: A row c = activation row c (clamped) of group
    // 2p (first MFMA) or 2p + 1 (second); D rows 4q .. 4q + 3 = activation
    // rows 4q .. 4q + 3.
    constexpr int H = W16 ? 2 : 1;   // MFMAs per word
    const int arow = MS == 1 ? 0 : min(W16 ? col : brow, M - 1);
    const uint8_t* xl = smem + (MS == 1 ? 0 : arow * RS) + (2 * kw * PPW + (W16 ? 0 : h)) * 272 + q * 64;
    const float* bl = MS == 1 ? bias + 2 * kw * PPW + h : bias + (2 * kw * PPW + (q >> 1)) * 8 + 4 * (q & 1);
    const float* scl[RB];
#pragma unroll
    for (int b = 0; b < RB; ++b) scl[b] = sc + (2 * (8 * (nb * RB + b) + brow) + h) * PS + kw * PPW;
    constexpr int NA = MS == 1 ? 1 : 4;   // accumulators per lane
    float acc[RB][NA];
    f32x4 d[RB][H];
#pragma unroll
    for (int b = 0; b < RB; ++b) {
#pragma unroll
        for (int e = 0; e < NA; ++e) acc[b][e] = 0.0f;
#pragma unroll
        for (int hh = 0; hh < H; ++hh) d[b][hh] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
    }
    u32x4 A0[H][4], A1[H][4];
#pragma unroll
    for (int hh = 0; hh < H; ++hh)
#pragma unroll
        for (int t = 0; t < 4; ++t) A0[hh][t] = *reinterpret_cast<const u32x4*>(xl + hh * 272 + t * 16);
#pragma unroll
    for (int j = 0; j < PPW; ++j) {
        u32x4 (&cur)[H][4] = (j & 1) ? A1 : A0;
        u32x4 (&nxt)[H][4] = (j & 1) ? A0 : A1;
        if (j + 1 < PPW) {
#pragma unroll
            for (int hh = 0; hh < H; ++hh)
#pragma unroll
                for (int t = 0; t < 4; ++t)
                    nxt[hh][t] = *reinterpret_cast<const u32x4*>(xl + (j + 1) * 544 + hh * 272 + t * 16);
        }
        f32x4 bj = {0.0f, 0.0f, 0.0f, 0.0f};
        if constexpr (MS == 1) bj.x = bl[2 * j];
        else if constexpr (!W16) bj = *reinterpret_cast<const f32x4*>(bl + 16 * j);
        Codes8 cw[RB][4];
#pragma unroll
        for (int b = 0; b < RB; ++b) {
            if constexpr (W16) {
                // B = fp16_rn(code * scale): the staged fp32 scale is an fp16
                // value, so the conversion back is exact (0 past K)
                const f16 s16 = (f16)scl[b][j];
                const f16x2 s2 = {s16, s16};
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    cw[b][t] = unpack8(wv[j % D][b][t]);
#pragma unroll
                    for (int e = 0; e < 4; ++e) cw[b][t].p[e] = cw[b][t].p[e] * s2;
                }
            } else {
#pragma unroll
                for (int t = 0; t < 4; ++t) cw[b][t] = unpack8_offset(wv[j % D][b][t]);
            }
        }
        if (j + D < PPW) {
            // the slot is free once decoded: request pair j + D
            __builtin_amdgcn_sched_barrier(0);
            issue(j + D);
            __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int b = 0; b < RB; ++b) {
            f32x4 dd[H];
#pragma unroll
            for (int hh = 0; hh < H; ++hh) dd[hh] = d[b][hh];
            if constexpr (MS == 1) dd[0].x = bj.x;   // registers 1..3 carry unused values
            else if constexpr (!W16) dd[0] = bj;
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const f16x8 bt = __builtin_bit_cast(f16x8, (u32x4){as_u32(cw[b][t].p[0]), as_u32(cw[b][t].p[1]),
                                                                   as_u32(cw[b][t].p[2]), as_u32(cw[b][t].p[3])});
#pragma unroll
                for (int hh = 0; hh < H; ++hh)
                    dd[hh] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, cur[hh][t]), bt, dd[hh],
                                                                    0, 0, 0);
            }
            if constexpr (!W16) {
                const float s = scl[b][j];
#pragma unroll
                for (int e = 0; e < NA; ++e) acc[b][e] = __builtin_fmaf(dd[0][e], s, acc[b][e]);
            }
#pragma unroll
            for (int hh = 0; hh < H; ++hh) d[b][hh] = dd[hh];
        }
    }

    // 4. halves (MS <= 8: lane l + 40 onto lane l; MS = 16: lane l + 8 onto
    // lane l), then the K slices in order. M = 1: lane c < 8 holds row c;
    // else lane 16 q + c (c < 8; q < 2 for MS <= 8) holds activation rows
    // 4q .. 4q + 3 of weight row c.
    constexpr int RED = MS == 1 ? 8 : W16 ? 128 : 64;
    const bool keep = MS == 1 ? lane < 8 : ((W16 || q < 2) && col < 8);
    const int rl = MS == 1 ? lane : (q * 8 + col) * 4;   // slot in a block's partials
    float v[RB][NA];
#pragma unroll
    for (int b = 0; b < RB; ++b)
#pragma unroll
        for (int e = 0; e < NA; ++e) {
            if constexpr (W16) v[b][e] = d[b][0][e] + __shfl(d[b][1][e], lane + 8);
            else v[b][e] = acc[b][e] + __shfl(acc[b][e], lane + 40);
        }
    auto store = [&](const float (&vv)[RB][NA]) {
#pragma unroll
        for (int b = 0; b < RO; ++b) {
            const int n = nw + 8 * b + brow;
            if (n >= N) continue;
#pragma unroll
            for (int e = 0; e < NA; ++e) {
                const int m = MS == 1 ? 0 : 4 * q + e;
                if (MS == 1 || m < M) {
                    if constexpr (SPLIT && W16) store_through(part + ((size_t)sl * M + m) * N + n, vv[b][e]);
                    else if constexpr (SPLIT) part[((size_t)sl * M + m) * N + n] = vv[b][e];
                    else if constexpr (SILU) store_through(out + (size_t)m * N + n, gemm_silu_mul(vv[0][e], vv[1][e]));
                    else if constexpr (RESID) store_through(out + n, (f16)((float)resv[b] + (float)(f16)vv[b][e]));
                    else store_through(out + (size_t)m * N + n, (f16)vv[b][e]);
                }
            }
        }
    };
    if constexpr (SK == 1) {
        if (keep) store(v);
    } else {
        if (keep) {
#pragma unroll
            for (int b = 0; b < RB; ++b)
#pragma unroll
                for (int e = 0; e < NA; ++e) red[((nb * RB + b) * SK + kw) * RED + rl + e] = v[b][e];
        }
        __syncthreads();
        if (kw != 0 || !keep) return;
        float t[RB][NA];
#pragma unroll
        for (int b = 0; b < RB; ++b)
#pragma unroll
            for (int e = 0; e < NA; ++e) {
                t[b][e] = red[((nb * RB + b) * SK) * RED + rl + e];
#pragma unroll
                for (int s = 1; s < SK; ++s) t[b][e] += red[((nb * RB + b) * SK + s) * RED + rl + e];
            }
        store(t);
    }
}

}  // namespace w4a16

// M = 1 GEMV on the matrix cores in the paired layout, with a ring of weight
// loads in flight per wavefront, for gfx950. Kept apart from w4a16_kernels.h
// so its instantiations build in their own translation unit.
#pragma once

#include "w4a16_device.h"

namespace w4a16 {

// ---------------------------------------------------------------------------
// Paired-layout M = 1 GEMV, G = 128, G even.
//
// Operand layout of v_mfma_f32_16x16x32_f16 (lane l = 16 q + c): lane l
// supplies A row c, k = 8q .. 8q + 7 and B column c, k = 8q .. 8q + 7, and
// receives D rows 4q .. 4q + 3 of column c. Column c of B is weight row
// c & 7 of an 8-row block, group 2p + (c >> 3) of group pair p: the lane
// loads bytes 16q .. 16q + 15 of that group, so one load instruction reads
// 8 rows x 128 contiguous bytes, and its four 32-bit words are the B
// operands of the pair's four MFMAs (word t: k = 32q + 8t .. + 7 of the
// group). Every A row c holds the activations of the group of half c >> 3,
// so D[i][c] is a wanted dot product when i and c lie in the same half:
// lanes 0..7 (D row 0, group 2p) and lanes 40..47 (D row 8, group 2p + 1)
// each keep register 0, and the halves of row c are added at the end (lane
// c + 40 onto lane c).
//
// Offset decode: B holds the codes without fix-ups (even k as 1024 + v, odd
// k as 1024 + 16 v with v = s + 8, one shift and four v_bitop3 per word); A
// holds the activations permuted to the same pair order with the odd-k
// halves scaled by 1/16 (exact for normal fp16), so the chain's sum is
// sum(x s) + 1032 sum(x_even) + 1152 sum(x_odd / 16). The activation term is
// computed once per group while staging and each chain starts from its
// negative, loaded into the accumulator's register 0 straight from LDS. The
// group scale then multiplies register 0 in one fp32 FMA. VALU work per
// 8 rows x 128 weights: 20 decode instructions and one FMA (the VALU kernels
// add 16 dot2 instructions and per-chunk staging on top).
//
// Workgroup = SK x SN wavefronts; wavefront (kw, nb) owns RB blocks of 8 rows
// and pairs kw PPW .. kw PPW + PPW - 1. Order of requests: the workgroup's
// activation units, its scale words, then the wavefront's first D pairs of
// weights (a wavefront's loads return in issue order). Staging writes the
// permuted units, the per-group bias and the workgroup's scales as fp32 split
// by half (s[row][h][p] = scale of group 2p + h), one barrier, then pair j is
// decoded as its load arrives, pair j + D is requested into the registers
// it freed, and pair j goes through the MFMAs. Requesting every pair up
// front (D = PPW) measured slower: the memory pipeline accepts requests at
// its own pace, so a wavefront that issues all of them sits at the issue of
// its later loads while its first pairs have long arrived, the staging and
// every multiply wait until the last request is out (about 3.5 us into a
// 4096 x 14336 call, from in-kernel timestamps) and the arithmetic then runs
// as a burst after the stream (7.05 against 6.34 us at that shape). Pairs
// past K (SK PPW > G/2) re-read the last pair with zero activations, zero
// bias and zero scale. SK > 1: the K slices' partial sums are added in slice
// order through LDS.
// ---------------------------------------------------------------------------
__host__ __device__ constexpr int64_t pair_m1_lds_bytes(int SK, int SN, int RB, int PPW) {
    return (int64_t)2 * SK * PPW * 16 * 16         // staged activation units
           + (int64_t)2 * SK * PPW * 4              // per-group bias
           + (int64_t)8 * RB * SN * 2 * SK * PPW * 4  // fp32 scales [rows][2][SK PPW]
           + (SK > 1 ? (int64_t)SN * RB * SK * 8 * 4 : 0);
}

template <int SK, int SN, int RB, int PPW, int D = PPW>
__global__ void __launch_bounds__(64 * SK * SN)
gemv_pair_m1(const f16* __restrict__ x, const uint8_t* __restrict__ w, const f16* __restrict__ scales,
           f16* __restrict__ out, int N, int K) {
    constexpr int W = SK * SN;
    constexpr int T = 64 * W;
    constexpr int PS = SK * PPW;              // pairs staged
    constexpr int US = PS * 32;               // activation units staged (16 per group)
    constexpr int XU = (US + T - 1) / T;      // staging units per thread
    constexpr int R = 8 * RB * SN;            // rows per workgroup
    constexpr int SD = R * PS;                // scale words (pairs) per workgroup
    constexpr int SU = (SD + T - 1) / T;      // scale words per thread
    extern __shared__ __align__(16) uint8_t smem[];
    u32x4* xs = reinterpret_cast<u32x4*>(smem);
    float* bias = reinterpret_cast<float*>(smem + US * 16);
    float* sc = bias + 2 * PS;                // [R][2][PS]
    float* red = sc + R * 2 * PS;             // [SN RB][SK][8]

    const int G = K >> 7;
    const int P = G >> 1;
    const int units = K >> 3;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int col = lane & 15, q = lane >> 4;
    const int brow = col & 7, h = col >> 3;
    const int kw = wave % SK, nb = wave / SK;
    const int n0 = blockIdx.x * R;
    const int nw = n0 + nb * RB * 8;
    const uint32_t row_bytes = (uint32_t)(K >> 1);

    // 1. requests: activation units (clamped; units past K are zeroed when
    // staged), the workgroup's scale words, then the wavefront's weights
    u32x4 a[XU];
#pragma unroll
    for (int u = 0; u < XU; ++u) {
        const int i = min((int)threadIdx.x + u * T, units - 1);
        a[u] = *reinterpret_cast<const u32x4*>(x + (size_t)i * 8);
    }
    const uint32_t* s32 = reinterpret_cast<const uint32_t*>(scales);
    uint32_t sw[SU];
#pragma unroll
    for (int u = 0; u < SU; ++u) {
        const int d = threadIdx.x + u * T;
        const int r = d / PS, p = d - r * PS;
        const int n = min(n0 + r, N - 1);
        sw[u] = s32[(size_t)n * P + min(p, P - 1)];
    }
    // weights of pair j go to ring slot j % D; the first D are requested
    // now, pair j + D after pair j is decoded
    static_assert(D >= 1 && D <= PPW, "ring depth 1 .. PPW");
    u32x4 wv[D][RB];
    auto issue = [&](int j) {
        const uint32_t pg = (uint32_t)min(kw * PPW + j, P - 1);
#pragma unroll
        for (int b = 0; b < RB; ++b) {
            const int n = min(nw + 8 * b + brow, N - 1);
            wv[j % D][b] = load_stream(reinterpret_cast<const u32x4*>(w + (size_t)n * row_bytes + pg * 128u +
                                                                     (uint32_t)(h * 64 + q * 16)));
        }
    };
#pragma unroll
    for (int j = 0; j < D; ++j) issue(j);
    __builtin_amdgcn_sched_barrier(0);

    // 2. staging: unit i covers x[8i .. 8i + 7] (group i / 16); the 16 units
    // of a group sit in one DPP row, whose sum is the group's bias
    const f16x2 sixteenth = {(f16)0.0625f, (f16)0.0625f};
    const f16x2 c_even = {(f16)1032.0f, (f16)1032.0f};
    const f16x2 c_odd = {(f16)1152.0f, (f16)1152.0f};
#pragma unroll
    for (int u = 0; u < XU; ++u) {
        const int i = threadIdx.x + u * T;
        u32x4 v = permute8(a[u]);
        v.y = as_u32(as_f16x2(v.y) * sixteenth);
        v.w = as_u32(as_f16x2(v.w) * sixteenth);
        if (i >= units) v = (u32x4){0u, 0u, 0u, 0u};
        float cs = __builtin_amdgcn_fdot2(as_f16x2(v.x), c_even, 0.0f, false);
        cs = __builtin_amdgcn_fdot2(as_f16x2(v.y), c_odd, cs, false);
        cs = __builtin_amdgcn_fdot2(as_f16x2(v.z), c_even, cs, false);
        cs = __builtin_amdgcn_fdot2(as_f16x2(v.w), c_odd, cs, false);
        cs += dpp<0xB1>(cs);
        cs += dpp<0x4E>(cs);
        cs += dpp<0x141>(cs);
        cs += dpp<0x140>(cs);
        if (i < US) {
            xs[i] = v;
            if ((i & 15) == 0) bias[i >> 4] = -cs;
        }
    }
#pragma unroll
    for (int u = 0; u < SU; ++u) {
        const int d = threadIdx.x + u * T;
        const int r = d / PS, p = d - r * PS;
        if (d < SD) {
            const bool ok = p < P;
            const f16x2 sv = as_f16x2(sw[u]);
            sc[(2 * r) * PS + p] = ok ? (float)sv.x : 0.0f;
            sc[(2 * r + 1) * PS + p] = ok ? (float)sv.y : 0.0f;
        }
    }
    __syncthreads();

    // 3. pairs in arrival order; A fragments of pair j + 1 read during pair j
    const int xo = (2 * kw * PPW + h) * 16 + q * 4;   // this lane's first unit
    const int bo = 2 * kw * PPW + h;                  // this lane's first bias
    const float* scl[RB];
#pragma unroll
    for (int b = 0; b < RB; ++b) scl[b] = sc + (2 * (8 * (nb * RB + b) + brow) + h) * PS + kw * PPW;
    float acc[RB];
    f32x4 d[RB];
#pragma unroll
    for (int b = 0; b < RB; ++b) {
        acc[b] = 0.0f;
        d[b] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
    }
    u32x4 A0[4], A1[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) A0[t] = xs[xo + t];
#pragma unroll
    for (int j = 0; j < PPW; ++j) {
        u32x4 (&cur)[4] = (j & 1) ? A1 : A0;
        u32x4 (&nxt)[4] = (j & 1) ? A0 : A1;
        if (j + 1 < PPW) {
#pragma unroll
            for (int t = 0; t < 4; ++t) nxt[t] = xs[xo + 32 * (j + 1) + t];
        }
        const float bj = bias[bo + 2 * j];
        Codes8 cw[RB][4];
#pragma unroll
        for (int b = 0; b < RB; ++b)
#pragma unroll
            for (int t = 0; t < 4; ++t) cw[b][t] = unpack8_offset(wv[j % D][b][t]);
        if (j + D < PPW) {
            // the slot is free once decoded: request pair j + D
            __builtin_amdgcn_sched_barrier(0);
            issue(j + D);
            __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int b = 0; b < RB; ++b) {
            f32x4 dd = d[b];
            dd.x = bj;
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const f16x8 bt = __builtin_bit_cast(f16x8, (u32x4){as_u32(cw[b][t].p[0]), as_u32(cw[b][t].p[1]),
                                                                   as_u32(cw[b][t].p[2]), as_u32(cw[b][t].p[3])});
                dd = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, cur[t]), bt, dd, 0, 0, 0);
            }
            acc[b] = __builtin_fmaf(dd.x, scl[b][j], acc[b]);
            d[b] = dd;
        }
    }

    // 4. halves (lane c + 40 onto lane c), then the K slices in order
#pragma unroll
    for (int b = 0; b < RB; ++b) {
        const float v = acc[b] + __shfl(acc[b], lane + 40);
        const int n = nw + 8 * b + lane;
        if constexpr (SK == 1) {
            if (lane < 8 && n < N) out[n] = (f16)v;
        } else {
            if (lane < 8) red[((nb * RB + b) * SK + kw) * 8 + lane] = v;
        }
    }
    if constexpr (SK > 1) {
        __syncthreads();
        if (kw != 0 || lane >= 8) return;
#pragma unroll
        for (int b = 0; b < RB; ++b) {
            float v = red[((nb * RB + b) * SK) * 8 + lane];
#pragma unroll
            for (int s = 1; s < SK; ++s) v += red[((nb * RB + b) * SK + s) * 8 + lane];
            const int n = nw + 8 * b + lane;
            if (n < N) out[n] = (f16)v;
        }
    }
}

}  // namespace w4a16

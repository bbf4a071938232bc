// Paired-group MFMA GEMV for small batches (M = 2..8) on gfx950. Kept apart
// from w4a16_kernels.h so its instantiations build in their own translation
// unit (w4a16_pair.hip).
#pragma once

#include "w4a16_device.h"

namespace w4a16 {

// ---------------------------------------------------------------------------
// Paired-group MFMA kernel for small batches (runtime M = 2..8), G = 128,
// activations staged in LDS (K up to 8192 at M = 8).
//
// The 16x16x32 MFMA has 16 A rows for M <= 8 activation rows, so its A rows
// hold the activation rows twice, for the two groups of a group pair, and its
// 16 B columns are 8 weight rows x the same two groups: lane l = 16 q + c
// supplies weight row c & 7, group 2 p + (c >> 3) of pair p, bytes 16 q ..
// 16 q + 15 of that group. One load instruction then reads 8 rows x 128
// contiguous bytes (whole cache lines), which MI355X streams as fast as 1 KiB
// contiguous loads; the 16 rows x 64 bytes of a plain MFMA tile read 10-55%
// slower (pure reads at 4096 x 14336 / 8192 x 8192: 5.9 / 8.8 us against
// 7.0 / 12.8 us). D[i][c] is a wanted product when i and c lie in the same
// half (i, c < 8: group 2 p; i, c >= 8: group 2 p + 1); the cross-half blocks
// are dropped, and the halves of an output, in lanes l and l + 40, are added
// in the final LDS reduction.
//
// Workgroup = SK x SN wavefronts; wavefront (kw, nb) takes RB blocks of 8
// rows and pairs kw, kw + SK, ... (GPW of them), so each A fragment read from
// LDS feeds RB MFMAs. Loads are issued up front and the offset decode is that
// of gemv_mfma_oneshot (codes without fix-ups in B, pos-1 activations scaled
// by 1/16 in A, each chain started from the staged per-(group, row) bias).
//
// Staged activations: 16-byte unit (m, g, t, q) (activation row m, k = 128 g
// + 32 q + 8 t .. + 7) at line ((g >> 1) * 4 + t) * 4 + q, slot (m + MS (g & 1)
// + 4 q + t) mod 2 MS of a line of 2 MS units (MS = 4 row slots for M <= 4, 8
// for M <= 8). Staging writes (16 lanes: one (m, g), all (q, t)) and fragment
// reads (16 lanes: one (q, t), all (m, g & 1)) then fall on distinct bank
// slots, where the row-stride layout of gemv_mfma_oneshot conflicts up to
// 8-way on the writes. The staged pairs are padded with zeros up to SK * GPW
// so the fragment reads of every step are a fixed offset from a per-lane
// base (no clamps).
// ---------------------------------------------------------------------------
__host__ __device__ constexpr int pair_row_slots(int M) { return M <= 4 ? 4 : 8; }

// LDS of gemv_mfma_pair: staged units of `pairs` group pairs (>= (G + 1) / 2;
// pairs past the last group and a missing odd group are zero-filled so the
// fragment reads need no clamp), the fp32 bias of every group of those pairs,
// and one f32x4 per lane, block and wavefront for the final reduction.
__host__ __device__ constexpr int64_t pair_lds_bytes(int64_t M, int64_t pairs, int64_t waves, int64_t rb) {
    return pairs * 16 * (2 * pair_row_slots((int)M)) * 16 + pairs * 2 * 64 + waves * rb * 64 * 16;
}

template <int SK, int SN, int RB, int GPW, int MS>
__global__ void __launch_bounds__(64 * SK * SN)
gemv_mfma_pair(const f16* __restrict__ x, const uint8_t* __restrict__ w, const f16* __restrict__ scales,
               f16* __restrict__ out, int M, int N, int K) {
    constexpr int S = SK * SN;
    constexpr int T = 64 * S;
    constexpr int kFirst = 8;
    constexpr int LS = 2 * MS;               // units per line
    constexpr int P = SK * GPW;              // staged pairs
    extern __shared__ __align__(16) uint8_t smem[];
    const int G = K >> 7;
    u32x4* xs = reinterpret_cast<u32x4*>(smem);                                  // [P * 16][LS] units
    float* base = reinterpret_cast<float*>(smem + P * 16 * LS * 16);             // [2 P][16] fp32
    f32x4* red = reinterpret_cast<f32x4*>(smem + P * 16 * LS * 16 + P * 2 * 64); // [S][RB][64]
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int col = lane & 15, q = lane >> 4;
    const int brow = col & 7, bhalf = col >> 3;
    const int kw = wave % SK, nb = wave / SK;
    const int n0 = (blockIdx.x * SN + nb) * RB * 8;
    const uint32_t row_bytes = (uint32_t)(K >> 1);
    auto group = [&](int j, int h) { return 2 * (kw + SK * j) + h; };

    // 1. activation units (8 halves): i = m * K/8 + uk
    const int upr = K >> 3;
    const int units = M * upr;
    const float inv_upr = 1.0f / (float)upr;
    u32x4 a[kFirst];
#pragma unroll
    for (int p = 0; p < kFirst; ++p) {
        const int i = min((int)threadIdx.x + p * T, units - 1);
        a[p] = *reinterpret_cast<const u32x4*>(x + (size_t)i * 8);
    }
    // 2. scales and weights of every (pair, block): clamped addresses, groups
    // past G weighted 0 below
    const uint16_t* sbase = reinterpret_cast<const uint16_t*>(scales);
    uint32_t sv[GPW][RB];
    u32x4 wv[GPW][RB];
#pragma unroll
    for (int j = 0; j < GPW; ++j)
#pragma unroll
        for (int b = 0; b < RB; ++b) {
            const int n = min(n0 + 8 * b + brow, N - 1);
            sv[j][b] = sbase[(size_t)n * G + min(group(j, bhalf), G - 1)];
        }
#pragma unroll
    for (int j = 0; j < GPW; ++j)
#pragma unroll
        for (int b = 0; b < RB; ++b) {
            const int n = min(n0 + 8 * b + brow, N - 1);
            wv[j][b] = load_stream(reinterpret_cast<const u32x4*>(
                w + (size_t)n * row_bytes + (uint32_t)min(group(j, bhalf), G - 1) * 64u + q * 16));
        }
    __builtin_amdgcn_sched_barrier(0);

    // 3. stage A units and the per-(group, row) bias; zero the padding groups
    const f16x2 sixteenth = {(f16)0.0625f, (f16)0.0625f};
    const f16x2 b0 = {(f16)1032.0f, (f16)1032.0f};
    const f16x2 b1 = {(f16)1152.0f, (f16)1152.0f};
    auto put = [&](int i, u32x4 v, bool valid) {
        // m = i / upr, exact: (i + 1/2) / upr is at least 1 / (2 upr) away from an integer
        const int m = (int)(((float)i + 0.5f) * inv_upr);
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
        // the 16 units of (m, g) sit in 16 consecutive lanes (a DPP row)
        c += dpp<0xB1>(c);
        c += dpp<0x4E>(c);
        c += dpp<0x141>(c);
        c += dpp<0x140>(c);
        if (valid) {
            xs[(((g >> 1) * 4 + t) * 4 + qq) * LS + ((m + MS * (g & 1) + 4 * qq + t) & (LS - 1))] = pv;
            if ((uk & 15) == 0) base[g * 16 + m] = -c;
        }
    };
#pragma unroll
    for (int p = 0; p < kFirst; ++p) {
        const int i = threadIdx.x + p * T;
        put(min(i, units - 1), a[p], i < units);
    }
    for (int i0 = threadIdx.x + kFirst * T; i0 < ((units + T - 1) / T) * T; i0 += T) {
        const int i = min(i0, units - 1);
        put(i, *reinterpret_cast<const u32x4*>(x + (size_t)i * 8), i0 < units);
    }
    {
        // groups G .. 2P - 1: every (t, q) line slot of those groups' row slots
        const int pad_units = (2 * P - G) * 16 * MS;
        const u32x4 zero4 = {0u, 0u, 0u, 0u};
        for (int i = threadIdx.x; i < pad_units; i += T) {
            const int g = G + i / (16 * MS);
            const int r = i % (16 * MS);
            const int m = r / 16, uk = r % 16, qq = uk >> 2, t = uk & 3;
            xs[(((g >> 1) * 4 + t) * 4 + qq) * LS + ((m + MS * (g & 1) + 4 * qq + t) & (LS - 1))] = zero4;
        }
        for (int i = threadIdx.x; i < (2 * P - G) * 16; i += T) base[G * 16 + i] = 0.0f;
    }
    __syncthreads();

    // 4. pairs: A fragments of pair j+1 read while pair j runs on the MFMAs.
    // A row `col` = activation row arow of group group(j, bhalf); D rows 4 q ..
    // 4 q + 3 = activation rows dm .. dm + 3 of group group(j, q >> 1).
    const int arow = brow % M;
    const u32x4* xlane = xs + (kw * 16 + q) * LS;
    int toff[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) toff[t] = 4 * t * LS + ((arow + MS * bhalf + 4 * q + t) & (LS - 1));
    const float* blane = base + (2 * kw + (q >> 1)) * 16 + 4 * (q & 1);
    auto fetch = [&](u32x4 (&av)[4], f32x4& bv, int j) {
#pragma unroll
        for (int t = 0; t < 4; ++t) av[t] = xlane[j * SK * 16 * LS + toff[t]];
        bv = *reinterpret_cast<const f32x4*>(blane + j * SK * 32);
    };
    f32x4 acc[RB];
#pragma unroll
    for (int b = 0; b < RB; ++b) acc[b] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
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
        const bool in_range = group(j, bhalf) < G;
#pragma unroll
        for (int b = 0; b < RB; ++b) {
            f32x4 d = cb;
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const Codes8 cw = unpack8_offset(wv[j][b][t]);
                const f16x8 bt = __builtin_bit_cast(
                    f16x8, (u32x4){as_u32(cw.p[0]), as_u32(cw.p[1]), as_u32(cw.p[2]), as_u32(cw.p[3])});
                d = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, cur[t]), bt, d, 0, 0, 0);
            }
            const float sc = in_range ? (float)__builtin_bit_cast(f16, (uint16_t)sv[j][b]) : 0.0f;
            acc[b] = d * sc + acc[b];
        }
    }

    // 5. reduce the SK partial tiles and the two halves (lane l + 40 onto
    // lane l, q < 2, c < 8), store rows m < M
#pragma unroll
    for (int b = 0; b < RB; ++b) red[(wave * RB + b) * 64 + lane] = acc[b];
    __syncthreads();
    if (kw != 0 || q >= 2 || col >= 8) return;
#pragma unroll
    for (int b = 0; b < RB; ++b) {
        f32x4 v = acc[b] + red[(wave * RB + b) * 64 + lane + 40];
#pragma unroll
        for (int s2 = 1; s2 < SK; ++s2)
            v += red[((wave + s2) * RB + b) * 64 + lane] + red[((wave + s2) * RB + b) * 64 + lane + 40];
        const int nn = n0 + 8 * b + col;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int m = q * 4 + e;
            if (m < M && nn < N) out[(size_t)m * N + nn] = (f16)v[e];
        }
    }
}

}  // namespace w4a16

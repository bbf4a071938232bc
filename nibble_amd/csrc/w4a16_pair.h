// Paired-group MFMA GEMV for small batches (M = 2..8) on gfx950. Kept apart
// from w4a16_kernels.h so its instantiations build in their own translation
// unit (w4a16_pair.hip).
#pragma once

#include "w4a16_device.h"

namespace w4a16 {

// ---------------------------------------------------------------------------
// Paired-group MFMA kernel for small batches (runtime M = 2..8), G = 128,
// activations staged in LDS, whole or in chunks of group pairs.
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
// for M <= 8), g counted within the staged chunk. Staging writes (16 lanes:
// one (m, g), all (q, t)) and fragment reads (16 lanes: one (q, t), all (m,
// g & 1)) then fall on distinct bank slots, where the row-stride layout of
// gemv_mfma_oneshot conflicts up to 8-way on the writes. Groups past K are
// staged as zeros (weight 0), so the fragment reads of every step are a fixed
// offset from a per-lane base (no clamps).
//
// MB: the per-(group, row) bias comes from 4 more MFMAs per step (A against
// the constant -(1032, 1032, 1152, 1152, ...), shared by the RB blocks)
// instead of staging dot products and an LDS table.
//
// 16 row slots (M = 9..16): the A rows are the activation rows of one group,
// so a step runs two MFMAs against the same B (the pair's two groups); a
// lane keeps the D of the MFMA whose group matches its B column, and the
// halves of an output sit in lanes l and l + 8. These put the dequantized
// weights in B (exact codes times the group scale, rounded to fp16 once, as
// w4a16_dequantize_f16 writes them; activations staged unscaled, no bias)
// and accumulate in the MFMA: the result is the reference's prefill path
// (dequantize, fp16 GEMM with fp32 accumulation) up to summation order,
// where an fp32 scale applied to per-group sums of codes, or the offset
// decode's sums of ~1032 |x|, would miss its 1e-3 tolerance.
//
// Chunks (C pairs < SK * GPW): rows too long for LDS are staged C pairs at a
// time into two alternating buffers, one barrier per chunk: chunk c + 1 is
// written to the other buffer after chunk c's MFMAs. Loads are requested
// chunk by chunk (activations, then that chunk's scales and weights), the
// first LA chunks up front and chunk c + LA when chunk c starts.
// ---------------------------------------------------------------------------
__host__ __device__ constexpr int pair_row_slots(int M) { return M <= 4 ? 4 : M <= 8 ? 8 : 16; }

// LDS of gemv_mfma_pair: one or two buffers (one when a single chunk of
// `chunk` pairs covers the `pairs` a workgroup steps over) of staged units
// and fp32 per-(group, row) biases, then one f32x4 per lane, block and
// wavefront for the final reduction.
__host__ __device__ constexpr int64_t pair_lds_bytes(int64_t M, int64_t pairs, int64_t chunk, int64_t waves,
                                                     int64_t rb) {
    return (chunk < pairs ? 2 : 1) * (chunk * 16 * (2 * pair_row_slots((int)M)) * 16 + chunk * 2 * 64) +
           waves * rb * 64 * 16;
}

template <int SK, int SN, int RB, int GPW, int MS, int C, int LA = 64, bool MB = false, bool SILU = false>
__global__ void __launch_bounds__(64 * SK * SN)
gemv_mfma_pair(const f16* __restrict__ x, const uint8_t* __restrict__ w, const f16* __restrict__ scales,
               f16* __restrict__ out, int M, int N, int K) {
    constexpr int S = SK * SN;
    constexpr int T = 64 * S;
    constexpr int LS = 2 * MS;                 // units per line
    constexpr int P = SK * GPW;                // pairs the workgroup steps over
    static_assert(C % SK == 0 && C <= P, "a chunk is a whole number of steps");
    static_assert(LA >= 1, "at least the first chunk is requested up front");
    static_assert(MS == 4 || MS == 8 || MS == 16, "4, 8 or 16 row slots");
    static_assert(MS != 16 || !MB, "16 row slots take the bias from the staging");
    static_assert(!SILU || (MS == 16 && RB == 2), "the SiLU-multiply form pairs a gate block and its up block");
    constexpr bool W16 = MS == 16;   // M = 9..16: one activation group per MFMA, two MFMAs per step, exact decode
    constexpr int H = W16 ? 2 : 1;   // A fragment sets per step
    constexpr int NC = (P + C - 1) / C;        // chunks
    constexpr int NB = NC > 1 ? 2 : 1;         // staging buffers
    constexpr int JPC = C / SK;                // steps per chunk
    constexpr int CU = 2 * C * 16;             // staged units per activation row per chunk
    constexpr int UPT = (MS * CU + T - 1) / T; // staging units per thread per chunk (M <= MS)
    constexpr int XS = C * 16 * LS;            // units per staging buffer
    extern __shared__ __align__(16) uint8_t smem[];
    const int G = K >> 7;
    u32x4* xs = reinterpret_cast<u32x4*>(smem);                                       // [NB][XS] units
    float* base = reinterpret_cast<float*>(smem + NB * XS * 16);                     // [NB][2 C][16] fp32
    f32x4* red = reinterpret_cast<f32x4*>(smem + NB * XS * 16 + NB * C * 2 * 64);   // [S][RB][64]
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int col = lane & 15, q = lane >> 4;
    const int brow = col & 7, bhalf = col >> 3;
    const int kw = wave % SK, nb = wave / SK;
    constexpr int RO = SILU ? 1 : RB;   // output blocks of 8 rows per wavefront
    const int n0 = (blockIdx.x * SN + nb) * RO * 8;
    // weight row of block b for this lane: SILU (N = inter, 2 inter weight
    // rows) takes gate row n and up row inter + n of the same output column
    auto wrow = [&](int b) -> int {
        if constexpr (SILU) return (b ? N : 0) + min(n0 + brow, N - 1);
        else return min(n0 + 8 * b + brow, N - 1);
    };
    const uint32_t row_bytes = (uint32_t)(K >> 1);
    const int upr = K >> 3;                    // 16-byte units per activation row
    auto group = [&](int j, int h) { return 2 * (kw + SK * j) + h; };

    // staging unit i of chunk c: activation row i / CU, unit i % CU of the
    // chunk's 2 C groups; units of groups past K and rows past M read x[0]
    auto load_chunk = [&](u32x4 (&a)[UPT], int c) {
#pragma unroll
        for (int p = 0; p < UPT; ++p) {
            const int i = threadIdx.x + p * T;
            const int m = i / CU, ul = i % CU;
            const int g = 2 * c * C + (ul >> 4);
            const bool valid = m < M && g < G;
            a[p] = *reinterpret_cast<const u32x4*>(x + (valid ? ((size_t)m * upr + (size_t)g * 16 + (ul & 15)) * 8 : 0));
        }
    };
    const f16x2 sixteenth = {(f16)0.0625f, (f16)0.0625f};
    const f16x2 b0 = {(f16)1032.0f, (f16)1032.0f};
    const f16x2 b1 = {(f16)1152.0f, (f16)1152.0f};
    auto put_chunk = [&](const u32x4 (&a)[UPT], int c, int buf) {
        u32x4* xb = xs + buf * XS;
        float* bb = base + buf * C * 32;
#pragma unroll
        for (int p = 0; p < UPT; ++p) {
            const int i = threadIdx.x + p * T;
            const int m = i / CU, ul = i % CU;
            const int gl = ul >> 4, qq = (ul >> 2) & 3, t = ul & 3;
            const bool zero = 2 * c * C + gl >= G;
            u32x4 pv = permute8(a[p]);
            if (!W16) {
                pv.y = as_u32(as_f16x2(pv.y) * sixteenth);
                pv.w = as_u32(as_f16x2(pv.w) * sixteenth);
            }
            if (zero) pv = (u32x4){0u, 0u, 0u, 0u};
            float cs = 0.0f;
            if (!MB && !W16) {
                cs = __builtin_amdgcn_fdot2(as_f16x2(pv.x), b0, cs, false);
                cs = __builtin_amdgcn_fdot2(as_f16x2(pv.y), b1, cs, false);
                cs = __builtin_amdgcn_fdot2(as_f16x2(pv.z), b0, cs, false);
                cs = __builtin_amdgcn_fdot2(as_f16x2(pv.w), b1, cs, false);
                // the 16 units of (m, g) sit in 16 consecutive lanes (a DPP row)
                cs += dpp<0xB1>(cs);
                cs += dpp<0x4E>(cs);
                cs += dpp<0x141>(cs);
                cs += dpp<0x140>(cs);
            }
            if (m < M) {
                xb[(((gl >> 1) * 4 + t) * 4 + qq) * LS + ((m + MS * (gl & 1) + 4 * qq + t) & (LS - 1))] = pv;
                if (!MB && !W16 && (ul & 15) == 0) bb[gl * 16 + m] = -cs;
            }
        }
    };

    // 1. loads, chunk by chunk in the order they are consumed: a chunk's
    // activations, then its steps' scales and weights (clamped addresses;
    // groups past K weighted 0 below). The first LA chunks are requested up
    // front and chunk c + LA at the start of chunk c, so a chunk's
    // activations never queue behind weights of much later chunks (a
    // wavefront's loads return in issue order).
    const uint16_t* sbase = reinterpret_cast<const uint16_t*>(scales);
    u32x4 a[NC][UPT];
    uint32_t sv[GPW][RB];
    u32x4 wv[GPW][RB];
    auto issue = [&](int cc) {
        load_chunk(a[cc], cc);
        __builtin_amdgcn_sched_barrier(0);   // keep the activations ahead of the weights
#pragma unroll
        for (int jl = 0; jl < JPC; ++jl) {
            const int j = cc * JPC + jl;
            if (j < GPW) {
#pragma unroll
                for (int b = 0; b < RB; ++b) {
                    const int n = wrow(b);
                    sv[j][b] = sbase[(size_t)n * G + min(group(j, bhalf), G - 1)];
                }
            }
        }
#pragma unroll
        for (int jl = 0; jl < JPC; ++jl) {
            const int j = cc * JPC + jl;
            if (j < GPW) {
#pragma unroll
                for (int b = 0; b < RB; ++b) {
                    const int n = wrow(b);
                    wv[j][b] = load_stream(reinterpret_cast<const u32x4*>(
                        w + (size_t)n * row_bytes + (uint32_t)min(group(j, bhalf), G - 1) * 64u + q * 16));
                }
            }
        }
    };
#pragma unroll
    for (int cc = 0; cc < NC && cc < LA; ++cc) issue(cc);
    __builtin_amdgcn_sched_barrier(0);
    put_chunk(a[0], 0, 0);
    __syncthreads();

    // 2. chunks of pairs: A fragments of step j+1 read while step j runs on
    // the MFMAs. A row `col` = activation row arow of group group(j, bhalf);
    // D rows 4 q .. 4 q + 3 = activation rows dm .. dm + 3 of group
    // group(j, q >> 1).
    // M <= 8: A row `col` = activation row arow of group group(j, bhalf).
    // M > 8 (16 row slots): A row `col` = activation row col of group
    // group(j, h) in the step's h-th MFMA; B columns col < 8 hold group
    // group(j, 0) and col >= 8 group group(j, 1), so a lane keeps the D of
    // the MFMA whose group matches its B column.
    const int arow = W16 ? col % M : brow % M;
    int toff[H][4];
#pragma unroll
    for (int h = 0; h < H; ++h)
#pragma unroll
        for (int t = 0; t < 4; ++t)
            toff[h][t] = (kw * 16 + q) * LS + 4 * t * LS + ((arow + MS * (W16 ? h : bhalf) + 4 * q + t) & (LS - 1));
    const int boff = W16 ? 2 * kw * 16 + 4 * q : (2 * kw + (q >> 1)) * 16 + 4 * (q & 1);
    f32x4 acc[RB];
#pragma unroll
    for (int b = 0; b < RB; ++b) acc[b] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const int buf = c % NB;
        const u32x4* xb = xs + buf * XS;
        const float* bb = base + buf * C * 32;
        if (c + LA < NC) issue(c + LA);
        auto fetch = [&](u32x4 (&av)[H][4], f32x4 (&bv)[H], int jl) {
#pragma unroll
            for (int h = 0; h < H; ++h) {
#pragma unroll
                for (int t = 0; t < 4; ++t) av[h][t] = xb[jl * SK * 16 * LS + toff[h][t]];
                if (!MB && !W16) bv[h] = *reinterpret_cast<const f32x4*>(bb + jl * SK * 32 + boff + 16 * h);
            }
        };
        const int steps = (c + 1) * JPC <= GPW ? JPC : GPW - c * JPC;
        u32x4 A0[H][4], A1[H][4];
        f32x4 B0[H], B1[H];
#pragma unroll
        for (int h = 0; h < H; ++h) B0[h] = B1[h] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
        fetch(A0, B0, 0);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int jl = 0; jl < JPC; ++jl) {
            if (jl < steps) {
                const int j = c * JPC + jl;
                u32x4 (&curh)[H][4] = (jl & 1) ? A1 : A0;
                u32x4 (&nxt)[H][4] = (jl & 1) ? A0 : A1;
                f32x4 (&cbh)[H] = (jl & 1) ? B1 : B0;
                f32x4 (&nbv)[H] = (jl & 1) ? B0 : B1;
                u32x4 (&cur)[4] = curh[0];
                f32x4& cb = cbh[0];
                if (jl + 1 < steps) fetch(nxt, nbv, jl + 1);
                __builtin_amdgcn_sched_barrier(0);
                const bool in_range = group(j, bhalf) < G;
                if (MB) {
                    // the bias rows on the matrix cores: A against the
                    // constant -(1032, 1032, 1152, 1152, ...) of the offset
                    // decode (exact products, fp32 sums)
                    const f16x8 cneg = {(f16)-1032.0f, (f16)-1032.0f, (f16)-1152.0f, (f16)-1152.0f,
                                        (f16)-1032.0f, (f16)-1032.0f, (f16)-1152.0f, (f16)-1152.0f};
                    f32x4 db = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                    for (int t = 0; t < 4; ++t)
                        db = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, cur[t]), cneg, db, 0, 0,
                                                                    0);
                    cb = db;
                }
#pragma unroll
                for (int b = 0; b < RB; ++b) {
                    // 16 row slots: B = fp16_rn(code * scale), the dequantized
                    // weights bit for bit (scale 0 past K), summed unscaled
                    const f16 sc16 = in_range ? __builtin_bit_cast(f16, (uint16_t)sv[j][b]) : (f16)0.0f;
                    const f16x2 sc2 = {sc16, sc16};
                    f32x4 dh[H];
#pragma unroll
                    for (int h = 0; h < H; ++h) dh[h] = W16 ? acc[b] : cbh[h];
#pragma unroll
                    for (int t = 0; t < 4; ++t) {
                        Codes8 cw = W16 ? unpack8(wv[j][b][t]) : unpack8_offset(wv[j][b][t]);
                        if (W16) {
#pragma unroll
                            for (int e = 0; e < 4; ++e) cw.p[e] = cw.p[e] * sc2;
                        }
                        const f16x8 bt = __builtin_bit_cast(
                            f16x8, (u32x4){as_u32(cw.p[0]), as_u32(cw.p[1]), as_u32(cw.p[2]), as_u32(cw.p[3])});
#pragma unroll
                        for (int h = 0; h < H; ++h)
                            dh[h] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, curh[h][t]), bt,
                                                                           dh[h], 0, 0, 0);
                    }
                    if (W16) {
                        acc[b] = bhalf ? dh[H - 1] : dh[0];
                    } else {
                        const float sc = in_range ? (float)sc16 : 0.0f;
                        acc[b] = dh[0] * sc + acc[b];
                    }
                }
            }
        }
        if (c + 1 < NC) {
            put_chunk(a[c + 1], c + 1, (c + 1) % NB);
            __syncthreads();
        }
    }

    // 3. reduce the SK partial tiles and the two halves (lane l + 40 onto
    // lane l, q < 2, c < 8; with 16 row slots lane l + 8 onto lane l, c < 8),
    // store rows m < M
    constexpr int HALF = W16 ? 8 : 40;
#pragma unroll
    for (int b = 0; b < RB; ++b) red[(wave * RB + b) * 64 + lane] = acc[b];
    __syncthreads();
    if (kw != 0 || (!W16 && q >= 2) || col >= 8) return;
    f32x4 v[RB];
#pragma unroll
    for (int b = 0; b < RB; ++b) {
        v[b] = acc[b] + red[(wave * RB + b) * 64 + lane + HALF];
#pragma unroll
        for (int s2 = 1; s2 < SK; ++s2)
            v[b] += red[((wave + s2) * RB + b) * 64 + lane] + red[((wave + s2) * RB + b) * 64 + lane + HALF];
    }
#pragma unroll
    for (int b = 0; b < RO; ++b) {
        const int nn = n0 + 8 * b + col;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int m = q * 4 + e;
            if (m < M && nn < N) out[(size_t)m * N + nn] = SILU ? gemm_silu_mul(v[0][e], v[1][e]) : (f16)v[b][e];
        }
    }
}

}  // namespace w4a16

namespace w4a16 {

// ---------------------------------------------------------------------------
// Streaming paired-group MFMA kernel (runtime M = 2..8, whole rows staged).
//
// The paired kernel above stages all M K activations in every workgroup, so
// a layer of N rows in workgroups of R rows stages them N / R times; with
// wide layers (N >> 256 R) that staging costs as much as the weights. Here
// the grid is at most the workgroups resident at once: each workgroup stages
// the activations once (the layout and per-(group, row) biases of the kernel
// above) and its W wavefronts then stream 8-row blocks (tasks, dealt
// round-robin over the grid's wavefronts) pair by pair, each wavefront over
// whole rows, with D pairs of loads in flight in a ring of registers (one
// 1 KiB load of 8 rows x 128 bytes and one scale per lane per pair). A
// wavefront folds the two halves of its tile (lane l + 40 onto lane l) with
// a lane shuffle and stores its block, so there is no barrier after the
// staging. The loop's tail is peeled, so no load sits behind a branch; a
// wavefront with no task requests D pairs of the grid's last block and
// stores nothing.
//
// SPLIT (split K, for rows whose M K activations do not fit in LDS): the
// pairs of a row are cut into S slices of ceil(P / S) pairs; workgroup b
// takes slice b mod S (it stages only that slice's activations) and the
// tasks of that slice with its gridDim / S peers, and stores fp32 partial
// sums to part[slice][m][n]; pair_split_reduce adds the S slices in slice
// order and rounds to fp16.
// ---------------------------------------------------------------------------
__host__ __device__ constexpr int64_t pair_stream_lds_bytes(int64_t M, int64_t pairs) {
    return pairs * 16 * (2 * pair_row_slots((int)M)) * 16 + pairs * 2 * 64;
}

template <int MS, int D, bool SPLIT = false>
__global__ void __launch_bounds__(1024)
gemv_pair_stream(const f16* __restrict__ x, const uint8_t* __restrict__ w, const f16* __restrict__ scales,
                 f16* __restrict__ out, int M, int N, int K, float* __restrict__ part, int S) {
    constexpr int LS = 2 * MS;   // units per line
    constexpr int B = 8;         // staging units per thread requested at a time
    extern __shared__ __align__(16) uint8_t smem[];
    const int Gall = K >> 7;                                                 // groups per row
    const int Pall = (Gall + 1) >> 1;                                        // pairs per row
    int sl = 0, peer = blockIdx.x, peers = gridDim.x, pair0 = 0, P = Pall;
    if (SPLIT) {   // slice sl: pairs pair0 .. pair0 + P - 1 (the host keeps every slice non-empty)
        const int PS = (Pall + S - 1) / S;
        sl = blockIdx.x % S;
        peer = blockIdx.x / S;
        peers = gridDim.x / S;
        pair0 = sl * PS;
        P = min(PS, Pall - pair0);
    }
    const int g0 = 2 * pair0;              // first group of the slice
    const int G = min(2 * P, Gall - g0);   // groups of the slice
    u32x4* xs = reinterpret_cast<u32x4*>(smem);                              // [P * 16 lines][LS]
    float* base = reinterpret_cast<float*>(smem + (size_t)P * 16 * LS * 16); // [2 P][16]
    const int T = blockDim.x;
    const int W = T >> 6;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int col = lane & 15, q = lane >> 4;
    const int brow = col & 7, bhalf = col >> 3;
    const uint32_t row_bytes = (uint32_t)(K >> 1);
    const int upr = K >> 3;            // 16-byte units per activation row
    const int CU = 32 * P;             // staged units per activation row (2 P groups x 16)
    const int NB = (N + 7) >> 3;       // 8-row blocks
    const int task0 = peer * W + wave;
    const int stride = peers * W;
    const int my_tasks = task0 < NB ? (NB - 1 - task0) / stride + 1 : 0;
    const int units = my_tasks * P;

    // staging unit i: activation row i / CU, unit i % CU; units of groups
    // past K and rows past M read x[0]; every 16 consecutive units are one
    // (row, group) and sit in one DPP row of 16 lanes
    const f16x2 sixteenth = {(f16)0.0625f, (f16)0.0625f};
    const f16x2 b0 = {(f16)1032.0f, (f16)1032.0f};
    const f16x2 b1 = {(f16)1152.0f, (f16)1152.0f};
    auto stage_load = [&](u32x4 (&a)[B], int first) {
#pragma unroll
        for (int p = 0; p < B; ++p) {
            const int i = first + (int)threadIdx.x + p * T;
            const int m = i / CU, ul = i % CU;
            const int g = ul >> 4;
            const bool valid = m < M && g < G && i < MS * CU;
            a[p] = *reinterpret_cast<const u32x4*>(
                x + (valid ? ((size_t)m * upr + (size_t)(g0 + g) * 16 + (ul & 15)) * 8 : 0));
        }
    };
    auto stage_put = [&](const u32x4 (&a)[B], int first) {
#pragma unroll
        for (int p = 0; p < B; ++p) {
            const int i = first + (int)threadIdx.x + p * T;
            const int m = i / CU, ul = i % CU;
            const int gl = ul >> 4, qq = (ul >> 2) & 3, t = ul & 3;
            u32x4 pv = permute8(a[p]);
            pv.y = as_u32(as_f16x2(pv.y) * sixteenth);
            pv.w = as_u32(as_f16x2(pv.w) * sixteenth);
            if (gl >= G) pv = (u32x4){0u, 0u, 0u, 0u};
            float cs = 0.0f;
            cs = __builtin_amdgcn_fdot2(as_f16x2(pv.x), b0, cs, false);
            cs = __builtin_amdgcn_fdot2(as_f16x2(pv.y), b1, cs, false);
            cs = __builtin_amdgcn_fdot2(as_f16x2(pv.z), b0, cs, false);
            cs = __builtin_amdgcn_fdot2(as_f16x2(pv.w), b1, cs, false);
            cs += dpp<0xB1>(cs);
            cs += dpp<0x4E>(cs);
            cs += dpp<0x141>(cs);
            cs += dpp<0x140>(cs);
            if (m < M && i < MS * CU) {
                xs[(((gl >> 1) * 4 + t) * 4 + qq) * LS + ((m + MS * (gl & 1) + 4 * qq + t) & (LS - 1))] = pv;
                if ((ul & 15) == 0) base[gl * 16 + m] = -cs;
            }
        }
    };

    // ring of D pairs in flight: unit (task, pair); 32-bit byte offsets (the
    // host checks that the weights are below 4 GiB)
    u32x4 wv[D];
    uint32_t sv[D];
    const uint8_t* sbytes = reinterpret_cast<const uint8_t*>(scales);
    auto load = [&](int d, int task, int pr) {
        const uint32_t n = (uint32_t)min(task * 8 + brow, N - 1);
        const uint32_t gi = (uint32_t)min(g0 + 2 * pr + bhalf, Gall - 1);
        sv[d] = *reinterpret_cast<const uint16_t*>(sbytes + (n * (uint32_t)Gall + gi) * 2u);
        wv[d] = load_stream(reinterpret_cast<const u32x4*>(w + (n * row_bytes + gi * 64u + (uint32_t)q * 16u)));
    };

    // 1. the first staging batch, then the ring's first D pairs, then the rest
    // of the staging (a wavefront's loads return in issue order)
    const int total = MS * CU;
    int lt = min(task0, NB - 1), lp = 0;   // next unit to request
    {
        u32x4 a[B];
        stage_load(a, 0);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int d = 0; d < D; ++d) {
            load(d, lt, lp);
            if (++lp == P) { lp = 0; lt += stride; }
        }
        __builtin_amdgcn_sched_barrier(0);
        stage_put(a, 0);
        for (int first = B * T; first < total; first += B * T) {
            stage_load(a, first);
            stage_put(a, first);
        }
    }
    __syncthreads();
    if (units == 0) return;

    // 2. stream: per pair 4 A fragments and the bias from LDS, 4 MFMAs
    const int arow = brow % M;
    int toff[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) toff[t] = q * LS + 4 * t * LS + ((arow + MS * bhalf + 4 * q + t) & (LS - 1));
    const int boff = (q >> 1) * 16 + 4 * (q & 1);
    f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    int ct = task0, cp = 0;   // unit being computed

    auto compute = [&](int d) {
        u32x4 av[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) av[t] = xs[cp * 16 * LS + toff[t]];
        f32x4 dv = *reinterpret_cast<const f32x4*>(base + cp * 32 + boff);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const Codes8 cw = unpack8_offset(wv[d][t]);
            const f16x8 bt = __builtin_bit_cast(
                f16x8, (u32x4){as_u32(cw.p[0]), as_u32(cw.p[1]), as_u32(cw.p[2]), as_u32(cw.p[3])});
            dv = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, av[t]), bt, dv, 0, 0, 0);
        }
        const float sc = 2 * cp + bhalf < G ? (float)__builtin_bit_cast(f16, (uint16_t)sv[d]) : 0.0f;
        acc = dv * sc + acc;
        if (cp == P - 1) {
            // fold the two halves (lane l + 40 onto lane l, q < 2, col < 8) and store
            f32x4 v;
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = acc[e] + __shfl(acc[e], (lane + 40) & 63);
            const int nn = ct * 8 + col;
            if (q < 2 && col < 8 && nn < N) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int m = 4 * q + e;
                    if (m < M) {
                        if (SPLIT)
                            part[((size_t)sl * M + m) * N + nn] = v[e];
                        else
                            out[(size_t)m * N + nn] = (f16)v[e];
                    }
                }
            }
            acc = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
            cp = 0;
            ct += stride;
        } else {
            ++cp;
        }
    };

    int u = 0;
    if (units >= D) {
        for (; u + 2 * D <= units; u += D) {
#pragma unroll
            for (int d = 0; d < D; ++d) {
                compute(d);
                load(d, lt, lp);
                if (++lp == P) { lp = 0; lt += stride; }
            }
        }
#pragma unroll
        for (int d = 0; d < D; ++d) {
            compute(d);
            if (u + D + d < units) {
                load(d, lt, lp);
                if (++lp == P) { lp = 0; lt += stride; }
            }
        }
#pragma unroll
        for (int d = 0; d < D; ++d)
            if (u + D + d < units) compute(d);
    } else {
#pragma unroll
        for (int d = 0; d < D; ++d)
            if (d < units) compute(d);
    }
}

// out[i] = fp16(part[0][i] + part[1][i] + ... + part[S - 1][i]) over the
// MN = M N outputs, 4 per thread (16-byte loads when MN % 4 == 0). S is a
// template argument so that a thread's S loads are all requested before the
// first add (a runtime loop would wait for each in turn).
template <int S>
__global__ void __launch_bounds__(256)
pair_split_reduce(const float* __restrict__ part, f16* __restrict__ out, int MN) {
    const int i = (blockIdx.x * 256 + threadIdx.x) * 4;
    if (i >= MN) return;
    // 8-byte stores need whole quads and an 8-byte aligned output (the C ABI
    // asks only for 2-byte alignment)
    if ((MN & 3) == 0 && (reinterpret_cast<uintptr_t>(out) & 7u) == 0) {
        f32x4 v[S];
#pragma unroll
        for (int s = 0; s < S; ++s) v[s] = *reinterpret_cast<const f32x4*>(part + (size_t)s * MN + i);
        f32x4 acc = v[0];
#pragma unroll
        for (int s = 1; s < S; ++s) acc += v[s];
        const f16x2 lo = {(f16)acc[0], (f16)acc[1]}, hi = {(f16)acc[2], (f16)acc[3]};
        *reinterpret_cast<uint2*>(out + i) = make_uint2(as_u32(lo), as_u32(hi));
        return;
    }
    for (int e = i; e < min(i + 4, MN); ++e) {
        float acc = part[e];
#pragma unroll
        for (int s = 1; s < S; ++s) acc += part[(size_t)s * MN + e];
        out[e] = (f16)acc;
    }
}

}  // namespace w4a16

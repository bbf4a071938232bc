// W4A16 GEMM for prompts (M > 16 activation rows) on gfx950, group size 128.
//
// out[m][n] = fp16( sum_k x[m][k] * W[n][k] ), W[n][k] = fp16_rn(code * scale)
// decoded in registers: the B operand of every MFMA is bit-identical to what
// w4a16_dequantize_f16 writes, so the result is the reference's prefill path
// (dequantize, then an fp16 GEMM with fp32 accumulation) without the fp16
// weight round trip through HBM (0.5 byte per weight read instead of 0.5
// read + 2 written + 2 read).
//
// v_mfma_f32_16x16x32_f16 tiles: D[m][n] over 16 activation rows x 16 weight
// rows. Within a 128-weight group, step t (0..3) of lane l = 16 q + c takes
// k = 32 q + 8 t .. + 7 (the MFMA needs the same k set for its A and B
// lanes, not a particular order): lane (q, c) then reads its whole share of
// the group's weights for row c as ONE 16-byte load (bytes 16 q .. 16 q + 15
// of the row's 64-byte group), word t of which is step t; its A fragment of
// step t is the 16 contiguous bytes x[m][128 g + 32 q + 8 t ..], loaded
// straight from memory in natural order (no staging, no permutation).
//
// Decode of one word (8 weights, nibble i = weight i): per byte, v_perm puts
// the byte in both halves, v_bitop3 keeps the low nibble in the low half and
// the high nibble 4 bits up in the high half, flips bit 3 (two's complement
// to offset binary) and ORs in the binary16 1024.0 pattern; one packed fma
// (x {1, 1/16}, - {1032, 72}) gives the exact codes and one packed multiply
// by the group scale rounds code * scale once (RNE), as the dequantize kernel
// does. 16 VALU per 8 weights, shared by the MT activation tiles.
//
// Workgroup = SK wavefronts splitting the K / 128 groups (wavefront kw takes
// groups kw, kw + SK, ...); each wavefront computes MT x RB tiles (16 MT
// activation rows, 16 RB weight rows), so each A fragment feeds RB MFMAs and
// each decoded B fragment feeds MT. Loads of the next group are issued before
// the current group's MFMAs (two register buffers). The SK partial tiles are
// summed through LDS in a fixed order (deterministic) and stored as fp16.
//
// Grid: nbp * mblocks workgroups, nbp = the weight-row blocks rounded up to a
// multiple of 8. Workgroup b runs on XCD b % 8 (round-robin dispatch); it
// takes weight block 8 (s / mblocks) + b % 8 and activation block s % mblocks
// (s = b / 8), so every activation block of one weight block runs on the same
// XCD, one after another, and re-reads those weights from that XCD's L2.
// Workgroups past the last weight block return at once.
#pragma once

#include "w4a16_device.h"

namespace w4a16 {

// LDS of gemm_w4a16: the partial tiles of wavefronts 1 .. SK - 1.
__host__ __device__ constexpr int64_t gemm_lds_bytes(int mt, int rb, int sk) {
    return (int64_t)(sk - 1) * mt * rb * 64 * 16;
}

template <int MT, int RB>
struct GemmGroup {
    u32x4 a[MT][4];   // A fragments of the 4 steps, per activation tile
    u32x4 w[RB];      // 32 packed weights per lane, per weight tile
    uint32_t s[RB];   // fp16 bits of the group scale
};

// SiLU-multiply epilogue of a [gate; up] weight pair (PAIRED): N is the
// output width `inter`, the packed weights hold 2 inter rows (gate rows, then
// up rows), and a wavefront's RB weight tiles are RB / 2 gate tiles and the
// up tiles of the same columns; out[m][n] = fp16(fp16(silu(fp16(g))) *
// fp16(u)), the roundings of silu(gate) * up on the op's fp16 outputs
// (gemm_silu_mul, w4a16_device.h).

template <int MT, int RB, int SK, bool PAIRED = false>
__global__ void __launch_bounds__(64 * SK)
gemm_w4a16(const f16* __restrict__ x, const uint8_t* __restrict__ w, const f16* __restrict__ scales,
           f16* __restrict__ out, int M, int N, int K, int nblocks) {
    static_assert(!PAIRED || RB % 2 == 0, "paired tiles come in gate / up pairs");
    constexpr int RO = PAIRED ? RB / 2 : RB;   // output tiles per wavefront
    const int b = blockIdx.x;
    const int mblocks = (int)gridDim.x / ((nblocks + 7) & ~7);
    const int s = b >> 3;
    const int nbk = 8 * (s / mblocks) + (b & 7);
    const int mbk = s % mblocks;
    if (nbk >= nblocks) return;   // padding workgroup: whole workgroup, before any barrier

    extern __shared__ __align__(16) uint8_t smem[];
    f32x4* red = reinterpret_cast<f32x4*>(smem);   // [SK - 1][MT][RB][64]
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int c = lane & 15, q = lane >> 4;
    const int G = K >> 7;
    const uint32_t row_bytes = (uint32_t)(K >> 1);
    const int n0 = nbk * 16 * RO;
    const int m0 = mbk * 16 * MT;
    const int ng = wave < G ? (G - 1 - wave) / SK + 1 : 0;   // groups of this wavefront

    // per-lane 32-bit byte offsets (the host checks that every buffer is
    // below 4 GiB); rows past the end re-read the last row and are not stored
    const uint8_t* sbase = reinterpret_cast<const uint8_t*>(scales);
    const uint8_t* xbase = reinterpret_cast<const uint8_t*>(x);
    uint32_t wrow[RB], srow[RB], xrow[MT];
#pragma unroll
    for (int r = 0; r < RB; ++r) {
        // PAIRED: tiles RO .. RB - 1 are the up rows (N .. 2 N - 1) of tiles 0 .. RO - 1
        const uint32_t n = PAIRED && r >= RO ? (uint32_t)(N + min(n0 + 16 * (r - RO) + c, N - 1))
                                             : (uint32_t)min(n0 + 16 * r + c, N - 1);
        wrow[r] = n * row_bytes + 16u * q;
        srow[r] = n * (uint32_t)G * 2u;
    }
#pragma unroll
    for (int t = 0; t < MT; ++t) {
        const uint32_t m = (uint32_t)min(m0 + 16 * t + c, M - 1);
        xrow[t] = (m * (uint32_t)K + 32u * q) * 2u;
    }

    auto load = [&](GemmGroup<MT, RB>& buf, int j) {
        const uint32_t g = (uint32_t)(wave + SK * j);
#pragma unroll
        for (int r = 0; r < RB; ++r) buf.s[r] = *reinterpret_cast<const uint16_t*>(sbase + srow[r] + g * 2u);
#pragma unroll
        for (int r = 0; r < RB; ++r) buf.w[r] = *reinterpret_cast<const u32x4*>(w + wrow[r] + g * 64u);
#pragma unroll
        for (int t = 0; t < MT; ++t)
#pragma unroll
            for (int st = 0; st < 4; ++st)
                buf.a[t][st] = *reinterpret_cast<const u32x4*>(xbase + xrow[t] + g * 256u + 16u * st);
    };

    f32x4 acc[MT][RB];
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int r = 0; r < RB; ++r) acc[t][r] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};

    auto compute = [&](const GemmGroup<MT, RB>& buf) {
        const f16x2 mul = {(f16)1.0f, (f16)0.0625f};
        const f16x2 off = {(f16)-1032.0f, (f16)-72.0f};
#pragma unroll
        for (int st = 0; st < 4; ++st) {
#pragma unroll
            for (int r = 0; r < RB; ++r) {
                const f16 sc = __builtin_bit_cast(f16, (uint16_t)buf.s[r]);
                const f16x2 sc2 = {sc, sc};
                const uint32_t word = buf.w[r][st];
                f16x2 p[4];
#pragma unroll
                for (int by = 0; by < 4; ++by) {
                    // byte `by` in both halves, low nibble low, high nibble 4 bits up
                    const uint32_t sel = (0x0Cu << 24) | ((uint32_t)by << 16) | (0x0Cu << 8) | (uint32_t)by;
                    const uint32_t v = __builtin_amdgcn_bitop3_b32(perm(word, word, sel), 0x00F0000Fu,
                                                                   0x64806408u, 0x6A);
                    p[by] = __builtin_elementwise_fma(as_f16x2(v), mul, off) * sc2;
                }
                const f16x8 bt = __builtin_bit_cast(
                    f16x8, (u32x4){as_u32(p[0]), as_u32(p[1]), as_u32(p[2]), as_u32(p[3])});
#pragma unroll
                for (int t = 0; t < MT; ++t)
                    acc[t][r] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, buf.a[t][st]), bt,
                                                                       acc[t][r], 0, 0, 0);
            }
        }
    };

    // groups j = 0 .. ng - 1, two register buffers; the loop's tail is
    // peeled so no load sits behind a branch inside it
    if (ng > 0) {
        GemmGroup<MT, RB> b0, b1;
        load(b0, 0);
        int j = 0;
        for (; j + 2 < ng; j += 2) {
            load(b1, j + 1);
            compute(b0);
            load(b0, j + 2);
            compute(b1);
        }
        if (j + 1 < ng) {
            load(b1, j + 1);
            compute(b0);
            compute(b1);
        } else {
            compute(b0);
        }
    }

    // SK partial tiles: wavefronts 1.. write, wavefront 0 sums in order 0..SK-1
    if (SK > 1) {
        if (wave > 0) {
#pragma unroll
            for (int t = 0; t < MT; ++t)
#pragma unroll
                for (int r = 0; r < RB; ++r) red[(((wave - 1) * MT + t) * RB + r) * 64 + lane] = acc[t][r];
        }
        __syncthreads();
        if (wave > 0) return;
#pragma unroll
        for (int t = 0; t < MT; ++t)
#pragma unroll
            for (int r = 0; r < RB; ++r)
#pragma unroll
                for (int kw = 1; kw < SK; ++kw) acc[t][r] += red[(((kw - 1) * MT + t) * RB + r) * 64 + lane];
    }
    // D rows 4 q .. 4 q + 3 (activation rows), column c (weight row)
#pragma unroll
    for (int t = 0; t < MT; ++t) {
#pragma unroll
        for (int r = 0; r < RO; ++r) {
            const int n = n0 + 16 * r + c;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int m = m0 + 16 * t + 4 * q + e;
                if (m < M && n < N)
                    out[(size_t)m * N + n] = PAIRED ? gemm_silu_mul(acc[t][r][e], acc[t][r + RO][e])
                                                    : (f16)acc[t][r][e];
            }
        }
    }
}

}  // namespace w4a16

namespace w4a16 {

// ---------------------------------------------------------------------------
// W4A16 GEMM with the activation block staged in LDS (large M).
//
// gemm_w4a16 above reads each wavefront's A fragments from memory, so every
// workgroup of 16 RB weight rows re-reads its 16 MT activation rows over all
// of K (at M = 256 on 4096 x 14336: 470 MB of L2 reads, about half of the
// kernel's time). Here a workgroup of SN x SK wavefronts covers 16 RB SN
// weight rows: wavefront (sn, sk) owns weight tiles sn * RB .. and the groups
// g = sk, sk + SK, ...; round r stages groups r SK .. r SK + SK - 1 of the
// workgroup's activation rows in LDS once (double-buffered, one barrier per
// round, round r + 1 requested while round r is computed), and the SN
// wavefronts of each sk read their A fragments from it. Weights come from a
// ring of DB rounds in flight per wavefront (HBM latency is longer than one
// round's MFMAs). The rounds run to a multiple of DB; groups past K are
// staged as zeros and their weight loads clamped, so no load sits behind a
// branch. Decode, tile layout, k order and the SK reduction are those of
// gemm_w4a16; the grid mapping is the same with 16 RB SN weight rows per
// block.
//
// LDS: two buffers of [SK][16 MT][kGemmRow] halves (rows of one group padded
// from 128 to 136 halves: the 16 rows of a fragment read fall on distinct
// banks); after the last round the same memory holds the SK reduction's
// [SK - 1][SN][MT][RB][64] f32x4.
// ---------------------------------------------------------------------------
constexpr int kGemmRow = 136;
constexpr int kGemmRing = 4;   // rounds of weights in flight per wavefront

__host__ __device__ constexpr int64_t gemm2_lds_bytes(int mt, int rb, int sn, int sk) {
    return (int64_t)2 * sk * 16 * mt * kGemmRow * 2 > (int64_t)(sk - 1) * sn * mt * rb * 64 * 16
               ? (int64_t)2 * sk * 16 * mt * kGemmRow * 2
               : (int64_t)(sk - 1) * sn * mt * rb * 64 * 16;
}

template <int MT, int RB, int SN, int SK, bool PAIRED = false>
__global__ void __launch_bounds__(64 * SN * SK)
gemm2_w4a16(const f16* __restrict__ x, const uint8_t* __restrict__ w, const f16* __restrict__ scales,
            f16* __restrict__ out, int M, int N, int K, int nblocks) {
    static_assert(!PAIRED || RB % 2 == 0, "paired tiles come in gate / up pairs");
    constexpr int RO = PAIRED ? RB / 2 : RB;   // output tiles per wavefront (PAIRED: as gemm_w4a16)
    constexpr int T = 64 * SN * SK;
    constexpr int DB = kGemmRing;
    constexpr int UNITS = SK * 16 * MT * 16;   // 16-byte units staged per round
    static_assert(UNITS % T == 0, "whole staging units per thread");
    constexpr int UPT = UNITS / T;
    constexpr int BUF = SK * 16 * MT * kGemmRow;   // halves per staging buffer
    const int b = blockIdx.x;
    const int mblocks = (int)gridDim.x / ((nblocks + 7) & ~7);
    const int s = b >> 3;
    const int nbk = 8 * (s / mblocks) + (b & 7);
    const int mbk = s % mblocks;
    if (nbk >= nblocks) return;   // padding workgroup: whole workgroup, before any barrier

    extern __shared__ __align__(16) uint8_t smem[];
    f16* as = reinterpret_cast<f16*>(smem);                                   // [2][SK][16 MT][kGemmRow]
    f32x4* red = reinterpret_cast<f32x4*>(smem);   // [SK - 1][SN][MT][RB][64], after the last round
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int c = lane & 15, q = lane >> 4;
    const int sk = wave % SK, sn = wave / SK;
    const int G = K >> 7;
    const int R = (G + SK - 1) / SK;
    const int RP = (R + DB - 1) / DB * DB;   // rounds run, a multiple of the ring
    const uint32_t row_bytes = (uint32_t)(K >> 1);
    const int n0 = nbk * 16 * RO * SN + sn * 16 * RO;
    const int m0 = mbk * 16 * MT;

    // staging: unit u = (group gl, row, 16-byte part p) of the round
    const uint8_t* xbase = reinterpret_cast<const uint8_t*>(x);
    auto stage_load = [&](u32x4 (&a)[UPT], int r) {
#pragma unroll
        for (int p = 0; p < UPT; ++p) {
            const int u = threadIdx.x + p * T;
            const int gl = u / (16 * MT * 16), rem = u % (16 * MT * 16);
            const int row = rem >> 4, part = rem & 15;
            const int g = min(r * SK + gl, G - 1);
            const uint32_t m = (uint32_t)min(m0 + row, M - 1);
            a[p] = *reinterpret_cast<const u32x4*>(xbase + (m * (uint32_t)K + (uint32_t)g * 128u + part * 8u) * 2u);
        }
    };
    auto stage_put = [&](const u32x4 (&a)[UPT], int r, int buf) {
#pragma unroll
        for (int p = 0; p < UPT; ++p) {
            const int u = threadIdx.x + p * T;
            const int gl = u / (16 * MT * 16), rem = u % (16 * MT * 16);
            const int row = rem >> 4, part = rem & 15;
            const bool live = r * SK + gl < G;
            *reinterpret_cast<u32x4*>(as + (size_t)buf * BUF + ((size_t)gl * 16 * MT + row) * kGemmRow + part * 8) =
                live ? a[p] : (u32x4){0u, 0u, 0u, 0u};
        }
    };

    // weights: ring slot d holds round r's group g = r SK + sk (clamped)
    const uint8_t* sbase = reinterpret_cast<const uint8_t*>(scales);
    uint32_t wrow[RB], srow[RB];
#pragma unroll
    for (int t = 0; t < RB; ++t) {
        const uint32_t n = PAIRED && t >= RO ? (uint32_t)(N + min(n0 + 16 * (t - RO) + c, N - 1))
                                             : (uint32_t)min(n0 + 16 * t + c, N - 1);
        wrow[t] = n * row_bytes + 16u * q;
        srow[t] = n * (uint32_t)G * 2u;
    }
    u32x4 wv[DB][RB];
    uint32_t sv[DB][RB];
    auto load_w = [&](int d, int r) {
        const uint32_t g = (uint32_t)min(r * SK + sk, G - 1);
#pragma unroll
        for (int t = 0; t < RB; ++t) sv[d][t] = *reinterpret_cast<const uint16_t*>(sbase + srow[t] + g * 2u);
#pragma unroll
        for (int t = 0; t < RB; ++t) wv[d][t] = *reinterpret_cast<const u32x4*>(w + wrow[t] + g * 64u);
    };

    f32x4 acc[MT][RB];
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int r = 0; r < RB; ++r) acc[t][r] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};

    const f16x2 mul = {(f16)1.0f, (f16)0.0625f};
    const f16x2 off = {(f16)-1032.0f, (f16)-72.0f};
    auto compute = [&](int d, int buf) {
        const f16* ab = as + (size_t)buf * BUF + (size_t)sk * 16 * MT * kGemmRow;
#pragma unroll
        for (int st = 0; st < 4; ++st) {
            u32x4 af[MT];
#pragma unroll
            for (int t = 0; t < MT; ++t)
                af[t] = *reinterpret_cast<const u32x4*>(ab + (16 * t + c) * kGemmRow + 32 * q + 8 * st);
#pragma unroll
            for (int r = 0; r < RB; ++r) {
                const f16 sc = __builtin_bit_cast(f16, (uint16_t)sv[d][r]);
                const f16x2 sc2 = {sc, sc};
                const uint32_t word = wv[d][r][st];
                f16x2 pr[4];
#pragma unroll
                for (int by = 0; by < 4; ++by) {
                    const uint32_t sel = (0x0Cu << 24) | ((uint32_t)by << 16) | (0x0Cu << 8) | (uint32_t)by;
                    const uint32_t v = __builtin_amdgcn_bitop3_b32(perm(word, word, sel), 0x00F0000Fu, 0x64806408u,
                                                                   0x6A);
                    pr[by] = __builtin_elementwise_fma(as_f16x2(v), mul, off) * sc2;
                }
                const f16x8 bt = __builtin_bit_cast(
                    f16x8, (u32x4){as_u32(pr[0]), as_u32(pr[1]), as_u32(pr[2]), as_u32(pr[3])});
#pragma unroll
                for (int t = 0; t < MT; ++t)
                    acc[t][r] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, af[t]), bt,
                                                                       acc[t][r], 0, 0, 0);
            }
        }
    };

    // prologue: round 0 staged, the ring's first DB rounds requested
    {
        u32x4 a[UPT];
        stage_load(a, 0);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int d = 0; d < DB; ++d) load_w(d, d);
        __builtin_amdgcn_sched_barrier(0);
        stage_put(a, 0, 0);
    }
    __syncthreads();
    for (int r0 = 0; r0 < RP; r0 += DB) {
#pragma unroll
        for (int d = 0; d < DB; ++d) {
            const int r = r0 + d;
            u32x4 a[UPT];
            stage_load(a, r + 1);   // past the last round: clamped, staged as zeros, never read
            compute(d, r & 1);
            load_w(d, r + DB);
            stage_put(a, r + 1, (r + 1) & 1);
            __syncthreads();
        }
    }

    // SK partial tiles: wavefronts sk > 0 write, sk = 0 sums in order
    if (SK > 1) {
        if (sk > 0) {
#pragma unroll
            for (int t = 0; t < MT; ++t)
#pragma unroll
                for (int r = 0; r < RB; ++r)
                    red[((((sk - 1) * SN + sn) * MT + t) * RB + r) * 64 + lane] = acc[t][r];
        }
        __syncthreads();
        if (sk > 0) return;
#pragma unroll
        for (int t = 0; t < MT; ++t)
#pragma unroll
            for (int r = 0; r < RB; ++r)
#pragma unroll
                for (int k2 = 1; k2 < SK; ++k2) acc[t][r] += red[((((k2 - 1) * SN + sn) * MT + t) * RB + r) * 64 + lane];
    }
#pragma unroll
    for (int t = 0; t < MT; ++t) {
#pragma unroll
        for (int r = 0; r < RO; ++r) {
            const int n = n0 + 16 * r + c;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int m = m0 + 16 * t + 4 * q + e;
                if (m < M && n < N)
                    out[(size_t)m * N + n] = PAIRED ? gemm_silu_mul(acc[t][r][e], acc[t][r + RO][e])
                                                    : (f16)acc[t][r][e];
            }
        }
    }
}

// ---------------------------------------------------------------------------
// W4A16 GEMM on 32x32 tiles (large M).
//
// gemm2_w4a16 on v_mfma_f32_32x32x16_f16: every decoded B fragment (8
// weights per lane) and every A fragment read from LDS now feed an MFMA of
// 32 x 32 x 16 instead of 16 x 16 x 32, so the decode VALU work and the LDS
// reads per FLOP are halved. Lane layout (checked on the device): A lane l
// holds row l % 32, k = 8 (l / 32) .. + 7 of its 32 x 16 step; B lane l holds
// column l % 32 of the same k; D register e of lane l is row
// 8 (e / 4) + 4 (l / 32) + e % 4, column l % 32.
//
// Within a 128-weight group, step s (0..7) of lane half h = l / 32 takes
// k = 64 h + 8 s .. + 7, so a lane's weights of one group are bytes 32 h ..
// 32 h + 31 of its row's 64-byte group (two 16-byte loads, word s % 4 of
// the first or second) and its A fragment of step s is the 16 contiguous
// bytes at halves 64 h + 8 s of its activation row's staged group. Decode,
// staging (rows of 136 halves), the ring of weight rounds, the XCD-aware grid
// and the fixed-order SK reduction are those of gemm2_w4a16, with tiles of
// 32 rows.
// ---------------------------------------------------------------------------
__host__ __device__ constexpr int64_t gemm3_lds_bytes(int mt, int rb, int sn, int sk) {
    return (int64_t)2 * sk * 32 * mt * kGemmRow * 2 > (int64_t)(sk - 1) * sn * mt * rb * 64 * 64
               ? (int64_t)2 * sk * 32 * mt * kGemmRow * 2
               : (int64_t)(sk - 1) * sn * mt * rb * 64 * 64;
}

typedef float f32x16 __attribute__((ext_vector_type(16)));

template <int MT, int RB, int SN, int SK, bool PAIRED = false, int LA = 2>
__global__ void __launch_bounds__(64 * SN * SK)
gemm3_w4a16(const f16* __restrict__ x, const uint8_t* __restrict__ w, const f16* __restrict__ scales,
            f16* __restrict__ out, int M, int N, int K, int nblocks) {
    static_assert(!PAIRED || RB % 2 == 0, "paired tiles come in gate / up pairs");
    constexpr int RO = PAIRED ? RB / 2 : RB;   // output tiles per wavefront
    constexpr int T = 64 * SN * SK;
    constexpr int DB = kGemmRing;
    constexpr int UNITS = SK * 32 * MT * 16;   // 16-byte units staged per round
    static_assert(UNITS % T == 0, "whole staging units per thread");
    constexpr int UPT = UNITS / T;
    constexpr int BUF = SK * 32 * MT * kGemmRow;   // halves per staging buffer
    const int b = blockIdx.x;
    const int mblocks = (int)gridDim.x / ((nblocks + 7) & ~7);
    const int sidx = b >> 3;
    const int nbk = 8 * (sidx / mblocks) + (b & 7);
    const int mbk = sidx % mblocks;
    if (nbk >= nblocks) return;   // padding workgroup: whole workgroup, before any barrier

    extern __shared__ __align__(16) uint8_t smem[];
    f16* as = reinterpret_cast<f16*>(smem);                                   // [2][SK][32 MT][kGemmRow]
    f32x16* red = reinterpret_cast<f32x16*>(smem);   // [SK - 1][SN][MT][RB][64], after the last round
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int c = lane & 31, h = lane >> 5;
    const int sk = wave % SK, sn = wave / SK;
    const int G = K >> 7;
    const int R = (G + SK - 1) / SK;
    const int RP = (R + DB - 1) / DB * DB;   // rounds run, a multiple of the ring
    const uint32_t row_bytes = (uint32_t)(K >> 1);
    const int n0 = nbk * 32 * RO * SN + sn * 32 * RO;
    const int m0 = mbk * 32 * MT;

    // staging: unit u = (group gl, row, 16-byte part p) of the round
    const uint8_t* xbase = reinterpret_cast<const uint8_t*>(x);
    auto stage_load = [&](u32x4 (&a)[UPT], int r) {
#pragma unroll
        for (int p = 0; p < UPT; ++p) {
            const int u = threadIdx.x + p * T;
            const int gl = u / (32 * MT * 16), rem = u % (32 * MT * 16);
            const int row = rem >> 4, part = rem & 15;
            const int g = min(r * SK + gl, G - 1);
            const uint32_t m = (uint32_t)min(m0 + row, M - 1);
            a[p] = *reinterpret_cast<const u32x4*>(xbase + (m * (uint32_t)K + (uint32_t)g * 128u + part * 8u) * 2u);
        }
    };
    auto stage_put = [&](const u32x4 (&a)[UPT], int r, int buf) {
#pragma unroll
        for (int p = 0; p < UPT; ++p) {
            const int u = threadIdx.x + p * T;
            const int gl = u / (32 * MT * 16), rem = u % (32 * MT * 16);
            const int row = rem >> 4, part = rem & 15;
            const bool live = r * SK + gl < G;
            *reinterpret_cast<u32x4*>(as + (size_t)buf * BUF + ((size_t)gl * 32 * MT + row) * kGemmRow + part * 8) =
                live ? a[p] : (u32x4){0u, 0u, 0u, 0u};
        }
    };

    // weights: ring slot d holds round r's group g = r SK + sk (clamped), 32
    // bytes per lane and weight tile (two 16-byte loads)
    const uint8_t* sbase = reinterpret_cast<const uint8_t*>(scales);
    uint32_t wrow[RB], srow[RB];
#pragma unroll
    for (int t = 0; t < RB; ++t) {
        const uint32_t n = PAIRED && t >= RO ? (uint32_t)(N + min(n0 + 32 * (t - RO) + c, N - 1))
                                             : (uint32_t)min(n0 + 32 * t + c, N - 1);
        wrow[t] = n * row_bytes + 32u * h;
        srow[t] = n * (uint32_t)G * 2u;
    }
    u32x4 wv[DB][RB][2];
    uint32_t sv[DB][RB];
    auto load_w = [&](int d, int r) {
        const uint32_t g = (uint32_t)min(r * SK + sk, G - 1);
#pragma unroll
        for (int t = 0; t < RB; ++t) sv[d][t] = *reinterpret_cast<const uint16_t*>(sbase + srow[t] + g * 2u);
#pragma unroll
        for (int t = 0; t < RB; ++t) {
            wv[d][t][0] = *reinterpret_cast<const u32x4*>(w + wrow[t] + g * 64u);
            wv[d][t][1] = *reinterpret_cast<const u32x4*>(w + wrow[t] + g * 64u + 16u);
        }
    };

    f32x16 acc[MT][RB];
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int r = 0; r < RB; ++r)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[t][r][e] = 0.0f;

    const f16x2 mul = {(f16)1.0f, (f16)0.0625f};
    const f16x2 off = {(f16)-1032.0f, (f16)-72.0f};
    auto compute = [&](int d, int buf) {
        const f16* ab = as + (size_t)buf * BUF + (size_t)sk * 32 * MT * kGemmRow;
        // A fragments one step ahead: step st + 1's LDS reads are in flight
        // while step st decodes and runs its MFMAs
        u32x4 afn[MT];
#pragma unroll
        for (int t = 0; t < MT; ++t) afn[t] = *reinterpret_cast<const u32x4*>(ab + (32 * t + c) * kGemmRow + 64 * h);
#pragma unroll
        for (int st = 0; st < 8; ++st) {
            u32x4 af[MT];
#pragma unroll
            for (int t = 0; t < MT; ++t) af[t] = afn[t];
            if (st < 7) {
#pragma unroll
                for (int t = 0; t < MT; ++t)
                    afn[t] = *reinterpret_cast<const u32x4*>(ab + (32 * t + c) * kGemmRow + 64 * h + 8 * (st + 1));
            }
#pragma unroll
            for (int r = 0; r < RB; ++r) {
                const f16 sc = __builtin_bit_cast(f16, (uint16_t)sv[d][r]);
                const f16x2 sc2 = {sc, sc};
                const uint32_t word = wv[d][r][st >> 2][st & 3];
                f16x2 pr[4];
#pragma unroll
                for (int by = 0; by < 4; ++by) {
                    const uint32_t sel = (0x0Cu << 24) | ((uint32_t)by << 16) | (0x0Cu << 8) | (uint32_t)by;
                    const uint32_t v = __builtin_amdgcn_bitop3_b32(perm(word, word, sel), 0x00F0000Fu, 0x64806408u,
                                                                   0x6A);
                    pr[by] = __builtin_elementwise_fma(as_f16x2(v), mul, off) * sc2;
                }
                const f16x8 bt = __builtin_bit_cast(
                    f16x8, (u32x4){as_u32(pr[0]), as_u32(pr[1]), as_u32(pr[2]), as_u32(pr[3])});
#pragma unroll
                for (int t = 0; t < MT; ++t)
                    acc[t][r] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, af[t]), bt,
                                                                       acc[t][r], 0, 0, 0);
            }
        }
    };

    // prologue: round 0 staged, round 1 requested, the ring's first DB rounds
    // of weights requested. Staging runs two rounds ahead: round r's loop
    // requests round r + 2 into the register set round r came from and puts
    // round r + 1 (requested a round earlier) into LDS, so a staging load has
    // two rounds of MFMAs to arrive.
    // (LA = 1: round r requests round r + 1 and puts it after its MFMAs, for
    // shapes whose registers only hold one staging set.)
    static_assert(LA == 1 || LA == 2, "staging runs one or two rounds ahead");
    u32x4 a[LA][UPT];
    stage_load(a[0], 0);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int d = 0; d < DB; ++d) load_w(d, d);
    if constexpr (LA == 2) stage_load(a[LA - 1], 1);
    __builtin_amdgcn_sched_barrier(0);
    stage_put(a[0], 0, 0);
    __syncthreads();
    static_assert(DB % 2 == 0, "the staging register sets alternate within the weight ring");
    for (int r0 = 0; r0 < RP; r0 += DB) {
#pragma unroll
        for (int d = 0; d < DB; ++d) {
            const int r = r0 + d;
            // past the last round: clamped, staged as zeros, never read
            if constexpr (LA == 2) stage_load(a[d & 1], r + 2);
            else stage_load(a[0], r + 1);
            compute(d, r & 1);
            load_w(d, r + DB);
            stage_put(a[LA == 2 ? (d + 1) & 1 : 0], r + 1, (r + 1) & 1);
            __syncthreads();
        }
    }

    // SK partial tiles: wavefronts sk > 0 write, sk = 0 sums in order
    if (SK > 1) {
        if (sk > 0) {
#pragma unroll
            for (int t = 0; t < MT; ++t)
#pragma unroll
                for (int r = 0; r < RB; ++r)
                    red[((((sk - 1) * SN + sn) * MT + t) * RB + r) * 64 + lane] = acc[t][r];
        }
        __syncthreads();
        if (sk > 0) return;
#pragma unroll
        for (int t = 0; t < MT; ++t)
#pragma unroll
            for (int r = 0; r < RB; ++r)
#pragma unroll
                for (int k2 = 1; k2 < SK; ++k2) acc[t][r] += red[((((k2 - 1) * SN + sn) * MT + t) * RB + r) * 64 + lane];
    }
#pragma unroll
    for (int t = 0; t < MT; ++t) {
#pragma unroll
        for (int r = 0; r < RO; ++r) {
            const int n = n0 + 32 * r + c;
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int m = m0 + 32 * t + 8 * (e >> 2) + 4 * h + (e & 3);
                if (m < M && n < N)
                    out[(size_t)m * N + n] = PAIRED ? gemm_silu_mul(acc[t][r][e], acc[t][r + RO][e])
                                                    : (f16)acc[t][r][e];
            }
        }
    }
}

}  // namespace w4a16

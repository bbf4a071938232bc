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
// Workgroup = S wavefronts (blockDim = 64 S) on R consecutive output rows.
// The activations are staged once per workgroup in LDS, permuted to the
// unpack8 pair order and laid out unit-major: unit q (8 halves) of chunk c of
// activation row m lives at xs[(m*4 + q) * C + c], so the 64 lanes of a
// wavefront reading unit q of 64 consecutive chunks hit 64 consecutive
// 16-byte slots.
// Thread t handles chunks t, t + 64 S, ... of every one of the R rows: each
// chunk is one 16-byte load per row, decoded once and dotted with the M
// activation rows by v_dot2_f32_f16 (fp16 products, fp32 accumulation). The
// chunk dot is scaled by its group's scale in fp32 (reference
// csrc/int4_linear_kernel.cu:390 scales per-lane chunk partials the same way).
// Reduction: DPP within each wavefront, LDS across the S wavefronts.
// Rows past N re-read row N-1 and are not stored (keeps every access in
// bounds and every wavefront on the same path).
// ---------------------------------------------------------------------------
template <int M, int R, int U>
__global__ void __launch_bounds__(512)
gemv_valu(const f16* __restrict__ x, const uint8_t* __restrict__ w,
          const f16* __restrict__ scales, f16* __restrict__ out, int N, int K) {
    extern __shared__ __align__(16) uint8_t smem[];
    u32x4* xs = reinterpret_cast<u32x4*>(smem);

    const int T = blockDim.x;
    const int tid = threadIdx.x;
    const int C = K >> 5;   // chunks per row
    const int G = K >> 7;   // groups per row

    // Stage activations (16 B per unit, permuted).
    const int units_per_row = K >> 3;
    for (int i = tid; i < M * units_per_row; i += T) {
        const int m = i / units_per_row;
        const int j = i - m * units_per_row;
        const u32x4 a = *reinterpret_cast<const u32x4*>(x + (size_t)i * 8);
        xs[(m * 4 + (j & 3)) * C + (j >> 2)] = permute8(a);
    }
    __syncthreads();

    const int n0 = blockIdx.x * R;
    const u32x4* wrow[R];
    const f16* srow[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int n = min(n0 + r, N - 1);
        wrow[r] = reinterpret_cast<const u32x4*>(w + (size_t)n * (size_t)(K >> 1));
        srow[r] = scales + (size_t)n * G;
    }

    float acc[R][M];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int m = 0; m < M; ++m) acc[r][m] = 0.0f;

    for (int c0 = tid; c0 < C; c0 += U * T) {
        u32x4 wv[U][R];
        f16 sv[U][R];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int c = c0 + u * T;
            if (c < C) {
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    wv[u][r] = load_stream(wrow[r] + c);
                    sv[u][r] = srow[r][c >> 2];
                }
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int c = c0 + u * T;
            if (c < C) {
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    u32x4 xa[M];
#pragma unroll
                    for (int m = 0; m < M; ++m) xa[m] = xs[(m * 4 + q) * C + c];
#pragma unroll
                    for (int r = 0; r < R; ++r) {
                        const Codes8 cw = unpack8(wv[u][r][q]);
                        const float s = (float)sv[u][r];
#pragma unroll
                        for (int m = 0; m < M; ++m) {
                            float d = 0.0f;
                            d = __builtin_amdgcn_fdot2(as_f16x2(xa[m].x), cw.p[0], d, false);
                            d = __builtin_amdgcn_fdot2(as_f16x2(xa[m].y), cw.p[1], d, false);
                            d = __builtin_amdgcn_fdot2(as_f16x2(xa[m].z), cw.p[2], d, false);
                            d = __builtin_amdgcn_fdot2(as_f16x2(xa[m].w), cw.p[3], d, false);
                            acc[r][m] = __builtin_fmaf(d, s, acc[r][m]);
                        }
                    }
                }
            }
        }
    }

    const int S = T >> 6;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    float* red = reinterpret_cast<float*>(smem + (size_t)M * K * 2);
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int m = 0; m < M; ++m) {
            const float v = wave_sum(acc[r][m]);
            if (S == 1) {
                if (lane == 0 && n0 + r < N) out[(size_t)m * N + n0 + r] = (f16)v;
            } else if (lane == 0) {
                red[wave * (R * M) + r * M + m] = v;
            }
        }
    if (S > 1) {
        __syncthreads();
        if (tid < R * M) {
            const int r = tid / M;
            const int m = tid - r * M;
            float v = 0.0f;
            for (int s = 0; s < S; ++s) v += red[s * (R * M) + tid];
            if (n0 + r < N) out[(size_t)m * N + n0 + r] = (f16)v;
        }
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
// wavefronts splitting the groups of K (wave w takes groups w, w+S, ...),
// reduced through LDS at the end. Activation rows m >= M and rows past N
// follow the same path with zero A / clamped rows and are not stored.
// ---------------------------------------------------------------------------
template <int RB, int U>
__global__ void __launch_bounds__(512)
gemv_mfma(const f16* __restrict__ x, const uint8_t* __restrict__ w,
          const f16* __restrict__ scales, f16* __restrict__ out, int M, int N, int K) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int S = blockDim.x >> 6;
    const int wave = threadIdx.x >> 6;
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
// Dequantize: out[n][k] = fp16_rn(code * scale), one thread per 16-byte chunk
// (32 weights, inside one group since G % 32 == 0), 64 bytes written per
// thread in natural k order. Codes are exact in f16, and an IEEE binary16
// multiply of exact operands rounds the exact product once (round to nearest
// even, subnormals kept), which is the value of reference
// w4a16/reference.py:38-46 followed by .to(torch.float16).
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(256)
dequantize_kernel(const uint8_t* __restrict__ w, const f16* __restrict__ scales,
                  f16* __restrict__ out, int64_t chunks, int chunks_per_row,
                  int chunks_per_group, int groups_per_row) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= chunks) return;
    const int64_t n = i / chunks_per_row;
    const int c = (int)(i - n * chunks_per_row);
    const u32x4 d = load_stream(reinterpret_cast<const u32x4*>(w) + i);
    const f16 s = scales[n * groups_per_row + c / chunks_per_group];
    const f16x2 ss = {s, s};
    u32x4* o = reinterpret_cast<u32x4*>(out) + i * 4;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const uint32_t u = d[q] ^ 0x88888888u;
        u32x4 v;
        v.x = as_u32(unpack_byte_pair<0>(u) * ss);
        v.y = as_u32(unpack_byte_pair<1>(u) * ss);
        v.z = as_u32(unpack_byte_pair<2>(u) * ss);
        v.w = as_u32(unpack_byte_pair<3>(u) * ss);
        o[q] = v;
    }
}

}  // namespace w4a16

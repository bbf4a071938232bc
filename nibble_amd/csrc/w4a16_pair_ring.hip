// Launcher of the paired-layout ring GEMV (w4a16_pair_ring.h, M = 1..16) and
// its instantiations, in a translation unit of their own. Called by the
// dispatcher in w4a16_hip.hip.
#include "w4a16_hip.h"

#include <hip/hip_runtime.h>

#include <string>

#include "w4a16_pair_ring.h"

namespace w4a16_internal {
void set_last_error(const std::string& message);   // w4a16_hip.hip
int ensure_lds(const void* kernel, int bytes);     // w4a16_hip.hip: raise the dynamic-LDS limit once
int launch_split_reduce(int slices, const float* part, w4a16::f16* o, int64_t mn, hipStream_t stream);   // w4a16_pair.hip
}  // namespace w4a16_internal

namespace {

constexpr int kMaxLdsBytes = 160 * 1024;

int fail(int code, const std::string& message) {
    w4a16_internal::set_last_error(message);
    return code;
}

using Kern = void (*)(const w4a16::f16*, const uint8_t*, const w4a16::f16*, w4a16::f16*, int, int, int, float*, int,
                      w4a16::RingFusion);

int row_slots(int M) { return M <= 1 ? 1 : M <= 4 ? 4 : M <= 8 ? 8 : 16; }

// Instantiated (row slots, wavefronts splitting K, wavefronts on 8-row
// blocks, pairs per wavefront, pairs in flight): the launch shapes the M = 1
// and M = 2..8 sweeps chose per row length (K = 256 x pairs).
Kern pick(int ms, int sk, int sn, int ppw, int depth) {
#define W4A16_P(MS, SK, SN, PPW, D) \
    if (ms == MS && sk == SK && sn == SN && ppw == PPW && depth == D) return w4a16::gemv_pair_ring<MS, SK, SN, 1, PPW, D>;
    // M = 1
    W4A16_P(1, 1, 3, 8, 8)    // K = 2048 (tuned entry)
    W4A16_P(1, 1, 3, 8, 7)    // K = 2048, N < 8192
    W4A16_P(1, 1, 3, 8, 6)    // K = 2048, 8192 <= N < 16384
    W4A16_P(1, 1, 8, 8, 4)    // K = 2048, N >= 16384
    W4A16_P(1, 2, 2, 8, 8)    // K = 4096 (tuned entry)
    W4A16_P(1, 2, 2, 8, 7)    // K = 4096, N < 8192
    W4A16_P(1, 1, 8, 16, 6)   // K = 4096, N >= 8192
    W4A16_P(1, 4, 1, 6, 6)    // K = 5376 .. 6144
    W4A16_P(1, 2, 4, 16, 4)   // K = 8192 (tuned entry)
    W4A16_P(1, 2, 4, 16, 6)   // K = 8192, N < 16384
    W4A16_P(1, 1, 7, 32, 6)   // K = 8192, N >= 16384
    W4A16_P(1, 2, 2, 28, 10)  // K = 14080 .. 14336
    W4A16_P(1, 2, 4, 56, 6)   // K = 28416 .. 28672
    // M = 2..4
    W4A16_P(4, 4, 1, 2, 2)    // K = 2048, N <= 2048
    W4A16_P(4, 1, 4, 8, 6)    // K = 2048 (tuned entry)
    W4A16_P(4, 1, 4, 8, 7)    // K = 2048, N <= 8192
    W4A16_P(4, 2, 2, 8, 4)    // K = 4096 (tuned entry)
    W4A16_P(4, 2, 2, 8, 6)    // K = 4096, N < 8192
    W4A16_P(4, 1, 8, 16, 6)   // K = 4096, N >= 8192
    W4A16_P(4, 8, 1, 3, 3)    // K = 5376 .. 6144 (M = 3, 4)
    W4A16_P(4, 2, 4, 16, 4)   // K = 8192, N <= 8192
    W4A16_P(4, 4, 2, 14, 6)   // K = 14080 .. 14336
    // M = 5..8
    W4A16_P(8, 4, 1, 2, 2)    // K = 2048, N <= 2048
    W4A16_P(8, 1, 4, 8, 6)    // K = 2048, N <= 8192
    W4A16_P(8, 4, 2, 4, 4)    // K = 4096, N < 8192
    W4A16_P(8, 1, 8, 16, 6)   // K = 4096, N >= 8192
    W4A16_P(8, 2, 4, 16, 4)   // K = 8192 (tuned entry)
    W4A16_P(8, 2, 4, 16, 5)   // K = 8192, N <= 8192
    W4A16_P(8, 11, 1, 2, 2)   // K = 5376 .. 5632, N <= 2048 (M = 6..8)
    // M = 9..16 (exact decode)
    W4A16_P(16, 8, 1, 1, 1)   // K = 2048, N <= 2048
    W4A16_P(16, 4, 2, 2, 2)   // K = 2048, N <= 4096
    W4A16_P(16, 2, 4, 4, 4)   // K = 2048, N > 4096
    W4A16_P(16, 1, 4, 8, 4)   // K = 2048: the SiLU form's K split over plain rows
#undef W4A16_P
    return nullptr;
}

// Split-K instantiations (slices > 1; row slots, wavefronts, pairs per
// wavefront per slice, pairs in flight) and their 8-row blocks per
// wavefront: M = 9..16 on 5632 x 2048 (8 slices of 3 pairs), 14336 x 4096
// (4 of 14) and 8192 x 8192 (2 of 16); M = 3..4 on 28672 x 8192 (4 of 28);
// M = 5..8 with two blocks per wavefront (half the activation staging per
// row) on 28672 x 8192 (8 of 14), 8192 x 28672 (2 of 16) and, on 4
// wavefronts, 14336 x 4096 (8 of 7).
struct SplitPick {
    Kern kern;
    int rb;
};
SplitPick pick_split(int ms, int sk, int sn, int ppw, int depth) {
#define W4A16_P(MS, SK, SN, RB, PPW, D)                               \
    if (ms == MS && sk == SK && sn == SN && ppw == PPW && depth == D) \
        return SplitPick{w4a16::gemv_pair_ring<MS, SK, SN, RB, PPW, D, true>, RB};
    W4A16_P(4, 1, 8, 1, 28, 4)
    W4A16_P(8, 1, 8, 2, 14, 2)
    W4A16_P(8, 1, 8, 2, 16, 3)
    W4A16_P(16, 1, 8, 1, 3, 3)
    W4A16_P(16, 1, 8, 1, 14, 4)
    W4A16_P(16, 1, 8, 1, 16, 4)
    W4A16_P(8, 1, 4, 2, 7, 2)
#undef W4A16_P
    return SplitPick{nullptr, 1};
}

// SiLU form (16 row slots, a gate and an up block per wavefront):
// (wavefronts splitting K, wavefronts on output blocks, pairs per
// wavefront, pairs in flight). Measured at M = 16 / 9, 2048 x 2 x 5632,
// graph timing of 22 calls over 24 weight copies (one box, two passes):
// (4, 3, 2, 1) 7.35-7.47 / 7.11-7.20 us; (4, 3, 2, 2) 7.75-7.88 / 7.40;
// (2, 3, 4, 2) 7.82-8.03 / 7.50-7.57; (2, 4, 4, 2) 7.88 / 7.57; (3, 3, 3, 1)
// 8.07-8.19 / 7.77; (1, 4, 8, 4) 8.20-8.50 / 7.93-7.98; (4, 4, 2, 1) 8.45 /
// 8.24-8.37; (1, 3, 8, 4) 8.66-8.73 / 8.16-8.19; (4, 2, 2, 1) 8.74 / 8.27;
// (2, 2, 4, 2) 8.96 / 8.53; (3, 5, 3, 1) 11.1 / 10.8. Three wavefronts on
// output blocks give 235 workgroups (one per CU; four give 176), and four
// on K give each CU 12 wavefronts requesting its 64 KB of activations.
Kern pick_silu(int sk, int sn, int ppw, int depth) {
#define W4A16_P(SK, SN, PPW, D) \
    if (sk == SK && sn == SN && ppw == PPW && depth == D) return w4a16::gemv_pair_ring<16, SK, SN, 2, PPW, D, false, true>;
    W4A16_P(4, 3, 2, 1)   // K = 2048
#undef W4A16_P
    return nullptr;
}

// Pairs per wavefront for `slices` K slices of `sk` wavefronts each.
int ppw_of(int64_t K, int sk, int slices) {
    const int64_t P = K / 256;
    const int64_t per_slice = (P + slices - 1) / slices;
    return (int)((per_slice + sk - 1) / sk);
}

}  // namespace

namespace w4a16_internal {

// Pairs per wavefront for K split over `sk` wavefronts (G = K / 128 even).
int pair_ring_ppw(int64_t K, int sk) { return sk > 0 ? (int)((K / 256 + sk - 1) / sk) : 0; }

int64_t pair_ring_workspace_bytes(int64_t M, int64_t N, int slices) {
    return slices > 1 ? (int64_t)slices * M * N * 4 : 0;
}

// Slices > 1 must leave none empty: (slices - 1) ceil(P / slices) < P.
bool pair_ring_slices_valid(int64_t K, int slices) {
    const int64_t P = K / 256;
    return slices == 1 || (slices >= 2 && slices <= 16 && (int64_t)(slices - 1) * ((P + slices - 1) / slices) < P);
}

bool pair_ring_instantiated(int64_t M, int64_t K, int sk, int sn, int depth, int slices) {
    if (M < 1 || M > 16 || K < 256 || K % 256 != 0 || sk < 1) return false;
    if (slices < 1) slices = 1;
    if (!pair_ring_slices_valid(K, slices)) return false;
    const int ppw = ppw_of(K, sk, slices);
    const int ms = row_slots((int)M);
    const SplitPick k = slices > 1 ? pick_split(ms, sk, sn, ppw, depth) : SplitPick{pick(ms, sk, sn, ppw, depth), 1};
    return k.kern != nullptr && w4a16::pair_ring_lds_bytes(ms, sk, sn, k.rb, ppw) <= kMaxLdsBytes;
}

bool pair_ring_silu_instantiated(int64_t M, int64_t K, int sk, int sn, int depth) {
    if (M < 9 || M > 16 || K < 256 || K % 256 != 0 || sk < 1) return false;
    const int ppw = ppw_of(K, sk, 1);
    return pick_silu(sk, sn, ppw, depth) != nullptr && w4a16::pair_ring_lds_bytes(16, sk, sn, 2, ppw) <= kMaxLdsBytes;
}

int launch_pair_ring(int sk, int sn, int depth, int slices, int M, const w4a16::f16* x, const uint8_t* w,
                     const w4a16::f16* s, w4a16::f16* o, int N, int K, void* part, int64_t part_bytes,
                     hipStream_t stream, bool reduce) {
    if (M < 1 || M > 16) return fail(W4A16_ERR_CONFIG, "paired ring kernel: 1 <= M <= 16");
    if (K < 256 || K % 256 != 0)
        return fail(W4A16_ERR_CONFIG, "paired ring kernel: K must be a multiple of 256 (an even group count)");
    if (reinterpret_cast<uintptr_t>(s) & 3u)
        return fail(W4A16_ERR_CONFIG, "paired ring kernel: scales must be 4-byte aligned");
    if (slices < 1) slices = 1;
    if (!pair_ring_slices_valid(K, slices))
        return fail(W4A16_ERR_CONFIG, "paired ring kernel: max_blocks (K slices) 1..16, each slice non-empty");
    if (sk < 1) return fail(W4A16_ERR_CONFIG, "paired ring kernel: splits (wavefronts splitting K) must be positive");
    const int ppw = ppw_of(K, sk, slices);
    const int ms = row_slots(M);
    const SplitPick pk = slices > 1 ? pick_split(ms, sk, sn, ppw, depth) : SplitPick{pick(ms, sk, sn, ppw, depth), 1};
    const Kern kern = pk.kern;
    if (kern == nullptr)
        return fail(W4A16_ERR_CONFIG,
                    "paired ring kernel: (splits, rows, pairs per wavefront, unroll) not instantiated for this M; "
                    "M = 1: (1,3,8,8) (1,3,8,7) (1,3,8,6) (1,8,8,4) (2,2,8,8) (2,2,8,7) (1,8,16,6) (4,1,6,6) "
                    "(2,4,16,4) (2,4,16,6) (1,7,32,6) "
                    "(2,2,28,10) (2,4,56,6); M = 2..4: (4,1,2,2) (1,4,8,6) (2,2,8,4) (1,8,16,6) (8,1,3,3) "
                    "(2,4,16,4) (4,2,14,6) (1,4,8,7) (2,2,8,6); M = 5..8: (4,1,2,2) (1,4,8,6) (4,2,4,4) (1,8,16,6) (2,4,16,4) "
                    "(2,4,16,5); "
                    "M = 5..8 also (11,1,2,2); M = 9..16: (8,1,1,1) (4,2,2,2) (2,4,4,4) (1,4,8,4), and with K slices "
                    "(1,8,3,3) (1,8,14,4) "
                    "(1,8,16,4); M = 2..4 with K slices (1,8,28,4); M = 5..8 with K slices and two 8-row blocks "
                    "per wavefront (1,8,14,2) (1,8,16,3) (1,4,7,2)");
    const int64_t lds = w4a16::pair_ring_lds_bytes(ms, sk, sn, pk.rb, ppw);
    if (lds > kMaxLdsBytes) return fail(W4A16_ERR_CONFIG, "paired ring kernel: staging exceeds LDS");
    const int64_t need = pair_ring_workspace_bytes(M, N, slices);
    if (slices > 1 && (part == nullptr || part_bytes < need || (reinterpret_cast<uintptr_t>(part) & 15u)))
        return fail(W4A16_ERR_CONFIG, "paired ring kernel: K slices need a 16-byte aligned workspace of " +
                                          std::to_string(need) + " bytes (w4a16_linear_workspace_bytes)");
    int rc = ensure_lds(reinterpret_cast<const void*>(kern), (int)lds);
    if (rc != W4A16_OK) return rc;
    const int rows = 8 * sn * pk.rb;
    const int blocks = (N + rows - 1) / rows * slices;
    hipLaunchKernelGGL(kern, dim3(blocks), dim3(64 * sk * sn), (size_t)lds, stream, x, w, s, o, M, N, K,
                       static_cast<float*>(part), slices, w4a16::RingFusion{});
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(W4A16_ERR_LAUNCH, std::string("kernel launch failed: ") + hipGetErrorString(e));
    if (slices > 1 && reduce)
        return launch_split_reduce(slices, static_cast<const float*>(part), o, (int64_t)M * N, stream);
    return W4A16_OK;
}

// Fused decode-step GEMVs at M = 1 (the caller checks pointers and
// alignment; scales 4-byte aligned). kind 0: the SiLU form (N = inter, 2 N
// weight rows), RMSNorm when fz.norm_weight is set, K = 2048; kind 1: the
// residual add, K = 5632; kind 2: RMSNorm, K = 2048 (wide layers). Shapes
// from graph timing against the one-shot fused GEMVs (decode step of the
// 1.1B model): gate|up 2048 x 2 x 5632 with RMSNorm (1, 3, 8 pairs, 6 in
// flight, 2 blocks per wavefront) 4.39-4.41 us against 4.48-4.52 with 4 in
// flight (3: 4.82-4.87, 5: 4.72-4.75, 8: 4.87) and 4.85 on the one-shot
// form; down 5632 x 2048 with the residual (8 wavefronts on K, 3 pairs each)
// 3.31 against 3.45; lm_head 2048 x 32000 with RMSNorm (1, 4, 8 pairs, 6 in
// flight) 7.47-7.53 against 7.88-7.95 with all 8 in flight, 7.53-7.71 with
// 4, 7.92-8.17 on (1, 8, 8) and 8.18 on the one-shot form (12 rotated
// weight copies). Other shapes measured with 22-call graphs over 24 copies
// (wavefronts on K, on blocks, pairs, in flight): gate|up (2, 3, 4, 4)
// 4.80-4.86 and (4, 3, 2, 1) 5.22-5.26 against 4.46-4.52; down (4, 1, 6, 6)
// 3.67 and (11, 1, 2, 1) 3.75 against 3.56-3.58; lm_head (2, 4, 4, 4)
// 8.17-8.64. Returns W4A16_ERR_CONFIG for other shapes.
int launch_pair_ring_fused(int kind, const w4a16::f16* x, const w4a16::RingFusion& fz, const uint8_t* w,
                           const w4a16::f16* s, w4a16::f16* o, int N, int K, hipStream_t stream) {
    using namespace w4a16;
    Kern kern = nullptr;
    int sk = 1, sn = 1, rb = 1, ppw = 1;
    if (kind == 0 && K == 2048) {
        kern = fz.norm_weight ? gemv_pair_ring<1, 1, 3, 2, 8, 6, false, true, true>
                              : gemv_pair_ring<1, 1, 3, 2, 8, 6, false, true, false>;
        sk = 1, sn = 3, rb = 2, ppw = 8;
    } else if (kind == 1 && K == 5632 && fz.norm_weight == nullptr) {
        kern = gemv_pair_ring<1, 8, 1, 1, 3, 3, false, false, false, true>;
        sk = 8, sn = 1, rb = 1, ppw = 3;
    } else if (kind == 2 && K == 2048 && fz.norm_weight != nullptr) {
        kern = gemv_pair_ring<1, 1, 4, 1, 8, 6, false, false, true>;
        sk = 1, sn = 4, rb = 1, ppw = 8;
    }
    if (kern == nullptr) return fail(W4A16_ERR_CONFIG, "fused ring GEMV: shape not instantiated");
    const int64_t lds = pair_ring_lds_bytes(1, sk, sn, rb, ppw);
    int rc = ensure_lds(reinterpret_cast<const void*>(kern), (int)lds);
    if (rc != W4A16_OK) return rc;
    const int rows = 8 * sn;
    const int blocks = (N + rows - 1) / rows;
    hipLaunchKernelGGL(kern, dim3(blocks), dim3(64 * sk * sn), (size_t)lds, stream, x, w, s, o, 1, N, K,
                       (float*)nullptr, 1, fz);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(W4A16_ERR_LAUNCH, std::string("kernel launch failed: ") + hipGetErrorString(e));
    return W4A16_OK;
}

// The prompt's attention + o projection as the ring kernel's ATTN form
// (the caller checks shapes, pointers and alignment: T = 1..16, start + T <=
// 32, K = 64 x query heads, a multiple of 256, fz filled in): K / 256 slices
// of one pair (four query heads), sn wavefronts of rb 8-row blocks per
// workgroup, fp32 partial sums to part[slice][T][N]. Instantiated (sn, rb):
// (8, 1), (4, 1), (4, 2). Graph timing on the 1.1B model's o projection
// (16 tokens, 2048 x 2048): (8, 1) 6.09 us, (4, 2) 6.32, (8, 2) 6.87, (16,
// 1) 6.88, (4, 1) 8.27, against 4.17 + 4.64 for the attention and the o op
// as two launches.
int launch_pair_ring_attn(int sn, int rb, const w4a16::RingFusion& fz, int T, const uint8_t* w,
                          const w4a16::f16* s, int N, int K, float* part, hipStream_t stream) {
    using namespace w4a16;
    Kern kern = nullptr;
    if (sn == 4 && rb == 1) kern = gemv_pair_ring<16, 1, 4, 1, 1, 1, true, false, false, false, true>;
    else if (sn == 8 && rb == 1) kern = gemv_pair_ring<16, 1, 8, 1, 1, 1, true, false, false, false, true>;
    else if (sn == 4 && rb == 2) kern = gemv_pair_ring<16, 1, 4, 2, 1, 1, true, false, false, false, true>;
    if (kern == nullptr) return fail(W4A16_ERR_CONFIG, "attention + o ring kernel: shape not instantiated");
    const int64_t lds = (pair_ring_lds_bytes(16, 1, sn, rb, 1) + 15) / 16 * 16 + pair_ring_attn_lds_bytes();
    int rc = ensure_lds(reinterpret_cast<const void*>(kern), (int)lds);
    if (rc != W4A16_OK) return rc;
    const int rows = 8 * sn * rb;
    const int slices = K / 256;
    const int blocks = (N + rows - 1) / rows * slices;
    hipLaunchKernelGGL(kern, dim3(blocks), dim3(64 * sn), (size_t)lds, stream, (const f16*)nullptr, w, s,
                       (f16*)nullptr, T, N, K, part, slices, fz);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(W4A16_ERR_LAUNCH, std::string("kernel launch failed: ") + hipGetErrorString(e));
    return W4A16_OK;
}

int launch_pair_ring_silu(int sk, int sn, int depth, int M, const w4a16::f16* x, const uint8_t* w,
                          const w4a16::f16* s, w4a16::f16* o, int inter, int K, hipStream_t stream) {
    if (M < 9 || M > 16) return fail(W4A16_ERR_CONFIG, "paired ring SiLU kernel: 9 <= M <= 16");
    if (K < 256 || K % 256 != 0)
        return fail(W4A16_ERR_CONFIG, "paired ring SiLU kernel: K must be a multiple of 256 (an even group count)");
    if (reinterpret_cast<uintptr_t>(s) & 3u)
        return fail(W4A16_ERR_CONFIG, "paired ring SiLU kernel: scales must be 4-byte aligned");
    if (sk < 1) return fail(W4A16_ERR_CONFIG, "paired ring SiLU kernel: splits must be positive");
    const int ppw = ppw_of(K, sk, 1);
    Kern kern = pick_silu(sk, sn, ppw, depth);
    if (kern == nullptr) return fail(W4A16_ERR_CONFIG, "paired ring SiLU kernel: shape not instantiated");
    const int64_t lds = w4a16::pair_ring_lds_bytes(16, sk, sn, 2, ppw);
    if (lds > kMaxLdsBytes) return fail(W4A16_ERR_CONFIG, "paired ring SiLU kernel: staging exceeds LDS");
    int rc = ensure_lds(reinterpret_cast<const void*>(kern), (int)lds);
    if (rc != W4A16_OK) return rc;
    const int rows = 8 * sn;
    const int blocks = (inter + rows - 1) / rows;
    hipLaunchKernelGGL(kern, dim3(blocks), dim3(64 * sk * sn), (size_t)lds, stream, x, w, s, o, M, inter, K,
                       (float*)nullptr, 1, w4a16::RingFusion{});
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(W4A16_ERR_LAUNCH, std::string("kernel launch failed: ") + hipGetErrorString(e));
    return W4A16_OK;
}

}  // namespace w4a16_internal

// Launcher of the paired-layout ring GEMV (w4a16_pair_ring.h, M = 1..8) and
// its instantiations, in a translation unit of their own. Called by the
// dispatcher in w4a16_hip.hip.
#include "w4a16_hip.h"

#include <hip/hip_runtime.h>

#include <string>

#include "w4a16_pair_ring.h"

namespace w4a16_internal {
void set_last_error(const std::string& message);   // w4a16_hip.hip
int ensure_lds(const void* kernel, int bytes);     // w4a16_hip.hip: raise the dynamic-LDS limit once
}  // namespace w4a16_internal

namespace {

constexpr int kMaxLdsBytes = 160 * 1024;

int fail(int code, const std::string& message) {
    w4a16_internal::set_last_error(message);
    return code;
}

using Kern = void (*)(const w4a16::f16*, const uint8_t*, const w4a16::f16*, w4a16::f16*, int, int, int);

int row_slots(int M) { return M <= 1 ? 1 : M <= 4 ? 4 : 8; }

// Instantiated (row slots, wavefronts splitting K, wavefronts on 8-row
// blocks, pairs per wavefront, pairs in flight): the launch shapes the M = 1
// and M = 2..8 sweeps chose per row length (K = 256 x pairs).
Kern pick(int ms, int sk, int sn, int ppw, int depth) {
#define W4A16_P(MS, SK, SN, PPW, D) \
    if (ms == MS && sk == SK && sn == SN && ppw == PPW && depth == D) return w4a16::gemv_pair_ring<MS, SK, SN, 1, PPW, D>;
    // M = 1
    W4A16_P(1, 1, 3, 8, 8)    // K = 2048, N < 16384
    W4A16_P(1, 1, 8, 8, 4)    // K = 2048, N >= 16384
    W4A16_P(1, 2, 2, 8, 8)    // K = 4096, N < 8192
    W4A16_P(1, 1, 8, 16, 6)   // K = 4096, N >= 8192
    W4A16_P(1, 4, 1, 6, 6)    // K = 5376 .. 6144
    W4A16_P(1, 2, 4, 16, 4)   // K = 8192, N < 16384
    W4A16_P(1, 1, 7, 32, 6)   // K = 8192, N >= 16384
    W4A16_P(1, 2, 2, 28, 10)  // K = 14080 .. 14336
    W4A16_P(1, 2, 4, 56, 6)   // K = 28416 .. 28672
    // M = 2..4
    W4A16_P(4, 4, 1, 2, 2)    // K = 2048, N <= 2048
    W4A16_P(4, 1, 4, 8, 6)    // K = 2048, N <= 8192
    W4A16_P(4, 2, 2, 8, 4)    // K = 4096, N < 8192
    W4A16_P(4, 1, 8, 16, 6)   // K = 4096, N >= 8192
    W4A16_P(4, 8, 1, 3, 3)    // K = 5376 .. 6144 (M = 3, 4)
    W4A16_P(4, 2, 4, 16, 4)   // K = 8192, N <= 8192
    W4A16_P(4, 4, 2, 14, 6)   // K = 14080 .. 14336
    // M = 5..8
    W4A16_P(8, 4, 1, 2, 2)    // K = 2048, N <= 2048
    W4A16_P(8, 1, 4, 8, 6)    // K = 2048, N <= 8192
    W4A16_P(8, 4, 2, 4, 4)    // K = 4096, N < 8192
    W4A16_P(8, 1, 8, 16, 6)   // K = 4096, N >= 8192
    W4A16_P(8, 2, 4, 16, 4)   // K = 8192, N <= 8192
#undef W4A16_P
    return nullptr;
}

}  // namespace

namespace w4a16_internal {

// Pairs per wavefront for K split over `sk` wavefronts (G = K / 128 even).
int pair_ring_ppw(int64_t K, int sk) { return sk > 0 ? (int)((K / 256 + sk - 1) / sk) : 0; }

bool pair_ring_instantiated(int64_t M, int64_t K, int sk, int sn, int depth) {
    if (M < 1 || M > 8 || K < 256 || K % 256 != 0) return false;
    const int ppw = pair_ring_ppw(K, sk);
    const int ms = row_slots((int)M);
    return pick(ms, sk, sn, ppw, depth) != nullptr && w4a16::pair_ring_lds_bytes(ms, sk, sn, 1, ppw) <= kMaxLdsBytes;
}

int launch_pair_ring(int sk, int sn, int depth, int M, const w4a16::f16* x, const uint8_t* w, const w4a16::f16* s,
                     w4a16::f16* o, int N, int K, hipStream_t stream) {
    if (M < 1 || M > 8) return fail(W4A16_ERR_CONFIG, "paired ring kernel: 1 <= M <= 8");
    if (K < 256 || K % 256 != 0)
        return fail(W4A16_ERR_CONFIG, "paired ring kernel: K must be a multiple of 256 (an even group count)");
    if (reinterpret_cast<uintptr_t>(s) & 3u)
        return fail(W4A16_ERR_CONFIG, "paired ring kernel: scales must be 4-byte aligned");
    const int ppw = pair_ring_ppw(K, sk);
    const int ms = row_slots(M);
    Kern kern = pick(ms, sk, sn, ppw, depth);
    if (kern == nullptr)
        return fail(W4A16_ERR_CONFIG,
                    "paired ring kernel: (splits, rows, pairs per wavefront, unroll) not instantiated for this M; "
                    "M = 1: (1,3,8,8) (1,8,8,4) (2,2,8,8) (1,8,16,6) (4,1,6,6) (2,4,16,4) (1,7,32,6) "
                    "(2,2,28,10) (2,4,56,6); M = 2..4: (4,1,2,2) (1,4,8,6) (2,2,8,4) (1,8,16,6) (8,1,3,3) "
                    "(2,4,16,4) (4,2,14,6); M = 5..8: (4,1,2,2) (1,4,8,6) (4,2,4,4) (1,8,16,6) (2,4,16,4)");
    const int64_t lds = w4a16::pair_ring_lds_bytes(ms, sk, sn, 1, ppw);
    if (lds > kMaxLdsBytes) return fail(W4A16_ERR_CONFIG, "paired ring kernel: staging exceeds LDS");
    int rc = ensure_lds(reinterpret_cast<const void*>(kern), (int)lds);
    if (rc != W4A16_OK) return rc;
    const int rows = 8 * sn;
    const int blocks = (N + rows - 1) / rows;
    hipLaunchKernelGGL(kern, dim3(blocks), dim3(64 * sk * sn), (size_t)lds, stream, x, w, s, o, M, N, K);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(W4A16_ERR_LAUNCH, std::string("kernel launch failed: ") + hipGetErrorString(e));
    return W4A16_OK;
}

}  // namespace w4a16_internal

// Launcher of the paired-group MFMA GEMV (w4a16_pair.h) and its
// instantiations, in a translation unit of their own so they compile in
// parallel with w4a16_hip.hip. Called by the dispatcher in w4a16_hip.hip.
#include "w4a16_hip.h"

#include <hip/hip_runtime.h>

#include <string>

#include "w4a16_pair.h"

namespace w4a16_internal {
void set_last_error(const std::string& message);   // w4a16_hip.hip
int ensure_lds(const void* kernel, int bytes);     // w4a16_hip.hip: raise the dynamic-LDS limit once
}  // namespace w4a16_internal

namespace {

constexpr int kMaxLdsBytes = 160 * 1024;

int fail(int code, const char* message) {
    w4a16_internal::set_last_error(message);
    return code;
}

using Kern = void (*)(const w4a16::f16*, const uint8_t*, const w4a16::f16*, w4a16::f16*, int, int, int);

// Instantiated shapes: SK in {2, 4, 8} wavefronts splitting K, SN in {1, 2,
// 4, 8} row-block wavefronts with SK * SN <= 16, one 8-row block per
// wavefront, 1..8 group pairs per wavefront, 4 or 8 row slots.
template <int MS>
Kern pick(int sk, int sn, int rb, int gpw) {
    using namespace w4a16;
    if (rb != 1) return nullptr;
#define W4A16_G(SK, SN)                                                                                        \
    if (sk == SK && sn == SN) {                                                                                \
        switch (gpw) {                                                                                         \
            case 1: return gemv_mfma_pair<SK, SN, 1, 1, MS>;                                                   \
            case 2: return gemv_mfma_pair<SK, SN, 1, 2, MS>;                                                   \
            case 3: return gemv_mfma_pair<SK, SN, 1, 3, MS>;                                                   \
            case 4: return gemv_mfma_pair<SK, SN, 1, 4, MS>;                                                   \
            case 5: return gemv_mfma_pair<SK, SN, 1, 5, MS>;                                                   \
            case 6: return gemv_mfma_pair<SK, SN, 1, 6, MS>;                                                   \
            case 7: return gemv_mfma_pair<SK, SN, 1, 7, MS>;                                                   \
            case 8: return gemv_mfma_pair<SK, SN, 1, 8, MS>;                                                   \
            default: return nullptr;                                                                           \
        }                                                                                                      \
    }
    W4A16_G(2, 1) W4A16_G(2, 2) W4A16_G(2, 4) W4A16_G(2, 8)
    W4A16_G(4, 1) W4A16_G(4, 2) W4A16_G(4, 4)
    W4A16_G(8, 1) W4A16_G(8, 2)
#undef W4A16_G
    return nullptr;
}

}  // namespace

namespace w4a16_internal {

int64_t mfma_pair_lds_bytes(int64_t M, int64_t K, int sk, int sn, int rb, int gpw) {
    (void)K;
    return w4a16::pair_lds_bytes(M, (int64_t)sk * gpw, (int64_t)sk * sn, rb);
}

// Launch gemv_mfma_pair<sk, sn, rb, gpw> over [M, K] x [N, K]^T. The caller
// has checked pointers, group size 128 and 16-byte alignment.
int launch_mfma_pair(int sk, int sn, int rb, int gpw, int M, const void* x, const uint8_t* w, const void* s,
                     void* o, int N, int K, hipStream_t stream) {
    if (M < 2 || M > 8) return fail(W4A16_ERR_CONFIG, "paired MFMA kernel needs 2 <= M <= 8");
    if (K < 128 || K % 128 != 0) return fail(W4A16_ERR_CONFIG, "paired MFMA kernel: K must be a positive multiple of 128");
    const int G = K / 128;
    const int pairs = (G + 1) / 2;
    if (gpw == 0 && sk > 0) gpw = (pairs + sk - 1) / sk;   // the fewest pairs per wavefront that cover K
    if (gpw < 1 || (int64_t)sk * gpw < pairs)
        return fail(W4A16_ERR_CONFIG, "paired MFMA kernel: splits * unroll must cover the K / 256 group pairs");
    const Kern kern = M <= 4 ? pick<4>(sk, sn, rb, gpw) : pick<8>(sk, sn, rb, gpw);
    if (kern == nullptr)
        return fail(W4A16_ERR_CONFIG,
                    "paired MFMA kernel: splits 2, 4 or 8, wavefront blocks 1, 2, 4 or 8 with splits * blocks "
                    "<= 16, rows 1, unroll 1..8");
    const int64_t lds = mfma_pair_lds_bytes(M, K, sk, sn, rb, gpw);
    if (lds > kMaxLdsBytes) return fail(W4A16_ERR_CONFIG, "paired MFMA kernel: activations do not fit in LDS");
    const int rc = ensure_lds(reinterpret_cast<const void*>(kern), (int)lds);
    if (rc != W4A16_OK) return rc;
    const int rows = 8 * rb * sn;
    const int blocks = (N + rows - 1) / rows;
    hipLaunchKernelGGL(kern, dim3(blocks), dim3(64 * sk * sn), (size_t)lds, stream,
                       static_cast<const w4a16::f16*>(x), w, static_cast<const w4a16::f16*>(s),
                       static_cast<w4a16::f16*>(o), M, N, K);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_last_error(std::string("kernel launch failed: ") + hipGetErrorString(e));
        return W4A16_ERR_LAUNCH;
    }
    return W4A16_OK;
}

}  // namespace w4a16_internal

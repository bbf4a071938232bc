// Launcher of the W4A16 GEMM for prompts (w4a16_gemm.h) and its
// instantiations, in a translation unit of their own. Called by the
// dispatcher in w4a16_hip.hip.
#include "w4a16_hip.h"

#include <hip/hip_runtime.h>

#include <string>

#include "w4a16_gemm.h"

namespace w4a16_internal {
void set_last_error(const std::string& message);   // w4a16_hip.hip
int ensure_lds(const void* kernel, int bytes);     // w4a16_hip.hip: raise the dynamic-LDS limit once
}  // namespace w4a16_internal

namespace {

int fail(int code, const std::string& message) {
    w4a16_internal::set_last_error(message);
    return code;
}

using Kern = void (*)(const w4a16::f16*, const uint8_t*, const w4a16::f16*, w4a16::f16*, int, int, int, int);

// Instantiated shapes: MT in {1, 2, 4} activation tiles and RB in {1, 2, 4}
// weight tiles per wavefront, SK in {2, 4, 8} wavefronts splitting K, except
// MT = RB = 4 with 8 wavefronts (its 16 tiles spill within the 256 VGPRs of
// a 512-thread workgroup).
template <int MT, int RB>
Kern pick_sk(int sk) {
    using namespace w4a16;
    if (sk == 2) return gemm_w4a16<MT, RB, 2>;
    if (sk == 4) return gemm_w4a16<MT, RB, 4>;
    if constexpr (MT * RB < 16) {
        if (sk == 8) return gemm_w4a16<MT, RB, 8>;
    }
    return nullptr;
}

template <int MT>
Kern pick_rb(int rb, int sk) {
    if (rb == 1) return pick_sk<MT, 1>(sk);
    if (rb == 2) return pick_sk<MT, 2>(sk);
    if (rb == 4) return pick_sk<MT, 4>(sk);
    return nullptr;
}

Kern pick(int mt, int rb, int sk) {
    if (mt == 1) return pick_rb<1>(rb, sk);
    if (mt == 2) return pick_rb<2>(rb, sk);
    if (mt == 4) return pick_rb<4>(rb, sk);
    return nullptr;
}

}  // namespace

namespace w4a16_internal {

bool gemm_instantiated(int mt, int rb, int sk) { return pick(mt, rb, sk) != nullptr; }

// Every byte offset the kernel forms fits in 32 bits.
bool gemm_fits(int64_t M, int64_t N, int64_t K) {
    const int64_t lim = (int64_t)1 << 32;
    return K % 128 == 0 && K > 0 && N * (K / 2) < lim && M * K * 2 < lim && N * (K / 128) * 2 < lim;
}

// Launch gemm_w4a16 over [M, K] x [N, K]^T: mt activation tiles and rb
// weight tiles of 16 rows per wavefront, sk wavefronts splitting K. The
// caller has checked pointers, group size 128 and 16-byte alignment.
int launch_gemm(int mt, int rb, int sk, int M, const void* x, const uint8_t* w, const void* s, void* o, int N, int K,
                hipStream_t stream) {
    if (M < 1 || N < 1 || !gemm_fits(M, N, K))
        return fail(W4A16_ERR_CONFIG, "GEMM kernel: K must be a positive multiple of 128 and every operand below 4 GiB");
    const Kern kern = pick(mt, rb, sk);
    if (kern == nullptr)
        return fail(W4A16_ERR_CONFIG, "GEMM kernel: rows (activation tiles) 1, 2 or 4, max_blocks (weight tiles) 1, 2 "
                                      "or 4, splits 2, 4 or 8 (not 8 with rows = max_blocks = 4)");
    const int lds = (int)w4a16::gemm_lds_bytes(mt, rb, sk);
    int rc = ensure_lds(reinterpret_cast<const void*>(kern), lds);
    if (rc != W4A16_OK) return rc;
    const int nblocks = (N + 16 * rb - 1) / (16 * rb);
    const int mblocks = (M + 16 * mt - 1) / (16 * mt);
    const int64_t grid = (int64_t)((nblocks + 7) & ~7) * mblocks;
    if (grid > INT32_MAX) return fail(W4A16_ERR_TOO_LARGE, "GEMM kernel: too many workgroups");
    hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(64 * sk), (size_t)lds, stream,
                       static_cast<const w4a16::f16*>(x), w, static_cast<const w4a16::f16*>(s),
                       static_cast<w4a16::f16*>(o), M, N, K, nblocks);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(W4A16_ERR_LAUNCH, std::string("kernel launch failed: ") + hipGetErrorString(e));
    return W4A16_OK;
}

// LDS-staged GEMM (gemm2_w4a16): mt activation tiles and rb weight tiles per
// wavefront, sn wavefronts on weight tiles sharing each staged round, sk
// wavefronts splitting K. Instantiated: mt 2 or 4, rb 2 or 4, sn 2 or 4,
// sk 1, 2 or 4, except sk = 4 with sn = 4 and mt * rb >= 8 or with mt = rb =
// 4 (they spill).
namespace {
template <int MT, int RB, int SN>
Kern pick2_sk(int sk) {
    using namespace w4a16;
    if (sk == 1) return gemm2_w4a16<MT, RB, SN, 1>;
    if (sk == 2) return gemm2_w4a16<MT, RB, SN, 2>;
    // 16 wavefronts with 8+ tiles each, or 8 with 16 tiles, spill
    if constexpr (!((SN == 4 && MT * RB >= 8) || (MT * RB == 16))) {
        if (sk == 4) return gemm2_w4a16<MT, RB, SN, 4>;
    }
    return nullptr;
}
template <int MT, int RB>
Kern pick2_sn(int sn, int sk) {
    if (sn == 2) return pick2_sk<MT, RB, 2>(sk);
    if (sn == 4) return pick2_sk<MT, RB, 4>(sk);
    return nullptr;
}
template <int MT>
Kern pick2_rb(int rb, int sn, int sk) {
    if (rb == 2) return pick2_sn<MT, 2>(sn, sk);
    if (rb == 4) return pick2_sn<MT, 4>(sn, sk);
    return nullptr;
}
Kern pick2(int mt, int rb, int sn, int sk) {
    if (mt == 2) return pick2_rb<2>(rb, sn, sk);
    if (mt == 4) return pick2_rb<4>(rb, sn, sk);
    return nullptr;
}
}  // namespace

bool gemm2_instantiated(int mt, int rb, int sn, int sk) { return pick2(mt, rb, sn, sk) != nullptr; }

int launch_gemm2(int mt, int rb, int sn, int sk, int M, const void* x, const uint8_t* w, const void* s, void* o, int N,
                 int K, hipStream_t stream) {
    if (M < 1 || N < 1 || !gemm_fits(M, N, K))
        return fail(W4A16_ERR_CONFIG, "LDS GEMM kernel: K must be a positive multiple of 128 and every operand below 4 GiB");
    const Kern kern = pick2(mt, rb, sn, sk);
    if (kern == nullptr)
        return fail(W4A16_ERR_CONFIG, "LDS GEMM kernel: rows (activation tiles) 2 or 4, max_blocks (weight tiles) 2 or "
                                      "4, unroll (wavefronts sharing the staging) 2 or 4, splits 1, 2 or 4 (splits 4 "
                                      "needs unroll 2 and rows * max_blocks < 16, or rows * max_blocks < 8)");
    const int64_t lds = w4a16::gemm2_lds_bytes(mt, rb, sn, sk);
    if (lds > 160 * 1024) return fail(W4A16_ERR_CONFIG, "LDS GEMM kernel: staging exceeds LDS");
    int rc = ensure_lds(reinterpret_cast<const void*>(kern), (int)lds);
    if (rc != W4A16_OK) return rc;
    const int nblocks = (N + 16 * rb * sn - 1) / (16 * rb * sn);
    const int mblocks = (M + 16 * mt - 1) / (16 * mt);
    const int64_t grid = (int64_t)((nblocks + 7) & ~7) * mblocks;
    if (grid > INT32_MAX) return fail(W4A16_ERR_TOO_LARGE, "LDS GEMM kernel: too many workgroups");
    hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(64 * sn * sk), (size_t)lds, stream,
                       static_cast<const w4a16::f16*>(x), w, static_cast<const w4a16::f16*>(s),
                       static_cast<w4a16::f16*>(o), M, N, K, nblocks);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(W4A16_ERR_LAUNCH, std::string("kernel launch failed: ") + hipGetErrorString(e));
    return W4A16_OK;
}

// gemm_w4a16 with the SiLU-multiply epilogue of a [gate; up] pair: N = inter
// output columns, the weights 2 inter rows; rb weight tiles per wavefront
// (2 or 4: rb / 2 gate tiles and their up tiles).
namespace {
template <int MT, int RB>
Kern pick_silu_sk(int sk) {
    using namespace w4a16;
    if (sk == 2) return gemm_w4a16<MT, RB, 2, true>;
    if (sk == 4) return gemm_w4a16<MT, RB, 4, true>;
    if constexpr (MT * RB < 16) {
        if (sk == 8) return gemm_w4a16<MT, RB, 8, true>;
    }
    return nullptr;
}
Kern pick_silu(int mt, int rb, int sk) {
    if (rb == 2) {
        if (mt == 1) return pick_silu_sk<1, 2>(sk);
        if (mt == 2) return pick_silu_sk<2, 2>(sk);
        if (mt == 4) return pick_silu_sk<4, 2>(sk);
    }
    if (rb == 4) {
        if (mt == 1) return pick_silu_sk<1, 4>(sk);
        if (mt == 2) return pick_silu_sk<2, 4>(sk);
        if (mt == 4) return pick_silu_sk<4, 4>(sk);
    }
    return nullptr;
}
}  // namespace

bool gemm_silu_instantiated(int mt, int rb, int sk) { return pick_silu(mt, rb, sk) != nullptr; }

// gemm2_w4a16 with the SiLU-multiply epilogue: the LDS-staged GEMM's shapes
// for prompts of 128+ rows (4 activation tiles, one gate and one up tile per
// wavefront).
namespace {
Kern pick2_silu(int mt, int rb, int sn, int sk) {
    using namespace w4a16;
    if (mt != 4 || rb != 2) return nullptr;
    if (sn == 4 && sk == 1) return gemm2_w4a16<4, 2, 4, 1, true>;
    if (sn == 2 && sk == 2) return gemm2_w4a16<4, 2, 2, 2, true>;
    if (sn == 2 && sk == 4) return gemm2_w4a16<4, 2, 2, 4, true>;
    return nullptr;
}
}  // namespace

bool gemm2_silu_instantiated(int mt, int rb, int sn, int sk) { return pick2_silu(mt, rb, sn, sk) != nullptr; }

int launch_gemm2_silu(int mt, int rb, int sn, int sk, int M, const void* x, const uint8_t* w, const void* s, void* o,
                      int inter, int K, hipStream_t stream) {
    if (M < 1 || inter < 1 || !gemm_fits(M, 2 * (int64_t)inter, K))
        return fail(W4A16_ERR_CONFIG, "LDS GEMM kernel: K must be a positive multiple of 128 and every operand below 4 GiB");
    const Kern kern = pick2_silu(mt, rb, sn, sk);
    if (kern == nullptr) return fail(W4A16_ERR_CONFIG, "paired LDS GEMM kernel: no instantiation for this shape");
    const int64_t lds = w4a16::gemm2_lds_bytes(mt, rb, sn, sk);
    int rc = ensure_lds(reinterpret_cast<const void*>(kern), (int)lds);
    if (rc != W4A16_OK) return rc;
    const int nblocks = (inter + 8 * rb * sn - 1) / (8 * rb * sn);
    const int mblocks = (M + 16 * mt - 1) / (16 * mt);
    const int64_t grid = (int64_t)((nblocks + 7) & ~7) * mblocks;
    if (grid > INT32_MAX) return fail(W4A16_ERR_TOO_LARGE, "LDS GEMM kernel: too many workgroups");
    hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(64 * sn * sk), (size_t)lds, stream,
                       static_cast<const w4a16::f16*>(x), w, static_cast<const w4a16::f16*>(s),
                       static_cast<w4a16::f16*>(o), M, inter, K, nblocks);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(W4A16_ERR_LAUNCH, std::string("kernel launch failed: ") + hipGetErrorString(e));
    return W4A16_OK;
}

// GEMM on 32x32 tiles (gemm3_w4a16): mt activation tiles and rb weight
// tiles of 32 rows per wavefront, sn wavefronts on weight tiles sharing each
// staged round, sk wavefronts splitting K. Instantiated (M = 256 sweep of
// 4096 x 14336, 2048 x 11264 / 5632, 14336 x 4096, M = 128 4096 x 14336 and
// M = 512..2048 sweep): (mt, rb, sn, sk) = (4, 2, 4, 1), (4, 1, 4, 1),
// (2, 1, 4, 2), (2, 2, 2, 2), (2, 2, 4, 1), (4, 1, 2, 2), (2, 1, 2, 4) and
// (2, 1, 1, 4) (staging one round ahead: two register sets of 16 units would
// not fit); the SiLU-multiply form (rb / 2
// gate tiles and their up tiles) as (2, 2, 4, 1), (2, 2, 2, 2) and (2, 2, 1, 4)
// (one staging set).
namespace {
Kern pick3(int mt, int rb, int sn, int sk, bool paired) {
    using namespace w4a16;
    if (paired) {
        if (mt == 2 && rb == 2 && sn == 4 && sk == 1) return gemm3_w4a16<2, 2, 4, 1, true>;
        if (mt == 2 && rb == 2 && sn == 2 && sk == 2) return gemm3_w4a16<2, 2, 2, 2, true>;
        if (mt == 2 && rb == 2 && sn == 1 && sk == 4) return gemm3_w4a16<2, 2, 1, 4, true, 1>;
        return nullptr;
    }
    if (mt == 4 && rb == 2 && sn == 4 && sk == 1) return gemm3_w4a16<4, 2, 4, 1>;
    if (mt == 4 && rb == 1 && sn == 4 && sk == 1) return gemm3_w4a16<4, 1, 4, 1>;
    if (mt == 2 && rb == 1 && sn == 4 && sk == 2) return gemm3_w4a16<2, 1, 4, 2>;
    if (mt == 2 && rb == 2 && sn == 2 && sk == 2) return gemm3_w4a16<2, 2, 2, 2>;
    if (mt == 2 && rb == 2 && sn == 4 && sk == 1) return gemm3_w4a16<2, 2, 4, 1>;
    if (mt == 4 && rb == 1 && sn == 2 && sk == 2) return gemm3_w4a16<4, 1, 2, 2>;
    if (mt == 2 && rb == 1 && sn == 2 && sk == 4) return gemm3_w4a16<2, 1, 2, 4>;
    if (mt == 2 && rb == 1 && sn == 1 && sk == 4) return gemm3_w4a16<2, 1, 1, 4, false, 1>;   // one staging set: registers
    return nullptr;
}
}  // namespace

bool gemm3_instantiated(int mt, int rb, int sn, int sk, bool paired) { return pick3(mt, rb, sn, sk, paired) != nullptr; }

// paired: the SiLU-multiply epilogue over a [gate; up] pair, N = inter output
// columns and 2 inter weight rows.
int launch_gemm3(int mt, int rb, int sn, int sk, bool paired, int M, const void* x, const uint8_t* w, const void* s,
                 void* o, int N, int K, hipStream_t stream) {
    if (M < 1 || N < 1 || !gemm_fits(M, paired ? 2 * (int64_t)N : N, K))
        return fail(W4A16_ERR_CONFIG, "32x32 GEMM kernel: K must be a positive multiple of 128 and every operand below 4 GiB");
    const Kern kern = pick3(mt, rb, sn, sk, paired);
    if (kern == nullptr)
        return fail(W4A16_ERR_CONFIG, paired ? "paired 32x32 GEMM kernel: (rows, max_blocks, unroll, splits) must be "
                                               "(2, 2, 4, 1), (2, 2, 2, 2) or (2, 2, 1, 4)"
                                             : "32x32 GEMM kernel: (rows, max_blocks, unroll, splits) must be (4, 2, 4, "
                                               "1), (4, 1, 4, 1), (2, 1, 4, 2), (2, 2, 2, 2), (2, 2, 4, 1), (4, 1, 2, 2), "
                                               "(2, 1, 2, 4) or (2, 1, 1, 4)");
    const int64_t lds = w4a16::gemm3_lds_bytes(mt, rb, sn, sk);
    if (lds > 160 * 1024) return fail(W4A16_ERR_CONFIG, "32x32 GEMM kernel: staging exceeds LDS");
    int rc = ensure_lds(reinterpret_cast<const void*>(kern), (int)lds);
    if (rc != W4A16_OK) return rc;
    const int cols = (paired ? 16 : 32) * rb * sn;   // output columns per workgroup
    const int nblocks = (N + cols - 1) / cols;
    const int mblocks = (M + 32 * mt - 1) / (32 * mt);
    const int64_t grid = (int64_t)((nblocks + 7) & ~7) * mblocks;
    if (grid > INT32_MAX) return fail(W4A16_ERR_TOO_LARGE, "32x32 GEMM kernel: too many workgroups");
    hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(64 * sn * sk), (size_t)lds, stream,
                       static_cast<const w4a16::f16*>(x), w, static_cast<const w4a16::f16*>(s),
                       static_cast<w4a16::f16*>(o), M, N, K, nblocks);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(W4A16_ERR_LAUNCH, std::string("kernel launch failed: ") + hipGetErrorString(e));
    return W4A16_OK;
}

int launch_gemm_silu(int mt, int rb, int sk, int M, const void* x, const uint8_t* w, const void* s, void* o, int inter,
                     int K, hipStream_t stream) {
    if (M < 1 || inter < 1 || !gemm_fits(M, 2 * (int64_t)inter, K))
        return fail(W4A16_ERR_CONFIG, "GEMM kernel: K must be a positive multiple of 128 and every operand below 4 GiB");
    const Kern kern = pick_silu(mt, rb, sk);
    if (kern == nullptr) return fail(W4A16_ERR_CONFIG, "paired GEMM kernel: no instantiation for this shape");
    const int lds = (int)w4a16::gemm_lds_bytes(mt, rb, sk);
    int rc = ensure_lds(reinterpret_cast<const void*>(kern), lds);
    if (rc != W4A16_OK) return rc;
    const int nblocks = (inter + 8 * rb - 1) / (8 * rb);
    const int mblocks = (M + 16 * mt - 1) / (16 * mt);
    const int64_t grid = (int64_t)((nblocks + 7) & ~7) * mblocks;
    if (grid > INT32_MAX) return fail(W4A16_ERR_TOO_LARGE, "GEMM kernel: too many workgroups");
    hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(64 * sk), (size_t)lds, stream,
                       static_cast<const w4a16::f16*>(x), w, static_cast<const w4a16::f16*>(s),
                       static_cast<w4a16::f16*>(o), M, inter, K, nblocks);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(W4A16_ERR_LAUNCH, std::string("kernel launch failed: ") + hipGetErrorString(e));
    return W4A16_OK;
}

}  // namespace w4a16_internal

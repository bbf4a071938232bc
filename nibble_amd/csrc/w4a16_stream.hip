// Launcher of the streaming M = 1 GEMV (w4a16_stream.h) and its
// instantiations, in a translation unit of their own. Called by the
// dispatcher in w4a16_hip.hip.
#include "w4a16_hip.h"

#include <hip/hip_runtime.h>

#include <map>
#include <mutex>
#include <string>
#include <tuple>

#include "w4a16_stream.h"

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

using Kern = void (*)(const w4a16::f16*, const uint8_t*, const w4a16::f16*, w4a16::f16*, int, int);

// Instantiated shapes: R in {1, 2, 4} rows per task with D in {2, 3, 4} steps
// in flight, or R = 8 with D = 2 (deeper rings of 8 rows spill), W in {4, 8}
// wavefronts per workgroup; the activation units per thread cover K <= 16384
// (half) or K <= 32768 (full).
template <int W>
Kern pick_w(int rows, int depth, bool full) {
    using namespace w4a16;
    constexpr int kHalf = 32 / W, kFull = 64 / W;
#define W4A16_S(R, D)                                                                                         \
    if (rows == R && depth == D) return full ? gemv_stream<R, D, W, kFull> : gemv_stream<R, D, W, kHalf>;
    W4A16_S(1, 2) W4A16_S(1, 3) W4A16_S(1, 4)
    W4A16_S(2, 2) W4A16_S(2, 3) W4A16_S(2, 4)
    W4A16_S(4, 2) W4A16_S(4, 3) W4A16_S(4, 4)
    W4A16_S(8, 2)
#undef W4A16_S
    return nullptr;
}

Kern pick(int rows, int waves, int depth, int K) {
    const bool full = K > 16384;
    if (waves == 4) return pick_w<4>(rows, depth, full);
    if (waves == 8) return pick_w<8>(rows, depth, full);
    return nullptr;
}

// Workgroups of `kern` resident per CU with `lds` bytes of dynamic LDS, times
// the CU count; cached per (kernel, device, lds).
int resident_blocks(Kern kern, int waves, int lds, int* blocks) {
    static std::mutex mu;
    static std::map<std::tuple<const void*, int, int>, int> cache;
    int device = 0;
    if (hipGetDevice(&device) != hipSuccess) return fail(W4A16_ERR_LAUNCH, "hipGetDevice failed");
    const auto key = std::make_tuple(reinterpret_cast<const void*>(kern), device, lds);
    std::lock_guard<std::mutex> lock(mu);
    const auto it = cache.find(key);
    if (it != cache.end()) {
        *blocks = it->second;
        return W4A16_OK;
    }
    int per_cu = 0, cus = 0;
    hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void*>(kern),
                                                                64 * waves, (size_t)lds);
    if (e != hipSuccess)
        return fail(W4A16_ERR_LAUNCH, std::string("hipOccupancyMaxActiveBlocksPerMultiprocessor: ") +
                                          hipGetErrorString(e));
    e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device);
    if (e != hipSuccess)
        return fail(W4A16_ERR_LAUNCH, std::string("hipDeviceGetAttribute: ") + hipGetErrorString(e));
    if (per_cu < 1 || cus < 1) return fail(W4A16_ERR_CONFIG, "streaming kernel: no workgroup fits on a CU");
    *blocks = per_cu * cus;
    cache[key] = *blocks;
    return W4A16_OK;
}

}  // namespace

namespace w4a16_internal {

int64_t stream_lds_bytes(int64_t K) { return K * 2 + (K / 32) * 4; }

bool stream_instantiated(int rows, int waves, int depth, int64_t K) {
    return K <= 32768 && pick(rows, waves, depth, (int)K) != nullptr;
}

// Launch gemv_stream over [1, K] x [N, K]^T: `rows` rows per task, `waves`
// wavefronts per workgroup, `depth` 1 KiB steps per row in flight; the grid
// is the workgroups resident at once (or `max_blocks` when > 0), at most one
// per `waves` tasks. The caller has checked pointers, group size 128 and
// 16-byte alignment.
int launch_stream(int rows, int waves, int depth, int max_blocks, const void* x, const uint8_t* w, const void* s,
                  void* o, int N, int K, hipStream_t stream) {
    if (K < 128 || K % 128 != 0 || K > 32768)
        return fail(W4A16_ERR_CONFIG, "streaming kernel: K must be a multiple of 128 up to 32768");
    const Kern kern = pick(rows, waves, depth, K);
    if (kern == nullptr)
        return fail(W4A16_ERR_CONFIG, "streaming kernel: rows 1, 2 or 4 with unroll (steps in flight) 2, 3 or 4, or "
                                      "rows 8 with unroll 2; splits (wavefronts) 4 or 8");
    const int lds = (int)stream_lds_bytes(K);
    if (lds > kMaxLdsBytes) return fail(W4A16_ERR_CONFIG, "streaming kernel: activations do not fit in LDS");
    int rc = ensure_lds(reinterpret_cast<const void*>(kern), lds);
    if (rc != W4A16_OK) return rc;
    int blocks = max_blocks;
    if (blocks <= 0) {
        rc = resident_blocks(kern, waves, lds, &blocks);
        if (rc != W4A16_OK) return rc;
    }
    const int tasks = (N + rows - 1) / rows;
    const int need = (tasks + waves - 1) / waves;
    if (blocks > need) blocks = need;
    hipLaunchKernelGGL(kern, dim3(blocks), dim3(64 * waves), (size_t)lds, stream, static_cast<const w4a16::f16*>(x),
                       w, static_cast<const w4a16::f16*>(s), static_cast<w4a16::f16*>(o), N, K);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(W4A16_ERR_LAUNCH, std::string("kernel launch failed: ") + hipGetErrorString(e));
    return W4A16_OK;
}

}  // namespace w4a16_internal

// Launcher of the paired-group MFMA GEMV (w4a16_pair.h) and its
// instantiations, in a translation unit of their own so they compile in
// parallel with w4a16_hip.hip. Called by the dispatcher in w4a16_hip.hip.
#include "w4a16_hip.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <string>
#include <utility>

#include "w4a16_pair.h"

namespace w4a16_internal {
void set_last_error(const std::string& message);   // w4a16_hip.hip
int ensure_lds(const void* kernel, int bytes);     // w4a16_hip.hip: raise the dynamic-LDS limit once
}  // namespace w4a16_internal

namespace {

constexpr int kMaxLdsBytes = 160 * 1024;
constexpr int kChunkPairs = 8;   // group pairs per staged chunk (K = 2048 per chunk)
// Chunks whose loads are in flight ahead of the one being computed. M = 4
// and 8 sweeps (14336 x 4096, 8192 x 8192, 8192 x 28672, 28672 x 8192): 2
// beats 1 by 5-25% (M = 8, 14336 x 4096: 11.6 against 14.0 us) and beats
// requesting every chunk up front, where the later chunks' activations queue
// behind all of the weights.
constexpr int kLookahead = 2;

int fail(int code, const std::string& message) {
    w4a16_internal::set_last_error(message);
    return code;
}

using Kern = void (*)(const w4a16::f16*, const uint8_t*, const w4a16::f16*, w4a16::f16*, int, int, int);

// Instantiated shapes, whole rows staged (chunk = splits * unroll pairs):
// SK in {2, 4, 8} wavefronts splitting K, SN in {1, 2, 4, 8} row-block
// wavefronts with SK * SN <= 16, one 8-row block per wavefront, 1..8 group
// pairs per wavefront, 4 or 8 row slots.
template <int MS>
Kern pick_whole(int sk, int sn, int gpw) {
    using namespace w4a16;
#define W4A16_G(SK, SN)                                                                                        \
    if (sk == SK && sn == SN) {                                                                                \
        switch (gpw) {                                                                                         \
            case 1: return gemv_mfma_pair<SK, SN, 1, 1, MS, SK * 1>;                                           \
            case 2: return gemv_mfma_pair<SK, SN, 1, 2, MS, SK * 2>;                                           \
            case 3: return gemv_mfma_pair<SK, SN, 1, 3, MS, SK * 3>;                                           \
            case 4: return gemv_mfma_pair<SK, SN, 1, 4, MS, SK * 4>;                                           \
            case 5: return gemv_mfma_pair<SK, SN, 1, 5, MS, SK * 5>;                                           \
            case 6: return gemv_mfma_pair<SK, SN, 1, 6, MS, SK * 6>;                                           \
            case 7: return gemv_mfma_pair<SK, SN, 1, 7, MS, SK * 7>;                                           \
            case 8: return gemv_mfma_pair<SK, SN, 1, 8, MS, SK * 8>;                                           \
            default: return nullptr;                                                                           \
        }                                                                                                      \
    }
    W4A16_G(2, 1) W4A16_G(2, 2) W4A16_G(2, 4) W4A16_G(2, 8)
    W4A16_G(4, 1) W4A16_G(4, 2) W4A16_G(4, 4)
    W4A16_G(8, 1) W4A16_G(8, 2)
#undef W4A16_G
    return nullptr;
}

// Chunked staging (two buffers of kChunkPairs pairs): SK = 4 with SN in {1,
// 2, 4} and 7 or 8 pairs per wavefront, or SK = 8 with SN in {1, 2} and
// 3..8, 10, 12, 14 or 16. The SK = 8 kernels with 10 or more pairs per
// wavefront (rows longer than 16384) take each step's bias from 4 more MFMAs
// instead of the staging (MB): 3-7% faster at 28672 x 8192 (M = 4 and 8);
// neutral to 4% slower at 14336, 4-20% slower on shorter rows.
template <int MS>
Kern pick_chunked(int sk, int sn, int gpw) {
    using namespace w4a16;
    constexpr int C = kChunkPairs;
#define W4A16_G4(SN)                                                                                           \
    if (sk == 4 && sn == SN) {                                                                                 \
        if (gpw == 7) return gemv_mfma_pair<4, SN, 1, 7, MS, C, kLookahead>;                                               \
        if (gpw == 8) return gemv_mfma_pair<4, SN, 1, 8, MS, C, kLookahead>;                                               \
        return nullptr;                                                                                        \
    }
#define W4A16_G8(SN)                                                                                           \
    if (sk == 8 && sn == SN) {                                                                                 \
        switch (gpw) {                                                                                         \
            case 3: return gemv_mfma_pair<8, SN, 1, 3, MS, C, kLookahead>;                                                 \
            case 4: return gemv_mfma_pair<8, SN, 1, 4, MS, C, kLookahead>;                                                 \
            case 5: return gemv_mfma_pair<8, SN, 1, 5, MS, C, kLookahead>;                                                 \
            case 6: return gemv_mfma_pair<8, SN, 1, 6, MS, C, kLookahead>;                                                 \
            case 7: return gemv_mfma_pair<8, SN, 1, 7, MS, C, kLookahead>;                                                 \
            case 8: return gemv_mfma_pair<8, SN, 1, 8, MS, C, kLookahead>;                                                 \
            default: break;                                                                                    \
        }                                                                                                      \
        if constexpr (MS != 16) {                                                                              \
            switch (gpw) {                                                                                     \
                case 10: return gemv_mfma_pair<8, SN, 1, 10, MS, C, kLookahead, true>;                         \
                case 12: return gemv_mfma_pair<8, SN, 1, 12, MS, C, kLookahead, true>;                         \
                case 14: return gemv_mfma_pair<8, SN, 1, 14, MS, C, kLookahead, true>;                         \
                case 16: return gemv_mfma_pair<8, SN, 1, 16, MS, C, kLookahead, true>;                         \
                default: break;                                                                                \
            }                                                                                                  \
        }                                                                                                      \
        return nullptr;                                                                                        \
    }
    W4A16_G4(1) W4A16_G4(2) W4A16_G4(4) W4A16_G8(1) W4A16_G8(2)
#undef W4A16_G4
#undef W4A16_G8
    return nullptr;
}

// Staged pairs per chunk when the caller leaves it to the launcher: whole
// rows up to 16 pairs (K <= 4096) or while the workgroup's LDS stays within
// half of the CU's (two workgroups per CU), else kChunkPairs. Measured at M
// = 4 and 8: 8-pair chunks beat whole rows from K = 5632 (M = 8: 5632 x 2048
// 5.6 against 6.2 us, 8192 x 8192 12.3 against 13.7) and beat 16-pair chunks
// on the longest rows (M = 4, 28672 x 8192: 39.6 against 56.1 us).
int auto_chunk(int64_t M, int sk, int sn, int gpw) {
    const int64_t pairs = (int64_t)sk * gpw;
    if (pairs <= 16 || w4a16::pair_lds_bytes(M, pairs, pairs, (int64_t)sk * sn, 1) <= kMaxLdsBytes / 2)
        return (int)pairs;
    return kChunkPairs;
}

}  // namespace

namespace w4a16_internal {

int mfma_pair_auto_chunk(int64_t M, int sk, int sn, int gpw) { return auto_chunk(M, sk, sn, gpw); }

Kern pick(int64_t M, int sk, int sn, int chunk, int gpw) {
    if (chunk == sk * gpw)
        return M <= 4 ? pick_whole<4>(sk, sn, gpw) : M <= 8 ? pick_whole<8>(sk, sn, gpw) : pick_whole<16>(sk, sn, gpw);
    if (chunk == kChunkPairs)
        return M <= 4 ? pick_chunked<4>(sk, sn, gpw) : M <= 8 ? pick_chunked<8>(sk, sn, gpw)
                                                      : pick_chunked<16>(sk, sn, gpw);
    return nullptr;
}

bool mfma_pair_instantiated(int64_t M, int sk, int sn, int chunk, int gpw) {
    if (chunk == 0) chunk = auto_chunk(M, sk, sn, gpw);
    return pick(M, sk, sn, chunk, gpw) != nullptr;
}

// chunk: staged pairs per chunk, 0 = auto_chunk
int64_t mfma_pair_lds_bytes(int64_t M, int64_t K, int sk, int sn, int chunk, int gpw) {
    (void)K;
    const int64_t pairs = (int64_t)sk * gpw;
    if (chunk == 0) chunk = auto_chunk(M, sk, sn, gpw);
    return w4a16::pair_lds_bytes(M, pairs, chunk, (int64_t)sk * sn, 1);
}

// Launch gemv_mfma_pair over [M, K] x [N, K]^T: sk wavefronts splitting the
// pairs, sn row-block wavefronts per workgroup, gpw pairs per wavefront,
// `chunk` staged pairs per chunk (0 = auto_chunk; sk * gpw = whole rows).
// The caller has checked pointers, group size 128 and 16-byte alignment.
int launch_mfma_pair(int sk, int sn, int chunk, int gpw, int M, const void* x, const uint8_t* w, const void* s,
                     void* o, int N, int K, hipStream_t stream) {
    if (M < 2 || M > 16) return fail(W4A16_ERR_CONFIG, "paired MFMA kernel needs 2 <= M <= 16");
    if (K < 128 || K % 128 != 0) return fail(W4A16_ERR_CONFIG, "paired MFMA kernel: K must be a positive multiple of 128");
    const int G = K / 128;
    const int pairs = (G + 1) / 2;
    if (gpw == 0 && sk > 0) gpw = (pairs + sk - 1) / sk;   // the fewest pairs per wavefront that cover K
    if (gpw < 1 || (int64_t)sk * gpw < pairs)
        return fail(W4A16_ERR_CONFIG, "paired MFMA kernel: splits * unroll must cover the K / 256 group pairs");
    if (sk != 2 && sk != 4 && sk != 8) return fail(W4A16_ERR_CONFIG, "paired MFMA kernel: splits 2, 4 or 8");
    if (chunk == 0) chunk = auto_chunk(M, sk, sn, gpw);
    const Kern kern = pick(M, sk, sn, chunk, gpw);
    if (kern == nullptr)
        return fail(W4A16_ERR_CONFIG,
                    "paired MFMA kernel: no instantiation for this shape (whole rows, rows = splits * unroll: "
                    "splits 2, 4 or 8, blocks 1, 2, 4 or 8 with splits * blocks <= 16, unroll 1..8; chunks, rows = "
                    "8: splits 4 with blocks 1, 2 or 4 and unroll 7 or 8, or splits 8 with blocks 1 or 2 and "
                    "unroll 3..8, 10, 12, 14 or 16)");
    const int64_t lds = w4a16::pair_lds_bytes(M, (int64_t)sk * gpw, chunk, (int64_t)sk * sn, 1);
    if (lds > kMaxLdsBytes) return fail(W4A16_ERR_CONFIG, "paired MFMA kernel: activations do not fit in LDS");
    const int rc = ensure_lds(reinterpret_cast<const void*>(kern), (int)lds);
    if (rc != W4A16_OK) return rc;
    const int rows = 8 * sn;
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

// SiLU-multiply form of the 16-row-slot paired kernel (M = 9..16): each
// wavefront takes a block of 8 gate rows and the 8 up rows of the same
// output columns (inter + n), whole rows staged; out[m][n] = fp16(fp16(
// silu(fp16(g))) * fp16(u)). Instantiated: (sk, sn) in (2, 2), (2, 4),
// (4, 1), (4, 2), (8, 1), (8, 2), 1..8 pairs per wavefront.
namespace {
Kern pick_silu(int sk, int sn, int gpw) {
    using namespace w4a16;
#define W4A16_S(SK, SN)                                                                                        \
    if (sk == SK && sn == SN) {                                                                                \
        switch (gpw) {                                                                                         \
            case 1: return gemv_mfma_pair<SK, SN, 2, 1, 16, SK * 1, 64, false, true>;                          \
            case 2: return gemv_mfma_pair<SK, SN, 2, 2, 16, SK * 2, 64, false, true>;                          \
            case 3: return gemv_mfma_pair<SK, SN, 2, 3, 16, SK * 3, 64, false, true>;                          \
            case 4: return gemv_mfma_pair<SK, SN, 2, 4, 16, SK * 4, 64, false, true>;                          \
            case 5: return gemv_mfma_pair<SK, SN, 2, 5, 16, SK * 5, 64, false, true>;                          \
            case 6: return gemv_mfma_pair<SK, SN, 2, 6, 16, SK * 6, 64, false, true>;                          \
            case 7: return gemv_mfma_pair<SK, SN, 2, 7, 16, SK * 7, 64, false, true>;                          \
            case 8: return gemv_mfma_pair<SK, SN, 2, 8, 16, SK * 8, 64, false, true>;                          \
            default: return nullptr;                                                                           \
        }                                                                                                      \
    }
    W4A16_S(2, 2) W4A16_S(2, 4) W4A16_S(4, 1) W4A16_S(4, 2) W4A16_S(8, 1) W4A16_S(8, 2)
#undef W4A16_S
    return nullptr;
}
}  // namespace

int64_t mfma_pair_silu_lds_bytes(int64_t K, int sk, int sn, int gpw) {
    (void)K;
    const int64_t pairs = (int64_t)sk * gpw;
    return w4a16::pair_lds_bytes(16, pairs, pairs, (int64_t)sk * sn, 2);
}

bool mfma_pair_silu_instantiated(int sk, int sn, int gpw) { return pick_silu(sk, sn, gpw) != nullptr; }

// out [M, inter] = silu(x W_gate^T) * (x W_up^T) over the packed [gate; up]
// rows; M = 9..16. The caller has checked pointers, group size 128 and
// 16-byte alignment.
int launch_mfma_pair_silu(int sk, int sn, int gpw, int M, const void* x, const uint8_t* w, const void* s, void* o,
                          int inter, int K, hipStream_t stream) {
    if (M < 9 || M > 16) return fail(W4A16_ERR_CONFIG, "paired SiLU kernel needs 9 <= M <= 16");
    if (K < 128 || K % 128 != 0) return fail(W4A16_ERR_CONFIG, "paired SiLU kernel: K must be a positive multiple of 128");
    const int pairs = (K / 128 + 1) / 2;
    if (gpw < 1 || (int64_t)sk * gpw < pairs)
        return fail(W4A16_ERR_CONFIG, "paired SiLU kernel: splits * unroll must cover the K / 256 group pairs");
    const Kern kern = pick_silu(sk, sn, gpw);
    if (kern == nullptr) return fail(W4A16_ERR_CONFIG, "paired SiLU kernel: no instantiation for this shape");
    const int64_t lds = mfma_pair_silu_lds_bytes(K, sk, sn, gpw);
    if (lds > kMaxLdsBytes) return fail(W4A16_ERR_CONFIG, "paired SiLU kernel: activations do not fit in LDS");
    const int rc = ensure_lds(reinterpret_cast<const void*>(kern), (int)lds);
    if (rc != W4A16_OK) return rc;
    const int cols = 8 * sn;   // output columns per workgroup
    hipLaunchKernelGGL(kern, dim3((inter + cols - 1) / cols), dim3(64 * sk * sn), (size_t)lds, stream,
                       static_cast<const w4a16::f16*>(x), w, static_cast<const w4a16::f16*>(s),
                       static_cast<w4a16::f16*>(o), M, inter, K);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_last_error(std::string("kernel launch failed: ") + hipGetErrorString(e));
        return W4A16_ERR_LAUNCH;
    }
    return W4A16_OK;
}

// Streaming paired kernel (gemv_pair_stream): whole rows staged once per
// workgroup. depth = pairs in flight per wavefront (2, 3, 4 or 6); waves =
// wavefronts per workgroup (0: the fewest that cover the 8-row blocks with
// the workgroups that fit on the device at once by LDS, at most 16);
// max_blocks = grid cap (0: one workgroup per `waves` blocks).
int64_t pair_stream_lds(int64_t M, int64_t K) { return w4a16::pair_stream_lds_bytes(M, (K / 128 + 1) / 2); }

namespace {
using StreamKern = void (*)(const w4a16::f16*, const uint8_t*, const w4a16::f16*, w4a16::f16*, int, int, int,
                           float*, int);
template <int MS, bool SPLIT = false>
StreamKern pick_stream(int depth) {
    using namespace w4a16;
    switch (depth) {
        case 2: return gemv_pair_stream<MS, 2, SPLIT>;
        case 3: return gemv_pair_stream<MS, 3, SPLIT>;
        case 4: return gemv_pair_stream<MS, 4, SPLIT>;
        case 6: return gemv_pair_stream<MS, 6, SPLIT>;   // deeper rings spill within 128 VGPRs (1024 threads)
        default: return nullptr;
    }
}

using ReduceKern = void (*)(const float*, w4a16::f16*, int);
template <int... S>
ReduceKern reduce_table(int slices, std::integer_sequence<int, S...>) {
    static constexpr ReduceKern table[] = {w4a16::pair_split_reduce<S + 2>...};
    return table[slices - 2];
}
// pair_split_reduce<slices> for slices 2..16 (the launcher checks the range)
ReduceKern pick_reduce(int slices) { return reduce_table(slices, std::make_integer_sequence<int, 15>{}); }

int cu_count() {
    int cus = 0, device = 0;
    if (hipGetDevice(&device) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess || cus < 1)
        cus = 256;
    return cus;
}
}  // namespace

bool pair_stream_instantiated(int depth) { return pick_stream<8>(depth) != nullptr; }

int pair_stream_waves(int64_t M, int64_t N, int64_t K) {
    const int cus = cu_count();
    const int64_t per_cu = std::max<int64_t>(1, kMaxLdsBytes / std::max<int64_t>(1, pair_stream_lds(M, K)));
    const int64_t blocks = (N + 7) / 8;
    const int64_t resident = per_cu * cus;
    return (int)std::min<int64_t>(16, std::max<int64_t>(1, (blocks + resident - 1) / resident));
}

int launch_pair_stream(int depth, int waves, int max_blocks, int M, const void* x, const uint8_t* w, const void* s,
                       void* o, int N, int K, hipStream_t stream) {
    if (M < 2 || M > 8) return fail(W4A16_ERR_CONFIG, "streaming paired kernel needs 2 <= M <= 8");
    if (K < 128 || K % 128 != 0 || K > 32768)
        return fail(W4A16_ERR_CONFIG, "streaming paired kernel: K must be a multiple of 128 up to 32768");
    if ((int64_t)N * (K / 2) >= ((int64_t)1 << 32))
        return fail(W4A16_ERR_TOO_LARGE, "streaming paired kernel: weights must be below 4 GiB");
    const StreamKern kern = M <= 4 ? pick_stream<4>(depth) : pick_stream<8>(depth);
    if (kern == nullptr) return fail(W4A16_ERR_CONFIG, "streaming paired kernel: unroll (pairs in flight) 2, 3, 4 or 6");
    if (waves == 0) waves = pair_stream_waves(M, N, K);
    if (waves < 1 || waves > 16) return fail(W4A16_ERR_CONFIG, "streaming paired kernel: rows (wavefronts) 1..16");
    const int64_t lds = pair_stream_lds(M, K);
    if (lds > kMaxLdsBytes) return fail(W4A16_ERR_CONFIG, "streaming paired kernel: activations do not fit in LDS");
    const int rc = ensure_lds(reinterpret_cast<const void*>(kern), (int)lds);
    if (rc != W4A16_OK) return rc;
    const int blocks = (N + 7) / 8;
    int grid = (blocks + waves - 1) / waves;
    if (max_blocks > 0 && grid > max_blocks) grid = max_blocks;
    hipLaunchKernelGGL(kern, dim3(grid), dim3(64 * waves), (size_t)lds, stream, static_cast<const w4a16::f16*>(x), w,
                       static_cast<const w4a16::f16*>(s), static_cast<w4a16::f16*>(o), M, N, K, nullptr, 1);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_last_error(std::string("kernel launch failed: ") + hipGetErrorString(e));
        return W4A16_ERR_LAUNCH;
    }
    return W4A16_OK;
}

// Split-K streaming paired kernel: `slices` K slices of ceil(P / slices)
// pairs (P = K / 256 rounded up), each staged by its own workgroups; fp32
// partial sums in `part` ([slices][M][N], pair_split_workspace_bytes), then
// pair_split_reduce into `o`. waves = 0: the fewest wavefronts per workgroup
// (at most 16) with which slices x ceil(N / 8 / waves) workgroups fit on
// the device at once by LDS; max_blocks > 0 caps the workgroups per slice.
int64_t pair_split_lds(int64_t M, int64_t K, int slices) {
    const int64_t pairs = (K / 128 + 1) / 2;
    return w4a16::pair_stream_lds_bytes(M, (pairs + slices - 1) / slices);
}

int64_t pair_split_workspace_bytes(int64_t M, int64_t N, int slices) { return (int64_t)slices * M * N * 4; }

bool pair_split_valid(int64_t K, int slices) {
    const int64_t pairs = (K / 128 + 1) / 2;
    return slices >= 2 && slices <= 16 && (int64_t)(slices - 1) * ((pairs + slices - 1) / slices) < pairs;
}

int pair_split_waves(int64_t M, int64_t N, int64_t K, int slices) {
    const int64_t per_cu = std::max<int64_t>(1, kMaxLdsBytes / std::max<int64_t>(1, pair_split_lds(M, K, slices)));
    const int64_t resident = per_cu * cu_count();
    const int64_t blocks = (N + 7) / 8 * slices;
    return (int)std::min<int64_t>(16, std::max<int64_t>(1, (blocks + resident - 1) / resident));
}

// o = fp16(part[0] + .. + part[slices - 1]) over mn outputs, slices 2..16
// (the paired ring kernel's K slices).
int launch_split_reduce(int slices, const float* part, w4a16::f16* o, int64_t mn, hipStream_t stream) {
    if (slices < 2 || slices > 16) return fail(W4A16_ERR_CONFIG, "split-K reduce: 2..16 slices");
    hipLaunchKernelGGL(pick_reduce(slices), dim3((unsigned)((mn + 1023) / 1024)), dim3(256), 0, stream, part, o, (int)mn);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(W4A16_ERR_LAUNCH, std::string("kernel launch failed: ") + hipGetErrorString(e));
    return W4A16_OK;
}

int launch_pair_split(int depth, int waves, int slices, int max_blocks, int M, const void* x, const uint8_t* w,
                      const void* s, void* o, int N, int K, void* part, int64_t part_bytes, hipStream_t stream) {
    if (M < 2 || M > 8) return fail(W4A16_ERR_CONFIG, "split-K paired kernel needs 2 <= M <= 8");
    if (K < 128 || K % 128 != 0 || K > 65536)
        return fail(W4A16_ERR_CONFIG, "split-K paired kernel: K must be a multiple of 128 up to 65536");
    if ((int64_t)N * (K / 2) >= ((int64_t)1 << 32))
        return fail(W4A16_ERR_TOO_LARGE, "split-K paired kernel: weights must be below 4 GiB");
    if (!pair_split_valid(K, slices))
        return fail(W4A16_ERR_CONFIG, "split-K paired kernel: splits (K slices) 2..16, each slice non-empty");
    const StreamKern kern = M <= 4 ? pick_stream<4, true>(depth) : pick_stream<8, true>(depth);
    if (kern == nullptr) return fail(W4A16_ERR_CONFIG, "split-K paired kernel: unroll (pairs in flight) 2, 3, 4 or 6");
    if (waves == 0) waves = pair_split_waves(M, N, K, slices);
    if (waves < 1 || waves > 16) return fail(W4A16_ERR_CONFIG, "split-K paired kernel: rows (wavefronts) 1..16");
    const int64_t need = pair_split_workspace_bytes(M, N, slices);
    if (part == nullptr || part_bytes < need || (reinterpret_cast<uintptr_t>(part) & 15u))
        return fail(W4A16_ERR_CONFIG, "split-K paired kernel: needs a 16-byte aligned workspace of " +
                                          std::to_string(need) + " bytes (w4a16_linear_workspace_bytes)");
    const int64_t lds = pair_split_lds(M, K, slices);
    if (lds > kMaxLdsBytes) return fail(W4A16_ERR_CONFIG, "split-K paired kernel: a slice does not fit in LDS");
    const int rc = ensure_lds(reinterpret_cast<const void*>(kern), (int)lds);
    if (rc != W4A16_OK) return rc;
    int per_slice = ((N + 7) / 8 + waves - 1) / waves;
    if (max_blocks > 0 && per_slice > max_blocks) per_slice = max_blocks;
    hipLaunchKernelGGL(kern, dim3(per_slice * slices), dim3(64 * waves), (size_t)lds, stream,
                       static_cast<const w4a16::f16*>(x), w, static_cast<const w4a16::f16*>(s),
                       static_cast<w4a16::f16*>(o), M, N, K, static_cast<float*>(part), slices);
    hipError_t e = hipGetLastError();
    if (e == hipSuccess) {
        const int64_t mn = (int64_t)M * N;
        hipLaunchKernelGGL(pick_reduce(slices), dim3((unsigned)((mn + 1023) / 1024)), dim3(256), 0, stream,
                           static_cast<const float*>(part), static_cast<w4a16::f16*>(o), (int)mn);
        e = hipGetLastError();
    }
    if (e != hipSuccess) {
        set_last_error(std::string("kernel launch failed: ") + hipGetErrorString(e));
        return W4A16_ERR_LAUNCH;
    }
    return W4A16_OK;
}

}  // namespace w4a16_internal

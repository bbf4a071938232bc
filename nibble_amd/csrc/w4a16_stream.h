// Streaming VALU GEMV for long rows at M = 1 (gfx950), group size 128.
//
// The grid is sized to the workgroups that are resident on the chip at
// once, so every workgroup stages the activation row in LDS a single time
// (offset-decode layout and per-chunk bias, as the one-shot kernel) and then
// stays until its rows are done. Each wavefront owns tasks of R output rows
// (task t covers rows t R .. t R + R - 1; tasks are dealt round-robin over
// the grid's wavefronts) and walks them along K in steps of one 1 KiB load
// per row (lane l takes chunk 64 s + l of step s; lanes past the row's last
// chunk re-read it and add 0). D steps are in flight at any time in a ring of
// registers: after computing the step in slot d the wavefront requests the
// step D later into the same slot, so each wavefront keeps D R KiB of loads
// outstanding while the VALU works, with no barrier after the staging.
//
// Compared with the one-shot kernel (every load of a wavefront requested at
// once, one wavefront per R rows): rows of 16384 weights and more need more
// activation LDS per workgroup than leaves room for the grid to be resident
// in one round, and the one-shot kernel then runs its grid in rounds that
// each start with a fresh staging and an HBM round trip. Here the staging is
// paid once per workgroup and the weight stream never drains.
//
// Loads are unconditional: past the last unit of a wavefront nothing more is
// requested (the loop's tail is peeled), and a wavefront with no task
// requests its first D steps on the grid's last task, computes nothing and
// stores nothing. Branches around loads would make the compiler wait for
// every outstanding load at the join. Rows shorter than D steps are fine:
// the ring simply holds steps of the next task (the first D requests may run
// past a wavefront's last task; their rows are clamped to N - 1 and their
// data is not used).
#pragma once

#include "w4a16_device.h"

namespace w4a16 {

template <int R>
struct StreamStep {
    u32x4 w[R];
    uint32_t s[R];   // fp16 bits of the chunk's group scale
};

// A = activation units of 16 bytes per thread, all requested ahead of the
// weights: the row's K / 8 units need K <= 512 A W, which the host checks.
template <int R, int D, int W, int A>
__global__ void __launch_bounds__(64 * W)
gemv_stream(const f16* __restrict__ x, const uint8_t* __restrict__ w, const f16* __restrict__ scales,
            f16* __restrict__ out, int N, int K) {
    extern __shared__ __align__(16) uint8_t smem[];
    u32x4* xs = reinterpret_cast<u32x4*>(smem);
    float* cbias = reinterpret_cast<float*>(smem + (size_t)K * 2);   // [C], after xs
    const int C = K >> 5;
    const int G = K >> 7;
    const uint32_t row_bytes = (uint32_t)(K >> 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int steps = (C + 63) >> 6;
    const int tasks = (N + R - 1) / R;
    const int task0 = blockIdx.x * W + wave;
    const int stride = gridDim.x * W;
    const int my_tasks = task0 < tasks ? (tasks - 1 - task0) / stride + 1 : 0;
    const int units = my_tasks * steps;

    // 1. the activation row: units i = 4 c + q (chunk c, quarter q), all
    // requested before any weight (a wavefront's loads return in order)
    constexpr int T = 64 * W;
    const int aunits = 4 * C;
    u32x4 a[A];
#pragma unroll
    for (int p = 0; p < A; ++p) {
        const int i = min((int)threadIdx.x + p * T, aunits - 1);
        a[p] = *reinterpret_cast<const u32x4*>(x + (size_t)i * 8);
    }

    // 2. the first D steps of this wavefront's first task
    auto load = [&](StreamStep<R>& b, int task, int step) {
        const uint32_t c = (uint32_t)min(step * 64 + lane, C - 1);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int n = min(task * R + r, N - 1);
            b.s[r] = reinterpret_cast<const uint16_t*>(scales)[(size_t)n * G + (c >> 2)];
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int n = min(task * R + r, N - 1);
            const uint8_t* wrow = w + (size_t)n * row_bytes;   // wavefront-uniform
            b.w[r] = load_stream(reinterpret_cast<const u32x4*>(wrow + c * 16u));
        }
    };
    StreamStep<R> ring[D];
    int lt = min(task0, tasks - 1), ls = 0;   // next step to request
#pragma unroll
    for (int d = 0; d < D; ++d) {
        load(ring[d], lt, ls);
        if (++ls == steps) { ls = 0; lt += stride; }
    }
    __builtin_amdgcn_sched_barrier(0);

    // 3. stage: offset layout, xs[q * C + c], and the chunk's bias
#pragma unroll
    for (int p = 0; p < A; ++p) {
        const int i = threadIdx.x + p * T;
        float bias;
        const u32x4 v = stage_offset(a[p], bias);
        if (i < aunits) {
            xs[(i & 3) * C + (i >> 2)] = v;
            if ((i & 3) == 0) cbias[i >> 2] = bias;
        }
    }
    __syncthreads();
    if (units == 0) return;

    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.0f;
    int ct = task0, cs = 0;   // step being computed

    auto compute = [&](const StreamStep<R>& b) {
        const int c = cs * 64 + lane;
        const int cc = min(c, C - 1);
        const float bias = cbias[cc];
        float d[R];
#pragma unroll
        for (int r = 0; r < R; ++r) d[r] = bias;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const u32x4 xv = xs[q * C + cc];
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const Codes8 cw = unpack8_offset(b.w[r][q]);
                d[r] = __builtin_amdgcn_fdot2(as_f16x2(xv.x), cw.p[0], d[r], false);
                d[r] = __builtin_amdgcn_fdot2(as_f16x2(xv.y), cw.p[1], d[r], false);
                d[r] = __builtin_amdgcn_fdot2(as_f16x2(xv.z), cw.p[2], d[r], false);
                d[r] = __builtin_amdgcn_fdot2(as_f16x2(xv.w), cw.p[3], d[r], false);
            }
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const float s = (float)__builtin_bit_cast(f16, (uint16_t)b.s[r]);
            acc[r] = __builtin_fmaf(c < C ? d[r] : 0.0f, s, acc[r]);
        }
        if (cs == steps - 1) {
            // row sums: lane r stores row r of the task
            float mine = 0.0f;
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const float v = wave_sum(acc[r]);
                acc[r] = 0.0f;
                mine = lane == r ? v : mine;
            }
            const int n = ct * R + lane;
            if (lane < R && n < N) out[n] = (f16)mine;
            cs = 0;
            ct += stride;
        } else {
            ++cs;
        }
    };

    if (units < D) {   // fewer steps than the ring holds (short rows, one task)
#pragma unroll
        for (int d = 0; d < D; ++d)
            if (d < units) compute(ring[d]);
        return;
    }
    // 4. full rounds: every slot is refilled with a step that exists
    int u = 0;
    for (; u + 2 * D <= units; u += D) {
#pragma unroll
        for (int d = 0; d < D; ++d) {
            compute(ring[d]);
            load(ring[d], lt, ls);
            if (++ls == steps) { ls = 0; lt += stride; }
        }
    }
    // 5. the last D .. 2 D - 1 steps
#pragma unroll
    for (int d = 0; d < D; ++d) {
        compute(ring[d]);
        if (u + D + d < units) {
            load(ring[d], lt, ls);
            if (++ls == steps) { ls = 0; lt += stride; }
        }
    }
#pragma unroll
    for (int d = 0; d < D; ++d)
        if (u + D + d < units) compute(ring[d]);
}

}  // namespace w4a16

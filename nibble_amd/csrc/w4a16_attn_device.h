// Device-side building blocks shared by the attention kernels (the decode
// step's, the prompt's and the attention prologue of the ring GEMV): lane
// reductions across a wavefront and across its four 16-lane rows, the
// transposing LDS read that feeds V^T to the matrix cores, and the rotary
// embedding of one 8-dim unit.
#pragma once

#include "w4a16_device.h"

namespace w4a16 {

__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp<0xB1>(v));
    v = fmaxf(v, dpp<0x4E>(v));
    v = fmaxf(v, dpp<0x141>(v));
    v = fmaxf(v, dpp<0x140>(v));
    const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
    const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
    const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
    const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
    return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

__device__ __forceinline__ void wave_lds_sync() {
    // LDS operations of one wavefront complete in order; this only keeps the
    // compiler from moving LDS accesses across the point
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

typedef short v4i16 __attribute__((ext_vector_type(4)));

// Max / sum of v over lanes l, l ^ 16, l ^ 32 and l ^ 48 (the four 16-lane
// rows), in every lane: v_permlane16_swap / v_permlane32_swap hand each lane
// its partner's value without LDS. Sums pair the rows as (r0 + r1) + (r2 + r3)
// in every lane, so all lanes hold the same bits.
__device__ __forceinline__ float row_pair_max(float v) {
    const auto a = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, v), __builtin_bit_cast(uint32_t, v),
                                                    false, false);
    v = fmaxf(__builtin_bit_cast(float, (uint32_t)a[0]), __builtin_bit_cast(float, (uint32_t)a[1]));
    const auto b = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, v), __builtin_bit_cast(uint32_t, v),
                                                    false, false);
    return fmaxf(__builtin_bit_cast(float, (uint32_t)b[0]), __builtin_bit_cast(float, (uint32_t)b[1]));
}

__device__ __forceinline__ float row_pair_sum(float v) {
    const auto a = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, v), __builtin_bit_cast(uint32_t, v),
                                                    false, false);
    v = __builtin_bit_cast(float, (uint32_t)a[0]) + __builtin_bit_cast(float, (uint32_t)a[1]);
    const auto b = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, v), __builtin_bit_cast(uint32_t, v),
                                                    false, false);
    return __builtin_bit_cast(float, (uint32_t)b[0]) + __builtin_bit_cast(float, (uint32_t)b[1]);
}

// ds_read_b64_tr_b16 at an LDS address (see attn_o_kernel for the lane mapping)
__device__ __forceinline__ uint2 lds_read_tr16(const f16* p) {
    const v4i16 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) v4i16*)(reinterpret_cast<uintptr_t>(p)));
    return __builtin_bit_cast(uint2, v);
}

// Rotary embedding, half-split convention, of head dims d = 8 b .. 8 b + 7
// (a, fp16 pairs) and 32 + d (z): lo = fp16(scale (a c - z s)) and hi =
// fp16(scale (z c + a s)) in fp32, c / s the rotary tables' values at dims d.
// scale is 1 for keys and the score scale 1/8 for queries (a power of two:
// the fp16 rounding of the scaled value is the scaled rounding).
__device__ __forceinline__ void rope8(u32x4 a, u32x4 z, const float (&c)[8], const float (&s)[8], float scale,
                                      u32x4& lo, u32x4& hi) {
#pragma unroll
    for (int h = 0; h < 4; ++h) {
        const f16x2 x = as_f16x2(a[h]), y = as_f16x2(z[h]);
        const float c0 = c[2 * h], c1 = c[2 * h + 1], s0 = s[2 * h], s1 = s[2 * h + 1];
        const f16x2 l = {(f16)(scale * ((float)x.x * c0 - (float)y.x * s0)),
                         (f16)(scale * ((float)x.y * c1 - (float)y.y * s1))};
        const f16x2 u = {(f16)(scale * ((float)y.x * c0 + (float)x.x * s0)),
                         (f16)(scale * ((float)y.y * c1 + (float)x.y * s1))};
        lo[h] = as_u32(l);
        hi[h] = as_u32(u);
    }
}

}  // namespace w4a16

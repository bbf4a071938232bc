// Device-side building blocks for the gfx950 W4A16 kernels: fp16 vector
// types, the exact nibble -> fp16 unpack, the activation permutation that
// matches it, and a DPP wavefront reduction.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace w4a16 {

typedef _Float16 f16;
typedef f16 f16x2 __attribute__((ext_vector_type(2)));
typedef f16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f16x2 as_f16x2(uint32_t v) { return __builtin_bit_cast(f16x2, v); }
__device__ __forceinline__ uint32_t as_u32(f16x2 v) { return __builtin_bit_cast(uint32_t, v); }

// Stores of results a later launch reads, written through to memory:
// system-scope stores (vector stores with the sc0 sc1 bits), which the L2
// does not keep dirty, so the release at the end of the launch has none of
// them left to write back. 16-byte values go out as two 8-byte stores (there
// is no 16-byte atomic store). Used where a wavefront stores contiguous runs
// (the ring kernel's 8-row outputs, whole normalised rows); where one lane
// of each wavefront stores two scattered fp16 values (the one-shot GEMV's
// q|k|v + rotary + KV append, attention + o's residual rows), ordinary stores
// measured faster: each scattered write-through store is its own partial-line
// write, which the L2 otherwise merges (decode 2779 tok/s with them plain,
// 2662 / 2669 with either written through, 2563 with both).
__device__ __forceinline__ void store_through(f16* p, f16 v) {
    __hip_atomic_store(reinterpret_cast<short*>(p), __builtin_bit_cast(short, v), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_SYSTEM);
}
__device__ __forceinline__ void store_through(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
__device__ __forceinline__ void store_through(int64_t* p, int64_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
__device__ __forceinline__ void store_through(uint2* p, uint2 v) {
    __hip_atomic_store(reinterpret_cast<uint64_t*>(p), (uint64_t)v.x | ((uint64_t)v.y << 32), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_SYSTEM);
}
__device__ __forceinline__ void store_through(u32x4* p, u32x4 v) {
    uint64_t* q = reinterpret_cast<uint64_t*>(p);
    __hip_atomic_store(q, (uint64_t)v.x | ((uint64_t)v.y << 32), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    __hip_atomic_store(q + 1, (uint64_t)v.z | ((uint64_t)v.w << 32), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// v_perm_b32: byte i of the result is byte sel[i] of the 8-byte value {hi:lo}
// (selector 0-3 = lo bytes, 4-7 = hi bytes, 0x0c = zero byte).
__device__ __forceinline__ uint32_t perm(uint32_t hi, uint32_t lo, uint32_t sel) {
    return __builtin_amdgcn_perm(hi, lo, sel);
}

// ---------------------------------------------------------------------------
// Nibble unpack.
//
// Packing (reference w4a16/quantization.py:17-26): byte j of a row holds
// weight 2j in its low nibble and 2j+1 in its high nibble, two's complement,
// so nibble i of a little-endian 32-bit word is weight i of that word.
//
// Flipping bit 3 turns a two's-complement nibble s into the offset value
// s+8 in [0, 15]. OR-ing a 4-bit value v into the mantissa of binary16 1024.0
// (0x6400, exponent 2^10, unit last place 1) gives exactly 1024 + v; placed
// one nibble higher it gives 1024 + 16 v. One packed f16 add or fma then
// recovers s exactly:
//   (1024 + v) - 1032          = v - 8 = s
//   (1024 + 16 v) / 16 - 72    = v - 8 = s
// All intermediate values are integers below 2048 (or exact multiples of
// 1/16 of them), so every step is exact in binary16.
//
// unpack8 returns the 8 codes of one word as four f16 pairs in the order
// (s0,s4) (s1,s5) (s2,s6) (s3,s7); the activation side uses the same order
// (permute8 below), so a pairwise dot of the two is the plain dot product.
// ---------------------------------------------------------------------------
struct Codes8 {
    f16x2 p[4];
};

__device__ __forceinline__ Codes8 unpack8(uint32_t word) {
    // v_bitop3 computes (word & mask) ^ c in one instruction; c = the 0x6400
    // magic OR the nibble's bit-3 flip (two's complement -> offset binary),
    // which never overlaps the mask bits.
    const uint32_t v = word >> 8;
    const f16x2 bias_lo = {(f16)-1032.0f, (f16)-1032.0f};
    const f16x2 mul_hi = {(f16)0.0625f, (f16)0.0625f};
    const f16x2 bias_hi = {(f16)-72.0f, (f16)-72.0f};
    Codes8 c;
    c.p[0] = as_f16x2(__builtin_amdgcn_bitop3_b32(word, 0x000F000Fu, 0x64086408u, 0x6A)) + bias_lo;
    c.p[1] = __builtin_elementwise_fma(
        as_f16x2(__builtin_amdgcn_bitop3_b32(word, 0x00F000F0u, 0x64806480u, 0x6A)), mul_hi, bias_hi);
    c.p[2] = as_f16x2(__builtin_amdgcn_bitop3_b32(v, 0x000F000Fu, 0x64086408u, 0x6A)) + bias_lo;
    c.p[3] = __builtin_elementwise_fma(
        as_f16x2(__builtin_amdgcn_bitop3_b32(v, 0x00F000F0u, 0x64806480u, 0x6A)), mul_hi, bias_hi);
    return c;
}

// Natural-order unpack of one byte b (0..3) of a word: returns the f16 pair
// (weight 2b, weight 2b+1) = (low nibble, high nibble), exact.
template <int B>
__device__ __forceinline__ f16x2 unpack_byte_pair(uint32_t u_offset) {
    // byte B copied to result bytes 0 and 2, zero elsewhere
    constexpr uint32_t sel = (0x0Cu << 24) | (uint32_t(B) << 16) | (0x0Cu << 8) | uint32_t(B);
    const uint32_t t = (perm(u_offset, u_offset, sel) & 0x00F0000Fu) | 0x64006400u;
    const f16x2 mul = {(f16)1.0f, (f16)0.0625f};
    const f16x2 bias = {(f16)-1032.0f, (f16)-72.0f};
    return __builtin_elementwise_fma(as_f16x2(t), mul, bias);
}

// out = fp16(fp16(silu(fp16(g))) * fp16(u)) for fp32 sums g, u: the
// roundings of silu(gate) * up on a GEMM's fp16 outputs.
__device__ __forceinline__ f16 gemm_silu_mul(float g, float u) {
    const float gh = (float)(f16)g;
    const f16 sg = (f16)(gh / (1.0f + __expf(-gh)));
    return (f16)((float)sg * (float)(f16)u);
}

// Activation permutation matching unpack8: 8 consecutive halves x0..x7 held
// as words a=(x0,x1) b=(x2,x3) c=(x4,x5) e=(x6,x7) become
// (x0,x4) (x1,x5) (x2,x6) (x3,x7).
__device__ __forceinline__ u32x4 permute8(u32x4 a) {
    u32x4 o;
    o.x = perm(a.z, a.x, 0x05040100u);
    o.y = perm(a.z, a.x, 0x07060302u);
    o.z = perm(a.w, a.y, 0x05040100u);
    o.w = perm(a.w, a.y, 0x07060302u);
    return o;
}

// ---------------------------------------------------------------------------
// Wavefront (64-lane) sum. DPP quad_perm / row mirrors reduce each row of 16
// lanes without touching LDS; the four row sums are then read as scalars.
// Every lane must be active.
// ---------------------------------------------------------------------------
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __builtin_bit_cast(
        float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

__device__ __forceinline__ float wave_sum(float v) {
    v += dpp<0xB1>(v);   // quad_perm [1,0,3,2]
    v += dpp<0x4E>(v);   // quad_perm [2,3,0,1]
    v += dpp<0x141>(v);  // row_half_mirror: lane i <- lane 7-i of its 8
    v += dpp<0x140>(v);  // row_mirror:      lane i <- lane 15-i of its 16
    const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
    const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
    const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
    const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
    return (r0 + r1) + (r2 + r3);
}

__device__ __forceinline__ u32x4 load_stream(const u32x4* p) {
    return __builtin_nontemporal_load(p);
}

// Decode without f16 fix-ups for the offset path: pairs (0,4) (2,6) as
// 1024 + v and pairs (1,5) (3,7) as 1024 + 16 v, v = s + 8.
__device__ __forceinline__ Codes8 unpack8_offset(uint32_t word) {
    const uint32_t v = word >> 8;
    Codes8 c;
    c.p[0] = as_f16x2(__builtin_amdgcn_bitop3_b32(word, 0x000F000Fu, 0x64086408u, 0x6A));
    c.p[1] = as_f16x2(__builtin_amdgcn_bitop3_b32(word, 0x00F000F0u, 0x64806480u, 0x6A));
    c.p[2] = as_f16x2(__builtin_amdgcn_bitop3_b32(v, 0x000F000Fu, 0x64086408u, 0x6A));
    c.p[3] = as_f16x2(__builtin_amdgcn_bitop3_b32(v, 0x00F000F0u, 0x64806480u, 0x6A));
    return c;
}

// One 16-byte activation unit for the offset decode: permuted to the
// unpack8 pair order with the odd-k pairs (.y, .w) scaled by 1/16; `bias`
// receives -(1032 sum_even x + 1152 sum_odd x/16) summed over the unit's DPP
// quad (the four units of one 32-weight chunk). Every lane of the wavefront
// must execute it (DPP), and the four lanes of a quad must hold the four
// units of one chunk.
__device__ __forceinline__ u32x4 stage_offset(u32x4 a, float& bias) {
    const f16x2 sixteenth = {(f16)0.0625f, (f16)0.0625f};
    u32x4 v = permute8(a);
    const f16x2 e0 = as_f16x2(v.x), e1 = as_f16x2(v.z);
    const f16x2 o0 = as_f16x2(v.y) * sixteenth, o1 = as_f16x2(v.w) * sixteenth;
    v.y = as_u32(o0);
    v.w = as_u32(o1);
    float part = 1032.0f * (((float)e0.x + (float)e0.y) + ((float)e1.x + (float)e1.y)) +
                 1152.0f * (((float)o0.x + (float)o0.y) + ((float)o1.x + (float)o1.y));
    part += dpp<0xB1>(part);   // quad_perm [1,0,3,2]
    part += dpp<0x4E>(part);   // quad_perm [2,3,0,1]
    bias = -part;
    return v;
}

}  // namespace w4a16

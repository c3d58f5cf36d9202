// vk_common.h — device helpers shared by the gfx950 kernels.
//
// Everything here is bit-exact with the reference's scalar definitions where
// a reference definition exists (cited per helper).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

typedef __bf16 vk_bf16x8 __attribute__((ext_vector_type(8)));
typedef float vk_f32x4 __attribute__((ext_vector_type(4)));
typedef float vk_f32x16 __attribute__((ext_vector_type(16)));

#define VK_WAVE 64

// Workgroup barrier for LDS hand-offs: this wave's LDS writes are complete,
// then all waves meet. Unlike __syncthreads() it does not fence global
// memory, so prefetched global loads stay in flight across it.
#define VK_LDS_BARRIER() asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory")

// binary16 -> f32, exact for every finite value; NaN decodes to the canonical
// quiet NaN 0x7FC00000 as f32::NAN does.
// crates/vokra-core/src/kv_quant/half.rs:53-69 (value-identical bit build).
__device__ __forceinline__ float vk_f16_to_f32(uint32_t h) {
    const uint32_t sign = (h >> 15) & 1u, exp = (h >> 10) & 0x1fu, mant = h & 0x3ffu;
    if (exp == 0x1fu) {
        return mant ? __uint_as_float(0x7fc00000u) : __uint_as_float((sign << 31) | 0x7f800000u);
    }
    if (exp == 0u) {
        const float v = (float)mant * 5.9604644775390625e-08f;  // mant * 2^-24, exact
        return sign ? -v : v;
    }
    return __uint_as_float((sign << 31) | ((exp + 112u) << 23) | (mant << 13));
}

// Branch-free binary16 -> f32 for hot loops (v_cvt_f32_f16): the same value
// as vk_f16_to_f32 for every non-NaN input, subnormals included; a NaN scale
// decodes to some quiet NaN rather than exactly 0x7FC00000.
__device__ __forceinline__ float vk_f16_to_f32_hw(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

// f32 -> binary16 with round-to-nearest-even; overflow -> inf, NaN -> 0x7E00
// with the sign kept, subnormals rounded. Same results as
// crates/vokra-core/src/kv_quant/half.rs:80-151 for every input.
__device__ __forceinline__ uint32_t vk_f32_to_f16_bits(float x) {
    const uint32_t bits = __float_as_uint(x);
    const uint32_t sign = (bits >> 31) & 1u;
    const int exp32 = (int)((bits >> 23) & 0xffu);
    const uint32_t mant = bits & 0x007fffffu;
    if (exp32 == 0xff) return (sign << 15) | 0x7c00u | (mant ? 0x200u : 0u);
    if (exp32 == 0 && mant == 0) return sign << 15;
    const int e16 = exp32 - 112;
    if (e16 >= 0x1f) return (sign << 15) | 0x7c00u;
    if (e16 >= 1) {
        const uint32_t rb = (mant >> 12) & 1u;
        const bool sticky = (mant & 0xfffu) != 0;
        uint32_t t = mant >> 13;
        uint32_t e = (uint32_t)e16;
        if (rb && (sticky || (t & 1u))) ++t;
        if (t == 0x400u) {
            t = 0;
            if (++e >= 0x1fu) return (sign << 15) | 0x7c00u;
        }
        return (sign << 15) | (e << 10) | (t & 0x3ffu);
    }
    if (e16 < -10) return sign << 15;
    const uint32_t mi = mant | 0x00800000u;
    const uint32_t sh = (uint32_t)(1 - e16) + 13u;
    const uint32_t rb = (mi >> (sh - 1)) & 1u;
    const bool sticky = (mi & ((1u << (sh - 1)) - 1u)) != 0;
    uint32_t t = mi >> sh;
    if (rb && (sticky || (t & 1u))) ++t;
    if (t >= 0x400u) return (sign << 15) | 0x400u;
    return (sign << 15) | (t & 0x3ffu);
}

// bf16 bit pattern of a small integer |v| <= 256 (exact: the f32 has at most
// 9 significant bits, so its low 16 bits are zero).
__device__ __forceinline__ uint32_t vk_int_to_bf16_bits(int v) {
    return __float_as_uint((float)v) >> 16;
}

// Rust `f32::round` (half away from zero) — roundf is exactly that.
__device__ __forceinline__ float vk_round_half_away(float x) { return roundf(x); }

// Max-reduce over groups of `G` consecutive lanes (G power of two <= 64).
template <int G>
__device__ __forceinline__ float vk_group_max(float v) {
#pragma unroll
    for (int o = 1; o < G; o <<= 1) v = fmaxf(v, __shfl_xor(v, o, VK_WAVE));
    return v;
}

template <int G>
__device__ __forceinline__ int vk_group_sum_i(int v) {
#pragma unroll
    for (int o = 1; o < G; o <<= 1) v += __shfl_xor(v, o, VK_WAVE);
    return v;
}

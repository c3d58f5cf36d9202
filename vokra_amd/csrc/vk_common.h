// vk_common.h — device helpers shared by the gfx950 kernels.
//
// Everything here is bit-exact with the reference's scalar definitions where
// a reference definition exists (cited per helper).
#pragma once

#include <hip/hip_runtime.h>
#include "vk_launch.h"
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

// The half-split rotation of one pair (a = x[j], b = x[j + hd / 2]) with
// cs = (cos, sin) of its angle, as rope_apply forms it: the four products,
// then x[j] = a c - b s and x[j + hd / 2] = a s + b c.
__device__ __forceinline__ float vk_rope_lo(float a, float b, float2 cs) {
    const float ac = a * cs.x, bs = b * cs.y;
    return ac - bs;
}
__device__ __forceinline__ float vk_rope_hi(float a, float b, float2 cs) {
    const float as = a * cs.y, bc = b * cs.x;
    return as + bc;
}

// A finite f32 whose fp16 rounding is infinite (|x| >= 65520): the fp16
// hi / lo operands of the attention kernels cannot represent it.
__device__ __forceinline__ bool vk_f16_overflow(float x) {
    const float a = fabsf(x);
    return a >= 65520.0f && a <= 3.40282347e38f;
}

// The partner of a lane in a butterfly step over groups of 2 o lanes (lane
// ^ o), through the cheapest cross-lane path that delivers it: DPP for
// o <= 8 (a VALU operand modifier, no LDS round trip), ds_swizzle for o = 16,
// ds_bpermute for o = 32. For o = 4 and 8 the DPP is a mirror (lane i <- the
// lane 7 - i or 15 - i of its 8 / 16), which is the xor partner's value once
// the earlier steps have made every lane of a 4- / 8-lane group equal, so the
// butterfly's reductions (which only ever reach that state) get the same
// operands.
template <int O>
__device__ __forceinline__ int vk_bfly_partner(int v) {
    if constexpr (O == 1) return __builtin_amdgcn_mov_dpp(v, 0xB1, 0xf, 0xf, true);  // quad_perm [1,0,3,2]
    else if constexpr (O == 2) return __builtin_amdgcn_mov_dpp(v, 0x4E, 0xf, 0xf, true);  // quad_perm [2,3,0,1]
    else if constexpr (O == 4) return __builtin_amdgcn_mov_dpp(v, 0x141, 0xf, 0xf, true);  // row_half_mirror
    else if constexpr (O == 8) return __builtin_amdgcn_mov_dpp(v, 0x140, 0xf, 0xf, true);  // row_mirror
    else if constexpr (O == 16) return __builtin_amdgcn_ds_swizzle(v, 0x401F);  // bit mode: lane ^ 16 in 32
    else return __shfl_xor(v, O, VK_WAVE);
}

// Lane J of each 16-lane row, to every lane of that row (DPP row_newbcast).
template <int J>
__device__ __forceinline__ int vk_row_bcast_i(int v) {
    return __builtin_amdgcn_mov_dpp(v, 0x150 + J, 0xf, 0xf, true);
}

// Max-reduce over groups of `G` consecutive lanes (G power of two <= 64);
// every lane of a group ends with the group's value. The inputs must be
// +0 or positive and not NaN (the callers reduce fmaxf(0, |x|), which maps a
// NaN to 0 as the reference's fold from 0.0 does): on those, the order of
// the f32 values is the order of their bit patterns, so the reduction runs
// as an integer max whose DPP operand needs no NaN canonicalization.
template <int G>
__device__ __forceinline__ float vk_group_max(float v) {
    int b = __float_as_int(v);
#define VK_GMAX_STEP(O) if constexpr (G > (O)) b = max(b, vk_bfly_partner<(O)>(b));
    VK_GMAX_STEP(1) VK_GMAX_STEP(2) VK_GMAX_STEP(4) VK_GMAX_STEP(8) VK_GMAX_STEP(16) VK_GMAX_STEP(32)
#undef VK_GMAX_STEP
    return __int_as_float(b);
}

// The same butterflies for any f32 values (fmaxf: NaN ignored unless every
// value is NaN; sums add the same two partials per step as a shuffle
// butterfly in ascending steps).
template <int G>
__device__ __forceinline__ float vk_group_maxf(float v) {
#define VK_GMAXF_STEP(O) if constexpr (G > (O)) v = fmaxf(v, __int_as_float(vk_bfly_partner<(O)>(__float_as_int(v))));
    VK_GMAXF_STEP(1) VK_GMAXF_STEP(2) VK_GMAXF_STEP(4) VK_GMAXF_STEP(8) VK_GMAXF_STEP(16) VK_GMAXF_STEP(32)
#undef VK_GMAXF_STEP
    return v;
}
template <int G>
__device__ __forceinline__ float vk_group_sumf(float v) {
#define VK_GSUMF_STEP(O) if constexpr (G > (O)) v += __int_as_float(vk_bfly_partner<(O)>(__float_as_int(v)));
    VK_GSUMF_STEP(1) VK_GSUMF_STEP(2) VK_GSUMF_STEP(4) VK_GSUMF_STEP(8) VK_GSUMF_STEP(16) VK_GSUMF_STEP(32)
#undef VK_GSUMF_STEP
    return v;
}

template <int G>
__device__ __forceinline__ int vk_group_sum_i(int v) {
#define VK_GSUM_STEP(O) if constexpr (G > (O)) v += vk_bfly_partner<(O)>(v);
    VK_GSUM_STEP(1) VK_GSUM_STEP(2) VK_GSUM_STEP(4) VK_GSUM_STEP(8) VK_GSUM_STEP(16) VK_GSUM_STEP(32)
#undef VK_GSUM_STEP
    return v;
}

// Activation-pass arithmetic of one 32-element block (the convention of
// vk_quantize_act_b32), for producers that quantize their own output rows.
// amax = max |v| over the block from 0 through fmaxf (NaN ignored); when
// amax == 0 the scale and every q are 0.
__device__ __forceinline__ float vk_act_scale(float amax, bool pow2) {  // amax != 0
    float s = amax / 127.0f;
    if (pow2) {
        int ex;
        const float f = frexpf(s, &ex);  // s = f * 2^ex, f in [0.5, 1)
        s = ldexpf(1.0f, f == 0.5f ? ex - 1 : ex);
    }
    return s;
}
__device__ __forceinline__ int vk_act_q(float v, float s) {
    const float r = vk_round_half_away(v / s);
    return (r != r) ? 0 : (int)fminf(fmaxf(r, -127.0f), 127.0f);
}
// bf16 bits of the A operand: q, or q * 2^e under the power-of-two convention
__device__ __forceinline__ uint32_t vk_act_bits(int q, float s, bool pow2) {
    return pow2 ? (__float_as_uint((float)q * s) >> 16) : vk_int_to_bf16_bits(q);
}
// uint16 offset of element e (0..31) of k-block kb of row `row` in the A
// fragments [m_pad / 16][nb][64 lanes][8]: lane = row % 16 + 16 (e / 8).
__device__ __forceinline__ size_t vk_afrag_u16(size_t row, int kb, int nb, int e) {
    return ((((row >> 4) * (size_t)nb + kb) * 64) + (row & 15) + 16 * (e >> 3)) * 8 + (e & 7);
}

// GELU through the Abramowitz & Stegun 7.1.26 erf
// (crates/vokra-backend-cpu/src/kernels/scalar.rs:126-172). Shared by the GELU
// kernel and the GEMM epilogues, so a fused epilogue equals the separate pass.
__device__ __forceinline__ float vk_erf_as(float x) {
    const float P = 0.3275911f, A1 = 0.254829592f, A2 = -0.284496736f, A3 = 1.421413741f, A4 = -1.453152027f,
                A5 = 1.061405429f;
    const float sign = x < 0.0f ? -1.0f : 1.0f;
    const float ax = fabsf(x);
    const float t = 1.0f / (1.0f + P * ax);
    const float poly = ((((A5 * t + A4) * t + A3) * t + A2) * t + A1) * t;
    return sign * (1.0f - poly * expf(-ax * ax));
}
__device__ __forceinline__ float vk_gelu_as(float x) { return 0.5f * x * (1.0f + vk_erf_as(x * 0.70710678118654752440f)); }

// What a GEMM epilogue applies after the bias: y = gelu(y) (an MLP's first
// linear) and/or y = resid + y (a residual connection; resid may be the output
// buffer itself: each element is read and written by the same thread). The
// results equal the separate GELU / add passes bit for bit.
__device__ __forceinline__ float vk_epi_apply(float v, const VkEpi& e, size_t idx) {
    if (e.gelu) v = vk_gelu_as(v);
    if (e.resid) v = e.resid[idx] + v;
    return v;
}

// Sum over a 256-thread workgroup (4 waves): wave shuffle tree, then
// (w0 + w1) + (w2 + w3). `red` is 4 floats of LDS. Every row-reduction kernel
// that must agree bit for bit with another uses this one. Its barriers wait
// for LDS only (not for global loads in flight), so a caller's prefetch of
// the next row stays in flight across the reduction.
__device__ __forceinline__ float vk_block_sum256(float v, float* red) {
    // the butterfly over the wave in steps 1, 2, .., 32 (the partners of the
    // first five through DPP / swizzle, see vk_bfly_partner)
    v += __int_as_float(vk_bfly_partner<1>(__float_as_int(v)));
    v += __int_as_float(vk_bfly_partner<2>(__float_as_int(v)));
    v += __int_as_float(vk_bfly_partner<4>(__float_as_int(v)));
    v += __int_as_float(vk_bfly_partner<8>(__float_as_int(v)));
    v += __int_as_float(vk_bfly_partner<16>(__float_as_int(v)));
    v += __shfl_xor(v, 32, VK_WAVE);
    VK_LDS_BARRIER();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    VK_LDS_BARRIER();
    return (red[0] + red[1]) + (red[2] + red[3]);
}

// LayerNorm statistics of one row by a 256-thread workgroup
// (crates/vokra-backend-cpu/src/kernels/scalar.rs:201-222: mean, population
// variance): thread t sums columns t, t + 256, ... in order, then
// vk_block_sum256. Returns mean and 1 / sqrt(var + eps). The LayerNorm kernel
// and the fused LayerNorm + activation pass both use these, so they agree bit
// for bit. Rows up to kLnRegCols are held in registers (x[j] = column
// t + 256 j), loaded together so their latencies overlap.
constexpr int kLnRegCols = 2048;
constexpr int kLnRegJ = kLnRegCols / 256;
__device__ __forceinline__ void vk_row_load256(const float* __restrict__ row, int cols, float (&x)[kLnRegJ]) {
#pragma unroll
    for (int j = 0; j < kLnRegJ; ++j) {
        const int c = (int)threadIdx.x + 256 * j;
        x[j] = c < cols ? row[c] : 0.0f;
    }
}
// The same columns, every load issued (columns past the row re-read its last
// element and are zeroed by a select): no branch around a load, so a wait
// for one row's loads does not also wait for younger ones.
__device__ __forceinline__ void vk_row_load256_all(const float* __restrict__ row, int cols, float (&x)[kLnRegJ]) {
#pragma unroll
    for (int j = 0; j < kLnRegJ; ++j) {
        const int c = (int)threadIdx.x + 256 * j;
        const float v = row[min(c, cols - 1)];
        x[j] = c < cols ? v : 0.0f;
    }
}
// Sum of x[c] * x[c] over this thread's columns c = t, t + 256, t + 512, ...
// in that order (each a multiply, then an add). The loads are issued eight
// columns at a time, so a row of up to 2048 columns is one memory round trip.
__device__ __forceinline__ float vk_sumsq_cols256(const float* __restrict__ row, int cols) {
    float s = 0.0f;
    for (int c0 = threadIdx.x; c0 < cols; c0 += 256 * 8) {
        float x[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) x[j] = c0 + 256 * j < cols ? row[c0 + 256 * j] : 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j)
            if (c0 + 256 * j < cols) s += x[j] * x[j];
    }
    return s;
}
__device__ __forceinline__ float2 vk_ln_stats256(const float (&x)[kLnRegJ], int cols, float eps, float* red) {
    const float inv_cols = 1.0f / (float)cols;
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < kLnRegJ; ++j)
        if ((int)threadIdx.x + 256 * j < cols) s += x[j];
    const float mean = vk_block_sum256(s, red) * inv_cols;
    float v = 0.0f;
#pragma unroll
    for (int j = 0; j < kLnRegJ; ++j) {
        const float dlt = x[j] - mean;
        if ((int)threadIdx.x + 256 * j < cols) v += dlt * dlt;
    }
    const float inv_std = 1.0f / sqrtf(vk_block_sum256(v, red) * inv_cols + eps);
    return make_float2(mean, inv_std);
}
// Same statistics, same order of operations, streaming any row length.
__device__ __forceinline__ float2 vk_ln_stats256(const float* __restrict__ row, int cols, float eps, float* red) {
    const float inv_cols = 1.0f / (float)cols;
    float s = 0.0f;
    for (int c = threadIdx.x; c < cols; c += 256) s += row[c];
    const float mean = vk_block_sum256(s, red) * inv_cols;
    float v = 0.0f;
    for (int c = threadIdx.x; c < cols; c += 256) {
        const float dlt = row[c] - mean;
        v += dlt * dlt;
    }
    const float inv_std = 1.0f / sqrtf(vk_block_sum256(v, red) * inv_cols + eps);
    return make_float2(mean, inv_std);
}
__device__ __forceinline__ float vk_ln_apply(float x, float2 st, float g, float b) {
    return (x - st.x) * st.y * g + b;
}

// Direct global -> LDS loads (global_load_lds_dwordx4 / _dword). M0 holds the
// wave-uniform LDS base; lane l writes base + l * size. They are issued from
// inline asm so the compiler does not fence every LDS read on them; their
// completion is tracked by hand with vmcnt (loads retire in issue order).
// Nothing else in the kernels that use them reads M0.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
// lds_base must be wave-uniform; it is passed through readfirstlane so that M0
// is always written from a scalar register (free when it already is one).
__device__ __forceinline__ void vk_dma_b128(const void* g, uint32_t lds_base) {
    const uint32_t m0v = __builtin_amdgcn_readfirstlane(lds_base);
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(m0v)
                 : "memory", "m0");
}
__device__ __forceinline__ void vk_dma_b32(const void* g, uint32_t lds_base) {
    const uint32_t m0v = __builtin_amdgcn_readfirstlane(lds_base);
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off" ::"v"(g), "s"(m0v)
                 : "memory", "m0");
}
#pragma clang diagnostic pop

__device__ __forceinline__ uint32_t vk_lds_addr(const void* p) {
    return (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const void*)p;
}

// Wait until at most N of this wave's vector-memory loads (the direct-to-LDS
// loads above included) are in flight.
template <int N>
__device__ __forceinline__ void vk_wait_vm() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}


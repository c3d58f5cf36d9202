// vk_attn.hip — fused scaled-dot-product attention for gfx950.
//
// Semantics (f32): for every batch b, query head h (kv head h / (Hq / Hkv)),
//   S = (q * scale) . k^T, masked to -inf for key j > q_off + i when causal,
//   P = softmax_rows(S), O = P . v
// which is crates/vokra-models/src/whisper/nn.rs:209-325 (q scaled before
// the product, per-head S, causal mask, softmax, P.V) and, with Hkv < Hq,
// the GQA loop of crates/vokra-models/src/voxtral/text_decoder.rs:1302-1360.
//
// Precision: every f32 operand x is split into two fp16 values x = hi + lo
// (hi = fp16(x), lo = fp16(x - hi)) and each product runs as three MFMAs,
// hi*hi + hi*lo + lo*hi, accumulated in f32: about 22 significant bits per
// product, i.e. f32-level results, at 3x the fp16 MFMA rate. q is split as
// q * scale * log2(e), so S comes out in base-2 units and P = 2^(S - max)
// (= e^(s - max) of the natural scores) takes one subtraction and one v_exp
// per score. Inputs must stay within the fp16 range (|x| < 65504 after that
// scaling).
//
// With LO = false (the decoder's half-precision cross-attention mode) K and V
// are taken as their fp16 hi parts only: two MFMAs per product (k_hi*q_hi +
// k_hi*q_lo, v_hi*p_hi + v_hi*p_lo) and half the K/V bytes.
//
// Kernel shape: one workgroup per (64-query tile, head, batch); each of the 4
// waves owns 16 queries. Both products are computed transposed,
//   S^T = K . Q^T  (A = K tile from LDS, B = the wave's Q in registers)
//   O^T = V^T . P^T (A = V^T tile from LDS, B = P from registers)
// so every lane holds the scores, softmax statistics and output of one query
// (lane % 16) and the softmax needs no transposes. K/V tiles of 64 keys are
// staged through LDS, the next tile's loads in flight during the current one;
// the loads are buffer loads whose addresses are a per-lane constant plus a
// wave-uniform tile offset (no vector address arithmetic in the key loop).
// The K tile rows are read into S^T in the order that leaves each lane the
// scores of 8 consecutive keys per 32-key step, which is the P^T operand
// layout of the second product, so a lane's V^T operand is one 16-byte read.
#include <hip/hip_fp16.h>

#include "vk_common.h"
#include "vk_launch.h"

namespace vk {

typedef _Float16 vk_h16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t vk_u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t vk_u32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 vk_h16x2a __attribute__((ext_vector_type(2)));
typedef short vk_i16x2 __attribute__((ext_vector_type(2)));

typedef float vk_f32x2 __attribute__((ext_vector_type(2)));
template <bool B>
struct AttnMask {
    static constexpr bool value = B;
};

namespace attn {
constexpr int QT = 64;   // queries per workgroup
constexpr int KT = 64;   // keys per LDS tile
constexpr int KPAD = 8;  // halves of row padding in the K tile
constexpr int VPAD = 8;  // halves of row padding in the V^T tile
constexpr float kLog2e = 1.44269504088896340736f;
// halves of one K tile (row r at r * (HD + KPAD) + kshift(r), kshift <= 192) and of one V^T tile
constexpr int k_tile_halves(int hd) { return KT * (hd + KPAD) + 192; }
constexpr int v_tile_halves(int hd) { return hd * (KT + VPAD); }
// static LDS bytes of a flash workgroup with np fp16 parts of K / V in use
constexpr int flash_lds_bytes(int hd, int np) { return np * (k_tile_halves(hd) + v_tile_halves(hd)) * 2; }
constexpr int kLdsPerCu = 160 * 1024;
constexpr int kRsrcRaw = 0x00020000;  // buffer resource word 3: raw (unswizzled) dword access
}  // namespace attn

// max / sum over the four lanes of a query (l, l ^ 16, l ^ 32, l ^ 48): each
// permlane swap leaves a lane holding its own value and its partner's, in
// either order (the sum of the two is the same either way)
__device__ __forceinline__ float attn_fmax_raw(float a, float b) {
    float r;  // plain v_max_f32: fmaxf would first quiet signalling NaNs, which scores never are
    asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
    return r;
}
// x - (float)h for h the low (H = 0) or high (H = 1) fp16 of hpair, in one
// v_fma_mix_f32 (x + h * -1, one rounding: the exact difference when h is
// x's own fp16 rounding), instead of a conversion and a subtraction
template <int H>
struct AttnHalf {};
__device__ __forceinline__ float attn_sub_f16(float x, uint32_t hpair, AttnHalf<0>) {
    float r;
    asm("v_fma_mix_f32 %0, %1, -1.0, %2 op_sel_hi:[1,0,0]" : "=v"(r) : "v"(hpair), "v"(x));
    return r;
}
__device__ __forceinline__ float attn_sub_f16(float x, uint32_t hpair, AttnHalf<1>) {
    float r;
    asm("v_fma_mix_f32 %0, %1, -1.0, %2 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(r) : "v"(hpair), "v"(x));
    return r;
}
__device__ __forceinline__ float attn_query_max(float v) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = attn_fmax_raw(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return attn_fmax_raw(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float attn_query_sum(float v) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// Set (to 1) by any kernel of this file that meets an operand outside the
// fp16 range; read and cleared by the host (range_check in vk_capi.hip). One per device.
static __device__ unsigned int vk_attn_range_flag;

__device__ __forceinline__ void attn_range_raise() { atomicOr(&vk_attn_range_flag, 1u); }

__device__ __forceinline__ void split_f16(float x, _Float16& hi, _Float16& lo) {
    hi = (_Float16)x;
    lo = (_Float16)(x - (float)hi);
}

// hi / lo fp16 of x[0..7] * scale packed as two uint4 (vk_split_rows's
// arithmetic for 8 consecutive elements).
__device__ __forceinline__ void split8_f16(const float* __restrict__ x, float scale, uint4& hi, uint4& lo) {
    const float4 u = reinterpret_cast<const float4*>(x)[0], w = reinterpret_cast<const float4*>(x)[1];
    const float a[8] = {u.x * scale, u.y * scale, u.z * scale, u.w * scale,
                        w.x * scale, w.y * scale, w.z * scale, w.w * scale};
    bool bad = false;
#pragma unroll
    for (int j = 0; j < 8; ++j) bad |= vk_f16_overflow(a[j]);
    if (bad) attn_range_raise();
    uint32_t h[4], l[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        _Float16 h0, l0, h1, l1;
        split_f16(a[2 * j], h0, l0);
        split_f16(a[2 * j + 1], h1, l1);
        h[j] = __builtin_bit_cast(uint16_t, h0) | ((uint32_t)__builtin_bit_cast(uint16_t, h1) << 16);
        l[j] = __builtin_bit_cast(uint16_t, l0) | ((uint32_t)__builtin_bit_cast(uint16_t, l1) << 16);
    }
    hi = make_uint4(h[0], h[1], h[2], h[3]);
    lo = make_uint4(l[0], l[1], l[2], l[3]);
}

// Compact low part (single-query attention's K / V): x = hi + lo with hi =
// fp16(x) and lo = q * 2^(e - 32), e = hi's exponent field, q = round((x - hi)
// * 2^(32 - e)) an integer of magnitude <= 64 stored in one byte (x - hi is
// exact and at most half an fp16 ulp, 2^(e - 26)). |x - hi - lo| <= 2^(e - 33),
// relative at most 2^-18 / (1 - 2^-12). Below e = 8 (|x| < 2^-7) lo is zero
// (absolute error at most 2^-19), as the decoder's fp16 scale 2^(e - 22) is
// not normal there.
__device__ __forceinline__ void split_q7(float x, _Float16& hi, int8_t& lo) {
    hi = (_Float16)x;
    const int e = (__builtin_bit_cast(uint16_t, hi) >> 10) & 31;
    lo = (e >= 8 && e < 31) ? (int8_t)(int)rintf(ldexpf(x - (float)hi, 32 - e)) : (int8_t)0;
}
// The fp16 low parts of two elements: hpair holds their fp16 high parts,
// bytes `sel` of qsrc their q. q / 1024 comes exactly from the fp16 bits
// 0x3C00 | (q + 128) (= 1 + (q + 128) / 1024) minus 1.125; times 2^(e - 22)
// (fp16 exponent field e - 7, zero below e = 8) it is q * 2^(e - 32), exact.
__device__ __forceinline__ uint32_t q7pair_f16(uint32_t hpair, uint32_t qsrc, uint32_t sel) {
    const uint32_t t = __builtin_amdgcn_perm(0u, qsrc, sel) ^ 0x3C803C80u;
    const vk_h16x2a q = __builtin_bit_cast(vk_h16x2a, t) + (vk_h16x2a){(_Float16)-1.125f, (_Float16)-1.125f};
    vk_i16x2 e = __builtin_bit_cast(vk_i16x2, hpair & 0x7C007C00u) - (vk_i16x2){0x1C00, 0x1C00};
    e = e > (vk_i16x2){0, 0} ? e : (vk_i16x2){0, 0};
    return __builtin_bit_cast(uint32_t, q * __builtin_bit_cast(vk_h16x2a, e));
}
// the eight fp16 low parts of the elements whose high parts are h (8 fp16)
// and whose q are the bytes of ql (8 int8)
__device__ __forceinline__ vk_u32x4 q7x8_f16(vk_u32x4 h, vk_u32x2 ql) {
    vk_u32x4 r;
    r.x = q7pair_f16(h.x, ql.x, 0x0c010c00u);
    r.y = q7pair_f16(h.y, ql.x, 0x0c030c02u);
    r.z = q7pair_f16(h.z, ql.y, 0x0c010c00u);
    r.w = q7pair_f16(h.w, ql.y, 0x0c030c02u);
    return r;
}

// ---------------------------------------------------------------------------
// Pre-pass: x [rows, cols] f32 -> hi / lo fp16 of x * scale (same layout).
__global__ void vk_split_rows(const float* __restrict__ x, size_t n4, float scale, uint2* __restrict__ hi,
                              uint2* __restrict__ lo) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n4) return;
    const float4 v = reinterpret_cast<const float4*>(x)[i];
    const float a[4] = {v.x * scale, v.y * scale, v.z * scale, v.w * scale};
    if (vk_f16_overflow(a[0]) || vk_f16_overflow(a[1]) || vk_f16_overflow(a[2]) || vk_f16_overflow(a[3]))
        attn_range_raise();
    _Float16 h[4], l[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) split_f16(a[j], h[j], l[j]);
    hi[i] = make_uint2(__builtin_bit_cast(uint16_t, h[0]) | ((uint32_t)__builtin_bit_cast(uint16_t, h[1]) << 16),
                       __builtin_bit_cast(uint16_t, h[2]) | ((uint32_t)__builtin_bit_cast(uint16_t, h[3]) << 16));
    lo[i] = make_uint2(__builtin_bit_cast(uint16_t, l[0]) | ((uint32_t)__builtin_bit_cast(uint16_t, l[1]) << 16),
                       __builtin_bit_cast(uint16_t, l[2]) | ((uint32_t)__builtin_bit_cast(uint16_t, l[3]) << 16));
}

// Pre-pass: v [B][T][H*HD] f32 -> transposed hi / lo [B][H][HD][T_pad] fp16,
// zero for t >= T. One workgroup per (64 x 64 tile of (t, c), head, batch).
__global__ __launch_bounds__(256) void vk_split_vt(const float* __restrict__ v, int t_kv, int t_pad, int h_kv,
                                                   int hd, uint16_t* __restrict__ vth, uint16_t* __restrict__ vtl) {
    __shared__ float tile[64][65];
    const int t0 = blockIdx.x * 64, c0 = (blockIdx.y % (hd / 64)) * 64, h = blockIdx.y / (hd / 64), b = blockIdx.z;
    const int tid = threadIdx.x;
    const size_t width = (size_t)h_kv * hd;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int r = (tid >> 6) + 4 * i, c = tid & 63;
        const int t = t0 + r;
        tile[r][c] = t < t_kv ? v[((size_t)b * t_kv + t) * width + (size_t)h * hd + c0 + c] : 0.0f;
        if (vk_f16_overflow(tile[r][c])) attn_range_raise();
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int c = (tid >> 6) + 4 * i, r = tid & 63;
        _Float16 hi, lo;
        split_f16(tile[r][c], hi, lo);
        const size_t o = (((size_t)b * h_kv + h) * hd + c0 + c) * t_pad + t0 + r;
        vth[o] = __builtin_bit_cast(uint16_t, hi);
        vtl[o] = __builtin_bit_cast(uint16_t, lo);
    }
}

// The same two pre-passes with the compact low part (one byte per element).
__device__ __forceinline__ void split4_q7(float4 v, float scale, uint2& hi, uint32_t& lo) {
    const float a[4] = {v.x * scale, v.y * scale, v.z * scale, v.w * scale};
    if (vk_f16_overflow(a[0]) || vk_f16_overflow(a[1]) || vk_f16_overflow(a[2]) || vk_f16_overflow(a[3]))
        attn_range_raise();
    _Float16 h[4];
    int8_t l[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) split_q7(a[j], h[j], l[j]);
    hi = make_uint2(__builtin_bit_cast(uint16_t, h[0]) | ((uint32_t)__builtin_bit_cast(uint16_t, h[1]) << 16),
                    __builtin_bit_cast(uint16_t, h[2]) | ((uint32_t)__builtin_bit_cast(uint16_t, h[3]) << 16));
    lo = (uint32_t)(uint8_t)l[0] | ((uint32_t)(uint8_t)l[1] << 8) | ((uint32_t)(uint8_t)l[2] << 16) |
         ((uint32_t)(uint8_t)l[3] << 24);
}

__global__ void vk_split_rows_q7(const float* __restrict__ x, size_t n4, float scale, uint2* __restrict__ hi,
                                 uint32_t* __restrict__ lo) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n4) return;
    split4_q7(reinterpret_cast<const float4*>(x)[i], scale, hi[i], lo[i]);
}

// x [B][T][H*hd] -> hi / lo [B][H][T][hd] (each head's keys contiguous); one
// thread per 4 output elements.
__global__ void vk_split_rows_q7_heads(const float* __restrict__ x, size_t n4, int t, int h, int hd4, float scale,
                                       uint2* __restrict__ hi, uint32_t* __restrict__ lo) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n4) return;
    const int d4 = (int)(i % hd4);
    const size_t r = i / hd4;  // (b * h + head) * t + key
    const int key = (int)(r % t);
    const size_t bh = r / t;
    const int head = (int)(bh % h);
    const size_t b = bh / h;
    const size_t src = ((b * t + key) * h + head) * hd4 + d4;
    split4_q7(reinterpret_cast<const float4*>(x)[src], scale, hi[i], lo[i]);
}

// tiled: V^T [B][H][T_pad / 64][hd][64] (each 64-key tile of a head
// contiguous) instead of [B][H][hd][T_pad]
__global__ __launch_bounds__(256) void vk_split_vt_q7(const float* __restrict__ v, int t_kv, int t_pad, int h_kv,
                                                      int hd, int tiled, uint16_t* __restrict__ vth,
                                                      int8_t* __restrict__ vtl) {
    __shared__ float tile[64][65];
    const int t0 = blockIdx.x * 64, c0 = (blockIdx.y % (hd / 64)) * 64, h = blockIdx.y / (hd / 64), b = blockIdx.z;
    const int tid = threadIdx.x;
    const size_t width = (size_t)h_kv * hd;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int r = (tid >> 6) + 4 * i, c = tid & 63;
        const int t = t0 + r;
        tile[r][c] = t < t_kv ? v[((size_t)b * t_kv + t) * width + (size_t)h * hd + c0 + c] : 0.0f;
        if (vk_f16_overflow(tile[r][c])) attn_range_raise();
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int c = (tid >> 6) + 4 * i, r = tid & 63;
        _Float16 hi;
        int8_t lo;
        split_q7(tile[r][c], hi, lo);
        const size_t slab = ((size_t)b * h_kv + h) * hd * t_pad;
        const size_t o = tiled ? slab + (size_t)t0 * hd + (size_t)(c0 + c) * 64 + r
                               : slab + (size_t)(c0 + c) * t_pad + t0 + r;
        vth[o] = __builtin_bit_cast(uint16_t, hi);
        vtl[o] = lo;
    }
}

// ---------------------------------------------------------------------------
// LOM: the K / V low parts in use: 0 none (fp16 high parts only), 1 fp16
// (kl, vtl as fp16 arrays), 2 compact (one byte per element, split_q7).
template <int HD, int LOM, bool ONEQ>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void vk_flash_attn(
    const uint4* __restrict__ qh, const uint4* __restrict__ ql,    // [B][Tq][Hq*HD] fp16, scaled
    const uint4* __restrict__ kh, const uint4* __restrict__ kl,    // [B][Tkv][Hkv*HD] fp16
    const uint4* __restrict__ vth, const uint4* __restrict__ vtl,  // [B][Hkv][HD][Tpad] fp16
    float* __restrict__ out, int tq, int tkv, int t_pad, int hq, int hkv, int causal, int q_off,
    const int* __restrict__ kv_index,
    const float* __restrict__ qf, float q_scale,  // qf != null: f32 q, split here (qh / ql unused)
    const VkQOut qo,                              // qo.afrag != null: quantize O (out may be null)
    const AttnLayout lay) {                       // K / V element strides
    using namespace attn;
    constexpr int KS = HD / 32;      // 32-wide K steps of S = K . Q^T
    constexpr int OS = HD / 16;      // 16-row output subtiles of O^T
    constexpr int KROW = HD + KPAD;  // halves per K tile row
    constexpr int VROW = KT + VPAD;  // halves per V^T tile row
    constexpr int KU4 = KT * HD / 8 / 256;  // uint4 per thread per K array
    constexpr int VU4 = HD * KT / 8 / 256;  // uint4 per thread per V^T array
    constexpr bool LO = LOM != 0;
    constexpr int NP = LO ? 2 : 1;                         // fp16 parts of K and V in use
    // K tile, hi (/ lo): row r at r * KROW + kshift(r) halves (see krow0)
    __shared__ __align__(16) _Float16 lk[NP][k_tile_halves(HD)];
    __shared__ __align__(16) _Float16 lv[NP][v_tile_halves(HD)];  // V^T tile, hi (/ lo)

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, g = lane >> 4, lq = lane & 15;
    const int qt = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
    const int kb = kv_index ? kv_index[b] : b;  // K/V batch of query batch b
    const int hk = h / (hq / hkv);
    const int q_idx = qt * QT + wave * 16 + lq;  // this lane's query
    // ONEQ (t_q = 1, decode): only wave 0 holds a live query; the other waves
    // only help stage the K/V tiles
    const bool active = !ONEQ || wave == 0;
    const int q_ld = min(q_idx, tq - 1);
    const size_t qw = (size_t)hq * HD / 8, kw = (size_t)hkv * HD / 8;  // row widths in uint4

    // this lane's query operand (B of S^T = K . Q^T): hd 32ks + 8g .. +7
    uint4 qa_h[KS], qa_l[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
        const size_t o = ((size_t)b * tq + q_ld) * qw + (size_t)h * HD / 8 + 4 * ks + g;
        if (qf) {
            split8_f16(qf + 8 * o, q_scale, qa_h[ks], qa_l[ks]);
        } else {
            qa_h[ks] = qh[o];
            qa_l[ks] = ql[o];
        }
    }
    // q is complete before the key loop: the loop's waits then only count
    // its own K / V loads
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
        asm volatile("" ::"v"(qa_h[ks].x), "v"(qa_h[ks].y), "v"(qa_h[ks].z), "v"(qa_h[ks].w), "v"(qa_l[ks].x),
                     "v"(qa_l[ks].y), "v"(qa_l[ks].z), "v"(qa_l[ks].w));

    // keys this workgroup has to visit
    int kv_end = tkv;
    if (causal) kv_end = min(tkv, q_off + min(qt * QT + QT, tq));
    const int n_tiles = (kv_end + KT - 1) / KT;

    // Staged loads of one K / V^T tile. K: the tile's rows start a buffer
    // resource whose extent ends with row t_kv - 1 of this (batch, kv head)
    // (a row past it reads as zero; such keys are masked); V^T: one resource
    // over this (batch, kv head)'s HD x Tpad slab, the tile a scalar offset
    // into it.
    // Per-lane byte offsets are loop constants. Native vectors (not HIP's
    // uint4 struct) keep the stage in registers.
    struct Stage {
        vk_u32x4 kh[KU4], kl[KU4], vh[VU4], vl[VU4];
        vk_u32x2 klq[KU4], vlq[VU4];  // LOM == 2
    };
    constexpr int KEB = LOM == 2 ? 1 : 2;  // bytes per element of the K / V low parts
    const size_t kslab = (size_t)kb * lay.kb + (size_t)hk * lay.kh;  // elements: key 0 of this (batch, kv head)
    const char* kslab_h = reinterpret_cast<const char*>(kh) + kslab * 2;
    const char* kslab_l = reinterpret_cast<const char*>(kl) + kslab * KEB;
    const size_t vslab = ((size_t)kb * hkv + hk) * HD * t_pad;  // elements
    const __amdgpu_buffer_rsrc_t rvh = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(reinterpret_cast<const char*>(vth) + vslab * 2), 0, HD * t_pad * 2, kRsrcRaw);
    const __amdgpu_buffer_rsrc_t rvl = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(reinterpret_cast<const char*>(vtl) + vslab * KEB), 0, HD * t_pad * KEB, kRsrcRaw);
    uint32_t ko[KU4], vo[VU4];  // element offsets of this thread's K / V^T chunks within a tile
#pragma unroll
    for (int i = 0; i < KU4; ++i) {
        const int idx = tid + 256 * i, r = idx / (HD / 8), c = idx % (HD / 8);
        ko[i] = (uint32_t)(r * lay.kt + 8 * c);
    }
#pragma unroll
    for (int i = 0; i < VU4; ++i) {
        const int idx = tid + 256 * i, r = idx / (KT / 8), c = idx % (KT / 8);
        vo[i] = (uint32_t)(r * lay.vd + 8 * c);
    }
    auto load = [&](int kt) __attribute__((always_inline)) -> Stage {
        Stage st;
        const int rows = min(tkv - kt * KT, KT);  // >= 1: kt < n_tiles
        const size_t k0 = (size_t)kt * KT * lay.kt;  // elements
        const int kext = (rows - 1) * lay.kt + HD;   // elements up to the end of row t_kv - 1
        const __amdgpu_buffer_rsrc_t rkh =
            __builtin_amdgcn_make_buffer_rsrc((void*)(kslab_h + k0 * 2), 0, kext * 2, kRsrcRaw);
        const __amdgpu_buffer_rsrc_t rkl =
            __builtin_amdgcn_make_buffer_rsrc((void*)(kslab_l + k0 * KEB), 0, kext * KEB, kRsrcRaw);
#pragma unroll
        for (int i = 0; i < KU4; ++i) {
            st.kh[i] = __builtin_amdgcn_raw_buffer_load_b128(rkh, ko[i] * 2, 0, 0);
            if (LOM == 1) st.kl[i] = __builtin_amdgcn_raw_buffer_load_b128(rkl, ko[i] * 2, 0, 0);
            if (LOM == 2) st.klq[i] = __builtin_amdgcn_raw_buffer_load_b64(rkl, ko[i], 0, 0);
        }
#pragma unroll
        for (int i = 0; i < VU4; ++i) {
            st.vh[i] = __builtin_amdgcn_raw_buffer_load_b128(rvh, vo[i] * 2, kt * lay.vtile * 2, 0);
            if (LOM == 1) st.vl[i] = __builtin_amdgcn_raw_buffer_load_b128(rvl, vo[i] * 2, kt * lay.vtile * 2, 0);
            if (LOM == 2) st.vlq[i] = __builtin_amdgcn_raw_buffer_load_b64(rvl, vo[i], kt * lay.vtile, 0);
        }
        return st;
    };

    // O = O^T * inv: lane holds query lq, hd 16os + 4g + r. The four lanes of
    // a query (l, l^16, l^32, l^48) hold its row; with qo, they quantize each
    // 32-wide block of it (os 2bq and 2bq+1) as the activation pass would.
    auto finish = [&](const vk_f32x4* o_acc, float inv) {
        float ov[OS][4];
#pragma unroll
        for (int os = 0; os < OS; ++os)
#pragma unroll
            for (int r = 0; r < 4; ++r) ov[os][r] = o_acc[os][r] * inv;
        const size_t row = (size_t)b * tq + q_idx;
        if (out && q_idx < tq) {
            float* orow = out + row * (size_t)hq * HD + (size_t)h * HD;
#pragma unroll
            for (int os = 0; os < OS; ++os)
                *reinterpret_cast<float4*>(orow + 16 * os + 4 * g) =
                    make_float4(ov[os][0], ov[os][1], ov[os][2], ov[os][3]);
        }
        if (!qo.afrag) return;
        const int nb = qo.k >> 5;
#pragma unroll
        for (int bq = 0; bq < HD / 32; ++bq) {
            float amax = 0.0f;
#pragma unroll
            for (int hf = 0; hf < 2; ++hf)
#pragma unroll
                for (int r = 0; r < 4; ++r) amax = fmaxf(amax, fabsf(ov[2 * bq + hf][r]));
            amax = fmaxf(amax, __shfl_xor(amax, 16, VK_WAVE));
            amax = fmaxf(amax, __shfl_xor(amax, 32, VK_WAVE));
            float sc = 0.0f;
            int qv[2][4] = {{0, 0, 0, 0}, {0, 0, 0, 0}};
            if (amax != 0.0f) {
                sc = vk_act_scale(amax, qo.pow2);
#pragma unroll
                for (int hf = 0; hf < 2; ++hf)
#pragma unroll
                    for (int r = 0; r < 4; ++r) qv[hf][r] = vk_act_q(ov[2 * bq + hf][r], sc);
            }
            int gs = 0;
#pragma unroll
            for (int hf = 0; hf < 2; ++hf)
#pragma unroll
                for (int r = 0; r < 4; ++r) gs += qv[hf][r];
            gs += __shfl_xor(gs, 16, VK_WAVE);
            gs += __shfl_xor(gs, 32, VK_WAVE);
            if (q_idx < tq) {
                const int kb = h * (HD / 32) + bq;
                uint16_t* f16 = reinterpret_cast<uint16_t*>(qo.afrag);
#pragma unroll
                for (int hf = 0; hf < 2; ++hf) {
                    // elements 16 hf + 4g .. +3: four consecutive uint16 of one lane's uint4
                    const size_t at = vk_afrag_u16(row, kb, nb, 16 * hf + 4 * g);
                    uint32_t w0 = vk_act_bits(qv[hf][0], sc, qo.pow2) | (vk_act_bits(qv[hf][1], sc, qo.pow2) << 16);
                    uint32_t w1 = vk_act_bits(qv[hf][2], sc, qo.pow2) | (vk_act_bits(qv[hf][3], sc, qo.pow2) << 16);
                    *reinterpret_cast<uint2*>(f16 + at) = make_uint2(w0, w1);
                }
                if (g == 0) {
                    qo.ascale[(size_t)kb * qo.m_pad + row] = sc;
                    qo.asum[(size_t)kb * qo.m_pad + row] = qo.pow2 ? (float)gs * sc : (float)gs;
                }
            }
        }
    };

    vk_f32x4 o_acc[OS];
#pragma unroll
    for (int s = 0; s < OS; ++s) o_acc[s] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (n_tiles == 0) {  // no keys: P . V over an empty set is zero
        finish(o_acc, 0.0f);
        return;
    }
    float m_run = -INFINITY, l_run = 0.0f;
    // S^T subtile n takes K tile row 32 (n / 2) + 4 (n % 2) + 8 (i / 4) + i % 4
    // as its row i: a lane (g = lane / 16) then holds, for subtile n and
    // accumulator entry r, key 32 (n / 2) + 8 g + 4 (n % 2) + r. The rows a
    // 16-lane read phase takes (i = 0..15) are 4 runs of 4 rows 8 apart; row r
    // starts kshift(r) = 4 (r & 24) + 3 (r & 32) halves past r * KROW, which
    // puts those 16 reads of 16 bytes on 64 distinct banks (and each 8-lane
    // half on 32) where the plain row pitch would pair them up; the 3 (r & 32)
    // term keeps rows 32.. clear of row 31's shifted span. For the rows read
    // here r & 24 = 8 (lq / 4) and r & 32 = 32 (n / 2).
    const int krow0 = 8 * (lq >> 2) + (lq & 3);
    const int kbase = krow0 * KROW + 32 * (lq >> 2) + 8 * g;

    // One tile's two products and softmax step for the active waves; MASK:
    // the tile holds keys past t_kv or (causal) past some query's position.
    // The two instantiations keep the whole-tile case free of the masking.
    auto tile = [&](int kt, auto mask_tag) __attribute__((always_inline)) {
        constexpr bool MASK = decltype(mask_tag)::value;
        // ---- S^T for 4 key subtiles of 16 (base-2 units)
        vk_f32x4 s[4];
#pragma unroll
        for (int n = 0; n < 4; ++n) {
            s[n] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                const int off = kbase + (32 * (n >> 1) + 4 * (n & 1)) * KROW + 96 * (n >> 1) + 32 * ks;
                const vk_h16x8 ah = *reinterpret_cast<const vk_h16x8*>(&lk[0][off]);
                const vk_h16x8 bh = __builtin_bit_cast(vk_h16x8, qa_h[ks]);
                const vk_h16x8 bl = __builtin_bit_cast(vk_h16x8, qa_l[ks]);
                s[n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bh, s[n], 0, 0, 0);
                s[n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bl, s[n], 0, 0, 0);
                if (LO) {
                    const vk_h16x8 al = *reinterpret_cast<const vk_h16x8*>(&lk[NP - 1][off]);
                    s[n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bh, s[n], 0, 0, 0);
                }
            }
        }
        // ---- mask, online softmax (per query = per lane, across lanes g)
        float mloc = -INFINITY;
#pragma unroll
        for (int n = 0; n < 4; ++n)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                if (MASK) {
                    const int key = kt * KT + 32 * (n >> 1) + 8 * g + 4 * (n & 1) + r;
                    const bool ok = key < tkv && (!causal || key <= q_off + q_idx);
                    s[n][r] = ok ? s[n][r] : -INFINITY;
                }
                mloc = fmaxf(mloc, s[n][r]);
            }
        mloc = attn_query_max(mloc);
        const float m_new = fmaxf(m_run, mloc);
        const float m_use = m_new == -INFINITY ? 0.0f : m_new;
        const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);
        float psum = 0.0f;
        // P^T operand halves: for 32-key step ks, the lane's keys 32ks + 8g + 4j + r
        // (subtile n = 2ks + j) are MFMA k-slots 8g + 4j + r
        vk_u32x4 ph[2], pl[2];
#pragma unroll
        for (int n = 0; n < 4; ++n) {
#pragma unroll
            for (int r = 0; r < 4; r += 2) {
                const vk_f32x2 p = {__builtin_amdgcn_exp2f(s[n][r] - m_use),
                                    __builtin_amdgcn_exp2f(s[n][r + 1] - m_use)};
                psum += p.x;
                psum += p.y;
                const vk_h16x2a hi = __builtin_convertvector(p, vk_h16x2a);
                const uint32_t hb = __builtin_bit_cast(uint32_t, hi);
                const vk_f32x2 d = {attn_sub_f16(p.x, hb, AttnHalf<0>{}), attn_sub_f16(p.y, hb, AttnHalf<1>{})};
                const vk_h16x2a lo = __builtin_convertvector(d, vk_h16x2a);
                ph[n >> 1][2 * (n & 1) + r / 2] = __builtin_bit_cast(uint32_t, hi);
                pl[n >> 1][2 * (n & 1) + r / 2] = __builtin_bit_cast(uint32_t, lo);
            }
        }
        psum = attn_query_sum(psum);
        l_run = l_run * alpha + psum;
        m_run = m_new;
        // o * 1.0f is o: when no lane's running max moved, the rescale is skipped
        if (__any(alpha != 1.0f)) {
#pragma unroll
            for (int os = 0; os < OS; ++os)
#pragma unroll
                for (int r = 0; r < 4; ++r) o_acc[os][r] *= alpha;
        }
        // ---- O^T += V^T . P^T over 2 key steps of 32
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            const vk_h16x8 bh = __builtin_bit_cast(vk_h16x8, ph[ks]);
            const vk_h16x8 bl = __builtin_bit_cast(vk_h16x8, pl[ks]);
#pragma unroll
            for (int os = 0; os < OS; ++os) {
                const int off = (16 * os + lq) * VROW + 32 * ks + 8 * g;
                const vk_h16x8 ah = *reinterpret_cast<const vk_h16x8*>(&lv[0][off]);
                o_acc[os] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bh, o_acc[os], 0, 0, 0);
                o_acc[os] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bl, o_acc[os], 0, 0, 0);
                if (LO) {
                    const vk_h16x8 al = *reinterpret_cast<const vk_h16x8*>(&lv[NP - 1][off]);
                    o_acc[os] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bh, o_acc[os], 0, 0, 0);
                }
            }
        }
    };

    // Stage a tile's loads (sx) into LDS.
    auto stage_in = [&](const Stage& sx) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < KU4; ++i) {
            const int idx = tid + 256 * i;
            const int r = idx / (HD / 8), c = idx % (HD / 8);
            const int at = r * KROW + 4 * (r & 24) + 3 * (r & 32) + 8 * c;
            *reinterpret_cast<vk_u32x4*>(&lk[0][at]) = sx.kh[i];
            if (LOM == 1) *reinterpret_cast<vk_u32x4*>(&lk[NP - 1][at]) = sx.kl[i];
            if (LOM == 2) *reinterpret_cast<vk_u32x4*>(&lk[NP - 1][at]) = q7x8_f16(sx.kh[i], sx.klq[i]);
        }
#pragma unroll
        for (int i = 0; i < VU4; ++i) {
            const int idx = tid + 256 * i;
            const int r = idx / (KT / 8), c = idx % (KT / 8);
            *reinterpret_cast<vk_u32x4*>(&lv[0][r * VROW + 8 * c]) = sx.vh[i];
            if (LOM == 1) *reinterpret_cast<vk_u32x4*>(&lv[NP - 1][r * VROW + 8 * c]) = sx.vl[i];
            if (LOM == 2) *reinterpret_cast<vk_u32x4*>(&lv[NP - 1][r * VROW + 8 * c]) = q7x8_f16(sx.vh[i], sx.vlq[i]);
        }
        VK_LDS_BARRIER();
    };
    // One tile per step: stage it, start the next tile's loads, run the
    // products. Tiles that need no masking (all keys below t_kv and,
    // causal, at or before the workgroup's first query) are a prefix of
    // the sequence: they run in a loop of their own, so the masked case
    // costs nothing there.
    Stage st = load(0);  // unconditional (clamped) loads keep the stage in registers
    auto step = [&](int kt, auto mask_tag) __attribute__((always_inline)) {
        stage_in(st);
        st = load(min(kt + 1, n_tiles - 1));
        if (active) tile(kt, mask_tag);
        VK_LDS_BARRIER();
    };
    int n_full = min(n_tiles, tkv / KT);
    if (causal) n_full = min(n_full, (q_off + qt * QT + 1) / KT);
    int kt = 0;
    for (; kt < n_full; ++kt) step(kt, AttnMask<false>{});
    for (; kt < n_tiles; ++kt) step(kt, AttnMask<true>{});
    if (active) finish(o_acc, l_run > 0.0f ? 1.0f / l_run : 0.0f);
}

}  // namespace vk

#include "vk_launch.h"

namespace vk {

float attn_q_scale(float scale) { return scale * attn::kLog2e; }

hipError_t launch_split_rows(hipStream_t s, const float* x, size_t n, float scale, void* hi, void* lo) {
    const size_t n4 = n / 4;
    if (n4 == 0) return hipSuccess;
    hipLaunchKernelGGL(vk_split_rows, dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, s, x, n4, scale, (uint2*)hi,
                       (uint2*)lo);
    return hipGetLastError();
}

hipError_t launch_split_rows_q7(hipStream_t s, const float* x, size_t n, float scale, void* hi, void* lo) {
    const size_t n4 = n / 4;
    if (n4 == 0) return hipSuccess;
    hipLaunchKernelGGL(vk_split_rows_q7, dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, s, x, n4, scale, (uint2*)hi,
                       (uint32_t*)lo);
    return hipGetLastError();
}

hipError_t launch_split_vt_q7(hipStream_t s, const float* v, int batch, int t_kv, int t_pad, int h_kv, int hd,
                              void* vth, void* vtl, bool tiled) {
    if (batch == 0 || t_pad == 0) return hipSuccess;
    hipLaunchKernelGGL(vk_split_vt_q7, dim3(t_pad / 64, h_kv * (hd / 64), batch), dim3(256), 0, s, v, t_kv, t_pad,
                       h_kv, hd, tiled ? 1 : 0, (uint16_t*)vth, (int8_t*)vtl);
    return hipGetLastError();
}

hipError_t launch_split_rows_q7_heads(hipStream_t s, const float* x, int batch, int t, int h, int hd, float scale,
                                      void* hi, void* lo) {
    const size_t n4 = (size_t)batch * t * h * hd / 4;
    if (n4 == 0) return hipSuccess;
    hipLaunchKernelGGL(vk_split_rows_q7_heads, dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, s, x, n4, t, h,
                       hd / 4, scale, (uint2*)hi, (uint32_t*)lo);
    return hipGetLastError();
}

hipError_t launch_split_vt(hipStream_t s, const float* v, int batch, int t_kv, int t_pad, int h_kv, int hd, void* vth,
                           void* vtl) {
    if (batch == 0 || t_pad == 0) return hipSuccess;
    hipLaunchKernelGGL(vk_split_vt, dim3(t_pad / 64, h_kv * (hd / 64), batch), dim3(256), 0, s, v, t_kv, t_pad, h_kv,
                       hd, (uint16_t*)vth, (uint16_t*)vtl);
    return hipGetLastError();
}

AttnLayout attn_layout_rows(int t_kv, int h_kv, int hd, int t_pad) {
    AttnLayout l;
    l.kt = h_kv * hd;
    l.kh = hd;
    l.kb = (long long)t_kv * h_kv * hd;
    l.vd = t_pad;
    l.vtile = attn::KT;
    return l;
}

AttnLayout attn_layout_heads(int t_kv, int h_kv, int hd, int t_pad) {
    AttnLayout l;
    l.kt = hd;
    l.kh = (long long)t_kv * hd;
    l.kb = (long long)t_kv * h_kv * hd;
    l.vd = attn::KT;
    l.vtile = attn::KT * hd;
    (void)t_pad;
    return l;
}

namespace {
// One flash launch's operands (the kernel's arguments).
struct FlashArgs {
    const void *qh, *ql, *kh, *kl, *vth, *vtl;
    float* out;
    int tq, tkv, t_pad, hq, hkv, causal, q_off;
    const int* kv_index;
    const float* qf;
    float q_scale;
    VkQOut qo;
    AttnLayout lay;
};

// Dynamic LDS that sets a single-query launch's residency. Those launches
// stream K / V from HBM and finish in rounds of (CUs x workgroups per CU); a
// last round that holds few workgroups per CU leaves HBM underused while it
// runs. When the grid needs more than one round at the kernel's full
// residency r, one fewer per CU is taken if that fills the last round better
// (decoder step, 64 streams x 20 heads = 1280 workgroups, compact K / V: r = 4
// gives rounds of 1024 + 256, 3 gives 768 + 512; 7.95 -> 7.43 ms per step;
// 2 per CU measured 8.17 ms). The padded total sits midway between the two
// residencies: a total just under a third of the LDS (54272 bytes) ran like
// 2 per CU.
int oneq_lds_pad(int r_full, int lds_static, size_t n_wg) {
    static const int cus = [] {  // CUs per device (the same on every gfx950 device)
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
            return 0;
        return n;
    }();
    if (cus <= 0) return 0;
    if (r_full <= 1 || n_wg <= (size_t)cus * r_full) return 0;
    auto fill = [&](int r) {  // share of the last round's slots in use
        const size_t per = (size_t)cus * r, last = n_wg % per;
        return last == 0 ? 1.0 : (double)last / (double)per;
    };
    if (fill(r_full - 1) <= fill(r_full)) return 0;
    // a workgroup's LDS total midway between what fits r_full - 1 and r_full
    // times, clear of the allocation granularity either way
    const int total = ((attn::kLdsPerCu / r_full + attn::kLdsPerCu / (r_full - 1)) / 2) & ~1023;
    return total > attn::kLdsPerCu / r_full && total > lds_static ? total - lds_static : 0;
}

template <int HD, int LOM, bool ONEQ>
void go_flash(hipStream_t s, dim3 grid, const FlashArgs& a) {
    int pad = 0;
    if (ONEQ) {
        static const int r_full = [] {  // workgroups per CU without padding (same for every gfx950 device)
            int r = 0;
            if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
                    &r, reinterpret_cast<const void*>(&vk_flash_attn<HD, LOM, ONEQ>), 256, 0) != hipSuccess)
                return 0;
            return r;
        }();
        pad = oneq_lds_pad(r_full, attn::flash_lds_bytes(HD, LOM != 0 ? 2 : 1),
                           (size_t)grid.x * grid.y * grid.z);
    }
    hipLaunchKernelGGL((vk_flash_attn<HD, LOM, ONEQ>), grid, dim3(256), pad, s, (const uint4*)a.qh,
                       (const uint4*)a.ql, (const uint4*)a.kh, (const uint4*)a.kl, (const uint4*)a.vth,
                       (const uint4*)a.vtl, a.out, a.tq, a.tkv, a.t_pad, a.hq, a.hkv, a.causal, a.q_off, a.kv_index,
                       a.qf, a.q_scale, a.qo, a.lay);
}

template <int HD>
void go_flash_hd(hipStream_t s, dim3 grid, int lo_mode, const FlashArgs& a) {
    const bool one = a.tq == 1;
    if (lo_mode == KV_LO_Q7)  // the compact form exists for single-query launches only
        go_flash<HD, 2, true>(s, grid, a);
    else if (lo_mode == KV_LO_F16)
        one ? go_flash<HD, 1, true>(s, grid, a) : go_flash<HD, 1, false>(s, grid, a);
    else
        one ? go_flash<HD, 0, true>(s, grid, a) : go_flash<HD, 0, false>(s, grid, a);
}

hipError_t flash_any(hipStream_t s, int hd, int batch, int lo_mode, const FlashArgs& a) {
    if (lo_mode == KV_LO_Q7 && a.tq != 1) return hipErrorInvalidValue;
    // buffer-resource extents (one kv head's V^T slab, 64 K rows) and the
    // per-lane 32-bit K offsets, in bytes
    if ((size_t)hd * a.t_pad * 2 > 0x7fffffffu || (size_t)attn::KT * a.lay.kt * 2 > 0x7fffffffu)
        return hipErrorInvalidValue;
    const dim3 grid((a.tq + attn::QT - 1) / attn::QT, a.hq, batch);
    if (hd == 64)
        go_flash_hd<64>(s, grid, lo_mode, a);
    else
        go_flash_hd<128>(s, grid, lo_mode, a);
    return hipGetLastError();
}
}  // namespace

hipError_t launch_flash_attn(hipStream_t s, int hd, const void* qh, const void* ql, const void* kh, const void* kl,
                             const void* vth, const void* vtl, float* out, int batch, int tq, int tkv, int t_pad,
                             int hq, int hkv, int causal, int q_off, const int* kv_index, int lo_mode) {
    const FlashArgs a = {qh,     ql,      kh,       kl,       vth,     vtl,  out,       tq,
                         tkv,    t_pad,   hq,       hkv,      causal,  q_off, kv_index, nullptr,
                         1.0f,   VkQOut{}, attn_layout_rows(tkv, hkv, hd, t_pad)};
    return flash_any(s, hd, batch, lo_mode, a);
}

hipError_t launch_flash_attn_f32q(hipStream_t s, int hd, const float* q, float q_scale, const void* kh, const void* kl,
                                  const void* vth, const void* vtl, float* out, int batch, int tq, int tkv, int t_pad,
                                  int hq, int hkv, int causal, int q_off, const int* kv_index, int lo_mode,
                                  const VkQOut* qo, const AttnLayout* lay) {
    const FlashArgs a = {nullptr, nullptr, kh,     kl,    vth,      vtl,
                         out,     tq,      tkv,    t_pad, hq,       hkv,
                         causal,  q_off,   kv_index, q,   attn_q_scale(q_scale), qo ? *qo : VkQOut{},
                         lay ? *lay : attn_layout_rows(tkv, hkv, hd, t_pad)};
    return flash_any(s, hd, batch, lo_mode, a);
}

// This device's address of this file's fp16-range flag (the host reads and
// clears it with one small kernel per check).
hipError_t attn_range_flag_addr(unsigned** p) { return hipGetSymbolAddress((void**)p, HIP_SYMBOL(vk_attn_range_flag)); }

}  // namespace vk

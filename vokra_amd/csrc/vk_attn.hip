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
// product, i.e. f32-level results, at 3x the fp16 MFMA rate. Inputs must stay
// within the fp16 range (|x| < 65504 after scaling).
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
// staged through LDS, the next tile's loads in flight during the current one.
#include <hip/hip_fp16.h>

#include "vk_common.h"
#include "vk_launch.h"

namespace vk {

typedef _Float16 vk_h16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t vk_u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t vk_u32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 vk_h16x2a __attribute__((ext_vector_type(2)));
typedef short vk_i16x2 __attribute__((ext_vector_type(2)));

namespace attn {
constexpr int QT = 64;   // queries per workgroup
constexpr int KT = 64;   // keys per LDS tile
constexpr int KPAD = 8;  // halves of row padding in the K tile
constexpr int VPAD = 8;  // halves of row padding in the V^T tile
}  // namespace attn

// Set (to 1) by any kernel of this file that meets an operand outside the
// fp16 range; read and cleared by the host (attn_range_take). One per device.
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
__global__ void vk_split_rows_q7(const float* __restrict__ x, size_t n4, float scale, uint2* __restrict__ hi,
                                 uint32_t* __restrict__ lo) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n4) return;
    const float4 v = reinterpret_cast<const float4*>(x)[i];
    const float a[4] = {v.x * scale, v.y * scale, v.z * scale, v.w * scale};
    if (vk_f16_overflow(a[0]) || vk_f16_overflow(a[1]) || vk_f16_overflow(a[2]) || vk_f16_overflow(a[3]))
        attn_range_raise();
    _Float16 h[4];
    int8_t l[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) split_q7(a[j], h[j], l[j]);
    hi[i] = make_uint2(__builtin_bit_cast(uint16_t, h[0]) | ((uint32_t)__builtin_bit_cast(uint16_t, h[1]) << 16),
                       __builtin_bit_cast(uint16_t, h[2]) | ((uint32_t)__builtin_bit_cast(uint16_t, h[3]) << 16));
    lo[i] = (uint32_t)(uint8_t)l[0] | ((uint32_t)(uint8_t)l[1] << 8) | ((uint32_t)(uint8_t)l[2] << 16) |
            ((uint32_t)(uint8_t)l[3] << 24);
}

__global__ __launch_bounds__(256) void vk_split_vt_q7(const float* __restrict__ v, int t_kv, int t_pad, int h_kv,
                                                      int hd, uint16_t* __restrict__ vth, int8_t* __restrict__ vtl) {
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
        const size_t o = (((size_t)b * h_kv + h) * hd + c0 + c) * t_pad + t0 + r;
        vth[o] = __builtin_bit_cast(uint16_t, hi);
        vtl[o] = lo;
    }
}

// ---------------------------------------------------------------------------
// LOM: the K / V low parts in use: 0 none (fp16 high parts only), 1 fp16
// (kl, vtl as fp16 arrays), 2 compact (one byte per element, split_q7).
template <int HD, int LOM, bool ONEQ>
__global__ __launch_bounds__(256) void vk_flash_attn(
    const uint4* __restrict__ qh, const uint4* __restrict__ ql,    // [B][Tq][Hq*HD] fp16, scaled
    const uint4* __restrict__ kh, const uint4* __restrict__ kl,    // [B][Tkv][Hkv*HD] fp16
    const uint4* __restrict__ vth, const uint4* __restrict__ vtl,  // [B][Hkv][HD][Tpad] fp16
    float* __restrict__ out, int tq, int tkv, int t_pad, int hq, int hkv, int causal, int q_off,
    const int* __restrict__ kv_index,
    const float* __restrict__ qf, float q_scale,  // qf != null: f32 q, split here (qh / ql unused)
    const VkQOut qo) {                            // qo.afrag != null: quantize O (out may be null)
    using namespace attn;
    constexpr int KS = HD / 32;      // 32-wide K steps of S = K . Q^T
    constexpr int OS = HD / 16;      // 16-row output subtiles of O^T
    constexpr int KROW = HD + KPAD;  // halves per K tile row
    constexpr int VROW = KT + VPAD;  // halves per V^T tile row
    constexpr int KU4 = KT * HD / 8 / 256;  // uint4 per thread per K array
    constexpr int VU4 = HD * KT / 8 / 256;  // uint4 per thread per V^T array
    constexpr bool LO = LOM != 0;
    constexpr int NP = LO ? 2 : 1;                         // fp16 parts of K and V in use
    __shared__ __align__(16) _Float16 lk[NP][KT * KROW];  // K tile, hi (/ lo)
    __shared__ __align__(16) _Float16 lv[NP][HD * VROW];  // V^T tile, hi (/ lo)

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

    // keys this workgroup has to visit
    int kv_end = tkv;
    if (causal) kv_end = min(tkv, q_off + min(qt * QT + QT, tq));
    const int n_tiles = (kv_end + KT - 1) / KT;

    // staged loads of one K / V^T tile (indices clamped into the arrays)
    // native vectors (not HIP's uint4 struct) so the stage stays in registers
    struct Stage {
        vk_u32x4 kh[KU4], kl[KU4], vh[VU4], vl[VU4];
        vk_u32x2 klq[KU4], vlq[VU4];  // LOM == 2
    };
    const vk_u32x4* kh4 = reinterpret_cast<const vk_u32x4*>(kh);
    const vk_u32x4* kl4 = reinterpret_cast<const vk_u32x4*>(kl);
    const vk_u32x4* vh4 = reinterpret_cast<const vk_u32x4*>(vth);
    const vk_u32x4* vl4 = reinterpret_cast<const vk_u32x4*>(vtl);
    const vk_u32x2* klq2 = reinterpret_cast<const vk_u32x2*>(kl);
    const vk_u32x2* vlq2 = reinterpret_cast<const vk_u32x2*>(vtl);
    auto load = [&](int kt) __attribute__((always_inline)) -> Stage {
        Stage st;
#pragma unroll
        for (int i = 0; i < KU4; ++i) {
            const int idx = tid + 256 * i;
            const int r = idx / (HD / 8), c = idx % (HD / 8);
            const int t = min(kt * KT + r, tkv - 1);
            const size_t o = ((size_t)kb * tkv + t) * kw + (size_t)hk * HD / 8 + c;
            st.kh[i] = kh4[o];
            if (LOM == 1) st.kl[i] = kl4[o];
            if (LOM == 2) st.klq[i] = klq2[o];
        }
#pragma unroll
        for (int i = 0; i < VU4; ++i) {
            const int idx = tid + 256 * i;
            const int r = idx / (KT / 8), c = idx % (KT / 8);
            const size_t o = (((size_t)kb * hkv + hk) * HD + r) * (t_pad / 8) + (size_t)kt * KT / 8 + c;
            st.vh[i] = vh4[o];
            if (LOM == 1) st.vl[i] = vl4[o];
            if (LOM == 2) st.vlq[i] = vlq2[o];
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

    // unconditional (clamped) loads keep the stage in registers
    Stage st = load(0);
    for (int kt = 0; kt < n_tiles; ++kt) {
        // ---- stage the tile into LDS
#pragma unroll
        for (int i = 0; i < KU4; ++i) {
            const int idx = tid + 256 * i;
            const int r = idx / (HD / 8), c = idx % (HD / 8);
            *reinterpret_cast<vk_u32x4*>(&lk[0][r * KROW + 8 * c]) = st.kh[i];
            if (LOM == 1) *reinterpret_cast<vk_u32x4*>(&lk[NP - 1][r * KROW + 8 * c]) = st.kl[i];
            if (LOM == 2) *reinterpret_cast<vk_u32x4*>(&lk[NP - 1][r * KROW + 8 * c]) = q7x8_f16(st.kh[i], st.klq[i]);
        }
#pragma unroll
        for (int i = 0; i < VU4; ++i) {
            const int idx = tid + 256 * i;
            const int r = idx / (KT / 8), c = idx % (KT / 8);
            *reinterpret_cast<vk_u32x4*>(&lv[0][r * VROW + 8 * c]) = st.vh[i];
            if (LOM == 1) *reinterpret_cast<vk_u32x4*>(&lv[NP - 1][r * VROW + 8 * c]) = st.vl[i];
            if (LOM == 2) *reinterpret_cast<vk_u32x4*>(&lv[NP - 1][r * VROW + 8 * c]) = q7x8_f16(st.vh[i], st.vlq[i]);
        }
        VK_LDS_BARRIER();
        st = load(min(kt + 1, n_tiles - 1));

        if (active) {
            // ---- S^T for 4 key subtiles of 16: lane holds keys 16n + 4g + r
            vk_f32x4 s[4];
#pragma unroll
            for (int n = 0; n < 4; ++n) {
                s[n] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int ks = 0; ks < KS; ++ks) {
                    const int off = (16 * n + lq) * KROW + 32 * ks + 8 * g;
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
            if (!causal && kt * KT + KT <= tkv) {  // a whole tile of live keys: nothing to mask
#pragma unroll
                for (int n = 0; n < 4; ++n)
#pragma unroll
                    for (int r = 0; r < 4; ++r) mloc = fmaxf(mloc, s[n][r]);
            } else {
#pragma unroll
                for (int n = 0; n < 4; ++n)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int key = kt * KT + 16 * n + 4 * g + r;
                        const bool ok = key < tkv && (!causal || key <= q_off + q_idx);
                        s[n][r] = ok ? s[n][r] : -INFINITY;
                        mloc = fmaxf(mloc, s[n][r]);
                    }
            }
            mloc = fmaxf(mloc, __shfl_xor(mloc, 16, VK_WAVE));
            mloc = fmaxf(mloc, __shfl_xor(mloc, 32, VK_WAVE));
            const float m_new = fmaxf(m_run, mloc);
            const float m_use = m_new == -INFINITY ? 0.0f : m_new;
            const float alpha = __expf(m_run - m_use);
            float psum = 0.0f;
            uint32_t ph[4][2], pl[4][2];  // P^T operand halves, [key subtile][pair]
#pragma unroll
            for (int n = 0; n < 4; ++n) {
                _Float16 h4[4], l4[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float p = __expf(s[n][r] - m_use);
                    psum += p;
                    split_f16(p, h4[r], l4[r]);
                }
                ph[n][0] = __builtin_bit_cast(uint16_t, h4[0]) | ((uint32_t)__builtin_bit_cast(uint16_t, h4[1]) << 16);
                ph[n][1] = __builtin_bit_cast(uint16_t, h4[2]) | ((uint32_t)__builtin_bit_cast(uint16_t, h4[3]) << 16);
                pl[n][0] = __builtin_bit_cast(uint16_t, l4[0]) | ((uint32_t)__builtin_bit_cast(uint16_t, l4[1]) << 16);
                pl[n][1] = __builtin_bit_cast(uint16_t, l4[2]) | ((uint32_t)__builtin_bit_cast(uint16_t, l4[3]) << 16);
            }
            psum += __shfl_xor(psum, 16, VK_WAVE);
            psum += __shfl_xor(psum, 32, VK_WAVE);
            l_run = l_run * alpha + psum;
            m_run = m_new;
            // o * 1.0f is o: when no lane's running max moved, the rescale is skipped
            if (__any(alpha != 1.0f)) {
#pragma unroll
                for (int os = 0; os < OS; ++os)
#pragma unroll
                    for (int r = 0; r < 4; ++r) o_acc[os][r] *= alpha;
            }
            // ---- O^T += V^T . P^T over 2 key steps of 32: MFMA k-index 8g + 4j + r
            //      is key 32ks + 16j + 4g + r (the lane's P values, in order)
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
                const vk_h16x8 bh = __builtin_bit_cast(
                    vk_h16x8, make_uint4(ph[2 * ks][0], ph[2 * ks][1], ph[2 * ks + 1][0], ph[2 * ks + 1][1]));
                const vk_h16x8 bl = __builtin_bit_cast(
                    vk_h16x8, make_uint4(pl[2 * ks][0], pl[2 * ks][1], pl[2 * ks + 1][0], pl[2 * ks + 1][1]));
#pragma unroll
                for (int os = 0; os < OS; ++os) {
                    const int row = (16 * os + lq) * VROW;
                    const int k0 = 32 * ks + 4 * g;
                    const uint2 h0 = *reinterpret_cast<const uint2*>(&lv[0][row + k0]);
                    const uint2 h1 = *reinterpret_cast<const uint2*>(&lv[0][row + k0 + 16]);
                    const vk_h16x8 ah = __builtin_bit_cast(vk_h16x8, make_uint4(h0.x, h0.y, h1.x, h1.y));
                    o_acc[os] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bh, o_acc[os], 0, 0, 0);
                    o_acc[os] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bl, o_acc[os], 0, 0, 0);
                    if (LO) {
                        const uint2 l0 = *reinterpret_cast<const uint2*>(&lv[NP - 1][row + k0]);
                        const uint2 l1 = *reinterpret_cast<const uint2*>(&lv[NP - 1][row + k0 + 16]);
                        const vk_h16x8 al = __builtin_bit_cast(vk_h16x8, make_uint4(l0.x, l0.y, l1.x, l1.y));
                        o_acc[os] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bh, o_acc[os], 0, 0, 0);
                    }
                }
            }
        }
        VK_LDS_BARRIER();
    }
    if (active) finish(o_acc, l_run > 0.0f ? 1.0f / l_run : 0.0f);
}

}  // namespace vk

#include "vk_launch.h"

namespace vk {

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
                              void* vth, void* vtl) {
    if (batch == 0 || t_pad == 0) return hipSuccess;
    hipLaunchKernelGGL(vk_split_vt_q7, dim3(t_pad / 64, h_kv * (hd / 64), batch), dim3(256), 0, s, v, t_kv, t_pad,
                       h_kv, hd, (uint16_t*)vth, (int8_t*)vtl);
    return hipGetLastError();
}

hipError_t launch_split_vt(hipStream_t s, const float* v, int batch, int t_kv, int t_pad, int h_kv, int hd, void* vth,
                           void* vtl) {
    if (batch == 0 || t_pad == 0) return hipSuccess;
    hipLaunchKernelGGL(vk_split_vt, dim3(t_pad / 64, h_kv * (hd / 64), batch), dim3(256), 0, s, v, t_kv, t_pad, h_kv,
                       hd, (uint16_t*)vth, (uint16_t*)vtl);
    return hipGetLastError();
}

template <int HD, int LOM>
static void go_flash1(hipStream_t s, dim3 grid, const void* qh, const void* ql, const void* kh, const void* kl,
                      const void* vth, const void* vtl, float* out, int tq, int tkv, int t_pad, int hq, int hkv,
                      int causal, int q_off, const int* kv_index, const float* qf, float q_scale, const VkQOut& qo) {
    if (tq == 1)
        hipLaunchKernelGGL((vk_flash_attn<HD, LOM, true>), grid, dim3(256), 0, s, (const uint4*)qh, (const uint4*)ql,
                           (const uint4*)kh, (const uint4*)kl, (const uint4*)vth, (const uint4*)vtl, out, tq, tkv,
                           t_pad, hq, hkv, causal, q_off, kv_index, qf, q_scale, qo);
    else
        hipLaunchKernelGGL((vk_flash_attn<HD, LOM, false>), grid, dim3(256), 0, s, (const uint4*)qh, (const uint4*)ql,
                           (const uint4*)kh, (const uint4*)kl, (const uint4*)vth, (const uint4*)vtl, out, tq, tkv,
                           t_pad, hq, hkv, causal, q_off, kv_index, qf, q_scale, qo);
}

template <int HD>
static void go_flash_hd(hipStream_t s, dim3 grid, const void* qh, const void* ql, const void* kh, const void* kl,
                        const void* vth, const void* vtl, float* out, int tq, int tkv, int t_pad, int hq, int hkv,
                        int causal, int q_off, const int* kv_index, const float* qf, float q_scale, int lo_mode,
                        const VkQOut& qo) {
    if (lo_mode == KV_LO_Q7 && tq == 1)  // the compact form exists for single-query launches only
        go_flash1<HD, 2>(s, grid, qh, ql, kh, kl, vth, vtl, out, tq, tkv, t_pad, hq, hkv, causal, q_off, kv_index, qf,
                         q_scale, qo);
    else if (lo_mode == KV_LO_F16)
        go_flash1<HD, 1>(s, grid, qh, ql, kh, kl, vth, vtl, out, tq, tkv, t_pad, hq, hkv, causal, q_off, kv_index, qf,
                         q_scale, qo);
    else
        go_flash1<HD, 0>(s, grid, qh, ql, kh, kl, vth, vtl, out, tq, tkv, t_pad, hq, hkv, causal, q_off, kv_index, qf,
                         q_scale, qo);
}

static hipError_t flash_any(hipStream_t s, int hd, const void* qh, const void* ql, const float* qf, float q_scale,
                            const void* kh, const void* kl, const void* vth, const void* vtl, float* out, int batch,
                            int tq, int tkv, int t_pad, int hq, int hkv, int causal, int q_off, const int* kv_index,
                            int lo_mode, const VkQOut& qo) {
    if (lo_mode == KV_LO_Q7 && tq != 1) return hipErrorInvalidValue;
    const dim3 grid((tq + attn::QT - 1) / attn::QT, hq, batch);
    if (hd == 64)
        go_flash_hd<64>(s, grid, qh, ql, kh, kl, vth, vtl, out, tq, tkv, t_pad, hq, hkv, causal, q_off, kv_index, qf,
                        q_scale, lo_mode, qo);
    else
        go_flash_hd<128>(s, grid, qh, ql, kh, kl, vth, vtl, out, tq, tkv, t_pad, hq, hkv, causal, q_off, kv_index, qf,
                         q_scale, lo_mode, qo);
    return hipGetLastError();
}

hipError_t launch_flash_attn(hipStream_t s, int hd, const void* qh, const void* ql, const void* kh, const void* kl,
                             const void* vth, const void* vtl, float* out, int batch, int tq, int tkv, int t_pad,
                             int hq, int hkv, int causal, int q_off, const int* kv_index, int lo_mode) {
    return flash_any(s, hd, qh, ql, nullptr, 1.0f, kh, kl, vth, vtl, out, batch, tq, tkv, t_pad, hq, hkv, causal,
                     q_off, kv_index, lo_mode, VkQOut{});
}

hipError_t launch_flash_attn_f32q(hipStream_t s, int hd, const float* q, float q_scale, const void* kh, const void* kl,
                                  const void* vth, const void* vtl, float* out, int batch, int tq, int tkv, int t_pad,
                                  int hq, int hkv, int causal, int q_off, const int* kv_index, int lo_mode,
                                  const VkQOut* qo) {
    return flash_any(s, hd, nullptr, nullptr, q, q_scale, kh, kl, vth, vtl, out, batch, tq, tkv, t_pad, hq, hkv,
                     causal, q_off, kv_index, lo_mode, qo ? *qo : VkQOut{});
}

// Reads and clears this file's fp16-range flag on the current device; the
// copies run on stream s, which is drained first.
hipError_t attn_range_take(hipStream_t s, unsigned* raised) {
    unsigned v = 0;
    hipError_t e = hipMemcpyFromSymbolAsync(&v, HIP_SYMBOL(vk_attn_range_flag), sizeof v, 0, hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e == hipSuccess && v) {
        const unsigned z = 0;
        e = hipMemcpyToSymbolAsync(HIP_SYMBOL(vk_attn_range_flag), &z, sizeof z, 0, hipMemcpyHostToDevice, s);
        if (e == hipSuccess) e = hipStreamSynchronize(s);
    }
    *raised = v;
    return e;
}

}  // namespace vk

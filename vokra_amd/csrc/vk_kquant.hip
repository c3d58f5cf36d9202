// vk_kquant.hip — Q4_K (256-element super-block) kernels for gfx950.
//
// Q4_K wire block (crates/vokra-core/src/gguf/tensor.rs:57-128, 144 bytes):
//   d (f16), dmin (f16), 12 bytes of packed 6-bit (scale, min) x 8 sub-blocks,
//   128 bytes of nibbles: 64-element chunk c holds element 64c + l in the low
//   nibble of byte 32c + l and element 64c + 32 + l in its high nibble.
//
// The INT8 matmul reproduces the reference's only integer path, the K-quant
// GEMV of crates/vokra-backend-cpu/src/kernels/kquant.rs:590-629:
//   activations: per 16 elements s = amax / 127, r = round(v / s) clamped to
//                +-127, gsum = sum r                       (kquant.rs:418-441)
//   weights:     q in 0..15, d_eff = d * sc, m_eff = dmin * m per 32 elements
//   combine:     acc += s * (d_eff * isum - m_eff * gsum) per 16-group, in
//                block then group order from acc = 0       (kquant.rs:447-449)
// The integer group sums isum come out of bf16 MFMAs exactly (every operand
// is an integer of at most 8 bits, every partial sum is below 2^24) and the
// float combine runs one thread per output in the reference's order with the
// same roundings, so outputs are bit-identical to the reference.
#include "vk_common.h"

#include <type_traits>

namespace vk {

namespace kq {
constexpr int QK = 256;      // elements per super-block
constexpr int BB = 144;      // bytes per super-block
constexpr int NG = 16;       // 16-element groups per super-block
}  // namespace kq

typedef short vk_s16x4 __attribute__((ext_vector_type(4)));

// crates/vokra-core/src/gguf/quant/mod.rs:140-149 get_scale_min_k4
__device__ __forceinline__ void scale_min_k4(int j, const uint8_t* s, int& d, int& m) {
    if (j < 4) {
        d = s[j] & 63;
        m = s[j + 4] & 63;
    } else {
        d = (s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4);
        m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
    }
}

// ---------------------------------------------------------------------------
// Dequantize (crates/vokra-core/src/gguf/quant/q4_k.rs:34-69): one thread per
// 4 outputs; y = d1 * q - m1 with two roundings, as the reference.
__global__ void vk_dequantize_q4k(const uint8_t* __restrict__ bytes, size_t nsb, float* __restrict__ out) {
    const size_t gid = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t sb = gid >> 6;
    if (sb >= nsb) return;
    const int t = (int)(gid & 63);
    const uint8_t* blk = bytes + sb * kq::BB;
    const float d = vk_f16_to_f32(blk[0] | (blk[1] << 8));
    const float dmin = vk_f16_to_f32(blk[2] | (blk[3] << 8));
    const int c = t >> 4, l = (t & 15) * 2;
    int sc0, m0, sc1, m1;
    scale_min_k4(2 * c, blk + 4, sc0, m0);
    scale_min_k4(2 * c + 1, blk + 4, sc1, m1);
    const float d1 = d * (float)sc0, mm1 = dmin * (float)m0;
    const float d2 = d * (float)sc1, mm2 = dmin * (float)m1;
    const uint32_t q0 = blk[16 + 32 * c + l], q1 = blk[16 + 32 * c + l + 1];
    float* y = out + sb * kq::QK + 64 * c;
    y[l] = d1 * (float)(q0 & 15u) - mm1;
    y[l + 1] = d1 * (float)(q1 & 15u) - mm1;
    y[32 + l] = d2 * (float)(q0 >> 4) - mm2;
    y[33 + l] = d2 * (float)(q1 >> 4) - mm2;
}

// Q5_K (crates/vokra-core/src/gguf/quant/q5_k.rs:36-80): Q4_K's layout with
// 32 bytes of fifth bits before the nibbles (176 bytes); element 64c + l takes
// qh[l] bit 2c, element 64c + 32 + l bit 2c + 1. One thread per 4 outputs.
__global__ void vk_dequantize_q5k(const uint8_t* __restrict__ bytes, size_t nsb, float* __restrict__ out) {
    const size_t gid = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t sb = gid >> 6;
    if (sb >= nsb) return;
    const int t = (int)(gid & 63);
    const uint8_t* blk = bytes + sb * 176;
    const float d = vk_f16_to_f32(blk[0] | (blk[1] << 8));
    const float dmin = vk_f16_to_f32(blk[2] | (blk[3] << 8));
    const int c = t >> 4, l = (t & 15) * 2;
    int sc0, m0, sc1, m1;
    scale_min_k4(2 * c, blk + 4, sc0, m0);
    scale_min_k4(2 * c + 1, blk + 4, sc1, m1);
    const float d1 = d * (float)sc0, mm1 = dmin * (float)m0;
    const float d2 = d * (float)sc1, mm2 = dmin * (float)m1;
    const uint8_t* qh = blk + 16;
    const uint32_t q0 = blk[48 + 32 * c + l], q1 = blk[48 + 32 * c + l + 1];
    const uint32_t lo_bit = 1u << (2 * c), hi_bit = 2u << (2 * c);
    float* y = out + sb * kq::QK + 64 * c;
    y[l] = d1 * (float)((q0 & 15u) + ((qh[l] & lo_bit) ? 16u : 0u)) - mm1;
    y[l + 1] = d1 * (float)((q1 & 15u) + ((qh[l + 1] & lo_bit) ? 16u : 0u)) - mm1;
    y[32 + l] = d2 * (float)((q0 >> 4) + ((qh[l] & hi_bit) ? 16u : 0u)) - mm2;
    y[33 + l] = d2 * (float)((q1 >> 4) + ((qh[l + 1] & hi_bit) ? 16u : 0u)) - mm2;
}

// Q6_K (crates/vokra-core/src/gguf/quant/q6_k.rs:34-72, 210 bytes): per
// 128-element half, 64 bytes of low nibbles, 32 bytes of 2-bit high parts,
// 8 int8 scales; y = d * sc * (q - 32) in that association. One thread per
// (half, l): the four outputs l, l + 32, l + 64, l + 96 of the half.
__global__ void vk_dequantize_q6k(const uint8_t* __restrict__ bytes, size_t nsb, float* __restrict__ out) {
    const size_t gid = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t sb = gid >> 6;
    if (sb >= nsb) return;
    const int t = (int)(gid & 63), half = t >> 5, l = t & 31;
    const uint8_t* blk = bytes + sb * 210;
    const float d = vk_f16_to_f32(blk[208] | (blk[209] << 8));
    const uint8_t* ql = blk + 64 * half;
    const uint8_t* qh = blk + 128 + 32 * half;
    const int8_t* sc = reinterpret_cast<const int8_t*>(blk + 192 + 8 * half);
    const int is = l / 16;
    const int q1 = (int)((ql[l] & 0xF) | ((qh[l] & 3) << 4)) - 32;
    const int q2 = (int)((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
    const int q3 = (int)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
    const int q4 = (int)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
    float* y = out + sb * kq::QK + 128 * half;
    y[l] = d * (float)sc[is] * (float)q1;
    y[l + 32] = d * (float)sc[is + 2] * (float)q2;
    y[l + 64] = d * (float)sc[is + 4] * (float)q3;
    y[l + 96] = d * (float)sc[is + 6] * (float)q4;
}

// ---------------------------------------------------------------------------
// Activation quantization, K-quant convention (kquant.rs:418-441): per row and
// 16-wide group g, amax = max |v| (NaN ignored), s = amax / 127, q =
// clamp(round_half_away(v / s), -127, 127) with NaN -> 0, gsum = sum q (all
// zero when amax == 0). Writes
//   afrag: bf16 integers in the 16x16x16 MFMA A-operand layout, per
//          (16-row tile mt, super-block sb, group pair gp) 64 lanes x 16 bytes:
//          lane l = row % 16 + 16 c holds K 4c..4c+3 of group 2gp (bytes 0..7)
//          and of group 2gp + 1 (bytes 8..15);
//   ascale: per run of 4 groups (g / 4), per row, the 4 groups' (s, (float)
//          gsum) pairs back to back: float2 index ((g / 4) * m_pad + row) * 4
//          + g % 4 (so a matmul lane reads its group's pair with one 8-byte
//          load).
// Rows m..m_pad-1 are written as zeros.
// One element of the pass, formed by the 16 lanes of its group together (an
// aligned run of 16 lanes, lane t holding element t of the group; v = 0 on
// the padding rows, which gives their zeros): the group's amax (NaN -> 0,
// then an integer max of the non-negative values: the same as a fmaxf chain
// from 0), s, q and integer sum, q's bf16 into its fragment slot, and from
// lane t = 0 the (s, gsum) pair.
__device__ __forceinline__ void vk_q16_lane(int row, int g, int t, float v, int m_pad, int nsb,
                                            uint2* __restrict__ afrag, float* __restrict__ ascale) {
    const float amax = vk_group_max<16>(fmaxf(0.0f, fabsf(v)));
    float s = 0.0f;
    int r = 0;
    if (amax != 0.0f) {
        s = amax / 127.0f;
        const float q = vk_round_half_away(v / s);
        // clamp(-127, 127) keeps NaN; `as i32` then maps NaN to 0
        r = (q != q) ? 0 : (int)fminf(fmaxf(q, -127.0f), 127.0f);
    }
    const int gsum = vk_group_sum_i<16>(r);
    const int mt = row >> 4, sb = g / kq::NG, gi = g % kq::NG;
    const size_t base = ((((size_t)mt * nsb + sb) * 8 + (gi >> 1)) * 64) * 2 + (gi & 1);
    const int lane = (row & 15) + 16 * (t >> 2);
    reinterpret_cast<uint16_t*>(afrag)[(base + (size_t)lane * 2) * 4 + (t & 3)] = (uint16_t)vk_int_to_bf16_bits(r);
    if (t == 0) {
        const size_t si = ((size_t)(g >> 2) * m_pad + row) * 4 + (g & 3);
        reinterpret_cast<float2*>(ascale)[si] = make_float2(s, (float)gsum);
    }
}

// The pass over an f32 matrix: one thread per element, grid (k / 256, m_pad).
__global__ __launch_bounds__(256) void vk_quantize_act_g16(const float* __restrict__ a, int m, int m_pad, int k,
                                                           uint2* __restrict__ afrag, float* __restrict__ ascale) {
    const int row = blockIdx.y, col = blockIdx.x * 256 + threadIdx.x;
    const float v = row < m ? a[(size_t)row * k + col] : 0.0f;
    vk_q16_lane(row, col >> 4, col & 15, v, m_pad, k / kq::QK, afrag, ascale);
}

// RMSNorm fused with the activation pass, grid (m_pad, k / 256): each
// workgroup forms its row's sum of squares exactly as vk_rms_norm_f32 forms
// it (thread t sums columns t, t + 256, ... in order, then vk_block_sum256),
// y = x * inv * gamma, and quantizes its 256-column slice of y as
// vk_quantize_act_g16 would, one element per thread (thread t's element,
// column 256 * slice + t, is one it summed). Rows m .. m_pad-1 write the zero
// padding. Bit-identical to the two launches.
constexpr int kRmsRowRegs = 2048;  // rows up to this many columns are read once, into registers
__global__ __launch_bounds__(256) void vk_rms_quantize_g16(const float* __restrict__ in,
                                                           const float* __restrict__ gamma, float eps, int m,
                                                           int m_pad, int k, uint2* __restrict__ afrag,
                                                           float* __restrict__ ascale) {
    __shared__ float red[4];
    const int row = blockIdx.x, part = blockIdx.y, col = part * 256 + (int)threadIdx.x;
    const bool live = row < m;  // uniform per workgroup
    const float* ir = in + (size_t)row * k;
    float v = 0.0f;
    if (live) {
        const float gc = gamma[col];  // requested ahead of the reduction
        float inv, xc = 0.0f;
        if (k <= kRmsRowRegs) {
            // the row read once: every column requested together
            float x[kRmsRowRegs / 256];
#pragma unroll
            for (int j = 0; j < kRmsRowRegs / 256; ++j) {
                const int c = (int)threadIdx.x + 256 * j;
                x[j] = c < k ? ir[c] : 0.0f;
            }
            float sq = 0.0f;
#pragma unroll
            for (int j = 0; j < kRmsRowRegs / 256; ++j) {
                if ((int)threadIdx.x + 256 * j < k) sq += x[j] * x[j];
                if (j == part) xc = x[j];
            }
            inv = 1.0f / sqrtf(vk_block_sum256(sq, red) / (float)k + eps);
        } else {
            inv = 1.0f / sqrtf(vk_block_sum256(vk_sumsq_cols256(ir, k), red) / (float)k + eps);
            xc = ir[col];
        }
        v = xc * inv * gc;
    }
    vk_q16_lane(row, col >> 4, col & 15, v, m_pad, k / kq::QK, afrag, ascale);
}

// SwiGLU fused with the activation pass: one thread per element, grid
// (k / 256, m_pad), silu(g) * u formed as vk_swiglu_f32 forms it, then
// quantized as vk_quantize_act_g16 would. Bit-identical to the two launches.
__global__ __launch_bounds__(256) void vk_swiglu_quantize_g16(const float* __restrict__ gt,
                                                              const float* __restrict__ up, int m, int m_pad, int k,
                                                              uint2* __restrict__ afrag, float* __restrict__ ascale) {
    const int row = blockIdx.y, col = blockIdx.x * 256 + threadIdx.x;
    float v = 0.0f;
    if (row < m) {
        const size_t o = (size_t)row * k + col;
        const float x = gt[o];
        const float sg = 1.0f / (1.0f + expf(-x));
        const float tt = x * sg;
        v = tt * up[o];
    }
    vk_q16_lane(row, col >> 4, col & 15, v, m_pad, k / kq::QK, afrag, ascale);
}

// ---------------------------------------------------------------------------
// Weight repack (upload time), one thread per (weight row = output column,
// super-block). Device layout per (16-column tile nt, super-block sb):
//   wq:  64 lanes x 32 bytes; lane l = col % 16 + 16 c holds 8 "nibble words",
//        word w covering groups 2w and 2w + 1: for j = 0..3 the pair
//        (K_lo, K_hi) = group 2w + j/2, elements 4c + 2(j%2) and +1, with
//        K_lo at bits 4j..4j+3 and K_hi at bits 16+4j..19+4j, so
//        ((W >> 4j) & 0x000F000F) | 0x43004300 is the bf16 pair (128 + q).
//   wdm: 4 sub-block pairs x 16 columns x 2 sub-blocks of float2 (d * sc,
//        dmin * m): sub-blocks 2p and 2p + 1 of a column side by side.
// Columns n..n_pad-1 are zero.
__device__ __forceinline__ uint32_t q4k_nibble(const uint8_t* qs, int e) {
    const int l = e & 63;
    const uint32_t b = qs[32 * (e >> 6) + (l & 31)];
    return l < 32 ? (b & 15u) : (b >> 4);
}

__global__ void vk_repack_w_q4k(const uint8_t* __restrict__ wq, int n, int n_pad, int nsb,
                                uint4* __restrict__ wq4, float2* __restrict__ wdm) {
    const size_t gid = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= (size_t)n_pad * nsb) return;
    const int col = (int)(gid / nsb), sb = (int)(gid % nsb);
    const int nt = col >> 4, cl = col & 15;
    const size_t tile = (size_t)nt * nsb + sb;
    const bool live = col < n;
    const uint8_t* blk = wq + ((size_t)(live ? col : 0) * nsb + sb) * kq::BB;
    const uint8_t* qs = blk + 16;
    for (int c = 0; c < 4; ++c) {
        uint32_t w[8];
        for (int wi = 0; wi < 8; ++wi) {
            uint32_t x = 0;
            for (int j = 0; j < 4; ++j) {
                const int g = 2 * wi + (j >> 1);
                const int e = 16 * g + 4 * c + 2 * (j & 1);
                if (live) x |= (q4k_nibble(qs, e) << (4 * j)) | (q4k_nibble(qs, e + 1) << (16 + 4 * j));
            }
            w[wi] = x;
        }
        const int lane = cl + 16 * c;
        wq4[(tile * 64 + lane) * 2] = make_uint4(w[0], w[1], w[2], w[3]);
        wq4[(tile * 64 + lane) * 2 + 1] = make_uint4(w[4], w[5], w[6], w[7]);
    }
    const float d = live ? vk_f16_to_f32(blk[0] | (blk[1] << 8)) : 0.0f;
    const float dmin = live ? vk_f16_to_f32(blk[2] | (blk[3] << 8)) : 0.0f;
    // sub-blocks 2p and 2p + 1 of a column side by side (one 16-byte load
    // per term wave p)
    for (int j = 0; j < 8; ++j) {
        int sc = 0, mn = 0;
        if (live) scale_min_k4(j, blk + 4, sc, mn);
        wdm[((tile * 4 + (j >> 1)) * 16 + cl) * 2 + (j & 1)] = make_float2(d * (float)sc, dmin * (float)mn);
    }
}

// Q5_K / Q6_K weights for the matmul (upload time), one thread per (weight
// row = output column, super-block): the super-block unpacked as
// unpack_block_i8 does (crates/vokra-backend-cpu/src/kernels/kquant.rs:
// 332-407) to q in 0..31 (Q5_K) or the biased q6 + 32 in 0..63 (Q6_K), with
// (d_eff, m_eff) per 16-element group: Q5_K's q45_sub_scales pair (d * sc,
// dmin * m) repeated over a sub-block's two groups, Q6_K's d * sc (int8) in
// q6_group_scales order and m_eff = d_eff * 32 (exact). Device layout per
// (16-column tile nt, super-block sb):
//   wq:  64 lanes x 64 bytes; lane l = col % 16 + 16 c holds 16 byte words,
//        word g = K 4c, 4c+2, 4c+1, 4c+3 of group g;
//   wdm: 8 group pairs x 16 columns x 2 groups of float2 (d_eff, m_eff)
//        (groups 2p and 2p + 1 of a column side by side: one 16-byte load).
// Columns n..n_pad-1 are zero.
__global__ void vk_repack_w_kq8(int wdtype, const uint8_t* __restrict__ wq, int n, int n_pad, int nsb,
                                uint4* __restrict__ wq4, float2* __restrict__ wdm) {
    const size_t gid = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= (size_t)n_pad * nsb) return;
    const int col = (int)(gid / nsb), sb = (int)(gid % nsb);
    const int nt = col >> 4, cl = col & 15;
    const size_t tile = (size_t)nt * nsb + sb;
    const bool live = col < n;
    const int bb = wdtype == 13 ? 176 : 210;
    const uint8_t* blk = wq + ((size_t)(live ? col : 0) * nsb + sb) * bb;
    uint8_t q[256];
    float de[16], me[16];
    if (!live) {
        for (int e = 0; e < 256; ++e) q[e] = 0;
        for (int g = 0; g < 16; ++g) de[g] = me[g] = 0.0f;
    } else if (wdtype == 13) {
        const float d = vk_f16_to_f32(blk[0] | (blk[1] << 8));
        const float dmin = vk_f16_to_f32(blk[2] | (blk[3] << 8));
        const uint8_t *qh = blk + 16, *qs = blk + 48;
        for (int j = 0; j < 8; ++j) {
            int sc, mn;
            scale_min_k4(j, blk + 4, sc, mn);
            de[2 * j] = de[2 * j + 1] = d * (float)sc;
            me[2 * j] = me[2 * j + 1] = dmin * (float)mn;
            const int chunk = j / 2, hi = j % 2;
            for (int t = 0; t < 32; ++t) {
                const uint8_t byte = qs[32 * chunk + t];
                uint8_t v = hi ? (uint8_t)(byte >> 4) : (uint8_t)(byte & 0xF);
                if (qh[t] & (1u << j)) v = (uint8_t)(v + 16);
                q[32 * j + t] = v;
            }
        }
    } else {
        const float d = vk_f16_to_f32(blk[208] | (blk[209] << 8));
        const int8_t* sc = reinterpret_cast<const int8_t*>(blk + 192);
        for (int half = 0; half < 2; ++half)
            for (int quarter = 0; quarter < 4; ++quarter)
                for (int sub = 0; sub < 2; ++sub) {
                    const int g = 8 * half + 2 * quarter + sub;  // (128 half + 32 quarter + 16 sub) / 16
                    de[g] = d * (float)sc[8 * half + sub + 2 * quarter];
                    me[g] = de[g] * 32.0f;
                }
        for (int half = 0; half < 2; ++half) {
            const uint8_t *ql = blk + 64 * half, *qh = blk + 128 + 32 * half;
            uint8_t* y = q + 128 * half;
            for (int l = 0; l < 32; ++l) {
                y[l] = (uint8_t)((ql[l] & 0xF) | ((qh[l] & 3) << 4));
                y[l + 32] = (uint8_t)((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4));
                y[l + 64] = (uint8_t)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4));
                y[l + 96] = (uint8_t)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4));
            }
        }
    }
    for (int c = 0; c < 4; ++c) {
        uint32_t w[16];
        for (int g = 0; g < 16; ++g) {
            const uint8_t* e = q + 16 * g + 4 * c;
            w[g] = (uint32_t)e[0] | ((uint32_t)e[2] << 8) | ((uint32_t)e[1] << 16) | ((uint32_t)e[3] << 24);
        }
        uint4* dst = wq4 + (tile * 64 + cl + 16 * c) * 4;
        for (int h = 0; h < 4; ++h) dst[h] = make_uint4(w[4 * h], w[4 * h + 1], w[4 * h + 2], w[4 * h + 3]);
    }
    for (int g = 0; g < 16; ++g) wdm[((tile * 8 + (g >> 1)) * 16 + cl) * 2 + (g & 1)] = make_float2(de[g], me[g]);
}

// bf16 operand (4 values, K 4c..4c+3 of one group) from a nibble word:
// pairs j0 and j0 + 1. mask = 0x000F000F and magic = 0x43004300 come in
// registers, so each half is one v_and_or_b32 (a three-operand instruction
// cannot take literals on this architecture).
__device__ __forceinline__ uint32_t q4k_and_or(uint32_t x, uint32_t mask, uint32_t magic) {
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(x), "v"(mask), "v"(magic));
    return r;
}
__device__ __forceinline__ vk_s16x4 q4k_operand(uint32_t w, int j0, uint32_t mask, uint32_t magic) {
    uint2 r;
    r.x = q4k_and_or(w >> (4 * j0), mask, magic);
    r.y = q4k_and_or(w >> (4 * j0 + 4), mask, magic);
    return __builtin_bit_cast(vk_s16x4, r);
}

// The B operand of group i (of the wave's 4): Q4_K from the nibble words;
// Q5_K / Q6_K from a byte word holding K 4c, 4c+2, 4c+1, 4c+3 of the group,
// so (w & 0x00ff00ff) | magic and ((w >> 8) & 0x00ff00ff) | magic are the
// bf16 pairs (128 + q) of K 4c, 4c+1 and 4c+2, 4c+3 (q <= 63).
template <int FMT, class W>
__device__ __forceinline__ vk_s16x4 kq_operand(const W& wv, int i, uint32_t nib_mask, uint32_t byte_mask,
                                               uint32_t magic) {
    if constexpr (FMT == 0) {
        return q4k_operand(i < 2 ? wv.x : wv.y, 2 * (i & 1), nib_mask, magic);
    } else {
        const uint32_t w = i == 0 ? wv.x : i == 1 ? wv.y : i == 2 ? wv.z : wv.w;
        uint2 r;
        r.x = q4k_and_or(w, byte_mask, magic);
        r.y = q4k_and_or(w >> 8, byte_mask, magic);
        return __builtin_bit_cast(vk_s16x4, r);
    }
}

// ---------------------------------------------------------------------------
// Matmul, one workgroup of 12 waves per 16 x 16 output tile (16 activation
// rows, 16 weight rows), K in chunks of two super-blocks (32 groups).
//
// The reference combine is, per output, acc += s * (d_eff * isum - m_eff *
// gsum) over the groups in order. Only the final add is a dependent chain;
// the term t = s * (d_eff * isum - m_eff * gsum) (four roundings) depends on
// one group alone. So:
//   phase 1 (chunk c): wave w takes 4 groups of the chunk; per group two
//     16x16x16 MFMAs, activations times a constant -128 (removing the +128
//     of the bf16 nibble trick) and then times the (128 + q) weights, give
//     isum exactly for 4 outputs per lane (the 8 MFMAs are issued before any
//     of their results is used), and the lane
//     turns them into the 4 terms with the reference's roundings; the terms
//     go to the LDS buffer of chunk c;
//   phase 2 (chunk c - 1): thread t of waves 8..11 adds the chunk's 32
//     terms of its output to acc, in group order;
//   one barrier per chunk: chunk c's terms are complete, chunk c - 1's free.
// Waves 0..7 only form terms and waves 8..11 only add, so each SIMD runs two
// term waves and one adding wave: the dependent adds of chunk c - 1 overlap
// the term arithmetic of chunk c instead of following it.
// Lane mapping: activations are the MFMA's A operand and weights its B
// operand, so lane l holds rows 4 (l / 16) .. +3 of weight column l % 16.
// Each 16-lane DPP row then needs the same 16 activation scales and 16 group
// sums (4 rows x 4 groups): every lane loads one (s, gsum) pair (a wave
// reads 512 contiguous bytes) and the values reach their users through
// row_newbcast DPP operands of the multiplies themselves, and a lane's own
// column needs only its two (d_eff, m_eff) pairs, stored side by side: one
// 8-byte and one 16-byte load per lane (Q5_K / Q6_K: two 16-byte loads for
// four per-group pairs) instead of 96 bytes of broadcast data, which keeps
// the texture path off the critical path (each vector-memory instruction of
// a step costs issue time on the CU's memory pipeline: 5 per step instead of
// 7 took 57.0 -> 53.8 us per config-4 layer).
// Term buffer layout per group: the float4 of lane l (its 4 rows) at 4 l, so
// a wave's stores cover 256 consecutive floats, and phase 2's thread t
// (t = thread index - 512) reads float t, the output (row 4 (t / 64) + t % 4,
// column (t / 4) % 16): no bank conflicts on either side.
// Operands are loaded two chunks ahead into two register sets, each load a
// wave-uniform base plus a 32-bit lane offset (a chunk past the end loads the
// last super-block again, unused). Up to three linears over the same
// activations share one grid (blockIdx.x runs over their column tiles in
// turn). Outputs are bit-identical to kquant_gemm_i8: the same terms, added
// in the same order.
namespace kq {
constexpr int CHG = 32;  // groups per chunk (two super-blocks)
constexpr int CHS = 2;   // super-blocks per chunk
template <int FMT>
struct Pipe {
    // FMT 0 (Q4_K): nibble words of this wave's 4 groups; FMT 1 (Q5_K,
    // Q6_K): one byte word per group
    typename std::conditional<FMT == 0, uint2, uint4>::type wv;
    uint4 af[2];         // activation fragments of its 4 groups (2 pairs)
    float s, a;          // one of the DPP row's 16 scales / group sums
    float2 dm[FMT == 0 ? 2 : 4];  // (d_eff, m_eff) of this lane's column: per sub-block / per group
};
// lane J of each 16-lane row, to every lane of that row
template <int J>
__device__ __forceinline__ float row_bcast(float x) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), 0x150 + J, 0xf, 0xf, true));
}
}  // namespace kq

template <int FMT>
__global__ __launch_bounds__(768) void vk_gemm_q4k(const uint4* __restrict__ afrag, const float* __restrict__ ascale,
                                                   VkQ4kSet set, int m, int nsb, int m_pad) {
    using namespace kq;
    __shared__ __align__(16) float lds_t[2][CHG][256];  // terms, [chunk parity][group][4 * lane + r]

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: scalar load bases
    // this workgroup's linear (uniform selects, no indexing into the set)
    const int bx = blockIdx.x, mt = blockIdx.y;
    const int li = (set.count > 2 && bx >= set.tile0[2]) ? 2 : (set.count > 1 && bx >= set.tile0[1]) ? 1 : 0;
    const VkQ4kLin L = li == 2 ? set.l[2] : li == 1 ? set.l[1] : set.l[0];
    const int nt = bx - (li == 2 ? set.tile0[2] : li == 1 ? set.tile0[1] : 0);
    const int q4 = wave & 3, sbw = (wave >> 2) & 1;  // a term wave's quarter of a super-block, and which one
    const int n_chunk = (nsb + CHS - 1) / CHS;
    // phase-2 thread: waves 8..11, output (row, col) of the term layout
    const int ot = tid - 512;
    const int orow = 4 * (ot >> 6) + (ot & 3), ocol = (ot >> 2) & 15;
    const bool owner = wave >= 8;

    // per-lane byte offsets (constant over the K loop)
    const uint32_t vo_w = FMT == 0 ? lane * 32 + 8 * q4 : lane * 64 + 16 * q4;
    const uint32_t vo_a = lane * 16;
    const uint32_t vo_d = (lane & 15) * 16;
    const uint32_t vo_s = ((uint32_t)(mt * 16) * 16 + lane * 4) * 2;

    // Buffer resources over the five operand arrays: every load is a
    // constant per-lane offset plus a wave-uniform offset computed on the
    // scalar unit, so no vector instruction forms an address in the K loop.
    const int n_pad = (L.n + 15) & ~15;
    const int rsrc_w3 = 0x00020000;  // raw (unswizzled) dword access
    const __amdgpu_buffer_rsrc_t rw =
        __builtin_amdgcn_make_buffer_rsrc((void*)L.wq4, 0, n_pad * nsb * (FMT == 0 ? 128 : 256), rsrc_w3);
    const __amdgpu_buffer_rsrc_t rd =
        __builtin_amdgcn_make_buffer_rsrc((void*)L.wdm, 0, n_pad * nsb * (FMT == 0 ? 64 : 128), rsrc_w3);
    const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc((void*)afrag, 0, m_pad * nsb * 512, rsrc_w3);
    // (s, gsum) pairs of the K-quant activation layout
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void*)ascale, 0, m_pad * nsb * 128, rsrc_w3);
    typedef unsigned int vk_u32x2 __attribute__((ext_vector_type(2)));
    typedef unsigned int vk_u32x4 __attribute__((ext_vector_type(4)));

    // chunk c's operands for this wave (super-block 2c + sbw, clamped into
    // the tensor: a super-block past the end loads the last one, unused).
    auto load = [&](int c) -> Pipe<FMT> {
        Pipe<FMT> p;
        const int sb = min(c * CHS + sbw, nsb - 1);
        const int ow = ((nt * nsb + sb) * 64) * (FMT == 0 ? 32 : 64);
        const int oa = (((mt * nsb + sb) * 8 + 2 * q4) * 64) * 16;
        // scales / sums of groups 4 q4 .. +3 of rows mt*16 .. +15: 256 bytes,
        // lane 16 k + j holding row 4 k + j / 4, group j % 4
        const int os = (sb * (NG / 4) + q4) * m_pad * 32;
        const int od = FMT == 0 ? ((nt * nsb + sb) * 4 + q4) * 256 : ((nt * nsb + sb) * 8 + 2 * q4) * 256;
        if constexpr (FMT == 0) {
            const vk_u32x2 w2 = __builtin_amdgcn_raw_buffer_load_b64(rw, vo_w, ow, 0);
            p.wv = make_uint2(w2.x, w2.y);
        } else {
            const vk_u32x4 w4 = __builtin_amdgcn_raw_buffer_load_b128(rw, vo_w, ow, 0);
            p.wv = make_uint4(w4.x, w4.y, w4.z, w4.w);
        }
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const vk_u32x4 x = __builtin_amdgcn_raw_buffer_load_b128(ra, vo_a + h * 1024, oa, 0);
            p.af[h] = make_uint4(x.x, x.y, x.z, x.w);
        }
        const vk_u32x2 sa = __builtin_amdgcn_raw_buffer_load_b64(rs, vo_s, os, 0);
        p.s = __uint_as_float(sa.x);
        p.a = __uint_as_float(sa.y);
#pragma unroll
        for (int jj = 0; jj < (FMT == 0 ? 2 : 4); jj += 2) {
            const vk_u32x4 x = __builtin_amdgcn_raw_buffer_load_b128(rd, vo_d, od + jj * 128, 0);
            p.dm[jj] = make_float2(__uint_as_float(x.x), __uint_as_float(x.y));
            p.dm[jj + 1] = make_float2(__uint_as_float(x.z), __uint_as_float(x.w));
        }
        return p;
    };
    // phase 1: the terms of this wave's 4 groups into buffer par (for a
    // super-block past the end the terms come from the clamped loads and
    // phase 2 never reads them)
    // the bf16 pair (-128, -128)
    uint32_t neg128_bf16;
    asm volatile("v_mov_b32 %0, 0xc300c300" : "=v"(neg128_bf16));
    uint32_t nib_mask, byte_mask, nib_magic;
    asm volatile("v_mov_b32 %0, 0x000f000f" : "=v"(nib_mask));
    asm volatile("v_mov_b32 %0, 0x00ff00ff" : "=v"(byte_mask));
    asm volatile("v_mov_b32 %0, 0x43004300" : "=v"(nib_magic));
    auto terms = [&](const Pipe<FMT>& p, int par) {
        vk_f32x4 isum[4];
        // The accumulator input -128 * gsum of each output comes from the
        // matrix core too: the product of the group's activations with a
        // constant -128 operand (exact: integers below 2^24), so no VALU
        // instruction forms it; the second product then adds the
        // (128 + q) weights. Both MFMAs of all 4 groups are issued before
        // any result is read.
        const vk_s16x4 neg128 = __builtin_bit_cast(vk_s16x4, make_uint2(neg128_bf16, neg128_bf16));
        vk_s16x4 aop[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint4 a4 = p.af[i >> 1];
            aop[i] = __builtin_bit_cast(vk_s16x4, (i & 1) ? make_uint2(a4.z, a4.w) : make_uint2(a4.x, a4.y));
            isum[i] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(aop[i], neg128, (vk_f32x4){0.0f, 0.0f, 0.0f, 0.0f},
                                                                0, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i)
            isum[i] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(
                aop[i], kq_operand<FMT>(p.wv, i, nib_mask, byte_mask, nib_magic), isum[i], 0, 0, 0);
        // The 16 terms of the wave's 4 groups breadth first, one rounding step
        // at a time over all of them (the issue order is pinned): each step's
        // 16 operations are independent, so no multiply waits on the one
        // before it.
        float x[4][4], y[4][4];
#define VK_Q4K_STEP1(i)                                                                                         \
        {                                                                                                       \
            const float2 dm = p.dm[FMT == 0 ? (i) >> 1 : (i)];                                                  \
            x[i][0] = dm.x * isum[i][0]; x[i][1] = dm.x * isum[i][1];                                           \
            x[i][2] = dm.x * isum[i][2]; x[i][3] = dm.x * isum[i][3];                                           \
            y[i][0] = dm.y * row_bcast<(i)>(p.a); y[i][1] = dm.y * row_bcast<4 + (i)>(p.a);                     \
            y[i][2] = dm.y * row_bcast<8 + (i)>(p.a); y[i][3] = dm.y * row_bcast<12 + (i)>(p.a);                \
        }
        VK_Q4K_STEP1(0) VK_Q4K_STEP1(1) VK_Q4K_STEP1(2) VK_Q4K_STEP1(3)
#undef VK_Q4K_STEP1
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) x[i][r] = x[i][r] - y[i][r];
        __builtin_amdgcn_sched_barrier(0);
#define VK_Q4K_STEP3(i)                                                                                         \
        {                                                                                                       \
            float4 t;                                                                                           \
            t.x = row_bcast<(i)>(p.s) * x[i][0]; t.y = row_bcast<4 + (i)>(p.s) * x[i][1];                        \
            t.z = row_bcast<8 + (i)>(p.s) * x[i][2]; t.w = row_bcast<12 + (i)>(p.s) * x[i][3];                  \
            *reinterpret_cast<float4*>(&lds_t[par][16 * sbw + 4 * q4 + (i)][4 * lane]) = t;                     \
        }
        VK_Q4K_STEP3(0) VK_Q4K_STEP3(1) VK_Q4K_STEP3(2) VK_Q4K_STEP3(3)
#undef VK_Q4K_STEP3
    };
    // phase 2: the ordered adds of chunk c (waves 0..3, one output per thread)
    float acc = 0.0f;
    auto chain = [&](int c, int par) {
        if (c < 0 || c >= n_chunk) return;
        const int ng = min(CHS, nsb - c * CHS) * NG;
        if (ng == CHG) {
#pragma unroll
            for (int g = 0; g < CHG; ++g) acc += lds_t[par][g][ot];
        } else {
#pragma unroll
            for (int g = 0; g < NG; ++g) acc += lds_t[par][g][ot];
        }
    };

    // The term waves issue every load unconditionally (chunks past the end
    // re-read the last super-block) and from one place, their loop body, so
    // the two register sets are refilled in the same order from the first
    // chunk on: loads issued on one side of a branch, or in another order
    // before the loop, make the compiler wait for all outstanding loads,
    // which would drain the next chunk's prefetch before each term pass. The
    // loop starts one step early (c = -2, an opaque value so it is not peeled
    // off) to issue the first two chunks' loads; each term pass then waits
    // for its own register set only. Both loops pass the same barriers.
    int c0;
    asm volatile("s_mov_b32 %0, -2" : "=s"(c0));
    if (!owner) {
        Pipe<FMT> pa{}, pb{};
        for (int c = c0; c < n_chunk; c += 2) {
            if (c >= 0) terms(pa, 0);  // chunk c
            pa = load(c + 2);
            VK_LDS_BARRIER();
            if (c >= 0) terms(pb, 1);  // chunk c + 1
            pb = load(c + 3);
            VK_LDS_BARRIER();
        }
        return;
    }
    for (int c = c0; c < n_chunk; c += 2) {
        chain(c - 1, 1);
        VK_LDS_BARRIER();
        chain(c, 0);
        VK_LDS_BARRIER();
    }
    chain(((n_chunk + 1) & ~1) - 1, 1);  // an even count leaves its last chunk
    const int r = mt * 16 + orow, col = nt * 16 + ocol;
    if (r < m && col < L.n) {
        const size_t o = (size_t)r * L.n + col;
        L.out[o] = vk_epi_apply(L.bias ? acc + L.bias[col] : acc, L.epi, o);
    }
}

}  // namespace vk

#include "vk_launch.h"

namespace vk {

hipError_t launch_dequantize_q4k(hipStream_t s, const uint8_t* bytes, size_t nsb, float* out) {
    if (nsb == 0) return hipSuccess;
    const size_t threads = nsb * 64;
    hipLaunchKernelGGL(vk_dequantize_q4k, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, s, bytes, nsb, out);
    return hipGetLastError();
}

hipError_t launch_dequantize_kq(hipStream_t s, int wdtype, const uint8_t* bytes, size_t nsb, float* out) {
    if (nsb == 0) return hipSuccess;
    const size_t threads = nsb * 64;
    const dim3 grid((unsigned)((threads + 255) / 256)), block(256);
    if (wdtype == 12) hipLaunchKernelGGL(vk_dequantize_q4k, grid, block, 0, s, bytes, nsb, out);
    else if (wdtype == 13) hipLaunchKernelGGL(vk_dequantize_q5k, grid, block, 0, s, bytes, nsb, out);
    else if (wdtype == 14) hipLaunchKernelGGL(vk_dequantize_q6k, grid, block, 0, s, bytes, nsb, out);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t launch_repack_w_kq8(hipStream_t s, int wdtype, const uint8_t* wq, int n, int n_pad, int nsb, uint4* wq4,
                               float2* wdm) {
    if (wdtype != 13 && wdtype != 14) return hipErrorInvalidValue;
    const size_t threads = (size_t)n_pad * nsb;
    if (threads == 0) return hipSuccess;
    hipLaunchKernelGGL(vk_repack_w_kq8, dim3((unsigned)((threads + 63) / 64)), dim3(64), 0, s, wdtype, wq, n, n_pad,
                       nsb, wq4, wdm);
    return hipGetLastError();
}

hipError_t launch_quantize_act_g16(hipStream_t s, const float* a, int m, int m_pad, int k, uint4* afrag,
                                   float* ascale) {
    if (k % kq::QK != 0 || m_pad % 16 != 0 || m_pad > 65535) return hipErrorInvalidValue;
    if (k == 0 || m_pad == 0) return hipSuccess;
    hipLaunchKernelGGL(vk_quantize_act_g16, dim3((unsigned)(k / 256), (unsigned)m_pad), dim3(256), 0, s, a, m,
                       m_pad, k, reinterpret_cast<uint2*>(afrag), ascale);
    return hipGetLastError();
}

hipError_t launch_rms_quantize_g16(hipStream_t s, const float* in, const float* gamma, float eps, int m, int m_pad,
                                   int k, uint4* afrag, float* ascale) {
    if (k % kq::QK != 0 || m_pad % 16 != 0 || k / 256 > 65535) return hipErrorInvalidValue;
    if (k == 0 || m_pad == 0) return hipSuccess;
    hipLaunchKernelGGL(vk_rms_quantize_g16, dim3((unsigned)m_pad, (unsigned)(k / 256)), dim3(256), 0, s, in, gamma,
                       eps, m, m_pad, k, reinterpret_cast<uint2*>(afrag), ascale);
    return hipGetLastError();
}

hipError_t launch_swiglu_quantize_g16(hipStream_t s, const float* g, const float* u, int m, int m_pad, int k,
                                      uint4* afrag, float* ascale) {
    if (k % kq::QK != 0 || m_pad % 16 != 0 || m_pad > 65535) return hipErrorInvalidValue;
    if (k == 0 || m_pad == 0) return hipSuccess;
    hipLaunchKernelGGL(vk_swiglu_quantize_g16, dim3((unsigned)(k / 256), (unsigned)m_pad), dim3(256), 0, s, g, u, m,
                       m_pad, k, reinterpret_cast<uint2*>(afrag), ascale);
    return hipGetLastError();
}

hipError_t launch_repack_w_q4k(hipStream_t s, const uint8_t* wq, int n, int n_pad, int nsb, uint4* wq4,
                               float2* wdm) {
    const size_t threads = (size_t)n_pad * nsb;
    if (threads == 0) return hipSuccess;
    hipLaunchKernelGGL(vk_repack_w_q4k, dim3((unsigned)((threads + 127) / 128)), dim3(128), 0, s, wq, n, n_pad, nsb,
                       wq4, wdm);
    return hipGetLastError();
}

hipError_t launch_gemm_q4k(hipStream_t s, const uint4* afrag, const float* ascale, const VkQ4kLin* lins, int n_lin,
                           int m, int nsb, int m_pad, int fmt) {
    if (n_lin < 1 || n_lin > 3 || fmt < 0 || fmt > 1) return hipErrorInvalidValue;
    VkQ4kSet set{};
    int tiles = 0;
    for (int i = 0; i < n_lin; ++i) {
        set.l[i] = lins[i];
        set.tile0[i] = tiles;
        tiles += (lins[i].n + 15) / 16;
    }
    set.count = n_lin;
    const dim3 grid((unsigned)tiles, (unsigned)((m + 15) / 16));
    if (fmt == 0)
        hipLaunchKernelGGL(vk_gemm_q4k<0>, grid, dim3(768), 0, s, afrag, ascale, set, m, nsb, m_pad);
    else
        hipLaunchKernelGGL(vk_gemm_q4k<1>, grid, dim3(768), 0, s, afrag, ascale, set, m, nsb, m_pad);
    return hipGetLastError();
}

}  // namespace vk

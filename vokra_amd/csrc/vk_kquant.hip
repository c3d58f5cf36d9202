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

// ---------------------------------------------------------------------------
// Activation quantization, K-quant convention (kquant.rs:418-441). One thread
// per (group g, row). Writes
//   afrag: bf16 integers in the 16x16x16 MFMA A-operand layout, per
//          (16-row tile mt, super-block sb, group pair gp) 64 lanes x 16 bytes:
//          lane l = row % 16 + 16 c holds K 4c..4c+3 of group 2gp (bytes 0..7)
//          and of group 2gp + 1 (bytes 8..15);
//   ascale / asum: per run of 4 groups (g / 4), per row, the 4 groups' s and
//          (float) gsum back to back: index ((g / 4) * m_pad + row) * 4 + g % 4.
// Rows m..m_pad-1 are written as zeros.
// One group's activation pass: the 16 values v of (row, group g) -> its
// fragment words, s and gsum (zeros when !live: the padding rows).
__device__ __forceinline__ void vk_q16_store(int row, int g, int m_pad, int nsb, const float (&v)[16], bool live,
                                             uint2* __restrict__ afrag, float* __restrict__ ascale,
                                             float* __restrict__ asum) {
    int r[16];
    float s = 0.0f;
    int gsum = 0;
#pragma unroll
    for (int t = 0; t < 16; ++t) r[t] = 0;
    if (live) {
        float amax = 0.0f;
#pragma unroll
        for (int t = 0; t < 16; ++t) amax = fmaxf(amax, fabsf(v[t]));
        if (amax != 0.0f) {
            s = amax / 127.0f;
#pragma unroll
            for (int t = 0; t < 16; ++t) {
                const float q = vk_round_half_away(v[t] / s);
                // clamp(-127, 127) keeps NaN; `as i32` then maps NaN to 0
                r[t] = (q != q) ? 0 : (int)fminf(fmaxf(q, -127.0f), 127.0f);
                gsum += r[t];
            }
        }
    }
    const int mt = row >> 4, sb = g / kq::NG, gi = g % kq::NG;
    const size_t base = ((((size_t)mt * nsb + sb) * 8 + (gi >> 1)) * 64) * 2 + (gi & 1);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const int lane = (row & 15) + 16 * c;
        const uint2 w = make_uint2(vk_int_to_bf16_bits(r[4 * c]) | (vk_int_to_bf16_bits(r[4 * c + 1]) << 16),
                                   vk_int_to_bf16_bits(r[4 * c + 2]) | (vk_int_to_bf16_bits(r[4 * c + 3]) << 16));
        afrag[base + (size_t)lane * 2] = w;
    }
    const size_t si = ((size_t)(g >> 2) * m_pad + row) * 4 + (g & 3);
    ascale[si] = s;
    asum[si] = (float)gsum;
}

__global__ void vk_quantize_act_g16(const float* __restrict__ a, int m, int m_pad, int k,
                                    uint2* __restrict__ afrag, float* __restrict__ ascale,
                                    float* __restrict__ asum) {
    const int ng = k / 16, nsb = k / kq::QK;
    const size_t gid = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= (size_t)ng * m_pad) return;
    const int g = (int)(gid / m_pad), row = (int)(gid % m_pad);
    float v[16];
    if (row < m) {
        const float4* src = reinterpret_cast<const float4*>(a + (size_t)row * k + 16 * g);
#pragma unroll
        for (int h = 0; h < 4; ++h) {
            const float4 x = src[h];
            v[4 * h] = x.x;
            v[4 * h + 1] = x.y;
            v[4 * h + 2] = x.z;
            v[4 * h + 3] = x.w;
        }
    }
    vk_q16_store(row, g, m_pad, nsb, v, row < m, afrag, ascale, asum);
}

// RMSNorm fused with the activation pass, one workgroup per row (rows m ..
// m_pad-1 write the zero padding): the row's sum of squares exactly as
// vk_rms_norm_f32 forms it (thread t sums columns t, t + 256, ... in order,
// then vk_block_sum256), y = x * inv * gamma, then each 16-wide group as
// vk_quantize_act_g16 would quantize y. Bit-identical to the two launches.
__global__ __launch_bounds__(256) void vk_rms_quantize_g16(const float* __restrict__ in,
                                                           const float* __restrict__ gamma, float eps, int m,
                                                           int m_pad, int k, uint2* __restrict__ afrag,
                                                           float* __restrict__ ascale, float* __restrict__ asum) {
    __shared__ float red[4];
    const int row = blockIdx.x, nsb = k / kq::QK;
    const bool live = row < m;  // uniform per workgroup
    float inv = 0.0f;
    const float* ir = in + (size_t)row * k;
    if (live) {
        float s = 0.0f;
        for (int c = threadIdx.x; c < k; c += 256) s += ir[c] * ir[c];
        inv = 1.0f / sqrtf(vk_block_sum256(s, red) / (float)k + eps);
    }
    for (int g = threadIdx.x; g < k / 16; g += 256) {
        float v[16];
        if (live) {
#pragma unroll
            for (int t = 0; t < 16; ++t) v[t] = ir[16 * g + t] * inv * gamma[16 * g + t];
        }
        vk_q16_store(row, g, m_pad, nsb, v, live, afrag, ascale, asum);
    }
}

// SwiGLU fused with the activation pass: one thread per (group, row), the
// 16 values silu(g) * u formed as vk_swiglu_f32 forms them, then quantized as
// vk_quantize_act_g16 would. Bit-identical to the two launches.
__global__ void vk_swiglu_quantize_g16(const float* __restrict__ gt, const float* __restrict__ up, int m, int m_pad,
                                       int k, uint2* __restrict__ afrag, float* __restrict__ ascale,
                                       float* __restrict__ asum) {
    const int ng = k / 16, nsb = k / kq::QK;
    const size_t gid = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= (size_t)ng * m_pad) return;
    const int g = (int)(gid / m_pad), row = (int)(gid % m_pad);
    float v[16];
    if (row < m) {
        const size_t o = (size_t)row * k + 16 * g;
#pragma unroll
        for (int t = 0; t < 16; ++t) {
            const float x = gt[o + t];
            const float sg = 1.0f / (1.0f + expf(-x));
            const float tt = x * sg;
            v[t] = tt * up[o + t];
        }
    }
    vk_q16_store(row, g, m_pad, nsb, v, row < m, afrag, ascale, asum);
}

// ---------------------------------------------------------------------------
// Weight repack (upload time), one thread per (weight row = output column,
// super-block). Device layout per (16-column tile nt, super-block sb):
//   wq:  64 lanes x 32 bytes; lane l = col % 16 + 16 c holds 8 "nibble words",
//        word w covering groups 2w and 2w + 1: for j = 0..3 the pair
//        (K_lo, K_hi) = group 2w + j/2, elements 4c + 2(j%2) and +1, with
//        K_lo at bits 4j..4j+3 and K_hi at bits 16+4j..19+4j, so
//        ((W >> 4j) & 0x000F000F) | 0x43004300 is the bf16 pair (128 + q).
//   wdm: 8 sub-blocks x 16 columns of float2 (d * sc, dmin * m).
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
    for (int j = 0; j < 8; ++j) {
        int sc = 0, mn = 0;
        if (live) scale_min_k4(j, blk + 4, sc, mn);
        wdm[(tile * 8 + j) * 16 + cl] = make_float2(d * (float)sc, dmin * (float)mn);
    }
}

// bf16 operand (4 values, K 4c..4c+3 of one group) from a nibble word:
// pairs j0 and j0 + 1.
__device__ __forceinline__ vk_s16x4 q4k_operand(uint32_t w, int j0) {
    uint2 r;
    r.x = ((w >> (4 * j0)) & 0x000F000Fu) | 0x43004300u;
    r.y = ((w >> (4 * j0 + 4)) & 0x000F000Fu) | 0x43004300u;
    return __builtin_bit_cast(vk_s16x4, r);
}

// ---------------------------------------------------------------------------
// Matmul, one workgroup of 8 waves per 16 x 16 output tile (16 activation
// rows, 16 weight rows), K in chunks of two super-blocks (32 groups).
//
// The reference combine is, per output, acc += s * (d_eff * isum - m_eff *
// gsum) over the groups in order. Only the final add is a dependent chain;
// the term t = s * (d_eff * isum - m_eff * gsum) (four roundings) depends on
// one group alone. So:
//   phase 1 (chunk c+1): wave w takes 4 groups of the chunk; per group one
//     16x16x16 MFMA with accumulator input -128 * gsum (removing the +128 of
//     the bf16 nibble trick) gives isum exactly for 4 outputs per lane (the
//     4 MFMAs are issued before any of their results is used), and the lane
//     turns them into the 4 terms with the reference's roundings; the terms
//     go to the LDS buffer of chunk c+1;
//   phase 2 (chunk c): thread t of waves 0..3 adds the chunk's 32 terms of
//     its output to acc, in group order;
//   one barrier per chunk: chunk c+1's terms are complete, chunk c's free.
// Term buffer layout per group: output (row, col) at (col / 4) * 64 + row * 4
// + col % 4, so a wave's float4 stores (lane l: row l % 16, cols 4 (l / 16)
// ..+3) cover 256 consecutive floats and phase 2's thread t reads float t:
// no bank conflicts on either side.
// Operands are loaded two chunks ahead into two register sets, each load a
// wave-uniform base plus a 32-bit lane offset (a chunk past the end loads the
// last super-block again, unused). Up to three linears over the same
// activations share one grid (blockIdx.x runs over their column tiles in
// turn). Outputs are bit-identical to kquant_gemm_i8: the same terms, added
// in the same order.
namespace kq {
constexpr int CHG = 32;  // groups per chunk (two super-blocks)
constexpr int CHS = 2;   // super-blocks per chunk
struct Pipe {
    uint2 wv;            // nibble words of this wave's 4 groups
    uint4 af[2];         // activation fragments of its 4 groups (2 pairs)
    float4 s, a;         // s and gsum of this lane's row for its 4 groups
    float4 dm[2][2];     // [sub-block][half]: (d_eff, m_eff) of cols rq + 2 half, +1
};
}  // namespace kq

__global__ __launch_bounds__(512) void vk_gemm_q4k(const uint4* __restrict__ afrag, const float* __restrict__ ascale,
                                                   const float* __restrict__ asum, VkQ4kSet set, int m, int nsb,
                                                   int m_pad) {
    using namespace kq;
    __shared__ __align__(16) float lds_t[2][CHG][256];  // terms, [chunk parity][group][(col/4)*64 + row*4 + col%4]

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: scalar load bases
    // this workgroup's linear (uniform selects, no indexing into the set)
    const int bx = blockIdx.x, mt = blockIdx.y;
    const int li = (set.count > 2 && bx >= set.tile0[2]) ? 2 : (set.count > 1 && bx >= set.tile0[1]) ? 1 : 0;
    const VkQ4kLin L = li == 2 ? set.l[2] : li == 1 ? set.l[1] : set.l[0];
    const int nt = bx - (li == 2 ? set.tile0[2] : li == 1 ? set.tile0[1] : 0);
    const int row_l = lane & 15, rq = 4 * (lane >> 4);  // MFMA lane: activation row, first weight column
    const int q4 = wave & 3, sbw = wave >> 2;           // this wave's quarter of a super-block, and which one
    const int n_chunk = (nsb + CHS - 1) / CHS;
    // phase-2 thread: waves 0..3, output (row, col) of the term layout
    const int orow = (tid >> 2) & 15, ocol = 4 * (tid >> 6) + (tid & 3);
    const bool owner = wave < 4;

    // per-lane byte offsets (constant over the K loop)
    const uint32_t vo_w = lane * 32 + 8 * q4;
    const uint32_t vo_a = lane * 16;
    const uint32_t vo_d = rq * 8;
    const uint32_t vo_s = (uint32_t)(mt * 16 + row_l) * 16;

    // chunk c's operands for this wave (super-block 2c + sbw, clamped into
    // the tensor: a super-block past the end loads the last one, unused).
    auto load = [&](int c) -> Pipe {
        Pipe p;
        const int sb = min(c * CHS + sbw, nsb - 1);
        const char* bw = reinterpret_cast<const char*>(L.wq4) + (size_t)((nt * nsb + sb) * 64) * 32;
        const char* ba = reinterpret_cast<const char*>(afrag) + (size_t)(((mt * nsb + sb) * 8 + 2 * q4) * 64) * 16;
        const size_t so_s = (size_t)(sb * (NG / 4) + q4) * m_pad * 16;
        const char* bs = reinterpret_cast<const char*>(ascale) + so_s;
        const char* bg = reinterpret_cast<const char*>(asum) + so_s;
        const char* bd = reinterpret_cast<const char*>(L.wdm) + (size_t)((nt * nsb + sb) * 8 + 2 * q4) * 128;
        p.wv = *reinterpret_cast<const uint2*>(bw + vo_w);
#pragma unroll
        for (int h = 0; h < 2; ++h) p.af[h] = *reinterpret_cast<const uint4*>(ba + vo_a + h * 1024);
        p.s = *reinterpret_cast<const float4*>(bs + vo_s);
        p.a = *reinterpret_cast<const float4*>(bg + vo_s);
#pragma unroll
        for (int jj = 0; jj < 2; ++jj)
#pragma unroll
            for (int h = 0; h < 2; ++h) p.dm[jj][h] = *reinterpret_cast<const float4*>(bd + vo_d + jj * 128 + h * 16);
        return p;
    };
    // phase 1: the terms of this wave's 4 groups of chunk c into buffer par
    auto terms = [&](const Pipe& p, int c, int par) {
        if (c * CHS + sbw >= nsb) return;  // a chunk with one super-block: waves 4..7 idle
        const float sv[4] = {p.s.x, p.s.y, p.s.z, p.s.w}, av[4] = {p.a.x, p.a.y, p.a.z, p.a.w};
        vk_f32x4 isum[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t word = (i < 2) ? p.wv.x : p.wv.y;
            const vk_s16x4 w = q4k_operand(word, 2 * (i & 1));
            const uint4 a4 = p.af[i >> 1];
            const uint2 ap = (i & 1) ? make_uint2(a4.z, a4.w) : make_uint2(a4.x, a4.y);
            const float c0 = -128.0f * av[i];
            const vk_f32x4 cin = {c0, c0, c0, c0};
            // transposed product: weights as the A operand, so lane l gets
            // activation row l % 16, columns rq..rq+3
            isum[i] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(w, __builtin_bit_cast(vk_s16x4, ap), cin, 0, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float4 d01 = p.dm[i >> 1][0], d23 = p.dm[i >> 1][1];  // (d, m) of cols rq .. rq + 3
            const float s = sv[i], a = av[i];
            float4 t;
            t.x = s * (d01.x * isum[i][0] - d01.y * a);
            t.y = s * (d01.z * isum[i][1] - d01.w * a);
            t.z = s * (d23.x * isum[i][2] - d23.y * a);
            t.w = s * (d23.z * isum[i][3] - d23.w * a);
            *reinterpret_cast<float4*>(&lds_t[par][16 * sbw + 4 * q4 + i][4 * lane]) = t;
        }
    };
    // phase 2: the ordered adds of chunk c (waves 0..3, one output per thread)
    float acc = 0.0f;
    auto chain = [&](int c, int par) {
        if (!owner) return;
        const int ng = min(CHS, nsb - c * CHS) * NG;
        if (ng == CHG) {
#pragma unroll
            for (int g = 0; g < CHG; ++g) acc += lds_t[par][g][tid];
        } else {
#pragma unroll
            for (int g = 0; g < NG; ++g) acc += lds_t[par][g][tid];
        }
    };

    Pipe pa = load(0);
    Pipe pb = load(n_chunk > 1 ? 1 : 0);
    terms(pa, 0, 0);
    if (n_chunk > 2) pa = load(2);
    VK_LDS_BARRIER();
    for (int c = 0; c < n_chunk; c += 2) {
        if (c + 1 < n_chunk) {
            terms(pb, c + 1, 1);
            if (c + 3 < n_chunk) pb = load(c + 3);
        }
        chain(c, 0);
        VK_LDS_BARRIER();
        if (c + 1 >= n_chunk) break;
        if (c + 2 < n_chunk) {
            terms(pa, c + 2, 0);
            if (c + 4 < n_chunk) pa = load(c + 4);
        }
        chain(c + 1, 1);
        VK_LDS_BARRIER();
    }
    if (owner) {
        const int r = mt * 16 + orow, col = nt * 16 + ocol;
        if (r < m && col < L.n) {
            const size_t o = (size_t)r * L.n + col;
            L.out[o] = vk_epi_apply(L.bias ? acc + L.bias[col] : acc, L.epi, o);
        }
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

hipError_t launch_quantize_act_g16(hipStream_t s, const float* a, int m, int m_pad, int k, uint4* afrag,
                                   float* ascale, float* asum) {
    const size_t threads = (size_t)(k / 16) * m_pad;
    if (threads == 0) return hipSuccess;
    hipLaunchKernelGGL(vk_quantize_act_g16, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, s, a, m, m_pad,
                       k, reinterpret_cast<uint2*>(afrag), ascale, asum);
    return hipGetLastError();
}

hipError_t launch_rms_quantize_g16(hipStream_t s, const float* in, const float* gamma, float eps, int m, int m_pad,
                                   int k, uint4* afrag, float* ascale, float* asum) {
    if (m_pad == 0) return hipSuccess;
    hipLaunchKernelGGL(vk_rms_quantize_g16, dim3((unsigned)m_pad), dim3(256), 0, s, in, gamma, eps, m, m_pad, k,
                       reinterpret_cast<uint2*>(afrag), ascale, asum);
    return hipGetLastError();
}

hipError_t launch_swiglu_quantize_g16(hipStream_t s, const float* g, const float* u, int m, int m_pad, int k,
                                      uint4* afrag, float* ascale, float* asum) {
    const size_t threads = (size_t)(k / 16) * m_pad;
    if (threads == 0) return hipSuccess;
    hipLaunchKernelGGL(vk_swiglu_quantize_g16, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, s, g, u, m,
                       m_pad, k, reinterpret_cast<uint2*>(afrag), ascale, asum);
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

hipError_t launch_gemm_q4k(hipStream_t s, const uint4* afrag, const float* ascale, const float* asum,
                           const VkQ4kLin* lins, int n_lin, int m, int nsb, int m_pad) {
    if (n_lin < 1 || n_lin > 3) return hipErrorInvalidValue;
    VkQ4kSet set{};
    int tiles = 0;
    for (int i = 0; i < n_lin; ++i) {
        set.l[i] = lins[i];
        set.tile0[i] = tiles;
        tiles += (lins[i].n + 15) / 16;
    }
    set.count = n_lin;
    const dim3 grid((unsigned)tiles, (unsigned)((m + 15) / 16));
    hipLaunchKernelGGL(vk_gemm_q4k, grid, dim3(512), 0, s, afrag, ascale, asum, set, m, nsb, m_pad);
    return hipGetLastError();
}

}  // namespace vk

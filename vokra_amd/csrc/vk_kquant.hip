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
constexpr int CS = 2;        // super-blocks per LDS chunk of the matmul
constexpr int CG = CS * NG;  // groups per chunk
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
//   ascale[g * m_pad + row] = s, asum[g * m_pad + row] = (float) gsum.
// Rows m..m_pad-1 are written as zeros.
__global__ void vk_quantize_act_g16(const float* __restrict__ a, int m, int m_pad, int k,
                                    uint2* __restrict__ afrag, float* __restrict__ ascale,
                                    float* __restrict__ asum) {
    const int ng = k / 16, nsb = k / kq::QK;
    const size_t gid = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= (size_t)ng * m_pad) return;
    const int g = (int)(gid / m_pad), row = (int)(gid % m_pad);
    int r[16];
    float s = 0.0f;
    int gsum = 0;
#pragma unroll
    for (int t = 0; t < 16; ++t) r[t] = 0;
    if (row < m) {
        const float4* src = reinterpret_cast<const float4*>(a + (size_t)row * k + 16 * g);
        float v[16];
#pragma unroll
        for (int h = 0; h < 4; ++h) {
            const float4 x = src[h];
            v[4 * h] = x.x;
            v[4 * h + 1] = x.y;
            v[4 * h + 2] = x.z;
            v[4 * h + 3] = x.w;
        }
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
    ascale[(size_t)g * m_pad + row] = s;
    asum[(size_t)g * m_pad + row] = (float)gsum;
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
// Matmul, one workgroup per 16 x 16 output tile (16 activation rows, 16
// weight rows), K in chunks of CS super-blocks.
// Phase 1: wave u takes half-super-block u of the chunk (8 groups): one
//   16x16x16 MFMA per group with accumulator input -128 * gsum (removing the
//   +128 of the bf16 nibble trick) gives isum exactly; isum goes to LDS.
// Phase 2: thread (row, col) runs the reference combine over the chunk's
//   groups in order.
template <bool HAS_BIAS>
__global__ __launch_bounds__(256) void vk_gemm_q4k(
    const uint4* __restrict__ afrag, const float* __restrict__ ascale, const float* __restrict__ asum,
    const uint4* __restrict__ wq4, const float2* __restrict__ wdm, const float* __restrict__ bias,
    float* __restrict__ out, int m, int n, int nsb, int m_pad) {
    using namespace kq;
    __shared__ float lds_p[CG][256];                  // isum, [group][row * 16 + col]
    __shared__ __align__(16) float lds_asg[CG][16];   // gsum, [group][row]   (phase 1)
    __shared__ float4 lds_sa[16][CG / 4];     // s,    [row][group]   (phase 2)
    __shared__ float4 lds_as[16][CG / 4];     // gsum, [row][group]   (phase 2)
    __shared__ float4 lds_dm[16][CG / 4];     // (d_eff, m_eff) x 2 sub-blocks, [col][sub-block pair]

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int nt = blockIdx.x, mt = blockIdx.y;
    const int rq = 4 * (lane >> 4);
    const int row = tid >> 4, col = tid & 15;
    float* sa_f = reinterpret_cast<float*>(lds_sa);
    float* as_f = reinterpret_cast<float*>(lds_as);
    float2* dm_f = reinterpret_cast<float2*>(lds_dm);

    float acc = 0.0f;
    for (int sb0 = 0; sb0 < nsb; sb0 += CS) {
        const int gsb = min(CS, nsb - sb0);   // super-blocks in this chunk
        // ---- phase 1 loads: this wave's half super-block (clamped in bounds)
        const int sbl = min(wave >> 1, gsb - 1), half = wave & 1;
        const int sb = sb0 + sbl;
        const uint4 wv = wq4[(((size_t)nt * nsb + sb) * 64 + lane) * 2 + half];
        uint4 af[4];
#pragma unroll
        for (int p = 0; p < 4; ++p) af[p] = afrag[(((size_t)mt * nsb + sb) * 8 + half * 4 + p) * 64 + lane];
        // ---- cooperative loads of the chunk's scales: 2 per thread
        float sv[2], tv[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int idx = min(tid + 256 * h, gsb * NG * 16 - 1);
            const int gl = idx >> 4, r = idx & 15;
            const size_t o = (size_t)(sb0 * NG + gl) * m_pad + mt * 16 + r;
            sv[h] = ascale[o];
            tv[h] = asum[o];
        }
        const int dmi = min(tid, gsb * 8 * 16 - 1);  // (sub-block, col) of the chunk
        const float2 dmv = wdm[(((size_t)nt * nsb + sb0) * 8 + (dmi >> 4)) * 16 + (dmi & 15)];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int idx = tid + 256 * h;
            if (idx < gsb * NG * 16) {
                const int gl = idx >> 4, r = idx & 15;
                lds_asg[gl][r] = tv[h];
                sa_f[r * CG + gl] = sv[h];
                as_f[r * CG + gl] = tv[h];
            }
        }
        if (tid < gsb * 8 * 16) dm_f[(tid & 15) * CG / 2 + (tid >> 4)] = dmv;
        VK_LDS_BARRIER();
        // ---- phase 1 compute
        if (wave >> 1 < gsb) {
            const uint32_t words[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
            for (int gi = 0; gi < 8; ++gi) {
                const int gl = sbl * NG + half * 8 + gi;  // group within the chunk
                const uint2 ap = (gi & 1) ? make_uint2(af[gi >> 1].z, af[gi >> 1].w)
                                          : make_uint2(af[gi >> 1].x, af[gi >> 1].y);
                const vk_s16x4 b = q4k_operand(words[gi >> 1], 2 * (gi & 1));
                const float4 t4 = *reinterpret_cast<const float4*>(&lds_asg[gl][rq]);
                const vk_f32x4 cin = {-128.0f * t4.x, -128.0f * t4.y, -128.0f * t4.z, -128.0f * t4.w};
                const vk_f32x4 p =
                    __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(vk_s16x4, ap), b, cin, 0, 0, 0);
#pragma unroll
                for (int r = 0; r < 4; ++r) lds_p[gl][(rq + r) * 16 + (lane & 15)] = p[r];
            }
        }
        VK_LDS_BARRIER();
        // ---- phase 2: the reference combine, 4 groups (2 sub-blocks) per step
        for (int q4 = 0; q4 < gsb * NG / 4; ++q4) {
            const float4 s4 = lds_sa[row][q4];
            const float4 a4 = lds_as[row][q4];
            const float4 dm4 = lds_dm[col][q4];  // (d0, m0, d1, m1)
            float p[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) p[u] = lds_p[4 * q4 + u][tid];
            acc += s4.x * (dm4.x * p[0] - dm4.y * a4.x);
            acc += s4.y * (dm4.x * p[1] - dm4.y * a4.y);
            acc += s4.z * (dm4.z * p[2] - dm4.w * a4.z);
            acc += s4.w * (dm4.z * p[3] - dm4.w * a4.w);
        }
        VK_LDS_BARRIER();
    }
    const int orow = mt * 16 + row, ocol = nt * 16 + col;
    if (orow < m && ocol < n) out[(size_t)orow * n + ocol] = HAS_BIAS ? acc + bias[ocol] : acc;
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

hipError_t launch_repack_w_q4k(hipStream_t s, const uint8_t* wq, int n, int n_pad, int nsb, uint4* wq4,
                               float2* wdm) {
    const size_t threads = (size_t)n_pad * nsb;
    if (threads == 0) return hipSuccess;
    hipLaunchKernelGGL(vk_repack_w_q4k, dim3((unsigned)((threads + 127) / 128)), dim3(128), 0, s, wq, n, n_pad, nsb,
                       wq4, wdm);
    return hipGetLastError();
}

hipError_t launch_gemm_q4k(hipStream_t s, const uint4* afrag, const float* ascale, const float* asum,
                           const uint4* wq4, const float2* wdm, const float* bias, float* out, int m, int n, int nsb,
                           int m_pad) {
    const dim3 grid((n + 15) / 16, (m + 15) / 16);
    if (bias)
        hipLaunchKernelGGL(vk_gemm_q4k<true>, grid, dim3(256), 0, s, afrag, ascale, asum, wq4, wdm, bias, out, m, n,
                           nsb, m_pad);
    else
        hipLaunchKernelGGL(vk_gemm_q4k<false>, grid, dim3(256), 0, s, afrag, ascale, asum, wq4, wdm, bias, out, m, n,
                           nsb, m_pad);
    return hipGetLastError();
}

}  // namespace vk

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
constexpr int CS = 4;        // super-blocks per LDS chunk of the matmul (one per wave)
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
// weight rows), K in chunks of CS super-blocks (CG = 64 groups).
// Phase 1: wave w takes super-block w of the chunk (16 groups): one
//   16x16x16 MFMA per group with accumulator input -128 * gsum (removing the
//   +128 of the bf16 nibble trick) gives isum exactly; isum goes to LDS.
//   Right after, the wave issues the global loads of the next chunk into
//   registers, so they are in flight during the combine.
// Phase 2: thread (row, col) runs the reference combine over the chunk's
//   groups in order; waves whose 4 rows are all padding skip it.
namespace kq {
struct Stage {
    uint4 wv[2];     // nibble words of this wave's super-block
    uint4 af[8];     // activation fragments of this wave's super-block
    float sv[4], tv[4];  // chunk scales / group sums (4 per thread)
    float2 dm[2];    // chunk (d_eff, m_eff) (2 per thread)
};
}  // namespace kq

template <bool HAS_BIAS>
__global__ __launch_bounds__(256) void vk_gemm_q4k(
    const uint4* __restrict__ afrag, const float* __restrict__ ascale, const float* __restrict__ asum,
    const uint4* __restrict__ wq4, const float2* __restrict__ wdm, const float* __restrict__ bias, VkEpi epi,
    float* out, int m, int n, int nsb, int m_pad) {
    using namespace kq;
    __shared__ __align__(16) float lds_p[CG][256];    // isum, [group][row * 16 + col]
    // rows padded by one float4 against bank conflicts on the transposing stores
    __shared__ float4 lds_sa[16][CG / 4 + 1];         // s,    [row][group]   (phase 2)
    __shared__ float4 lds_as[16][CG / 4 + 1];         // gsum, [row][group]   (phase 2)
    __shared__ float4 lds_dm[16][CG / 4 + 1];         // (d_eff, m_eff) x 2 sub-blocks, [col][pair]

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int nt = blockIdx.x, mt = blockIdx.y;
    const int rq = 4 * (lane >> 4);
    const int row = tid >> 4, col = tid & 15;
    float* sa_f = reinterpret_cast<float*>(lds_sa);
    float* as_f = reinterpret_cast<float*>(lds_as);
    float2* dm_f = reinterpret_cast<float2*>(lds_dm);
    const bool rows_live = mt * 16 + 4 * wave < m;    // this wave's phase-2 rows

    // Every load index is clamped into the chunk, so no load leaves its buffer.
    auto load = [&](int sb0) -> Stage {
        Stage st;
        const int gsb = min(CS, nsb - sb0);
        const int sb = sb0 + min(wave, gsb - 1);
#pragma unroll
        for (int h = 0; h < 2; ++h) st.wv[h] = wq4[(((size_t)nt * nsb + sb) * 64 + lane) * 2 + h];
#pragma unroll
        for (int p = 0; p < 8; ++p) st.af[p] = afrag[(((size_t)mt * nsb + sb) * 8 + p) * 64 + lane];
#pragma unroll
        for (int h = 0; h < 4; ++h) {
            const int idx = min(tid + 256 * h, gsb * 256 - 1);
            const size_t o = (size_t)(sb0 * NG + (idx >> 4)) * m_pad + mt * 16 + (idx & 15);
            st.sv[h] = ascale[o];
            st.tv[h] = asum[o];
        }
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int idx = min(tid + 256 * h, gsb * 128 - 1);
            st.dm[h] = wdm[(((size_t)nt * nsb + sb0) * 8 + (idx >> 4)) * 16 + (idx & 15)];
        }
        return st;
    };

    float acc = 0.0f;
    Stage st = load(0);
    for (int sb0 = 0; sb0 < nsb; sb0 += CS) {
        const int gsb = min(CS, nsb - sb0);   // super-blocks in this chunk
#pragma unroll
        for (int h = 0; h < 4; ++h) {
            const int idx = tid + 256 * h;
            if (idx < gsb * 256) {
                const int gl = idx >> 4, r = idx & 15;
                sa_f[r * (CG + 4) + gl] = st.sv[h];
                as_f[r * (CG + 4) + gl] = st.tv[h];
            }
        }
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int idx = tid + 256 * h;
            if (idx < gsb * 128) dm_f[(idx & 15) * (CG / 2 + 2) + (idx >> 4)] = st.dm[h];
        }
        VK_LDS_BARRIER();
        // ---- phase 1: this wave's super-block
        // (8 groups at a time: all LDS reads, then all MFMAs, then all writes,
        // so the latencies overlap instead of adding up per group)
        if (wave < gsb) {
#pragma unroll
            for (int half = 0; half < 2; ++half) {
                const uint32_t words[4] = {st.wv[half].x, st.wv[half].y, st.wv[half].z, st.wv[half].w};
                const int g0 = wave * NG + half * 8;
                float t[8];
#pragma unroll
                for (int gi = 0; gi < 8; ++gi) t[gi] = as_f[(lane & 15) * (CG + 4) + g0 + gi];
                vk_f32x4 p[8];
#pragma unroll
                for (int gi = 0; gi < 8; ++gi) {
                    const uint4 a4 = st.af[half * 4 + (gi >> 1)];
                    const uint2 ap = (gi & 1) ? make_uint2(a4.z, a4.w) : make_uint2(a4.x, a4.y);
                    const vk_s16x4 w = q4k_operand(words[gi >> 1], 2 * (gi & 1));
                    const float c = -128.0f * t[gi];
                    const vk_f32x4 cin = {c, c, c, c};
                    // transposed product: weights as the A operand, so lane l
                    // gets activation row l % 16, columns rq..rq+3
                    p[gi] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(w, __builtin_bit_cast(vk_s16x4, ap), cin, 0, 0,
                                                                      0);
                }
#pragma unroll
                for (int gi = 0; gi < 8; ++gi)
                    *reinterpret_cast<float4*>(&lds_p[g0 + gi][(lane & 15) * 16 + rq]) =
                        make_float4(p[gi][0], p[gi][1], p[gi][2], p[gi][3]);
            }
        }
        // ---- next chunk's loads (the last chunk reloads itself, unused)
        st = load(sb0 + CS < nsb ? sb0 + CS : sb0);
        VK_LDS_BARRIER();
        // ---- phase 2: the reference combine, 4 groups (2 sub-blocks) per step
        // (one super-block per step: its 28 LDS reads issue together)
        if (rows_live) {
            for (int sbl = 0; sbl < gsb; ++sbl) {
                float4 s4[4], a4[4], dm4[4];  // dm4 = (d0, m0, d1, m1)
                float p[16];
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    s4[u] = lds_sa[row][4 * sbl + u];
                    a4[u] = lds_as[row][4 * sbl + u];
                    dm4[u] = lds_dm[col][4 * sbl + u];
                }
#pragma unroll
                for (int u = 0; u < 16; ++u) p[u] = lds_p[NG * sbl + u][tid];
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    acc += s4[u].x * (dm4[u].x * p[4 * u] - dm4[u].y * a4[u].x);
                    acc += s4[u].y * (dm4[u].x * p[4 * u + 1] - dm4[u].y * a4[u].y);
                    acc += s4[u].z * (dm4[u].z * p[4 * u + 2] - dm4[u].w * a4[u].z);
                    acc += s4[u].w * (dm4[u].z * p[4 * u + 3] - dm4[u].w * a4[u].w);
                }
            }
        }
        VK_LDS_BARRIER();
    }
    const int orow = mt * 16 + row, ocol = nt * 16 + col;
    if (orow < m && ocol < n) {
        const size_t o = (size_t)orow * n + ocol;
        out[o] = vk_epi_apply(HAS_BIAS ? acc + bias[ocol] : acc, epi, o);
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
                           int m_pad, VkEpi epi) {
    const dim3 grid((n + 15) / 16, (m + 15) / 16);
    if (bias)
        hipLaunchKernelGGL(vk_gemm_q4k<true>, grid, dim3(256), 0, s, afrag, ascale, asum, wq4, wdm, bias, epi, out, m,
                           n, nsb, m_pad);
    else
        hipLaunchKernelGGL(vk_gemm_q4k<false>, grid, dim3(256), 0, s, afrag, ascale, asum, wq4, wdm, bias, epi, out, m,
                           n, nsb, m_pad);
    return hipGetLastError();
}

}  // namespace vk

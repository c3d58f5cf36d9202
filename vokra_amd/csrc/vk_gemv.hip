// vk_gemv.hip — decode-shaped (M <= 64) block GEMM for gfx950.
//
// Same numerics as vk_gemm_qblock (INT8 activations, exact per-block integer
// dots, combine acc = fmaf(sa * dw, P_b, acc) in block order), so the two
// kernels are bit-identical and the dispatcher picks by shape. Here the
// weights stream from HBM once in a compact device layout:
//
//  * Q4_0: per (16-row tile nt, group g of 4 blocks) one 1 KiB fragment, lane
//    l (row l%16, column chunk c = l/16) holding one 32-bit "nibble word" per
//    block: element 8c+2j at bits 4j..4j+3 and 8c+2j+1 at bits 16+4j..19+4j,
//    so ((X >> 4j) & 0x000F000F) | 0x43004300 is the bf16 pair (128 + nib).
//  * Q8_0: two 1 KiB fragments per (nt, g), lane l holding 8 bytes q + 128 per
//    block; v_cvt_f32_ubyte turns each into the exact bf16 of q + 128.
//  * scales: f16 per (row, block) at [nt][g][16][4] (one 8-byte load per lane).
//
// The weight offsets (+128 on every element, and the Q4_0 nibble bias 8) are
// removed through the MFMA accumulator input: C = -(128 + 8) * sum(A) for
// Q4_0 and -128 * sum(A) for Q8_0, itself an MFMA of the activations with a
// constant -136 / -128 operand (no per-row sums are read and no VALU forms
// it). Every product and partial sum is an integer (times a power of two for
// POW2 activations) below 2^24, so C and D = P_b are exact.
#include "vk_common.h"

#include <algorithm>

#include "vk_launch.h"

namespace vk {

namespace gemv {
constexpr int WAVES = 4;        // waves per workgroup, one 16-column tile each
constexpr int GB = 4;           // quant blocks per pipeline group
constexpr int FRAG_U4 = 64;
}  // namespace gemv

// ---------------------------------------------------------------------------
// Weight repack for the decode layout (upload time). One thread per (row,
// group of 4 blocks, column chunk c): reads the row's wire blocks directly.
__global__ void vk_repack_w_gemv(int mode, const uint8_t* __restrict__ wq, int n, int n_pad, int nb,
                                 uint4* __restrict__ wq4, uint2* __restrict__ wsc) {
    const int G = nb / gemv::GB;
    const size_t gid = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t total = (size_t)n_pad * G * 4;
    if (gid >= total) return;
    const int c = (int)(gid & 3);
    const size_t rg = gid >> 2;
    const int row = (int)(rg / G), g = (int)(rg % G);
    const int nt = row >> 4, lane = (row & 15) + 16 * c;
    const int bb = mode == 3 ? 34 : 18;
    uint32_t w[4] = {0, 0, 0, 0}, w2[4] = {0, 0, 0, 0};
    uint16_t sc[4] = {0, 0, 0, 0};
    for (int u = 0; u < gemv::GB; ++u) {
        if (row >= n) break;
        const uint8_t* p = wq + ((size_t)row * nb + g * gemv::GB + u) * bb;
        sc[u] = (uint16_t)(p[0] | (p[1] << 8));
        if (mode == 1) {
            // elements 8c .. 8c+7 are bytes 4c .. 4c+3 (lo nibble = even element)
            uint32_t x = 0;
            for (int j = 0; j < 4; ++j) {
                const uint32_t b = p[2 + 4 * c + j];
                x |= (b & 0x0fu) << (4 * j);
                x |= (b >> 4) << (16 + 4 * j);
            }
            w[u] = x;
        } else {
            uint32_t lo = 0, hi = 0;
            for (int j = 0; j < 4; ++j) {
                lo |= (uint32_t)((uint8_t)(p[2 + 8 * c + j] + 128u)) << (8 * j);
                hi |= (uint32_t)((uint8_t)(p[2 + 8 * c + 4 + j] + 128u)) << (8 * j);
            }
            if (u < 2) { w[2 * u] = lo; w[2 * u + 1] = hi; }
            else { w2[2 * (u - 2)] = lo; w2[2 * (u - 2) + 1] = hi; }
        }
    }
    const size_t fg = (size_t)nt * G + g;
    if (mode == 1) {
        wq4[fg * gemv::FRAG_U4 + lane] = make_uint4(w[0], w[1], w[2], w[3]);
    } else {
        wq4[(fg * 2) * gemv::FRAG_U4 + lane] = make_uint4(w[0], w[1], w[2], w[3]);
        wq4[(fg * 2 + 1) * gemv::FRAG_U4 + lane] = make_uint4(w2[0], w2[1], w2[2], w2[3]);
    }
    if (c == 0)
        wsc[fg * 16 + (row & 15)] = make_uint2((uint32_t)sc[0] | ((uint32_t)sc[1] << 16),
                                               (uint32_t)sc[2] | ((uint32_t)sc[3] << 16));
}

// bf16 operand (8 values) of one Q4_0 block from its nibble word.
__device__ __forceinline__ vk_bf16x8 q4_word_to_bf16(uint32_t x) {
    uint4 r;
    r.x = (x & 0x000F000Fu) | 0x43004300u;
    r.y = ((x >> 4) & 0x000F000Fu) | 0x43004300u;
    r.z = ((x >> 8) & 0x000F000Fu) | 0x43004300u;
    r.w = ((x >> 12) & 0x000F000Fu) | 0x43004300u;
    return __builtin_bit_cast(vk_bf16x8, r);
}

// bf16 operand of one Q8_0 block from 8 offset bytes (u = q + 128, exact).
__device__ __forceinline__ uint32_t u8pair_to_bf16(uint32_t x, int k) {
    // bytes k, k+1 of x -> two bf16 (high halves of the exact f32 values)
    const float a = (float)((x >> (8 * k)) & 0xffu), b = (float)((x >> (8 * (k + 1))) & 0xffu);
    return (__float_as_uint(a) >> 16) | (__float_as_uint(b) & 0xffff0000u);
}
__device__ __forceinline__ vk_bf16x8 q8_bytes_to_bf16(uint32_t lo, uint32_t hi) {
    uint4 r;
    r.x = u8pair_to_bf16(lo, 0);
    r.y = u8pair_to_bf16(lo, 2);
    r.z = u8pair_to_bf16(hi, 0);
    r.w = u8pair_to_bf16(hi, 2);
    return __builtin_bit_cast(vk_bf16x8, r);
}

// ---------------------------------------------------------------------------
// Decode kernel. One workgroup = one 16 x 16 output tile (16 activation rows,
// 16 weight rows). Phase 1: the 4 waves split the K blocks by 4-block group
// (group g -> wave g % 4), prefetch all their weight words and activation
// fragments for the chunk up front, and compute the exact block dots P_b
// (one MFMA per block) into LDS together with the block scales. Phase 2: one
// thread per output walks the chunk's blocks in order with the same
// fmaf(sa * dw, P_b, acc) as the tiled GEMM, so the result is bit-identical.
// K is processed in chunks of CB blocks so P fits LDS.
namespace gemv {
constexpr int CB = 48;                 // blocks per chunk (12 groups)
constexpr int GPW = CB / GB / WAVES;   // groups per wave per chunk (3)
}  // namespace gemv

// Up to three linears over the same activations in one launch (grid z picks
// the linear; q, k and v of an attention block share their input).
struct GemvSet {
    VkGemvLin lin[3];
};

// DEV: the linears come from a device array (any count, one per grid z) rather
// than the kernel arguments.
template <int MODE, bool POW2, bool DEV>
__global__ __launch_bounds__(256) void vk_gemv_qblock(
    const uint4* __restrict__ afrag, const float* __restrict__ ascale, const float* __restrict__ asum,
    const GemvSet set, const VkGemvLin* __restrict__ dlins, int m, int nb, int m_pad) {
    using namespace gemv;
    const VkGemvLin lin = DEV ? dlins[blockIdx.z] : set.lin[blockIdx.z];
    (void)asum;  // the operand sums come from the matrix core (OFFW below)
    const uint4* __restrict__ wq4 = lin.wq4;
    const uint2* __restrict__ wsc = lin.wsc;
    const int n = lin.n;
    if ((int)blockIdx.x * 16 >= n) return;  // this linear has fewer column tiles (whole workgroup)
    constexpr int WQ = MODE == 1 ? 1 : 2;  // weight uint4 per lane per group
    // the weight offsets (-136 for Q4_0: the +128 of the bf16 trick and the
    // nibble bias 8; -128 for Q8_0) as a bf16 pair: the MFMA of the
    // activations with it is the accumulator input OFFSET * sum(A), exact
    constexpr uint32_t OFFW = MODE == 1 ? 0xC308C308u : 0xC300C300u;
    __shared__ float lds_p[CB][256];       // exact block dots, [block][row*16 + col]
    __shared__ float lds_sa[CB][16];       // activation scales, [block][row]
    __shared__ float lds_dw[CB][16];       // weight scales, [block][col]

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int nt = blockIdx.x, mt = blockIdx.y;
    const int G = nb / GB;
    const int rq = 4 * (lane >> 4);        // first of this lane's 4 D rows

    float acc = 0.0f;                      // phase 2: output (row tid/16, col tid%16)
    // Operands of one chunk (everything for this wave's groups, plus the
    // chunk's activation scales and operand sums, 3 of each per thread). The
    // next chunk's are loaded into the same registers once phase 1 has used
    // them, so they are in flight during phase 2.
    uint4 wq[GPW][WQ];
    uint2 ws[GPW];
    uint4 af[GPW][GB];
    float sv[CB * 16 / 256];
    auto load_chunk = [&](int g0) {
        const int gn = min(CB / GB, G - g0);
#pragma unroll
        for (int j = 0; j < GPW; ++j) {
            const int gl = min(wave + WAVES * j, gn - 1);  // clamped: loads stay in bounds
            const int g = g0 + gl;
            const size_t fg = (size_t)nt * G + g;
#pragma unroll
            for (int h = 0; h < WQ; ++h) wq[j][h] = wq4[(fg * WQ + h) * FRAG_U4 + lane];
            ws[j] = wsc[fg * 16 + (lane & 15)];
#pragma unroll
            for (int u = 0; u < GB; ++u) af[j][u] = afrag[((size_t)mt * nb + g * GB + u) * FRAG_U4 + lane];
        }
#pragma unroll
        for (int h = 0; h < CB * 16 / 256; ++h) {
            const int idx = min(tid + 256 * h, gn * GB * 16 - 1);
            const int bl = idx >> 4, r = idx & 15;
            const size_t o = (size_t)(g0 * GB + bl) * m_pad + mt * 16 + r;
            sv[h] = ascale[o];
        }
    };
    load_chunk(0);
    for (int g0 = 0; g0 < G; g0 += CB / GB) {
        const int gn = min(CB / GB, G - g0);  // groups in this chunk
#pragma unroll
        for (int h = 0; h < CB * 16 / 256; ++h) {
            const int idx = tid + 256 * h;
            if (idx < gn * GB * 16) lds_sa[idx >> 4][idx & 15] = sv[h];
        }
        VK_LDS_BARRIER();
        // ---- phase 1 compute: exact P_b for this wave's groups
#pragma unroll
        for (int j = 0; j < GPW; ++j) {
            const int gl = wave + WAVES * j;
            if (gl >= gn) break;
            const uint32_t sc_bits[4] = {ws[j].x & 0xffffu, ws[j].x >> 16, ws[j].y & 0xffffu, ws[j].y >> 16};
#pragma unroll
            for (int u = 0; u < GB; ++u) {
                vk_bf16x8 bf;
                if (MODE == 1) {
                    const uint4 q = wq[j][0];
                    const uint32_t x = u == 0 ? q.x : (u == 1 ? q.y : (u == 2 ? q.z : q.w));
                    bf = q4_word_to_bf16(x);
                } else {
                    const uint4 q = wq[j][u >> 1];
                    bf = (u & 1) ? q8_bytes_to_bf16(q.z, q.w) : q8_bytes_to_bf16(q.x, q.y);
                }
                const int bl = gl * GB + u;  // block index within the chunk
                const vk_bf16x8 a8 = __builtin_bit_cast(vk_bf16x8, af[j][u]);
                const vk_f32x4 cin = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                    a8, __builtin_bit_cast(vk_bf16x8, make_uint4(OFFW, OFFW, OFFW, OFFW)),
                    (vk_f32x4){0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
                const vk_f32x4 p = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a8, bf, cin, 0, 0, 0);
#pragma unroll
                for (int r = 0; r < 4; ++r) lds_p[bl][(rq + r) * 16 + (lane & 15)] = p[r];
                if (lane < 16) lds_dw[bl][lane] = vk_f16_to_f32_hw(sc_bits[u]);
            }
        }
        VK_LDS_BARRIER();
        if (g0 + CB / GB < G) load_chunk(g0 + CB / GB);  // uniform
        // ---- phase 2: ordered combine, one thread per output
        const int row = tid >> 4, col = tid & 15;
        // gn*GB is a multiple of 4: the reads of 4 blocks are issued together
        // ahead of the dependent fmaf chain
        for (int bl = 0; bl < gn * GB; bl += 4) {
            float p[4], sd[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                p[u] = lds_p[bl + u][tid];
                sd[u] = POW2 ? lds_dw[bl + u][col] : lds_sa[bl + u][row] * lds_dw[bl + u][col];
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) acc = fmaf(sd[u], p[u], acc);
        }
        VK_LDS_BARRIER();
    }
    const int row = mt * 16 + (tid >> 4), col = nt * 16 + (tid & 15);
    if (row < m && col < n) {
        const size_t o = (size_t)row * n + col;
        lin.out[o] = vk_epi_apply(lin.bias ? acc + lin.bias[col] : acc, lin.epi, o);
    }
}

// ---------------------------------------------------------------------------
// Wave-per-tile decode kernel: one wave (its own workgroup) owns a 16 x 16
// output tile and walks the K blocks in order: the exact block dot P_b of the
// MFMA (accumulator input OFFSET * operand sum, as above) is folded right away,
// acc = fmaf(s_a * d_w, P_b, acc), for the lane's 4 outputs. No LDS exchange of
// block dots and no barriers; the operands of each 4-block group (A fragments,
// weight words, weight scales, activation scales and sums) stream global -> LDS
// through a private ring of RING groups with direct loads. Same products, same
// order: bit-identical to the two-phase kernel.
namespace gw {
#ifndef VK_GW_RING
#define VK_GW_RING 3
#endif
constexpr int RING = VK_GW_RING;        // groups in flight per wave (<= 8: the wait counts stay < 64)
constexpr int SLOT = 7 * 1024;          // bytes per ring slot: A 4 KiB, W <= 2 KiB, scales 768 B
constexpr int OFF_W = 4096, OFF_WS = 6144, OFF_SA = 6400;
}  // namespace gw

// One wave's 16 x 16 output tile (weight column tile nt, activation row tile
// mt) of the wave-per-tile kernel: acc[r] is output (16 mt + 4 (lane / 16) + r,
// 16 nt + lane % 16). ring: this wave's RING slots of LDS.
template <int MODE, bool POW2>
__device__ __forceinline__ void gemv_w_tile(const uint4* __restrict__ afrag, const float* __restrict__ ascale,
                                            const float* __restrict__ asum, const VkGemvLin& lin, int nt, int mt,
                                            int nb, int m_pad, uint8_t (&ring)[gw::RING][gw::SLOT], float (&acc)[4]) {
    using namespace gw;
    constexpr int WQ = MODE == 1 ? 1 : 2;           // weight KiB per group
    constexpr int LG = 4 + WQ + 2;                  // direct loads per lane per group
    // the weight offsets as a bf16 pair (see vk_gemv_qblock): the accumulator
    // input OFFSET * sum(A) is an MFMA of the activations with it
    constexpr uint32_t OFFW = MODE == 1 ? 0xC308C308u : 0xC300C300u;
    (void)asum;
    const int lane = threadIdx.x & 63, col = lane & 15;
    const int G = nb / gemv::GB;
    const uint32_t base = __builtin_amdgcn_readfirstlane(vk_lds_addr(&ring[0][0]));
    // per-lane sources (advanced by group)
    const uint4* a_src = afrag + (size_t)mt * nb * gemv::FRAG_U4 + lane;
    const uint4* w_src = lin.wq4 + (size_t)nt * G * WQ * gemv::FRAG_U4 + lane;
    const uint32_t* ws_src = reinterpret_cast<const uint32_t*>(lin.wsc + (size_t)nt * G * 16) + (lane & 31);
    const size_t s_off = (size_t)(lane >> 4) * m_pad + mt * 16 + (lane & 15);
    auto issue = [&](int g, int slot) {
        const uint32_t b = base + slot * SLOT;
#pragma unroll
        for (int u = 0; u < 4; ++u) vk_dma_b128(a_src + (size_t)(4 * g + u) * gemv::FRAG_U4, b + u * 1024);
#pragma unroll
        for (int h = 0; h < WQ; ++h) vk_dma_b128(w_src + (size_t)(g * WQ + h) * gemv::FRAG_U4, b + OFF_W + h * 1024);
        vk_dma_b32(ws_src + (size_t)g * 32, b + OFF_WS);
        vk_dma_b32(ascale + (size_t)4 * g * m_pad + s_off, b + OFF_SA);
    };
    acc[0] = acc[1] = acc[2] = acc[3] = 0.0f;
#pragma unroll
    for (int p = 0; p < RING - 1; ++p)
        if (p < G) issue(p, p);
    static_assert(RING >= 3 && RING <= 8 && (RING - 1) * LG < 64, "ring depth");
    int slot = 0;
#pragma unroll 1
    for (int g = 0; g < G; ++g) {
        // group g's loads are the oldest in flight: wait for exactly those
        const int ahead = G - 1 - g;
        if (ahead >= RING - 1) {
            issue(g + RING - 1, slot == 0 ? RING - 1 : slot - 1);
            vk_wait_vm<(RING - 1) * LG>();
        } else if (RING > 7 && ahead == 6) {
            vk_wait_vm<6 * LG>();
        } else if (RING > 6 && ahead == 5) {
            vk_wait_vm<5 * LG>();
        } else if (RING > 5 && ahead == 4) {
            vk_wait_vm<4 * LG>();
        } else if (RING > 4 && ahead == 3) {
            vk_wait_vm<3 * LG>();
        } else if (ahead == 2) {
            vk_wait_vm<2 * LG>();
        } else if (ahead == 1) {
            vk_wait_vm<LG>();
        } else {
            vk_wait_vm<0>();
        }
        const uint8_t* sl = &ring[slot][0];
        uint4 af[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) af[u] = reinterpret_cast<const uint4*>(sl + u * 1024)[lane];
        uint4 wq[WQ];
#pragma unroll
        for (int h = 0; h < WQ; ++h) wq[h] = reinterpret_cast<const uint4*>(sl + OFF_W + h * 1024)[lane];
        const uint2 ws = reinterpret_cast<const uint2*>(sl + OFF_WS)[col];
        float4 sa[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) sa[u] = reinterpret_cast<const float4*>(sl + OFF_SA)[u * 4 + (lane >> 4)];
        const uint32_t sc_bits[4] = {ws.x & 0xffffu, ws.x >> 16, ws.y & 0xffffu, ws.y >> 16};
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            vk_bf16x8 bf;
            if (MODE == 1) {
                const uint4 q = wq[0];
                const uint32_t x = u == 0 ? q.x : (u == 1 ? q.y : (u == 2 ? q.z : q.w));
                bf = q4_word_to_bf16(x);
            } else {
                const uint4 q = wq[u >> 1];
                bf = (u & 1) ? q8_bytes_to_bf16(q.z, q.w) : q8_bytes_to_bf16(q.x, q.y);
            }
            const vk_bf16x8 a8 = __builtin_bit_cast(vk_bf16x8, af[u]);
            const vk_f32x4 cin = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                a8, __builtin_bit_cast(vk_bf16x8, make_uint4(OFFW, OFFW, OFFW, OFFW)),
                (vk_f32x4){0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
            const vk_f32x4 p = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a8, bf, cin, 0, 0, 0);
            const float dw = vk_f16_to_f32_hw(sc_bits[u]);
            const float sar[4] = {sa[u].x, sa[u].y, sa[u].z, sa[u].w};
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[r] = fmaf(POW2 ? dw : sar[r] * dw, p[r], acc[r]);
        }
        slot = slot == RING - 1 ? 0 : slot + 1;
    }
}

template <int MODE, bool POW2, bool DEV>
__global__ __launch_bounds__(64) void vk_gemv_qblock_w(
    const uint4* __restrict__ afrag, const float* __restrict__ ascale, const float* __restrict__ asum,
    const GemvSet set, const VkGemvLin* __restrict__ dlins, int m, int nb, int m_pad) {
    __shared__ __align__(16) uint8_t ring[gw::RING][gw::SLOT];
    const VkGemvLin lin = DEV ? dlins[blockIdx.z] : set.lin[blockIdx.z];
    const int nt = blockIdx.x, mt = blockIdx.y;
    if (nt * 16 >= lin.n) return;  // this linear has fewer column tiles (the whole wave)
    const int lane = threadIdx.x, rq = 4 * (lane >> 4), col = lane & 15;
    float acc[4];
    gemv_w_tile<MODE, POW2>(afrag, ascale, asum, lin, nt, mt, nb, m_pad, ring, acc);
    const int c = nt * 16 + col;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int row = mt * 16 + rq + r;
        if (row < m && c < lin.n) {
            const size_t o = (size_t)row * lin.n + c;
            lin.out[o] = vk_epi_apply(lin.bias ? acc[r] + lin.bias[c] : acc[r], lin.epi, o);
        }
    }
}


// The wave-per-tile kernel for one linear whose outputs go straight into the
// activation pass of the next linear's input (qo; its f32 outputs are not
// written): a workgroup of two waves takes the two 16-column tiles of one
// 32-column block, so the block's absolute maximum and operand sum combine
// across the waves through LDS. Outputs, scales and sums equal the GEMV
// followed by vk_quantize_act_b32 (rows past m get zero fragments).
template <int MODE, bool POW2>
__global__ __launch_bounds__(128) void vk_gemv_qblock_wq(
    const uint4* __restrict__ afrag, const float* __restrict__ ascale, const float* __restrict__ asum,
    const VkGemvLin lin, int m, int nb, int m_pad, const VkQOut qo) {
    __shared__ __align__(16) uint8_t ring[2][gw::RING][gw::SLOT];
    __shared__ float xamax[2][16];
    __shared__ int xsum[2][16];
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63, rq = 4 * (lane >> 4), col = lane & 15;
    const int kb = blockIdx.x, nt = 2 * kb + w, mt = blockIdx.y;  // n % 32 == 0: both tiles exist
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (mt * 16 < m)  // row tiles past m only write zero fragments (uniform per workgroup)
        gemv_w_tile<MODE, POW2>(afrag, ascale, asum, lin, nt, mt, nb, m_pad, ring[w], acc);
    const int c = nt * 16 + col;
    float v[4], amax[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int row = mt * 16 + rq + r;
        const size_t o = (size_t)row * lin.n + c;
        v[r] = row < m ? vk_epi_apply(lin.bias ? acc[r] + lin.bias[c] : acc[r], lin.epi, o) : 0.0f;
        // from 0 and through fmaxf, as the separate pass (NaN ignored)
        amax[r] = vk_group_max<16>(fmaxf(0.0f, fabsf(v[r])));
    }
    if (col == 0)
#pragma unroll
        for (int r = 0; r < 4; ++r) xamax[w][rq + r] = amax[r];
    __syncthreads();
    float sc[4];
    int q[4], gs[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const float a = fmaxf(amax[r], xamax[w ^ 1][rq + r]);
        sc[r] = 0.0f;
        q[r] = 0;
        if (a != 0.0f) {
            sc[r] = vk_act_scale(a, qo.pow2);
            q[r] = vk_act_q(v[r], sc[r]);
        }
        gs[r] = vk_group_sum_i<16>(q[r]);
    }
    if (col == 0)
#pragma unroll
        for (int r = 0; r < 4; ++r) xsum[w][rq + r] = gs[r];
    __syncthreads();
    const int nbo = qo.k >> 5;
    uint16_t* f16 = reinterpret_cast<uint16_t*>(qo.afrag);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int row = mt * 16 + rq + r;  // < qo.m_pad
        f16[vk_afrag_u16((size_t)row, kb, nbo, 16 * w + col)] = (uint16_t)vk_act_bits(q[r], sc[r], qo.pow2);
        if (w == 0 && col == 0) {
            const int g = gs[r] + xsum[1][rq + r];  // the block's columns in order: wave 0's, then wave 1's
            qo.ascale[(size_t)kb * qo.m_pad + row] = sc[r];
            qo.asum[(size_t)kb * qo.m_pad + row] = qo.pow2 ? (float)g * sc[r] : (float)g;
        }
    }
}

}  // namespace vk

namespace vk {

hipError_t launch_repack_w_gemv(hipStream_t s, int mode, const uint8_t* wq, int n, int n_pad, int nb, uint4* wq4,
                                uint2* wsc) {
    const size_t threads = (size_t)n_pad * (nb / gemv::GB) * 4;
    if (threads == 0) return hipSuccess;
    const unsigned grid = (unsigned)((threads + 255) / 256);
    hipLaunchKernelGGL(vk_repack_w_gemv, dim3(grid), dim3(256), 0, s, mode, wq, n, n_pad, nb, wq4, wsc);
    return hipGetLastError();
}

// Which decode kernel: the wave-per-tile one streams weights faster once the
// grid is large (>= 512 tiles, or a grouped launch), the two-phase one has the
// shorter latency for a small grid (one memory round trip per workgroup).
// Measured at M=64: 320 tiles 6.5 us two-phase vs 7.3 wave-per-tile; the
// decoder step (q/k/v: 960 tiles) 10.46 -> 10.39 ms with 512 rather than 1024.
constexpr int kWptMinTiles = 512;

template <int MODE, bool POW2, bool DEV>
static hipError_t go(hipStream_t s, const uint4* afrag, const float* ascale, const float* asum, const GemvSet& set,
                     const VkGemvLin* dlins, int n_lin, int n_max, int m, int nb, int m_pad) {
    const int n_tiles = (n_max + 15) / 16, m_tiles = (m + 15) / 16;
    // linears from a device array always run the wave-per-tile kernel
    if constexpr (!DEV) {
        if ((size_t)n_tiles * m_tiles * n_lin < (size_t)kWptMinTiles) {
            hipLaunchKernelGGL((vk_gemv_qblock<MODE, POW2, false>), dim3(n_tiles, m_tiles, n_lin), dim3(256), 0, s,
                               afrag, ascale, asum, set, dlins, m, nb, m_pad);
            return hipGetLastError();
        }
    }
    hipLaunchKernelGGL((vk_gemv_qblock_w<MODE, POW2, DEV>), dim3(n_tiles, m_tiles, n_lin), dim3(64), 0, s, afrag,
                       ascale, asum, set, dlins, m, nb, m_pad);
    return hipGetLastError();
}

hipError_t launch_gemv_qblock(hipStream_t s, int mode, bool pow2, const uint4* afrag, const float* ascale,
                              const float* asum, const VkGemvLin* lins, int n_lin, int m, int nb, int m_pad) {
    if (n_lin < 1 || n_lin > 3 || m < 1) return hipErrorInvalidValue;
    GemvSet set = {};
    int n_max = 0;
    for (int i = 0; i < n_lin; ++i) {
        set.lin[i] = lins[i];
        n_max = std::max(n_max, lins[i].n);
    }
    if (n_max < 1) return hipSuccess;
    if (mode == 1)
        return pow2 ? go<1, true, false>(s, afrag, ascale, asum, set, nullptr, n_lin, n_max, m, nb, m_pad)
                    : go<1, false, false>(s, afrag, ascale, asum, set, nullptr, n_lin, n_max, m, nb, m_pad);
    return pow2 ? go<3, true, false>(s, afrag, ascale, asum, set, nullptr, n_lin, n_max, m, nb, m_pad)
                : go<3, false, false>(s, afrag, ascale, asum, set, nullptr, n_lin, n_max, m, nb, m_pad);
}

hipError_t launch_gemv_qblock_quant(hipStream_t s, int mode, bool pow2, const uint4* afrag, const float* ascale,
                                    const float* asum, const VkGemvLin& lin, int m, int nb, int m_pad,
                                    const VkQOut& qo) {
    // every padded row of the fragments is written (zero past m), as the
    // separate pass does; the row tiles read stay inside the input's padding
    if (m < 1 || lin.n < 32 || lin.n % 32 != 0 || qo.k != lin.n || !qo.afrag || qo.m_pad < m || qo.m_pad % 16 != 0 ||
        qo.m_pad > m_pad)
        return hipErrorInvalidValue;
    const dim3 grid((unsigned)(lin.n / 32), (unsigned)(qo.m_pad / 16)), block(128);
    if (mode == 1) {
        if (pow2) hipLaunchKernelGGL((vk_gemv_qblock_wq<1, true>), grid, block, 0, s, afrag, ascale, asum, lin, m, nb, m_pad, qo);
        else hipLaunchKernelGGL((vk_gemv_qblock_wq<1, false>), grid, block, 0, s, afrag, ascale, asum, lin, m, nb, m_pad, qo);
    } else {
        if (pow2) hipLaunchKernelGGL((vk_gemv_qblock_wq<3, true>), grid, block, 0, s, afrag, ascale, asum, lin, m, nb, m_pad, qo);
        else hipLaunchKernelGGL((vk_gemv_qblock_wq<3, false>), grid, block, 0, s, afrag, ascale, asum, lin, m, nb, m_pad, qo);
    }
    return hipGetLastError();
}

hipError_t launch_gemv_qblock_group(hipStream_t s, int mode, bool pow2, const uint4* afrag, const float* ascale,
                                    const float* asum, const VkGemvLin* d_lins, int n_lin, int n_max, int m, int nb,
                                    int m_pad) {
    if (n_lin < 1 || n_lin > 65535 || m < 1 || !d_lins) return hipErrorInvalidValue;
    if (n_max < 1) return hipSuccess;
    const GemvSet none = {};
    if (mode == 1)
        return pow2 ? go<1, true, true>(s, afrag, ascale, asum, none, d_lins, n_lin, n_max, m, nb, m_pad)
                    : go<1, false, true>(s, afrag, ascale, asum, none, d_lins, n_lin, n_max, m, nb, m_pad);
    return pow2 ? go<3, true, true>(s, afrag, ascale, asum, none, d_lins, n_lin, n_max, m, nb, m_pad)
                : go<3, false, true>(s, afrag, ascale, asum, none, d_lins, n_lin, n_max, m, nb, m_pad);
}

}  // namespace vk

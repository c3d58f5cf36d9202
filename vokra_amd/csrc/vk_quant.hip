// vk_quant.hip — block-quant kernels for gfx950 (CDNA4).
//
//  * vk_dequantize_q0        : wire Q4_0/Q5_0/Q8_0 blocks -> f32 (bit-exact,
//                              crates/vokra-core/src/kv_quant/mod.rs:307-359)
//  * vk_dequant_gemv_f32     : KvQuantDequantGemvOps (f32 semantics,
//                              crates/vokra-core/src/kv_quant/dequant_gemm.rs:49-98)
//  * vk_quantize_act_b32     : per-32-block INT8 activation quantization into
//                              the MFMA A-fragment layout
//  * vk_repack_w_b32         : wire weight blocks -> exact bf16 integers in the
//                              MFMA B-fragment layout + f32 block scales
//  * vk_gemm_qblock          : INT8-semantics block GEMM on bf16 MFMA
//
// Fragment layout ("frag16"): a 16-row x 32-column (one quant block) tile is
// stored as 64 lanes x 8 bf16, lane l holding row (l % 16), columns
// 8*(l/16) .. 8*(l/16)+7. That is exactly the per-lane operand of
// v_mfma_f32_16x16x32_bf16, so a wave loads a fragment with one coalesced
// 16-byte-per-lane read. Tiles are ordered [row_tile][block][lane][8].
#include "vk_common.h"

namespace vk {

// Block wire sizes of the KvQuant formats (kv_quant/mod.rs:101-110).
__host__ __device__ constexpr int q0_block_bytes(int mode) {
    return mode == 1 ? 18 : (mode == 2 ? 22 : (mode == 3 ? 34 : 0));
}

// Integer value of element i of a wire block (Q4_0 nib-8, Q5_0 v-16, Q8_0 q):
// q4_0.rs:73-87, q5_0.rs unpack, q8_0.rs:69-80.
__device__ __forceinline__ int q0_int(int mode, const uint8_t* blk, int i) {
    if (mode == 3) return (int)(int8_t)blk[2 + i];
    if (mode == 1) {
        const uint8_t b = blk[2 + (i >> 1)];
        return (int)((i & 1) ? (b >> 4) : (b & 0x0f)) - 8;
    }
    const uint8_t* qh = blk + 2;
    const uint8_t b = blk[6 + (i >> 1)];
    const uint32_t lo4 = (i & 1) ? (b >> 4) : (b & 0x0fu);
    const uint32_t hi1 = (qh[i >> 3] >> (i & 7)) & 1u;
    return (int)((hi1 << 4) | lo4) - 16;
}

__device__ __forceinline__ float q0_scale(const uint8_t* blk) {
    return vk_f16_to_f32((uint32_t)blk[0] | ((uint32_t)blk[1] << 8));
}

// ---------------------------------------------------------------------------
// Dequantize: 4 threads per block, 8 elements each, value = (float)q * d
// (the reference multiplies the integer-valued f32 by the decoded scale).
__global__ void vk_dequantize_q0(int mode, const uint8_t* __restrict__ bytes, size_t n_blocks,
                                 float* __restrict__ out) {
    const size_t gid = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t blk = gid >> 2;
    if (blk >= n_blocks) return;
    const int c = (int)(gid & 3);
    const int bb = q0_block_bytes(mode);
    const uint8_t* p = bytes + blk * (size_t)bb;
    const float d = q0_scale(p);
    float v[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = (float)q0_int(mode, p, 8 * c + e) * d;
    float4* o = reinterpret_cast<float4*>(out + blk * 32 + 8 * c);
    o[0] = make_float4(v[0], v[1], v[2], v[3]);
    o[1] = make_float4(v[4], v[5], v[6], v[7]);
}

// ---------------------------------------------------------------------------
// Plain 16-byte-per-lane copy (HBM bandwidth reference and the calibration
// kernel for rocprof FETCH_SIZE / WRITE_SIZE).
__global__ void vk_copy_u4(const uint4* __restrict__ src, uint4* __restrict__ dst, size_t n) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) dst[i] = src[i];
}

// ---------------------------------------------------------------------------
// Pack f32 -> wire blocks, one 32-lane half-wave per block (lane i owns
// element i). Same arithmetic as the reference packers: amax fold, d = amax/k
// (k = 127, 7, 15), inv = 1/d, q = round(clamp(x*inv, lo, hi)), f16(d) stored
// (q8_0.rs:40-64, q4_0.rs:44-68 + quantize_nibble :100-105, q5_0.rs pack).
__device__ __forceinline__ int vk_sat_round(float c) {
    // Rust `round() as i32` on an already clamped value: NaN -> 0.
    return (c != c) ? 0 : (int)roundf(c);
}

__global__ void vk_pack_q0(int mode, const float* __restrict__ x, size_t n_blocks, uint8_t* __restrict__ out) {
    const size_t gid = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t blk = gid >> 5;
    const int i = (int)(gid & 31);
    const bool live = blk < n_blocks;
    const float v = live ? x[blk * 32 + i] : 0.0f;
    const float amax = vk_group_max<32>(fmaxf(0.0f, fabsf(v)));  // NaN -> 0, as the fold from 0.0
    if (!live) return;
    const float div = mode == 3 ? 127.0f : (mode == 1 ? 7.0f : 15.0f);
    const float d = amax == 0.0f ? 0.0f : amax / div;
    const float inv = d == 0.0f ? 0.0f : 1.0f / d;
    const float sc = v * inv;
    uint8_t* p = out + blk * (size_t)q0_block_bytes(mode);
    if (i == 0) {
        const uint32_t h = vk_f32_to_f16_bits(d);
        p[0] = (uint8_t)(h & 0xff);
        p[1] = (uint8_t)(h >> 8);
    }
    // clamp-then-round; a NaN survives Rust's clamp and its cast gives 0
    // (fminf/fmaxf would replace the NaN, so it is tested first).
    if (mode == 3) {
        p[2 + i] = (uint8_t)(int8_t)vk_sat_round(sc != sc ? sc : fminf(fmaxf(sc, -127.0f), 127.0f));
        return;
    }
    int biased;
    if (mode == 1) biased = min(max(vk_sat_round(sc != sc ? sc : fminf(fmaxf(sc, -8.0f), 7.0f)) + 8, 0), 15);
    else biased = min(max(vk_sat_round(sc != sc ? sc : fminf(fmaxf(sc, -16.0f), 15.0f)) + 16, 0), 31);
    // Gather the packed fields: nibble pairs (2i, 2i+1) share a byte.
    const int lo4 = biased & 0x0f;
    const int partner = __shfl_xor(lo4, 1, VK_WAVE);
    if (mode == 1) {
        if ((i & 1) == 0) p[2 + (i >> 1)] = (uint8_t)(lo4 | (partner << 4));
        return;
    }
    if ((i & 1) == 0) p[6 + (i >> 1)] = (uint8_t)(lo4 | (partner << 4));
    const unsigned long long hb = __ballot(((biased >> 4) & 1) != 0);
    const uint32_t qh = (uint32_t)(hb >> (threadIdx.x & 32));
    if (i < 4) p[2 + i] = (uint8_t)((qh >> (8 * i)) & 0xff);
}

// ---------------------------------------------------------------------------
// f32-semantics dequant GEMV. Each work-item forms the partial dot of one
// (row, block) pair in element order; one lane per row then sums the row's
// block partials in block order. Rows per workgroup: floor(256 / n_bpr) (>= 1).
__global__ void vk_dequant_gemv_f32(int mode, const uint8_t* __restrict__ bytes, int n_rows,
                                    int n_bpr, int rows_per_wg, const float* __restrict__ x,
                                    float* __restrict__ y) {
    extern __shared__ float partial[];  // rows_per_wg * n_bpr
    const int row0 = blockIdx.x * rows_per_wg;
    const int rows_here = min(rows_per_wg, n_rows - row0);
    const int items = rows_here * n_bpr;
    const int bb = q0_block_bytes(mode);
    for (int it = threadIdx.x; it < items; it += blockDim.x) {
        const int r = it / n_bpr, b = it - r * n_bpr;
        const uint8_t* p = bytes + ((size_t)(row0 + r) * n_bpr + b) * bb;
        const float d = q0_scale(p);
        const float* xb = x + (size_t)b * 32;
        float acc = 0.0f;
#pragma unroll 8
        for (int i = 0; i < 32; ++i) acc = acc + ((float)q0_int(mode, p, i) * d) * xb[i];
        partial[it] = acc;
    }
    __syncthreads();
    for (int r = threadIdx.x; r < rows_here; r += blockDim.x) {
        float acc = 0.0f;
        for (int b = 0; b < n_bpr; ++b) acc = acc + partial[r * n_bpr + b];
        y[row0 + r] = acc;
    }
}

// ---------------------------------------------------------------------------
// INT8 activation quantization, 4 lanes per 32-element block (8 elements
// each). Convention "amax127" (kquant.rs:418-441 at group 32): s = amax/127,
// q = clamp(round(v / s), -127, 127); all-zero block -> s = 0, q = 0.
// Convention "pow2": s = 2^e, the smallest power of two >= amax/127, so the
// bf16 operand q * 2^e is exact and the MFMA folds the activation scale.
// Output: A fragments (bf16 of q, or of q * 2^e for pow2), scales [tile][nb][16]
// and block sums of q (same indexing). Rows >= m are written as zeros.
template <bool POW2>
__global__ void vk_quantize_act_b32(const float* __restrict__ a, int m, int m_pad, int k,
                                    uint4* __restrict__ afrag, float* __restrict__ ascale,
                                    float* __restrict__ asum) {
    // One wave per 16-row x 32-column fragment: lane l = mr + 16 c quantizes
    // row mr, elements 8c .. 8c+7, and stores its 16 bytes at lane l of the
    // fragment, so every wave writes one contiguous KiB.
    const int nb = k >> 5;
    // the fragment index is wave-uniform: its split into (mt, b) runs on the
    // scalar unit, ahead of the row loads that need it
    const int frag = __builtin_amdgcn_readfirstlane((int)(blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6)));
    if (frag >= (m_pad >> 4) * nb) return;  // whole waves exit together
    const int lane = (int)(threadIdx.x & 63), c = lane >> 4, mr = lane & 15;
    const int mt = frag / nb, b = frag - mt * nb;  // frag = mt * nb + b
    const int row = mt * 16 + mr;
    float v[8];
    if (row < m) {
        const float4* src = reinterpret_cast<const float4*>(a + (size_t)row * k + b * 32 + 8 * c);
        const float4 x0 = src[0], x1 = src[1];
        v[0] = x0.x; v[1] = x0.y; v[2] = x0.z; v[3] = x0.w;
        v[4] = x1.x; v[5] = x1.y; v[6] = x1.z; v[7] = x1.w;
    } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = 0.0f;
    }
    float amax = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(v[e]));
    // the four lanes of a row: l, l^16, l^32, l^48 (non-negative, not NaN: integer max)
    amax = __int_as_float(max(__float_as_int(amax), vk_bfly_partner<16>(__float_as_int(amax))));
    amax = __int_as_float(max(__float_as_int(amax), __shfl_xor(__float_as_int(amax), 32, VK_WAVE)));
    float s = 0.0f;
    int q[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    if (amax != 0.0f) {
        s = amax / 127.0f;
        if (POW2) {
            int ex;
            const float f = frexpf(s, &ex);  // s = f * 2^ex, f in [0.5, 1)
            s = ldexpf(1.0f, f == 0.5f ? ex - 1 : ex);
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            // Rust: (v / s).round().clamp(-127, 127) as i32 — a NaN survives
            // the clamp and the saturating cast maps it to 0.
            const float r = vk_round_half_away(v[e] / s);
            q[e] = (r != r) ? 0 : (int)fminf(fmaxf(r, -127.0f), 127.0f);
        }
    }
    int gs = 0;
#pragma unroll
    for (int e = 0; e < 8; ++e) gs += q[e];
    gs += vk_bfly_partner<16>(gs);
    gs += __shfl_xor(gs, 32, VK_WAVE);
    uint32_t w[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        uint32_t lo, hi;
        if (POW2) {
            lo = __float_as_uint((float)q[2 * e] * s) >> 16;
            hi = __float_as_uint((float)q[2 * e + 1] * s) >> 16;
        } else {
            lo = vk_int_to_bf16_bits(q[2 * e]);
            hi = vk_int_to_bf16_bits(q[2 * e + 1]);
        }
        w[e] = lo | (hi << 16);
    }
    afrag[(size_t)frag * 64 + lane] = make_uint4(w[0], w[1], w[2], w[3]);
    if (c == 0) {  // scales and operand sums are block-major: [nb][m_pad]
        ascale[(size_t)b * m_pad + row] = s;
        // sum of the A operand values of this block (exact: an integer times
        // a power of two), used to remove the weight-side offsets of the
        // decode kernel
        asum[(size_t)b * m_pad + row] = POW2 ? (float)gs * s : (float)gs;
    }
}

// ---------------------------------------------------------------------------
// LayerNorm fused with the activation pass: a 256-thread workgroup normalises
// a row exactly as vk_layer_norm_f32 (vk_ln_stats256 / vk_ln_apply) and
// quantizes it per 32-element block exactly as vk_quantize_act_b32 (thread t
// holds columns t + 256 j, a block is one half-wave). The result equals
// LayerNorm -> store -> quantize bit for bit, without the f32 round trip.
//  * TILE: a workgroup takes a 16-row fragment tile, row after row, stages
//    the bf16 operands in LDS in fragment order ((k / 32) KiB, dynamic) and
//    stores the tile as contiguous 1 KiB fragments;
//  * otherwise (a decode-sized batch): one row per workgroup, operands stored
//    straight to the fragments.
// Rows m .. m_pad-1 are zeros.
static_assert(kLnQuantMaxK <= kLnRegCols, "the fused pass holds its row in registers");
template <bool POW2, bool TILE>
__global__ __launch_bounds__(256) void vk_ln_quantize_b32(const float* __restrict__ in, int m, int m_pad, int k,
                                                          const float* __restrict__ gamma,
                                                          const float* __restrict__ beta, float eps,
                                                          uint4* __restrict__ afrag, float* __restrict__ ascale,
                                                          float* __restrict__ asum) {
    extern __shared__ uint4 lds_tile[];  // TILE: [nb][64] uint4 = the tile's fragments
    __shared__ float red[4];
    const int nb = k >> 5, t = threadIdx.x;
    const int mt = TILE ? (int)blockIdx.x : (int)blockIdx.x >> 4;
    uint16_t* tile16 = TILE ? reinterpret_cast<uint16_t*>(lds_tile)
                            : reinterpret_cast<uint16_t*>(afrag + (size_t)mt * nb * 64);
    // gamma and beta in registers up front: a global load inside the row
    // loop would make its wait (loads retire in order) also wait for the
    // next row's prefetch
    float gv[kLnRegJ], bv[kLnRegJ];
    vk_row_load256_all(gamma, k, gv);
    vk_row_load256_all(beta, k, bv);
    // TILE: rows r+1 .. r+LD are in flight while row r reduces (every row
    // load issued, rows past the matrix re-reading its last row), so the
    // workgroup waits one memory latency per LD rows, not per row. The row
    // loop stays rolled: unrolled over 16 rows the kernel is ~40 KB of code,
    // and three workgroups per CU at different rows thrash the instruction
    // cache.
    constexpr int LD = TILE ? 4 : 1;
    static_assert(16 % LD == 0, "whole row groups per tile");
    float xq[LD][kLnRegJ];
    const int row_first = mt * 16 + (TILE ? 0 : ((int)blockIdx.x & 15));
    const int row_last = max(m - 1, 0);
    const float* src = m > 0 ? in : gamma;  // with no rows, reads stay inside gamma (unused)
#pragma unroll
    for (int d = 0; d < LD; ++d) vk_row_load256_all(src + (size_t)min(row_first + d, row_last) * k, k, xq[d]);
    // rows r0 .. r0+LD-1 per pass, row r in slot r % LD (static register
    // indices: no copies that would wait for the younger rows' loads)
#pragma unroll 1
    for (int r0 = 0; r0 < (TILE ? 16 : 1); r0 += LD)
#pragma unroll
    for (int u = 0; u < LD; ++u) {
        const int r = r0 + u;
        const int mr = TILE ? r : (int)blockIdx.x & 15;
        const int row = mt * 16 + mr;
        const bool live = row < m;  // uniform per workgroup
        float x[kLnRegJ];
#pragma unroll
        for (int j = 0; j < kLnRegJ; ++j) x[j] = xq[u][j];
        if (TILE) vk_row_load256_all(src + (size_t)min(row + LD, row_last) * k, k, xq[u]);
        float2 st = make_float2(0.0f, 0.0f);
        if (live) st = vk_ln_stats256(x, k, eps, red);
#pragma unroll
        for (int j = 0; j < kLnRegJ; ++j) {
            const int c = t + 256 * j;
            if (c - (t & 31) >= k) break;  // k is a multiple of 32: whole half-waves
            const float v = live ? vk_ln_apply(x[j], st, gv[j], bv[j]) : 0.0f;
            // from 0 and through fmaxf, as the separate pass: NaN elements are ignored
            const float amax = vk_group_max<32>(fmaxf(0.0f, fabsf(v)));
            float s = 0.0f;
            int q = 0;
            if (amax != 0.0f) {
                s = amax / 127.0f;
                if (POW2) {
                    int ex;
                    const float f = frexpf(s, &ex);
                    s = ldexpf(1.0f, f == 0.5f ? ex - 1 : ex);
                }
                const float rr = vk_round_half_away(v / s);
                q = (rr != rr) ? 0 : (int)fminf(fmaxf(rr, -127.0f), 127.0f);
            }
            const int gs = vk_group_sum_i<32>(q);
            const int b = c >> 5, e = c & 31;
            tile16[((size_t)b * 64 + mr + 16 * (e >> 3)) * 8 + (e & 7)] =
                (uint16_t)(POW2 ? (__float_as_uint((float)q * s) >> 16) : vk_int_to_bf16_bits(q));
            if (e == 0) {
                ascale[(size_t)b * m_pad + row] = s;
                asum[(size_t)b * m_pad + row] = POW2 ? (float)gs * s : (float)gs;
            }
        }
    }
    if (TILE) {
        __syncthreads();
        uint4* dst = afrag + (size_t)mt * nb * 64;  // fragments (mt, 0 .. nb-1) are contiguous
        for (int i = t; i < nb * 64; i += 256) dst[i] = lds_tile[i];
    }
}

// ---------------------------------------------------------------------------
// Weight repack (upload time): wire blocks [n][nb] -> bf16 integer fragments
// [n_pad/16][nb][64][8] + f32 scales block-major [nb][n_pad]. Rows >= n are zero.
__global__ void vk_repack_w_b32(int mode, const uint8_t* __restrict__ wq, int n, int n_pad, int nb,
                                uint4* __restrict__ wfrag, float* __restrict__ wscale) {
    const size_t gid = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t total = (size_t)n_pad * nb * 4;
    if (gid >= total) return;
    const int c = (int)(gid & 3);
    const size_t rb = gid >> 2;
    const int row = (int)(rb / nb), b = (int)(rb % nb);
    const int bb = q0_block_bytes(mode);
    uint32_t w[4] = {0, 0, 0, 0};
    float d = 0.0f;
    if (row < n) {
        const uint8_t* p = wq + ((size_t)row * nb + b) * bb;
        d = q0_scale(p);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            w[e] = vk_int_to_bf16_bits(q0_int(mode, p, 8 * c + 2 * e)) |
                   (vk_int_to_bf16_bits(q0_int(mode, p, 8 * c + 2 * e + 1)) << 16);
        }
    }
    const int nt = row >> 4, nr = row & 15;
    const size_t frag = (size_t)nt * nb + b;
    wfrag[frag * 64 + (size_t)(nr + 16 * c)] = make_uint4(w[0], w[1], w[2], w[3]);
    if (c == 0) wscale[(size_t)b * n_pad + row] = d;
}

// ---------------------------------------------------------------------------
// Block GEMM, INT8 semantics on bf16 MFMA.
//   out[m, n] = sum_b fmaf(sa[m,b] * dw[n,b], P_b[m,n], .)   (+ bias[n])
// where P_b = v_mfma_f32_16x16x32_bf16 over one 32-element block of exact
// integer-valued bf16 operands: every partial sum is an integer below 2^24,
// so P_b equals the int32 block dot product exactly. With POW2 activations
// the A operand already carries 2^e and the combine is fmaf(dw, P_b, .),
// which is the same value (the power-of-two product sa * dw is exact).
//
// Workgroup tile 128 (m) x 128 (n): 4 waves in 2 x 2, wave tile 64 x 64 =
// 4 x 4 MFMA tiles, one quant block (K = 32) per pipeline stage; two
// workgroups per CU, so one's barrier wait overlaps the other's compute.
// Grids that would fill less than three quarters of the chip with such
// tiles run 32 x 32 wave tiles (64 x 64 workgroup tiles, four times the
// workgroups) with the same per-output arithmetic.
// Operands move global -> LDS directly (no staging registers) through a
// three-stage ring. Inside a wave the MFMAs of a block are interleaved with
// the VALU combine of earlier tiles, so the matrix core runs under the VALU
// work (two VALU ops per output per block: the larger cost of the two).
// Tile order is XCD-aware: workgroup i runs on XCD i % 8, so each XCD gets a
// contiguous run of tiles, ordered n-tile-major to share W tiles in its L2.
// The epilogue transposes each wave's 16 x 64 row strips through LDS so rows
// leave as full 256-byte dwordx4 stores (streaming: the result is not re-read
// by this kernel).
// Set (to 1) by a block GEMM whose split outputs (VkSplitOut) meet a value
// outside the fp16 range; read and cleared by the host (range_check in vk_capi.hip).
static __device__ unsigned int vk_gemm_range_flag;

namespace gemm {
constexpr int WM = 2, WN = 2;                 // waves per workgroup (m x n)
constexpr int THREADS = 64 * WM * WN;
constexpr int TM = 64 * WM, TN = 64 * WN;     // workgroup tile
constexpr int MT = TM / 16, NT = TN / 16;     // fragment tiles per workgroup tile
constexpr int FRAG_U4 = 64;                   // uint4 per 16x32 fragment (1 KiB)
constexpr int N_XCD = 8;
constexpr int NS = 3;                         // LDS stages
constexpr int LAG = 3;                        // MFMA -> combine distance (tiles)
}  // namespace gemm

// Wait until at most N of this thread's loads are in flight and every LDS
// access has completed, then barrier.
template <int N>
__device__ __forceinline__ void vk_wait_vm_barrier() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(N) : "memory");
}

// Up to three linears over the same activations and of the same width in one
// grid (q, k and v of an attention block): tile t of the launch belongs to
// linear t / (tiles per linear), so each one's outputs are those of its own
// launch.
struct GemmSet {
    VkGemmLin lin[3];
};

// WT: 16 x 16 MFMA tiles per wave side (4: 64 x 64 waves, 128 x 128
// workgroup tiles; 2: 32 x 32 waves, 64 x 64 workgroup tiles for grids that
// would not fill the chip). Per-output arithmetic is the same for both.
template <bool POW2, int WT, bool QOUT>
__global__ __launch_bounds__(gemm::THREADS, 2) void vk_gemm_qblock(
    const uint4* __restrict__ afrag, const float* __restrict__ ascale, const GemmSet set, int n_lin,
    int m, int n, int nb, int ldo, int m_pad, int n_pad) {
    using namespace gemm;
    static_assert(WT == 2 || WT == 4, "wave tile");
    constexpr int WAVES = WM * WN;
    constexpr int TM = 16 * WT * WM, TN = 16 * WT * WN;  // workgroup tile (hides the namespace's)
    constexpr int MT = TM / 16, NT = TN / 16;
    constexpr int NTILE = WT * WT;                        // MFMA tiles per wave
    constexpr int CPR = 4 * WT;                           // float4 per row of a wave's output strip
    constexpr int APT = MT * FRAG_U4 / THREADS, BPT = NT * FRAG_U4 / THREADS;  // uint4 loads per thread
    static_assert(APT * THREADS == MT * FRAG_U4 && BPT * THREADS == NT * FRAG_U4, "fragment split");
    static_assert(TM + TN <= THREADS, "one scale per thread");
    constexpr int LOADS = APT + BPT + 1;  // loads per thread per stage
    __shared__ __align__(16) uint4 lds_a[NS][MT * FRAG_U4];  // 3 x 8 KiB; reused by the epilogue
    __shared__ __align__(16) uint4 lds_b[NS][NT * FRAG_U4];  // 3 x 8 KiB
    // Block scales: [0, TM) activation rows, [TM, TM + TN) weight columns.
    __shared__ __align__(16) float lds_s[NS][THREADS];
    static_assert(sizeof(lds_a) >= (size_t)WAVES * 16 * 16 * WT * 4, "epilogue slots");

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WN, wn = wave - wm * WN;

    // XCD-aware tile index: workgroups L, L+8, L+16, ... share an XCD.
    const int tiles_m = m_pad / TM, tiles_n = n_pad / TN, tiles_lin = tiles_m * tiles_n, tiles = tiles_lin * n_lin;
    const int L = blockIdx.x;
    const int per_xcd = tiles / N_XCD;
    const int tt = (per_xcd * N_XCD == tiles) ? (L % N_XCD) * per_xcd + L / N_XCD : L;
    const int li = tt / tiles_lin, t = tt - li * tiles_lin;
    const int ntile = t / tiles_m, mtile = t - ntile * tiles_m;
    const int mt0 = mtile * MT, nt0 = ntile * NT;
    const uint4* __restrict__ wfrag = set.lin[li].wfrag;
    const float* __restrict__ wscale = set.lin[li].wscale;
    const float* __restrict__ bias = set.lin[li].bias;
    float* out = set.lin[li].out;
    const VkEpi epi = set.lin[li].epi;
    const VkQOut qo = set.lin[li].qo;  // used when QOUT (every linear of the launch has it)
    const VkSplitOut so = set.lin[li].so;

    // Per-thread slice of one stage: A fragments wave + q WAVES (q < APT), B
    // fragments likewise, and one scale (threads [0, TM): A rows, [TM, TM+TN):
    // W columns).
    const uint4* a_src = afrag + (size_t)(mt0 + wave) * nb * FRAG_U4 + lane;
    const uint4* b_src = wfrag + (size_t)(nt0 + wave) * nb * FRAG_U4 + lane;
    // (threads past TM + TN re-read a column scale into an unused slot)
    const float* s_src = tid < TM ? ascale + mt0 * 16 + tid : wscale + nt0 * 16 + (tid - TM) % TN;
    const int s_stride = tid < TM ? m_pad : n_pad;
    // wave-uniform LDS destinations (bytes)
    const uint32_t la = __builtin_amdgcn_readfirstlane(vk_lds_addr(&lds_a[0][wave * 64]));
    const uint32_t lb = __builtin_amdgcn_readfirstlane(vk_lds_addr(&lds_b[0][wave * 64]));
    const uint32_t ls = __builtin_amdgcn_readfirstlane(vk_lds_addr(&lds_s[0][wave * 64]));
    constexpr uint32_t A_STAGE = MT * FRAG_U4 * 16, B_STAGE = NT * FRAG_U4 * 16, S_STAGE = THREADS * 4;

    auto issue = [&](int b, int buf) {
        const size_t o = (size_t)b * FRAG_U4;
#pragma unroll
        for (int q = 0; q < APT; ++q)
            vk_dma_b128(a_src + (size_t)q * WAVES * nb * FRAG_U4 + o, la + buf * A_STAGE + q * WAVES * 1024);
#pragma unroll
        for (int q = 0; q < BPT; ++q)
            vk_dma_b128(b_src + (size_t)q * WAVES * nb * FRAG_U4 + o, lb + buf * B_STAGE + q * WAVES * 1024);
        vk_dma_b32(s_src + (size_t)b * s_stride, ls + buf * S_STAGE);
    };

    vk_f32x4 acc[WT][WT];
#pragma unroll
    for (int i = 0; i < WT; ++i)
#pragma unroll
        for (int j = 0; j < WT; ++j) acc[i][j] = (vk_f32x4){0.0f, 0.0f, 0.0f, 0.0f};

    const vk_f32x4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
    auto compute = [&](int buf) {
        vk_bf16x8 af[WT], bf[WT];
        float sa[WT][4], dw[WT];
#pragma unroll
        for (int i = 0; i < WT; ++i) {
            af[i] = __builtin_bit_cast(vk_bf16x8, lds_a[buf][(wm * WT + i) * FRAG_U4 + lane]);
            if (!POW2) {
                const float4 s4 = reinterpret_cast<const float4*>(lds_s[buf] + (wm * WT + i) * 16)[lane >> 4];
                sa[i][0] = s4.x; sa[i][1] = s4.y; sa[i][2] = s4.z; sa[i][3] = s4.w;
            }
        }
#pragma unroll
        for (int j = 0; j < WT; ++j) {
            bf[j] = __builtin_bit_cast(vk_bf16x8, lds_b[buf][(wn * WT + j) * FRAG_U4 + lane]);
            dw[j] = lds_s[buf][TM + (wn * WT + j) * 16 + (lane & 15)];
        }
        vk_f32x4 p[NTILE];
        auto combine = [&](int t) {
            const int i = t / WT, j = t % WT;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                if (POW2) acc[i][j][r] = fmaf(dw[j], p[t][r], acc[i][j][r]);
                else acc[i][j][r] = fmaf(sa[i][r] * dw[j], p[t][r], acc[i][j][r]);
            }
        };
        // Issue order is pinned (sched_barrier): MFMA t, then the combine of
        // tile t - LAG, whose product has retired; LAG + 1 products are live.
        // The combine order per output stays block order.
#pragma unroll
        for (int t = 0; t < NTILE; ++t) {
            p[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[t / WT], bf[t % WT], zero, 0, 0, 0);
            if (t >= LAG) combine(t - LAG);
            __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int t = NTILE - LAG; t < NTILE; ++t) combine(t);
    };

    // Stage ring of NS = 3: the loads for block b+2 are issued once every wave
    // has passed block b-1 (the barrier), into the buffer block b-1 used. At
    // the wait, this thread's loads for blocks b and b+1 may be outstanding:
    // vmcnt(LOADS) retires block b's. Loads past the last block re-read block
    // nb-1 into a buffer no later block reads, so every iteration issues
    // exactly LOADS loads. One block per iteration (no unrolling) keeps the
    // accumulators in fixed registers.
    const int last = nb - 1;
    issue(0, 0);
    issue(min(1, last), 1);
    int buf = 0, nbuf = 2;
#pragma unroll 1
    for (int b = 0; b < nb; ++b) {
        vk_wait_vm_barrier<LOADS>();
        issue(min(b + 2, last), nbuf);
        compute(buf);
        buf = buf == NS - 1 ? 0 : buf + 1;
        nbuf = nbuf == NS - 1 ? 0 : nbuf + 1;
    }
    // every load has landed and every wave is done reading before the
    // epilogue reuses the A buffers
    vk_wait_vm_barrier<0>();

    // Epilogue. D layout of v_mfma_f32_16x16x32_bf16: lane l holds rows
    // 4*(l/16)+r of column l%16. Each wave owns an LDS slot; per m-subtile it
    // writes the 16 x (16 WT) strip, then reads it back row-major.
    float* slot = reinterpret_cast<float*>(&lds_a[0][0]) + wave * (256 * WT);
    const int col0 = (nt0 + wn * WT) * 16;
    const bool vec_ok = (ldo % 4 == 0) && (col0 + 16 * WT <= n) &&
                        (((reinterpret_cast<uintptr_t>(out) | reinterpret_cast<uintptr_t>(bias) |
                           reinterpret_cast<uintptr_t>(epi.resid)) & 15) == 0);
    const int c4 = 4 * (lane % CPR);
    const float4 bv = (bias && vec_ok) ? *reinterpret_cast<const float4*>(bias + col0 + c4)
                                       : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
    for (int i = 0; i < WT; ++i) {
        const int row_base = (mt0 + wm * WT + i) * 16;
        // residual rows of this strip, loaded before the LDS round trip so the
        // latency overlaps it (rows past m read row m-1: in bounds, unused)
        float4 rv[WT];
        if (epi.resid && vec_ok) {
#pragma unroll
            for (int q = 0; q < WT; ++q) {
                const int row = min(row_base + (64 / CPR) * q + lane / CPR, m - 1);
                rv[q] = *reinterpret_cast<const float4*>(epi.resid + (size_t)row * ldo + col0 + c4);
            }
        }
#pragma unroll
        for (int j = 0; j < WT; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) slot[(4 * (lane >> 4) + r) * (16 * WT) + 16 * j + (lane & 15)] = acc[i][j][r];
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
        for (int q = 0; q < WT; ++q) {
            const int rr = (64 / CPR) * q + lane / CPR;
            const int row = row_base + rr;
            float4 v = *reinterpret_cast<const float4*>(slot + rr * (16 * WT) + c4);
            const size_t o = (size_t)row * ldo + col0 + c4;
            if (vec_ok) {
                if (bias) {
                    v.x = v.x + bv.x; v.y = v.y + bv.y; v.z = v.z + bv.z; v.w = v.w + bv.w;
                }
                if (epi.gelu) {
                    v.x = vk_gelu_as(v.x); v.y = vk_gelu_as(v.y); v.z = vk_gelu_as(v.z); v.w = vk_gelu_as(v.w);
                }
                if (epi.resid) {  // resid + y, as the separate add pass
                    v.x = rv[q].x + v.x; v.y = rv[q].y + v.y; v.z = rv[q].z + v.z; v.w = rv[q].w + v.w;
                }
                if (QOUT) {
                    // the activation pass over this row's 32-column block:
                    // 8 consecutive lanes hold it (columns 4 (lane % 8) ..)
                    float amax = fmaxf(fmaxf(fmaxf(0.0f, fabsf(v.x)), fmaxf(fabsf(v.y), fabsf(v.z))), fabsf(v.w));
                    amax = vk_group_max<8>(amax);
                    float sc = 0.0f;
                    int q4[4] = {0, 0, 0, 0};
                    if (amax != 0.0f) {
                        sc = vk_act_scale(amax, qo.pow2);
                        q4[0] = vk_act_q(v.x, sc); q4[1] = vk_act_q(v.y, sc);
                        q4[2] = vk_act_q(v.z, sc); q4[3] = vk_act_q(v.w, sc);
                    }
                    const int gs = vk_group_sum_i<8>((q4[0] + q4[1]) + (q4[2] + q4[3]));
                    if (row < m) {
                        const int col = col0 + c4, kb = col >> 5;
                        const size_t at = vk_afrag_u16((size_t)row, kb, qo.k >> 5, col & 31);
                        const uint32_t w0 = vk_act_bits(q4[0], sc, qo.pow2) | (vk_act_bits(q4[1], sc, qo.pow2) << 16);
                        const uint32_t w1 = vk_act_bits(q4[2], sc, qo.pow2) | (vk_act_bits(q4[3], sc, qo.pow2) << 16);
                        *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(qo.afrag) + at) = make_uint2(w0, w1);
                        if ((lane & 7) == 0) {
                            qo.ascale[(size_t)kb * qo.m_pad + row] = sc;
                            qo.asum[(size_t)kb * qo.m_pad + row] = qo.pow2 ? (float)gs * sc : (float)gs;
                        }
                    }
                }
                if (row < m && so.hi) {  // row-major split (k)
                    const float e4[4] = {v.x, v.y, v.z, v.w};
                    uint32_t hw[2], lw[2];
                    bool bad = false;
#pragma unroll
                    for (int u = 0; u < 2; ++u) {
                        const float x0 = e4[2 * u], x1 = e4[2 * u + 1];
                        bad |= vk_f16_overflow(x0) | vk_f16_overflow(x1);
                        const _Float16 h0 = (_Float16)x0, h1 = (_Float16)x1;
                        const _Float16 l0 = (_Float16)(x0 - (float)h0), l1 = (_Float16)(x1 - (float)h1);
                        hw[u] = __builtin_bit_cast(uint16_t, h0) | ((uint32_t)__builtin_bit_cast(uint16_t, h1) << 16);
                        lw[u] = __builtin_bit_cast(uint16_t, l0) | ((uint32_t)__builtin_bit_cast(uint16_t, l1) << 16);
                    }
                    if (bad) atomicOr(&vk_gemm_range_flag, 1u);
                    *reinterpret_cast<uint2*>(so.hi + o) = make_uint2(hw[0], hw[1]);
                    *reinterpret_cast<uint2*>(so.lo + o) = make_uint2(lw[0], lw[1]);
                } else if (row < m && out)
                    __builtin_nontemporal_store((vk_f32x4){v.x, v.y, v.z, v.w}, reinterpret_cast<vk_f32x4*>(out + o));
            } else if (row < m) {
                const float e[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const int col = col0 + c4 + u;
                    if (col >= n) continue;
                    const float y = vk_epi_apply(bias ? e[u] + bias[col] : e[u], epi, o + u);
                    if (so.hi) {  // row-major split (k)
                        if (vk_f16_overflow(y)) atomicOr(&vk_gemm_range_flag, 1u);
                        const _Float16 h = (_Float16)y;
                        so.hi[o + u] = __builtin_bit_cast(uint16_t, h);
                        so.lo[o + u] = __builtin_bit_cast(uint16_t, (_Float16)(y - (float)h));
                    } else {
                        out[o + u] = y;
                    }
                }
            }
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    }
}

template __global__ void vk_quantize_act_b32<false>(const float*, int, int, int, uint4*, float*, float*);
template __global__ void vk_quantize_act_b32<true>(const float*, int, int, int, uint4*, float*, float*);

template __global__ void vk_gemm_qblock<false, 4, false>(const uint4*, const float*, const GemmSet, int, int, int, int,
                                                       int, int, int);
template __global__ void vk_gemm_qblock<false, 4, true>(const uint4*, const float*, const GemmSet, int, int, int, int,
                                                       int, int, int);
template __global__ void vk_gemm_qblock<false, 2, false>(const uint4*, const float*, const GemmSet, int, int, int, int,
                                                       int, int, int);
template __global__ void vk_gemm_qblock<false, 2, true>(const uint4*, const float*, const GemmSet, int, int, int, int,
                                                       int, int, int);
template __global__ void vk_gemm_qblock<true, 4, false>(const uint4*, const float*, const GemmSet, int, int, int, int,
                                                       int, int, int);
template __global__ void vk_gemm_qblock<true, 4, true>(const uint4*, const float*, const GemmSet, int, int, int, int,
                                                       int, int, int);
template __global__ void vk_gemm_qblock<true, 2, false>(const uint4*, const float*, const GemmSet, int, int, int, int,
                                                       int, int, int);
template __global__ void vk_gemm_qblock<true, 2, true>(const uint4*, const float*, const GemmSet, int, int, int, int,
                                                       int, int, int);

}  // namespace vk

// ===========================================================================
// Host-side launchers (called by the C-ABI layer in vk_capi.hip).
// ===========================================================================
#include "vk_launch.h"

namespace vk {

hipError_t launch_dequantize_q0(hipStream_t s, int mode, const uint8_t* bytes, size_t n_blocks,
                                float* out) {
    if (n_blocks == 0) return hipSuccess;
    const size_t threads = n_blocks * 4;
    const unsigned grid = (unsigned)((threads + 255) / 256);
    hipLaunchKernelGGL(vk_dequantize_q0, dim3(grid), dim3(256), 0, s, mode, bytes, n_blocks, out);
    return hipGetLastError();
}

hipError_t launch_copy_u4(hipStream_t s, const void* src, void* dst, size_t n16) {
    if (n16 == 0) return hipSuccess;
    const size_t want = (n16 + 255) / 256;
    const unsigned grid = (unsigned)(want < 8192 ? want : 8192);
    hipLaunchKernelGGL(vk_copy_u4, dim3(grid), dim3(256), 0, s, (const uint4*)src, (uint4*)dst, n16);
    return hipGetLastError();
}

hipError_t launch_pack_q0(hipStream_t s, int mode, const float* x, size_t n_blocks, uint8_t* out) {
    if (n_blocks == 0) return hipSuccess;
    const size_t threads = n_blocks * 32;
    const unsigned grid = (unsigned)((threads + 255) / 256);
    hipLaunchKernelGGL(vk_pack_q0, dim3(grid), dim3(256), 0, s, mode, x, n_blocks, out);
    return hipGetLastError();
}

hipError_t launch_dequant_gemv_f32(hipStream_t s, int mode, const uint8_t* bytes, int n_rows,
                                   int n_bpr, const float* x, float* y) {
    if (n_rows == 0) return hipSuccess;
    const int rows_per_wg = n_bpr >= 256 ? 1 : 256 / n_bpr;
    const unsigned grid = (unsigned)((n_rows + rows_per_wg - 1) / rows_per_wg);
    const size_t lds = (size_t)rows_per_wg * n_bpr * sizeof(float);
    hipLaunchKernelGGL(vk_dequant_gemv_f32, dim3(grid), dim3(256), lds, s, mode, bytes, n_rows, n_bpr,
                       rows_per_wg, x, y);
    return hipGetLastError();
}

hipError_t launch_quantize_act_b32(hipStream_t s, bool pow2, const float* a, int m, int m_pad, int k,
                                   uint4* afrag, float* ascale, float* asum) {
    if (m_pad % 16 != 0) return hipErrorInvalidValue;  // whole fragments
    const size_t threads = (size_t)m_pad * (k / 32) * 4;
    if (threads == 0) return hipSuccess;
    if (threads > (size_t)INT32_MAX) return hipErrorInvalidValue;  // the kernel indexes in 32 bits
    const unsigned grid = (unsigned)((threads + 255) / 256);
    if (pow2)
        hipLaunchKernelGGL(vk_quantize_act_b32<true>, dim3(grid), dim3(256), 0, s, a, m, m_pad, k, afrag,
                           ascale, asum);
    else
        hipLaunchKernelGGL(vk_quantize_act_b32<false>, dim3(grid), dim3(256), 0, s, a, m, m_pad, k, afrag,
                           ascale, asum);
    return hipGetLastError();
}

hipError_t launch_ln_quantize_b32(hipStream_t s, bool pow2, const float* a, int m, int m_pad, int k,
                                  const float* gamma, const float* beta, float eps, uint4* afrag, float* ascale,
                                  float* asum) {
    if (m_pad % 16 != 0 || k % 32 != 0 || m > m_pad || k > kLnQuantMaxK) return hipErrorInvalidValue;
    if (m_pad == 0 || k == 0) return hipSuccess;
    // one row per workgroup unless there are enough 16-row tiles to fill the
    // chip with workgroups that stage whole tiles for contiguous stores
    const bool tile = m_pad / 16 >= 1024;
    const size_t lds = tile ? (size_t)(k / 32) * 1024 : 0;
    const dim3 grid(tile ? m_pad / 16 : m_pad), block(256);
    if (pow2 && tile)
        hipLaunchKernelGGL((vk_ln_quantize_b32<true, true>), grid, block, lds, s, a, m, m_pad, k, gamma, beta, eps,
                           afrag, ascale, asum);
    else if (pow2)
        hipLaunchKernelGGL((vk_ln_quantize_b32<true, false>), grid, block, lds, s, a, m, m_pad, k, gamma, beta, eps,
                           afrag, ascale, asum);
    else if (tile)
        hipLaunchKernelGGL((vk_ln_quantize_b32<false, true>), grid, block, lds, s, a, m, m_pad, k, gamma, beta, eps,
                           afrag, ascale, asum);
    else
        hipLaunchKernelGGL((vk_ln_quantize_b32<false, false>), grid, block, lds, s, a, m, m_pad, k, gamma, beta, eps,
                           afrag, ascale, asum);
    return hipGetLastError();
}

hipError_t launch_repack_w_b32(hipStream_t s, int mode, const uint8_t* wq, int n, int n_pad, int nb,
                               uint4* wfrag, float* wscale) {
    const size_t threads = (size_t)n_pad * nb * 4;
    if (threads == 0) return hipSuccess;
    const unsigned grid = (unsigned)((threads + 255) / 256);
    hipLaunchKernelGGL(vk_repack_w_b32, dim3(grid), dim3(256), 0, s, mode, wq, n, n_pad, nb, wfrag, wscale);
    return hipGetLastError();
}

// The C-ABI layer pads m and n to GEMM_TM / GEMM_TN: whole workgroup tiles.
static_assert(GEMM_TM % gemm::TM == 0 && GEMM_TN % gemm::TN == 0, "GEMM padding");

// Below three quarters of one resident round (256 CUs x 2 workgroups) of
// 128 x 128 tiles, 64 x 64 tiles win (measured: 120 tiles 26.5 -> 16.6 us,
// 360 tiles 37.8 -> 35.4 us; 480 tiles 39.5 -> 46.7 us, so those stay).
constexpr int kGemmSmallTileBelow = 384;  // 128 x 128 tiles per launch

hipError_t launch_gemm_qblock_multi(hipStream_t s, bool pow2, const uint4* afrag, const float* ascale,
                                    const VkGemmLin* lins, int n_lin, int m, int m_pad, int n, int n_pad, int nb) {
    if (m_pad % gemm::TM != 0 || n_pad % gemm::TN != 0 || nb < 1 || n_lin < 1 || n_lin > 3)
        return hipErrorInvalidValue;
    GemmSet set = {};
    for (int i = 0; i < n_lin; ++i) set.lin[i] = lins[i];
    // 128 x 128 workgroup tiles unless they leave CUs idle; then 64 x 64
    const int big = (n_pad / gemm::TN) * (m_pad / gemm::TM) * n_lin;
    const bool small = big < kGemmSmallTileBelow;
    bool qout = lins[0].qo.afrag != nullptr;
    for (int i = 1; i < n_lin; ++i)
        if ((lins[i].qo.afrag != nullptr) != qout) return hipErrorInvalidValue;
    const dim3 grid((unsigned)(small ? big * 4 : big)), block(gemm::THREADS);
#define VK_GQ(P, W, Q) hipLaunchKernelGGL((vk_gemm_qblock<P, W, Q>), grid, block, 0, s, afrag, ascale, set, n_lin, m, n, \
                                          nb, n, m_pad, n_pad)
    if (pow2) {
        if (small) { if (qout) VK_GQ(true, 2, true); else VK_GQ(true, 2, false); }
        else { if (qout) VK_GQ(true, 4, true); else VK_GQ(true, 4, false); }
    } else {
        if (small) { if (qout) VK_GQ(false, 2, true); else VK_GQ(false, 2, false); }
        else { if (qout) VK_GQ(false, 4, true); else VK_GQ(false, 4, false); }
    }
#undef VK_GQ
    return hipGetLastError();
}

// This device's address of this file's fp16-range flag (the host reads and
// clears it with one small kernel per check).
hipError_t gemm_range_flag_addr(unsigned** p) { return hipGetSymbolAddress((void**)p, HIP_SYMBOL(vk_gemm_range_flag)); }

hipError_t launch_gemm_qblock(hipStream_t s, bool pow2, const uint4* afrag, const float* ascale,
                              const uint4* wfrag, const float* wscale, const float* bias, float* out,
                              int m, int m_pad, int n, int n_pad, int nb, VkEpi epi, const VkQOut* qo) {
    // the fused pass runs in the vector epilogue: whole 128-column tiles and
    // 16-byte aligned rows
    if (qo && qo->afrag &&
        (n % 128 != 0 || n_pad != n || qo->k != n || qo->m_pad != m_pad ||
         ((reinterpret_cast<uintptr_t>(bias) | reinterpret_cast<uintptr_t>(epi.resid) |
           reinterpret_cast<uintptr_t>(out)) & 15) != 0))
        return hipErrorInvalidValue;
    const VkGemmLin lin = {wfrag, wscale, bias, out, epi, qo ? *qo : VkQOut{}};
    return launch_gemm_qblock_multi(s, pow2, afrag, ascale, &lin, 1, m, m_pad, n, n_pad, nb);
}

}  // namespace vk

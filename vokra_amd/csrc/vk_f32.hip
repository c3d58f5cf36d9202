// vk_f32.hip — f32 kernels of the path for gfx950: GEMM / GEMV (matrix cores
// in f32), row softmax, LayerNorm, RMSNorm, GELU, and the small per-step
// kernels of a decoder step (residual add, embedding gather, argmax).
//
// Semantics are the reference's scalar tier (crates/vokra-backend-cpu/src/
// kernels/scalar.rs); every per-element expression keeps the reference's
// operation order, reductions run in a different (tree) order, so results
// agree to f32 rounding rather than bit for bit.
#include <algorithm>

#include "vk_common.h"

namespace vk {

// ---------------------------------------------------------------------------
// GEMM: out[m][n] = bias[n] + sum_l a[m][l] * B(l, n) with B(l, n) = b[l][n]
// (BT = false, the reference's gemm_f32 layout, scalar.rs:41-72) or b[n][l]
// (BT = true: weights stored [out, in], e.g. tied embeddings). One workgroup
// per 64 x 64 output tile, K in chunks of 16 staged K-major in LDS, each wave a
// 32 x 32 sub-tile of v_mfma_f32_16x16x4_f32 (exact f32 products, f32 sums).
namespace g32 {
constexpr int T = 64, KC = 16, PAD = 4;
}

template <bool BT>
__global__ __launch_bounds__(256) void vk_gemm_f32(const float* __restrict__ a, const float* __restrict__ b,
                                                   const float* __restrict__ bias, VkEpi epi, float* out, int m,
                                                   int n, int k) {
    using namespace g32;
    __shared__ float as[KC][T + PAD];
    __shared__ float bs[KC][T + PAD];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n0 = blockIdx.x * T, m0 = blockIdx.y * T;
    const int wr = 32 * (wave >> 1), wc = 32 * (wave & 1);
    // this thread's 4 loads of each tile (out-of-range elements read as 0)
    const int ar = tid >> 2, ak = (tid & 3) * 4;         // A: row, first k
    const int bk = BT ? (tid & 3) * 4 : tid >> 4;        // B: first k (BT) or k
    const int bn = BT ? tid >> 2 : (tid & 15) * 4;       // B: n (BT) or first n
    float ra[4], rb[4];
    auto load = [&](int k0) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int gm = m0 + ar, gk = k0 + ak + j;
            ra[j] = (gm < m && gk < k) ? a[(size_t)gm * k + gk] : 0.0f;
            if (BT) {
                const int gn = n0 + bn, gk2 = k0 + bk + j;
                rb[j] = (gn < n && gk2 < k) ? b[(size_t)gn * k + gk2] : 0.0f;
            } else {
                const int gn = n0 + bn + j, gk2 = k0 + bk;
                rb[j] = (gn < n && gk2 < k) ? b[(size_t)gk2 * n + gn] : 0.0f;
            }
        }
    };
    vk_f32x4 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = {0.0f, 0.0f, 0.0f, 0.0f};
    load(0);
    for (int k0 = 0; k0 < k; k0 += KC) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            as[ak + j][ar] = ra[j];
            if (BT) bs[bk + j][bn] = rb[j];
            else bs[bk][bn + j] = rb[j];
        }
        __syncthreads();
        if (k0 + KC < k) load(k0 + KC);
#pragma unroll
        for (int s = 0; s < KC / 4; ++s) {
            const int kk = 4 * s + (lane >> 4);
            float av[2], bv[2];
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                av[t] = as[kk][wr + 16 * t + (lane & 15)];
                bv[t] = bs[kk][wc + 16 * t + (lane & 15)];
            }
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[i], bv[j], acc[i][j], 0, 0, 0);
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int gm = m0 + wr + 16 * i + 4 * (lane >> 4) + r, gn = n0 + wc + 16 * j + (lane & 15);
                if (gm < m && gn < n) {
                    const size_t o = (size_t)gm * n + gn;
                    out[o] = vk_epi_apply(bias ? bias[gn] + acc[i][j][r] : acc[i][j][r], epi, o);
                }
            }
}

__device__ __forceinline__ float vk_f4c(const float4& v, int s) {
    return s == 0 ? v.x : (s == 1 ? v.y : (s == 2 ? v.z : v.w));
}

// Tiled GEMM for K % 16 == 0: 128 x 128 workgroup tiles (four 64 x 64 waves),
// K in 16-wide stages moved global -> LDS by direct loads through a ring of
// three stages (two ahead of the MFMAs), XCD-aware tile order. Fragments of
// v_mfma_f32_16x16x4f32 are read as float4: lane group g = l / 16 holds k =
// 4g .. 4g+3 of the stage and MFMA s takes component s, so one 16-byte LDS read
// feeds four MFMAs (for BT = false the B values come as four 4-byte reads).
// Rows / columns past M / N read the last valid one (in bounds, discarded).
namespace g32f {
constexpr int TM = 128, TN = 128, KC = 16, NS = 3, N_XCD = 8;
}

template <bool BT>
__global__ __launch_bounds__(256, 2) void vk_gemm_f32_tiled(const float* __restrict__ a, const float* __restrict__ b,
                                                            const float* __restrict__ bias, VkEpi epi, float* out,
                                                            int m, int n, int k) {
    using namespace g32f;
    __shared__ __align__(16) float la[NS][TM * KC];  // [row][k], 8 KiB per stage
    __shared__ __align__(16) float lb[NS][TN * KC];  // BT: [col][k]; else [k][col]
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, g = lane >> 4, l16 = lane & 15;
    const int wm = wave >> 1, wn = wave & 1;
    const int tiles_m = (m + TM - 1) / TM, tiles_n = (n + TN - 1) / TN, tiles = tiles_m * tiles_n;
    const int L = blockIdx.x;
    const int per_xcd = tiles / N_XCD;
    const int t = (per_xcd * N_XCD == tiles) ? (L % N_XCD) * per_xcd + L / N_XCD : L;
    const int mt = t % tiles_m, nt = t / tiles_m;
    const int m0 = mt * TM, n0 = nt * TN;

    // direct loads: each wave moves 2 KiB of A and 2 KiB of B per stage (two
    // 1 KiB instructions each); lane l of instruction i lands at +16 l
    const float* asrc[2];
    const float* bsrc[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int r = 16 * (2 * wave + i) + (lane >> 2);  // A row of the tile (16 rows x 64 B per KiB)
        asrc[i] = a + (size_t)min(m0 + r, m - 1) * k + 4 * (lane & 3);
        if (BT) {
            bsrc[i] = b + (size_t)min(n0 + r, n - 1) * k + 4 * (lane & 3);
        } else {
            const int kr = 2 * (2 * wave + i) + (lane >> 5);          // k row of the stage (2 rows x 512 B per KiB)
            const int cq = min(n0 / 4 + (lane & 31), n / 4 - 1);      // column quad (n % 4 == 0)
            bsrc[i] = b + (size_t)kr * n + 4 * cq;
        }
    }
    // wave-uniform LDS destinations (M0 takes a scalar register)
    const uint32_t la0 = __builtin_amdgcn_readfirstlane(vk_lds_addr(&la[0][0]) + wave * 2048);
    const uint32_t lb0 = __builtin_amdgcn_readfirstlane(vk_lds_addr(&lb[0][0]) + wave * 2048);
    constexpr uint32_t STAGE = TM * KC * 4;
    auto issue = [&](int kc, int buf) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            vk_dma_b128(asrc[i] + kc, la0 + buf * STAGE + i * 1024);
            vk_dma_b128(BT ? bsrc[i] + kc : bsrc[i] + (size_t)kc * n, lb0 + buf * STAGE + i * 1024);
        }
    };
    vk_f32x4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = {0.0f, 0.0f, 0.0f, 0.0f};
    const int nk = k / KC;  // >= 2
    issue(0, 0);
    issue(KC, 1);
    int buf = 0, nbuf = 2;
#pragma unroll 1
    for (int kc = 0; kc < nk; ++kc) {
        // this thread's stage kc has landed (stage kc+1 may be in flight), then
        // every wave's has: the buffer of stage kc-1 is free for kc+2
        if (kc + 1 < nk) asm volatile("s_waitcnt vmcnt(4)\n\ts_barrier" ::: "memory");
        else asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
        if (kc + 2 < nk) issue((kc + 2) * KC, nbuf);
        float4 av[4];
        float bv[4][4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
            av[i] = *reinterpret_cast<const float4*>(&la[buf][(wm * 64 + 16 * i + l16) * KC + 4 * g]);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int col = wn * 64 + 16 * j + l16;
            if (BT) {
                const float4 v = *reinterpret_cast<const float4*>(&lb[buf][col * KC + 4 * g]);
                bv[j][0] = v.x; bv[j][1] = v.y; bv[j][2] = v.z; bv[j][3] = v.w;
            } else {
#pragma unroll
                for (int s2 = 0; s2 < 4; ++s2) bv[j][s2] = lb[buf][(4 * g + s2) * TN + col];
            }
        }
#pragma unroll
        for (int s2 = 0; s2 < 4; ++s2)
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(vk_f4c(av[i], s2), bv[j][s2], acc[i][j], 0, 0, 0);
        buf = buf == NS - 1 ? 0 : buf + 1;
        nbuf = nbuf == NS - 1 ? 0 : nbuf + 1;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int gm = m0 + wm * 64 + 16 * i + 4 * g + r, gn = n0 + wn * 64 + 16 * j + l16;
                if (gm < m && gn < n) {
                    const size_t o = (size_t)gm * n + gn;
                    out[o] = vk_epi_apply(bias ? bias[gn] + acc[i][j][r] : acc[i][j][r], epi, o);
                }
            }
}

// GEMV: out[i] = bias[i] + a[i][:] . x (scalar.rs:74-91). One wave per row,
// float4 loads when the row stride allows; the row streams from HBM once.
__global__ __launch_bounds__(256) void vk_gemv_f32(const float* __restrict__ a, const float* __restrict__ x,
                                                   const float* __restrict__ bias, float* __restrict__ out, int m,
                                                   int k) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= m) return;
    const float* ar = a + (size_t)row * k;
    float s = 0.0f;
    if ((k & 3) == 0) {
        const float4* a4 = reinterpret_cast<const float4*>(ar);
        const float4* x4 = reinterpret_cast<const float4*>(x);
        for (int i = lane; i < k / 4; i += 64) {
            const float4 u = a4[i], v = x4[i];
            s = fmaf(u.x, v.x, s);
            s = fmaf(u.y, v.y, s);
            s = fmaf(u.z, v.z, s);
            s = fmaf(u.w, v.w, s);
        }
    } else {
        for (int i = lane; i < k; i += 64) s = fmaf(ar[i], x[i], s);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o, VK_WAVE);
    if (lane == 0) out[row] = bias ? bias[row] + s : s;
}

// ---------------------------------------------------------------------------
// Row reductions over a 256-thread workgroup.
__device__ __forceinline__ float block_sum(float v, float* red) { return vk_block_sum256(v, red); }
__device__ __forceinline__ float block_max(float v, float* red) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, VK_WAVE));
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

// softmax (scalar.rs:177-199): e = exp(x - max), out = e * (1 / sum e).
__global__ __launch_bounds__(256) void vk_softmax_f32(const float* __restrict__ in, float* __restrict__ out,
                                                      int cols) {
    __shared__ float red[4];
    const float* ir = in + (size_t)blockIdx.x * cols;
    float* orow = out + (size_t)blockIdx.x * cols;
    float mx = -INFINITY;
    for (int c = threadIdx.x; c < cols; c += 256) mx = fmaxf(mx, ir[c]);
    mx = block_max(mx, red);
    float s = 0.0f;
    for (int c = threadIdx.x; c < cols; c += 256) {
        const float e = expf(ir[c] - mx);
        orow[c] = e;
        s += e;
    }
    const float inv = 1.0f / block_sum(s, red);
    for (int c = threadIdx.x; c < cols; c += 256) orow[c] *= inv;
}

// layer_norm (scalar.rs:201-222): population variance, then
// (x - mean) * inv_std * gamma + beta per element; one row per workgroup.
__global__ __launch_bounds__(256) void vk_layer_norm_f32(const float* __restrict__ in, float* __restrict__ out,
                                                         int cols, const float* __restrict__ gamma,
                                                         const float* __restrict__ beta, float eps) {
    __shared__ float red[4];
    const float* ir = in + (size_t)blockIdx.x * cols;
    float* orow = out + (size_t)blockIdx.x * cols;
    if (cols <= kLnRegCols) {
        float x[kLnRegJ];
        vk_row_load256(ir, cols, x);
        const float2 st = vk_ln_stats256(x, cols, eps, red);
#pragma unroll
        for (int j = 0; j < kLnRegJ; ++j) {
            const int c = (int)threadIdx.x + 256 * j;
            if (c < cols) orow[c] = vk_ln_apply(x[j], st, gamma[c], beta[c]);
        }
        return;
    }
    const float2 st = vk_ln_stats256(ir, cols, eps, red);
    for (int c = threadIdx.x; c < cols; c += 256) orow[c] = vk_ln_apply(ir[c], st, gamma[c], beta[c]);
}

// rms_norm (crates/vokra-models/src/voxtral/text_decoder.rs:801-822).
__global__ __launch_bounds__(256) void vk_rms_norm_f32(const float* __restrict__ in, float* __restrict__ out,
                                                       int cols, const float* __restrict__ gamma, float eps) {
    __shared__ float red[4];
    const float* ir = in + (size_t)blockIdx.x * cols;
    float* orow = out + (size_t)blockIdx.x * cols;
    const float inv = 1.0f / sqrtf(block_sum(vk_sumsq_cols256(ir, cols), red) / (float)cols + eps);
    for (int c = threadIdx.x; c < cols; c += 256) orow[c] = ir[c] * inv * gamma[c];
}

// GELU through the Abramowitz & Stegun 7.1.26 erf (vk_gelu_as, scalar.rs:126-172).
__global__ void vk_gelu_f32(const float* __restrict__ x, float* __restrict__ out, size_t n) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        out[i] = vk_gelu_as(x[i]);
}

// out = a + b (residual connections).
// out may be a or b (in place): each element is read and written by one thread.
__global__ void vk_add_f32(const float* a, const float* b, float* out, size_t n) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        out[i] = a[i] + b[i];
}

// h[i] = tok_emb[tokens[i]] + pos_emb[positions[i]] (whisper/decoder.rs:420-432);
// with pos_emb NULL, the embedding row alone (rotary models add no position
// vector, voxtral/text_decoder.rs:1080-1095).
__global__ void vk_embed_f32(const float* __restrict__ tok_emb, const float* __restrict__ pos_emb,
                             const int* __restrict__ tokens, const int* __restrict__ positions, int vocab,
                             int n_pos, int d, float* __restrict__ out) {
    const int i = blockIdx.x;
    const int t = min(max(tokens[i], 0), vocab - 1);
    if (!pos_emb) {
        for (int c = threadIdx.x; c < d; c += blockDim.x) out[(size_t)i * d + c] = tok_emb[(size_t)t * d + c];
        return;
    }
    const int p = min(max(positions[i], 0), n_pos - 1);
    for (int c = threadIdx.x; c < d; c += blockDim.x)
        out[(size_t)i * d + c] = tok_emb[(size_t)t * d + c] + pos_emb[(size_t)p * d + c];
}

// argmax per row, first strict maximum from -inf (decode/sampler.rs:197-206):
// NaN never wins, ties keep the lowest index.
__global__ __launch_bounds__(256) void vk_argmax_f32(const float* __restrict__ logits, int cols,
                                                     int* __restrict__ out) {
    __shared__ float rv[4];
    __shared__ int ri[4];
    const float* row = logits + (size_t)blockIdx.x * cols;
    float bv = -INFINITY;
    int bi = 0;
    for (int c = threadIdx.x; c < cols; c += 256)
        if (row[c] > bv) {
            bv = row[c];
            bi = c;
        }
    // reduce (value desc, index asc); a lane with no strict max keeps (-inf, 0)
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(bv, o, VK_WAVE);
        const int oi = __shfl_xor(bi, o, VK_WAVE);
        if (ov > bv || (ov == bv && oi < bi)) {
            bv = ov;
            bi = oi;
        }
    }
    if ((threadIdx.x & 63) == 0) {
        rv[threadIdx.x >> 6] = bv;
        ri[threadIdx.x >> 6] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        float v = rv[0];
        int idx = ri[0];
        for (int w = 1; w < 4; ++w)
            if (rv[w] > v || (rv[w] == v && ri[w] < idx)) {
                v = rv[w];
                idx = ri[w];
            }
        out[blockIdx.x] = idx;
    }
}

// ---------------------------------------------------------------------------
// Tied logits and greedy argmax in one pass over the embedding
// (whisper/decoder.rs:754-796 project_logits_into, then decode/sampler.rs:
// 197-206 argmax): logits[s][v] = emb[v][:] . x[s][:].
//
// One workgroup per 16*J vocabulary rows and up to 16*NCT streams (1621
// workgroups at the Whisper vocabulary: fine-grained enough to balance 256
// CUs). Its 4 waves split d into quarters and their partial dots are summed
// in wave order. Operands are v_mfma_f32_16x16x4f32 fragments taken straight
// from row-major memory: vocabulary rows on the 16-row side, streams on the
// 16-column side, lane l holding k = 4*(l/16) .. +3 of row l%16 of a 16-wide
// k chunk as one float4, MFMA s of the chunk taking component s of both
// operands (A and B agree on k). Each wave moves its chunks global -> LDS with
// direct loads (lane l lands at slot + 16*l and reads the same 16 bytes back)
// through a private three-slot ring, two chunks ahead of the MFMAs; a stream's
// x row is read by every workgroup from L2.
//
// The argmax keeps the sampler's rule: first strict maximum from -inf (NaN
// never wins, ties keep the lowest index, index 0 when nothing beats -inf).
// Each workgroup stores its (max, index) per stream; vk_argmax_parts scans
// those in vocabulary order with the same rule.
namespace lg {
#ifndef VK_LG_WAVES
#define VK_LG_WAVES 4
#endif
#ifndef VK_LG_J
#define VK_LG_J 2
#endif
#ifndef VK_LG_NSLOT
#define VK_LG_NSLOT 3
#endif
constexpr int WAVES = VK_LG_WAVES, J = VK_LG_J, NSLOT = VK_LG_NSLOT;
static_assert(NSLOT >= 2 && NSLOT <= 4, "ring depth");
static_assert(WAVES >= 1 && WAVES <= 16, "workgroup of 64 * WAVES threads");
}


// (value desc, index asc) merge of two argmax candidates
__device__ __forceinline__ void vk_am_merge(float& bv, int& bi, float ov, int oi) {
    if (ov > bv || (ov == bv && oi < bi)) {
        bv = ov;
        bi = oi;
    }
}

template <int NCT, bool WRITE>
__global__ __launch_bounds__(64 * lg::WAVES) void vk_logits_argmax(const float* __restrict__ x, const float* __restrict__ emb,
                                                           float* __restrict__ logits, float2* __restrict__ part,
                                                           int n, int vocab, int d, int n_vt) {
    using namespace lg;
    constexpr int Q = J + NCT;  // 1 KiB direct loads per wave per chunk
    __shared__ __align__(16) uint4 ring[WAVES][NSLOT][Q][64];
    // after the k loop the ring holds the partial dots of waves 1..3
    static_assert(sizeof(ring) >= sizeof(vk_f32x4) * (WAVES - 1) * J * NCT * 64, "reduction fits the ring");
    vk_f32x4* red = reinterpret_cast<vk_f32x4*>(&ring[0][0][0][0]);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int v0 = blockIdx.x * 16 * J, s0 = blockIdx.y * 16 * NCT;
    const int dq = d / WAVES;                    // this wave's k range: [wave*dq, wave*dq + dq)
    const int kq = wave * dq + 4 * (lane >> 4);  // the lane's first k within a chunk
    const float* ep[J];
    const float* xp[NCT];
#pragma unroll
    for (int j = 0; j < J; ++j) ep[j] = emb + (size_t)min(v0 + 16 * j + (lane & 15), vocab - 1) * d + kq;
#pragma unroll
    for (int c = 0; c < NCT; ++c) xp[c] = x + (size_t)min(s0 + 16 * c + (lane & 15), n - 1) * d + kq;
    const uint32_t base = __builtin_amdgcn_readfirstlane(vk_lds_addr(&ring[wave][0][0][0]));
    constexpr uint32_t SLOT = Q * 1024;
    auto issue = [&](int ck, int slot) {
#pragma unroll
        for (int j = 0; j < J; ++j) vk_dma_b128(ep[j] + 16 * ck, base + slot * SLOT + j * 1024);
#pragma unroll
        for (int c = 0; c < NCT; ++c) vk_dma_b128(xp[c] + 16 * ck, base + slot * SLOT + (J + c) * 1024);
    };
    vk_f32x4 acc[J][NCT];
#pragma unroll
    for (int j = 0; j < J; ++j)
#pragma unroll
        for (int c = 0; c < NCT; ++c) acc[j][c] = {0.0f, 0.0f, 0.0f, 0.0f};
    const int nk = dq / 16;  // 16-wide k chunks of this wave (>= NSLOT - 1)
#pragma unroll
    for (int p = 0; p < NSLOT - 1; ++p) issue(p, p);
    int slot = 0;
#pragma unroll 1
    for (int ck = 0; ck < nk; ++ck) {
        // chunk ck's loads are the oldest in flight: wait for exactly those
        const int ahead = nk - 1 - ck;  // chunks loaded after ck, once the ring is full
        if (ahead >= NSLOT - 1) {
            issue(ck + NSLOT - 1, slot == 0 ? NSLOT - 1 : slot - 1);
            vk_wait_vm<(NSLOT - 1) * Q>();
        } else if (NSLOT > 3 && ahead == 2) {
            vk_wait_vm<2 * Q>();
        } else if (ahead == 1) {
            vk_wait_vm<Q>();
        } else {
            vk_wait_vm<0>();
        }
        float4 ce[J], cx[NCT];
#pragma unroll
        for (int j = 0; j < J; ++j) ce[j] = *reinterpret_cast<const float4*>(&ring[wave][slot][j][lane]);
#pragma unroll
        for (int c = 0; c < NCT; ++c) cx[c] = *reinterpret_cast<const float4*>(&ring[wave][slot][J + c][lane]);
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int j = 0; j < J; ++j)
#pragma unroll
                for (int c = 0; c < NCT; ++c)
                    acc[j][c] = __builtin_amdgcn_mfma_f32_16x16x4f32(vk_f4c(ce[j], s), vk_f4c(cx[c], s), acc[j][c],
                                                                     0, 0, 0);
        slot = slot == NSLOT - 1 ? 0 : slot + 1;
    }
    __syncthreads();  // every wave is done with the ring (its loads have all landed)
    if (wave > 0) {
#pragma unroll
        for (int j = 0; j < J; ++j)
#pragma unroll
            for (int c = 0; c < NCT; ++c) red[((wave - 1) * J * NCT + j * NCT + c) * 64 + lane] = acc[j][c];
    }
    __syncthreads();
    if (wave > 0) return;
#pragma unroll
    for (int c = 0; c < NCT; ++c) {
        const int s = s0 + 16 * c + (lane & 15);
        float bv = -INFINITY;
        int bi = INT_MAX;
#pragma unroll
        for (int j = 0; j < J; ++j) {
            vk_f32x4 t = acc[j][c];
#pragma unroll
            for (int w = 0; w < WAVES - 1; ++w) {
                const vk_f32x4 o = red[(w * J * NCT + j * NCT + c) * 64 + lane];
#pragma unroll
                for (int r = 0; r < 4; ++r) t[r] += o[r];
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int v = v0 + 16 * j + 4 * (lane >> 4) + r;  // ascending within the lane
                if (v < vocab) {
                    if (WRITE && s < n) logits[(size_t)s * vocab + v] = t[r];
                    if (t[r] > bv) {
                        bv = t[r];
                        bi = v;
                    }
                }
            }
        }
        // lanes l, l^16, l^32, l^48 hold the same stream
        vk_am_merge(bv, bi, __shfl_xor(bv, 16, VK_WAVE), __shfl_xor(bi, 16, VK_WAVE));
        vk_am_merge(bv, bi, __shfl_xor(bv, 32, VK_WAVE), __shfl_xor(bi, 32, VK_WAVE));
        if (lane < 16 && s < n) part[(size_t)s * n_vt + blockIdx.x] = make_float2(bv, __int_as_float(bi));
    }
}

// One workgroup per stream: merge its n_vt (max, index) partials. A partial
// whose max is -inf holds no candidate; the result is index 0 when no value
// beats -inf, as in the sampler.
__global__ __launch_bounds__(256) void vk_argmax_parts(const float2* __restrict__ part, int n_vt,
                                                       int* __restrict__ out) {
    __shared__ float rv[4];
    __shared__ int ri[4];
    const float2* p = part + (size_t)blockIdx.x * n_vt;
    float bv = -INFINITY;
    int bi = INT_MAX;
    for (int t = threadIdx.x; t < n_vt; t += 256) {
        const float2 q = p[t];
        vk_am_merge(bv, bi, q.x, __float_as_int(q.y));
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) vk_am_merge(bv, bi, __shfl_xor(bv, o, VK_WAVE), __shfl_xor(bi, o, VK_WAVE));
    if ((threadIdx.x & 63) == 0) {
        rv[threadIdx.x >> 6] = bv;
        ri[threadIdx.x >> 6] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < 4; ++w) vk_am_merge(bv, bi, rv[w], ri[w]);
        out[blockIdx.x] = bv > -INFINITY ? bi : 0;
    }
}

// argmax over wide rows in two passes: workgroup (slice, row) scans columns
// [slice * AM_SLICE, +AM_SLICE) with the same strict-greater rule and stores
// its (max, index) pair; vk_argmax_parts then merges a row's pairs. Each
// thread visits its columns in increasing order, so "first strict maximum"
// survives the (value desc, index asc) merges.
constexpr int AM_SLICE = 2048;
__global__ __launch_bounds__(256) void vk_argmax_slices(const float* __restrict__ logits, int cols, int n_sl,
                                                        float2* __restrict__ part) {
    __shared__ float rv[4];
    __shared__ int ri[4];
    const float* row = logits + (size_t)blockIdx.y * cols;
    const int c0 = blockIdx.x * AM_SLICE + threadIdx.x;
    float v[AM_SLICE / 256];
#pragma unroll
    for (int j = 0; j < AM_SLICE / 256; ++j) v[j] = c0 + 256 * j < cols ? row[c0 + 256 * j] : -INFINITY;
    float bv = -INFINITY;
    int bi = INT_MAX;
#pragma unroll
    for (int j = 0; j < AM_SLICE / 256; ++j)
        if (v[j] > bv) {
            bv = v[j];
            bi = c0 + 256 * j;
        }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) vk_am_merge(bv, bi, __shfl_xor(bv, o, VK_WAVE), __shfl_xor(bi, o, VK_WAVE));
    if ((threadIdx.x & 63) == 0) {
        rv[threadIdx.x >> 6] = bv;
        ri[threadIdx.x >> 6] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < 4; ++w) vk_am_merge(bv, bi, rv[w], ri[w]);
        part[(size_t)blockIdx.y * n_sl + blockIdx.x] = make_float2(bv, __int_as_float(bi));
    }
}

}  // namespace vk

#include "vk_launch.h"

namespace vk {

hipError_t launch_gemm_f32(hipStream_t s, bool b_trans, const float* a, const float* b, const float* bias,
                           float* out, int m, int n, int k, VkEpi epi) {
    if (m == 0 || n == 0) return hipSuccess;
    // the tiled kernel: whole 16-wide K stages (at least two), 16-byte aligned
    // rows, and for B [k, n] whole column quads
    const bool aligned = ((reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(b)) & 15) == 0;
    if (k % g32f::KC == 0 && k >= 2 * g32f::KC && aligned && (b_trans || n % 4 == 0)) {
        const unsigned tiles = (unsigned)(((m + g32f::TM - 1) / g32f::TM) * ((n + g32f::TN - 1) / g32f::TN));
        if (b_trans)
            hipLaunchKernelGGL(vk_gemm_f32_tiled<true>, dim3(tiles), dim3(256), 0, s, a, b, bias, epi, out, m, n, k);
        else
            hipLaunchKernelGGL(vk_gemm_f32_tiled<false>, dim3(tiles), dim3(256), 0, s, a, b, bias, epi, out, m, n, k);
        return hipGetLastError();
    }
    const dim3 grid((n + g32::T - 1) / g32::T, (m + g32::T - 1) / g32::T);
    if (b_trans)
        hipLaunchKernelGGL(vk_gemm_f32<true>, grid, dim3(256), 0, s, a, b, bias, epi, out, m, n, k);
    else
        hipLaunchKernelGGL(vk_gemm_f32<false>, grid, dim3(256), 0, s, a, b, bias, epi, out, m, n, k);
    return hipGetLastError();
}

hipError_t launch_gemv_f32(hipStream_t s, const float* a, const float* x, const float* bias, float* out, int m,
                           int k) {
    if (m == 0) return hipSuccess;
    hipLaunchKernelGGL(vk_gemv_f32, dim3((unsigned)((m + 3) / 4)), dim3(256), 0, s, a, x, bias, out, m, k);
    return hipGetLastError();
}

hipError_t launch_softmax_f32(hipStream_t s, const float* in, float* out, int rows, int cols) {
    if (rows == 0 || cols == 0) return hipSuccess;
    hipLaunchKernelGGL(vk_softmax_f32, dim3(rows), dim3(256), 0, s, in, out, cols);
    return hipGetLastError();
}

hipError_t launch_layer_norm_f32(hipStream_t s, const float* in, float* out, int rows, int cols, const float* gamma,
                                 const float* beta, float eps) {
    if (rows == 0 || cols == 0) return hipSuccess;
    hipLaunchKernelGGL(vk_layer_norm_f32, dim3(rows), dim3(256), 0, s, in, out, cols, gamma, beta, eps);
    return hipGetLastError();
}

hipError_t launch_rms_norm_f32(hipStream_t s, const float* in, float* out, int rows, int cols, const float* gamma,
                               float eps) {
    if (rows == 0 || cols == 0) return hipSuccess;
    hipLaunchKernelGGL(vk_rms_norm_f32, dim3(rows), dim3(256), 0, s, in, out, cols, gamma, eps);
    return hipGetLastError();
}

hipError_t launch_gelu_f32(hipStream_t s, const float* x, float* out, size_t n) {
    if (n == 0) return hipSuccess;
    const unsigned grid = (unsigned)std::min<size_t>((n + 255) / 256, 8192);
    hipLaunchKernelGGL(vk_gelu_f32, dim3(grid), dim3(256), 0, s, x, out, n);
    return hipGetLastError();
}

hipError_t launch_add_f32(hipStream_t s, const float* a, const float* b, float* out, size_t n) {
    if (n == 0) return hipSuccess;
    const unsigned grid = (unsigned)std::min<size_t>((n + 255) / 256, 8192);
    hipLaunchKernelGGL(vk_add_f32, dim3(grid), dim3(256), 0, s, a, b, out, n);
    return hipGetLastError();
}

hipError_t launch_embed_f32(hipStream_t s, const float* tok_emb, const float* pos_emb, const int* tokens,
                            const int* positions, int vocab, int n_pos, int d, int rows, float* out) {
    if (rows == 0) return hipSuccess;
    hipLaunchKernelGGL(vk_embed_f32, dim3(rows), dim3(256), 0, s, tok_emb, pos_emb, tokens, positions, vocab, n_pos,
                       d, out);
    return hipGetLastError();
}

hipError_t launch_argmax_f32(hipStream_t s, const float* logits, int rows, int cols, int* out) {
    if (rows == 0) return hipSuccess;
    hipLaunchKernelGGL(vk_argmax_f32, dim3(rows), dim3(256), 0, s, logits, cols, out);
    return hipGetLastError();
}

int argmax_n_slices(int cols) { return (cols + AM_SLICE - 1) / AM_SLICE; }

hipError_t launch_argmax_sliced(hipStream_t s, const float* logits, int rows, int cols, float2* part, int* out) {
    if (rows == 0) return hipSuccess;
    if (cols < 1 || rows > 65535) return hipErrorInvalidValue;  // grid.y limit
    const int n_sl = argmax_n_slices(cols);
    hipLaunchKernelGGL(vk_argmax_slices, dim3((unsigned)n_sl, (unsigned)rows), dim3(256), 0, s, logits, cols, n_sl,
                       part);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(vk_argmax_parts, dim3((unsigned)rows), dim3(256), 0, s, part, n_sl, out);
    return hipGetLastError();
}

int logits_n_vt(int vocab) { return (vocab + 16 * lg::J - 1) / (16 * lg::J); }

template <int NCT>
static void go_logits(hipStream_t s, const float* x, const float* emb, float* logits, float2* part, int n, int vocab,
                      int d, int n_vt) {
    const dim3 grid((unsigned)n_vt, (unsigned)((n + 16 * NCT - 1) / (16 * NCT)));
    const dim3 block(64 * lg::WAVES);  // the kernel's wave count sets its k split and LDS ring
    if (logits)
        hipLaunchKernelGGL((vk_logits_argmax<NCT, true>), grid, block, 0, s, x, emb, logits, part, n, vocab, d, n_vt);
    else
        hipLaunchKernelGGL((vk_logits_argmax<NCT, false>), grid, block, 0, s, x, emb, logits, part, n, vocab, d, n_vt);
}

hipError_t launch_logits_argmax(hipStream_t s, const float* x, const float* emb, float* logits, float2* part,
                                int* next, int n, int vocab, int d) {
    if (n == 0) return hipSuccess;
    // the kernel's loads assume whole 16-wide chunks per wave quarter and
    // 16-byte aligned rows
    if (vocab < 1 || d < logits_min_d() || d % logits_d_multiple() != 0) return hipErrorInvalidValue;
    // whole chunks per wave, and enough of them to fill the ring
    if (d % (16 * lg::WAVES) != 0 || d / (16 * lg::WAVES) < lg::NSLOT - 1) return hipErrorInvalidValue;
    const int n_vt = logits_n_vt(vocab);
    if ((n + 63) / 64 > 65535) return hipErrorInvalidValue;  // grid.y limit
    if (n <= 16) go_logits<1>(s, x, emb, logits, part, n, vocab, d, n_vt);
    else if (n <= 32) go_logits<2>(s, x, emb, logits, part, n, vocab, d, n_vt);
    else if (n <= 48) go_logits<3>(s, x, emb, logits, part, n, vocab, d, n_vt);
    else go_logits<4>(s, x, emb, logits, part, n, vocab, d, n_vt);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(vk_argmax_parts, dim3((unsigned)n), dim3(256), 0, s, part, n_vt, next);
    return hipGetLastError();
}

}  // namespace vk

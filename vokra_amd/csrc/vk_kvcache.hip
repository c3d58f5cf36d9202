// vk_kvcache.hip — the quantized paged KV cache resident in HBM, and decode
// attention over it, for gfx950.
//
// Semantics follow QuantizedPagedKvCache (crates/vokra-core/src/cache/
// paged_quant.rs:240-545) with one codebook:
//   * a page holds `bs` time steps of one layer for every stream; the page
//     table entry of (layer, t) is layer * pages_per_layer + t / bs (:414-415);
//   * pages come from a LIFO free list that starts as [cap-1 .. 0] (pop gives
//     0, 1, 2, ...), release pushes back in table order (:152-216, :500-515);
//   * each K / V row (n_head * d_head values) is stored as Q8_0 blocks of 32,
//     packed exactly as BlockQ8_0::pack (kv_quant/q8_0.rs:40-64), and reads
//     return q * f32(f16(d)) (:69-80).
// Device layout (this build's, numerics unaffected): quants and scales in
// separate arrays, so a head's row slice is one aligned vector load:
//   q: [cap][bs][n_stream][width] int8,  d: [cap][bs][n_stream][width/32] f16
// The table, the free list and the allocator state live in device memory and
// are only touched by kernels: an append batch allocates on the GPU.
#include "vk_common.h"
#include "vk_launch.h"

namespace vk {

// Set (to 1) by the GQA decode kernel when q * scale is outside the fp16
// range of its operands; read and cleared by the host (range_check in vk_capi.hip).
static __device__ unsigned int vk_kv_range_flag;

// Device view of one cache, passed by value to every kernel.
struct KvDev {
    int8_t* kq;
    int8_t* vq;
    uint16_t* kd;
    uint16_t* vd;
    int* table;      // [n_layer * ppl], -1 = no page
    int* free_list;  // stack of page ids, top at free_len - 1
    int* meta;       // [0] free_len, [1] status of the last append, [2] items appended, [3] scratch,
                     // [4 ..) per item of the last append: 1 = overwritten by a later item
    int n_layer, n_stream, width, row_blocks, bs, ppl, cap, max_time;
    int hd, nh, hb;  // head size, heads per row, 32-blocks per head
};

enum : int { KV_OK = 0, KV_INVALID = 5, KV_EXHAUSTED = 10 };  // vokra_hip_status_t values

// Page layout: a page holds bs time steps of every stream; inside it the
// head rows are ordered [stream][head][t % bs], so one head's keys of a page
// are contiguous (bs x hd quants, bs x hd/32 scales) for the attention reads.
// Head row index of (page, t, stream, head); its hd quants start at
// hrow * hd in kq / vq and its hd/32 f16 scales at hrow * hb in kd / vd.
__device__ __forceinline__ size_t kv_hrow(const KvDev& c, int pid, int t, int s, int h) {
    return (((size_t)pid * c.n_stream + s) * c.nh + h) * c.bs + (t % c.bs);
}
// Offsets of row element e (0 .. width-1) of (page, t, stream): quant, scale.
__device__ __forceinline__ size_t kv_qoff(const KvDev& c, int pid, int t, int s, int e) {
    return kv_hrow(c, pid, t, s, e / c.hd) * c.hd + (e % c.hd);
}
__device__ __forceinline__ size_t kv_doff(const KvDev& c, int pid, int t, int s, int e) {
    return kv_hrow(c, pid, t, s, e / c.hd) * c.hb + (e % c.hd) / 32;
}

// ---------------------------------------------------------------------------
// Allocation for one append batch: items i = 0..n-1 behave as append_step
// calls in order. Item i needs a new page when its table entry is empty and
// no earlier item of the batch maps to the same entry; the r-th such item
// pops free_list[free_len - 1 - r]. The first invalid or unservable item
// ends the batch (items before it are appended, it and later ones are not).
// One workgroup of 1024 threads; n <= 1024.
__global__ __launch_bounds__(1024) void vk_kv_alloc(KvDev c, int layer, int n, const int* __restrict__ streams,
                                                    const int* __restrict__ times) {
    __shared__ int s_ti[1024];
    __shared__ int s_key[1024];
    __shared__ int s_scan[1024];
    __shared__ int s_fail;
    const int i = threadIdx.x;
    int s = 0, t = 0, ti = -1;
    bool valid = false;
    if (i < n) {
        s = streams[i];
        t = times[i];
        valid = layer >= 0 && layer < c.n_layer && s >= 0 && s < c.n_stream && t >= 0 && t < c.max_time;
        ti = valid ? layer * c.ppl + t / c.bs : -1;
    }
    if (i == 0) s_fail = n;
    s_ti[i] = ti;
    s_key[i] = valid ? s * c.max_time + t : -1 - i;  // distinct for invalid items
    __syncthreads();
    bool first = false;
    if (valid && c.table[ti] < 0) {
        first = true;
        for (int j = 0; j < i; ++j)
            if (s_ti[j] == ti) {
                first = false;
                break;
            }
    }
    // inclusive scan of `first` (Hillis-Steele over the block; the block is
    // the smallest power of two >= n, at least one wave)
    s_scan[i] = first ? 1 : 0;
    __syncthreads();
    for (int off = 1; off < (int)blockDim.x; off <<= 1) {
        const int v = i >= off ? s_scan[i - off] : 0;
        __syncthreads();
        s_scan[i] += v;
        __syncthreads();
    }
    const int free_len = c.meta[0];
    const int rank = s_scan[i] - (first ? 1 : 0);
    const bool fail = i < n && (!valid || (first && rank >= free_len));
    if (fail) atomicMin(&s_fail, i);
    __syncthreads();
    const int f = s_fail;
    if (first && i < f) c.table[ti] = c.free_list[free_len - 1 - rank];
    // a later item of the batch writing the same slot wins, as with
    // successive append_step calls
    if (i < n) {
        int over = 0;
        for (int j = i + 1; j < f; ++j)
            if (s_key[j] == s_key[i]) {
                over = 1;
                break;
            }
        c.meta[4 + i] = over;
    }
    if (i == 0) {
        const int used = f > 0 ? s_scan[f - 1] : 0;
        int status = KV_OK;
        if (f < n) {
            const int sf = streams[f], tf = times[f];
            const bool vf = layer >= 0 && layer < c.n_layer && sf >= 0 && sf < c.n_stream && tf >= 0 &&
                            tf < c.max_time;
            status = vf ? KV_EXHAUSTED : KV_INVALID;
        }
        c.meta[0] = free_len - used;
        c.meta[1] = status;
        c.meta[2] = f;
    }
}

// Allocation for the same items appended to layers layer0 .. layer0+nl-1 in
// that order (item q = l * n + i, as n append_step calls per layer, layer
// after layer), in one launch: the r-th item whose table entry is empty and
// which is the first of its layer's batch with that entry pops
// free_list[free_len - 1 - r]; the first invalid or unservable item ends the
// batch. Writes the table, free_len, the status and the appended count
// (meta[2], in items q); no per-item overwrite flags (its caller appends
// distinct streams). One workgroup of 1024 threads; nl * n <= 4096.
// q_base > 0 continues a batch split over several launches (q_base items
// before this one): a launch after a failed one allocates nothing and keeps
// the first failure's status and count.
__global__ __launch_bounds__(1024) void vk_kv_alloc_layers(KvDev c, int layer0, int nl, int n, int q_base,
                                                           const int* __restrict__ streams,
                                                           const int* __restrict__ times) {
    constexpr int QMAX = 4096, U = QMAX / 1024;
    __shared__ int s_ti[QMAX];
    __shared__ int s_rank[QMAX];
    __shared__ int s_scan[1024];
    __shared__ int s_bad, s_total;
    const int tid = threadIdx.x, N = nl * n;
    if (q_base > 0 && c.meta[1] != KV_OK) return;  // uniform: one value for the whole workgroup
    bool valid[U], first[U];
    int ti[U];
    if (tid == 0) { s_bad = N; s_total = 0; }
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int q = 1024 * u + tid;
        valid[u] = false;
        ti[u] = -1;
        if (q < N) {
            const int l = layer0 + q / n, i = q % n;
            const int s = streams[i], t = times[i];
            valid[u] = l >= 0 && l < c.n_layer && s >= 0 && s < c.n_stream && t >= 0 && t < c.max_time;
            ti[u] = valid[u] ? l * c.ppl + t / c.bs : -1;
            s_ti[q] = ti[u];
        }
    }
    __syncthreads();
    const int free_len = c.meta[0];
    int base = 0;  // first-flags of earlier chunks
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int q = 1024 * u + tid;
        first[u] = false;
        if (valid[u] && c.table[ti[u]] < 0) {
            first[u] = true;
            for (int j = q - q % n; j < q; ++j)  // earlier items of the same layer
                if (s_ti[j] == ti[u]) {
                    first[u] = false;
                    break;
                }
        }
        // inclusive scan of this chunk's flags (Hillis-Steele)
        s_scan[tid] = first[u] ? 1 : 0;
        __syncthreads();
        for (int off = 1; off < 1024; off <<= 1) {
            const int v = tid >= off ? s_scan[tid - off] : 0;
            __syncthreads();
            s_scan[tid] += v;
            __syncthreads();
        }
        const int rank = base + s_scan[tid] - (first[u] ? 1 : 0);
        if (q < N && (!valid[u] || (first[u] && rank >= free_len))) atomicMin(&s_bad, q);
        if (q < N) s_rank[q] = rank;
        base += s_scan[1023];
        __syncthreads();
    }
    const int bad = s_bad;
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int q = 1024 * u + tid;
        if (first[u] && q < bad) {
            c.table[ti[u]] = c.free_list[free_len - 1 - s_rank[q]];
            atomicAdd(&s_total, 1);
        }
    }
    __syncthreads();
    if (tid == 0) {
        int status = KV_OK;
        if (bad < N) {
            const int i = bad % n, l = layer0 + bad / n, sf = streams[i], tf = times[i];
            const bool vf = l >= 0 && l < c.n_layer && sf >= 0 && sf < c.n_stream && tf >= 0 && tf < c.max_time;
            status = vf ? KV_EXHAUSTED : KV_INVALID;
        }
        c.meta[0] = free_len - s_total;
        c.meta[1] = status;
        c.meta[2] = q_base + bad;
    }
}

// Packs the K and V rows of the appended items into their slots. One thread
// per (item, 32-element block, element); 32 consecutive threads form a block.
// Same arithmetic as BlockQ8_0::pack: amax = max |x|, d = amax / 127,
// q = round(clamp(x * (1/d), -127, 127)), scale stored as f16(d).
__device__ __forceinline__ void q8_0_pack_lane(float v, int lane32, int8_t* q, uint16_t* d) {
    const float amax = vk_group_max<32>(fmaxf(0.0f, fabsf(v)));  // NaN -> 0, as the fold from 0.0
    const float dd = amax == 0.0f ? 0.0f : amax / 127.0f;
    const float inv = dd == 0.0f ? 0.0f : 1.0f / dd;
    const float sc = v * inv;
    const float cl = sc != sc ? sc : fminf(fmaxf(sc, -127.0f), 127.0f);
    *q = (int8_t)((cl != cl) ? 0 : (int)roundf(cl));
    if (lane32 == 0) *d = (uint16_t)vk_f32_to_f16_bits(dd);
}

__global__ void vk_kv_write(KvDev c, int layer, int n, const int* __restrict__ streams,
                            const int* __restrict__ times, const float* __restrict__ k, const float* __restrict__ v) {
    const size_t gid = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int e = (int)(gid % (size_t)c.width);
    const int item = (int)(gid / (size_t)c.width);
    // `live` is uniform over each 32-thread block group (width % 32 == 0)
    const bool live = item < n && item < c.meta[2] && c.meta[4 + min(item, 1023)] == 0;
    float kv = 0.0f, vv = 0.0f;
    int s = 0, t = 0;
    if (live) {
        s = streams[item];
        t = times[item];
        kv = k[(size_t)item * c.width + e];
        vv = v[(size_t)item * c.width + e];
    }
    int8_t qk, qv;
    uint16_t dk = 0, dv = 0;
    q8_0_pack_lane(kv, e & 31, &qk, &dk);
    q8_0_pack_lane(vv, e & 31, &qv, &dv);
    if (!live) return;
    const int pid = c.table[layer * c.ppl + t / c.bs];
    const size_t qo = kv_qoff(c, pid, t, s, e);
    c.kq[qo] = qk;
    c.vq[qo] = qv;
    if ((e & 31) == 0) {
        const size_t dof = kv_doff(c, pid, t, s, e);
        c.kd[dof] = dk;
        c.vd[dof] = dv;
    }
}

// Packs item i's K and V rows (width floats each) at time times[i] into the
// page that an earlier vk_kv_alloc_layers launch gave (layer, times[i] /
// block_size); items whose entry is empty (allocation failed) or out of range
// are skipped. Same packing as vk_kv_write. One thread per (item, element).
// rope_cs (optional): [n][hd / 2] (cos, sin) of each item's position; k is
// then rotated (head size hd) on the way into the cache, as a RoPE pass over
// k before the write would leave it.
__global__ void vk_kv_write_allocated(KvDev c, int layer, int n, const int* __restrict__ streams,
                                      const int* __restrict__ times, const float* __restrict__ k,
                                      const float* __restrict__ v, const float2* __restrict__ rope_cs, int hd) {
    const size_t gid = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int e = (int)(gid % (size_t)c.width);
    const int item = (int)(gid / (size_t)c.width);
    bool live = false;
    int s = 0, t = 0, pid = -1;
    if (item < n) {  // uniform over each 32-thread block group (width % 32 == 0)
        s = streams[item];
        t = times[item];
        if (s >= 0 && s < c.n_stream && t >= 0 && t < c.max_time) {
            pid = c.table[layer * c.ppl + t / c.bs];
            live = pid >= 0;
        }
    }
    float kv = 0.0f, vv = 0.0f;
    if (live) {
        kv = k[(size_t)item * c.width + e];
        vv = v[(size_t)item * c.width + e];
        if (rope_cs) {
            const int half = hd >> 1, j = e % hd, jj = j % half;
            const float2 cs = rope_cs[(size_t)item * half + jj];
            if (j < half) kv = vk_rope_lo(kv, k[(size_t)item * c.width + e + half], cs);
            else kv = vk_rope_hi(k[(size_t)item * c.width + e - half], kv, cs);
        }
    }
    int8_t qk, qv;
    uint16_t dk = 0, dv = 0;
    q8_0_pack_lane(kv, e & 31, &qk, &dk);
    q8_0_pack_lane(vv, e & 31, &qv, &dv);
    if (!live) return;
    const size_t qo = kv_qoff(c, pid, t, s, e);
    c.kq[qo] = qk;
    c.vq[qo] = qv;
    if ((e & 31) == 0) {
        const size_t dof = kv_doff(c, pid, t, s, e);
        c.kd[dof] = dk;
        c.vd[dof] = dv;
    }
}

// read_step (paged_quant.rs:448-480): dequantized K and V rows of (layer, t, s)
// into out[0 .. width) and out[width .. 2 width); found[0] = 0 when the entry
// has no page (the reference's None).
__global__ void vk_kv_read(KvDev c, int layer, int t, int s, float* __restrict__ out, int* __restrict__ found) {
    const int pid = c.table[layer * c.ppl + t / c.bs];
    const int e = blockIdx.x * blockDim.x + threadIdx.x;
    if (e == 0) found[0] = pid >= 0 ? 1 : 0;
    if (pid < 0 || e >= c.width) return;
    const size_t qo = kv_qoff(c, pid, t, s, e), dof = kv_doff(c, pid, t, s, e);
    out[e] = (float)c.kq[qo] * vk_f16_to_f32(c.kd[dof]);
    out[c.width + e] = (float)c.vq[qo] * vk_f16_to_f32(c.vd[dof]);
}

// release_layer (paged_quant.rs:500-515): entries of `layer` in table order
// push their pages; meta[3] keeps the old free_len so the zeroing kernel
// finds the released pages at free_list[meta[3] .. meta[0]).
__global__ __launch_bounds__(1024) void vk_kv_release(KvDev c, int layer) {
    __shared__ int s_scan[1024];
    __shared__ int s_base;
    const int i = threadIdx.x;
    if (i == 0) {
        s_base = c.meta[0];
        c.meta[3] = c.meta[0];
    }
    __syncthreads();
    for (int p0 = 0; p0 < c.ppl; p0 += 1024) {
        const int p = p0 + i;
        const int ti = layer * c.ppl + p;
        const int pid = p < c.ppl ? c.table[ti] : -1;
        s_scan[i] = pid >= 0 ? 1 : 0;
        __syncthreads();
        for (int off = 1; off < 1024; off <<= 1) {
            const int v = i >= off ? s_scan[i - off] : 0;
            __syncthreads();
            s_scan[i] += v;
            __syncthreads();
        }
        if (pid >= 0) {
            c.free_list[s_base + s_scan[i] - 1] = pid;
            c.table[ti] = -1;
        }
        __syncthreads();
        if (i == 0) s_base += s_scan[1023];
        __syncthreads();
    }
    if (i == 0) c.meta[0] = s_base;
}

// Zeroes the pages at free_list[meta[3] .. meta[0]) (the ones just released).
__global__ void vk_kv_zero_released(KvDev c) {
    const int lo = c.meta[3], hi = c.meta[0];
    const size_t qpage = (size_t)c.bs * c.n_stream * c.width;
    const size_t dpage = (size_t)c.bs * c.n_stream * c.row_blocks;
    for (int r = lo + blockIdx.y; r < hi; r += gridDim.y) {
        const int pid = c.free_list[r];
        for (size_t x = (size_t)blockIdx.x * blockDim.x + threadIdx.x; x < qpage; x += (size_t)gridDim.x * blockDim.x) {
            c.kq[(size_t)pid * qpage + x] = 0;
            c.vq[(size_t)pid * qpage + x] = 0;
            if (x < dpage) {
                c.kd[(size_t)pid * dpage + x] = 0;
                c.vd[(size_t)pid * dpage + x] = 0;
            }
        }
    }
}

// reset (paged_quant.rs:489-493): empty table, free list [cap-1 .. 0] (or a
// caller-given order), status cleared. Page memory is cleared by fill kernels.
__global__ void vk_kv_reset_meta(KvDev c, const int* __restrict__ order) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < c.n_layer * c.ppl) c.table[i] = -1;
    if (i < c.cap) c.free_list[i] = order ? order[i] : c.cap - 1 - i;
    if (i == 0) {
        c.meta[0] = c.cap;
        c.meta[1] = KV_OK;
        c.meta[2] = 0;
        c.meta[3] = c.cap;
    }
}

__global__ void vk_fill_u32(uint32_t* __restrict__ p, size_t n, uint32_t v) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) p[i] = v;
}

__global__ void vk_kv_page_of(KvDev c, int layer, int t, int* __restrict__ out) {
    out[0] = c.table[layer * c.ppl + t / c.bs];
    out[1] = c.meta[0];
}

// ---------------------------------------------------------------------------
// Decode attention over the cache. For item i (stream s_i, keys 0..len_i-1)
// and query head h (kv head h / G):
//   s_j = (q_h * scale) . k_j,  p = softmax(s),  out_h = sum_j p_j v_j
// with k_j, v_j the cache's dequantized rows (head slice). One workgroup per
// (key split, kv head, item) handles the G query heads sharing the kv head;
// keys go in chunks of 256 (one per thread for the scores). With several
// splits, each writes (m, l, O) partials that vk_paged_attn_combine merges.
namespace pa {
constexpr int CH = 256;
constexpr int KPS = 512, MAX_SPLIT = 8;  // keys per split grow by KPS so an item never has more than 8
}

// Key split of one item, a function of its length only (never of the batch
// or of the grid): splits of pa_kps(len) keys, pa_splits(len) <= 8 of them.
// An item's results therefore do not depend on what else is in the launch.
__host__ __device__ __forceinline__ int pa_kps(int len) {
    return pa::KPS * (len > 0 ? (len + pa::KPS * pa::MAX_SPLIT - 1) / (pa::KPS * pa::MAX_SPLIT) : 1);
}
__host__ __device__ __forceinline__ int pa_splits(int len) {
    const int k = pa_kps(len);
    return len > k ? (len + k - 1) / k : 1;
}

// Fused append: the workgroup whose key range [k0, k1) holds the item's new
// time step packs that step's K and V head slices into the cache first,
// exactly as vk_kv_write would, then reads them back with the other keys. The
// page comes from an earlier allocation launch. Called by every thread of the
// workgroup (its barrier is uniform per workgroup).
template <int HD>
__device__ __forceinline__ void pa_append_slice(const KvDev& c, int layer, int s, int hk, int item, int k0, int k1,
                                                const float* __restrict__ ak, const float* __restrict__ av,
                                                const int* __restrict__ at, int wave, int lane) {
    constexpr int NB = HD / 32;
    const int t = at[item];
    if (t < k0 || t >= k1) return;
    const int pid = c.table[layer * c.ppl + t / c.bs];
    if (pid >= 0 && wave < 2) {
        const size_t hr = kv_hrow(c, pid, t, s, hk);
        const float* src = (wave == 0 ? ak : av) + (size_t)item * c.width + (size_t)hk * HD;
        int8_t* dq = (wave == 0 ? c.kq : c.vq) + hr * HD;
        uint16_t* dd = (wave == 0 ? c.kd : c.vd) + hr * NB;
#pragma unroll
        for (int e = lane; e < HD; e += 64) {
            int8_t qb;
            uint16_t db = 0;
            q8_0_pack_lane(src[e], e & 31, &qb, &db);
            dq[e] = qb;
            if ((e & 31) == 0) dd[e >> 5] = db;
        }
    }
    __threadfence_block();
    __syncthreads();
}

// The activation pass over one output row element (row = item, width hq * HD,
// column h * HD + e) for the kernels that write the attention output
// directly: a 32-wide block is one half-wave, so the calling wave's lanes
// must hold 64 consecutive columns.
__device__ __forceinline__ void pa_quantize_out(const VkQOut& qo, int item, int col, float val) {
    const float amax = vk_group_max<32>(fmaxf(0.0f, fabsf(val)));
    float sc = 0.0f;
    int qv = 0;
    if (amax != 0.0f) {
        sc = vk_act_scale(amax, qo.pow2);
        qv = vk_act_q(val, sc);
    }
    const int gs = vk_group_sum_i<32>(qv);
    const int kb = col >> 5;
    reinterpret_cast<uint16_t*>(qo.afrag)[vk_afrag_u16((size_t)item, kb, qo.k >> 5, col & 31)] =
        (uint16_t)vk_act_bits(qv, sc, qo.pow2);
    if ((col & 31) == 0) {
        qo.ascale[(size_t)kb * qo.m_pad + item] = sc;
        qo.asum[(size_t)kb * qo.m_pad + item] = qo.pow2 ? (float)gs * sc : (float)gs;
    }
}

template <int HD, int G>
__global__ __launch_bounds__(256) void vk_paged_attn(KvDev c, int layer, const int* __restrict__ streams,
                                                     const int* __restrict__ lens, const float* __restrict__ q,
                                                     float scale, int hq, int n_split,
                                                     float* __restrict__ out, float* __restrict__ part_ml,
                                                     float* __restrict__ part_o, const VkQOut qo,
                                                     const float* __restrict__ ak, const float* __restrict__ av,
                                                     const int* __restrict__ at) {
    constexpr int NB = HD / 32;            // blocks per head slice
    constexpr int NO = G * HD;             // outputs of the workgroup
    // P.V work unit: a quad of 4 consecutive outputs of one head (one 32-bit
    // LDS read of V quants feeds 4 FMAs; the quad shares its block's scale)
    constexpr int NQ = NO / 4;
    constexpr int OPT = NQ >= 256 ? NQ / 256 : 1;    // quads per thread
    constexpr int TPO = NQ >= 256 ? 1 : 256 / NQ;    // threads per quad
    __shared__ __align__(16) float lq[G][HD];
    __shared__ float lpd[G][pa::CH][NB];         // p_j * d_{j,b} for the V product
    __shared__ float lalpha[G];                  // chunk rescale factors (uniform)
    __shared__ float lml[G][2];                  // final (m, l) per head
    __shared__ __align__(16) int8_t lv[pa::CH][HD];  // V quants of the chunk
    __shared__ float red[G][8];
    __shared__ __align__(16) float lpart[256 * OPT][4];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int split = blockIdx.x, hk = blockIdx.y, item = blockIdx.z;
    const int s = streams[item];
    const int len = min(lens[item], c.max_time);
    const int kps = pa_kps(len), nsp = pa_splits(len);
    if (split >= nsp) return;  // uniform per workgroup, before any barrier
    const int k0 = split * kps, k1 = min(len, k0 + kps);

    if (ak) pa_append_slice<HD>(c, layer, s, hk, item, k0, k1, ak, av, at, wave, lane);
    for (int x = tid; x < G * HD; x += 256) {
        const int g = x / HD, e = x % HD;
        lq[g][e] = q[((size_t)item * hq + hk * G + g) * HD + e] * scale;
    }
    float m_run[G], l_run[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        m_run[g] = -INFINITY;
        l_run[g] = 0.0f;
    }
    float o_acc[OPT][4];
#pragma unroll
    for (int u = 0; u < OPT; ++u)
#pragma unroll
        for (int i = 0; i < 4; ++i) o_acc[u][i] = 0.0f;
    __syncthreads();

    // the page-table entry of this thread's key in the next chunk is read
    // while the current chunk computes (a split of two chunks: three memory
    // round trips, not four)
    int pid_next = c.table[layer * c.ppl + min(k0 + tid, k1 - 1) / c.bs];
    for (int j0 = k0; j0 < k1; j0 += pa::CH) {
        // ---- scores: thread = key
        const int j = j0 + tid;
        const bool kv_ok = j < k1;
        const int jt = kv_ok ? j : k0;
        int pid = pid_next;
        pid_next = c.table[layer * c.ppl + min(j0 + pa::CH + tid, k1 - 1) / c.bs];
        const bool has = kv_ok && pid >= 0;
        pid = max(pid, 0);
        const size_t hr = kv_hrow(c, pid, jt, s, hk);
        const uint16_t* kds = c.kd + hr * NB;
        const uint16_t* vds = c.vd + hr * NB;
        float sc[G];
#pragma unroll
        for (int g = 0; g < G; ++g) sc[g] = 0.0f;
        const uint4* kr = reinterpret_cast<const uint4*>(c.kq + hr * HD);
        const uint4* vr = reinterpret_cast<const uint4*>(c.vq + hr * HD);
        float dv[NB];
        if constexpr (G == 1) {
            // one head: every load of the key's row is issued before any is
            // used (one memory round trip after the page-table lookup)
            uint4 kw[NB][2], vw[NB][2];
            uint16_t kd16[NB], vd16[NB];
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                kw[b][0] = kr[2 * b];
                kw[b][1] = kr[2 * b + 1];
                vw[b][0] = vr[2 * b];
                vw[b][1] = vr[2 * b + 1];
                kd16[b] = kds[b];
                vd16[b] = vds[b];
            }
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                const float d = vk_f16_to_f32_hw(kd16[b]);
                const uint32_t w[8] = {kw[b][0].x, kw[b][0].y, kw[b][0].z, kw[b][0].w,
                                       kw[b][1].x, kw[b][1].y, kw[b][1].z, kw[b][1].w};
                const float4* qg = reinterpret_cast<const float4*>(&lq[0][32 * b]);
                float a = sc[0];
#pragma unroll
                for (int x4 = 0; x4 < 8; ++x4) {
                    const float4 q4 = qg[x4];
                    const uint32_t wx = w[x4];
                    a = fmaf(q4.x, (float)(int8_t)(wx & 0xff) * d, a);
                    a = fmaf(q4.y, (float)(int8_t)((wx >> 8) & 0xff) * d, a);
                    a = fmaf(q4.z, (float)(int8_t)((wx >> 16) & 0xff) * d, a);
                    a = fmaf(q4.w, (float)(int8_t)(wx >> 24) * d, a);
                }
                sc[0] = a;
                *reinterpret_cast<uint4*>(&lv[tid][32 * b]) = vw[b][0];
                *reinterpret_cast<uint4*>(&lv[tid][32 * b + 16]) = vw[b][1];
                dv[b] = has ? vk_f16_to_f32_hw(vd16[b]) : 0.0f;
            }
        } else {
#pragma unroll 1
            for (int b = 0; b < NB; ++b) {
                const float d = vk_f16_to_f32_hw(kds[b]);
                const uint4 w0 = kr[2 * b], w1 = kr[2 * b + 1];
                const uint32_t w[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
                float kf[32];  // the block's dequantized keys (exact products)
#pragma unroll
                for (int x = 0; x < 32; ++x) kf[x] = (float)(int8_t)((w[x >> 2] >> (8 * (x & 3))) & 0xff) * d;
#pragma unroll
                for (int g = 0; g < G; ++g) {
                    const float4* qg = reinterpret_cast<const float4*>(&lq[g][32 * b]);
                    float a = sc[g];
#pragma unroll 2
                    for (int x4 = 0; x4 < 8; ++x4) {
                        const float4 q4 = qg[x4];
                        a = fmaf(q4.x, kf[4 * x4], a);
                        a = fmaf(q4.y, kf[4 * x4 + 1], a);
                        a = fmaf(q4.z, kf[4 * x4 + 2], a);
                        a = fmaf(q4.w, kf[4 * x4 + 3], a);
                    }
                    sc[g] = a;
                }
                // stage V quants and its scale product for the P.V pass
                const uint4 v0 = vr[2 * b], v1 = vr[2 * b + 1];
                *reinterpret_cast<uint4*>(&lv[tid][32 * b]) = v0;
                *reinterpret_cast<uint4*>(&lv[tid][32 * b + 16]) = v1;
            }
#pragma unroll
            for (int b = 0; b < NB; ++b)
                dv[b] = has ? vk_f16_to_f32_hw(vds[b]) : 0.0f;
        }
        // ---- chunk max per head
#pragma unroll
        for (int g = 0; g < G; ++g) {
            sc[g] = has ? sc[g] : -INFINITY;
            const float mx = vk_group_maxf<64>(sc[g]);
            if (lane == 0) red[g][wave] = mx;
        }
        __syncthreads();
        float alpha[G];
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const float mx = fmaxf(fmaxf(red[g][0], red[g][1]), fmaxf(red[g][2], red[g][3]));
            const float m_new = fmaxf(m_run[g], mx);
            const float m_use = m_new == -INFINITY ? 0.0f : m_new;
            alpha[g] = __expf(m_run[g] - m_use);
            const float p = __expf(sc[g] - m_use);
            if (tid == 0) lalpha[g] = alpha[g];
#pragma unroll
            for (int b = 0; b < NB; ++b) lpd[g][tid][b] = p * dv[b];
            const float ps = vk_group_sumf<64>(p);
            if (lane == 0) red[g][4 + wave] = ps;
            m_run[g] = m_new;
        }
        __syncthreads();
#pragma unroll
        for (int g = 0; g < G; ++g) l_run[g] = l_run[g] * alpha[g] + ((red[g][4] + red[g][5]) + (red[g][6] + red[g][7]));
        // ---- O += P . V: quad oq = (g, e0..e0+3); TPO threads share a quad
        const int nk = min(pa::CH, k1 - j0);
#pragma unroll
        for (int u = 0; u < OPT; ++u) {
            const int oq = NQ >= 256 ? tid + 256 * u : tid / TPO;
            const int part = NQ >= 256 ? 0 : tid % TPO;
            const int g = (4 * oq) / HD, e0 = (4 * oq) % HD;
            float a[4] = {0.0f, 0.0f, 0.0f, 0.0f};
            for (int jj = part; jj < nk; jj += TPO) {
                const uint32_t w = *reinterpret_cast<const uint32_t*>(&lv[jj][e0]);
                const float pd = lpd[g][jj][e0 >> 5];
#pragma unroll
                for (int i = 0; i < 4; ++i) a[i] = fmaf(pd, (float)(int8_t)((w >> (8 * i)) & 0xffu), a[i]);
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) o_acc[u][i] = o_acc[u][i] * lalpha[g] + a[i];
        }
        __syncthreads();
    }
    // ---- reduce the TPO partials of each quad (fixed order), then write
#pragma unroll
    for (int u = 0; u < OPT; ++u)
#pragma unroll
        for (int i = 0; i < 4; ++i) lpart[tid + 256 * u][i] = o_acc[u][i];
    if (tid == 0)
#pragma unroll
        for (int g = 0; g < G; ++g) {
            lml[g][0] = m_run[g];
            lml[g][1] = l_run[g];
        }
    __syncthreads();
    for (int o = tid; o < NO; o += 256) {
        const int g = o / HD, e = o % HD, oq = o >> 2, i = o & 3;
        float a = 0.0f;
        if (NQ >= 256) {
            a = lpart[(oq % 256) + 256 * (oq / 256)][i];
        } else {
            for (int r = 0; r < TPO; ++r) a += lpart[oq * TPO + r][i];
        }
        const int h = hk * G + g;
        if (nsp == 1) {
            const float inv = lml[g][1] > 0.0f ? 1.0f / lml[g][1] : 0.0f;
            const float val = a * inv;
            out[((size_t)item * hq + h) * HD + e] = val;
            if (qo.afrag) pa_quantize_out(qo, item, h * HD + e, val);  // NO is a multiple of 64
        } else {
            const size_t pi = ((size_t)item * hq + h) * n_split + split;
            part_o[pi * HD + e] = a;
            if (e == 0) {
                part_ml[2 * pi] = lml[g][0];
                part_ml[2 * pi + 1] = lml[g][1];
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Decode attention with one query head per kv head and head_dim 64 (Whisper's
// self-attention). Same grid, key splits, outputs, partials and fused passes
// as vk_paged_attn<64, 1>, but the keys of a split are shared among the four
// waves rather than the threads of the workgroup: wave w takes the 64-key
// tiles w, w + 4, ... and keeps its own online softmax, so no barrier runs in
// the key loop; the four (m, l, O) states merge in wave order at the end.
// Per tile, in four passes of 16 keys:
//   scores, a quad of lanes per key (lane 4 k + u holds dims 16 u .. 16 u + 15
//     of key k of the pass): s = scale * sum_u d_{b(u)} * (sum_{e in quarter
//     u} q_e k_e), each quarter's dot taken exactly in integers (q as 22-bit
//     integers in three int8 digits against the int8 quants, v_dot4) and
//     scaled back in f32, each block's f16 scale applied to its quarter sums
//     (f32-level numerics, as the matrix-core kernel's); the quad adds its
//     four terms in a fixed butterfly, so its lanes agree bit for bit;
//   O += P . V, lane = (dims 4 dq .. 4 dq + 3, keys kg, kg + 4, ..): the V
//     quants reach the wave's own LDS copy of the tile, [key][64 B], by direct
//     global-to-LDS loads (one per pass, 1 KB of consecutive 16-byte chunks),
//     and the 64 lanes of one read cover four consecutive rows (no bank
//     conflicts), with p * d_v per key and block beside it.
namespace pw {
constexpr int HD = 64, NB = HD / 32, KT = 64, WAVES = 4, DQ = HD / 4, KG = 64 / DQ, KPL = KT / KG;
constexpr int PASS = 4, KPP = KT / PASS;  // passes per tile, keys per pass (a quad of lanes each)
}
// Sum over the 16 quads of a wave whose four lanes hold equal values (xor
// steps 4 .. 32 only; the mirrors of vk_bfly_partner are exact on such input).
__device__ __forceinline__ float pw_quad_group_sumf(float v) {
    v += __int_as_float(vk_bfly_partner<4>(__float_as_int(v)));
    v += __int_as_float(vk_bfly_partner<8>(__float_as_int(v)));
    v += __int_as_float(vk_bfly_partner<16>(__float_as_int(v)));
    v += __int_as_float(vk_bfly_partner<32>(__float_as_int(v)));
    return v;
}
__global__ __launch_bounds__(256, 5) void vk_paged_attn_w64(KvDev c, int layer, const int* __restrict__ streams,
                                                         const int* __restrict__ lens, const float* __restrict__ q,
                                                         float scale, int hq, int n_split, float* __restrict__ out,
                                                         float* __restrict__ part_ml, float* __restrict__ part_o,
                                                         const VkQOut qo, const float* __restrict__ ak,
                                                         const float* __restrict__ av, const int* __restrict__ at) {
    using namespace pw;
    __shared__ __align__(16) int8_t lv[WAVES][KT][HD];
    __shared__ __align__(16) float lpd[WAVES][KT][NB];
    __shared__ __align__(16) float lpo[WAVES][KG][HD];
    __shared__ float lml[WAVES][2];
    __shared__ __align__(16) int8_t lqd[WAVES][3][HD];  // q's integer digits
    __shared__ float2 lqs[WAVES][HD / 16];              // per quarter: 2^(ex - 22), qbad

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int split = blockIdx.x, hk = blockIdx.y, item = blockIdx.z;
    const int s = streams[item];
    const int len = min(lens[item], c.max_time);
    const int kps = pa_kps(len), nsp = pa_splits(len);
    if (split >= nsp) return;  // uniform per workgroup, before any barrier
    const int k0 = split * kps, k1 = min(len, k0 + kps);
    if (ak) pa_append_slice<HD>(c, layer, s, hk, item, k0, k1, ak, av, at, wave, lane);

    const int ku = lane >> 2, u = lane & 3, ub = u >> 1;  // score passes: key of the pass, quarter, block
    // head rows (kv_hrow) in 32 bits: the launcher checks that every slot
    // index fits and that the page size is a power of two
    const int bsh = __builtin_ctz(c.bs), bsm = c.bs - 1;
    // (through readfirstlane, so that the compiler keeps one 24-bit multiply
    // per key instead of refactoring it back into kv_hrow's three; the
    // launcher checks that both factors fit 24 bits)
    const uint32_t rows_pp = __builtin_amdgcn_readfirstlane((uint32_t)c.n_stream * c.nh * c.bs);
    const uint32_t row0 = __builtin_amdgcn_readfirstlane(((uint32_t)s * c.nh + hk) * c.bs);
    const int* tab = c.table + layer * c.ppl;
    const uint32_t lv_base = vk_lds_addr(&lv[wave][0][0]);
    const int8_t* kq_l = c.kq + 16 * u;  // the lane's 16-byte chunk of a head row
    const int8_t* vq_l = c.vq + 16 * u;
    const uint16_t* kd_l = c.kd + ub;    // and its block's scale
    const uint16_t* vd_l = c.vd + ub;
    const int nt = (k1 - k0 + KT - 1) / KT;

    // A tile's loads in two steps: the page entries of its keys, then its rows.
    int jt[PASS], pid[PASS];
    bool has[PASS];
    auto load_table = [&](int t) {
        const int j0 = k0 + t * KT;
#pragma unroll
        for (int p = 0; p < PASS; ++p) {
            const int j = j0 + KPP * p + ku;
            has[p] = j < k1;
            jt[p] = has[p] ? j : k0;
            pid[p] = tab[jt[p] >> bsh];
        }
    };
    uint4 kw[PASS];
    uint32_t kd[PASS], vd[PASS];
    bool hv[PASS];
    auto load_rows = [&]() {
#pragma unroll
        for (int p = 0; p < PASS; ++p) {
            hv[p] = has[p] && pid[p] >= 0;
            const uint64_t hr = __umul24((uint32_t)max(pid[p], 0), rows_pp) + row0 + (uint32_t)(jt[p] & bsm);
            // lane 4 k + u's 16 bytes of V land at row KPP p + k, chunk u, of the wave's copy
            vk_dma_b128(vq_l + hr * HD, lv_base + p * KPP * HD);
            kw[p] = *reinterpret_cast<const uint4*>(kq_l + hr * HD);
            kd[p] = kd_l[hr * NB];
            vd[p] = vd_l[hr * NB];
        }
    };

    // q as integers Q = q * 2^(22 - ex) per quarter u (|Q| <= 2^22, ex from
    // the quarter's largest |q|, clamped so that 2^(ex - 22) and its inverse
    // stay normal), split into three signed bytes Q = 2^16 D2 + 2^8 D1 + D0:
    // each quarter's block dot then runs as exact integer dot4 products of
    // the digits with the int8 key quants, and sum_e q_e k_e =
    // 2^(ex - 22) (2^16 S2 + 2^8 S1 + S0) to f32 rounding. qbad is 0, or NaN
    // when a q value of the quarter is not finite (it then reaches the
    // scores, as the f32 products would carry it). Each wave converts one
    // value per lane and regroups the digits through its own LDS rows.
    uint32_t qd[3][4];
    float qsc, qbad;
    {
        const float v = q[((size_t)item * hq + hk) * HD + lane];
        const float m = vk_group_max<16>(fmaxf(0.0f, fabsf(v)));  // a quarter is 16 lanes
        const float bad = vk_group_sumf<16>(0.0f * v);
        int ex = -100;
        if (m > 0.0f && m <= 3.40282347e38f) {
            frexpf(m, &ex);  // m < 2^ex
            ex = max(ex, -100);
        }
        const float x = v * ldexpf(1.0f, 22 - ex);
        const int qi = (x == x && fabsf(x) <= 4194304.0f) ? (int)rintf(x) : 0;
        const int b0 = (int)(int8_t)(qi & 0xff), r1 = (qi - b0) >> 8;
        const int b1 = (int)(int8_t)(r1 & 0xff), b2 = (r1 - b1) >> 8;
        lqd[wave][0][lane] = (int8_t)b0;
        lqd[wave][1][lane] = (int8_t)b1;
        lqd[wave][2][lane] = (int8_t)b2;
        if ((lane & 15) == 0) lqs[wave][lane >> 4] = make_float2(ldexpf(1.0f, ex - 22), bad);
#pragma unroll
        for (int g = 0; g < 3; ++g) {  // the wave's own writes: in order
            const uint4 w = *reinterpret_cast<const uint4*>(&lqd[wave][g][16 * u]);
            qd[g][0] = w.x;
            qd[g][1] = w.y;
            qd[g][2] = w.z;
            qd[g][3] = w.w;
        }
        qsc = lqs[wave][u].x;
        qbad = lqs[wave][u].y;
    }

    const int dq = lane % DQ, kg = lane / DQ;
    float m_run = -INFINITY, l_run = 0.0f;
    float o[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int t = wave; t < nt; t += WAVES) {
        load_table(t);
        load_rows();
        // the products consume the K quants only from here, so every load of
        // the tile is issued before the first wait
        asm volatile("" : "+v"(kw[0].x), "+v"(kw[0].y), "+v"(kw[0].z), "+v"(kw[0].w), "+v"(kw[1].x), "+v"(kw[1].y),
                          "+v"(kw[1].z), "+v"(kw[1].w), "+v"(kw[2].x), "+v"(kw[2].y), "+v"(kw[2].z), "+v"(kw[2].w),
                          "+v"(kw[3].x), "+v"(kw[3].y), "+v"(kw[3].z), "+v"(kw[3].w));
        // ---- scores of the tile's four passes
        float sc[PASS];
#pragma unroll
        for (int p = 0; p < PASS; ++p) {
            const int w[4] = {(int)kw[p].x, (int)kw[p].y, (int)kw[p].z, (int)kw[p].w};
            int sd[3];
#pragma unroll
            for (int g = 0; g < 3; ++g) {
                int acc = 0;
#pragma unroll
                for (int x = 0; x < 4; ++x) acc = __builtin_amdgcn_sdot4((int)qd[g][x], w[x], acc, false);
                sd[g] = acc;
            }
            const float a = fmaf((float)sd[2], 65536.0f, fmaf((float)sd[1], 256.0f, (float)sd[0]));
            float v = (vk_f16_to_f32_hw(kd[p]) * qsc) * a + qbad;
            v += __int_as_float(vk_bfly_partner<1>(__float_as_int(v)));
            v += __int_as_float(vk_bfly_partner<2>(__float_as_int(v)));
            sc[p] = hv[p] ? v * scale : -INFINITY;
        }
        // ---- the wave's online softmax over the tile
        float mx = fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3]));
        mx = fmaxf(mx, __int_as_float(vk_bfly_partner<4>(__float_as_int(mx))));
        mx = fmaxf(mx, __int_as_float(vk_bfly_partner<8>(__float_as_int(mx))));
        mx = fmaxf(mx, __int_as_float(vk_bfly_partner<16>(__float_as_int(mx))));
        mx = fmaxf(mx, __int_as_float(vk_bfly_partner<32>(__float_as_int(mx))));
        const float m_new = fmaxf(m_run, mx);
        const float m_use = m_new == -INFINITY ? 0.0f : m_new;
        const float alpha = __expf(m_run - m_use);
        float ps = 0.0f;
#pragma unroll
        for (int p = 0; p < PASS; ++p) {
            const float e = __expf(sc[p] - m_use);
            ps += e;
            // the quad's lanes of one block write the same value
            lpd[wave][KPP * p + ku][ub] = hv[p] ? e * vk_f16_to_f32_hw(vd[p]) : 0.0f;
        }
        l_run = l_run * alpha + pw_quad_group_sumf(ps);
        m_run = m_new;
        // ---- O += P . V from the wave's LDS rows: the direct loads of V have
        // landed once no load of the tile is in flight
        vk_wait_vm<0>();
        uint32_t wv[KPL];
        float pdv[KPL];
#pragma unroll
        for (int i = 0; i < KPL; ++i) {  // every read in flight before the first product
            wv[i] = *reinterpret_cast<const uint32_t*>(&lv[wave][kg + KG * i][4 * dq]);
            pdv[i] = lpd[wave][kg + KG * i][(4 * dq) / 32];
        }
        float a4[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int i = 0; i < KPL; ++i)
#pragma unroll
            for (int c4 = 0; c4 < 4; ++c4)
                a4[c4] = fmaf(pdv[i], (float)(int8_t)((wv[i] >> (8 * c4)) & 0xffu), a4[c4]);
#pragma unroll
        for (int c4 = 0; c4 < 4; ++c4) o[c4] = fmaf(o[c4], alpha, a4[c4]);
        // the rows' reads are done before the next tile's loads overwrite them
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    }
    // ---- merge: key groups, then waves, in order
    *reinterpret_cast<float4*>(&lpo[wave][kg][4 * dq]) = make_float4(o[0], o[1], o[2], o[3]);
    if (lane == 0) {
        lml[wave][0] = m_run;
        lml[wave][1] = l_run;
    }
    __syncthreads();
    if (wave != 0) return;
    const int e = lane;
    float m = lml[0][0];
#pragma unroll
    for (int w = 1; w < WAVES; ++w) m = fmaxf(m, lml[w][0]);
    float l = 0.0f, a = 0.0f;
#pragma unroll
    for (int w = 0; w < WAVES; ++w) {
        const float f = lml[w][0] == -INFINITY ? 0.0f : __expf(lml[w][0] - m);
        float ow = lpo[w][0][e];
#pragma unroll
        for (int g = 1; g < KG; ++g) ow += lpo[w][g][e];
        l = fmaf(f, lml[w][1], l);
        a = fmaf(f, ow, a);
    }
    if (nsp == 1) {
        const float val = a * (l > 0.0f ? 1.0f / l : 0.0f);
        out[((size_t)item * hq + hk) * HD + e] = val;
        if (qo.afrag) pa_quantize_out(qo, item, hk * HD + e, val);
    } else {
        const size_t pi = ((size_t)item * hq + hk) * n_split + split;
        part_o[pi * HD + e] = a;
        if (e == 0) {
            part_ml[2 * pi] = m;
            part_ml[2 * pi + 1] = l;
        }
    }
}

// ---------------------------------------------------------------------------
// Grouped-query decode attention on the matrix cores: head_dim 128 and G = 2..8
// query heads per kv head (config 4 is G = 8). Same contract as vk_paged_attn
// (one workgroup per (split, kv head, item), (m, l, O) partials for the
// combine when split), f32-level numerics through fp16 hi/lo operands:
//
//   S^T[key][head] = sum_b d_k[key][b] * (K_b . (q_hi + q_lo))_b
//     K quants are exact fp16 integers, so each block dot is the exact integer
//     dot against the two fp16 halves of q * scale; the key's f16 block scale
//     is applied to the block sum (v_mfma_f32_16x16x32_f16, keys on the 16-row
//     side, heads on the 16-column side, padded to 16);
//   O^T[dim][head] += V^T . (p * d_v)^T
//     the V block scale of each key folds into P, split hi/lo; V^T comes from
//     a per-wave LDS copy of the tile converted to fp16.
//
// Each wave owns the 32-key tiles j0 = k0 + 32 w + 128 i of the split and keeps
// its own online softmax; the four states merge in wave order at the end.
// Within a tile, MFMA row i of key subtile n is key 8 (i / 4) + 4 n + i % 4, so
// lane (g = l / 16, head l % 16) ends up holding the scores of keys 8g .. 8g+7,
// exactly the P^T operand slots 8g .. 8g+7 of the P.V product: no shuffles.
namespace pg {
constexpr int HD = 128, NB = HD / 32, KT = 32, WAVES = 4;
constexpr int VROW = KT + 8;  // fp16 per V^T row in LDS (padded; rows stay 16-byte aligned)
static_assert((VROW * 2) % 16 == 0, "16-byte LDS reads of V^T rows");
}  // namespace pg

typedef _Float16 vk_h16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 vk_h16x2_t __attribute__((ext_vector_type(2)));

// Two signed bytes (selected by `sel` from {hi_src:lo_src}) -> two exact fp16:
// 0x64uu with u = x + 128 is the fp16 1024 + u; subtracting 1152 leaves x.
__device__ __forceinline__ uint32_t vk_i8pair_f16(uint32_t hi_src, uint32_t lo_src, uint32_t sel) {
    const uint32_t t = __builtin_amdgcn_perm(hi_src, lo_src, sel) ^ 0x64806480u;
    vk_h16x2_t h = __builtin_bit_cast(vk_h16x2_t, t);
    h = h + (vk_h16x2_t){(_Float16)-1152.0f, (_Float16)-1152.0f};
    return __builtin_bit_cast(uint32_t, h);
}
// eight signed bytes (little-endian in w) -> eight fp16 in order
__device__ __forceinline__ vk_h16x8_t vk_i8x8_f16(uint2 w) {
    uint4 r;
    r.x = vk_i8pair_f16(0, w.x, 0x0c010c00u);
    r.y = vk_i8pair_f16(0, w.x, 0x0c030c02u);
    r.z = vk_i8pair_f16(0, w.y, 0x0c010c00u);
    r.w = vk_i8pair_f16(0, w.y, 0x0c030c02u);
    return __builtin_bit_cast(vk_h16x8_t, r);
}

// two workgroups per CU (measured best: 29.3 vs 30.5 us at config 4)
template <int G>
__global__ __launch_bounds__(256, 2) void vk_paged_attn_gqa(KvDev c, int layer, const int* __restrict__ streams,
                                                         const int* __restrict__ lens, const float* __restrict__ q,
                                                         float scale, int hq, int n_split,
                                                         float* __restrict__ out, float* __restrict__ part_ml,
                                                         float* __restrict__ part_o,
                                                         const float2* __restrict__ rope_cs,
                                                         const float* __restrict__ ak, const float* __restrict__ av,
                                                         const int* __restrict__ at) {
    using namespace pg;
    static_assert(G >= 2 && G <= 16, "query heads per kv head");
    __shared__ __align__(16) _Float16 lvt[WAVES][HD][VROW];  // per wave: V^T of its tile (reused by the merge)
    __shared__ float lm[WAVES][16], ll[WAVES][16];
    static_assert(sizeof(lvt) >= sizeof(vk_f32x4) * (WAVES - 1) * (HD / 16) * 64, "merge buffer fits");

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, g = lane >> 4, hh = lane & 15;
    const int split = blockIdx.x, hk = blockIdx.y, item = blockIdx.z;
    const int s = streams[item];
    const int len = min(lens[item], c.max_time);
    const int kps = pa_kps(len), nsp = pa_splits(len);
    if (split >= nsp) return;  // uniform per workgroup, before any barrier
    const int k0 = split * kps, k1 = min(len, k0 + kps);

    // Fused append (ak != null): the workgroup whose key range holds the
    // item's new step packs that step's K and V head slices into the cache
    // (the page comes from an earlier allocation launch), exactly as
    // vk_kv_write_allocated would: with rope_cs, k is rotated first (lane e
    // holds the pair e, e + 64 of the head). Wave 0 writes K, wave 1 V; the
    // tile loads below read the row back.
    if (ak) {
        const int t = at[item];
        if (t >= k0 && t < k1) {  // uniform per workgroup
            const int pid = c.table[layer * c.ppl + t / c.bs];
            if (pid >= 0 && wave < 2) {
                const size_t hr = kv_hrow(c, pid, t, s, hk);
                const float* src = (wave == 0 ? ak : av) + (size_t)item * c.width + (size_t)hk * HD;
                float lo = src[lane], hi = src[lane + HD / 2];
                if (wave == 0 && rope_cs) {
                    const float2 cs = rope_cs[(size_t)item * (HD / 2) + lane];
                    const float a = lo, b = hi;
                    lo = vk_rope_lo(a, b, cs);
                    hi = vk_rope_hi(a, b, cs);
                }
                int8_t* dq = (wave == 0 ? c.kq : c.vq) + hr * HD;
                uint16_t* dd = (wave == 0 ? c.kd : c.vd) + hr * NB;
                int8_t qlo, qhi;
                uint16_t dlo = 0, dhi = 0;
                q8_0_pack_lane(lo, lane & 31, &qlo, &dlo);
                q8_0_pack_lane(hi, lane & 31, &qhi, &dhi);
                dq[lane] = qlo;
                dq[lane + HD / 2] = qhi;
                if ((lane & 31) == 0) {
                    dd[lane >> 5] = dlo;
                    dd[2 + (lane >> 5)] = dhi;
                }
            }
            __threadfence_block();
            __syncthreads();
        }
    }

    // q * scale of head hh (zero for padding heads) as the S^T B operand:
    // lane (g, hh) holds dims 32b + 8g .. +7, split into fp16 hi + lo. With
    // rope_cs, q is first rotated: dims j and j + 64 (blocks b and b + 2) sit
    // in the same lane.
    vk_h16x8_t qh[NB], ql[NB];
    float x[NB][8];
#pragma unroll
    for (int b = 0; b < NB; ++b) {
#pragma unroll
        for (int i = 0; i < 8; ++i) x[b][i] = 0.0f;
        if (hh < G) {
            const float4* qp =
                reinterpret_cast<const float4*>(q + ((size_t)item * hq + hk * G + hh) * HD + 32 * b + 8 * g);
            const float4 u = qp[0], v = qp[1];
            x[b][0] = u.x; x[b][1] = u.y; x[b][2] = u.z; x[b][3] = u.w;
            x[b][4] = v.x; x[b][5] = v.y; x[b][6] = v.z; x[b][7] = v.w;
        }
    }
    if (rope_cs && hh < G) {
        static_assert(NB == 4, "the rotation pairs blocks b and b + 2");
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float2 cs = rope_cs[(size_t)item * (HD / 2) + 32 * b + 8 * g + i];
                const float a = x[b][i], bb = x[b + 2][i];
                x[b][i] = vk_rope_lo(a, bb, cs);
                x[b + 2][i] = vk_rope_hi(a, bb, cs);
            }
    }
#pragma unroll
    for (int b = 0; b < NB; ++b) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float xs = x[b][i] * scale;
            if (vk_f16_overflow(xs)) atomicOr(&vk_kv_range_flag, 1u);
            const _Float16 h = (_Float16)xs;
            qh[b][i] = h;
            ql[b][i] = (_Float16)(xs - (float)h);
        }
    }
    float m_run = -INFINITY, l_run = 0.0f;
    vk_f32x4 o[HD / 16];
#pragma unroll
    for (int et = 0; et < HD / 16; ++et) o[et] = {0.0f, 0.0f, 0.0f, 0.0f};
    const int trow = layer * c.ppl;
    const int va = lane & 7, vc = lane >> 3;  // V staging: keys 4va .. +3, dims 16vc .. +15
    const int jfirst = k0 + KT * wave;        // this wave's tiles: jfirst + KT * WAVES * t
    const int ntile =                         // wave-uniform: scalar branches around the loads
        __builtin_amdgcn_readfirstlane(jfirst < k1 ? (k1 - jfirst + KT * WAVES - 1) / (KT * WAVES) : 0);

    // The loads of a tile: its page-table entries one tile ahead, its K / V
    // rows and block scales one tile ahead of the tile being computed.
    // Lane l looks up key l % 32 (lanes 32..63 repeat lanes 0..31). Every
    // load is issued unconditionally (tile indices clamped to the wave's last
    // tile, keys to the split's last key), so the wait before a tile's
    // products counts only the younger loads and the prefetch stays in flight.
    struct Tile {
        uint2 kw[2][NB];  // K operand rows: subtile n, row hh <-> key 8 (hh / 4) + 4 n + hh % 4
        uint4 vw[4];      // V rows of keys 4va + t, dims 16vc .. +15
        uint2 kd, vd;     // f16 block scales of key 8 (lane / 16) + lane % 8
        int has;          // that key is cached
    };
    // the raw table entry of key lane % 32 of tile t (the key clamped into
    // the split); load_tile masks keys past the split, so nothing here waits
    auto page_of = [&](int t) -> int {
        const int jk = jfirst + KT * WAVES * t + (lane & 31);
        return c.table[trow + min(jk, k1 - 1) / c.bs];
    };
    auto load_tile = [&](int t, int raw) -> Tile {
        Tile T;
        const int jk = jfirst + KT * WAVES * t + (lane & 31);
        const int pid = jk < k1 ? raw : -1;
        const int slot_any = (int)kv_hrow(c, max(pid, 0), jk, s, hk);
        const int slot = pid >= 0 ? slot_any : 0;  // row 0: in bounds, masked
#pragma unroll
        for (int n = 0; n < 2; ++n) {
            const int sl = __shfl(slot, 8 * (hh >> 2) + 4 * n + (hh & 3), VK_WAVE);
            const uint2* kr = reinterpret_cast<const uint2*>(c.kq + (size_t)sl * HD);
#pragma unroll
            for (int b = 0; b < NB; ++b) T.kw[n][b] = kr[4 * b + g];
        }
        // the scales and presence of key 8 (lane / 16) + lane % 8: lane j < 8
        // of 16-lane row g then holds key 8 g + j, which the products take
        // through row_newbcast DPP moves instead of LDS permutes
        const int src = 8 * (lane >> 4) + (lane & 7);
        const int slot_s = __shfl(slot, src, VK_WAVE);
        T.has = __shfl(pid >= 0 ? 1 : 0, src, VK_WAVE);
        T.kd = *reinterpret_cast<const uint2*>(c.kd + (size_t)slot_s * NB);
        T.vd = *reinterpret_cast<const uint2*>(c.vd + (size_t)slot_s * NB);
#pragma unroll
        for (int t4 = 0; t4 < 4; ++t4) {
            const int sl = __shfl(slot, 4 * va + t4, VK_WAVE);
            T.vw[t4] = *reinterpret_cast<const uint4*>(c.vq + (size_t)sl * HD + 16 * vc);
        }
        return T;
    };
    auto compute = [&](const Tile& T) {
        // scales and presence of keys 8g + j (j = 4n + r) from the lanes that loaded them
        uint2 kds[8], vds[8];
        int kval[8];
#define VK_GQA_BC(J)                                                                                            \
        kds[J] = make_uint2((uint32_t)vk_row_bcast_i<J>((int)T.kd.x), (uint32_t)vk_row_bcast_i<J>((int)T.kd.y));   \
        vds[J] = make_uint2((uint32_t)vk_row_bcast_i<J>((int)T.vd.x), (uint32_t)vk_row_bcast_i<J>((int)T.vd.y));   \
        kval[J] = vk_row_bcast_i<J>(T.has);
        VK_GQA_BC(0) VK_GQA_BC(1) VK_GQA_BC(2) VK_GQA_BC(3) VK_GQA_BC(4) VK_GQA_BC(5) VK_GQA_BC(6) VK_GQA_BC(7)
#undef VK_GQA_BC

        // ---- S^T = K . (q hi + lo)^T per key subtile, block scales applied per block
        float sc[8];
#pragma unroll
        for (int n = 0; n < 2; ++n) {
            vk_f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                const vk_h16x8_t a = vk_i8x8_f16(T.kw[n][b]);
                vk_f32x4 d = {0.0f, 0.0f, 0.0f, 0.0f};
                d = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, qh[b], d, 0, 0, 0);
                d = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, ql[b], d, 0, 0, 0);
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const uint2 kd = kds[4 * n + r];
                    const uint32_t bits = (b < 2 ? kd.x : kd.y) >> (16 * (b & 1));
                    acc[r] = fmaf(vk_f16_to_f32_hw(bits & 0xffffu), d[r], acc[r]);
                }
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) sc[4 * n + r] = kval[4 * n + r] ? acc[r] : -INFINITY;
        }

        // ---- online softmax of head hh over the tile's 32 keys
        float mloc = sc[0];
#pragma unroll
        for (int j = 1; j < 8; ++j) mloc = fmaxf(mloc, sc[j]);
        mloc = fmaxf(mloc, __int_as_float(vk_bfly_partner<16>(__float_as_int(mloc))));
        mloc = fmaxf(mloc, __shfl_xor(mloc, 32, VK_WAVE));
        const float m_new = fmaxf(m_run, mloc);
        const float m_use = m_new == -INFINITY ? 0.0f : m_new;
        const float alpha = __expf(m_run - m_use);
        float p[8], psum = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            p[j] = __expf(sc[j] - m_use);
            psum += p[j];
        }
        psum += __int_as_float(vk_bfly_partner<16>(__float_as_int(psum)));
        psum += __shfl_xor(psum, 32, VK_WAVE);
        l_run = l_run * alpha + psum;
        m_run = m_new;
#pragma unroll
        for (int et = 0; et < HD / 16; ++et)
#pragma unroll
            for (int r = 0; r < 4; ++r) o[et][r] *= alpha;

        // ---- V^T of the tile into this wave's LDS, as fp16 (keys 4va .. +3 of dim 16vc + x)
#pragma unroll
        for (int x = 0; x < 16; ++x) {
            const int cw = x >> 2, sb = x & 3;  // component and byte of dim x in each row's 16 bytes
            const uint4* vw = T.vw;
            const uint32_t w0 = cw == 0 ? vw[0].x : cw == 1 ? vw[0].y : cw == 2 ? vw[0].z : vw[0].w;
            const uint32_t w1 = cw == 0 ? vw[1].x : cw == 1 ? vw[1].y : cw == 2 ? vw[1].z : vw[1].w;
            const uint32_t w2 = cw == 0 ? vw[2].x : cw == 1 ? vw[2].y : cw == 2 ? vw[2].z : vw[2].w;
            const uint32_t w3 = cw == 0 ? vw[3].x : cw == 1 ? vw[3].y : cw == 2 ? vw[3].z : vw[3].w;
            const uint32_t sel = 0x0c000c00u | ((uint32_t)(4 + sb) << 16) | (uint32_t)sb;
            uint2 h;
            h.x = vk_i8pair_f16(w1, w0, sel);
            h.y = vk_i8pair_f16(w3, w2, sel);
            *reinterpret_cast<uint2*>(&lvt[wave][16 * vc + x][4 * va]) = h;
        }

        // ---- O^T += V^T . (p d_v)^T, one V block scale per pair of 16-dim tiles
#pragma unroll
        for (int vb = 0; vb < NB; ++vb) {
            vk_h16x8_t bh, bl;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const uint32_t bits = (vb < 2 ? vds[j].x : vds[j].y) >> (16 * (vb & 1));
                const float pd = p[j] * vk_f16_to_f32_hw(bits & 0xffffu);
                const _Float16 h = (_Float16)pd;
                bh[j] = h;
                bl[j] = (_Float16)(pd - (float)h);
            }
#pragma unroll
            for (int e2 = 0; e2 < 2; ++e2) {
                const int et = 2 * vb + e2;
                const vk_h16x8_t a = *reinterpret_cast<const vk_h16x8_t*>(&lvt[wave][16 * et + hh][8 * g]);
                o[et] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bh, o[et], 0, 0, 0);
                o[et] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bl, o[et], 0, 0, 0);
            }
        }
    };

    // Two register sets, alternating (no copies between them); past the
    // wave's last tile the prefetch reloads that tile, unused. Loads retire
    // in issue order, so the issue order is page(t + 2), data(t + 1), then
    // tile t's products: each wait is for the oldest loads in flight only.
    if (ntile > 0 && ntile <= 4) {
        // splits of up to 512 keys: straight-line, every load unconditional
        // (only the products of tiles past the wave's last are skipped)
        const int last = ntile - 1;
        const int p0 = page_of(0), p1 = page_of(min(1, last));
        Tile ta = load_tile(0, p0);
        const int p2 = page_of(min(2, last));
        __builtin_amdgcn_sched_barrier(0);  // keep the issue order
        Tile tb = load_tile(min(1, last), p1);
        const int p3 = page_of(min(3, last));
        __builtin_amdgcn_sched_barrier(0);
        compute(ta);
        ta = load_tile(min(2, last), p2);
        __builtin_amdgcn_sched_barrier(0);
        if (ntile > 1) compute(tb);
        tb = load_tile(min(3, last), p3);
        __builtin_amdgcn_sched_barrier(0);
        if (ntile > 2) compute(ta);
        if (ntile > 3) compute(tb);
    } else if (ntile > 4) {
        const int last = ntile - 1;
        int pid_a = page_of(0);
        int pid_b = page_of(min(1, last));
        Tile ta = load_tile(0, pid_a), tb;
        for (int t = 0; t < ntile; t += 2) {
            pid_a = page_of(min(t + 2, last));
            __builtin_amdgcn_sched_barrier(0);
            tb = load_tile(min(t + 1, last), pid_b);
            __builtin_amdgcn_sched_barrier(0);
            compute(ta);
            if (t + 1 >= ntile) break;
            pid_b = page_of(min(t + 3, last));
            __builtin_amdgcn_sched_barrier(0);
            ta = load_tile(min(t + 2, last), pid_a);
            __builtin_amdgcn_sched_barrier(0);
            compute(tb);
        }
    }

    // ---- merge the four waves (fixed order), then write
    if (lane < 16) {
        lm[wave][lane] = m_run;
        ll[wave][lane] = l_run;
    }
    __syncthreads();  // all waves are done with their V^T tiles too
    float M = lm[0][hh];
#pragma unroll
    for (int w = 1; w < WAVES; ++w) M = fmaxf(M, lm[w][hh]);
    const float M_use = M == -INFINITY ? 0.0f : M;
    float L = 0.0f;
#pragma unroll
    for (int w = 0; w < WAVES; ++w) L += ll[w][hh] * __expf(lm[w][hh] - M_use);
    const float f = __expf(m_run - M_use);
    vk_f32x4* red = reinterpret_cast<vk_f32x4*>(&lvt[0][0][0]);
    if (wave > 0) {
#pragma unroll
        for (int et = 0; et < HD / 16; ++et) {
            vk_f32x4 t = o[et];
#pragma unroll
            for (int r = 0; r < 4; ++r) t[r] *= f;
            red[((wave - 1) * (HD / 16) + et) * 64 + lane] = t;
        }
    }
    __syncthreads();
    if (wave > 0 || hh >= G) return;
    const int h = hk * G + hh;
    const size_t pi = ((size_t)item * hq + h) * n_split + split;
    const float inv = L > 0.0f ? 1.0f / L : 0.0f;
#pragma unroll
    for (int et = 0; et < HD / 16; ++et) {
        vk_f32x4 t = o[et];
#pragma unroll
        for (int r = 0; r < 4; ++r) t[r] *= f;
#pragma unroll
        for (int w = 1; w < WAVES; ++w) {
            const vk_f32x4 u = red[((w - 1) * (HD / 16) + et) * 64 + lane];
#pragma unroll
            for (int r = 0; r < 4; ++r) t[r] += u[r];
        }
        const int e = 16 * et + 4 * g;
        if (nsp == 1)
            *reinterpret_cast<float4*>(out + ((size_t)item * hq + h) * HD + e) =
                make_float4(t[0] * inv, t[1] * inv, t[2] * inv, t[3] * inv);
        else
            *reinterpret_cast<float4*>(part_o + pi * HD + e) = make_float4(t[0], t[1], t[2], t[3]);
    }
    if (nsp > 1 && g == 0) {
        part_ml[2 * pi] = M;
        part_ml[2 * pi + 1] = L;
    }
}

// Merges split partials: m = max m_s, O = sum O_s e^(m_s - m), l likewise,
// over the item's own pa_splits(len) splits (partials at stride n_split);
// items with one split were written whole by the attention kernel.
template <int HD, bool Q16>
__global__ void vk_paged_attn_combine(int n_split, int hq, const int* __restrict__ lens, int max_time,
                                      const float* __restrict__ part_ml, const float* __restrict__ part_o,
                                      float* __restrict__ out, const VkQOut qo) {
    const size_t ih = blockIdx.x;  // (item, head)
    const int e = threadIdx.x;
    const int nsp = pa_splits(min(lens[ih / hq], max_time));
    float v;
    if (nsp == 1) {
        if (!Q16) return;
        v = out[ih * HD + e];  // written by the split kernel itself
    } else {
        // every split's partials are loaded up front (indices clamped to the
        // item's last split, so all loads stay in bounds and none waits on
        // another), then merged in split order
        float pm[pa::MAX_SPLIT], pl[pa::MAX_SPLIT], po[pa::MAX_SPLIT];
#pragma unroll
        for (int sp = 0; sp < pa::MAX_SPLIT; ++sp) {
            const size_t pi = ih * n_split + min(sp, nsp - 1);
            pm[sp] = part_ml[2 * pi];
            pl[sp] = part_ml[2 * pi + 1];
            po[sp] = part_o[pi * HD + e];
        }
        float m = -INFINITY;
#pragma unroll
        for (int sp = 0; sp < pa::MAX_SPLIT; ++sp)
            if (sp < nsp) m = fmaxf(m, pm[sp]);
        const float m_use = m == -INFINITY ? 0.0f : m;
        float l = 0.0f, o = 0.0f;
#pragma unroll
        for (int sp = 0; sp < pa::MAX_SPLIT; ++sp) {
            if (sp < nsp) {
                const float w = __expf(pm[sp] - m_use);
                l += pl[sp] * w;
                o += po[sp] * w;
            }
        }
        v = l > 0.0f ? o / l : 0.0f;
        out[ih * HD + e] = v;
    }
    if constexpr (Q16) {
        // the K-quant activation pass over this head's slice of the output
        // row: 16 consecutive threads hold one 16-wide group, quantized as
        // vk_q16_lane quantizes it (amax / 127, round half away, clamp,
        // integer group sum)
        const int row = (int)(ih / hq), h = (int)(ih % hq);
        const int g = h * (HD / 16) + (e >> 4), t = e & 15;
        const float amax = vk_group_max<16>(fmaxf(0.0f, fabsf(v)));  // NaN -> 0 first, as the pass does
        float sc = 0.0f;
        int r = 0;
        if (amax != 0.0f) {
            sc = amax / 127.0f;
            const float q = vk_round_half_away(v / sc);
            r = (q != q) ? 0 : (int)fminf(fmaxf(q, -127.0f), 127.0f);
        }
        const int gs = vk_group_sum_i<16>(r);
        const int nsb = qo.k / 256, mt = row >> 4, sb = g >> 4, gi = g & 15;
        const size_t base = ((((size_t)mt * nsb + sb) * 8 + (gi >> 1)) * 64) * 2 + (gi & 1);
        const int lane_f = (row & 15) + 16 * (t >> 2);
        reinterpret_cast<uint16_t*>(qo.afrag)[(base + (size_t)lane_f * 2) * 4 + (t & 3)] =
            (uint16_t)vk_int_to_bf16_bits(r);
        if (t == 0) {  // the K-quant layout's (s, gsum) pair
            const size_t si = ((size_t)(g >> 2) * qo.m_pad + row) * 4 + (g & 3);
            reinterpret_cast<float2*>(qo.ascale)[si] = make_float2(sc, (float)gs);
        }
    }
}

}  // namespace vk

#include "vk_launch.h"

namespace vk {

static KvDev kv_view(const KvView& v) {
    KvDev c;
    c.kq = (int8_t*)v.kq;
    c.vq = (int8_t*)v.vq;
    c.kd = (uint16_t*)v.kd;
    c.vd = (uint16_t*)v.vd;
    c.table = v.table;
    c.free_list = v.free_list;
    c.meta = v.meta;
    c.n_layer = v.n_layer;
    c.n_stream = v.n_stream;
    c.width = v.width;
    c.row_blocks = v.width / 32;
    c.bs = v.bs;
    c.ppl = v.ppl;
    c.cap = v.cap;
    c.max_time = v.max_time;
    c.hd = v.hd;
    c.nh = v.width / v.hd;
    c.hb = v.hd / 32;
    return c;
}

hipError_t launch_kv_append(hipStream_t s, const KvView& v, int layer, int n, const int* streams, const int* times,
                            const float* k, const float* vv) {
    const KvDev c = kv_view(v);
    if (n > 1024) return hipErrorInvalidValue;
    int block = 64;  // the smallest power of two >= n (at least one wave)
    while (block < n) block <<= 1;
    hipLaunchKernelGGL(vk_kv_alloc, dim3(1), dim3(block), 0, s, c, layer, n, streams, times);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const size_t threads = (size_t)n * v.width;
    if (threads == 0) return hipSuccess;
    hipLaunchKernelGGL(vk_kv_write, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, s, c, layer, n, streams,
                       times, k, vv);
    return hipGetLastError();
}

hipError_t launch_kv_write_allocated(hipStream_t s, const KvView& v, int layer, int n, const int* streams,
                                    const int* times, const float* k, const float* vv, const float2* rope_cs,
                                    int hd) {
    const KvDev c = kv_view(v);
    const size_t threads = (size_t)n * v.width;
    if (threads == 0) return hipSuccess;
    if (rope_cs && (hd < 2 || hd % 2 != 0 || v.width % hd != 0)) return hipErrorInvalidValue;
    hipLaunchKernelGGL(vk_kv_write_allocated, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, s, c, layer, n,
                       streams, times, k, vv, rope_cs, hd);
    return hipGetLastError();
}

hipError_t launch_kv_alloc_layers(hipStream_t s, const KvView& v, int layer0, int n_layers, int n, int q_base,
                                  const int* streams, const int* times) {
    if (n_layers < 1 || n < 0 || (size_t)n_layers * n > 4096 || q_base < 0) return hipErrorInvalidValue;
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(vk_kv_alloc_layers, dim3(1), dim3(1024), 0, s, kv_view(v), layer0, n_layers, n, q_base, streams,
                       times);
    return hipGetLastError();
}

hipError_t launch_kv_read(hipStream_t s, const KvView& v, int layer, int t, int st, float* out, int* found) {
    hipLaunchKernelGGL(vk_kv_read, dim3((unsigned)((v.width + 255) / 256)), dim3(256), 0, s, kv_view(v), layer, t, st,
                       out, found);
    return hipGetLastError();
}

hipError_t launch_kv_release(hipStream_t s, const KvView& v, int layer) {
    const KvDev c = kv_view(v);
    hipLaunchKernelGGL(vk_kv_release, dim3(1), dim3(1024), 0, s, c, layer);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(vk_kv_zero_released, dim3(64, 64), dim3(256), 0, s, c);
    return hipGetLastError();
}

hipError_t launch_kv_reset(hipStream_t s, const KvView& v, const int* order, size_t pool_bytes, size_t scale_bytes) {
    const KvDev c = kv_view(v);
    const int n = max(v.n_layer * v.ppl, v.cap);
    hipLaunchKernelGGL(vk_kv_reset_meta, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, c, order);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    for (void* p : {v.kq, v.vq})
        hipLaunchKernelGGL(vk_fill_u32, dim3(2048), dim3(256), 0, s, (uint32_t*)p, pool_bytes / 4, 0u);
    for (void* p : {(void*)v.kd, (void*)v.vd})
        hipLaunchKernelGGL(vk_fill_u32, dim3(512), dim3(256), 0, s, (uint32_t*)p, scale_bytes / 4, 0u);
    return hipGetLastError();
}

hipError_t launch_kv_page_of(hipStream_t s, const KvView& v, int layer, int t, int* out) {
    hipLaunchKernelGGL(vk_kv_page_of, dim3(1), dim3(1), 0, s, kv_view(v), layer, t, out);
    return hipGetLastError();
}

// Returns whether the kernel that ran also quantized the output (qo). A fused
// append (ak) runs in either kernel; the rotation of the appended k (rope_cs)
// only in the matrix-core one.
template <int HD, int G>
static bool go_pa(hipStream_t s, const KvDev& c, int layer, int n, const int* streams, const int* lens,
                  const float* q, float scale, int hq, int hkv, int n_split, float* out, float* pml,
                  float* po, const VkQOut& qo, const float* ak, const float* av, const int* at,
                  const float2* rope_cs) {
    // head_dim 128 with several query heads per kv head: the matrix-core
    // kernel (its slots travel through 32-bit lane shuffles; it moves q and
    // O as float4)
    const bool small_slots = (size_t)c.cap * c.bs * c.n_stream * c.nh <= (size_t)INT32_MAX;
    const bool aligned = ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(out) |
                           reinterpret_cast<uintptr_t>(po)) & 15) == 0;
    if constexpr (HD == pg::HD && G >= 2) {
        if (small_slots && aligned) {
            hipLaunchKernelGGL((vk_paged_attn_gqa<G>), dim3(n_split, hkv, n), dim3(256), 0, s, c, layer, streams,
                               lens, q, scale, hq, n_split, out, pml, po, rope_cs, ak, av, at);
            return false;
        }
    }
    // head_dim 64, one query head per kv head: the wave-split kernel (32-bit
    // head rows from a 24-bit page multiply, page size a power of two, q rows
    // 16-byte aligned)
    if constexpr (HD == pw::HD && G == 1) {
        if (small_slots && (c.bs & (c.bs - 1)) == 0 && (reinterpret_cast<uintptr_t>(q) & 15) == 0 &&
            c.cap < (1 << 24) && (size_t)c.n_stream * c.nh * c.bs < (1u << 24)) {
            hipLaunchKernelGGL(vk_paged_attn_w64, dim3(n_split, hkv, n), dim3(256), 0, s, c, layer, streams, lens,
                               q, scale, hq, n_split, out, pml, po, n_split == 1 ? qo : VkQOut{}, ak, av, at);
            return n_split == 1 && qo.afrag;
        }
    }
    hipLaunchKernelGGL((vk_paged_attn<HD, G>), dim3(n_split, hkv, n), dim3(256), 0, s, c, layer, streams, lens, q,
                       scale, hq, n_split, out, pml, po, n_split == 1 ? qo : VkQOut{}, ak, av, at);
    return n_split == 1 && qo.afrag;
}

int paged_attn_grid_splits(int max_len) {
    // pa_splits(len) = ceil(len / 512) up to 4096 keys and never above 8
    // beyond (it is not monotone there): this bounds it for every len <= max_len
    const int k = (max_len + pa::KPS - 1) / pa::KPS;
    return k < 1 ? 1 : (k > pa::MAX_SPLIT ? pa::MAX_SPLIT : k);
}

bool paged_attn_rotates_q(const KvView& v, int hq, int hd, const float* q, const float* out, const float* part_o) {
    const int hkv = v.width / hd, g = hkv > 0 ? hq / hkv : 0;
    const bool small_slots = (size_t)v.cap * v.bs * v.n_stream * hkv <= (size_t)INT32_MAX;
    const bool aligned = ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(out) |
                           reinterpret_cast<uintptr_t>(part_o)) & 15) == 0;
    return hd == pg::HD && (g == 2 || g == 4 || g == 8) && small_slots && aligned;
}

hipError_t launch_paged_attn(hipStream_t s, const KvView& v, int layer, int n, const int* streams, const int* lens,
                             const float* q, float scale, int hq, int hd, int n_split, float* out,
                             float* part_ml, float* part_o, const VkQOut* qo, const float* ak, const float* av,
                             const int* at, const float2* rope_cs) {
    const KvDev c = kv_view(v);
    const int hkv = v.width / hd, g = hq / hkv;
    // the rotation of q (and of an appended k) rides only on the matrix-core GQA kernel
    if (rope_cs && !paged_attn_rotates_q(v, hq, hd, q, out, part_o)) return hipErrorInvalidValue;
    const VkQOut qz = qo ? *qo : VkQOut{};
    const VkQOut qb = qz.g16 ? VkQOut{} : qz;  // the split kernels' own fused pass is the 32-wide one
    bool fused = false;
#define VK_PA(HDV, GV)                                                                                          \
    if (hd == HDV && g == GV) {                                                                                 \
        fused = go_pa<HDV, GV>(s, c, layer, n, streams, lens, q, scale, hq, hkv, n_split, out,                  \
                               part_ml, part_o, qb, ak, av, at, rope_cs);                                       \
    } else
    VK_PA(64, 1) VK_PA(64, 2) VK_PA(64, 4) VK_PA(64, 8) VK_PA(128, 1) VK_PA(128, 2) VK_PA(128, 4) VK_PA(128, 8) {
        return hipErrorInvalidValue;
    }
#undef VK_PA
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    // the K-quant activation pass rides on the combine (which then also reads
    // back the rows of single-split items)
    const bool g16 = qz.afrag && qz.g16;
    if (n_split > 1) {
#define VK_PA_COMBINE(HDV, QV)                                                                                  \
        hipLaunchKernelGGL((vk_paged_attn_combine<HDV, QV>), dim3((unsigned)(n * hq)), dim3(HDV), 0, s, n_split, hq, \
                           lens, c.max_time, part_ml, part_o, out, qz)
        if (hd == 64) {
            if (g16) VK_PA_COMBINE(64, true); else VK_PA_COMBINE(64, false);
        } else {
            if (g16) VK_PA_COMBINE(128, true); else VK_PA_COMBINE(128, false);
        }
#undef VK_PA_COMBINE
        e = hipGetLastError();
        if (e != hipSuccess) return e;
        if (g16) return hipSuccess;
    }
    // kernels without the fused pass: the separate activation pass over out
    if (g16) return launch_quantize_act_g16(s, out, n, qz.m_pad, qz.k, qz.afrag, qz.ascale);
    if (qz.afrag && !fused)
        return launch_quantize_act_b32(s, qz.pow2 != 0, out, n, qz.m_pad, qz.k, qz.afrag, qz.ascale, qz.asum);
    return hipSuccess;
}

// This device's address of this file's fp16-range flag (the host reads and
// clears it with one small kernel per check).
hipError_t kv_range_flag_addr(unsigned** p) { return hipGetSymbolAddress((void**)p, HIP_SYMBOL(vk_kv_range_flag)); }

}  // namespace vk

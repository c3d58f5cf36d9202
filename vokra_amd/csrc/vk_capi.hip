// vk_capi.hip — C++ host layer behind include/vokra_hip.h.
//
// Mirrors the reference's device-context surface (CudaContext in
// crates/vokra-backend-cuda/src/context.rs): a context owns one device and one
// stream; per-op "copy mode" calls validate, upload, launch, synchronize and
// read back; resident ("_dev") calls only enqueue. Validation follows the
// reference's own rules and happens before any device work.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <algorithm>
#include <new>
#include <string>
#include <utility>
#include <mutex>
#include <vector>

#include "../../include/vokra_hip.h"
#include "vk_launch.h"

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}

int hip_fail(hipError_t e, const char* what) {
    return fail(VOKRA_HIP_ERROR_BACKEND_UNAVAILABLE, "%s: %s", what, hipGetErrorString(e));
}

// Workspace of the no-allocation GEMM entry point: activation fragments,
// scales and sums of one call. Each device holds its own copy for the life of
// the process; host code uses the per-device address from
// hipGetSymbolAddress (kept in g_scratch_dev), never the array's name.
constexpr size_t kScratchBytes = 32u << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];
constexpr int kMaxDevices = 64;
void* g_scratch_dev[kMaxDevices] = {};
std::mutex g_scratch_mu;

// The device address of `scratch` on `device` (current), looked up once.
int scratch_address(int device, void** out) {
    if (device < 0 || device >= kMaxDevices)
        return fail(VOKRA_HIP_ERROR_BACKEND_UNAVAILABLE, "device %d beyond the scratch table", device);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_dev[device]) {
        void* ptr = nullptr;
        hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)");
        if (!ptr) return fail(VOKRA_HIP_ERROR_BACKEND_UNAVAILABLE, "hipGetSymbolAddress(scratch) returned NULL");
        g_scratch_dev[device] = ptr;
    }
    *out = g_scratch_dev[device];
    return VOKRA_HIP_OK;
}

#define VK_TRY(call, what)                                 \
    do {                                                   \
        hipError_t _e = (call);                            \
        if (_e != hipSuccess) return hip_fail(_e, (what)); \
    } while (0)

size_t round_up(size_t v, size_t m) { return (v + m - 1) / m * m; }

bool mul_ok(size_t a, size_t b, size_t* out) {
    if (a != 0 && b > SIZE_MAX / a) return false;
    *out = a * b;
    return true;
}

int kv_block_bytes(int mode) {
    switch (mode) {
    case VOKRA_HIP_KV_Q4_0: return 18;
    case VOKRA_HIP_KV_Q5_0: return 22;
    case VOKRA_HIP_KV_Q8_0: return 34;
    default: return 0;
    }
}

// Super-block bytes of a K-quant weight dtype (gguf/tensor.rs:117-125), 0 if
// the dtype is not a K-quant.
size_t kq_block_bytes(int wd) {
    return wd == VOKRA_HIP_W_Q4_K ? 144 : wd == VOKRA_HIP_W_Q5_K ? 176 : wd == VOKRA_HIP_W_Q6_K ? 210 : 0;
}

// Block-format weight dtype -> KvQuant discriminant used by the kernels.
int wd_kv_mode(int wd) {
    switch (wd) {
    case VOKRA_HIP_W_Q4_0: return VOKRA_HIP_KV_Q4_0;
    case VOKRA_HIP_W_Q5_0: return VOKRA_HIP_KV_Q5_0;
    case VOKRA_HIP_W_Q8_0: return VOKRA_HIP_KV_Q8_0;
    default: return 0;
    }
}

// A device buffer that only grows (hot calls reuse it without allocating).
struct DevBuf {
    void* p = nullptr;
    size_t cap = 0;
    hipError_t ensure(size_t bytes) {
        if (bytes <= cap) return hipSuccess;
        if (p) {
            hipError_t e = hipFree(p);
            if (e != hipSuccess) return e;
            p = nullptr;
            cap = 0;
        }
        hipError_t e = hipMalloc(&p, bytes);
        if (e == hipSuccess) cap = bytes;
        return e;
    }
    void release() {
        if (p) (void)hipFree(p);
        p = nullptr;
        cap = 0;
    }
};

}  // namespace

// Quantized activations in the MFMA A-fragment layout (rows padded to the
// GEMM tile), their per-block scales and block sums.
struct vokra_hip_qact {
    vokra_hip_ctx* ctx = nullptr;
    size_t max_m = 0, k = 0, m = 0, m_pad = 0;
    bool growable = false;
    int act_quant = VOKRA_HIP_ACT_AMAX127;
    DevBuf frag, scale, gsum;
};

struct vokra_hip_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    int act_quant = VOKRA_HIP_ACT_AMAX127;
    bool decode_kernel = true;  // route m <= 64 to the decode kernel
    // Copy-mode staging and the context's own activation workspace.
    DevBuf in0, in1, in2, out0;
    vokra_hip_qact act;
    // attention workspace: fp16 hi / lo splits of q, k and transposed v
    DevBuf at_qh, at_ql, at_kh, at_kl, at_vh, at_vl;
    // front end: window, DFT basis, filter bank (for fe_mels bands), frames,
    // spectrum, power, mel energies, per-block maxima; im2col columns
    DevBuf fe_win, fe_basis, fe_fb, fe_frames, fe_spec, fe_pow, fe_mel, fe_part, cv_col;
    int fe_mels = 0;
    DevBuf lg_part;  // per-workgroup (max, index) partials of the fused logits argmax
    // RoPE frequency table of the last (rope_base, head_dim) the _dev entry saw
    DevBuf rope_theta, rope_pos;
    void* scratch = nullptr;  // this device's address of the no-allocation workspace
    unsigned *flag_attn = nullptr, *flag_kv = nullptr, *flag_gemm = nullptr;  // this device's range flags
    unsigned* flags_host = nullptr;  // pinned: the flags' values at the last check
    float rope_base = 0.0f;
    size_t rope_hd = 0;
};

struct vokra_hip_qweight {
    vokra_hip_ctx* ctx = nullptr;
    int wdtype = 0;
    size_t n = 0, k = 0, n_pad = 0, nb = 0;
    DevBuf frag, scale;  // MFMA-fragment bf16 integers + f32 scales (prefill GEMM)
    bool has_gemv = false;
    DevBuf gq, gsc;      // compact decode layout (Q4_0 / Q8_0, k % 128 == 0); Q4_K: nibble words + (d, m)
    bool kquant = false; // K-quants: one matmul kernel for every m
    int kfmt = 0;        // its weight layout: 0 nibble words (Q4_K), 1 byte words (Q5_K, Q6_K)
};

// Largest activation count routed to the decode kernel.
constexpr size_t kGemvMaxM = 64;

struct vokra_hip_event {
    hipEvent_t ev = nullptr;
};

// Paged quantized KV cache (layout and kernels in vk_kvcache.hip).
struct vokra_hip_kv {
    vokra_hip_ctx* ctx = nullptr;
    size_t n_layer = 0, n_head = 0, d_head = 0, n_stream = 0, max_time = 0, bs = 0, ppl = 0, cap = 0, width = 0;
    size_t pool_bytes = 0, scale_bytes = 0;
    DevBuf kq, vq, kd, vd, table, free_list, meta;
    DevBuf items, rows, qbuf, obuf;  // copy-mode staging
    DevBuf part_ml, part_o;          // split-K partials of paged attention
    vk::KvView view() const {
        vk::KvView v;
        v.kq = kq.p;
        v.vq = vq.p;
        v.kd = kd.p;
        v.vd = vd.p;
        v.table = (int*)table.p;
        v.free_list = (int*)free_list.p;
        v.meta = (int*)meta.p;
        v.n_layer = (int)n_layer;
        v.n_stream = (int)n_stream;
        v.width = (int)width;
        v.hd = (int)d_head;
        v.bs = (int)bs;
        v.ppl = (int)ppl;
        v.cap = (int)cap;
        v.max_time = (int)max_time;
        return v;
    }
    void release_all() {
        for (DevBuf* b : {&kq, &vq, &kd, &vd, &table, &free_list, &meta, &items, &rows, &qbuf, &obuf, &part_ml, &part_o})
            b->release();
    }
};

struct vokra_hip_graph {
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
};

namespace {

hipError_t set_dev(const vokra_hip_ctx* c) { return hipSetDevice(c->device); }

// Sized for every convention: bf16 fragments of m_pad x k, one scale and one
// sum per 16 elements (block formats use half of it).
int qact_reserve(vokra_hip_qact* qa, size_t m, size_t k) {
    const size_t m_pad = round_up(m, vk::GEMM_TM);
    const size_t ng = k / 16;
    VK_TRY(qa->frag.ensure(m_pad * k * 2), "hipMalloc(activation fragments)");
    // the K-quant (16-wide) layout keeps (scale, sum) pairs in `scale`
    VK_TRY(qa->scale.ensure(m_pad * ng * 2 * sizeof(float)), "hipMalloc(activation scales)");
    VK_TRY(qa->gsum.ensure(m_pad * ng * sizeof(float)), "hipMalloc(activation sums)");
    return VOKRA_HIP_OK;
}

// Quantize [m, k] device activations into qa (the INT8 activation pass).
int quantize_activations(vokra_hip_ctx* c, vokra_hip_qact* qa, const float* d_a, size_t m, size_t k,
                         int act_quant) {
    if (qa->growable) {
        int st = qact_reserve(qa, m, k);
        if (st) return st;
    }
    if (act_quant == VOKRA_HIP_ACT_KQUANT) {
        if (k % 256 != 0)
            return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT,
                        "K-quant INT8 GEMV needs k to be a positive multiple of 256, got %zu", k);
        if (reinterpret_cast<uintptr_t>(d_a) % 16 != 0)
            return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "activations must be 16-byte aligned");
        const size_t m_pad = round_up(m, 16);
        VK_TRY(vk::launch_quantize_act_g16(c->stream, d_a, (int)m, (int)m_pad, (int)k, (uint4*)qa->frag.p,
                                           (float*)qa->scale.p),
               "launch(vk_quantize_act_g16)");
        qa->m = m;
        qa->k = k;
        qa->m_pad = m_pad;
        qa->act_quant = act_quant;
        return VOKRA_HIP_OK;
    }
    const size_t m_pad = round_up(m, vk::GEMM_TM);
    VK_TRY(vk::launch_quantize_act_b32(c->stream, act_quant == VOKRA_HIP_ACT_POW2, d_a, (int)m, (int)m_pad,
                                       (int)k, (uint4*)qa->frag.p, (float*)qa->scale.p, (float*)qa->gsum.p),
           "launch(vk_quantize_act_b32)");
    qa->m = m;
    qa->k = k;
    qa->m_pad = m_pad;
    qa->act_quant = act_quant;
    return VOKRA_HIP_OK;
}

int check_block_shapes(int wdtype, size_t n, size_t k, size_t wq_len) {
    const int mode = wd_kv_mode(wdtype);
    if (const size_t bb = kq_block_bytes(wdtype)) {
        // validate_gemv_i8 (crates/vokra-backend-cpu/src/kernels/kquant.rs:545-578)
        if (k == 0 || k % 256 != 0)
            return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT,
                        "K-quant INT8 GEMV needs k to be a positive multiple of 256, got %zu", k);
        size_t want;
        if (!mul_ok(n, (k / 256) * bb, &want))
            return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "K-quant weight byte-length overflow");
        if (wq_len != want)
            return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "K-quant weight payload is %zu bytes, want %zu (m=%zu rows x %zu)",
                        wq_len, want, n, (k / 256) * bb);
        if (n > (size_t)INT32_MAX / 2 || k > (size_t)INT32_MAX)
            return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "gemm_q_f32: dimension exceeds int32");
        return VOKRA_HIP_OK;
    }
    if (mode == 0) return fail(VOKRA_HIP_ERROR_UNSUPPORTED_OP, "gemm_q_f32: unsupported weight dtype %d", wdtype);
    if (k == 0 || k % 32 != 0)
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT,
                    "gemm_q_f32 needs k to be a positive multiple of 32, got %zu", k);
    size_t rb, want;
    if (!mul_ok(n, k / 32, &rb) || !mul_ok(rb, (size_t)kv_block_bytes(mode), &want))
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "gemm_q_f32: weight byte-length overflow");
    if (wq_len != want)
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT,
                    "block weight payload is %zu bytes, want %zu (n=%zu rows x %zu blocks)", wq_len, want, n,
                    k / 32);
    if (n > (size_t)INT32_MAX || k > (size_t)INT32_MAX)
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "gemm_q_f32: dimension exceeds int32");
    return VOKRA_HIP_OK;
}

int upload_weight(vokra_hip_ctx* c, int wdtype, size_t n, size_t k, const uint8_t* d_wq, vokra_hip_qweight* w) {
    w->ctx = c;
    w->wdtype = wdtype;
    w->n = n;
    w->k = k;
    if (kq_block_bytes(wdtype)) {
        const size_t nsb = k / 256;
        w->kquant = true;
        w->nb = nsb;
        w->n_pad = round_up(n ? n : 1, 16);
        if (wdtype == VOKRA_HIP_W_Q4_K) {
            w->kfmt = 0;
            VK_TRY(w->gq.ensure(w->n_pad * nsb * 128), "hipMalloc(Q4_K nibble words)");
            VK_TRY(w->gsc.ensure(w->n_pad * nsb * 8 * sizeof(float) * 2), "hipMalloc(Q4_K scales)");
            VK_TRY(vk::launch_repack_w_q4k(c->stream, d_wq, (int)n, (int)w->n_pad, (int)nsb, (uint4*)w->gq.p,
                                           (float2*)w->gsc.p),
                   "launch(vk_repack_w_q4k)");
        } else {
            w->kfmt = 1;
            VK_TRY(w->gq.ensure(w->n_pad * nsb * 256), "hipMalloc(K-quant byte words)");
            VK_TRY(w->gsc.ensure(w->n_pad * nsb * 16 * sizeof(float) * 2), "hipMalloc(K-quant scales)");
            VK_TRY(vk::launch_repack_w_kq8(c->stream, wdtype, d_wq, (int)n, (int)w->n_pad, (int)nsb, (uint4*)w->gq.p,
                                           (float2*)w->gsc.p),
                   "launch(vk_repack_w_kq8)");
        }
        return VOKRA_HIP_OK;
    }
    w->nb = k / 32;
    w->n_pad = round_up(n ? n : 1, vk::GEMM_TN);
    VK_TRY(w->frag.ensure(w->n_pad * k * 2), "hipMalloc(weight fragments)");
    VK_TRY(w->scale.ensure(w->n_pad * w->nb * sizeof(float)), "hipMalloc(weight scales)");
    VK_TRY(vk::launch_repack_w_b32(c->stream, wd_kv_mode(wdtype), d_wq, (int)n, (int)w->n_pad, (int)w->nb,
                                   (uint4*)w->frag.p, (float*)w->scale.p),
           "launch(vk_repack_w_b32)");
    const int mode = wd_kv_mode(wdtype);
    w->has_gemv = (mode == VOKRA_HIP_KV_Q4_0 || mode == VOKRA_HIP_KV_Q8_0) && w->nb % 4 == 0;
    if (w->has_gemv) {
        const size_t qbytes = w->n_pad * w->nb * (mode == VOKRA_HIP_KV_Q4_0 ? 16 : 32);
        VK_TRY(w->gq.ensure(qbytes), "hipMalloc(decode weights)");
        VK_TRY(w->gsc.ensure(w->n_pad * w->nb * 2), "hipMalloc(decode scales)");
        VK_TRY(vk::launch_repack_w_gemv(c->stream, mode, d_wq, (int)n, (int)w->n_pad, (int)w->nb, (uint4*)w->gq.p,
                                        (uint2*)w->gsc.p),
               "launch(vk_repack_w_gemv)");
    }
    return VOKRA_HIP_OK;
}

void release_weight(vokra_hip_qweight* w) {
    w->frag.release();
    w->scale.release();
    w->gq.release();
    w->gsc.release();
}

// Whether w runs on the decode kernel for these activations.
bool gemv_route(const vokra_hip_ctx* c, const vokra_hip_qweight* w, const vokra_hip_qact* qa) {
    return !w->kquant && w->has_gemv && qa->m <= kGemvMaxM && c->decode_kernel;
}

int run_gemm_qact(vokra_hip_ctx* c, const vokra_hip_qweight* w, const vokra_hip_qact* qa, const float* d_bias,
                  float* d_out, VkEpi epi = {nullptr, 0}) {
    if (w->kquant) {
        if (qa->act_quant != VOKRA_HIP_ACT_KQUANT)
            return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "gemm_qact: K-quant weights need KQUANT activations");
        const VkQ4kLin lin = {(const uint4*)w->gq.p, (const float2*)w->gsc.p, d_bias, d_out, epi, (int)w->n};
        VK_TRY(vk::launch_gemm_q4k(c->stream, (const uint4*)qa->frag.p, (const float*)qa->scale.p, &lin, 1,
                                   (int)qa->m, (int)w->nb, (int)qa->m_pad, w->kfmt),
               "launch(vk_gemm_q4k)");
        return VOKRA_HIP_OK;
    }
    if (qa->act_quant == VOKRA_HIP_ACT_KQUANT)
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "gemm_qact: block-format weights need AMAX127 or POW2 activations");
    // Both kernels produce bit-identical outputs; the decode kernel streams
    // the compact weights once, the GEMM reuses bf16 tiles across many rows.
    if (gemv_route(c, w, qa)) {
        const VkGemvLin lin = {(const uint4*)w->gq.p, (const uint2*)w->gsc.p, d_bias, d_out, epi, (int)w->n};
        VK_TRY(vk::launch_gemv_qblock(c->stream, wd_kv_mode(w->wdtype), qa->act_quant == VOKRA_HIP_ACT_POW2,
                                      (const uint4*)qa->frag.p, (const float*)qa->scale.p,
                                      (const float*)qa->gsum.p, &lin, 1, (int)qa->m, (int)w->nb, (int)qa->m_pad),
               "launch(vk_gemv_qblock)");
        return VOKRA_HIP_OK;
    }
    VK_TRY(vk::launch_gemm_qblock(c->stream, qa->act_quant == VOKRA_HIP_ACT_POW2, (const uint4*)qa->frag.p,
                                  (const float*)qa->scale.p, (const uint4*)w->frag.p, (const float*)w->scale.p,
                                  d_bias, d_out, (int)qa->m, (int)qa->m_pad, (int)w->n, (int)w->n_pad,
                                  (int)w->nb, epi),
           "launch(vk_gemm_qblock)");
    return VOKRA_HIP_OK;
}

int run_gemm(vokra_hip_ctx* c, const vokra_hip_qweight* w, size_t m, const float* d_a, const float* d_bias,
             float* d_out, int act_quant) {
    int st = quantize_activations(c, &c->act, d_a, m, w->k, w->kquant ? VOKRA_HIP_ACT_KQUANT : act_quant);
    if (st) return st;
    return run_gemm_qact(c, w, &c->act, d_bias, d_out);
}

// Shape checks of the attention entry points (no reference counterpart
// rejects these: the reference's loops accept any shape; these are the
// limits of the kernels).
int check_attn(size_t batch, size_t tq, size_t tkv, size_t hq, size_t hkv, size_t hd) {
    if (hd != 64 && hd != 128)
        return fail(VOKRA_HIP_ERROR_UNSUPPORTED_OP, "attn_f32: head_dim %zu is not wired (64 or 128)", hd);
    if (hq == 0 || hkv == 0 || hq % hkv != 0)
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT,
                    "attn_f32: n_head_q=%zu must be a positive multiple of n_head_kv=%zu", hq, hkv);
    if (batch == 0 || batch > 65535 || hq > 65535)
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "attn_f32: batch and n_head_q must be in 1..65535");
    if (tq > (size_t)INT32_MAX / 2 || tkv > (size_t)INT32_MAX / 2)
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "attn_f32: sequence length exceeds int32");
    return VOKRA_HIP_OK;
}

// With qo (a fused activation pass over the output rows), d_out is still
// written when keep_out is set or q is unaligned (the pass then runs on it).
int run_attn(vokra_hip_ctx* c, size_t batch, size_t tq, size_t tkv, size_t hq, size_t hkv, size_t hd,
             const float* d_q, const float* d_k, const float* d_v, float scale, int causal, size_t q_off,
             float* d_out, const VkQOut* qo = nullptr, bool keep_out = true) {
    const size_t t_pad = round_up(tkv, 64);
    const size_t nq = batch * tq * hq * hd, nk = batch * tkv * hkv * hd, nv = batch * hkv * hd * t_pad;
    // an aligned f32 q is split inside the attention kernel (same values as
    // the split pass)
    const bool q_in_kernel = ((uintptr_t)d_q & 15) == 0;
    if (!q_in_kernel) {
        VK_TRY(c->at_qh.ensure(nq * 2 + 16), "hipMalloc(attention q)");
        VK_TRY(c->at_ql.ensure(nq * 2 + 16), "hipMalloc(attention q)");
    }
    // a single query row (decode) reads K / V with one-byte low parts (the
    // compact form: a quarter fewer bytes; relative error 2^-18), several
    // rows with fp16 low parts
    const bool q7 = tq == 1;
    const int lo_mode = q7 ? vk::KV_LO_Q7 : vk::KV_LO_F16;
    VK_TRY(c->at_kh.ensure(nk * 2 + 16), "hipMalloc(attention k)");
    VK_TRY(c->at_kl.ensure(nk * (q7 ? 1 : 2) + 16), "hipMalloc(attention k)");
    VK_TRY(c->at_vh.ensure(nv * 2 + 16), "hipMalloc(attention v)");
    VK_TRY(c->at_vl.ensure(nv * (q7 ? 1 : 2) + 16), "hipMalloc(attention v)");
    if (!q_in_kernel)
        VK_TRY(vk::launch_split_rows(c->stream, d_q, nq, vk::attn_q_scale(scale), c->at_qh.p, c->at_ql.p),
               "launch(vk_split_rows q)");
    if (q7) {
        VK_TRY(vk::launch_split_rows_q7(c->stream, d_k, nk, 1.0f, c->at_kh.p, c->at_kl.p), "launch(vk_split_rows_q7 k)");
        VK_TRY(vk::launch_split_vt_q7(c->stream, d_v, (int)batch, (int)tkv, (int)t_pad, (int)hkv, (int)hd, c->at_vh.p,
                                      c->at_vl.p),
               "launch(vk_split_vt_q7)");
    } else {
        VK_TRY(vk::launch_split_rows(c->stream, d_k, nk, 1.0f, c->at_kh.p, c->at_kl.p), "launch(vk_split_rows k)");
        VK_TRY(vk::launch_split_vt(c->stream, d_v, (int)batch, (int)tkv, (int)t_pad, (int)hkv, (int)hd, c->at_vh.p,
                                   c->at_vl.p),
               "launch(vk_split_vt)");
    }
    if (q_in_kernel) {
        VK_TRY(vk::launch_flash_attn_f32q(c->stream, (int)hd, d_q, scale, c->at_kh.p, c->at_kl.p, c->at_vh.p,
                                          c->at_vl.p, (qo && !keep_out) ? nullptr : d_out, (int)batch, (int)tq,
                                          (int)tkv, (int)t_pad, (int)hq, (int)hkv, causal ? 1 : 0, (int)q_off,
                                          nullptr, lo_mode, qo),
               "launch(vk_flash_attn)");
        return VOKRA_HIP_OK;
    }
    VK_TRY(vk::launch_flash_attn(c->stream, (int)hd, c->at_qh.p, c->at_ql.p, c->at_kh.p, c->at_kl.p, c->at_vh.p,
                                 c->at_vl.p, d_out, (int)batch, (int)tq, (int)tkv, (int)t_pad, (int)hq, (int)hkv,
                                 causal ? 1 : 0, (int)q_off, nullptr, lo_mode),
           "launch(vk_flash_attn)");
    if (qo)
        VK_TRY(vk::launch_quantize_act_b32(c->stream, qo->pow2 != 0, d_out, (int)(batch * tq), qo->m_pad, qo->k,
                                           qo->afrag, qo->ascale, qo->asum),
               "launch(vk_quantize_act_b32)");
    return VOKRA_HIP_OK;
}

int kv_meta(vokra_hip_kv* kv, int* meta4) {
    VK_TRY(hipMemcpyAsync(meta4, kv->meta.p, 4 * sizeof(int), hipMemcpyDeviceToHost, kv->ctx->stream),
           "hipMemcpyAsync(kv meta)");
    VK_TRY(hipStreamSynchronize(kv->ctx->stream), "hipStreamSynchronize");
    return VOKRA_HIP_OK;
}

// Status of the last append batch, in the reference's error vocabulary.
int kv_append_status(vokra_hip_kv* kv, size_t n, const int* h_streams, const int* h_times, size_t* appended) {
    int m[4];
    int st = kv_meta(kv, m);
    if (st) return st;
    if (appended) *appended = (size_t)m[2];
    if (m[1] == VOKRA_HIP_OK) return VOKRA_HIP_OK;
    if (m[1] == VOKRA_HIP_ERROR_KV_CACHE_EXHAUSTED)
        return fail(VOKRA_HIP_ERROR_KV_CACHE_EXHAUSTED,
                    "paged KV cache exhausted: arena has %zu pages, %zu in use - pre-allocate a larger "
                    "max_time/n_stream at session construction (item %d of %zu)",
                    kv->cap, kv->cap - (size_t)m[0], m[2], n);
    if (h_streams && h_times && (size_t)m[2] < n) {
        // check_bounds order and wording (paged_quant.rs:518-544)
        const long t = h_times[m[2]], st = h_streams[m[2]];
        if (t < 0 || (size_t)t >= kv->max_time)
            return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "t %ld >= max_time %zu", t, kv->max_time);
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "stream %ld >= n_stream %zu", st, kv->n_stream);
    }
    return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "append item %d: layer, stream or t out of range", m[2]);
}

int run_paged_attn(vokra_hip_ctx* c, vokra_hip_kv* kv, size_t layer, size_t n, const int* d_streams,
                   const int* d_lens, size_t max_len, size_t hq, const float* d_q, float scale, float* d_out,
                   const VkQOut* qo = nullptr, const float* d_ak = nullptr, const float* d_av = nullptr,
                   const int* d_at = nullptr, const float2* rope_cs = nullptr) {
    // each item splits its keys by its own length (at most 8 splits of >= 512
    // keys), so its results never depend on the rest of the batch
    const int n_split = vk::paged_attn_grid_splits((int)std::min<size_t>(max_len ? max_len : 1, kv->max_time));
    if (n_split > 1) {
        VK_TRY(kv->part_ml.ensure(n * hq * n_split * 2 * sizeof(float)), "hipMalloc(paged attention partials)");
        VK_TRY(kv->part_o.ensure(n * hq * n_split * kv->d_head * sizeof(float)), "hipMalloc(paged attention partials)");
    }
    VK_TRY(vk::launch_paged_attn(c->stream, kv->view(), (int)layer, (int)n, d_streams, d_lens, d_q, scale, (int)hq,
                                 (int)kv->d_head, n_split, d_out, (float*)kv->part_ml.p, (float*)kv->part_o.p,
                                 qo, d_ak, d_av, d_at, rope_cs),
           "launch(vk_paged_attn)");
    return VOKRA_HIP_OK;
}

int check_paged_attn(const vokra_hip_kv* kv, size_t layer, size_t n, size_t hq) {
    if (layer >= kv->n_layer)
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "layer %zu >= n_layer %zu", layer, kv->n_layer);
    if (n > 65535) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "paged_attn: at most 65535 items per call");
    if (hq == 0 || hq % kv->n_head != 0 || hq / kv->n_head > 8)
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT,
                    "paged_attn: n_head_q=%zu must be 1..8 times the cache's n_head=%zu", hq, kv->n_head);
    const size_t g = hq / kv->n_head;
    if (g != 1 && g != 2 && g != 4 && g != 8)
        return fail(VOKRA_HIP_ERROR_UNSUPPORTED_OP, "paged_attn: query heads per kv head must be 1, 2, 4 or 8");
    return VOKRA_HIP_OK;
}

}  // namespace

// Internal accessors for the sessions (vk_session.hip), which are built on
// this file's entry points.
namespace vk {
hipStream_t ctx_stream(const vokra_hip_ctx* c) { return c->stream; }

// Drains the context stream and turns a raised fp16-range flag of the
// attention kernels into INVALID_ARGUMENT (the explicit failure of
// compute.rs:649-696 instead of an inf / NaN result).
// Reads and clears the three fp16-range flags in one launch: their values go
// to the context's pinned host words, so a check is one kernel and one stream
// drain (it was a copy and a drain per flag).
__global__ void vk_take_range_flags(unsigned* __restrict__ a, unsigned* __restrict__ b, unsigned* __restrict__ g,
                                    unsigned* __restrict__ host) {
    if (threadIdx.x == 0) {
        host[0] = atomicExch(a, 0u);
        host[1] = atomicExch(b, 0u);
        host[2] = atomicExch(g, 0u);
    }
}

int range_check(vokra_hip_ctx* c) {
    hipLaunchKernelGGL(vk_take_range_flags, dim3(1), dim3(64), 0, c->stream, c->flag_attn, c->flag_kv, c->flag_gemm,
                       c->flags_host);
    VK_TRY(hipGetLastError(), "launch(vk_take_range_flags)");
    VK_TRY(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    const unsigned a = c->flags_host[0], b = c->flags_host[1], g = c->flags_host[2];
    if (a || b || g)
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT,
                    "attention: an operand is outside the fp16 range of the split products (|x| >= 65520 after "
                    "scaling); the results of the calls since the last check are not valid");
    return VOKRA_HIP_OK;
}
int ctx_fail(int code, const char* fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    return fail(code, "%s", buf);
}

static int check_gemm_qact(const vokra_hip_ctx* c, const vokra_hip_qweight* w, const vokra_hip_qact* qa,
                           const float* d_out) {
    if (!c || !w || !qa || !d_out) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "gemm_qact: NULL argument");
    if (w->ctx != c || qa->ctx != c)
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "gemm_qact: weight/activations belong to another context");
    if (qa->m == 0) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "gemm_qact: activations were never quantized");
    if (qa->k != w->k)
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "gemm_qact: activation k=%zu != weight k=%zu", qa->k, w->k);
    return VOKRA_HIP_OK;
}

int gemm_qact_epi(vokra_hip_ctx* c, const vokra_hip_qweight* w, const vokra_hip_qact* qa, const float* d_bias,
                  float* d_out, VkEpi epi) {
    int st = check_gemm_qact(c, w, qa, d_out);
    if (st) return st;
    VK_TRY(set_dev(c), "hipSetDevice");
    return run_gemm_qact(c, w, qa, d_bias, d_out, epi);
}

int gemm_qact_multi(vokra_hip_ctx* c, int n, const vokra_hip_qweight* const* ws, const vokra_hip_qact* qa,
                    const float* const* biases, float* const* outs) {
    if (n < 1 || n > 3 || !ws || !outs) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "gemm_qact_multi: bad list");
    bool one_launch = true;
    for (int i = 0; i < n; ++i) {
        int st = check_gemm_qact(c, ws[i], qa, outs[i]);
        if (st) return st;
        one_launch = one_launch && gemv_route(c, ws[i], qa) && ws[i]->wdtype == ws[0]->wdtype &&
                     qa->act_quant != VOKRA_HIP_ACT_KQUANT;
    }
    VK_TRY(set_dev(c), "hipSetDevice");
    bool q4k_all = qa->act_quant == VOKRA_HIP_ACT_KQUANT;
    for (int i = 0; i < n && q4k_all; ++i)
        q4k_all = ws[i]->kquant && ws[i]->nb == ws[0]->nb && ws[i]->kfmt == ws[0]->kfmt;
    if (q4k_all && n > 1) {
        // K-quant linears over the same activations: one grid
        VkQ4kLin lins[3];
        for (int i = 0; i < n; ++i)
            lins[i] = {(const uint4*)ws[i]->gq.p, (const float2*)ws[i]->gsc.p, biases ? biases[i] : nullptr, outs[i],
                       {nullptr, 0}, (int)ws[i]->n};
        VK_TRY(vk::launch_gemm_q4k(c->stream, (const uint4*)qa->frag.p, (const float*)qa->scale.p, lins, n,
                                   (int)qa->m, (int)ws[0]->nb, (int)qa->m_pad, ws[0]->kfmt),
               "launch(vk_gemm_q4k x n)");
        return VOKRA_HIP_OK;
    }
    if (!one_launch) {
        // block formats of one width on the prefill route: one block-GEMM grid
        bool one_gemm = qa->act_quant != VOKRA_HIP_ACT_KQUANT;
        for (int i = 0; i < n && one_gemm; ++i)
            one_gemm = !ws[i]->kquant && !gemv_route(c, ws[i], qa) && ws[i]->n == ws[0]->n &&
                       ws[i]->n_pad == ws[0]->n_pad;
        if (one_gemm && n > 1) {
            VkGemmLin lins[3];
            for (int i = 0; i < n; ++i)
                lins[i] = {(const uint4*)ws[i]->frag.p, (const float*)ws[i]->scale.p, biases ? biases[i] : nullptr,
                           outs[i], {nullptr, 0}};
            VK_TRY(vk::launch_gemm_qblock_multi(c->stream, qa->act_quant == VOKRA_HIP_ACT_POW2,
                                                (const uint4*)qa->frag.p, (const float*)qa->scale.p, lins, n,
                                                (int)qa->m, (int)qa->m_pad, (int)ws[0]->n, (int)ws[0]->n_pad,
                                                (int)ws[0]->nb),
                   "launch(vk_gemm_qblock x n)");
            return VOKRA_HIP_OK;
        }
        for (int i = 0; i < n; ++i) {
            int st = run_gemm_qact(c, ws[i], qa, biases ? biases[i] : nullptr, outs[i]);
            if (st) return st;
        }
        return VOKRA_HIP_OK;
    }
    VkGemvLin lins[3];
    for (int i = 0; i < n; ++i)
        lins[i] = {(const uint4*)ws[i]->gq.p, (const uint2*)ws[i]->gsc.p, biases ? biases[i] : nullptr, outs[i],
                   {nullptr, 0}, (int)ws[i]->n};
    VK_TRY(vk::launch_gemv_qblock(c->stream, wd_kv_mode(ws[0]->wdtype), qa->act_quant == VOKRA_HIP_ACT_POW2,
                                  (const uint4*)qa->frag.p, (const float*)qa->scale.p, (const float*)qa->gsum.p, lins,
                                  n, (int)qa->m, (int)ws[0]->nb, (int)qa->m_pad),
           "launch(vk_gemv_qblock x n)");
    return VOKRA_HIP_OK;
}

int gemm_qact_qkv_split(vokra_hip_ctx* c, const vokra_hip_qweight* const* ws, const vokra_hip_qact* qa,
                        const float* const* biases, float* q_out, const VkSplitOut& ks, float* v_out, bool* fused) {
    *fused = false;
    for (int i = 0; i < 3; ++i) {
        int st = check_gemm_qact(c, ws[i], qa, q_out);
        if (st) return st;
    }
    // the one-grid block-GEMM route with whole 128-column tiles only
    bool ok = qa->act_quant != VOKRA_HIP_ACT_KQUANT;
    for (int i = 0; i < 3 && ok; ++i)
        ok = !ws[i]->kquant && !gemv_route(c, ws[i], qa) && ws[i]->n == ws[0]->n && ws[i]->n_pad == ws[i]->n &&
             ws[i]->n % 128 == 0;
    if (!ok) return VOKRA_HIP_OK;
    VK_TRY(set_dev(c), "hipSetDevice");
    VkGemmLin lins[3];
    for (int i = 0; i < 3; ++i)
        lins[i] = {(const uint4*)ws[i]->frag.p, (const float*)ws[i]->scale.p, biases ? biases[i] : nullptr,
                   i == 0 ? q_out : i == 2 ? v_out : nullptr, {nullptr, 0}, VkQOut{}, i == 1 ? ks : VkSplitOut{}};
    VK_TRY(vk::launch_gemm_qblock_multi(c->stream, qa->act_quant == VOKRA_HIP_ACT_POW2, (const uint4*)qa->frag.p,
                                        (const float*)qa->scale.p, lins, 3, (int)qa->m, (int)qa->m_pad,
                                        (int)ws[0]->n, (int)ws[0]->n_pad, (int)ws[0]->nb),
           "launch(vk_gemm_qblock q, split k, v)");
    *fused = true;
    return VOKRA_HIP_OK;
}

int qact_ln_quantize(vokra_hip_ctx* c, vokra_hip_qact* qa, size_t m, const float* d_in, const float* gamma,
                     const float* beta, float eps, int act_quant, float* d_scratch) {
    if (!c || !qa || !d_in || !gamma || !beta)
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "ln_quantize: NULL argument");
    if (qa->ctx != c) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "ln_quantize: qact belongs to another context");
    if (m == 0 || m > qa->max_m)
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "ln_quantize: m=%zu outside 1..%zu", m, qa->max_m);
    VK_TRY(set_dev(c), "hipSetDevice");
    const size_t k = qa->k;
    if (act_quant == VOKRA_HIP_ACT_KQUANT || k > (size_t)vk::kLnQuantMaxK) {
        // two passes through d_scratch [m, k]
        if (!d_scratch) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "ln_quantize: this width needs a scratch buffer");
        VK_TRY(vk::launch_layer_norm_f32(c->stream, d_in, d_scratch, (int)m, (int)k, gamma, beta, eps),
               "launch(vk_layer_norm_f32)");
        return quantize_activations(c, qa, d_scratch, m, k, act_quant);
    }
    if (act_quant != VOKRA_HIP_ACT_AMAX127 && act_quant != VOKRA_HIP_ACT_POW2)
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "ln_quantize: unknown activation convention %d", act_quant);
    if (qa->growable) {
        int st = qact_reserve(qa, m, k);
        if (st) return st;
    }
    const size_t m_pad = round_up(m, vk::GEMM_TM);
    VK_TRY(vk::launch_ln_quantize_b32(c->stream, act_quant == VOKRA_HIP_ACT_POW2, d_in, (int)m, (int)m_pad, (int)k,
                                      gamma, beta, eps, (uint4*)qa->frag.p, (float*)qa->scale.p,
                                      (float*)qa->gsum.p),
           "launch(vk_ln_quantize_b32)");
    qa->m = m;
    qa->m_pad = m_pad;
    qa->act_quant = act_quant;
    return VOKRA_HIP_OK;
}

// RMSNorm (or SwiGLU) of m rows of width k fused with the K-quant activation
// pass into qa: one launch, the same bits as the unfused pair.
static int qact_g16_prepare(vokra_hip_ctx* c, vokra_hip_qact* qa, size_t m, size_t k, const char* what) {
    if (!c || !qa || qa->ctx != c) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "%s: bad activation buffer", what);
    if (m == 0 || m > qa->max_m)
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "%s: m=%zu outside 1..%zu", what, m, qa->max_m);
    if (k == 0 || k % 256 != 0)
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT,
                    "K-quant INT8 GEMV needs k to be a positive multiple of 256, got %zu", k);
    if (qa->growable) {
        int st = qact_reserve(qa, m, k);
        if (st) return st;
    } else if (k != qa->k) {
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "%s: width %zu, the activation buffer holds %zu", what, k, qa->k);
    }
    VK_TRY(set_dev(c), "hipSetDevice");
    return VOKRA_HIP_OK;
}

int qact_rms_quantize_g16(vokra_hip_ctx* c, vokra_hip_qact* qa, size_t m, size_t k, const float* d_in,
                          const float* gamma, float eps) {
    int st = qact_g16_prepare(c, qa, m, k, "rms_quantize");
    if (st) return st;
    const size_t m_pad = round_up(m, 16);
    VK_TRY(vk::launch_rms_quantize_g16(c->stream, d_in, gamma, eps, (int)m, (int)m_pad, (int)k, (uint4*)qa->frag.p,
                                       (float*)qa->scale.p),
           "launch(vk_rms_quantize_g16)");
    qa->m = m;
    qa->k = k;
    qa->m_pad = m_pad;
    qa->act_quant = VOKRA_HIP_ACT_KQUANT;
    return VOKRA_HIP_OK;
}

int qact_swiglu_quantize_g16(vokra_hip_ctx* c, vokra_hip_qact* qa, size_t m, size_t k, const float* d_g,
                             const float* d_u) {
    int st = qact_g16_prepare(c, qa, m, k, "swiglu_quantize");
    if (st) return st;
    const size_t m_pad = round_up(m, 16);
    VK_TRY(vk::launch_swiglu_quantize_g16(c->stream, d_g, d_u, (int)m, (int)m_pad, (int)k, (uint4*)qa->frag.p,
                                          (float*)qa->scale.p),
           "launch(vk_swiglu_quantize_g16)");
    qa->m = m;
    qa->k = k;
    qa->m_pad = m_pad;
    qa->act_quant = VOKRA_HIP_ACT_KQUANT;
    return VOKRA_HIP_OK;
}

// The output side of an activation pass over m rows of qa's width, for a
// producer kernel that quantizes its own rows; qo->afrag stays NULL for the
// K-quant convention (its groups of 16 have no fused form). qact_commit then
// records what quantize_activations would.
static int qact_bind(vokra_hip_ctx* c, vokra_hip_qact* qa, size_t m, int act_quant, VkQOut* qo) {
    *qo = VkQOut{};
    if (!qa || qa->ctx != c) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "qact: bad activation buffer");
    if (m == 0 || m > qa->max_m)
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "qact_quantize: m=%zu outside 1..%zu", m, qa->max_m);
    if (act_quant == VOKRA_HIP_ACT_KQUANT) return VOKRA_HIP_OK;
    if (act_quant != VOKRA_HIP_ACT_AMAX127 && act_quant != VOKRA_HIP_ACT_POW2)
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "qact_quantize: unknown activation convention %d", act_quant);
    if (qa->growable) {
        int st = qact_reserve(qa, m, qa->k);
        if (st) return st;
    }
    *qo = VkQOut{(uint4*)qa->frag.p, (float*)qa->scale.p, (float*)qa->gsum.p, (int)round_up(m, vk::GEMM_TM),
                 (int)qa->k, act_quant == VOKRA_HIP_ACT_POW2 ? 1 : 0};
    return VOKRA_HIP_OK;
}
static void qact_commit(vokra_hip_qact* qa, size_t m, int act_quant) {
    qa->m = m;
    qa->m_pad = round_up(m, vk::GEMM_TM);
    qa->act_quant = act_quant;
}

int attn_quantize(vokra_hip_ctx* c, size_t batch, size_t tq, size_t tkv, size_t hq, size_t hkv, size_t hd,
                  const float* d_q, const float* d_k, const float* d_v, float scale, int causal, size_t q_off,
                  float* d_out, vokra_hip_qact* qa, int act_quant) {
    VkQOut qo;
    int st = qact_bind(c, qa, batch * tq, act_quant, &qo);
    if (st) return st;
    if (!qo.afrag) {
        st = vokra_hip_attn_f32_dev(c, batch, tq, tkv, hq, hkv, hd, d_q, d_k, d_v, scale, causal, q_off, d_out);
        return st ? st : vokra_hip_qact_quantize_dev(c, qa, batch * tq, d_out, act_quant);
    }
    if (qa->k != hq * hd) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "attn: qact width != n_head_q * head_dim");
    st = check_attn(batch, tq, tkv, hq, hkv, hd);
    if (st) return st;
    if (!d_q || !d_out || (tkv && (!d_k || !d_v))) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "attn: NULL buffer");
    if ((reinterpret_cast<uintptr_t>(d_q) | reinterpret_cast<uintptr_t>(d_k) | reinterpret_cast<uintptr_t>(d_out)) & 15)
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "attn: q, k and out must be 16-byte aligned");
    VK_TRY(set_dev(c), "hipSetDevice");
    st = run_attn(c, batch, tq, tkv, hq, hkv, hd, d_q, d_k, d_v, scale, causal, q_off, d_out, &qo, false);
    if (st) return st;
    qact_commit(qa, batch * tq, act_quant);
    return VOKRA_HIP_OK;
}

int attn_quantize_split(vokra_hip_ctx* c, size_t batch, size_t t, size_t h, size_t hd, const float* d_q,
                        const void* kh, const void* kl, const void* vth, const void* vtl, size_t t_pad, float scale,
                        float* d_out, vokra_hip_qact* qa, int act_quant) {
    VkQOut qo;
    int st = qact_bind(c, qa, batch * t, act_quant, &qo);
    if (st) return st;
    if (!qo.afrag || qa->k != h * hd || t < 2 || check_attn(batch, t, t, h, h, hd) ||
        (reinterpret_cast<uintptr_t>(d_q) & 15))
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "attn: split operands need the fused activation pass");
    VK_TRY(set_dev(c), "hipSetDevice");
    VK_TRY(vk::launch_flash_attn_f32q(c->stream, (int)hd, d_q, scale, kh, kl, vth, vtl, nullptr, (int)batch, (int)t,
                                      (int)t, (int)t_pad, (int)h, (int)h, 0, 0, nullptr, vk::KV_LO_F16, &qo),
           "launch(vk_flash_attn)");
    qact_commit(qa, batch * t, act_quant);
    return VOKRA_HIP_OK;
}

bool paged_attn_rotates_q(const vokra_hip_kv* kv, size_t n, size_t hq, const float* d_q, const float* d_out) {
    // part_o is 16-byte aligned whenever it is allocated (hipMalloc)
    (void)n;
    return kv && vk::paged_attn_rotates_q(kv->view(), (int)hq, (int)kv->d_head, d_q, d_out, nullptr);
}

int paged_attn_quantize(vokra_hip_ctx* c, vokra_hip_kv* kv, size_t layer, size_t n, const int* d_streams,
                        const int* d_lens, size_t max_len, size_t hq, const float* d_q, float scale, float* d_out,
                        vokra_hip_qact* qa, int act_quant, const float2* rope_cs, const float* d_ak,
                        const float* d_av, const int* d_at) {
    if (rope_cs && act_quant != VOKRA_HIP_ACT_KQUANT)
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "paged_attn_quantize: the fused rotation needs K-quant activations");
    if (d_ak && (!d_av || !d_at || act_quant != VOKRA_HIP_ACT_KQUANT))
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "paged_attn_quantize: the fused append needs K, V, times and K-quant activations");
    if (act_quant == VOKRA_HIP_ACT_KQUANT && kv && kv->ctx == c) {
        // the K-quant activation pass runs inside the split combine (or as
        // its own launch when no item splits)
        const size_t k = hq * kv->d_head;
        int st = qact_g16_prepare(c, qa, n, k, "paged_attn_quantize");
        if (st) return st;
        st = check_paged_attn(kv, layer, n, hq);
        if (st) return st;
        if (!d_streams || !d_lens || !d_q || !d_out)
            return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "paged_attn: NULL buffer");
        if (max_len > kv->max_time) max_len = kv->max_time;
        const size_t m_pad = round_up(n, 16);
        const VkQOut qo{(uint4*)qa->frag.p, (float*)qa->scale.p, (float*)qa->gsum.p, (int)m_pad, (int)k, 0, 1};
        if (rope_cs && !paged_attn_rotates_q(kv, n, hq, d_q, d_out))
            return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "paged_attn_quantize: no fused rotation for this shape");
        st = run_paged_attn(c, kv, layer, n, d_streams, d_lens, max_len, hq, d_q, scale, d_out, &qo, d_ak, d_av,
                            d_at, rope_cs);
        if (st) return st;
        qa->m = n;
        qa->k = k;
        qa->m_pad = m_pad;
        qa->act_quant = VOKRA_HIP_ACT_KQUANT;
        return VOKRA_HIP_OK;
    }
    VkQOut qo;
    int st = qact_bind(c, qa, n, act_quant, &qo);
    if (st) return st;
    if (!qo.afrag || qa->k != hq * kv->d_head) {
        st = vokra_hip_paged_attn_dev(c, kv, layer, n, d_streams, d_lens, max_len, hq, d_q, scale, d_out);
        return st ? st : vokra_hip_qact_quantize_dev(c, qa, n, d_out, act_quant);
    }
    if (!kv || kv->ctx != c) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "paged_attn: bad context or cache");
    st = check_paged_attn(kv, layer, n, hq);
    if (st) return st;
    if (!d_streams || !d_lens || !d_q || !d_out) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "paged_attn: NULL buffer");
    if (max_len > kv->max_time) max_len = kv->max_time;
    VK_TRY(set_dev(c), "hipSetDevice");
    st = run_paged_attn(c, kv, layer, n, d_streams, d_lens, max_len, hq, d_q, scale, d_out, &qo);
    if (st) return st;
    qact_commit(qa, n, act_quant);
    return VOKRA_HIP_OK;
}

int gemm_qact_quantize(vokra_hip_ctx* c, const vokra_hip_qweight* w, const vokra_hip_qact* qa, const float* d_bias,
                       float* d_out, VkEpi epi, vokra_hip_qact* qa_out, int act_quant) {
    int st = check_gemm_qact(c, w, qa, d_out);
    if (st) return st;
    if (!qa_out || qa_out->k != w->n)
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "gemm_qact_quantize: output activations must be %zu wide", w->n);
    VkQOut qo;
    st = qact_bind(c, qa_out, qa->m, act_quant, &qo);
    if (st) return st;
    const bool fused = qo.afrag && !w->kquant && qa->act_quant != VOKRA_HIP_ACT_KQUANT && !gemv_route(c, w, qa) &&
                       w->n % 128 == 0 && w->n_pad == w->n && qa_out->k == w->n &&
                       ((reinterpret_cast<uintptr_t>(d_bias) | reinterpret_cast<uintptr_t>(epi.resid)) & 15) == 0;
    VK_TRY(set_dev(c), "hipSetDevice");
    // the decode route: two 16-column tiles per workgroup hold each 32-column
    // block, so the pass runs in the GEMV's epilogue
    const bool fused_gemv = qo.afrag && !w->kquant && qa->act_quant != VOKRA_HIP_ACT_KQUANT && gemv_route(c, w, qa) &&
                            w->n % 32 == 0 && qa_out->k == w->n && qo.m_pad <= qa->m_pad && qo.m_pad % 16 == 0;
    if (fused_gemv) {
        const VkGemvLin lin = {(const uint4*)w->gq.p, (const uint2*)w->gsc.p, d_bias, nullptr, epi, (int)w->n};
        VK_TRY(vk::launch_gemv_qblock_quant(c->stream, wd_kv_mode(w->wdtype), qa->act_quant == VOKRA_HIP_ACT_POW2,
                                            (const uint4*)qa->frag.p, (const float*)qa->scale.p,
                                            (const float*)qa->gsum.p, lin, (int)qa->m, (int)w->nb, (int)qa->m_pad, qo),
               "launch(vk_gemv_qblock_wq)");
        qact_commit(qa_out, qa->m, act_quant);
        return VOKRA_HIP_OK;
    }
    if (!fused) {
        st = run_gemm_qact(c, w, qa, d_bias, d_out, epi);
        return st ? st : quantize_activations(c, qa_out, d_out, qa->m, w->n, act_quant);
    }
    VK_TRY(vk::launch_gemm_qblock(c->stream, qa->act_quant == VOKRA_HIP_ACT_POW2, (const uint4*)qa->frag.p,
                                  (const float*)qa->scale.p, (const uint4*)w->frag.p, (const float*)w->scale.p,
                                  d_bias, nullptr, (int)qa->m, (int)qa->m_pad, (int)w->n, (int)w->n_pad, (int)w->nb,
                                  epi, &qo),
           "launch(vk_gemm_qblock + activation pass)");
    qact_commit(qa_out, qa->m, act_quant);
    return VOKRA_HIP_OK;
}

int kv_alloc_layers(vokra_hip_ctx* c, vokra_hip_kv* kv, size_t first_layer, size_t layer0, size_t n_layers, size_t n,
                    const int* d_streams, const int* d_times) {
    if (!c || !kv || kv->ctx != c) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "kv_append: bad context or cache");
    if (n_layers == 0 || layer0 < first_layer || layer0 + n_layers > kv->n_layer || n * n_layers > 4096 ||
        (layer0 - first_layer) * n > 0x7fffffff)
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "kv_append: %zu layers from %zu of %zu, %zu items", n_layers,
                    layer0, kv->n_layer, n);
    if (n && (!d_streams || !d_times)) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "kv_append: NULL buffer");
    VK_TRY(set_dev(c), "hipSetDevice");
    // the launches of one step continue one batch: items of earlier layers
    // count first, and a failure stops every later launch
    const int q_base = (int)((layer0 - first_layer) * n);
    VK_TRY(vk::launch_kv_alloc_layers(c->stream, kv->view(), (int)layer0, (int)n_layers, (int)n, q_base, d_streams,
                                      d_times),
           "launch(vk_kv_alloc_layers)");
    return VOKRA_HIP_OK;
}

int kv_write_allocated(vokra_hip_ctx* c, vokra_hip_kv* kv, size_t layer, size_t n, const int* d_streams,
                       const int* d_times, const float* d_k, const float* d_v, const float2* rope_cs) {
    if (!c || !kv || kv->ctx != c) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "kv_append: bad context or cache");
    if (layer >= kv->n_layer || n > 65535)
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "kv_append: layer %zu of %zu, %zu items", layer, kv->n_layer, n);
    if (n && (!d_streams || !d_times || !d_k || !d_v)) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "kv_append: NULL buffer");
    VK_TRY(set_dev(c), "hipSetDevice");
    VK_TRY(vk::launch_kv_write_allocated(c->stream, kv->view(), (int)layer, (int)n, d_streams, d_times, d_k, d_v,
                                         rope_cs, (int)kv->d_head),
           "launch(vk_kv_write_allocated)");
    return VOKRA_HIP_OK;
}

int paged_attn_append_quantize(vokra_hip_ctx* c, vokra_hip_kv* kv, size_t layer, size_t n, const int* d_streams,
                               const int* d_times, const float* d_k, const float* d_v, const int* d_lens,
                               size_t max_len, size_t hq, const float* d_q, float scale, float* d_out,
                               vokra_hip_qact* qa, int act_quant) {
    if (!kv || kv->ctx != c) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "paged_attn: bad context or cache");
    int st = check_paged_attn(kv, layer, n, hq);
    if (st) return st;
    if (n == 0) return VOKRA_HIP_OK;
    if (!d_streams || !d_times || !d_k || !d_v || !d_lens || !d_q || !d_out)
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "paged_attn: NULL buffer");
    VkQOut qo;
    st = qact_bind(c, qa, n, act_quant, &qo);
    if (st) return st;
    if (qa->k != hq * kv->d_head) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "paged_attn: qact width");
    if (max_len > kv->max_time) max_len = kv->max_time;
    VK_TRY(set_dev(c), "hipSetDevice");
    st = run_paged_attn(c, kv, layer, n, d_streams, d_lens, max_len, hq, d_q, scale, d_out, qo.afrag ? &qo : nullptr,
                        d_k, d_v, d_times);
    if (st) return st;
    if (qo.afrag) {
        qact_commit(qa, n, act_quant);
        return VOKRA_HIP_OK;
    }
    return vokra_hip_qact_quantize_dev(c, qa, n, d_out, act_quant);
}

int qact_output(vokra_hip_ctx* c, vokra_hip_qact* qa, size_t m, int act_quant, VkQOut* qo) {
    return qact_bind(c, qa, m, act_quant, qo);
}
void qact_outputs_written(vokra_hip_qact* qa, size_t m, int act_quant) { qact_commit(qa, m, act_quant); }
}  // namespace vk

extern "C" {

int vokra_hip_kv_create(vokra_hip_ctx_t* c, size_t n_layer, size_t n_head, size_t d_head, size_t n_stream,
                        size_t max_time, size_t block_size, int mode, vokra_hip_kv_t** out) {
    if (!c || !out) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "kv_create: NULL argument");
    *out = nullptr;
    // QuantizedPagedKvCache::new (crates/vokra-core/src/cache/paged_quant.rs:260-307)
    if (mode == VOKRA_HIP_KV_FP32)
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT,
                    "QuantizedPagedKvCache::new: mode=Fp32 - use PagedKvCache<f32> for FP32");
    if (!n_layer || !n_head || !d_head || !n_stream || !max_time || !block_size)
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "QuantizedPagedKvCache::new: every axis must be > 0");
    if ((n_head * d_head) % 32 != 0)
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT,
                    "QuantizedPagedKvCache::new: n_head*d_head=%zu not a multiple of 32", n_head * d_head);
    if (mode != VOKRA_HIP_KV_Q8_0)
        return fail(VOKRA_HIP_ERROR_UNSUPPORTED_OP, "kv_create: the device cache stores Q8_0 rows (mode %d)", mode);
    if (d_head != 64 && d_head != 128)
        return fail(VOKRA_HIP_ERROR_UNSUPPORTED_OP, "kv_create: d_head %zu is not wired (64 or 128)", d_head);
    const size_t ppl = (max_time + block_size - 1) / block_size;
    const size_t cap = ppl * n_layer;
    if (cap > (size_t)INT32_MAX / 2 || n_stream > 65535 || max_time > (size_t)INT32_MAX / 2)
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "kv_create: cache too large for int32 indexing");
    VK_TRY(set_dev(c), "hipSetDevice");
    auto* kv = new vokra_hip_kv();
    kv->ctx = c;
    kv->n_layer = n_layer;
    kv->n_head = n_head;
    kv->d_head = d_head;
    kv->n_stream = n_stream;
    kv->max_time = max_time;
    kv->bs = block_size;
    kv->ppl = ppl;
    kv->cap = cap;
    kv->width = n_head * d_head;
    kv->pool_bytes = cap * block_size * n_stream * kv->width;
    kv->scale_bytes = round_up(cap * block_size * n_stream * (kv->width / 32) * 2, 4);
    hipError_t e = hipSuccess;
    for (auto pr : {std::make_pair(&kv->kq, kv->pool_bytes), std::make_pair(&kv->vq, kv->pool_bytes),
                    std::make_pair(&kv->kd, kv->scale_bytes), std::make_pair(&kv->vd, kv->scale_bytes),
                    std::make_pair(&kv->table, n_layer * ppl * sizeof(int)),
                    std::make_pair(&kv->free_list, cap * sizeof(int)), std::make_pair(&kv->meta, (4 + 1024) * sizeof(int))})
        if (e == hipSuccess) e = pr.first->ensure(pr.second);
    if (e == hipSuccess) e = vk::launch_kv_reset(c->stream, kv->view(), nullptr, kv->pool_bytes, kv->scale_bytes);
    if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    if (e != hipSuccess) {
        kv->release_all();
        delete kv;
        return hip_fail(e, "kv_create");
    }
    *out = kv;
    return VOKRA_HIP_OK;
}

void vokra_hip_kv_destroy(vokra_hip_kv_t* kv) {
    if (!kv) return;
    if (kv->ctx) {
        (void)hipSetDevice(kv->ctx->device);
        (void)hipStreamSynchronize(kv->ctx->stream);
    }
    kv->release_all();
    delete kv;
}

int vokra_hip_kv_append_dev(vokra_hip_ctx_t* c, vokra_hip_kv_t* kv, size_t layer, size_t n, const int32_t* d_streams,
                            const int32_t* d_times, const float* d_k, const float* d_v) {
    if (!c || !kv || kv->ctx != c) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "kv_append: bad context or cache");
    if (n > 1024) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "kv_append: at most 1024 items per call, got %zu", n);
    if (layer >= kv->n_layer)
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "layer %zu >= n_layer %zu", layer, kv->n_layer);
    if (n && (!d_streams || !d_times || !d_k || !d_v))
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "kv_append: NULL buffer");
    VK_TRY(set_dev(c), "hipSetDevice");
    VK_TRY(vk::launch_kv_append(c->stream, kv->view(), (int)layer, (int)n, d_streams, d_times, d_k, d_v),
           "launch(vk_kv_append)");
    return VOKRA_HIP_OK;
}

int vokra_hip_kv_status(vokra_hip_ctx_t* c, vokra_hip_kv_t* kv, size_t* n_appended) {
    if (!c || !kv || kv->ctx != c) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "kv_status: bad context or cache");
    VK_TRY(set_dev(c), "hipSetDevice");
    return kv_append_status(kv, SIZE_MAX, nullptr, nullptr, n_appended);
}

int vokra_hip_kv_append(vokra_hip_ctx_t* c, vokra_hip_kv_t* kv, size_t layer, size_t n, const int32_t* streams,
                        const int32_t* times, const float* k_rows, const float* v_rows) {
    if (!c || !kv || kv->ctx != c) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "kv_append: bad context or cache");
    if (n > 1024) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "kv_append: at most 1024 items per call, got %zu", n);
    if (layer >= kv->n_layer)
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "layer %zu >= n_layer %zu", layer, kv->n_layer);
    if (n == 0) return VOKRA_HIP_OK;
    if (!streams || !times || !k_rows || !v_rows) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "kv_append: NULL buffer");
    VK_TRY(set_dev(c), "hipSetDevice");
    const size_t rb = n * kv->width * sizeof(float);
    VK_TRY(kv->items.ensure(2 * n * sizeof(int)), "hipMalloc");
    VK_TRY(kv->rows.ensure(2 * rb), "hipMalloc");
    int* d_items = (int*)kv->items.p;
    float* d_rows = (float*)kv->rows.p;
    VK_TRY(hipMemcpyAsync(d_items, streams, n * sizeof(int), hipMemcpyHostToDevice, c->stream), "hipMemcpyAsync");
    VK_TRY(hipMemcpyAsync(d_items + n, times, n * sizeof(int), hipMemcpyHostToDevice, c->stream), "hipMemcpyAsync");
    VK_TRY(hipMemcpyAsync(d_rows, k_rows, rb, hipMemcpyHostToDevice, c->stream), "hipMemcpyAsync");
    VK_TRY(hipMemcpyAsync((char*)d_rows + rb, v_rows, rb, hipMemcpyHostToDevice, c->stream), "hipMemcpyAsync");
    VK_TRY(vk::launch_kv_append(c->stream, kv->view(), (int)layer, (int)n, d_items, d_items + n, d_rows,
                                (const float*)((char*)d_rows + rb)),
           "launch(vk_kv_append)");
    return kv_append_status(kv, n, streams, times, nullptr);
}

int vokra_hip_kv_read(vokra_hip_ctx_t* c, vokra_hip_kv_t* kv, size_t layer, size_t t, size_t s, float* k_out,
                      float* v_out, int* found) {
    if (!c || !kv || kv->ctx != c || !found) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "kv_read: bad argument");
    *found = 0;
    // read_step returns None out of range (paged_quant.rs:455-462)
    if (layer >= kv->n_layer || t >= kv->max_time || s >= kv->n_stream) return VOKRA_HIP_OK;
    if (!k_out || !v_out) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "kv_read: NULL buffer");
    VK_TRY(set_dev(c), "hipSetDevice");
    VK_TRY(kv->obuf.ensure(2 * kv->width * sizeof(float) + 16), "hipMalloc");
    float* d_out = (float*)kv->obuf.p;
    int* d_found = (int*)(d_out + 2 * kv->width);
    VK_TRY(vk::launch_kv_read(c->stream, kv->view(), (int)layer, (int)t, (int)s, d_out, d_found), "launch(vk_kv_read)");
    int f = 0;
    VK_TRY(hipMemcpyAsync(&f, d_found, sizeof(int), hipMemcpyDeviceToHost, c->stream), "hipMemcpyAsync");
    VK_TRY(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    if (f) {
        VK_TRY(hipMemcpyAsync(k_out, d_out, kv->width * sizeof(float), hipMemcpyDeviceToHost, c->stream), "hipMemcpyAsync");
        VK_TRY(hipMemcpyAsync(v_out, d_out + kv->width, kv->width * sizeof(float), hipMemcpyDeviceToHost, c->stream),
               "hipMemcpyAsync");
        VK_TRY(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    }
    *found = f;
    return VOKRA_HIP_OK;
}

int vokra_hip_kv_reset(vokra_hip_ctx_t* c, vokra_hip_kv_t* kv) {
    if (!c || !kv || kv->ctx != c) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "kv_reset: bad context or cache");
    VK_TRY(set_dev(c), "hipSetDevice");
    VK_TRY(vk::launch_kv_reset(c->stream, kv->view(), nullptr, kv->pool_bytes, kv->scale_bytes), "launch(vk_kv_reset)");
    return VOKRA_HIP_OK;
}

int vokra_hip_kv_set_free_order(vokra_hip_ctx_t* c, vokra_hip_kv_t* kv, const int32_t* order, size_t n) {
    if (!c || !kv || kv->ctx != c || !order) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "kv_set_free_order: bad argument");
    if (n != kv->cap) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "kv_set_free_order: need %zu page ids, got %zu", kv->cap, n);
    std::vector<char> seen(kv->cap, 0);
    for (size_t i = 0; i < n; ++i) {
        if (order[i] < 0 || (size_t)order[i] >= kv->cap || seen[order[i]])
            return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "kv_set_free_order: not a permutation of 0..%zu", kv->cap - 1);
        seen[order[i]] = 1;
    }
    VK_TRY(set_dev(c), "hipSetDevice");
    VK_TRY(kv->items.ensure(n * sizeof(int)), "hipMalloc");
    VK_TRY(hipMemcpyAsync(kv->items.p, order, n * sizeof(int), hipMemcpyHostToDevice, c->stream), "hipMemcpyAsync");
    VK_TRY(vk::launch_kv_reset(c->stream, kv->view(), (const int*)kv->items.p, kv->pool_bytes, kv->scale_bytes),
           "launch(vk_kv_reset)");
    VK_TRY(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    return VOKRA_HIP_OK;
}

int vokra_hip_kv_release_layer(vokra_hip_ctx_t* c, vokra_hip_kv_t* kv, size_t layer) {
    if (!c || !kv || kv->ctx != c) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "kv_release_layer: bad context or cache");
    if (layer >= kv->n_layer)
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "release_layer: layer %zu >= n_layer %zu", layer, kv->n_layer);
    VK_TRY(set_dev(c), "hipSetDevice");
    VK_TRY(vk::launch_kv_release(c->stream, kv->view(), (int)layer), "launch(vk_kv_release)");
    return VOKRA_HIP_OK;
}

int vokra_hip_kv_pages(vokra_hip_ctx_t* c, vokra_hip_kv_t* kv, size_t* free_pages, size_t* pages_in_use) {
    if (!c || !kv || kv->ctx != c) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "kv_pages: bad context or cache");
    VK_TRY(set_dev(c), "hipSetDevice");
    int m[4];
    int st = kv_meta(kv, m);
    if (st) return st;
    if (free_pages) *free_pages = (size_t)m[0];
    if (pages_in_use) *pages_in_use = kv->cap - (size_t)m[0];
    return VOKRA_HIP_OK;
}

int vokra_hip_kv_page_of(vokra_hip_ctx_t* c, vokra_hip_kv_t* kv, size_t layer, size_t t, long* page) {
    if (!c || !kv || kv->ctx != c || !page) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "kv_page_of: bad argument");
    *page = -1;
    if (layer >= kv->n_layer || t >= kv->max_time) return VOKRA_HIP_OK;
    VK_TRY(set_dev(c), "hipSetDevice");
    VK_TRY(kv->obuf.ensure(2 * kv->width * sizeof(float) + 16), "hipMalloc");
    int* d = (int*)kv->obuf.p;
    VK_TRY(vk::launch_kv_page_of(c->stream, kv->view(), (int)layer, (int)t, d), "launch(vk_kv_page_of)");
    int h[2];
    VK_TRY(hipMemcpyAsync(h, d, sizeof h, hipMemcpyDeviceToHost, c->stream), "hipMemcpyAsync");
    VK_TRY(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    *page = h[0];
    return VOKRA_HIP_OK;
}

int vokra_hip_paged_attn_dev(vokra_hip_ctx_t* c, vokra_hip_kv_t* kv, size_t layer, size_t n, const int32_t* d_streams,
                             const int32_t* d_lens, size_t max_len, size_t n_head_q, const float* d_q, float scale,
                             float* d_out) {
    if (!c || !kv || kv->ctx != c) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "paged_attn: bad context or cache");
    int st = check_paged_attn(kv, layer, n, n_head_q);
    if (st) return st;
    if (n == 0) return VOKRA_HIP_OK;
    if (!d_streams || !d_lens || !d_q || !d_out) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "paged_attn: NULL buffer");
    if (max_len > kv->max_time) max_len = kv->max_time;
    VK_TRY(set_dev(c), "hipSetDevice");
    return run_paged_attn(c, kv, layer, n, d_streams, d_lens, max_len, n_head_q, d_q, scale, d_out);
}

int vokra_hip_paged_attn(vokra_hip_ctx_t* c, vokra_hip_kv_t* kv, size_t layer, size_t n, const int32_t* streams,
                         const int32_t* lens, size_t n_head_q, const float* q, float scale, float* out) {
    if (!c || !kv || kv->ctx != c) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "paged_attn: bad context or cache");
    int st = check_paged_attn(kv, layer, n, n_head_q);
    if (st) return st;
    if (n == 0) return VOKRA_HIP_OK;
    if (!streams || !lens || !q || !out) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "paged_attn: NULL buffer");
    size_t max_len = 0;
    for (size_t i = 0; i < n; ++i) {
        if (streams[i] < 0 || (size_t)streams[i] >= kv->n_stream)
            return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "stream %d >= n_stream %zu", streams[i], kv->n_stream);
        if (lens[i] < 0 || (size_t)lens[i] > kv->max_time)
            return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "paged_attn: length %d outside 0..max_time %zu", lens[i],
                        kv->max_time);
        if ((size_t)lens[i] > max_len) max_len = (size_t)lens[i];
    }
    VK_TRY(set_dev(c), "hipSetDevice");
    const size_t qb = n * n_head_q * kv->d_head * sizeof(float);
    VK_TRY(kv->items.ensure(2 * n * sizeof(int)), "hipMalloc");
    VK_TRY(kv->qbuf.ensure(qb), "hipMalloc");
    VK_TRY(kv->rows.ensure(qb), "hipMalloc");
    int* d_items = (int*)kv->items.p;
    VK_TRY(hipMemcpyAsync(d_items, streams, n * sizeof(int), hipMemcpyHostToDevice, c->stream), "hipMemcpyAsync");
    VK_TRY(hipMemcpyAsync(d_items + n, lens, n * sizeof(int), hipMemcpyHostToDevice, c->stream), "hipMemcpyAsync");
    VK_TRY(hipMemcpyAsync(kv->qbuf.p, q, qb, hipMemcpyHostToDevice, c->stream), "hipMemcpyAsync");
    st = run_paged_attn(c, kv, layer, n, d_items, d_items + n, max_len, n_head_q, (const float*)kv->qbuf.p, scale,
                        (float*)kv->rows.p);
    if (st) {
        (void)hipStreamSynchronize(c->stream);
        return st;
    }
    VK_TRY(hipMemcpyAsync(out, kv->rows.p, qb, hipMemcpyDeviceToHost, c->stream), "hipMemcpyAsync");
    VK_TRY(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    return vk::range_check(c);
}

// ---- f32 kernels (A11, A12) -------------------------------------------------

namespace {
// crates/vokra-backend-cpu/src/kernels/mod.rs:228-236 expect_len
int expect_len(const char* name, size_t got, size_t want) {
    if (got == want) return VOKRA_HIP_OK;
    return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "%s length %zu does not match expected %zu", name, got, want);
}
bool fits_int(size_t v) { return v <= (size_t)INT32_MAX; }

// Upload `n` host floats into staging buffer `b` (nothing for n == 0).
int stage_in(vokra_hip_ctx* c, DevBuf& b, const float* h, size_t n) {
    VK_TRY(b.ensure(n * sizeof(float) + 16), "hipMalloc");
    if (n) VK_TRY(hipMemcpyAsync(b.p, h, n * sizeof(float), hipMemcpyHostToDevice, c->stream), "hipMemcpyAsync(H2D)");
    return VOKRA_HIP_OK;
}
int stage_out(vokra_hip_ctx* c, float* h, const void* d, size_t n) {
    if (n) VK_TRY(hipMemcpyAsync(h, d, n * sizeof(float), hipMemcpyDeviceToHost, c->stream), "hipMemcpyAsync(D2H)");
    VK_TRY(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    return VOKRA_HIP_OK;
}

int upload_table(vokra_hip_ctx* c, DevBuf& b, const std::vector<float>& h) {
    VK_TRY(b.ensure(h.size() * sizeof(float)), "hipMalloc(front-end table)");
    VK_TRY(hipMemcpyAsync(b.p, h.data(), h.size() * sizeof(float), hipMemcpyHostToDevice, c->stream),
           "hipMemcpyAsync(front-end table)");
    // the host vector goes out of scope when this returns
    VK_TRY(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    return VOKRA_HIP_OK;
}

// log_mel of `batch` clips of n_samples each (device), out [batch][n_mels][3000].
int run_log_mel(vokra_hip_ctx* c, const float* d_pcm, size_t batch, size_t n_samples, size_t n_mels, float* d_out) {
    const int NFR = vk::fe_n_frames(), NB = vk::fe_n_bins(), NFFT = vk::fe_n_fft();
    if (!c->fe_win.p) {
        std::vector<float> w, b;
        vk::fe_hann_periodic(w);
        vk::fe_dft_basis(b);
        int st = upload_table(c, c->fe_win, w);
        if (!st) st = upload_table(c, c->fe_basis, b);
        if (st) return st;
    }
    if (c->fe_mels != (int)n_mels) {
        std::vector<float> fb;
        vk::fe_mel_filterbank((int)n_mels, fb);
        int st = upload_table(c, c->fe_fb, fb);
        if (st) return st;
        c->fe_mels = (int)n_mels;
    }
    const size_t rows = batch * (size_t)NFR;
    VK_TRY(c->fe_frames.ensure(rows * NFFT * sizeof(float)), "hipMalloc(frames)");
    VK_TRY(c->fe_spec.ensure(rows * 2 * NB * sizeof(float)), "hipMalloc(spectrum)");
    VK_TRY(c->fe_pow.ensure(rows * NB * sizeof(float)), "hipMalloc(power)");
    VK_TRY(c->fe_mel.ensure(rows * n_mels * sizeof(float)), "hipMalloc(mel)");
    VK_TRY(c->fe_part.ensure(batch * vk::logmel_n_partial() * sizeof(float)), "hipMalloc(partials)");
    float* frames = (float*)c->fe_frames.p;
    VK_TRY(vk::launch_stft_frames(c->stream, d_pcm, (int)batch, (int)n_samples, (const float*)c->fe_win.p, frames),
           "launch(vk_stft_frames)");
    VK_TRY(vk::launch_gemm_f32(c->stream, true, frames, (const float*)c->fe_basis.p, nullptr, (float*)c->fe_spec.p,
                               (int)rows, 2 * NB, NFFT),
           "launch(vk_gemm_f32 stft)");
    VK_TRY(vk::launch_power_spec(c->stream, (const float*)c->fe_spec.p, (float*)c->fe_pow.p, rows),
           "launch(vk_power_spec)");
    VK_TRY(vk::launch_gemm_f32(c->stream, true, (const float*)c->fe_pow.p, (const float*)c->fe_fb.p, nullptr,
                               (float*)c->fe_mel.p, (int)rows, (int)n_mels, NB),
           "launch(vk_gemm_f32 mel)");
    VK_TRY(vk::launch_logmel_finish(c->stream, (const float*)c->fe_mel.p, (int)batch, (int)n_mels, d_out,
                                    (float*)c->fe_part.p),
           "launch(vk_logmel)");
    return VOKRA_HIP_OK;
}

int check_log_mel(size_t batch, size_t n_samples, size_t n_mels) {
    if (n_mels == 0 || n_mels > 1024) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "log_mel: n_mels must be 1..1024");
    if (batch == 0 || batch > 4096) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "log_mel: batch must be 1..4096");
    if (n_samples > (size_t)INT32_MAX / 2) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "log_mel: clip too long");
    return VOKRA_HIP_OK;
}

// conv1d shape rules of kernels::conv1d_f32 (mod.rs:754-790).
int conv1d_out(size_t in_len, size_t kernel, size_t stride, size_t padding, size_t* out_len) {
    if (stride == 0) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "conv1d stride must be >= 1");
    if (kernel == 0) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "conv1d kernel must be >= 1");
    const size_t padded = in_len + 2 * padding;
    if (padded < kernel)
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "conv1d padded length %zu is smaller than kernel %zu", padded,
                    kernel);
    *out_len = (padded - kernel) / stride + 1;
    return VOKRA_HIP_OK;
}
}  // namespace

int vokra_hip_gemm_f32_dev(vokra_hip_ctx_t* c, size_t m, size_t n, size_t k, const float* d_a, const float* d_b,
                           int b_trans, const float* d_bias, float* d_out) {
    if (!c) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "gemm_f32: ctx is NULL");
    if (!fits_int(m) || !fits_int(n) || !fits_int(k))
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "gemm_f32: dimension exceeds int32");
    if (m == 0 || n == 0) return VOKRA_HIP_OK;
    if (!d_out || (k && (!d_a || !d_b))) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "gemm_f32: NULL buffer");
    VK_TRY(set_dev(c), "hipSetDevice");
    VK_TRY(vk::launch_gemm_f32(c->stream, b_trans != 0, d_a, d_b, d_bias, d_out, (int)m, (int)n, (int)k),
           "launch(vk_gemm_f32)");
    return VOKRA_HIP_OK;
}

int vokra_hip_gemm_f32(vokra_hip_ctx_t* c, size_t m, size_t n, size_t k, const float* a, size_t a_len, const float* b,
                       size_t b_len, const float* bias, float* out, size_t out_len) {
    if (!c) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "gemm_f32: ctx is NULL");
    size_t mk, kn, mn;
    if (!mul_ok(m, k, &mk) || !mul_ok(k, n, &kn) || !mul_ok(m, n, &mn))
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "gemm: dimension product overflows");
    int st = expect_len("gemm a", a_len, mk);
    if (!st) st = expect_len("gemm b", b_len, kn);
    if (!st) st = expect_len("gemm out", out_len, mn);
    if (st) return st;
    if (mn == 0) return VOKRA_HIP_OK;
    VK_TRY(set_dev(c), "hipSetDevice");
    if ((st = stage_in(c, c->in0, a, mk)) || (st = stage_in(c, c->in1, b, kn)) ||
        (st = stage_in(c, c->in2, bias, bias ? n : 0)))
        return st;
    VK_TRY(c->out0.ensure(mn * sizeof(float)), "hipMalloc");
    st = vokra_hip_gemm_f32_dev(c, m, n, k, (const float*)c->in0.p, (const float*)c->in1.p, 0,
                                bias ? (const float*)c->in2.p : nullptr, (float*)c->out0.p);
    if (st) return st;
    return stage_out(c, out, c->out0.p, mn);
}

int vokra_hip_gemv_f32_dev(vokra_hip_ctx_t* c, size_t m, size_t k, const float* d_a, const float* d_x,
                           const float* d_bias, float* d_out) {
    if (!c) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "gemv_f32: ctx is NULL");
    if (!fits_int(m) || !fits_int(k)) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "gemv_f32: dimension exceeds int32");
    if (m == 0) return VOKRA_HIP_OK;
    if (!d_out || (k && (!d_a || !d_x))) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "gemv_f32: NULL buffer");
    if ((k & 3) == 0 && ((reinterpret_cast<uintptr_t>(d_a) | reinterpret_cast<uintptr_t>(d_x)) & 15))
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "gemv_f32: a and x must be 16-byte aligned");
    VK_TRY(set_dev(c), "hipSetDevice");
    VK_TRY(vk::launch_gemv_f32(c->stream, d_a, d_x, d_bias, d_out, (int)m, (int)k), "launch(vk_gemv_f32)");
    return VOKRA_HIP_OK;
}

int vokra_hip_gemv_f32(vokra_hip_ctx_t* c, size_t m, size_t k, const float* a, size_t a_len, const float* x,
                       size_t x_len, const float* bias, float* out, size_t out_len) {
    if (!c) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "gemv_f32: ctx is NULL");
    size_t mk;
    if (!mul_ok(m, k, &mk)) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "gemv: dimension product overflows");
    int st = expect_len("gemv a", a_len, mk);
    if (!st) st = expect_len("gemv x", x_len, k);
    if (!st) st = expect_len("gemv out", out_len, m);
    if (st) return st;
    if (m == 0) return VOKRA_HIP_OK;
    VK_TRY(set_dev(c), "hipSetDevice");
    if ((st = stage_in(c, c->in0, a, mk)) || (st = stage_in(c, c->in1, x, k)) ||
        (st = stage_in(c, c->in2, bias, bias ? m : 0)))
        return st;
    VK_TRY(c->out0.ensure(m * sizeof(float)), "hipMalloc");
    st = vokra_hip_gemv_f32_dev(c, m, k, (const float*)c->in0.p, (const float*)c->in1.p,
                                bias ? (const float*)c->in2.p : nullptr, (float*)c->out0.p);
    if (st) return st;
    return stage_out(c, out, c->out0.p, m);
}

// Row ops: op 0 softmax, 1 layer_norm, 2 rms_norm; gamma/beta as the op needs.
static int row_op_dev(vokra_hip_ctx_t* c, int op, const float* d_in, float* d_out, size_t rows, size_t cols,
                      const float* d_gamma, const float* d_beta, float eps) {
    if (!fits_int(rows) || !fits_int(cols)) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "row op: dimension exceeds int32");
    if (rows == 0 || cols == 0) return VOKRA_HIP_OK;
    if (!d_in || !d_out || (op >= 1 && !d_gamma) || (op == 1 && !d_beta))
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "row op: NULL buffer");
    VK_TRY(set_dev(c), "hipSetDevice");
    hipError_t e = op == 0 ? vk::launch_softmax_f32(c->stream, d_in, d_out, (int)rows, (int)cols)
                 : op == 1 ? vk::launch_layer_norm_f32(c->stream, d_in, d_out, (int)rows, (int)cols, d_gamma, d_beta, eps)
                           : vk::launch_rms_norm_f32(c->stream, d_in, d_out, (int)rows, (int)cols, d_gamma, eps);
    VK_TRY(e, "launch(row op)");
    return VOKRA_HIP_OK;
}

static int row_op(vokra_hip_ctx_t* c, int op, const float* in, size_t in_len, float* out, size_t out_len, size_t rows,
                  size_t cols, const float* gamma, size_t gamma_len, const float* beta, size_t beta_len, float eps) {
    if (!c) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "row op: ctx is NULL");
    size_t rc;
    if (!mul_ok(rows, cols, &rc)) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "rows*cols overflows");
    // validate_rows_cols / validate_layer_norm (kernels/mod.rs:488-536)
    int st = expect_len("input", in_len, rc);
    if (!st) st = expect_len("out", out_len, rc);
    if (!st && op >= 1) st = expect_len("gamma", gamma_len, cols);
    if (!st && op == 1) st = expect_len("beta", beta_len, cols);
    if (st) return st;
    if (rc == 0) return VOKRA_HIP_OK;
    VK_TRY(set_dev(c), "hipSetDevice");
    if ((st = stage_in(c, c->in0, in, rc)) || (st = stage_in(c, c->in1, gamma, op >= 1 ? cols : 0)) ||
        (st = stage_in(c, c->in2, beta, op == 1 ? cols : 0)))
        return st;
    VK_TRY(c->out0.ensure(rc * sizeof(float)), "hipMalloc");
    st = row_op_dev(c, op, (const float*)c->in0.p, (float*)c->out0.p, rows, cols, (const float*)c->in1.p,
                    (const float*)c->in2.p, eps);
    if (st) return st;
    return stage_out(c, out, c->out0.p, rc);
}

int vokra_hip_softmax_f32(vokra_hip_ctx_t* c, const float* in, size_t in_len, float* out, size_t out_len, size_t rows,
                          size_t cols) {
    return row_op(c, 0, in, in_len, out, out_len, rows, cols, nullptr, 0, nullptr, 0, 0.0f);
}
int vokra_hip_layer_norm_f32(vokra_hip_ctx_t* c, const float* in, size_t in_len, float* out, size_t out_len,
                             size_t rows, size_t cols, const float* gamma, size_t gamma_len, const float* beta,
                             size_t beta_len, float eps) {
    return row_op(c, 1, in, in_len, out, out_len, rows, cols, gamma, gamma_len, beta, beta_len, eps);
}
int vokra_hip_rms_norm_f32(vokra_hip_ctx_t* c, const float* in, size_t in_len, float* out, size_t out_len, size_t rows,
                           size_t cols, const float* gamma, size_t gamma_len, float eps) {
    return row_op(c, 2, in, in_len, out, out_len, rows, cols, gamma, gamma_len, nullptr, 0, eps);
}
int vokra_hip_softmax_f32_dev(vokra_hip_ctx_t* c, const float* d_in, float* d_out, size_t rows, size_t cols) {
    if (!c) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "softmax: ctx is NULL");
    return row_op_dev(c, 0, d_in, d_out, rows, cols, nullptr, nullptr, 0.0f);
}
int vokra_hip_layer_norm_f32_dev(vokra_hip_ctx_t* c, const float* d_in, float* d_out, size_t rows, size_t cols,
                                 const float* d_gamma, const float* d_beta, float eps) {
    if (!c) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "layer_norm: ctx is NULL");
    return row_op_dev(c, 1, d_in, d_out, rows, cols, d_gamma, d_beta, eps);
}
int vokra_hip_rms_norm_f32_dev(vokra_hip_ctx_t* c, const float* d_in, float* d_out, size_t rows, size_t cols,
                               const float* d_gamma, float eps) {
    if (!c) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "rms_norm: ctx is NULL");
    return row_op_dev(c, 2, d_in, d_out, rows, cols, d_gamma, nullptr, eps);
}

int vokra_hip_gelu_f32_dev(vokra_hip_ctx_t* c, const float* d_x, float* d_out, size_t n) {
    if (!c) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "gelu: ctx is NULL");
    if (n == 0) return VOKRA_HIP_OK;
    if (!d_x || !d_out) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "gelu: NULL buffer");
    VK_TRY(set_dev(c), "hipSetDevice");
    VK_TRY(vk::launch_gelu_f32(c->stream, d_x, d_out, n), "launch(vk_gelu_f32)");
    return VOKRA_HIP_OK;
}
int vokra_hip_gelu_f32(vokra_hip_ctx_t* c, const float* x, float* out, size_t n) {
    if (!c) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "gelu: ctx is NULL");
    if (n == 0) return VOKRA_HIP_OK;
    if (!x || !out) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "gelu: NULL buffer");
    VK_TRY(set_dev(c), "hipSetDevice");
    int st = stage_in(c, c->in0, x, n);
    if (st) return st;
    VK_TRY(c->out0.ensure(n * sizeof(float)), "hipMalloc");
    if ((st = vokra_hip_gelu_f32_dev(c, (const float*)c->in0.p, (float*)c->out0.p, n))) return st;
    return stage_out(c, out, c->out0.p, n);
}

// ---- speech-LLM text-decoder elementwise ops ---------------------------------

namespace {
// theta_j = rope_base.powf(-2.0 * (j as f32) / (head_dim as f32)), on the host
// with the reference's f32 expression (text_decoder.rs:880), uploaded once per
// (rope_base, head_dim).
int rope_table(vokra_hip_ctx* c, float base, size_t hd) {
    if (c->rope_theta.p && c->rope_base == base && c->rope_hd == hd) return VOKRA_HIP_OK;
    std::vector<float> th(hd / 2);
    for (size_t j = 0; j < th.size(); ++j) th[j] = powf(base, -2.0f * (float)j / (float)hd);
    VK_TRY(c->rope_theta.ensure(th.size() * sizeof(float)), "hipMalloc(rope table)");
    VK_TRY(hipMemcpyAsync(c->rope_theta.p, th.data(), th.size() * sizeof(float), hipMemcpyHostToDevice, c->stream),
           "hipMemcpyAsync(rope table)");
    VK_TRY(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    c->rope_base = base;
    c->rope_hd = hd;
    return VOKRA_HIP_OK;
}

int rope_check(size_t head_dim, size_t n_head, float rope_base) {
    if (head_dim % 2 != 0)
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "rope_apply: head_dim (%zu) must be even", head_dim);
    if (head_dim == 0 || n_head == 0) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "rope_apply: head_dim and n_head > 0");
    if (!(rope_base > 0.0f)) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "rope_apply: rope_base must be > 0");
    return VOKRA_HIP_OK;
}
}  // namespace

int vokra_hip_rope_f32_dev(vokra_hip_ctx_t* c, float* d_x, size_t rows, size_t n_head, size_t head_dim,
                           float rope_base, const int32_t* d_positions) {
    if (!c) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "rope_apply: ctx is NULL");
    int st = rope_check(head_dim, n_head, rope_base);
    if (st) return st;
    if (rows == 0) return VOKRA_HIP_OK;
    if (!d_x || !d_positions) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "rope_apply: NULL buffer");
    if (rows * n_head * (head_dim / 2) > (size_t)INT32_MAX)
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "rope_apply: too many elements");
    VK_TRY(set_dev(c), "hipSetDevice");
    if ((st = rope_table(c, rope_base, head_dim))) return st;
    VK_TRY(vk::launch_rope_rows(c->stream, d_x, (int)rows, (int)n_head, (int)head_dim, (const float*)c->rope_theta.p,
                                d_positions, 0),
           "launch(vk_rope_rows)");
    return VOKRA_HIP_OK;
}

int vokra_hip_rope_f32(vokra_hip_ctx_t* c, float* x, size_t x_len, size_t seq_len, size_t n_head, size_t head_dim,
                       float rope_base, size_t position_offset) {
    if (!c) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "rope_apply: ctx is NULL");
    int st = rope_check(head_dim, n_head, rope_base);
    if (st) return st;
    if (x_len != seq_len * n_head * head_dim)
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "rope_apply: x len %zu != seq_len*n_head*head_dim %zu", x_len,
                    seq_len * n_head * head_dim);
    if (seq_len == 0) return VOKRA_HIP_OK;
    if (!x) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "rope_apply: NULL buffer");
    if (position_offset + seq_len > (size_t)INT32_MAX)
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "rope_apply: position too large");
    VK_TRY(set_dev(c), "hipSetDevice");
    std::vector<int32_t> pos(seq_len);
    for (size_t i = 0; i < seq_len; ++i) pos[i] = (int32_t)(position_offset + i);
    VK_TRY(c->rope_pos.ensure(seq_len * sizeof(int32_t)), "hipMalloc");
    VK_TRY(hipMemcpyAsync(c->rope_pos.p, pos.data(), seq_len * sizeof(int32_t), hipMemcpyHostToDevice, c->stream),
           "hipMemcpyAsync(H2D)");
    if ((st = stage_in(c, c->in0, x, x_len))) return st;
    if ((st = vokra_hip_rope_f32_dev(c, (float*)c->in0.p, seq_len, n_head, head_dim, rope_base,
                                     (const int32_t*)c->rope_pos.p)))
        return st;
    return stage_out(c, x, c->in0.p, x_len);
}

int vokra_hip_swiglu_f32_dev(vokra_hip_ctx_t* c, const float* d_gate, const float* d_up, size_t n, float* d_out) {
    if (!c) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "swiglu: ctx is NULL");
    if (n == 0) return VOKRA_HIP_OK;
    if (!d_gate || !d_up || !d_out) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "swiglu: NULL buffer");
    VK_TRY(set_dev(c), "hipSetDevice");
    VK_TRY(vk::launch_swiglu_f32(c->stream, d_gate, d_up, d_out, n), "launch(vk_swiglu_f32)");
    return VOKRA_HIP_OK;
}

int vokra_hip_swiglu_f32(vokra_hip_ctx_t* c, const float* gate, size_t gate_len, const float* up, size_t up_len,
                         float* out) {
    if (!c) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "swiglu: ctx is NULL");
    if (gate_len != up_len)  // hadamard_inplace's rejection (text_decoder.rs:836-843)
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "hadamard_inplace: length mismatch %zu != %zu", gate_len, up_len);
    if (gate_len == 0) return VOKRA_HIP_OK;
    if (!gate || !up || !out) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "swiglu: NULL buffer");
    VK_TRY(set_dev(c), "hipSetDevice");
    int st = stage_in(c, c->in0, gate, gate_len);
    if (!st) st = stage_in(c, c->in1, up, up_len);
    if (st) return st;
    VK_TRY(c->out0.ensure(gate_len * sizeof(float)), "hipMalloc");
    if ((st = vokra_hip_swiglu_f32_dev(c, (const float*)c->in0.p, (const float*)c->in1.p, gate_len, (float*)c->out0.p)))
        return st;
    return stage_out(c, out, c->out0.p, gate_len);
}

int vokra_hip_add_f32_dev(vokra_hip_ctx_t* c, const float* d_a, const float* d_b, float* d_out, size_t n) {
    if (!c) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "add: ctx is NULL");
    if (n == 0) return VOKRA_HIP_OK;
    if (!d_a || !d_b || !d_out) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "add: NULL buffer");
    VK_TRY(set_dev(c), "hipSetDevice");
    VK_TRY(vk::launch_add_f32(c->stream, d_a, d_b, d_out, n), "launch(vk_add_f32)");
    return VOKRA_HIP_OK;
}

int vokra_hip_argmax_f32_dev(vokra_hip_ctx_t* c, const float* d_logits, size_t rows, size_t cols, int32_t* d_out) {
    if (!c) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "argmax: ctx is NULL");
    if (!fits_int(rows) || !fits_int(cols)) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "argmax: dimension exceeds int32");
    if (rows == 0) return VOKRA_HIP_OK;
    if (!d_logits || !d_out) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "argmax: NULL buffer");
    VK_TRY(set_dev(c), "hipSetDevice");
    if (rows <= 65535 && cols > 0) {  // many workgroups per row, then an in-order merge of the slices
        VK_TRY(c->lg_part.ensure(rows * (size_t)vk::argmax_n_slices((int)cols) * sizeof(float2)),
               "hipMalloc(argmax partials)");
        VK_TRY(vk::launch_argmax_sliced(c->stream, d_logits, (int)rows, (int)cols, (float2*)c->lg_part.p, d_out),
               "launch(vk_argmax_slices)");
        return VOKRA_HIP_OK;
    }
    VK_TRY(vk::launch_argmax_f32(c->stream, d_logits, (int)rows, (int)cols, d_out), "launch(vk_argmax_f32)");
    return VOKRA_HIP_OK;
}

namespace vk {
int check_logits_argmax(size_t rows, size_t vocab, size_t d, const float* x, const float* emb, const float* logits,
                        const int32_t* next) {
    if (!fits_int(rows) || !fits_int(vocab) || !fits_int(d))
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "logits_argmax: dimension exceeds int32");
    if (vocab == 0) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "logits_argmax: vocab must be positive");
    if (d < (size_t)logits_min_d() || d % logits_d_multiple() != 0)
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "logits_argmax: d must be a positive multiple of %d",
                    logits_d_multiple());
    size_t vd;
    if (!mul_ok(vocab, d, &vd)) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "logits_argmax: dimension product overflows");
    if (rows && (!x || !emb || !next)) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "logits_argmax: NULL buffer");
    if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(emb)) & 15)
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "logits_argmax: x and emb must be 16-byte aligned");
    (void)logits;
    return VOKRA_HIP_OK;
}
}  // namespace vk

int vokra_hip_logits_argmax_dev(vokra_hip_ctx_t* c, size_t rows, size_t vocab, size_t d, const float* d_x,
                                const float* d_emb, float* d_logits, int32_t* d_next) {
    if (!c) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "logits_argmax: ctx is NULL");
    int st = vk::check_logits_argmax(rows, vocab, d, d_x, d_emb, d_logits, d_next);
    if (st) return st;
    if (rows == 0) return VOKRA_HIP_OK;
    VK_TRY(set_dev(c), "hipSetDevice");
    VK_TRY(c->lg_part.ensure(rows * (size_t)vk::logits_n_vt((int)vocab) * sizeof(float2)),
           "hipMalloc(logits argmax partials)");
    VK_TRY(vk::launch_logits_argmax(c->stream, d_x, d_emb, d_logits, (float2*)c->lg_part.p, d_next, (int)rows,
                                    (int)vocab, (int)d),
           "launch(vk_logits_argmax)");
    return VOKRA_HIP_OK;
}

int vokra_hip_attn_f32_dev(vokra_hip_ctx_t* c, size_t batch, size_t t_q, size_t t_kv, size_t n_head_q,
                           size_t n_head_kv, size_t head_dim, const float* d_q, const float* d_k, const float* d_v,
                           float scale, int causal, size_t q_offset, float* d_out) {
    if (!c) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "attn_f32: ctx is NULL");
    int st = check_attn(batch, t_q, t_kv, n_head_q, n_head_kv, head_dim);
    if (st) return st;
    if (q_offset > (size_t)INT32_MAX / 2) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "attn_f32: q_offset too large");
    if (t_q == 0) return VOKRA_HIP_OK;
    if (!d_q || !d_out || (t_kv && (!d_k || !d_v)))
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "attn_f32: NULL buffer");
    if ((reinterpret_cast<uintptr_t>(d_q) | reinterpret_cast<uintptr_t>(d_k) | reinterpret_cast<uintptr_t>(d_out)) & 15)
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "attn_f32: q, k and out must be 16-byte aligned");
    VK_TRY(set_dev(c), "hipSetDevice");
    return run_attn(c, batch, t_q, t_kv, n_head_q, n_head_kv, head_dim, d_q, d_k, d_v, scale, causal, q_offset,
                    d_out);
}

int vokra_hip_attn_f32(vokra_hip_ctx_t* c, size_t batch, size_t t_q, size_t t_kv, size_t n_head_q, size_t n_head_kv,
                       size_t head_dim, const float* q, const float* k, const float* v, float scale, int causal,
                       size_t q_offset, float* out) {
    if (!c) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "attn_f32: ctx is NULL");
    int st = check_attn(batch, t_q, t_kv, n_head_q, n_head_kv, head_dim);
    if (st) return st;
    if (q_offset > (size_t)INT32_MAX / 2) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "attn_f32: q_offset too large");
    if (t_q == 0) return VOKRA_HIP_OK;
    if (!q || !out || (t_kv && (!k || !v))) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "attn_f32: NULL buffer");
    const size_t nq = batch * t_q * n_head_q * head_dim, nkv = batch * t_kv * n_head_kv * head_dim;
    VK_TRY(set_dev(c), "hipSetDevice");
    VK_TRY(c->in0.ensure(nq * 4), "hipMalloc");
    VK_TRY(c->in1.ensure(nkv * 4 + 16), "hipMalloc");
    VK_TRY(c->in2.ensure(nkv * 4 + 16), "hipMalloc");
    VK_TRY(c->out0.ensure(nq * 4), "hipMalloc");
    VK_TRY(hipMemcpyAsync(c->in0.p, q, nq * 4, hipMemcpyHostToDevice, c->stream), "hipMemcpyAsync(H2D)");
    if (nkv) {
        VK_TRY(hipMemcpyAsync(c->in1.p, k, nkv * 4, hipMemcpyHostToDevice, c->stream), "hipMemcpyAsync(H2D)");
        VK_TRY(hipMemcpyAsync(c->in2.p, v, nkv * 4, hipMemcpyHostToDevice, c->stream), "hipMemcpyAsync(H2D)");
    }
    st = run_attn(c, batch, t_q, t_kv, n_head_q, n_head_kv, head_dim, (const float*)c->in0.p, (const float*)c->in1.p,
                  (const float*)c->in2.p, scale, causal, q_offset, (float*)c->out0.p);
    if (st) {
        (void)hipStreamSynchronize(c->stream);
        return st;
    }
    VK_TRY(hipMemcpyAsync(out, c->out0.p, nq * 4, hipMemcpyDeviceToHost, c->stream), "hipMemcpyAsync(D2H)");
    VK_TRY(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    return vk::range_check(c);
}

const char* vokra_hip_last_error(void) { return g_last_error.c_str(); }

int vokra_hip_probe(int* n_devices) {
    if (!n_devices) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "probe: n_devices is NULL");
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    *n_devices = (e == hipSuccess) ? n : 0;
    if (e != hipSuccess) return hip_fail(e, "hipGetDeviceCount");
    if (n == 0) return fail(VOKRA_HIP_ERROR_BACKEND_UNAVAILABLE, "no HIP device visible");
    return VOKRA_HIP_OK;
}

int vokra_hip_create(int device, vokra_hip_ctx_t** out) {
    if (!out) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "create: out is NULL");
    *out = nullptr;
    int n = 0;
    int st = vokra_hip_probe(&n);
    if (st) return st;
    if (device < 0 || device >= n)
        return fail(VOKRA_HIP_ERROR_BACKEND_UNAVAILABLE, "device %d out of range (%d visible)", device, n);
    hipDeviceProp_t prop;
    VK_TRY(hipGetDeviceProperties(&prop, device), "hipGetDeviceProperties");
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return fail(VOKRA_HIP_ERROR_BACKEND_UNAVAILABLE, "device %d is %s; this library is built for gfx950",
                    device, prop.gcnArchName);
    VK_TRY(hipSetDevice(device), "hipSetDevice");
    void* scr = nullptr;
    if ((st = scratch_address(device, &scr))) return st;
    auto* c = new vokra_hip_ctx();
    c->device = device;
    c->act.ctx = c;
    c->act.growable = true;
    c->scratch = scr;
    hipError_t e = hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking);
    if (e == hipSuccess) e = vk::attn_range_flag_addr(&c->flag_attn);
    if (e == hipSuccess) e = vk::kv_range_flag_addr(&c->flag_kv);
    if (e == hipSuccess) e = vk::gemm_range_flag_addr(&c->flag_gemm);
    if (e == hipSuccess) e = hipHostMalloc((void**)&c->flags_host, 4 * sizeof(unsigned), hipHostMallocDefault);
    if (e == hipSuccess && (!c->flag_attn || !c->flag_kv || !c->flag_gemm)) e = hipErrorInvalidSymbol;
    if (e != hipSuccess) {
        if (c->stream) (void)hipStreamDestroy(c->stream);
        if (c->flags_host) (void)hipHostFree(c->flags_host);
        delete c;
        return hip_fail(e, "hipStreamCreate / range flags");
    }
    *out = c;
    return VOKRA_HIP_OK;
}

void vokra_hip_destroy(vokra_hip_ctx_t* c) {
    if (!c) return;
    (void)hipSetDevice(c->device);
    (void)hipStreamSynchronize(c->stream);
    for (DevBuf* b : {&c->in0, &c->in1, &c->in2, &c->out0, &c->act.frag, &c->act.scale, &c->act.gsum, &c->at_qh,
                      &c->at_ql, &c->at_kh, &c->at_kl, &c->at_vh, &c->at_vl, &c->fe_win, &c->fe_basis, &c->fe_fb,
                      &c->fe_frames, &c->fe_spec, &c->fe_pow, &c->fe_mel, &c->fe_part, &c->cv_col, &c->lg_part,
                      &c->rope_theta, &c->rope_pos})
        b->release();
    (void)hipStreamDestroy(c->stream);
    if (c->flags_host) (void)hipHostFree(c->flags_host);
    delete c;
}

int vokra_hip_synchronize(vokra_hip_ctx_t* c) {
    if (!c) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "synchronize: ctx is NULL");
    VK_TRY(set_dev(c), "hipSetDevice");
    return vk::range_check(c);  // drains the stream
}

int vokra_hip_device_alloc(vokra_hip_ctx_t* c, size_t bytes, void** dptr) {
    if (!c || !dptr) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "device_alloc: NULL argument");
    VK_TRY(set_dev(c), "hipSetDevice");
    VK_TRY(hipMalloc(dptr, bytes ? bytes : 1), "hipMalloc");
    return VOKRA_HIP_OK;
}

int vokra_hip_device_free(vokra_hip_ctx_t* c, void* dptr) {
    if (!c) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "device_free: ctx is NULL");
    VK_TRY(set_dev(c), "hipSetDevice");
    VK_TRY(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    VK_TRY(hipFree(dptr), "hipFree");
    return VOKRA_HIP_OK;
}

int vokra_hip_memcpy_htod(vokra_hip_ctx_t* c, void* dst, const void* src, size_t bytes) {
    if (!c) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "memcpy_htod: ctx is NULL");
    VK_TRY(set_dev(c), "hipSetDevice");
    VK_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, c->stream), "hipMemcpyAsync(H2D)");
    VK_TRY(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    return VOKRA_HIP_OK;
}

int vokra_hip_memcpy_dtoh(vokra_hip_ctx_t* c, void* dst, const void* src, size_t bytes) {
    if (!c) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "memcpy_dtoh: ctx is NULL");
    VK_TRY(set_dev(c), "hipSetDevice");
    VK_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, c->stream), "hipMemcpyAsync(D2H)");
    VK_TRY(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    return VOKRA_HIP_OK;
}

int vokra_hip_event_create(vokra_hip_ctx_t* c, vokra_hip_event_t** ev) {
    if (!c || !ev) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "event_create: NULL argument");
    VK_TRY(set_dev(c), "hipSetDevice");
    auto* e = new vokra_hip_event();
    hipError_t r = hipEventCreate(&e->ev);
    if (r != hipSuccess) {
        delete e;
        return hip_fail(r, "hipEventCreate");
    }
    *ev = e;
    return VOKRA_HIP_OK;
}

int vokra_hip_event_record(vokra_hip_ctx_t* c, vokra_hip_event_t* ev) {
    if (!c || !ev) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "event_record: NULL argument");
    VK_TRY(hipEventRecord(ev->ev, c->stream), "hipEventRecord");
    return VOKRA_HIP_OK;
}

int vokra_hip_event_elapsed_ms(vokra_hip_event_t* a, vokra_hip_event_t* b, float* ms) {
    if (!a || !b || !ms) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "event_elapsed: NULL argument");
    VK_TRY(hipEventSynchronize(b->ev), "hipEventSynchronize");
    VK_TRY(hipEventElapsedTime(ms, a->ev, b->ev), "hipEventElapsedTime");
    return VOKRA_HIP_OK;
}

void vokra_hip_event_destroy(vokra_hip_event_t* ev) {
    if (!ev) return;
    (void)hipEventDestroy(ev->ev);
    delete ev;
}

int vokra_hip_dequantize_bytes(vokra_hip_ctx_t* c, int mode, const uint8_t* bytes, size_t n_bytes, float* out,
                               size_t out_len) {
    if (!c) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "dequantize_bytes: ctx is NULL");
    const int bb = kv_block_bytes(mode);
    if (bb == 0)
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT,
                    "kv_quant::dequantize_bytes: mode %d has no on-wire block layout", mode);
    if (n_bytes % (size_t)bb != 0)
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT,
                    "kv_quant::dequantize_bytes: bytes.len()=%zu not a multiple of block_bytes=%d", n_bytes, bb);
    const size_t nblk = n_bytes / (size_t)bb;
    if (out_len != nblk * 32)
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT,
                    "dequantize_bytes_into: out.len()=%zu != n_blocks(%zu)*BLOCK_SIZE", out_len, nblk);
    if (nblk == 0) return VOKRA_HIP_OK;
    if (!bytes || !out) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "dequantize_bytes: NULL buffer");
    VK_TRY(set_dev(c), "hipSetDevice");
    VK_TRY(c->in0.ensure(n_bytes), "hipMalloc");
    VK_TRY(c->out0.ensure(out_len * sizeof(float)), "hipMalloc");
    VK_TRY(hipMemcpyAsync(c->in0.p, bytes, n_bytes, hipMemcpyHostToDevice, c->stream), "hipMemcpyAsync(H2D)");
    VK_TRY(vk::launch_dequantize_q0(c->stream, mode, (const uint8_t*)c->in0.p, nblk, (float*)c->out0.p),
           "launch(vk_dequantize_q0)");
    VK_TRY(hipMemcpyAsync(out, c->out0.p, out_len * sizeof(float), hipMemcpyDeviceToHost, c->stream),
           "hipMemcpyAsync(D2H)");
    VK_TRY(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    return VOKRA_HIP_OK;
}

int vokra_hip_kquant_dequantize(vokra_hip_ctx_t* c, int wdtype, const uint8_t* bytes, size_t n_bytes,
                                size_t n_elements, float* out) {
    if (!c) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "kquant_dequantize: ctx is NULL");
    const size_t bb = kq_block_bytes(wdtype);
    if (!bb) return fail(VOKRA_HIP_ERROR_UNSUPPORTED_OP, "kquant_dequantize: dtype %d is not wired on this arm", wdtype);
    // GgmlType::payload_size + TensorSizeMismatch (gguf/quant/mod.rs:42-50)
    if (n_elements % 256 != 0)
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT,
                    "K-quant payload needs n_elements a multiple of 256, got %zu", n_elements);
    const size_t nsb = n_elements / 256;
    if (n_bytes != nsb * bb)
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "tensor <dequant %d>: expected %zu bytes, got %zu", wdtype,
                    nsb * bb, n_bytes);
    if (nsb == 0) return VOKRA_HIP_OK;
    if (!bytes || !out) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "kquant_dequantize: NULL buffer");
    VK_TRY(set_dev(c), "hipSetDevice");
    VK_TRY(c->in0.ensure(n_bytes), "hipMalloc");
    VK_TRY(c->out0.ensure(n_elements * sizeof(float)), "hipMalloc");
    VK_TRY(hipMemcpyAsync(c->in0.p, bytes, n_bytes, hipMemcpyHostToDevice, c->stream), "hipMemcpyAsync(H2D)");
    VK_TRY(vk::launch_dequantize_kq(c->stream, wdtype, (const uint8_t*)c->in0.p, nsb, (float*)c->out0.p),
           "launch(K-quant dequantize)");
    VK_TRY(hipMemcpyAsync(out, c->out0.p, n_elements * sizeof(float), hipMemcpyDeviceToHost, c->stream),
           "hipMemcpyAsync(D2H)");
    VK_TRY(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    return VOKRA_HIP_OK;
}

int vokra_hip_dequant_gemv_f32(vokra_hip_ctx_t* c, int mode, const uint8_t* blocks, size_t n_bytes,
                               size_t n_rows, size_t n_bpr, const float* x, size_t x_len, float* y) {
    if (!c) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "fused_dequant_gemv: ctx is NULL");
    // validate_dequant_gemv (crates/vokra-core/src/kv_quant/gpu_ops.rs:95-131)
    if (mode == VOKRA_HIP_KV_FP32)
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT,
                    "fused_dequant_gemv: mode=Fp32 has no on-wire block layout; use dense_gemv_f32 instead");
    const int bb = kv_block_bytes(mode);
    if (bb == 0) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "fused_dequant_gemv: unknown mode %d", mode);
    size_t per_row = 0;
    if (!mul_ok(n_bpr, 32, &per_row) || x_len != per_row)
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT,
                    "fused_dequant_gemv: x.len()=%zu != n_blocks_per_row(%zu)*32", x_len, n_bpr);
    size_t rb, expected;
    if (!mul_ok(n_rows, n_bpr, &rb) || !mul_ok(rb, (size_t)bb, &expected))
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "fused_dequant_gemv: byte-length overflow");
    if (n_bytes != expected)
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT,
                    "fused_dequant_gemv: blocks_bytes.len()=%zu != n_rows(%zu)*n_blocks_per_row(%zu)*block_bytes(%d) "
                    "= %zu",
                    n_bytes, n_rows, n_bpr, bb, expected);
    if (n_rows == 0) return VOKRA_HIP_OK;  // the reference returns an empty Vec
    if (n_bpr == 0) {
        for (size_t i = 0; i < n_rows; ++i) y[i] = 0.0f;
        return VOKRA_HIP_OK;
    }
    if (n_rows > (size_t)INT32_MAX || n_bpr > 4096)
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT,
                    "fused_dequant_gemv: n_rows must fit int32 and n_blocks_per_row <= 4096");
    if (!blocks || !x || !y) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "fused_dequant_gemv: NULL buffer");
    VK_TRY(set_dev(c), "hipSetDevice");
    VK_TRY(c->in0.ensure(n_bytes), "hipMalloc");
    VK_TRY(c->in1.ensure(x_len * sizeof(float)), "hipMalloc");
    VK_TRY(c->out0.ensure(n_rows * sizeof(float)), "hipMalloc");
    VK_TRY(hipMemcpyAsync(c->in0.p, blocks, n_bytes, hipMemcpyHostToDevice, c->stream), "hipMemcpyAsync(H2D)");
    VK_TRY(hipMemcpyAsync(c->in1.p, x, x_len * sizeof(float), hipMemcpyHostToDevice, c->stream),
           "hipMemcpyAsync(H2D)");
    VK_TRY(vk::launch_dequant_gemv_f32(c->stream, mode, (const uint8_t*)c->in0.p, (int)n_rows, (int)n_bpr,
                                       (const float*)c->in1.p, (float*)c->out0.p),
           "launch(vk_dequant_gemv_f32)");
    VK_TRY(hipMemcpyAsync(y, c->out0.p, n_rows * sizeof(float), hipMemcpyDeviceToHost, c->stream),
           "hipMemcpyAsync(D2H)");
    VK_TRY(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    return VOKRA_HIP_OK;
}

int vokra_hip_set_act_quant(vokra_hip_ctx_t* c, int act_quant) {
    if (!c) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "set_act_quant: ctx is NULL");
    if (act_quant != VOKRA_HIP_ACT_AMAX127 && act_quant != VOKRA_HIP_ACT_POW2)
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "set_act_quant: unknown convention %d", act_quant);
    c->act_quant = act_quant;
    return VOKRA_HIP_OK;
}

int vokra_hip_qweight_upload(vokra_hip_ctx_t* c, int wdtype, size_t n, size_t k, const uint8_t* wq, size_t wq_len,
                             vokra_hip_qweight_t** out) {
    if (!c || !out) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "qweight_upload: NULL argument");
    *out = nullptr;
    int st = check_block_shapes(wdtype, n, k, wq_len);
    if (st) return st;
    if (n == 0) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "qweight_upload: n == 0");
    if (!wq) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "qweight_upload: NULL payload");
    VK_TRY(set_dev(c), "hipSetDevice");
    VK_TRY(c->in2.ensure(wq_len), "hipMalloc");
    VK_TRY(hipMemcpyAsync(c->in2.p, wq, wq_len, hipMemcpyHostToDevice, c->stream), "hipMemcpyAsync(H2D)");
    auto* w = new vokra_hip_qweight();
    st = upload_weight(c, wdtype, n, k, (const uint8_t*)c->in2.p, w);
    if (st == VOKRA_HIP_OK) {
        hipError_t e = hipStreamSynchronize(c->stream);
        if (e != hipSuccess) st = hip_fail(e, "hipStreamSynchronize");
    }
    if (st) {
        vokra_hip_qweight_free(w);
        return st;
    }
    *out = w;
    return VOKRA_HIP_OK;
}

void vokra_hip_qweight_free(vokra_hip_qweight_t* w) {
    if (!w) return;
    if (w->ctx) {
        (void)hipSetDevice(w->ctx->device);
        (void)hipStreamSynchronize(w->ctx->stream);
    }
    release_weight(w);
    delete w;
}

int vokra_hip_set_decode_kernel(vokra_hip_ctx_t* c, int enable) {
    if (!c) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "set_decode_kernel: ctx is NULL");
    c->decode_kernel = enable != 0;
    return VOKRA_HIP_OK;
}

int vokra_hip_gemm_q_f32_dev(vokra_hip_ctx_t* c, const vokra_hip_qweight_t* w, size_t m, const float* d_a,
                             const float* d_bias, float* d_out, int act_quant) {
    if (!c || !w) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "gemm_q_f32_dev: NULL context or weight");
    if (w->ctx != c) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "gemm_q_f32_dev: weight belongs to another context");
    if (m == 0)
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT,
                    "batched gemm_q_f32 needs at least one activation vector, got m = 0");
    if (m > (size_t)INT32_MAX / 2) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "gemm_q_f32_dev: m too large");
    if (act_quant != VOKRA_HIP_ACT_AMAX127 && act_quant != VOKRA_HIP_ACT_POW2 && act_quant != VOKRA_HIP_ACT_KQUANT)
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "gemm_q_f32_dev: unknown activation convention %d", act_quant);
    if (act_quant == VOKRA_HIP_ACT_KQUANT && !w->kquant)
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "gemm_q_f32_dev: KQUANT activations need K-quant weights");
    if (!d_a || !d_out) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "gemm_q_f32_dev: NULL buffer");
    VK_TRY(set_dev(c), "hipSetDevice");
    return run_gemm(c, w, m, d_a, d_bias, d_out, act_quant);
}

int vokra_hip_gemm_q_f32_dev_noalloc(vokra_hip_ctx_t* c, const vokra_hip_qweight_t* w, size_t m, const float* d_a,
                                     const float* d_bias, float* d_out, int act_quant) {
    if (!c || !w) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "gemm_q_f32_dev_noalloc: NULL context or weight");
    if (w->ctx != c)
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "gemm_q_f32_dev_noalloc: weight belongs to another context");
    if (m == 0)
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT,
                    "batched gemm_q_f32 needs at least one activation vector, got m = 0");
    if (act_quant != VOKRA_HIP_ACT_AMAX127 && act_quant != VOKRA_HIP_ACT_POW2 && act_quant != VOKRA_HIP_ACT_KQUANT)
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "gemm_q_f32_dev_noalloc: unknown activation convention %d",
                    act_quant);
    if (act_quant == VOKRA_HIP_ACT_KQUANT && !w->kquant)
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "gemm_q_f32_dev_noalloc: KQUANT activations need K-quant weights");
    if (!d_a || !d_out) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "gemm_q_f32_dev_noalloc: NULL buffer");
    // the workspace regions of qact_reserve(m, k), 256-byte aligned, in the static array
    const size_t k = w->k;
    if (m > ((size_t)1 << 30) / (k ? k : 1))
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "gemm_q_f32_dev_noalloc: m=%zu k=%zu too large", m, k);
    const size_t m_pad = round_up(m, vk::GEMM_TM), ng = k / 16;
    const size_t frag = round_up(m_pad * k * 2, 256), sc = round_up(m_pad * ng * sizeof(float), 256);
    const size_t need = frag + 2 * sc;
    if (need > kScratchBytes)
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT,
                    "gemm_q_f32_dev_noalloc: m=%zu k=%zu needs %zu bytes of workspace, the maximum is %zu "
                    "(use vokra_hip_gemm_q_f32_dev)",
                    m, k, need, kScratchBytes);
    if (!c->scratch) return fail(VOKRA_HIP_ERROR_BACKEND_UNAVAILABLE, "gemm_q_f32_dev_noalloc: no workspace address");
    VK_TRY(set_dev(c), "hipSetDevice");
    // a non-owning activation buffer over the workspace: fixed capacity,
    // never grown or freed (DevBuf frees only through release())
    vokra_hip_qact qa;
    qa.ctx = c;
    qa.max_m = m;
    qa.k = k;
    qa.growable = false;
    unsigned char* base = static_cast<unsigned char*>(c->scratch);
    qa.frag.p = base;
    qa.frag.cap = frag;
    // block formats use scale and gsum as two arrays; the K-quant layout
    // keeps (scale, sum) pairs in one array over both regions
    qa.scale.p = base + frag;
    qa.scale.cap = 2 * sc;
    qa.gsum.p = base + frag + sc;
    qa.gsum.cap = sc;
    int st = quantize_activations(c, &qa, d_a, m, k, w->kquant ? VOKRA_HIP_ACT_KQUANT : act_quant);
    if (st) return st;
    return run_gemm_qact(c, w, &qa, d_bias, d_out);
}

int vokra_hip_gemm_q_f32(vokra_hip_ctx_t* c, int wdtype, size_t m, size_t n, size_t k, const float* a, size_t a_len,
                         const uint8_t* wq, size_t wq_len, const float* bias, float* out, size_t out_len) {
    if (!c) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "gemm_q_f32: ctx is NULL");
    // kernels::gemm_q_f32 argument checks (kernels/mod.rs:351-358)
    size_t mk, mn;
    if (!mul_ok(m, k, &mk) || a_len != mk)
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "gemm_q a: length %zu != m*k", a_len);
    if (!mul_ok(m, n, &mn) || out_len != mn)
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "gemm_q out: length %zu != m*n", out_len);
    int st = check_block_shapes(wdtype, n, k, wq_len);
    if (st) return st;
    if (m == 0)
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT,
                    "batched gemm_q_f32 needs at least one activation vector, got m = 0");
    if (n == 0) return VOKRA_HIP_OK;
    if (!a || !wq || !out) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "gemm_q_f32: NULL buffer");
    VK_TRY(set_dev(c), "hipSetDevice");
    VK_TRY(c->in0.ensure(a_len * sizeof(float)), "hipMalloc");
    VK_TRY(c->in1.ensure(bias ? n * sizeof(float) : 4), "hipMalloc");
    VK_TRY(c->in2.ensure(wq_len), "hipMalloc");
    VK_TRY(c->out0.ensure(out_len * sizeof(float)), "hipMalloc");
    VK_TRY(hipMemcpyAsync(c->in0.p, a, a_len * sizeof(float), hipMemcpyHostToDevice, c->stream), "hipMemcpyAsync");
    VK_TRY(hipMemcpyAsync(c->in2.p, wq, wq_len, hipMemcpyHostToDevice, c->stream), "hipMemcpyAsync");
    if (bias)
        VK_TRY(hipMemcpyAsync(c->in1.p, bias, n * sizeof(float), hipMemcpyHostToDevice, c->stream),
               "hipMemcpyAsync");
    vokra_hip_qweight w;
    st = upload_weight(c, wdtype, n, k, (const uint8_t*)c->in2.p, &w);
    if (st == VOKRA_HIP_OK)
        st = run_gemm(c, &w, m, (const float*)c->in0.p, bias ? (const float*)c->in1.p : nullptr, (float*)c->out0.p,
                      c->act_quant);
    if (st == VOKRA_HIP_OK) {
        hipError_t e = hipMemcpyAsync(out, c->out0.p, out_len * sizeof(float), hipMemcpyDeviceToHost, c->stream);
        if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
        if (e != hipSuccess) st = hip_fail(e, "gemm_q_f32 readback");
    } else {
        (void)hipStreamSynchronize(c->stream);
    }
    release_weight(&w);
    return st;
}

int vokra_hip_capture_begin(vokra_hip_ctx_t* c) {
    if (!c) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "capture_begin: ctx is NULL");
    VK_TRY(set_dev(c), "hipSetDevice");
    VK_TRY(hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
    return VOKRA_HIP_OK;
}

int vokra_hip_capture_end(vokra_hip_ctx_t* c, vokra_hip_graph_t** out) {
    if (!c || !out) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "capture_end: NULL argument");
    *out = nullptr;
    VK_TRY(set_dev(c), "hipSetDevice");
    auto* g = new vokra_hip_graph();
    hipError_t e = hipStreamEndCapture(c->stream, &g->graph);
    if (e == hipSuccess) e = hipGraphInstantiate(&g->exec, g->graph, nullptr, nullptr, 0);
    // the executable graph goes to the device now, so its first launch costs
    // what every later one does
    if (e == hipSuccess) e = hipGraphUpload(g->exec, c->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    if (e != hipSuccess) {
        vokra_hip_graph_destroy(g);
        return hip_fail(e, "hipStreamEndCapture/hipGraphInstantiate/hipGraphUpload");
    }
    *out = g;
    return VOKRA_HIP_OK;
}

int vokra_hip_graph_launch(vokra_hip_ctx_t* c, vokra_hip_graph_t* g) {
    if (!c || !g) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "graph_launch: NULL argument");
    VK_TRY(set_dev(c), "hipSetDevice");
    VK_TRY(hipGraphLaunch(g->exec, c->stream), "hipGraphLaunch");
    return VOKRA_HIP_OK;
}

void vokra_hip_graph_destroy(vokra_hip_graph_t* g) {
    if (!g) return;
    if (g->exec) (void)hipGraphExecDestroy(g->exec);
    if (g->graph) (void)hipGraphDestroy(g->graph);
    delete g;
}

int vokra_hip_copy_dev(vokra_hip_ctx_t* c, void* d_dst, const void* d_src, size_t bytes) {
    if (!c) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "copy_dev: ctx is NULL");
    if (bytes % 16 != 0 || ((reinterpret_cast<uintptr_t>(d_dst) | reinterpret_cast<uintptr_t>(d_src)) & 15))
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "copy_dev: needs 16-byte aligned pointers and size");
    if (bytes == 0) return VOKRA_HIP_OK;
    if (!d_dst || !d_src) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "copy_dev: NULL buffer");
    VK_TRY(set_dev(c), "hipSetDevice");
    VK_TRY(vk::launch_copy_u4(c->stream, d_src, d_dst, bytes / 16), "launch(vk_copy_u4)");
    return VOKRA_HIP_OK;
}

int vokra_hip_quantize_bytes_dev(vokra_hip_ctx_t* c, int mode, const float* d_x, size_t n, uint8_t* d_out) {
    if (!c) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "quantize_bytes: ctx is NULL");
    if (kv_block_bytes(mode) == 0)
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "pack_matrix_to_bytes: mode %d has no packed layout", mode);
    if (n % 32 != 0)
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT,
                    "kv_quant::pack_slice: input.len()=%zu not a multiple of 32", n);
    if (n == 0) return VOKRA_HIP_OK;
    if (!d_x || !d_out) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "quantize_bytes: NULL buffer");
    VK_TRY(set_dev(c), "hipSetDevice");
    VK_TRY(vk::launch_pack_q0(c->stream, mode, d_x, n / 32, d_out), "launch(vk_pack_q0)");
    return VOKRA_HIP_OK;
}

int vokra_hip_quantize_bytes(vokra_hip_ctx_t* c, int mode, const float* x, size_t n, uint8_t* out, size_t out_len) {
    if (!c) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "quantize_bytes: ctx is NULL");
    const int bb = kv_block_bytes(mode);
    if (bb == 0)
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "pack_matrix_to_bytes: mode %d has no packed layout", mode);
    if (n % 32 != 0)
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT,
                    "kv_quant::pack_slice: input.len()=%zu not a multiple of 32", n);
    if (out_len != n / 32 * (size_t)bb)
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "quantize_bytes: out_len %zu != %zu blocks x %d bytes",
                    out_len, n / 32, bb);
    if (n == 0) return VOKRA_HIP_OK;
    if (!x || !out) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "quantize_bytes: NULL buffer");
    VK_TRY(set_dev(c), "hipSetDevice");
    VK_TRY(c->in0.ensure(n * sizeof(float)), "hipMalloc");
    VK_TRY(c->out0.ensure(out_len), "hipMalloc");
    VK_TRY(hipMemcpyAsync(c->in0.p, x, n * sizeof(float), hipMemcpyHostToDevice, c->stream), "hipMemcpyAsync(H2D)");
    VK_TRY(vk::launch_pack_q0(c->stream, mode, (const float*)c->in0.p, n / 32, (uint8_t*)c->out0.p),
           "launch(vk_pack_q0)");
    VK_TRY(hipMemcpyAsync(out, c->out0.p, out_len, hipMemcpyDeviceToHost, c->stream), "hipMemcpyAsync(D2H)");
    VK_TRY(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    return VOKRA_HIP_OK;
}

int vokra_hip_qact_create(vokra_hip_ctx_t* c, size_t max_m, size_t k, vokra_hip_qact_t** out) {
    if (!c || !out) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "qact_create: NULL argument");
    *out = nullptr;
    if (max_m == 0 || k == 0 || k % 32 != 0 || max_m > (size_t)INT32_MAX / 2 || k > (size_t)INT32_MAX)
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT,
                    "qact_create: need max_m > 0 and k a positive multiple of 32 (got %zu, %zu)", max_m, k);
    VK_TRY(set_dev(c), "hipSetDevice");
    auto* qa = new vokra_hip_qact();
    qa->ctx = c;
    qa->max_m = max_m;
    qa->k = k;
    int st = qact_reserve(qa, max_m, k);
    if (st) {
        vokra_hip_qact_free(qa);
        return st;
    }
    *out = qa;
    return VOKRA_HIP_OK;
}

void vokra_hip_qact_free(vokra_hip_qact_t* qa) {
    if (!qa) return;
    if (qa->ctx) {
        (void)hipSetDevice(qa->ctx->device);
        (void)hipStreamSynchronize(qa->ctx->stream);
    }
    qa->frag.release();
    qa->scale.release();
    qa->gsum.release();
    delete qa;
}

int vokra_hip_qact_quantize_dev(vokra_hip_ctx_t* c, vokra_hip_qact_t* qa, size_t m, const float* d_a,
                                int act_quant) {
    if (!c || !qa || !d_a) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "qact_quantize: NULL argument");
    if (qa->ctx != c) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "qact_quantize: qact belongs to another context");
    if (m == 0 || m > qa->max_m)
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "qact_quantize: m=%zu outside 1..%zu", m, qa->max_m);
    if (act_quant != VOKRA_HIP_ACT_AMAX127 && act_quant != VOKRA_HIP_ACT_POW2 && act_quant != VOKRA_HIP_ACT_KQUANT)
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "qact_quantize: unknown activation convention %d", act_quant);
    VK_TRY(set_dev(c), "hipSetDevice");
    return quantize_activations(c, qa, d_a, m, qa->k, act_quant);
}

int vokra_hip_gemm_qact_dev(vokra_hip_ctx_t* c, const vokra_hip_qweight_t* w, const vokra_hip_qact_t* qa,
                            const float* d_bias, float* d_out) {
    return vk::gemm_qact_epi(c, w, qa, d_bias, d_out, VkEpi{nullptr, 0});
}

// ---- grouped decode linears ---------------------------------------------------

struct vokra_hip_linear_group {
    vokra_hip_ctx* ctx = nullptr;
    size_t k = 0, nb = 0, n_max = 0;
    int wdtype = 0;
    std::vector<const vokra_hip_qweight*> ws;
    std::vector<const float*> biases;
    std::vector<float*> outs;
    DevBuf desc;  // VkGemvLin[count], read by the decode kernel
};

int vokra_hip_linear_group_create(vokra_hip_ctx_t* c, size_t count, const vokra_hip_qweight_t* const* weights,
                                  const float* const* d_biases, float* const* d_outs, vokra_hip_linear_group_t** out) {
    if (!c || !out) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "linear_group_create: NULL argument");
    *out = nullptr;
    if (count == 0 || count > 65535)
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "linear_group_create: count %zu outside 1..65535", count);
    if (!weights || !d_outs) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "linear_group_create: NULL list");
    std::vector<VkGemvLin> lins(count);
    size_t n_max = 0;
    for (size_t i = 0; i < count; ++i) {
        const vokra_hip_qweight* w = weights[i];
        if (!w || !d_outs[i]) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "linear_group_create: NULL entry %zu", i);
        if (w->ctx != c)
            return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "linear_group_create: weight %zu belongs to another context", i);
        if (w->kquant || !w->has_gemv)
            return fail(VOKRA_HIP_ERROR_UNSUPPORTED_OP,
                        "linear_group_create: weight %zu has no decode layout (Q4_0 / Q8_0 with k %% 128 == 0)", i);
        if (w->wdtype != weights[0]->wdtype || w->k != weights[0]->k)
            return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT,
                        "linear_group_create: weight %zu differs from weight 0 in dtype or k", i);
        if (!fits_int(w->n)) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "linear_group_create: n exceeds int32");
        lins[i] = {(const uint4*)w->gq.p, (const uint2*)w->gsc.p, d_biases ? d_biases[i] : nullptr, d_outs[i],
                   {nullptr, 0}, (int)w->n};
        n_max = std::max(n_max, w->n);
    }
    VK_TRY(set_dev(c), "hipSetDevice");
    vokra_hip_linear_group* g = new (std::nothrow) vokra_hip_linear_group;
    if (!g) return fail(VOKRA_HIP_ERROR_OTHER, "linear_group_create: out of host memory");
    g->ctx = c;
    g->k = weights[0]->k;
    g->nb = weights[0]->nb;
    g->n_max = n_max;
    g->wdtype = weights[0]->wdtype;
    g->ws.assign(weights, weights + count);
    g->biases.resize(count);
    for (size_t i = 0; i < count; ++i) g->biases[i] = d_biases ? d_biases[i] : nullptr;
    g->outs.assign(d_outs, d_outs + count);
    hipError_t e = g->desc.ensure(count * sizeof(VkGemvLin));
    if (e == hipSuccess)
        e = hipMemcpyAsync(g->desc.p, lins.data(), count * sizeof(VkGemvLin), hipMemcpyHostToDevice, c->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    if (e != hipSuccess) {
        g->desc.release();
        delete g;
        return fail(VOKRA_HIP_ERROR_BACKEND_UNAVAILABLE, "linear_group_create: %s", hipGetErrorString(e));
    }
    *out = g;
    return VOKRA_HIP_OK;
}

int vokra_hip_linear_group_run(vokra_hip_ctx_t* c, vokra_hip_linear_group_t* g, const vokra_hip_qact_t* qa) {
    if (!c || !g || !qa) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "linear_group_run: NULL argument");
    if (g->ctx != c || qa->ctx != c)
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "linear_group_run: group/activations belong to another context");
    if (qa->m == 0) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "linear_group_run: activations were never quantized");
    if (qa->k != g->k)
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "linear_group_run: activation k=%zu != weight k=%zu", qa->k, g->k);
    if (qa->act_quant == VOKRA_HIP_ACT_KQUANT)
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT,
                    "linear_group_run: block-format weights need AMAX127 or POW2 activations");
    VK_TRY(set_dev(c), "hipSetDevice");
    if (qa->m > kGemvMaxM || !c->decode_kernel) {  // prefill rows: the block GEMM, one launch per linear
        for (size_t i = 0; i < g->ws.size(); ++i) {
            int st = run_gemm_qact(c, g->ws[i], qa, g->biases[i], g->outs[i]);
            if (st) return st;
        }
        return VOKRA_HIP_OK;
    }
    VK_TRY(vk::launch_gemv_qblock_group(c->stream, wd_kv_mode(g->wdtype), qa->act_quant == VOKRA_HIP_ACT_POW2,
                                        (const uint4*)qa->frag.p, (const float*)qa->scale.p, (const float*)qa->gsum.p,
                                        (const VkGemvLin*)g->desc.p, (int)g->ws.size(), (int)g->n_max, (int)qa->m,
                                        (int)g->nb, (int)qa->m_pad),
           "launch(vk_gemv_qblock group)");
    return VOKRA_HIP_OK;
}

void vokra_hip_linear_group_destroy(vokra_hip_linear_group_t* g) {
    if (!g) return;
    (void)hipSetDevice(g->ctx->device);
    (void)hipStreamSynchronize(g->ctx->stream);
    g->desc.release();
    delete g;
}

// ---- Whisper front end ------------------------------------------------------

int vokra_hip_log_mel_dev(vokra_hip_ctx_t* c, const float* d_pcm, size_t batch, size_t n_samples, size_t n_mels,
                          float* d_out) {
    if (!c) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "log_mel: ctx is NULL");
    int st = check_log_mel(batch, n_samples, n_mels);
    if (st) return st;
    if (!d_out || (n_samples && !d_pcm)) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "log_mel: NULL buffer");
    VK_TRY(set_dev(c), "hipSetDevice");
    return run_log_mel(c, d_pcm, batch, n_samples, n_mels, d_out);
}

int vokra_hip_log_mel(vokra_hip_ctx_t* c, const float* pcm, size_t batch, size_t n_samples, size_t n_mels, float* out,
                      size_t out_len) {
    if (!c) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "log_mel: ctx is NULL");
    int st = check_log_mel(batch, n_samples, n_mels);
    if (st) return st;
    const size_t want = batch * n_mels * (size_t)vk::fe_n_frames();
    if ((st = expect_len("log_mel out", out_len, want))) return st;
    if (!out || (n_samples && !pcm)) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "log_mel: NULL buffer");
    VK_TRY(set_dev(c), "hipSetDevice");
    if ((st = stage_in(c, c->in0, pcm, batch * n_samples))) return st;
    VK_TRY(c->out0.ensure(want * sizeof(float)), "hipMalloc");
    if ((st = run_log_mel(c, (const float*)c->in0.p, batch, n_samples, n_mels, (float*)c->out0.p))) return st;
    return stage_out(c, out, c->out0.p, want);
}

int vokra_hip_conv1d_f32_dev(vokra_hip_ctx_t* c, const float* d_in, size_t in_ch, size_t in_len, const float* d_w,
                             size_t out_ch, size_t kernel, const float* d_bias, size_t stride, size_t padding,
                             float* d_out) {
    if (!c) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "conv1d: ctx is NULL");
    size_t out_len = 0, kk = 0, col_n = 0;
    int st = conv1d_out(in_len, kernel, stride, padding, &out_len);
    if (st) return st;
    if (!mul_ok(in_ch, kernel, &kk) || !mul_ok(kk, out_len, &col_n) || !fits_int(kk) || !fits_int(out_len) ||
        !fits_int(out_ch) || !fits_int(in_len) || !fits_int(stride) || !fits_int(padding))
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "conv1d: extent exceeds int32");
    if (out_ch == 0 || out_len == 0) return VOKRA_HIP_OK;
    if (!d_out || !d_w || (in_ch && !d_in)) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "conv1d: NULL buffer");
    VK_TRY(set_dev(c), "hipSetDevice");
    VK_TRY(c->cv_col.ensure(col_n * sizeof(float) + 16), "hipMalloc(im2col)");
    VK_TRY(vk::launch_im2col(c->stream, false, d_in, 0, in_len, 1, 1, (int)in_ch, (int)in_len, (int)kernel, (int)stride,
                             (int)padding, (int)out_len, (float*)c->cv_col.p),
           "launch(vk_im2col)");
    VK_TRY(vk::launch_gemm_f32(c->stream, false, d_w, (const float*)c->cv_col.p, nullptr, d_out, (int)out_ch,
                               (int)out_len, (int)kk),
           "launch(vk_gemm_f32 conv)");
    if (d_bias)
        VK_TRY(vk::launch_add_row_bias(c->stream, d_out, d_bias, (int)out_ch, (int)out_len), "launch(vk_add_row_bias)");
    return VOKRA_HIP_OK;
}

int vokra_hip_conv1d_f32(vokra_hip_ctx_t* c, const float* input, size_t in_len_total, size_t in_ch, size_t in_len,
                         const float* weight, size_t w_len, size_t out_ch, size_t kernel, const float* bias,
                         size_t stride, size_t padding, float* out, size_t out_len_total) {
    if (!c) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "conv1d: ctx is NULL");
    size_t out_len = 0, n_in = 0, n_w = 0, n_out = 0, kk = 0;
    int st = conv1d_out(in_len, kernel, stride, padding, &out_len);
    if (st) return st;
    if (!mul_ok(in_ch, in_len, &n_in) || !mul_ok(in_ch, kernel, &kk) || !mul_ok(out_ch, kk, &n_w) ||
        !mul_ok(out_ch, out_len, &n_out))
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "conv1d: extent overflows");
    if ((st = expect_len("conv1d input", in_len_total, n_in)) || (st = expect_len("conv1d weight", w_len, n_w)) ||
        (st = expect_len("conv1d out", out_len_total, n_out)))
        return st;
    if (n_out == 0) return VOKRA_HIP_OK;
    VK_TRY(set_dev(c), "hipSetDevice");
    if ((st = stage_in(c, c->in0, input, n_in)) || (st = stage_in(c, c->in1, weight, n_w)) ||
        (st = stage_in(c, c->in2, bias, bias ? out_ch : 0)))
        return st;
    VK_TRY(c->out0.ensure(n_out * sizeof(float)), "hipMalloc");
    st = vokra_hip_conv1d_f32_dev(c, (const float*)c->in0.p, in_ch, in_len, (const float*)c->in1.p, out_ch, kernel,
                                  bias ? (const float*)c->in2.p : nullptr, stride, padding, (float*)c->out0.p);
    if (st) return st;
    return stage_out(c, out, c->out0.p, n_out);
}

}  // extern "C"


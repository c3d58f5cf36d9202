// vk_session.hip — device-resident model sessions built on the library's own
// entry points: the pre-norm encoder (crates/vokra-models/src/whisper/
// encoder.rs:41-245) and the batched Whisper decoder step (decoder.rs:413-796).
//
// Everything a forward or a step touches stays in HBM: quantized weights are
// uploaded once, activations live in session workspaces, the self-attention
// K/V go to the paged Q8_0 cache, and the cross-attention K/V of each
// (stream, layer) are projected once per utterance and stored already split
// into fp16 hi/lo halves for the fused attention kernel.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <vector>

#include "../../include/vokra_hip.h"
#include "vk_launch.h"

namespace vk {

// Per-step indices: lens[i] = positions[i] + 1 (keys 0..t after the append)
// and, per layer, the cross K/V batch of item i, streams[i] * n_layer + l.
__global__ void vk_step_index(const int* __restrict__ streams, const int* __restrict__ positions, int n, int n_layer,
                              int* __restrict__ lens, int* __restrict__ kvidx) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    lens[i] = positions[i] + 1;
    for (int l = 0; l < n_layer; ++l) kvidx[l * n + i] = streams[i] * n_layer + l;
}

}  // namespace vk

namespace {

constexpr float kLnEps = 1e-5f;  // LAYER_NORM_DEFAULT_EPS (crates/vokra-backend-cpu/src/kernels/scalar.rs:26)

#define SS_TRY(x)                \
    do {                         \
        int _st = (x);           \
        if (_st) return _st;     \
    } while (0)
#define SS_HIP(x, what)                                                                    \
    do {                                                                                   \
        hipError_t _e = (x);                                                               \
        if (_e != hipSuccess) return vk::ctx_fail(VOKRA_HIP_ERROR_BACKEND_UNAVAILABLE, "%s", what); \
    } while (0)

size_t wire_bytes(int wdtype, size_t n, size_t k) {
    switch (wdtype) {
    case VOKRA_HIP_W_Q4_0: return n * (k / 32) * 18;
    case VOKRA_HIP_W_Q5_0: return n * (k / 32) * 22;
    case VOKRA_HIP_W_Q8_0: return n * (k / 32) * 34;
    case VOKRA_HIP_W_Q4_K: return n * (k / 256) * 144;
    case VOKRA_HIP_W_Q5_K: return n * (k / 256) * 176;
    case VOKRA_HIP_W_Q6_K: return n * (k / 256) * 210;
    default: return 0;
    }
}

// A device buffer owned by a session.
struct DBuf {
    void* p = nullptr;
    int alloc(vokra_hip_ctx_t* c, size_t n) { return vokra_hip_device_alloc(c, n ? n : 16, &p); }
    int upload(vokra_hip_ctx_t* c, const void* h, size_t n) {
        SS_TRY(alloc(c, n));
        return n ? vokra_hip_memcpy_htod(c, p, h, n) : VOKRA_HIP_OK;
    }
    void release(vokra_hip_ctx_t* c) {
        if (p) (void)vokra_hip_device_free(c, p);
        p = nullptr;
    }
    float* f() const { return (float*)p; }
    int* i() const { return (int*)p; }
};

// A quantized linear: resident weight [n, k] plus an optional f32 bias.
struct QLin {
    vokra_hip_qweight_t* w = nullptr;
    DBuf bias;
    bool has_bias = false;
    int make(vokra_hip_ctx_t* c, int wdtype, size_t n, size_t k, const uint8_t* wq, const float* b) {
        if (!wq) return vk::ctx_fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "session: a weight pointer is NULL");
        SS_TRY(vokra_hip_qweight_upload(c, wdtype, n, k, wq, wire_bytes(wdtype, n, k), &w));
        has_bias = b != nullptr;
        if (has_bias) SS_TRY(bias.upload(c, b, n * sizeof(float)));
        return VOKRA_HIP_OK;
    }
    int run(vokra_hip_ctx_t* c, const vokra_hip_qact_t* qa, float* d_out, VkEpi epi = {nullptr, 0}) const {
        return vk::gemm_qact_epi(c, w, qa, b(), d_out, epi);
    }
    // the same, then the activation pass over the outputs into qa_out (fused
    // into the GEMM epilogue where it has a fused form; d_out is scratch)
    int run_quantize(vokra_hip_ctx_t* c, const vokra_hip_qact_t* qa, float* d_out, VkEpi epi,
                     vokra_hip_qact_t* qa_out, int act) const {
        return vk::gemm_qact_quantize(c, w, qa, b(), d_out, epi, qa_out, act);
    }
    const float* b() const { return has_bias ? bias.f() : nullptr; }
    void release(vokra_hip_ctx_t* c) {
        vokra_hip_qweight_free(w);
        w = nullptr;
        bias.release(c);
    }
};

int upload_vec(vokra_hip_ctx_t* c, DBuf& b, const float* h, size_t n, const char* what) {
    if (!h) return vk::ctx_fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "%s", what);
    return b.upload(c, h, n * sizeof(float));
}

bool is_kquant(int wdtype) {
    return wdtype == VOKRA_HIP_W_Q4_K || wdtype == VOKRA_HIP_W_Q5_K || wdtype == VOKRA_HIP_W_Q6_K;
}
int act_of(int wdtype) { return is_kquant(wdtype) ? VOKRA_HIP_ACT_KQUANT : VOKRA_HIP_ACT_AMAX127; }

int check_model_dims(int wdtype, size_t d, size_t n_head, size_t d_ff) {
    if (wire_bytes(wdtype, 1, 256) == 0) return vk::ctx_fail(VOKRA_HIP_ERROR_UNSUPPORTED_OP, "session: unknown weight dtype");
    if (!d || !n_head || d % n_head != 0)
        return vk::ctx_fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "session: d_model must be a multiple of n_head");
    const size_t hd = d / n_head;
    if (hd != 64 && hd != 128) return vk::ctx_fail(VOKRA_HIP_ERROR_UNSUPPORTED_OP, "session: head_dim must be 64 or 128");
    const size_t q = is_kquant(wdtype) ? 256 : 32;
    if (d % q != 0 || d_ff % q != 0 || !d_ff)
        return vk::ctx_fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "session: d_model and d_ff must be multiples of the quant block");
    return VOKRA_HIP_OK;
}

struct EncLayer {
    DBuf ln1g, ln1b, ln2g, ln2b;
    QLin q, k, v, o, fc1, fc2;
};

struct DecLayer {
    DBuf ln1g, ln1b, ln2g, ln2b, ln3g, ln3b;
    QLin q, k, v, o, cq, ck, cv, co, fc1, fc2;
};

}  // namespace

struct vokra_hip_encoder {
    vokra_hip_ctx_t* ctx = nullptr;
    int wdtype = 0;
    size_t n_layer = 0, d = 0, n_head = 0, hd = 0, d_ff = 0, max_rows = 0;
    std::vector<EncLayer> layers;
    DBuf lnpg, lnpb, h, x, q, k, v, attn, f;
    vokra_hip_qact_t *qa_d = nullptr, *qa_f = nullptr;
    // conv stem (optional): weights, positional embedding, im2col / conv1 workspaces
    size_t n_mels = 0, n_frames = 0, n_ctx = 0, stem_batch = 0;
    DBuf c1w, c1b, c2w, c2b, pos, col1, c1, col2;
    // attention V^T as fp16 hi / lo [batch][d / hd][hd][t_pad] (the v split
    // pass's output; k's hi / lo, written by the q/k/v GEMM, take k's own
    // buffer)
    DBuf vt_hi, vt_lo;
    size_t vt_cap = 0;
    void release() {
        for (auto& L : layers) {
            for (DBuf* b : {&L.ln1g, &L.ln1b, &L.ln2g, &L.ln2b}) b->release(ctx);
            for (QLin* w : {&L.q, &L.k, &L.v, &L.o, &L.fc1, &L.fc2}) w->release(ctx);
        }
        for (DBuf* b : {&lnpg, &lnpb, &h, &x, &q, &k, &v, &attn, &f, &c1w, &c1b, &c2w, &c2b, &pos, &col1, &c1, &col2,
                        &vt_hi, &vt_lo})
            b->release(ctx);
        vt_cap = 0;
        vokra_hip_qact_free(qa_d);
        vokra_hip_qact_free(qa_f);
        qa_d = qa_f = nullptr;
    }
};

struct vokra_hip_decoder {
    vokra_hip_ctx_t* ctx = nullptr;
    int wdtype = 0;
    size_t n_layer = 0, d = 0, n_head = 0, hd = 0, d_ff = 0, vocab = 0, n_text = 0, n_audio = 0, n_stream = 0;
    size_t t_pad = 0;
    std::vector<DecLayer> layers;
    DBuf tok_emb, pos_emb, lnpg, lnpb;
    vokra_hip_kv_t* kv = nullptr;
    DBuf ckh, ckl, cvh, cvl;  // cross K and V^T per (stream, layer): fp16 high parts, one-byte low parts
    int cross_precision = VOKRA_HIP_CROSS_F32;  // F16: cross-attention reads the hi parts only
    DBuf h, x, q, k, v, attn, f, logits, lpart, lens, kvidx, next, tk, tv, stage;
    vokra_hip_qact_t *qa_d = nullptr, *qa_f = nullptr;
    // host mirror of each stream's state: cross K/V set from an encoder
    // output, and the number of positions in its self-KV history
    std::vector<char> enc_set;
    std::vector<int32_t> length;
    void release() {
        for (auto& L : layers) {
            for (DBuf* b : {&L.ln1g, &L.ln1b, &L.ln2g, &L.ln2b, &L.ln3g, &L.ln3b}) b->release(ctx);
            for (QLin* w : {&L.q, &L.k, &L.v, &L.o, &L.cq, &L.ck, &L.cv, &L.co, &L.fc1, &L.fc2}) w->release(ctx);
        }
        for (DBuf* b : {&tok_emb, &pos_emb, &lnpg, &lnpb, &ckh, &ckl, &cvh, &cvl, &h, &x, &q, &k, &v, &attn, &f,
                        &logits, &lpart, &lens, &kvidx, &next, &tk, &tv, &stage})
            b->release(ctx);
        vokra_hip_kv_destroy(kv);
        kv = nullptr;
        vokra_hip_qact_free(qa_d);
        vokra_hip_qact_free(qa_f);
        qa_d = qa_f = nullptr;
    }
};

namespace {

int enc_setup(vokra_hip_encoder* e, const vokra_hip_prenorm_layer_t* layers, const float* lpg, const float* lpb) {
    vokra_hip_ctx_t* c = e->ctx;
    const size_t d = e->d, ff = e->d_ff;
    e->layers.resize(e->n_layer);
    for (size_t l = 0; l < e->n_layer; ++l) {
        const vokra_hip_prenorm_layer_t& s = layers[l];
        EncLayer& L = e->layers[l];
        SS_TRY(upload_vec(c, L.ln1g, s.ln1_gamma, d, "encoder: ln1_gamma is NULL"));
        SS_TRY(upload_vec(c, L.ln1b, s.ln1_beta, d, "encoder: ln1_beta is NULL"));
        SS_TRY(upload_vec(c, L.ln2g, s.ln2_gamma, d, "encoder: ln2_gamma is NULL"));
        SS_TRY(upload_vec(c, L.ln2b, s.ln2_beta, d, "encoder: ln2_beta is NULL"));
        SS_TRY(L.q.make(c, e->wdtype, d, d, s.wq, s.bq));
        SS_TRY(L.k.make(c, e->wdtype, d, d, s.wk, s.bk));
        SS_TRY(L.v.make(c, e->wdtype, d, d, s.wv, s.bv));
        SS_TRY(L.o.make(c, e->wdtype, d, d, s.wo, s.bo));
        SS_TRY(L.fc1.make(c, e->wdtype, ff, d, s.w1, s.b1));
        SS_TRY(L.fc2.make(c, e->wdtype, d, ff, s.w2, s.b2));
    }
    SS_TRY(upload_vec(c, e->lnpg, lpg, d, "encoder: ln_post_gamma is NULL"));
    SS_TRY(upload_vec(c, e->lnpb, lpb, d, "encoder: ln_post_beta is NULL"));
    const size_t rd = e->max_rows * d * sizeof(float);
    for (DBuf* b : {&e->h, &e->x, &e->q, &e->k, &e->v, &e->attn}) SS_TRY(b->alloc(c, rd));
    SS_TRY(e->f.alloc(c, e->max_rows * ff * sizeof(float)));
    SS_TRY(vokra_hip_qact_create(c, e->max_rows, d, &e->qa_d));
    SS_TRY(vokra_hip_qact_create(c, e->max_rows, ff, &e->qa_f));
    return VOKRA_HIP_OK;
}

// V^T hi / lo buffers of at least `bytes` each (the split pass writes every
// element, zeros past each row's frames)
int enc_vt_ensure(vokra_hip_encoder* e, size_t bytes) {
    if (bytes <= e->vt_cap) return VOKRA_HIP_OK;
    e->vt_hi.release(e->ctx);
    e->vt_lo.release(e->ctx);
    e->vt_cap = 0;
    SS_TRY(e->vt_hi.alloc(e->ctx, bytes));
    SS_TRY(e->vt_lo.alloc(e->ctx, bytes));
    e->vt_cap = bytes;
    return VOKRA_HIP_OK;
}

int enc_forward(vokra_hip_encoder* e, size_t batch, size_t frames, const float* d_x, float* d_out) {
    vokra_hip_ctx_t* c = e->ctx;
    const size_t rows = batch * frames, d = e->d;
    const int act = act_of(e->wdtype);
    const float scale = powf((float)e->hd, -0.5f);  // (hd as f32).powf(-0.5), nn.rs:267
    const size_t t_pad = (frames + 63) / 64 * 64;
    SS_HIP(hipMemcpyAsync(e->h.p, d_x, rows * d * sizeof(float), hipMemcpyDeviceToDevice, vk::ctx_stream(c)),
           "encoder: hipMemcpyAsync");
    // Per block the entry-point sequence is LN -> quantize -> q/k/v -> attention
    // -> quantize -> out-proj -> + h, LN -> quantize -> fc1 -> GELU -> quantize
    // -> fc2 -> + h; LN + quantize, out-proj + residual and fc1 + GELU run as
    // one kernel each (vk::qact_ln_quantize, VkEpi), with the same results.
    const VkEpi add_h = {e->h.f(), 0}, gelu = {nullptr, 1};
    for (const EncLayer& L : e->layers) {
        // attention block (encoder.rs:180-220)
        SS_TRY(vk::qact_ln_quantize(c, e->qa_d, rows, e->h.f(), L.ln1g.f(), L.ln1b.f(), kLnEps, act, e->x.f()));
        const vokra_hip_qweight_t* qkv[3] = {L.q.w, L.k.w, L.v.w};
        const float* qkv_b[3] = {L.q.b(), L.k.b(), L.v.b()};
        // k leaves the GEMM as the attention kernel's fp16 hi / lo operands
        // (no k split pass); q stays f32 (the kernel splits it), v is split
        // and transposed by its pass
        bool fused = false;
        uint16_t* kh = (uint16_t*)e->k.p;
        uint16_t* kl = kh + rows * d;
        if (frames >= 2) {
            SS_TRY(enc_vt_ensure(e, batch * d * t_pad * sizeof(uint16_t)));
            SS_TRY(vk::gemm_qact_qkv_split(c, qkv, e->qa_d, qkv_b, e->q.f(), VkSplitOut{kh, kl}, e->v.f(), &fused));
        }
        if (fused) {
            SS_HIP(vk::launch_split_vt(vk::ctx_stream(c), e->v.f(), (int)batch, (int)frames, (int)t_pad,
                                       (int)e->n_head, (int)e->hd, e->vt_hi.p, e->vt_lo.p),
                   "launch(vk_split_vt)");
            SS_TRY(vk::attn_quantize_split(c, batch, frames, e->n_head, e->hd, e->q.f(), kh, kl, e->vt_hi.p,
                                           e->vt_lo.p, t_pad, scale, e->attn.f(), e->qa_d, act));
        } else {
            float* qkv_o[3] = {e->q.f(), e->k.f(), e->v.f()};
            SS_TRY(vk::gemm_qact_multi(c, 3, qkv, e->qa_d, qkv_b, qkv_o));
            SS_TRY(vk::attn_quantize(c, batch, frames, frames, e->n_head, e->n_head, e->hd, e->q.f(), e->k.f(),
                                     e->v.f(), scale, 0, 0, e->attn.f(), e->qa_d, act));
        }
        SS_TRY(L.o.run(c, e->qa_d, e->h.f(), add_h));
        // MLP block (nn.rs:134-181)
        SS_TRY(vk::qact_ln_quantize(c, e->qa_d, rows, e->h.f(), L.ln2g.f(), L.ln2b.f(), kLnEps, act, e->x.f()));
        SS_TRY(L.fc1.run_quantize(c, e->qa_d, e->f.f(), gelu, e->qa_f, act));
        SS_TRY(L.fc2.run(c, e->qa_f, e->h.f(), add_h));
    }
    return vokra_hip_layer_norm_f32_dev(c, e->h.f(), d_out, rows, d, e->lnpg.f(), e->lnpb.f(), kLnEps);
}

// The conv stem of WhisperEncoder::encode (crates/vokra-models/src/whisper/
// encoder.rs:58-104) as im2col + f32 GEMM with bias and GELU in the GEMM
// epilogue, conv outputs kept time-major ([frames, d]), then + pos_emb, into
// d_x [batch, n_ctx, d].
int enc_stem(vokra_hip_encoder* e, size_t batch, const float* d_mel, float* d_x) {
    vokra_hip_ctx_t* c = e->ctx;
    hipStream_t s = vk::ctx_stream(c);
    const size_t d = e->d, nm = e->n_mels, nf = e->n_frames, nc = e->n_ctx;
    if (batch > e->stem_batch) {  // workspaces grow with the largest batch seen
        for (DBuf* b : {&e->col1, &e->c1, &e->col2}) b->release(c);
        SS_TRY(e->col1.alloc(c, batch * nf * nm * 3 * sizeof(float)));
        SS_TRY(e->c1.alloc(c, batch * nf * d * sizeof(float)));
        SS_TRY(e->col2.alloc(c, batch * nc * d * 3 * sizeof(float)));
        e->stem_batch = batch;
    }
    const VkEpi gelu = {nullptr, 1};
    // conv1: [n_mels, n_frames] per clip, kernel 3, stride 1, pad 1
    SS_HIP(vk::launch_im2col(s, true, d_mel, nm * nf, nf, 1, (int)batch, (int)nm, (int)nf, 3, 1, 1, (int)nf,
                             e->col1.f()),
           "launch(vk_im2col conv1)");
    SS_HIP(vk::launch_gemm_f32(s, true, e->col1.f(), e->c1w.f(), e->c1b.f(), e->c1.f(), (int)(batch * nf), (int)d,
                               (int)(nm * 3), gelu),
           "launch(vk_gemm_f32 conv1)");
    // conv2: the time-major conv1 output read as [d, n_frames], kernel 3, stride 2, pad 1
    SS_HIP(vk::launch_im2col(s, true, e->c1.f(), nf * d, 1, d, (int)batch, (int)d, (int)nf, 3, 2, 1, (int)nc,
                             e->col2.f()),
           "launch(vk_im2col conv2)");
    SS_HIP(vk::launch_gemm_f32(s, true, e->col2.f(), e->c2w.f(), e->c2b.f(), d_x, (int)(batch * nc), (int)d,
                               (int)(d * 3), gelu),
           "launch(vk_gemm_f32 conv2)");
    SS_HIP(vk::launch_add_pos(s, d_x, e->pos.f(), batch * nc, (int)d, (int)nc), "launch(vk_add_pos)");
    return VOKRA_HIP_OK;
}

// The whole of WhisperEncoder::encode: the stem, then the blocks (enc_forward).
int enc_encode(vokra_hip_encoder* e, size_t batch, const float* d_mel, float* d_out) {
    SS_TRY(enc_stem(e, batch, d_mel, e->x.f()));
    return enc_forward(e, batch, e->n_ctx, e->x.f(), d_out);  // copies x into h before reusing x
}

int dec_setup(vokra_hip_decoder* m, const vokra_hip_decoder_layer_t* layers, const float* tok_emb,
              const float* pos_emb, const float* lpg, const float* lpb, size_t block_size) {
    vokra_hip_ctx_t* c = m->ctx;
    const size_t d = m->d, ff = m->d_ff;
    m->layers.resize(m->n_layer);
    for (size_t l = 0; l < m->n_layer; ++l) {
        const vokra_hip_decoder_layer_t& s = layers[l];
        DecLayer& L = m->layers[l];
        SS_TRY(upload_vec(c, L.ln1g, s.ln1_gamma, d, "decoder: ln1_gamma is NULL"));
        SS_TRY(upload_vec(c, L.ln1b, s.ln1_beta, d, "decoder: ln1_beta is NULL"));
        SS_TRY(upload_vec(c, L.ln2g, s.ln2_gamma, d, "decoder: ln2_gamma is NULL"));
        SS_TRY(upload_vec(c, L.ln2b, s.ln2_beta, d, "decoder: ln2_beta is NULL"));
        SS_TRY(upload_vec(c, L.ln3g, s.ln3_gamma, d, "decoder: ln3_gamma is NULL"));
        SS_TRY(upload_vec(c, L.ln3b, s.ln3_beta, d, "decoder: ln3_beta is NULL"));
        SS_TRY(L.q.make(c, m->wdtype, d, d, s.wq, s.bq));
        SS_TRY(L.k.make(c, m->wdtype, d, d, s.wk, s.bk));
        SS_TRY(L.v.make(c, m->wdtype, d, d, s.wv, s.bv));
        SS_TRY(L.o.make(c, m->wdtype, d, d, s.wo, s.bo));
        SS_TRY(L.cq.make(c, m->wdtype, d, d, s.cwq, s.cbq));
        SS_TRY(L.ck.make(c, m->wdtype, d, d, s.cwk, s.cbk));
        SS_TRY(L.cv.make(c, m->wdtype, d, d, s.cwv, s.cbv));
        SS_TRY(L.co.make(c, m->wdtype, d, d, s.cwo, s.cbo));
        SS_TRY(L.fc1.make(c, m->wdtype, ff, d, s.w1, s.b1));
        SS_TRY(L.fc2.make(c, m->wdtype, d, ff, s.w2, s.b2));
    }
    SS_TRY(upload_vec(c, m->tok_emb, tok_emb, m->vocab * d, "decoder: token_emb is NULL"));
    SS_TRY(upload_vec(c, m->pos_emb, pos_emb, m->n_text * d, "decoder: pos_emb is NULL"));
    SS_TRY(upload_vec(c, m->lnpg, lpg, d, "decoder: ln_post_gamma is NULL"));
    SS_TRY(upload_vec(c, m->lnpb, lpb, d, "decoder: ln_post_beta is NULL"));
    SS_TRY(vokra_hip_kv_create(c, m->n_layer, m->n_head, m->hd, m->n_stream, m->n_text, block_size, VOKRA_HIP_KV_Q8_0,
                               &m->kv));
    const size_t sl = m->n_stream * m->n_layer;
    SS_TRY(m->ckh.alloc(c, sl * m->n_audio * d * 2));
    SS_TRY(m->ckl.alloc(c, sl * m->n_audio * d));
    SS_TRY(m->cvh.alloc(c, sl * d * m->t_pad * 2));
    SS_TRY(m->cvl.alloc(c, sl * d * m->t_pad));
    // zero cross K/V: a stream stepped through the _dev path before its
    // encoder output is set attends over zeros, never over stale memory
    for (DBuf* b : {&m->ckh, &m->ckl})
        SS_HIP(hipMemsetAsync(b->p, 0, sl * m->n_audio * d * (b == &m->ckh ? 2 : 1), vk::ctx_stream(c)),
               "hipMemsetAsync(cross k)");
    for (DBuf* b : {&m->cvh, &m->cvl})
        SS_HIP(hipMemsetAsync(b->p, 0, sl * d * m->t_pad * (b == &m->cvh ? 2 : 1), vk::ctx_stream(c)),
               "hipMemsetAsync(cross v)");
    m->enc_set.assign(m->n_stream, 0);
    m->length.assign(m->n_stream, 0);
    const size_t rows = m->n_stream, rd = rows * d * sizeof(float);
    for (DBuf* b : {&m->h, &m->x, &m->q, &m->k, &m->v, &m->attn}) SS_TRY(b->alloc(c, rd));
    SS_TRY(m->f.alloc(c, rows * ff * sizeof(float)));
    SS_TRY(m->logits.alloc(c, rows * m->vocab * sizeof(float)));
    // (max, index) pairs of the fused logits pass or of the sliced argmax
    SS_TRY(m->lpart.alloc(c, rows * (size_t)std::max(vk::logits_n_vt((int)m->vocab), vk::argmax_n_slices((int)m->vocab)) *
                                 sizeof(float2)));
    SS_TRY(m->lens.alloc(c, rows * sizeof(int)));
    SS_TRY(m->kvidx.alloc(c, m->n_layer * rows * sizeof(int)));
    SS_TRY(m->next.alloc(c, rows * sizeof(int)));
    SS_TRY(m->tk.alloc(c, m->n_audio * d * sizeof(float)));
    SS_TRY(m->tv.alloc(c, m->n_audio * d * sizeof(float)));
    SS_TRY(m->stage.alloc(c, std::max(m->n_audio * d * sizeof(float), 3 * rows * sizeof(int))));
    SS_TRY(vokra_hip_qact_create(c, std::max(rows, m->n_audio), d, &m->qa_d));
    SS_TRY(vokra_hip_qact_create(c, rows, ff, &m->qa_f));
    return VOKRA_HIP_OK;
}

int dec_set_encoder(vokra_hip_decoder* m, size_t stream, const float* d_enc) {
    vokra_hip_ctx_t* c = m->ctx;
    hipStream_t s = vk::ctx_stream(c);
    const size_t d = m->d, na = m->n_audio;
    SS_TRY(vokra_hip_qact_quantize_dev(c, m->qa_d, na, d_enc, act_of(m->wdtype)));
    for (size_t l = 0; l < m->n_layer; ++l) {
        const DecLayer& L = m->layers[l];
        SS_TRY(L.ck.run(c, m->qa_d, m->tk.f()));
        SS_TRY(L.cv.run(c, m->qa_d, m->tv.f()));
        const size_t sl = stream * m->n_layer + l;
        uint16_t* kh = (uint16_t*)m->ckh.p + sl * na * d;
        int8_t* kl = (int8_t*)m->ckl.p + sl * na * d;
        uint16_t* vh = (uint16_t*)m->cvh.p + sl * d * m->t_pad;
        int8_t* vl = (int8_t*)m->cvl.p + sl * d * m->t_pad;
        // head-major K and tiled V^T: each 64-frame tile of a head is one
        // contiguous block for the single-query cross-attention stream
        SS_HIP(vk::launch_split_rows_q7_heads(s, m->tk.f(), 1, (int)na, (int)m->n_head, (int)m->hd, 1.0f, kh, kl),
               "launch(vk_split_rows_q7_heads cross k)");
        SS_HIP(vk::launch_split_vt_q7(s, m->tv.f(), 1, (int)na, (int)m->t_pad, (int)m->n_head, (int)m->hd, vh, vl,
                                      true),
               "launch(vk_split_vt_q7 cross v)");
    }
    return VOKRA_HIP_OK;
}

int dec_step(vokra_hip_decoder* m, size_t n, const int* d_streams, const int* d_tokens, const int* d_positions,
             int* d_next, float* d_logits) {
    vokra_hip_ctx_t* c = m->ctx;
    hipStream_t s = vk::ctx_stream(c);
    const size_t d = m->d;
    const int act = act_of(m->wdtype);
    const float scale = powf((float)m->hd, -0.5f);
    SS_HIP(vk::launch_embed_f32(s, m->tok_emb.f(), m->pos_emb.f(), d_tokens, d_positions, (int)m->vocab,
                                (int)m->n_text, (int)d, (int)n, m->h.f()),
           "launch(vk_embed_f32)");
    hipLaunchKernelGGL(vk::vk_step_index, dim3((unsigned)((n + 63) / 64)), dim3(64), 0, s, d_streams, d_positions, (int)n,
                       (int)m->n_layer, m->lens.i(), m->kvidx.i());
    SS_HIP(hipGetLastError(), "launch(vk_step_index)");
    // the self-attention cache pages of this step, every layer in layer order
    // (the same pages as one append per layer); each layer's attention kernel
    // then packs its new K / V rows into them
    for (size_t l0 = 0, per = std::max<size_t>(1, 4096 / n); l0 < m->n_layer; l0 += per)
        SS_TRY(vk::kv_alloc_layers(c, m->kv, 0, l0, std::min(per, m->n_layer - l0), n, d_streams, d_positions));
    // The same fusions as the encoder (LN + quantize, out-proj + residual,
    // fc1 + GELU, q/k/v in one launch); results equal the entry-point sequence.
    const VkEpi add_h = {m->h.f(), 0}, gelu = {nullptr, 1};
    for (size_t l = 0; l < m->n_layer; ++l) {
        const DecLayer& L = m->layers[l];
        // causal self-attention over the paged cache (decoder.rs:462-490)
        SS_TRY(vk::qact_ln_quantize(c, m->qa_d, n, m->h.f(), L.ln1g.f(), L.ln1b.f(), kLnEps, act, m->x.f()));
        const vokra_hip_qweight_t* qkv[3] = {L.q.w, L.k.w, L.v.w};
        const float* qkv_b[3] = {L.q.b(), L.k.b(), L.v.b()};
        float* qkv_o[3] = {m->q.f(), m->k.f(), m->v.f()};
        SS_TRY(vk::gemm_qact_multi(c, 3, qkv, m->qa_d, qkv_b, qkv_o));
        SS_TRY(vk::paged_attn_append_quantize(c, m->kv, l, n, d_streams, d_positions, m->k.f(), m->v.f(), m->lens.i(),
                                              m->n_text, m->n_head, m->q.f(), scale, m->attn.f(), m->qa_d, act));
        SS_TRY(L.o.run(c, m->qa_d, m->h.f(), add_h));
        // cross-attention over the stream's encoder frames (decoder.rs:492-510)
        SS_TRY(vk::qact_ln_quantize(c, m->qa_d, n, m->h.f(), L.ln2g.f(), L.ln2b.f(), kLnEps, act, m->x.f()));
        SS_TRY(L.cq.run(c, m->qa_d, m->q.f()));
        // (q * scale split into fp16 hi / lo inside the kernel, which also
        // runs the activation pass over its output rows when that has a
        // fused form)
        VkQOut qo;
        SS_TRY(vk::qact_output(c, m->qa_d, n, act, &qo));
        const vk::AttnLayout lay = vk::attn_layout_heads((int)m->n_audio, (int)m->n_head, (int)m->hd, (int)m->t_pad);
        SS_HIP(vk::launch_flash_attn_f32q(s, (int)m->hd, m->q.f(), scale, m->ckh.p, m->ckl.p, m->cvh.p, m->cvl.p,
                                          qo.afrag ? nullptr : m->attn.f(), (int)n, 1, (int)m->n_audio,
                                          (int)m->t_pad, (int)m->n_head, (int)m->n_head, 0, 0, m->kvidx.i() + l * n,
                                          m->cross_precision == VOKRA_HIP_CROSS_F32 ? vk::KV_LO_Q7 : vk::KV_LO_NONE,
                                          qo.afrag ? &qo : nullptr, &lay),
               "launch(vk_flash_attn cross)");
        if (qo.afrag) vk::qact_outputs_written(m->qa_d, n, act);
        else SS_TRY(vokra_hip_qact_quantize_dev(c, m->qa_d, n, m->attn.f(), act));
        SS_TRY(L.co.run(c, m->qa_d, m->h.f(), add_h));
        // MLP (decoder.rs:512-525)
        SS_TRY(vk::qact_ln_quantize(c, m->qa_d, n, m->h.f(), L.ln3g.f(), L.ln3b.f(), kLnEps, act, m->x.f()));
        SS_TRY(L.fc1.run_quantize(c, m->qa_d, m->f.f(), gelu, m->qa_f, act));
        SS_TRY(L.fc2.run(c, m->qa_f, m->h.f(), add_h));
    }
    // ln_post, then tied logits (decoder.rs:754-796) and greedy argmax in one
    // pass over the embedding; the logits are written only when asked for
    SS_TRY(vokra_hip_layer_norm_f32_dev(c, m->h.f(), m->x.f(), n, d, m->lnpg.f(), m->lnpb.f(), kLnEps));
    if (d % vk::logits_d_multiple() == 0) {
        SS_HIP(vk::launch_logits_argmax(s, m->x.f(), m->tok_emb.f(), d_logits, (float2*)m->lpart.p, d_next, (int)n,
                                        (int)m->vocab, (int)d),
               "launch(vk_logits_argmax)");
        return VOKRA_HIP_OK;
    }
    float* lg = d_logits ? d_logits : m->logits.f();
    SS_TRY(vokra_hip_gemm_f32_dev(c, n, m->vocab, d, m->x.f(), m->tok_emb.f(), 1, nullptr, lg));
    SS_HIP(vk::launch_argmax_sliced(s, lg, (int)n, (int)m->vocab, (float2*)m->lpart.p, d_next),
           "launch(vk_argmax_slices)");
    return VOKRA_HIP_OK;
}

}  // namespace

extern "C" {

int vokra_hip_encoder_create(vokra_hip_ctx_t* c, int wdtype, size_t n_layer, size_t d_model, size_t n_head,
                             size_t d_ff, const vokra_hip_prenorm_layer_t* layers, const float* ln_post_gamma,
                             const float* ln_post_beta, size_t max_rows, vokra_hip_encoder_t** out) {
    if (!c || !out || (n_layer && !layers))
        return vk::ctx_fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "encoder_create: NULL argument");
    *out = nullptr;
    SS_TRY(check_model_dims(wdtype, d_model, n_head, d_ff));
    if (!max_rows) return vk::ctx_fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "encoder_create: max_rows must be > 0");
    auto* e = new vokra_hip_encoder();
    e->ctx = c;
    e->wdtype = wdtype;
    e->n_layer = n_layer;
    e->d = d_model;
    e->n_head = n_head;
    e->hd = d_model / n_head;
    e->d_ff = d_ff;
    e->max_rows = max_rows;
    int st = enc_setup(e, layers, ln_post_gamma, ln_post_beta);
    if (st) {
        e->release();
        delete e;
        return st;
    }
    *out = e;
    return VOKRA_HIP_OK;
}

void vokra_hip_encoder_destroy(vokra_hip_encoder_t* e) {
    if (!e) return;
    e->release();
    delete e;
}

int vokra_hip_encoder_forward_dev(vokra_hip_ctx_t* c, vokra_hip_encoder_t* e, size_t batch, size_t frames,
                                  const float* d_x, float* d_out) {
    if (!c || !e || e->ctx != c) return vk::ctx_fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "encoder_forward: bad context");
    if (batch * frames == 0) return VOKRA_HIP_OK;
    if (batch * frames > e->max_rows)
        return vk::ctx_fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "encoder_forward: batch * frames exceeds max_rows");
    if (!d_x || !d_out) return vk::ctx_fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "encoder_forward: NULL buffer");
    return enc_forward(e, batch, frames, d_x, d_out);
}

int vokra_hip_encoder_set_stem(vokra_hip_ctx_t* c, vokra_hip_encoder_t* e, size_t n_mels, size_t n_frames,
                               const float* conv1_w, const float* conv1_b, const float* conv2_w, const float* conv2_b,
                               const float* pos_emb) {
    if (!c || !e || e->ctx != c) return vk::ctx_fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "encoder_set_stem: bad context");
    if (!conv1_w || !conv1_b || !conv2_w || !conv2_b || !pos_emb)
        return vk::ctx_fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "encoder_set_stem: NULL weight");
    if (n_mels == 0 || n_mels > 1024 || n_frames < 2 || n_frames > 65536)
        return vk::ctx_fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "encoder_set_stem: n_mels 1..1024, n_frames 2..65536");
    const size_t d = e->d, n_ctx = (n_frames + 2 - 3) / 2 + 1;  // conv_out_len(n_frames, 3, 2, 1)
    for (DBuf* b : {&e->c1w, &e->c1b, &e->c2w, &e->c2b, &e->pos}) b->release(c);
    SS_TRY(upload_vec(c, e->c1w, conv1_w, d * n_mels * 3, "encoder_set_stem: conv1_w"));
    SS_TRY(upload_vec(c, e->c1b, conv1_b, d, "encoder_set_stem: conv1_b"));
    SS_TRY(upload_vec(c, e->c2w, conv2_w, d * d * 3, "encoder_set_stem: conv2_w"));
    SS_TRY(upload_vec(c, e->c2b, conv2_b, d, "encoder_set_stem: conv2_b"));
    SS_TRY(upload_vec(c, e->pos, pos_emb, n_ctx * d, "encoder_set_stem: pos_emb"));
    e->n_mels = n_mels;
    e->n_frames = n_frames;
    e->n_ctx = n_ctx;
    return VOKRA_HIP_OK;
}

int vokra_hip_encoder_encode_dev(vokra_hip_ctx_t* c, vokra_hip_encoder_t* e, size_t batch, const float* d_log_mel,
                                 float* d_out) {
    if (!c || !e || e->ctx != c) return vk::ctx_fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "encoder_encode: bad context");
    if (!e->n_ctx) return vk::ctx_fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "encoder_encode: no conv stem (set_stem)");
    if (batch == 0) return VOKRA_HIP_OK;
    if (batch * e->n_ctx > e->max_rows)
        return vk::ctx_fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "encoder_encode: batch * n_ctx exceeds max_rows");
    if (!d_log_mel || !d_out) return vk::ctx_fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "encoder_encode: NULL buffer");
    return enc_encode(e, batch, d_log_mel, d_out);
}

int vokra_hip_encoder_stem_dev(vokra_hip_ctx_t* c, vokra_hip_encoder_t* e, size_t batch, const float* d_log_mel,
                               float* d_x) {
    if (!c || !e || e->ctx != c) return vk::ctx_fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "encoder_stem: bad context");
    if (!e->n_ctx) return vk::ctx_fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "encoder_stem: no conv stem (set_stem)");
    if (batch == 0) return VOKRA_HIP_OK;
    if (batch * e->n_ctx > e->max_rows)
        return vk::ctx_fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "encoder_stem: batch * n_ctx exceeds max_rows");
    if (!d_log_mel || !d_x) return vk::ctx_fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "encoder_stem: NULL buffer");
    return enc_stem(e, batch, d_log_mel, d_x);
}

int vokra_hip_encoder_encode(vokra_hip_ctx_t* c, vokra_hip_encoder_t* e, size_t batch, const float* log_mel,
                             float* out) {
    if (!c || !e || e->ctx != c) return vk::ctx_fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "encoder_encode: bad context");
    if (!e->n_ctx) return vk::ctx_fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "encoder_encode: no conv stem (set_stem)");
    if (batch == 0) return VOKRA_HIP_OK;
    if (!log_mel || !out) return vk::ctx_fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "encoder_encode: NULL buffer");
    const size_t n_in = batch * e->n_mels * e->n_frames, n_out = batch * e->n_ctx * e->d;
    DBuf in, o;
    int st = in.upload(c, log_mel, n_in * sizeof(float));
    if (!st) st = o.alloc(c, n_out * sizeof(float));
    if (!st) st = vokra_hip_encoder_encode_dev(c, e, batch, in.f(), o.f());
    if (!st) st = vokra_hip_memcpy_dtoh(c, out, o.p, n_out * sizeof(float));
    in.release(c);
    o.release(c);
    return st ? st : vk::range_check(c);
}

int vokra_hip_encoder_forward(vokra_hip_ctx_t* c, vokra_hip_encoder_t* e, size_t batch, size_t frames, const float* x,
                              float* out) {
    if (!c || !e || e->ctx != c) return vk::ctx_fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "encoder_forward: bad context");
    const size_t n = batch * frames * e->d;
    if (n == 0) return VOKRA_HIP_OK;
    if (batch * frames > e->max_rows)
        return vk::ctx_fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "encoder_forward: batch * frames exceeds max_rows");
    if (!x || !out) return vk::ctx_fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "encoder_forward: NULL buffer");
    DBuf in, o;
    int st = in.upload(c, x, n * sizeof(float));
    if (!st) st = o.alloc(c, n * sizeof(float));
    if (!st) st = enc_forward(e, batch, frames, in.f(), o.f());
    if (!st) st = vokra_hip_memcpy_dtoh(c, out, o.p, n * sizeof(float));
    in.release(c);
    o.release(c);
    return st ? st : vk::range_check(c);
}

int vokra_hip_decoder_create(vokra_hip_ctx_t* c, int wdtype, size_t n_layer, size_t d_model, size_t n_head,
                             size_t d_ff, size_t n_vocab, size_t n_text_ctx, size_t n_audio_ctx, size_t n_stream,
                             size_t block_size, const vokra_hip_decoder_layer_t* layers, const float* token_emb,
                             const float* pos_emb, const float* ln_post_gamma, const float* ln_post_beta,
                             vokra_hip_decoder_t** out) {
    if (!c || !out || !layers) return vk::ctx_fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "decoder_create: NULL argument");
    *out = nullptr;
    SS_TRY(check_model_dims(wdtype, d_model, n_head, d_ff));
    if (!n_layer || !n_vocab || !n_text_ctx || !n_audio_ctx || !n_stream || n_stream > 1024 || n_vocab > 0x7fffffff)
        return vk::ctx_fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT,
                            "decoder_create: n_layer, n_vocab, n_text_ctx, n_audio_ctx > 0 and n_stream in 1..1024");
    auto* m = new vokra_hip_decoder();
    m->ctx = c;
    m->wdtype = wdtype;
    m->n_layer = n_layer;
    m->d = d_model;
    m->n_head = n_head;
    m->hd = d_model / n_head;
    m->d_ff = d_ff;
    m->vocab = n_vocab;
    m->n_text = n_text_ctx;
    m->n_audio = n_audio_ctx;
    m->n_stream = n_stream;
    m->t_pad = (n_audio_ctx + 63) / 64 * 64;
    int st = dec_setup(m, layers, token_emb, pos_emb, ln_post_gamma, ln_post_beta, block_size);
    if (st) {
        m->release();
        delete m;
        return st;
    }
    *out = m;
    return VOKRA_HIP_OK;
}

void vokra_hip_decoder_destroy(vokra_hip_decoder_t* m) {
    if (!m) return;
    m->release();
    delete m;
}

int vokra_hip_decoder_set_encoder_dev(vokra_hip_ctx_t* c, vokra_hip_decoder_t* m, size_t stream, const float* d_enc) {
    if (!c || !m || m->ctx != c || !d_enc)
        return vk::ctx_fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "decoder_set_encoder: bad argument");
    if (stream >= m->n_stream)
        return vk::ctx_fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "decoder_set_encoder: stream out of range");
    SS_TRY(dec_set_encoder(m, stream, d_enc));
    m->enc_set[stream] = 1;
    return VOKRA_HIP_OK;
}

int vokra_hip_decoder_set_encoder(vokra_hip_ctx_t* c, vokra_hip_decoder_t* m, size_t stream, const float* enc) {
    if (!c || !m || m->ctx != c || !enc)
        return vk::ctx_fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "decoder_set_encoder: bad argument");
    if (stream >= m->n_stream)
        return vk::ctx_fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "decoder_set_encoder: stream out of range");
    SS_TRY(vokra_hip_memcpy_htod(c, m->stage.p, enc, m->n_audio * m->d * sizeof(float)));
    SS_TRY(dec_set_encoder(m, stream, m->stage.f()));
    SS_TRY(vokra_hip_synchronize(c));
    m->enc_set[stream] = 1;
    return VOKRA_HIP_OK;
}

int vokra_hip_decoder_set_cross_precision(vokra_hip_ctx_t* c, vokra_hip_decoder_t* m, int precision) {
    if (!c || !m || m->ctx != c)
        return vk::ctx_fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "decoder_set_cross_precision: bad argument");
    if (precision != VOKRA_HIP_CROSS_F32 && precision != VOKRA_HIP_CROSS_F16)
        return vk::ctx_fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "decoder_set_cross_precision: unknown precision");
    m->cross_precision = precision;  // both fp16 parts are always stored: switching needs no re-upload
    return VOKRA_HIP_OK;
}

int vokra_hip_decoder_reset(vokra_hip_ctx_t* c, vokra_hip_decoder_t* m) {
    if (!c || !m || m->ctx != c) return vk::ctx_fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "decoder_reset: bad argument");
    SS_TRY(vokra_hip_kv_reset(c, m->kv));
    std::fill(m->length.begin(), m->length.end(), 0);
    return VOKRA_HIP_OK;
}

int vokra_hip_decoder_set_free_order(vokra_hip_ctx_t* c, vokra_hip_decoder_t* m, const int32_t* order, size_t n) {
    if (!c || !m || m->ctx != c) return vk::ctx_fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "decoder_set_free_order: bad argument");
    SS_TRY(vokra_hip_kv_set_free_order(c, m->kv, order, n));
    std::fill(m->length.begin(), m->length.end(), 0);
    return VOKRA_HIP_OK;
}

int vokra_hip_decoder_kv_pages(vokra_hip_ctx_t* c, vokra_hip_decoder_t* m, size_t* free_pages, size_t* pages_in_use) {
    if (!c || !m || m->ctx != c) return vk::ctx_fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "decoder_kv_pages: bad argument");
    return vokra_hip_kv_pages(c, m->kv, free_pages, pages_in_use);
}

int vokra_hip_decoder_status(vokra_hip_ctx_t* c, vokra_hip_decoder_t* m, size_t* n_appended) {
    if (!c || !m || m->ctx != c) return vk::ctx_fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "decoder_status: bad argument");
    size_t a = 0;
    const int st = vokra_hip_kv_status(c, m->kv, &a);
    if (n_appended) *n_appended = a;
    return st ? st : vk::range_check(c);
}

int vokra_hip_decoder_step_dev(vokra_hip_ctx_t* c, vokra_hip_decoder_t* m, size_t n, const int32_t* d_streams,
                               const int32_t* d_tokens, const int32_t* d_positions, int32_t* d_next, float* d_logits) {
    if (!c || !m || m->ctx != c) return vk::ctx_fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "decoder_step: bad context");
    if (n == 0) return VOKRA_HIP_OK;
    if (n > m->n_stream) return vk::ctx_fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "decoder_step: more items than streams");
    if (!d_streams || !d_tokens || !d_positions || !d_next)
        return vk::ctx_fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "decoder_step: NULL buffer");
    return dec_step(m, n, d_streams, d_tokens, d_positions, d_next, d_logits);
}

int vokra_hip_decoder_step(vokra_hip_ctx_t* c, vokra_hip_decoder_t* m, size_t n, const int32_t* streams,
                           const int32_t* tokens, const int32_t* positions, int32_t* next_tokens, float* logits) {
    if (!c || !m || m->ctx != c) return vk::ctx_fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "decoder_step: bad context");
    if (n == 0) return VOKRA_HIP_OK;
    if (n > m->n_stream) return vk::ctx_fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "decoder_step: more items than streams");
    if (!streams || !tokens || !positions || !next_tokens)
        return vk::ctx_fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "decoder_step: NULL buffer");
    // WhisperDecoder::step_into's checks (decoder.rs:420-441), per stream
    std::vector<char> seen(m->n_stream, 0);
    for (size_t i = 0; i < n; ++i) {
        if (streams[i] < 0 || (size_t)streams[i] >= m->n_stream || seen[streams[i]])
            return vk::ctx_fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "decoder_step: streams must be distinct and < n_stream");
        seen[streams[i]] = 1;
        if (!m->enc_set[streams[i]])
            return vk::ctx_fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT,
                                "decoder_step: stream %d has no encoder output (call set_encoder first)", streams[i]);
        if (tokens[i] < 0 || (size_t)tokens[i] >= m->vocab)
            return vk::ctx_fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "whisper decoder: token id >= n_vocab");
        if (positions[i] < 0 || (size_t)positions[i] + 1 > m->n_text)
            return vk::ctx_fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "whisper decoder: position exceeds n_text_ctx");
        // the step position is the stream's current length (decoder.rs:427-434
        // takes start = self_kv.positions()); 0 restarts the stream
        if (positions[i] != 0 && positions[i] != m->length[streams[i]])
            return vk::ctx_fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT,
                                "decoder_step: stream %d is at position %d, got %d (0 restarts it)", streams[i],
                                m->length[streams[i]], positions[i]);
    }
    std::vector<int32_t> items(3 * n);
    memcpy(items.data(), streams, n * 4);
    memcpy(items.data() + n, tokens, n * 4);
    memcpy(items.data() + 2 * n, positions, n * 4);
    int* dv = m->stage.i();
    SS_TRY(vokra_hip_memcpy_htod(c, dv, items.data(), 3 * n * 4));
    SS_TRY(dec_step(m, n, dv, dv + n, dv + 2 * n, m->next.i(), logits ? m->logits.f() : nullptr));
    size_t appended = 0;
    SS_TRY(vokra_hip_kv_status(c, m->kv, &appended));
    for (size_t i = 0; i < n; ++i) m->length[streams[i]] = positions[i] + 1;  // the rows are appended
    SS_TRY(vokra_hip_memcpy_dtoh(c, next_tokens, m->next.p, n * 4));
    if (logits) SS_TRY(vokra_hip_memcpy_dtoh(c, logits, m->logits.p, n * m->vocab * sizeof(float)));
    return vk::range_check(c);
}

}  // extern "C"

// ---------------------------------------------------------------------------
// Speech-LLM text decoder (crates/vokra-models/src/voxtral/text_decoder.rs:
// 1147-1420 per stream, as driven by TextDecoderSession::step_into,
// text_decoder_session.rs:207-240), batched over streams: RMSNorm, q / k / v,
// RoPE at each stream's position, the paged Q8_0 cache, grouped-query decode
// attention, o-proj + residual, RMSNorm, SwiGLU FFN + residual, final
// RMSNorm, LM head and greedy argmax, all device-resident.

namespace vk {

// lens[i] = positions[i] + 1: the keys 0..t a step attends after its append.
__global__ void vk_lens_of(const int* __restrict__ positions, int n, int* __restrict__ lens) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) lens[i] = positions[i] + 1;
}

}  // namespace vk

namespace {

struct TextLayer {
    DBuf attn_g, ffn_g;
    QLin q, k, v, o, gate, up, down;
};

}  // namespace

struct vokra_hip_text_decoder {
    vokra_hip_ctx_t* ctx = nullptr;
    int wdtype = 0;
    size_t n_layer = 0, d = 0, hq = 0, hkv = 0, hd = 0, ff = 0, vocab = 0, n_ctx = 0, n_stream = 0;
    float rope_base = 0.0f, eps = 0.0f, scale = 0.0f;
    std::vector<TextLayer> layers;
    DBuf tok_emb, final_g, theta, h, x, q, k, v, attn, g, u, logits, lpart, lens, next, stage, rope_cs;
    QLin lm_head;
    bool tied = true;
    vokra_hip_kv_t* kv = nullptr;
    vokra_hip_qact_t *qa_d = nullptr, *qa_q = nullptr, *qa_f = nullptr;
    std::vector<int32_t> position;  // host clock per stream (TextDecoderSession::position)
    void release() {
        for (auto& L : layers) {
            for (DBuf* b : {&L.attn_g, &L.ffn_g}) b->release(ctx);
            for (QLin* w : {&L.q, &L.k, &L.v, &L.o, &L.gate, &L.up, &L.down}) w->release(ctx);
        }
        for (DBuf* b : {&tok_emb, &final_g, &theta, &h, &x, &q, &k, &v, &attn, &g, &u, &logits, &lpart, &lens, &next,
                        &stage, &rope_cs})
            b->release(ctx);
        lm_head.release(ctx);
        vokra_hip_kv_destroy(kv);
        kv = nullptr;
        for (vokra_hip_qact_t** qa : {&qa_d, &qa_q, &qa_f}) {
            vokra_hip_qact_free(*qa);
            *qa = nullptr;
        }
    }
};

namespace {

int td_setup(vokra_hip_text_decoder* m, const vokra_hip_text_decoder_layer_t* layers, const float* tok_emb,
             const float* final_g, const uint8_t* lm_head, size_t block_size) {
    vokra_hip_ctx_t* c = m->ctx;
    const size_t d = m->d, qh = m->hq * m->hd, kvh = m->hkv * m->hd, ff = m->ff;
    m->layers.resize(m->n_layer);
    for (size_t l = 0; l < m->n_layer; ++l) {
        const vokra_hip_text_decoder_layer_t& s = layers[l];
        TextLayer& L = m->layers[l];
        SS_TRY(upload_vec(c, L.attn_g, s.attn_norm_gamma, d, "text_decoder: attn_norm_gamma is NULL"));
        SS_TRY(upload_vec(c, L.ffn_g, s.ffn_norm_gamma, d, "text_decoder: ffn_norm_gamma is NULL"));
        SS_TRY(L.q.make(c, m->wdtype, qh, d, s.wq, nullptr));
        SS_TRY(L.k.make(c, m->wdtype, kvh, d, s.wk, nullptr));
        SS_TRY(L.v.make(c, m->wdtype, kvh, d, s.wv, nullptr));
        SS_TRY(L.o.make(c, m->wdtype, d, qh, s.wo, nullptr));
        SS_TRY(L.gate.make(c, m->wdtype, ff, d, s.w_gate, nullptr));
        SS_TRY(L.up.make(c, m->wdtype, ff, d, s.w_up, nullptr));
        SS_TRY(L.down.make(c, m->wdtype, d, ff, s.w_down, nullptr));
    }
    SS_TRY(upload_vec(c, m->tok_emb, tok_emb, m->vocab * d, "text_decoder: token_emb is NULL"));
    SS_TRY(upload_vec(c, m->final_g, final_g, d, "text_decoder: final_norm_gamma is NULL"));
    m->tied = lm_head == nullptr;
    if (!m->tied) SS_TRY(m->lm_head.make(c, m->wdtype, m->vocab, d, lm_head, nullptr));
    // the rotary frequencies, evaluated as the reference does per element:
    // rope_base.powf(-2.0 * (j as f32) / (head_dim as f32))
    std::vector<float> th(m->hd / 2);
    for (size_t j = 0; j < th.size(); ++j) th[j] = powf(m->rope_base, -2.0f * (float)j / (float)m->hd);
    SS_TRY(m->theta.upload(c, th.data(), th.size() * sizeof(float)));
    SS_TRY(vokra_hip_kv_create(c, m->n_layer, m->hkv, m->hd, m->n_stream, m->n_ctx, block_size, VOKRA_HIP_KV_Q8_0,
                               &m->kv));
    const size_t rows = m->n_stream;
    SS_TRY(m->h.alloc(c, rows * d * sizeof(float)));
    SS_TRY(m->x.alloc(c, rows * d * sizeof(float)));
    SS_TRY(m->q.alloc(c, rows * qh * sizeof(float)));
    SS_TRY(m->attn.alloc(c, rows * qh * sizeof(float)));
    SS_TRY(m->k.alloc(c, rows * kvh * sizeof(float)));
    SS_TRY(m->v.alloc(c, rows * kvh * sizeof(float)));
    SS_TRY(m->g.alloc(c, rows * ff * sizeof(float)));
    SS_TRY(m->u.alloc(c, rows * ff * sizeof(float)));
    SS_TRY(m->logits.alloc(c, rows * m->vocab * sizeof(float)));
    // (max, index) pairs of the fused logits pass or of the sliced argmax
    SS_TRY(m->lpart.alloc(c, rows * (size_t)std::max(vk::logits_n_vt((int)m->vocab), vk::argmax_n_slices((int)m->vocab)) *
                                 sizeof(float2)));
    SS_TRY(m->lens.alloc(c, rows * sizeof(int)));
    SS_TRY(m->next.alloc(c, rows * sizeof(int)));
    SS_TRY(m->stage.alloc(c, 3 * rows * sizeof(int)));
    SS_TRY(m->rope_cs.alloc(c, rows * (m->hd / 2) * sizeof(float2)));  // (cos, sin) of one step's positions
    SS_TRY(vokra_hip_qact_create(c, rows, d, &m->qa_d));
    SS_TRY(vokra_hip_qact_create(c, rows, qh, &m->qa_q));
    SS_TRY(vokra_hip_qact_create(c, rows, ff, &m->qa_f));
    m->position.assign(m->n_stream, 0);
    return VOKRA_HIP_OK;
}

// RMSNorm of rows n of in into scratch, then the activation pass into qa.
// (one fused launch for the K-quant convention)
int td_rms_quantize(vokra_hip_text_decoder* m, vokra_hip_qact_t* qa, size_t n, const float* in, const float* gamma) {
    if (act_of(m->wdtype) == VOKRA_HIP_ACT_KQUANT)
        return vk::qact_rms_quantize_g16(m->ctx, qa, n, m->d, in, gamma, m->eps);
    hipStream_t s = vk::ctx_stream(m->ctx);
    SS_HIP(vk::launch_rms_norm_f32(s, in, m->x.f(), (int)n, (int)m->d, gamma, m->eps), "launch(vk_rms_norm_f32)");
    return vokra_hip_qact_quantize_dev(m->ctx, qa, n, m->x.f(), act_of(m->wdtype));
}

int td_step(vokra_hip_text_decoder* m, size_t n, const int* d_streams, const int* d_tokens, const int* d_positions,
            int* d_next, float* d_logits) {
    vokra_hip_ctx_t* c = m->ctx;
    hipStream_t s = vk::ctx_stream(c);
    const int act = act_of(m->wdtype);
    const size_t d = m->d, ff = m->ff;
    SS_HIP(vk::launch_embed_f32(s, m->tok_emb.f(), nullptr, d_tokens, nullptr, (int)m->vocab, 1, (int)d, (int)n,
                                m->h.f()),
           "launch(vk_embed_f32)");
    hipLaunchKernelGGL(vk::vk_lens_of, dim3((unsigned)((n + 63) / 64)), dim3(64), 0, s, d_positions, (int)n,
                       m->lens.i());
    SS_HIP(hipGetLastError(), "launch(vk_lens_of)");
    // this step's cache pages for every layer, in layer order
    for (size_t l0 = 0, per = std::max<size_t>(1, 4096 / n); l0 < m->n_layer; l0 += per)
        SS_TRY(vk::kv_alloc_layers(c, m->kv, 0, l0, std::min(per, m->n_layer - l0), n, d_streams, d_positions));
    const VkEpi add_h = {m->h.f(), 0};
    // RoPE fused into the GQA kernel's K/V cache write (k) and q load: one
    // (cos, sin) table for the step's positions serves every layer
    const bool rope_fused =
        act == VOKRA_HIP_ACT_KQUANT && vk::paged_attn_rotates_q(m->kv, n, m->hq, m->q.f(), m->attn.f());
    const float2* cs = rope_fused ? (const float2*)m->rope_cs.p : nullptr;
    if (rope_fused)
        SS_HIP(vk::launch_rope_table(s, d_positions, m->theta.f(), (int)n, (int)(m->hd / 2), (float2*)m->rope_cs.p),
               "launch(vk_rope_table)");
    for (size_t l = 0; l < m->n_layer; ++l) {
        const TextLayer& L = m->layers[l];
        // pre-norm self-attention (text_decoder.rs:1212-1351)
        SS_TRY(td_rms_quantize(m, m->qa_d, n, m->h.f(), L.attn_g.f()));
        {  // q, k and v over the same activations: one launch
            const vokra_hip_qweight_t* qkv[3] = {L.q.w, L.k.w, L.v.w};
            const float* qkv_b[3] = {L.q.b(), L.k.b(), L.v.b()};
            float* qkv_o[3] = {m->q.f(), m->k.f(), m->v.f()};
            SS_TRY(vk::gemm_qact_multi(c, 3, qkv, m->qa_d, qkv_b, qkv_o));
        }
        if (!rope_fused)
            SS_HIP(vk::launch_rope_rows_qk(s, m->q.f(), m->k.f(), (int)n, (int)m->hq, (int)m->hkv, (int)m->hd,
                                           m->theta.f(), d_positions),
                   "launch(vk_rope_rows_qk)");
        // with the fused rotation the attention launch also packs this step's
        // K / V rows into the cache
        if (!rope_fused)
            SS_TRY(vk::kv_write_allocated(c, m->kv, l, n, d_streams, d_positions, m->k.f(), m->v.f(), nullptr));
        SS_TRY(vk::paged_attn_quantize(c, m->kv, l, n, d_streams, m->lens.i(), m->n_ctx, m->hq, m->q.f(), m->scale,
                                       m->attn.f(), m->qa_q, act, cs, rope_fused ? m->k.f() : nullptr,
                                       rope_fused ? m->v.f() : nullptr, rope_fused ? d_positions : nullptr));
        SS_TRY(L.o.run(c, m->qa_q, m->h.f(), add_h));
        // pre-norm SwiGLU FFN (text_decoder.rs:1385-1418)
        SS_TRY(td_rms_quantize(m, m->qa_d, n, m->h.f(), L.ffn_g.f()));
        {  // gate and up over the same activations: one launch
            const vokra_hip_qweight_t* gu[2] = {L.gate.w, L.up.w};
            const float* gu_b[2] = {L.gate.b(), L.up.b()};
            float* gu_o[2] = {m->g.f(), m->u.f()};
            SS_TRY(vk::gemm_qact_multi(c, 2, gu, m->qa_d, gu_b, gu_o));
        }
        if (act == VOKRA_HIP_ACT_KQUANT) {
            SS_TRY(vk::qact_swiglu_quantize_g16(c, m->qa_f, n, ff, m->g.f(), m->u.f()));
        } else {
            SS_HIP(vk::launch_swiglu_f32(s, m->g.f(), m->u.f(), m->g.f(), n * ff), "launch(vk_swiglu_f32)");
            SS_TRY(vokra_hip_qact_quantize_dev(c, m->qa_f, n, m->g.f(), act));
        }
        SS_TRY(L.down.run(c, m->qa_f, m->h.f(), add_h));
    }
    // final RMSNorm, LM head, greedy argmax (text_decoder.rs:1423-1451,
    // text_decoder_session.rs argmax)
    SS_HIP(vk::launch_rms_norm_f32(s, m->h.f(), m->x.f(), (int)n, (int)d, m->final_g.f(), m->eps),
           "launch(vk_rms_norm_f32 final)");
    if (!m->tied) {
        SS_TRY(vokra_hip_qact_quantize_dev(c, m->qa_d, n, m->x.f(), act));
        float* lg = d_logits ? d_logits : m->logits.f();
        SS_TRY(m->lm_head.run(c, m->qa_d, lg));
        SS_HIP(vk::launch_argmax_sliced(s, lg, (int)n, (int)m->vocab, (float2*)m->lpart.p, d_next),
               "launch(vk_argmax_slices)");
        return VOKRA_HIP_OK;
    }
    if (d % vk::logits_d_multiple() == 0) {
        SS_HIP(vk::launch_logits_argmax(s, m->x.f(), m->tok_emb.f(), d_logits, (float2*)m->lpart.p, d_next, (int)n,
                                        (int)m->vocab, (int)d),
               "launch(vk_logits_argmax)");
        return VOKRA_HIP_OK;
    }
    float* lg = d_logits ? d_logits : m->logits.f();
    SS_TRY(vokra_hip_gemm_f32_dev(c, n, m->vocab, d, m->x.f(), m->tok_emb.f(), 1, nullptr, lg));
    SS_HIP(vk::launch_argmax_sliced(s, lg, (int)n, (int)m->vocab, (float2*)m->lpart.p, d_next),
           "launch(vk_argmax_slices)");
    return VOKRA_HIP_OK;
}

}  // namespace

extern "C" {

int vokra_hip_text_decoder_create(vokra_hip_ctx_t* c, int wdtype, size_t n_layer, size_t d_model, size_t n_head_q,
                                  size_t n_head_kv, size_t head_dim, size_t ffn_dim, size_t vocab, size_t n_ctx,
                                  size_t n_stream, size_t block_size, float rope_base, float rms_norm_eps,
                                  const vokra_hip_text_decoder_layer_t* layers, const float* token_emb,
                                  const float* final_norm_gamma, const uint8_t* lm_head,
                                  vokra_hip_text_decoder_t** out) {
    if (!c || !out || !layers) return vk::ctx_fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "text_decoder_create: NULL argument");
    *out = nullptr;
    // TextDecoderSession::new's checks (text_decoder_session.rs:90-140)
    if (!n_layer || !d_model || !vocab || !n_head_q || !n_head_kv || !head_dim)
        return vk::ctx_fail(VOKRA_HIP_ERROR_MODEL_LOAD,
                            "voxtral::TextDecoderSession: config carries 0-sentinel (n_layer, d, vocab, heads, head_dim)");
    if (n_head_q % n_head_kv != 0)
        return vk::ctx_fail(VOKRA_HIP_ERROR_MODEL_LOAD,
                            "voxtral::TextDecoderSession: n_head_q (%zu) must be divisible by n_head_kv (%zu) - GQA",
                            n_head_q, n_head_kv);
    const size_t grp = n_head_q / n_head_kv;
    if (head_dim != 64 && head_dim != 128)
        return vk::ctx_fail(VOKRA_HIP_ERROR_UNSUPPORTED_OP, "text_decoder_create: head_dim must be 64 or 128");
    if (grp != 1 && grp != 2 && grp != 4 && grp != 8)
        return vk::ctx_fail(VOKRA_HIP_ERROR_UNSUPPORTED_OP,
                            "text_decoder_create: query heads per kv head must be 1, 2, 4 or 8");
    if (wire_bytes(wdtype, 1, 256) == 0)
        return vk::ctx_fail(VOKRA_HIP_ERROR_UNSUPPORTED_OP, "text_decoder_create: unknown weight dtype");
    const size_t qb = is_kquant(wdtype) ? 256 : 32;
    if (d_model % qb || ffn_dim % qb || !ffn_dim || (n_head_q * head_dim) % qb || (n_head_kv * head_dim) % 32)
        return vk::ctx_fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT,
                            "text_decoder_create: d_model, ffn_dim and n_head_q * head_dim must be multiples of the "
                            "quant block");
    if (!n_ctx || !n_stream || n_stream > 1024 || vocab > 0x7fffffff || !(rope_base > 0.0f) || !(rms_norm_eps >= 0.0f))
        return vk::ctx_fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT,
                            "text_decoder_create: n_ctx > 0, n_stream in 1..1024, rope_base > 0, rms_norm_eps >= 0");
    auto* m = new vokra_hip_text_decoder();
    m->ctx = c;
    m->wdtype = wdtype;
    m->n_layer = n_layer;
    m->d = d_model;
    m->hq = n_head_q;
    m->hkv = n_head_kv;
    m->hd = head_dim;
    m->ff = ffn_dim;
    m->vocab = vocab;
    m->n_ctx = n_ctx;
    m->n_stream = n_stream;
    m->rope_base = rope_base;
    m->eps = rms_norm_eps;
    m->scale = 1.0f / sqrtf((float)head_dim);  // 1.0f32 / (head_dim as f32).sqrt(), text_decoder.rs:1176
    int st = td_setup(m, layers, token_emb, final_norm_gamma, lm_head, block_size);
    if (st) {
        m->release();
        delete m;
        return st;
    }
    *out = m;
    return VOKRA_HIP_OK;
}

void vokra_hip_text_decoder_destroy(vokra_hip_text_decoder_t* m) {
    if (!m) return;
    m->release();
    delete m;
}

int vokra_hip_text_decoder_reset(vokra_hip_ctx_t* c, vokra_hip_text_decoder_t* m) {
    if (!c || !m || m->ctx != c) return vk::ctx_fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "text_decoder_reset: bad argument");
    SS_TRY(vokra_hip_kv_reset(c, m->kv));
    std::fill(m->position.begin(), m->position.end(), 0);
    return VOKRA_HIP_OK;
}

int vokra_hip_text_decoder_set_free_order(vokra_hip_ctx_t* c, vokra_hip_text_decoder_t* m, const int32_t* order,
                                          size_t n) {
    if (!c || !m || m->ctx != c)
        return vk::ctx_fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "text_decoder_set_free_order: bad argument");
    SS_TRY(vokra_hip_kv_set_free_order(c, m->kv, order, n));
    std::fill(m->position.begin(), m->position.end(), 0);
    return VOKRA_HIP_OK;
}

int vokra_hip_text_decoder_kv_pages(vokra_hip_ctx_t* c, vokra_hip_text_decoder_t* m, size_t* free_pages,
                                    size_t* pages_in_use) {
    if (!c || !m || m->ctx != c)
        return vk::ctx_fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "text_decoder_kv_pages: bad argument");
    return vokra_hip_kv_pages(c, m->kv, free_pages, pages_in_use);
}

int vokra_hip_text_decoder_position(vokra_hip_ctx_t* c, vokra_hip_text_decoder_t* m, size_t stream, size_t* position) {
    if (!c || !m || m->ctx != c || !position || stream >= m->n_stream)
        return vk::ctx_fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "text_decoder_position: bad argument");
    *position = (size_t)m->position[stream];
    return VOKRA_HIP_OK;
}

int vokra_hip_text_decoder_kv_restore(vokra_hip_ctx_t* c, vokra_hip_text_decoder_t* m, size_t stream, size_t n_pos,
                                      const float* k_rows, const float* v_rows) {
    if (!c || !m || m->ctx != c) return vk::ctx_fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "text_decoder_kv_restore: bad argument");
    if (stream >= m->n_stream) return vk::ctx_fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "text_decoder_kv_restore: stream out of range");
    if (n_pos > m->n_ctx)
        return vk::ctx_fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "text_decoder_kv_restore: position %zu > n_ctx %zu", n_pos,
                            m->n_ctx);
    if (n_pos && (!k_rows || !v_rows)) return vk::ctx_fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "text_decoder_kv_restore: NULL rows");
    const size_t w = m->hkv * m->hd;
    std::vector<int32_t> st(1024, (int32_t)stream), tt(1024);
    for (size_t l = 0; l < m->n_layer; ++l)
        for (size_t t0 = 0; t0 < n_pos; t0 += 1024) {
            const size_t cnt = std::min<size_t>(1024, n_pos - t0);
            for (size_t i = 0; i < cnt; ++i) tt[i] = (int32_t)(t0 + i);
            const size_t off = (l * n_pos + t0) * w;
            SS_TRY(vokra_hip_kv_append(c, m->kv, l, cnt, st.data(), tt.data(), k_rows + off, v_rows + off));
        }
    m->position[stream] = (int32_t)n_pos;
    return VOKRA_HIP_OK;
}

int vokra_hip_text_decoder_step_dev(vokra_hip_ctx_t* c, vokra_hip_text_decoder_t* m, size_t n, const int32_t* d_streams,
                                    const int32_t* d_tokens, const int32_t* d_positions, int32_t* d_next,
                                    float* d_logits) {
    if (!c || !m || m->ctx != c) return vk::ctx_fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "text_decoder_step: bad context");
    if (n == 0) return VOKRA_HIP_OK;
    if (n > m->n_stream) return vk::ctx_fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "text_decoder_step: more items than streams");
    if (!d_streams || !d_tokens || !d_positions || !d_next)
        return vk::ctx_fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "text_decoder_step: NULL buffer");
    return td_step(m, n, d_streams, d_tokens, d_positions, d_next, d_logits);
}

int vokra_hip_text_decoder_step(vokra_hip_ctx_t* c, vokra_hip_text_decoder_t* m, size_t n, const int32_t* streams,
                                const int32_t* tokens, int32_t* next_tokens, float* logits) {
    if (!c || !m || m->ctx != c) return vk::ctx_fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "text_decoder_step: bad context");
    if (n == 0) return VOKRA_HIP_OK;
    if (n > m->n_stream) return vk::ctx_fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "text_decoder_step: more items than streams");
    if (!streams || !tokens || !next_tokens)
        return vk::ctx_fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "text_decoder_step: NULL buffer");
    // forward_step's checks (text_decoder.rs:1007-1045), per stream
    std::vector<char> seen(m->n_stream, 0);
    std::vector<int32_t> items(3 * n);
    for (size_t i = 0; i < n; ++i) {
        if (streams[i] < 0 || (size_t)streams[i] >= m->n_stream || seen[streams[i]])
            return vk::ctx_fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT,
                                "text_decoder_step: streams must be distinct and < n_stream");
        seen[streams[i]] = 1;
        if (tokens[i] < 0 || (size_t)tokens[i] >= m->vocab)
            return vk::ctx_fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT,
                                "voxtral text_decoder.forward_step: token id %d >= vocab %zu", tokens[i], m->vocab);
        const int32_t p = m->position[streams[i]];
        if ((size_t)p + 1 > m->n_ctx)
            return vk::ctx_fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "voxtral text_decoder.forward_step: position %d > n_ctx %zu",
                                p + 1, m->n_ctx);
        items[i] = streams[i];
        items[n + i] = tokens[i];
        items[2 * n + i] = p;
    }
    int* dv = m->stage.i();
    SS_TRY(vokra_hip_memcpy_htod(c, dv, items.data(), 3 * n * 4));
    SS_TRY(td_step(m, n, dv, dv + n, dv + 2 * n, m->next.i(), logits ? m->logits.f() : nullptr));
    size_t appended = 0;
    SS_TRY(vokra_hip_kv_status(c, m->kv, &appended));
    for (size_t i = 0; i < n; ++i) m->position[streams[i]] += 1;  // the rows are appended
    SS_TRY(vokra_hip_memcpy_dtoh(c, next_tokens, m->next.p, n * 4));
    if (logits) SS_TRY(vokra_hip_memcpy_dtoh(c, logits, m->logits.p, n * m->vocab * sizeof(float)));
    return vk::range_check(c);
}

int vokra_hip_text_decoder_status(vokra_hip_ctx_t* c, vokra_hip_text_decoder_t* m, size_t* n_appended) {
    if (!c || !m || m->ctx != c) return vk::ctx_fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "text_decoder_status: bad argument");
    size_t a = 0;
    const int st = vokra_hip_kv_status(c, m->kv, &a);
    if (n_appended) *n_appended = a;
    return st ? st : vk::range_check(c);
}

}  // extern "C"

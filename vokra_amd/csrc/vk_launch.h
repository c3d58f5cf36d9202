// vk_launch.h — host launchers for the gfx950 kernels. Each launcher checks
// nothing: the C-ABI layer validates shapes before calling it.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

// What a GEMM epilogue applies after the bias (vk_common.h vk_epi_apply):
// gelu != 0 -> y = gelu(y); resid != NULL -> y = resid + y (may alias the output).
struct VkEpi {
    const float* resid;
    int gelu;
};
// The activation pass fused into the kernel that produces its input: for
// every row < m it writes, the producer stores the A fragments, scales and
// block sums launch_quantize_act_b32 would store (afrag == NULL: no fusion).
// Rows m .. m_pad-1 are not written (only their own GEMM rows read them).
struct VkQOut {
    uint4* afrag;
    float* ascale;
    float* asum;
    int m_pad;  // the fragments' padded row count
    int k;      // the quantized row width (a multiple of 32)
    int pow2;   // the power-of-two scale convention
    int g16;    // the K-quant layout instead: 16-wide groups (vk_q16_lane), m_pad a multiple of 16,
                // (scale, sum) pairs in ascale (asum not used by it)
};
// One linear of a multi-linear block-GEMM launch: bf16 fragments + scales,
// optional bias, output [m, n].
// With hi != null a block-GEMM linear's outputs (bias added) leave as the
// flash-attention kernel's fp16 operands, hi = fp16(x), lo = fp16(x - hi),
// row-major [rows][n], in place of f32 (vk_split_rows's arithmetic).
struct VkSplitOut {
    uint16_t* hi;
    uint16_t* lo;
};
struct VkGemmLin {
    const uint4* wfrag;
    const float* wscale;
    const float* bias;
    float* out;  // may be null when qo or so is set
    VkEpi epi;
    VkQOut qo;   // qo.afrag != null: the activation pass over the outputs (n % 128 == 0)
    VkSplitOut so;
};
// One linear of a decode-kernel launch: compact weights, optional bias, output [m, n].
struct VkGemvLin {
    const uint4* wq4;
    const uint2* wsc;
    const float* bias;
    float* out;
    VkEpi epi;
    int n;
};
// One linear of a Q4_K matmul launch (repacked weights, optional bias,
// output [m, n]); up to three linears over the same activations share a grid,
// tile0[i] being linear i's first column tile.
struct VkQ4kLin {
    const uint4* wq4;
    const float2* wdm;
    const float* bias;
    float* out;
    VkEpi epi;
    int n;
};
struct VkQ4kSet {
    VkQ4kLin l[3];
    int tile0[3];
    int count;
};

namespace vk {
constexpr int GEMM_TM = 128;  // block GEMM padding of m (a multiple of its workgroup tile)
constexpr int GEMM_TN = 128;  // block GEMM padding of n (a multiple of its workgroup tile)

hipError_t launch_dequantize_q0(hipStream_t s, int mode, const uint8_t* bytes, size_t n_blocks, float* out);
hipError_t launch_pack_q0(hipStream_t s, int mode, const float* x, size_t n_blocks, uint8_t* out);
hipError_t launch_copy_u4(hipStream_t s, const void* src, void* dst, size_t n16);
hipError_t launch_dequant_gemv_f32(hipStream_t s, int mode, const uint8_t* bytes, int n_rows, int n_bpr,
                                   const float* x, float* y);
hipError_t launch_quantize_act_b32(hipStream_t s, bool pow2, const float* a, int m, int m_pad, int k,
                                   uint4* afrag, float* ascale, float* asum);
// LayerNorm of [m, k] rows fused with the b32 activation pass (same results
// as launch_layer_norm_f32 followed by launch_quantize_act_b32); k <= kLnQuantMaxK
// (its LDS tile is k / 32 KiB).
constexpr int kLnQuantMaxK = 2048;  // = kLnRegCols (vk_common.h)
hipError_t launch_ln_quantize_b32(hipStream_t s, bool pow2, const float* a, int m, int m_pad, int k,
                                  const float* gamma, const float* beta, float eps, uint4* afrag, float* ascale,
                                  float* asum);
hipError_t launch_repack_w_b32(hipStream_t s, int mode, const uint8_t* wq, int n, int n_pad, int nb,
                               uint4* wfrag, float* wscale);
hipError_t launch_gemm_qblock(hipStream_t s, bool pow2, const uint4* afrag, const float* ascale,
                              const uint4* wfrag, const float* wscale, const float* bias, float* out, int m,
                              int m_pad, int n, int n_pad, int nb, VkEpi epi = {nullptr, 0},
                              const VkQOut* qo = nullptr);
// n_lin (1..3) linears of the same n over the same activations, one grid.
hipError_t launch_gemm_qblock_multi(hipStream_t s, bool pow2, const uint4* afrag, const float* ascale,
                                    const VkGemmLin* lins, int n_lin, int m, int m_pad, int n, int n_pad, int nb);
}  // namespace vk

namespace vk {
hipError_t launch_repack_w_gemv(hipStream_t s, int mode, const uint8_t* wq, int n, int n_pad, int nb, uint4* wq4,
                                uint2* wsc);
// n_lin (1..3) linears over the same activations, one launch.
hipError_t launch_gemv_qblock(hipStream_t s, int mode, bool pow2, const uint4* afrag, const float* ascale,
                              const float* asum, const VkGemvLin* lins, int n_lin, int m, int nb, int m_pad);
// One linear whose outputs feed the activation pass of the next input (qo:
// k == n, n % 32 == 0) instead of f32 out: the same fragments, scales and sums
// as launch_gemv_qblock followed by vk_quantize_act_b32.
hipError_t launch_gemv_qblock_quant(hipStream_t s, int mode, bool pow2, const uint4* afrag, const float* ascale,
                                    const float* asum, const VkGemvLin& lin, int m, int nb, int m_pad,
                                    const VkQOut& qo);
// n_lin (1..65535) linears described by a device array d_lins, one launch;
// n_max is the largest n among them.
hipError_t launch_gemv_qblock_group(hipStream_t s, int mode, bool pow2, const uint4* afrag, const float* ascale,
                                    const float* asum, const VkGemvLin* d_lins, int n_lin, int n_max, int m, int nb,
                                    int m_pad);
}  // namespace vk

namespace vk {
hipError_t launch_dequantize_q4k(hipStream_t s, const uint8_t* bytes, size_t nsb, float* out);
// K-quant activation pass: fragments, and (scale, sum) pairs in ascale
hipError_t launch_quantize_act_g16(hipStream_t s, const float* a, int m, int m_pad, int k, uint4* afrag,
                                   float* ascale);
hipError_t launch_repack_w_q4k(hipStream_t s, const uint8_t* wq, int n, int n_pad, int nsb, uint4* wq4,
                               float2* wdm);
hipError_t launch_gemm_q4k(hipStream_t s, const uint4* afrag, const float* ascale, const VkQ4kLin* lins, int n_lin,
                           int m, int nsb, int m_pad, int fmt);
// Q4_K / Q5_K / Q6_K (ggml tags 12 / 13 / 14) -> f32, bit-exact with gguf/quant.
hipError_t launch_dequantize_kq(hipStream_t s, int wdtype, const uint8_t* bytes, size_t nsb, float* out);
// Q5_K / Q6_K weights into the byte-word layout of the matmul's format 1.
hipError_t launch_repack_w_kq8(hipStream_t s, int wdtype, const uint8_t* wq, int n, int n_pad, int nsb, uint4* wq4,
                               float2* wdm);
// RMSNorm + the K-quant activation pass, and SwiGLU + the activation pass, in
// one launch each (bit-identical to vk_rms_norm_f32 / vk_swiglu_f32 followed by
// vk_quantize_act_g16); m_pad = round_up(m, 16), k % 256 == 0.
hipError_t launch_rms_quantize_g16(hipStream_t s, const float* in, const float* gamma, float eps, int m, int m_pad,
                                   int k, uint4* afrag, float* ascale);
hipError_t launch_swiglu_quantize_g16(hipStream_t s, const float* g, const float* u, int m, int m_pad, int k,
                                      uint4* afrag, float* ascale);
}  // namespace vk

namespace vk {
hipError_t launch_split_rows(hipStream_t s, const float* x, size_t n, float scale, void* hi, void* lo);
hipError_t launch_split_vt(hipStream_t s, const float* v, int batch, int t_kv, int t_pad, int h_kv, int hd, void* vth,
                           void* vtl);
// The same two splits with one-byte low parts (the compact form, vk_attn.hip
// split_q7): lo holds n bytes / one byte per V^T element.
hipError_t launch_split_rows_q7(hipStream_t s, const float* x, size_t n, float scale, void* hi, void* lo);
hipError_t launch_split_vt_q7(hipStream_t s, const float* v, int batch, int t_kv, int t_pad, int h_kv, int hd,
                              void* vth, void* vtl, bool tiled = false);
// x [B][T][H*hd] -> hi / lo [B][H][T][hd] (the attn_layout_heads K form)
hipError_t launch_split_rows_q7_heads(hipStream_t s, const float* x, int batch, int t, int h, int hd, float scale,
                                      void* hi, void* lo);
// Element strides of a flash launch's K / V operands: K element (b, t, h, d)
// at b * kb + h * kh + t * kt + d; V^T element (b, h, d, t) at
// (b * h_kv + h) * hd * t_pad + (t / 64) * vtile + d * vd + t % 64.
struct AttnLayout {
    long long kb, kh;
    int kt, vd, vtile;
};
// K [B][T][H*hd], V^T [B][H][hd][T_pad] (the split passes' default forms)
AttnLayout attn_layout_rows(int t_kv, int h_kv, int hd, int t_pad);
// K [B][H][T][hd], V^T [B][H][T_pad / 64][hd][64]: every 64-key tile of a
// head is one contiguous block (launch_split_rows_q7_heads, tiled V^T split)
AttnLayout attn_layout_heads(int t_kv, int h_kv, int hd, int t_pad);
// K / V low parts of a flash-attention launch: none (fp16 high parts only;
// kl, vtl unused), fp16, or the compact one-byte form (single-query launches).
enum { KV_LO_NONE = 0, KV_LO_F16 = 1, KV_LO_Q7 = 2 };
// The factor the flash kernel takes q in: its scores come out in base-2 units,
// so q is split (launch_split_rows) as q * attn_q_scale(scale) = q * scale *
// log2(e).
float attn_q_scale(float scale);
// qh / ql: the split of q * attn_q_scale(scale). hd * t_pad * 2 and
// 64 * hkv * hd * 2 must stay below 2^31 (buffer-resource extents).
hipError_t launch_flash_attn(hipStream_t s, int hd, const void* qh, const void* ql, const void* kh, const void* kl,
                             const void* vth, const void* vtl, float* out, int batch, int tq, int tkv, int t_pad,
                             int hq, int hkv, int causal, int q_off, const int* kv_index = nullptr,
                             int lo_mode = KV_LO_F16);
// The same with q given as f32 [B][Tq][Hq*hd] (16-byte aligned) and the
// softmax scale: the kernel splits q * attn_q_scale(q_scale) itself exactly
// as launch_split_rows would. With qo, the
// kernel also quantizes O (rows b * tq + i, width hq * hd) into qo's
// activation fragments, and out may be null.
hipError_t launch_flash_attn_f32q(hipStream_t s, int hd, const float* q, float q_scale, const void* kh, const void* kl,
                                  const void* vth, const void* vtl, float* out, int batch, int tq, int tkv, int t_pad,
                                  int hq, int hkv, int causal, int q_off, const int* kv_index = nullptr,
                                  int lo_mode = KV_LO_F16, const VkQOut* qo = nullptr,
                                  const AttnLayout* lay = nullptr);  // null: attn_layout_rows
}  // namespace vk

namespace vk {
// Device pointers and shape of one paged KV cache (see vk_kvcache.hip).
struct KvView {
    void *kq, *vq, *kd, *vd;
    int *table, *free_list, *meta;
    int n_layer, n_stream, width, hd, bs, ppl, cap, max_time;
};
hipError_t launch_kv_append(hipStream_t s, const KvView& v, int layer, int n, const int* streams, const int* times,
                            const float* k, const float* vv);
hipError_t launch_kv_read(hipStream_t s, const KvView& v, int layer, int t, int st, float* out, int* found);
hipError_t launch_kv_release(hipStream_t s, const KvView& v, int layer);
hipError_t launch_kv_reset(hipStream_t s, const KvView& v, const int* order, size_t pool_bytes, size_t scale_bytes);
hipError_t launch_kv_page_of(hipStream_t s, const KvView& v, int layer, int t, int* out);
// The grid's split count for keys up to max_len; each item uses its own
// length's split (pa_splits), at most this many.
int paged_attn_grid_splits(int max_len);
hipError_t launch_paged_attn(hipStream_t s, const KvView& v, int layer, int n, const int* streams, const int* lens,
                             const float* q, float scale, int hq, int hd, int n_split, float* out,
                             float* part_ml, float* part_o,
                             const VkQOut* qo = nullptr,  // also the activation pass over out (rows = items)
                             // fused append: item i's K / V rows (ak, av [n][width]) at time at[i] are
                             // packed into pages allocated beforehand (distinct streams; the generic
                             // kernel runs every head shape then)
                             const float* ak = nullptr, const float* av = nullptr, const int* at = nullptr,
                             // RoPE of q on load ([n][hd / 2] (cos, sin)): only where
                             // paged_attn_rotates_q holds, and without a fused append
                             const float2* rope_cs = nullptr);
// Whether launch_paged_attn runs the matrix-core GQA kernel for this shape and
// these buffers (the one that can rotate q on load).
bool paged_attn_rotates_q(const KvView& v, int hq, int hd, const float* q, const float* out, const float* part_o);
// The allocation of launch_kv_append for the same items appended to layers
// layer0 .. layer0 + n_layers - 1 in that order, in one launch (n_layers * n <= 4096).
// Read and clear the fp16-range flags of the attention kernels (vk_attn.hip)
// and of the GQA decode kernel (vk_kvcache.hip) on the current device.
// device addresses (current device) of the fp16-range flags of the attention
// kernels, the GEMM epilogue's split outputs and the cache's K/V packing
hipError_t attn_range_flag_addr(unsigned** p);
hipError_t gemm_range_flag_addr(unsigned** p);
hipError_t kv_range_flag_addr(unsigned** p);
// Packs rows into pages given by an earlier launch_kv_alloc_layers (items
// whose page is missing are skipped).
// rope_cs (optional, [n][hd / 2] (cos, sin)): k is rotated on the way in.
hipError_t launch_kv_write_allocated(hipStream_t s, const KvView& v, int layer, int n, const int* streams,
                                    const int* times, const float* k, const float* vv,
                                    const float2* rope_cs = nullptr, int hd = 0);
// cs[r][j] = (cos, sin) of positions[r] * theta[j], j < half: the angles of
// launch_rope_rows_qk for one step, for the fused rotations.
hipError_t launch_rope_table(hipStream_t s, const int* positions, const float* theta, int rows, int half, float2* cs);
// RoPE in place over x [rows][n_head * hd]: row r at positions[r] (or
// pos_offset + r when positions is NULL), theta [hd / 2] from the host.
hipError_t launch_rope_rows(hipStream_t s, float* x, int rows, int n_head, int hd, const float* theta,
                            const int* positions, int pos_offset);
// RoPE of q [rows][hq * hd] and k [rows][hkv * hd] at positions[r], one launch
// (the same values as two launch_rope_rows calls).
hipError_t launch_rope_rows_qk(hipStream_t s, float* q, float* k, int rows, int hq, int hkv, int hd,
                               const float* theta, const int* positions);
// out = silu(g) * u elementwise (out may alias g).
hipError_t launch_swiglu_f32(hipStream_t s, const float* g, const float* u, float* out, size_t n);
hipError_t launch_kv_alloc_layers(hipStream_t s, const KvView& v, int layer0, int n_layers, int n, int q_base,
                                  const int* streams, const int* times);
}  // namespace vk

namespace vk {
hipError_t launch_gemm_f32(hipStream_t s, bool b_trans, const float* a, const float* b, const float* bias,
                           float* out, int m, int n, int k,
                           VkEpi epi = {nullptr, 0});
hipError_t launch_gemv_f32(hipStream_t s, const float* a, const float* x, const float* bias, float* out, int m,
                           int k);
hipError_t launch_softmax_f32(hipStream_t s, const float* in, float* out, int rows, int cols);
hipError_t launch_layer_norm_f32(hipStream_t s, const float* in, float* out, int rows, int cols, const float* gamma,
                                 const float* beta, float eps);
hipError_t launch_rms_norm_f32(hipStream_t s, const float* in, float* out, int rows, int cols, const float* gamma,
                               float eps);
hipError_t launch_gelu_f32(hipStream_t s, const float* x, float* out, size_t n);
hipError_t launch_add_f32(hipStream_t s, const float* a, const float* b, float* out, size_t n);
hipError_t launch_embed_f32(hipStream_t s, const float* tok_emb, const float* pos_emb, const int* tokens,
                            const int* positions, int vocab, int n_pos, int d, int rows, float* out);
hipError_t launch_argmax_f32(hipStream_t s, const float* logits, int rows, int cols, int* out);
// The same argmax over 2048-column slices (many workgroups per row): part
// holds rows * argmax_n_slices(cols) pairs; rows at most 65535.
int argmax_n_slices(int cols);
hipError_t launch_argmax_sliced(hipStream_t s, const float* logits, int rows, int cols, float2* part, int* out);
// Fused tied logits + argmax: d a multiple of 128 (an even number of 16-wide
// k chunks in each of the kernel's four d quarters), rows of x and emb
// 16-byte aligned; logits may be null. part holds rows * logits_n_vt(vocab)
// float2.
constexpr int logits_min_d() { return 128; }
constexpr int logits_d_multiple() { return 128; }
int logits_n_vt(int vocab);
hipError_t launch_logits_argmax(hipStream_t s, const float* x, const float* emb, float* logits, float2* part,
                                int* next, int n, int vocab, int d);
}  // namespace vk

struct vokra_hip_ctx;
struct vokra_hip_qact;
struct vokra_hip_qweight;
struct vokra_hip_kv;
namespace vk {
hipStream_t ctx_stream(const vokra_hip_ctx* c);
int range_check(vokra_hip_ctx* c);  // INVALID_ARGUMENT when an fp16-range flag is raised
int ctx_fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
// Fused forms of entry-point sequences for the sessions (vk_capi.hip); each
// gives the same results as the sequence it replaces.
//   gemm_qact_epi    = vokra_hip_gemm_qact_dev, then GELU and/or + resid
//   gemm_qact_multi  = n (<= 3) vokra_hip_gemm_qact_dev over the same activations
//   qact_ln_quantize = vokra_hip_layer_norm_f32_dev into d_scratch, then
//                      vokra_hip_qact_quantize_dev (one kernel for AMAX127 / POW2)
int gemm_qact_epi(vokra_hip_ctx* c, const vokra_hip_qweight* w, const vokra_hip_qact* qa, const float* d_bias,
                  float* d_out, VkEpi epi);
int gemm_qact_multi(vokra_hip_ctx* c, int n, const vokra_hip_qweight* const* ws, const vokra_hip_qact* qa,
                    const float* const* biases, float* const* outs);
int qact_ln_quantize(vokra_hip_ctx* c, vokra_hip_qact* qa, size_t m, const float* d_in, const float* gamma,
                     const float* beta, float eps, int act_quant, float* d_scratch);
//   qact_rms_quantize_g16    = RMSNorm (vk_rms_norm_f32) of m rows of width k,
//                              then vokra_hip_qact_quantize_dev KQUANT
//   qact_swiglu_quantize_g16 = vk_swiglu_f32 of g, u [m, k], then the same pass
int qact_rms_quantize_g16(vokra_hip_ctx* c, vokra_hip_qact* qa, size_t m, size_t k, const float* d_in,
                          const float* gamma, float eps);
int qact_swiglu_quantize_g16(vokra_hip_ctx* c, vokra_hip_qact* qa, size_t m, size_t k, const float* d_g,
                             const float* d_u);
//   attn_quantize       = vokra_hip_attn_f32_dev into d_out, then
//                         vokra_hip_qact_quantize_dev of its batch * t_q rows
//                         (d_out is then scratch: the fused kernel may skip it)
//   paged_attn_quantize = vokra_hip_paged_attn_dev into d_out, then
//                         vokra_hip_qact_quantize_dev of its n rows
//   gemm_qact_quantize  = gemm_qact_epi into d_out, then vokra_hip_qact_quantize_dev
//                         of its rows into qa_out (d_out is then scratch: the
//                         fused block-GEMM epilogue skips it)
int gemm_qact_quantize(vokra_hip_ctx* c, const vokra_hip_qweight* w, const vokra_hip_qact* qa, const float* d_bias,
                       float* d_out, VkEpi epi, vokra_hip_qact* qa_out, int act_quant);
int attn_quantize(vokra_hip_ctx* c, size_t batch, size_t tq, size_t tkv, size_t hq, size_t hkv, size_t hd,
                  const float* d_q, const float* d_k, const float* d_v, float scale, int causal, size_t q_off,
                  float* d_out, vokra_hip_qact* qa, int act_quant);
//   gemm_qact_qkv_split + launch_split_vt + attn_quantize_split =
//   gemm_qact_multi of q, k, v, then attn_quantize (non-causal self-attention),
//   with k leaving the GEMM already as the attention kernel's fp16 hi / lo
//   operands (vk_split_rows's values). *fused is false (and nothing ran) when
//   the three linears do not take the one-grid block-GEMM route; the caller
//   then runs the pair it replaces.
int gemm_qact_qkv_split(vokra_hip_ctx* c, const vokra_hip_qweight* const* ws, const vokra_hip_qact* qa,
                        const float* const* biases, float* q_out, const VkSplitOut& ks, float* v_out, bool* fused);
int attn_quantize_split(vokra_hip_ctx* c, size_t batch, size_t t, size_t h, size_t hd, const float* d_q,
                        const void* kh, const void* kl, const void* vth, const void* vtl, size_t t_pad, float scale,
                        float* d_out, vokra_hip_qact* qa, int act_quant);
int paged_attn_quantize(vokra_hip_ctx* c, vokra_hip_kv* kv, size_t layer, size_t n, const int* d_streams,
                        const int* d_lens, size_t max_len, size_t hq, const float* d_q, float scale, float* d_out,
                        vokra_hip_qact* qa, int act_quant, const float2* rope_cs = nullptr,
                        const float* d_ak = nullptr, const float* d_av = nullptr, const int* d_at = nullptr);
// With d_ak / d_av / d_at (K-quant activations only): the items' K / V rows
// at times d_at are first packed into pages an earlier kv_alloc_layers gave,
// k rotated by rope_cs when given, inside the attention launch (= a
// kv_write_allocated before it).
// Whether paged_attn_quantize can rotate q itself for this cache and buffers.
bool paged_attn_rotates_q(const vokra_hip_kv* kv, size_t n, size_t hq, const float* d_q, const float* d_out);
//   kv_alloc_layers + paged_attn_append_quantize (one per layer, in layer
//   order) = per layer vokra_hip_kv_append_dev of the items' K / V rows at
//   d_times, then paged_attn_quantize; for distinct streams whose new time
//   step lies inside d_lens, and a cache with room for every append.
int kv_alloc_layers(vokra_hip_ctx* c, vokra_hip_kv* kv, size_t first_layer, size_t layer0, size_t n_layers, size_t n,
                    const int* d_streams, const int* d_times);
//   kv_alloc_layers + kv_write_allocated (per layer) = per layer
//   vokra_hip_kv_append_dev of the items' rows at d_times.
int kv_write_allocated(vokra_hip_ctx* c, vokra_hip_kv* kv, size_t layer, size_t n, const int* d_streams,
                       const int* d_times, const float* d_k, const float* d_v, const float2* rope_cs = nullptr);
int paged_attn_append_quantize(vokra_hip_ctx* c, vokra_hip_kv* kv, size_t layer, size_t n, const int* d_streams,
                               const int* d_times, const float* d_k, const float* d_v, const int* d_lens,
                               size_t max_len, size_t hq, const float* d_q, float scale, float* d_out,
                               vokra_hip_qact* qa, int act_quant);
// For a session's own fused producer: the output binding of an activation
// pass over m rows of qa (qo->afrag NULL: no fused form, run the pass), and
// the record of it once the producer is launched.
int qact_output(vokra_hip_ctx* c, vokra_hip_qact* qa, size_t m, int act_quant, VkQOut* qo);
void qact_outputs_written(vokra_hip_qact* qa, size_t m, int act_quant);
}  // namespace vk

namespace vk {
// Whisper front end (vk_frontend.hip): frame grid 3000 x 400, 201 bins.
int fe_n_frames();
int fe_n_bins();
int fe_n_fft();
int logmel_n_partial();
}  // namespace vk
#include <vector>
namespace vk {
void fe_hann_periodic(std::vector<float>& w);
void fe_dft_basis(std::vector<float>& b);
void fe_mel_filterbank(int n_mels, std::vector<float>& w);
hipError_t launch_stft_frames(hipStream_t s, const float* pcm, int batch, int n_samples, const float* win,
                              float* frames);
hipError_t launch_power_spec(hipStream_t s, const float* spec, float* power, size_t rows);
hipError_t launch_logmel_finish(hipStream_t s, const float* mel, int batch, int n_mels, float* out, float* partial);
hipError_t launch_im2col(hipStream_t s, bool trans, const float* x, size_t sb, size_t sc, size_t sp, int batch,
                         int in_ch, int in_len, int kernel, int stride, int padding, int out_len, float* col);
hipError_t launch_add_row_bias(hipStream_t s, float* out, const float* bias, int rows, int cols);
hipError_t launch_add_pos(hipStream_t s, float* out, const float* pos, size_t rows, int d, int period);
}  // namespace vk

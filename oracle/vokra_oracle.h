/*
 * vokra_oracle.h — CPU restatement of the reference (ayutaz/vokra) arithmetic
 * on the quantized-transformer hot path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the parity checker for the HIP
 * kernels in vokra_amd/csrc. Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it; the product path never does.
 *
 * Every function names the reference file:line it restates (paths relative to
 * the ayutaz/vokra repository root). The reference is Rust; the semantics that
 * matter for bit parity are reproduced explicitly:
 *   - f32::round       -> roundf (half away from zero)
 *   - `as i8/i32` casts saturate and map NaN to 0 (explicit clamps below)
 *   - f32::max         -> fmaxf (NaN-ignoring)
 *   - Iterator::sum    -> sequential left fold from -0.0 (Rust >= 1.82)
 *   - no FMA contraction anywhere (built with -ffp-contract=off)
 *
 * Status codes mirror vokra_status_t (include/vokra.h:56-66 in the reference).
 */
#ifndef VOKRA_ORACLE_H
#define VOKRA_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    VO_OK = 0,
    VO_UNSUPPORTED_OP = 3,
    VO_BACKEND_UNAVAILABLE = 4,
    VO_INVALID_ARGUMENT = 5,
    VO_KV_CACHE_EXHAUSTED = 10,
};

/* KvQuant discriminants in declaration order (kv_quant/mod.rs:81-91). */
enum { VO_KV_FP32 = 0, VO_KV_Q4_0 = 1, VO_KV_Q5_0 = 2, VO_KV_Q8_0 = 3 };

/* Weight dtypes for gemm_q_f32, numbered by their ggml type tags
 * (gguf/tensor.rs:57-95 for the K-quants; 2/6/8 are ggml's Q4_0/Q5_0/Q8_0). */
enum { VO_W_Q4_0 = 2, VO_W_Q5_0 = 6, VO_W_Q8_0 = 8, VO_W_Q4_K = 12, VO_W_Q5_K = 13, VO_W_Q6_K = 14 };

/* ---- binary16 (A1) ---------------------------------------------------- */
float vo_f16_bits_to_f32(uint16_t h);
uint16_t vo_f32_to_f16_bits(float x);
float vo_gguf_f16_to_f32(uint16_t h);
uint16_t vo_convert_f32_to_f16(float x);

/* ---- Q_0 block codecs (A2, A3, A4, A5) ---------------------------------- */
size_t vo_kv_block_bytes(int mode);
void vo_pack_block(int mode, const float *in32, uint8_t *out);
void vo_unpack_block(int mode, const uint8_t *blk, float *out32);
int vo_dequantize_bytes(int mode, const uint8_t *bytes, size_t n_bytes, float *out, size_t out_len);
int vo_pack_matrix_to_bytes(int mode, const float *a, size_t n_rows, size_t n_bpr, uint8_t *out);

/* ---- dequant GEMV (A6, A7) -------------------------------------------- */
int vo_validate_dequant_gemv(int mode, size_t n_bytes, size_t n_rows, size_t n_bpr, size_t x_len);
int vo_dequant_gemv_scalar(int mode, const uint8_t *bytes, size_t n_bytes, size_t n_rows,
                           size_t n_bpr, const float *x, size_t x_len, float *y);
void vo_dense_gemv_f32(const float *a, size_t n_rows, const float *x, size_t x_len, float *y);

/* ---- block-format INT8 GEMM (Q8_0 / Q4_0 / Q5_0 weights, gemm_q_f32) -- */
void vo_quantize_act_b32(const float *x, size_t k, int8_t *q, float *scale, int32_t *gsum);
void vo_quantize_act_b32_mode(const float *x, size_t k, int8_t *q, float *scale, int32_t *gsum, int pow2);
int vo_gemm_qblock_i8_mode(int wdtype, size_t m, size_t n, size_t k, const float *a,
                           const uint8_t *wq, size_t wq_len, const float *bias, float *out, int pow2);
int vo_qblock_block_dots_mode(int wdtype, size_t m, size_t n, size_t k, const float *a,
                              const uint8_t *wq, int32_t *dots, int pow2);
int vo_qblock_weight_ints(int wdtype, const uint8_t *blk, int8_t *q32, float *d);
int vo_gemm_qblock_i8(int wdtype, size_t m, size_t n, size_t k, const float *a,
                      const uint8_t *wq, size_t wq_len, const float *bias, float *out);
int vo_qblock_block_dots(int wdtype, size_t m, size_t n, size_t k, const float *a,
                         const uint8_t *wq, int32_t *dots);
float vo_qblock_error_bound(int wdtype, const uint8_t *w_row, const float *x, size_t k);

/* ---- K-quant (A8, A9, A10) ---------------------------------------------- */
int vo_kquant_dequantize(int wdtype, const uint8_t *bytes, size_t n_bytes, size_t n_elements, float *out);
int vo_kquant_quantize(int wdtype, const float *data, size_t n, uint8_t *out);
void vo_kquant_quantize_activations(const float *x, size_t k, int8_t *q, float *scales, int32_t *gsums);
int vo_kquant_gemv_i8(int wdtype, size_t m, size_t k, const uint8_t *w, size_t w_len,
                      const float *x, size_t x_len, float *out, size_t out_len);
int vo_kquant_gemm_i8(int wdtype, size_t m, size_t k, size_t n_act, const uint8_t *w,
                      size_t w_len, const float *x, size_t x_len, float *out, size_t out_len);
float vo_int8_error_bound(int wdtype, const uint8_t *w_row, const float *x, size_t k);
int vo_gemm_q_f32(int wdtype, size_t m, size_t n, size_t k, const float *a, size_t a_len,
                  const uint8_t *wq, size_t wq_len, const float *bias, float *out, size_t out_len);

/* ---- f32 scalar kernels (A11, A12) -------------------------------------- */
void vo_gemm_f32(size_t m, size_t n, size_t k, const float *a, const float *b, const float *bias, float *out);
void vo_gemm_f32_mt(size_t m, size_t n, size_t k, const float *a, const float *b, const float *bias,
                    float *out, int n_threads);
void vo_gemv_f32(size_t m, size_t k, const float *a, const float *x, const float *bias, float *out);
void vo_softmax_f32(const float *in, float *out, size_t rows, size_t cols);
void vo_layer_norm_f32(const float *in, float *out, size_t rows, size_t cols, const float *gamma,
                       const float *beta, float eps);
void vo_gelu_f32(const float *x, float *out, size_t n);
float vo_erf_as(float x);
void vo_rms_norm_f32(const float *x, const float *gamma, float eps, size_t rows, size_t d, float *out);
int vo_rope_apply(float *x, size_t x_len, size_t seq_len, size_t head_dim, float rope_base, size_t position_offset);
void vo_silu_inplace(float *x, size_t n);
int vo_hadamard_inplace(float *a, size_t a_len, const float *b, size_t b_len);

/* ---- attention (A13, A14) ----------------------------------------------- */
int vo_sdpa_whisper(size_t t_q, size_t t_kv, size_t n_head, size_t hd, const float *q,
                    const float *k, const float *v, int causal, size_t q_pos_offset, float *out);
int vo_gqa_attention(size_t t, size_t t_kv, size_t n_head_q, size_t n_head_kv, size_t hd,
                     const float *q, const float *k_cache, const float *v_cache, float scale,
                     size_t position_offset, float *out);

/* ---- paged quantized KV cache (A15) ------------------------------------- */
typedef struct vo_paged_cache vo_paged_cache;
int vo_paged_create(size_t n_layer, size_t n_head, size_t d_head, size_t n_stream, size_t max_time,
                    size_t block_size, int mode, vo_paged_cache **out);
void vo_paged_destroy(vo_paged_cache *c);
int vo_paged_append_step(vo_paged_cache *c, size_t layer, size_t t, size_t s, const float *k_row,
                         const float *v_row);
int vo_paged_read_step(const vo_paged_cache *c, size_t layer, size_t t, size_t s, float *k_out,
                       float *v_out);
int vo_paged_release_layer(vo_paged_cache *c, size_t layer);
void vo_paged_reset(vo_paged_cache *c);
size_t vo_paged_free_pages(const vo_paged_cache *c);
size_t vo_paged_pages_in_use(const vo_paged_cache *c);
long vo_paged_page_of(const vo_paged_cache *c, size_t layer, size_t t);

/* ---- decode, RNG ------------------------------------------------------- */
uint32_t vo_argmax(const float *logits, size_t n);
void vo_xorshift_rand_vec(uint64_t seed, size_t n, float *out);
void vo_splitmix_gaussian(uint64_t seed, size_t n, float *out);

/* Whisper log-mel front end and conv1d */
void vo_hann_periodic(size_t len, float *w);
void vo_mel_filterbank(size_t sr, size_t n_fft, size_t n_mels, double fmin, double fmax, float *w);
int vo_log_mel(const float *pcm, size_t n_pcm, size_t n_mels, float *out);
int vo_conv1d_f32(const float *input, size_t in_ch, size_t in_len, const float *weight, size_t out_ch,
                  size_t kernel, const float *bias, size_t stride, size_t padding, float *out);

#ifdef __cplusplus
}
#endif
#endif

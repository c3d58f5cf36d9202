/*
 * vokra_hip.h — C ABI of the MI355X (gfx950) quantized-transformer hot path.
 *
 * A drop-in device arm for the reference's backend seams. Every entry point
 * names the reference interface it replaces (paths relative to the
 * ayutaz/vokra repository root). Plain pointers and sizes only.
 *
 * Error convention (crates/vokra-core/src/error.rs:21-104 mapped as in
 * include/vokra.h:56-66): every fallible call returns a vokra_hip_status_t;
 * the message of the last failure on the calling thread is available from
 * vokra_hip_last_error(). A missing or failed device is
 * VOKRA_HIP_ERROR_BACKEND_UNAVAILABLE, a shape mismatch
 * VOKRA_HIP_ERROR_INVALID_ARGUMENT, an uncovered dtype
 * VOKRA_HIP_ERROR_UNSUPPORTED_OP. Nothing ever falls back to the CPU.
 *
 * Buffers: the "copy mode" calls take host pointers and behave like the
 * reference's per-op GPU methods (upload, launch, synchronize, read back;
 * crates/vokra-backend-cuda/src/context.rs:1701-1768). The "_dev" calls take
 * device pointers, enqueue on the context's stream and return without
 * synchronizing; argument errors are still reported synchronously.
 */
#ifndef VOKRA_HIP_H
#define VOKRA_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum vokra_hip_status_t {
    VOKRA_HIP_OK = 0,
    VOKRA_HIP_ERROR_IO = 1,                  /* VokraError::Io */
    VOKRA_HIP_ERROR_MODEL_LOAD = 2,          /* VokraError::ModelLoad */
    VOKRA_HIP_ERROR_UNSUPPORTED_OP = 3,      /* VokraError::UnsupportedOp */
    VOKRA_HIP_ERROR_BACKEND_UNAVAILABLE = 4, /* VokraError::BackendUnavailable */
    VOKRA_HIP_ERROR_INVALID_ARGUMENT = 5,    /* VokraError::InvalidArgument */
    VOKRA_HIP_ERROR_OTHER = 9,
    VOKRA_HIP_ERROR_KV_CACHE_EXHAUSTED = 10  /* VokraError::KvCacheExhausted */
} vokra_hip_status_t;

/* KvQuant in declaration order (crates/vokra-core/src/kv_quant/mod.rs:81-91). */
typedef enum vokra_hip_kv_quant_t {
    VOKRA_HIP_KV_FP32 = 0,
    VOKRA_HIP_KV_Q4_0 = 1,
    VOKRA_HIP_KV_Q5_0 = 2,
    VOKRA_HIP_KV_Q8_0 = 3
} vokra_hip_kv_quant_t;

/* Weight dtypes of gemm_q_f32, numbered by ggml type tag. The reference's
 * KQuantDtype (crates/vokra-backend-cpu/src/kernels/kquant.rs:56-63) covers
 * the K-quants; the block formats are this arm's extension of the seam. */
typedef enum vokra_hip_wdtype_t {
    VOKRA_HIP_W_Q4_0 = 2,
    VOKRA_HIP_W_Q5_0 = 6,
    VOKRA_HIP_W_Q8_0 = 8,
    VOKRA_HIP_W_Q4_K = 12,
    VOKRA_HIP_W_Q5_K = 13,
    VOKRA_HIP_W_Q6_K = 14
} vokra_hip_wdtype_t;

/* Activation quantization convention of the INT8 matmul.
 * AMAX127: per 32-element block s = amax/127, q = clamp(round(v/s), +-127)
 *          (the K-quant convention of kquant.rs:418-441 at group 32).
 * POW2:    per 32-element block s = smallest power of two >= amax/127
 *          (shared-exponent int8, as in the OCP MXINT8 format).
 * KQUANT:  per 16-element group exactly kquant.rs:418-441 (s = amax/127,
 *          q = clamp(round(v/s), +-127), plus the group sum); the only
 *          convention of Q4_K weights, which always use it. */
typedef enum vokra_hip_act_quant_t {
    VOKRA_HIP_ACT_AMAX127 = 0,
    VOKRA_HIP_ACT_POW2 = 1,
    VOKRA_HIP_ACT_KQUANT = 2
} vokra_hip_act_quant_t;

typedef struct vokra_hip_ctx vokra_hip_ctx_t;
typedef struct vokra_hip_qweight vokra_hip_qweight_t;
typedef struct vokra_hip_event vokra_hip_event_t;

/* ---- lifecycle ---------------------------------------------------------- */

/* Number of visible HIP devices; BACKEND_UNAVAILABLE when the runtime has
 * none. Replaces the CUDA device probe (crates/vokra-backend-cuda/src/probe.rs). */
int vokra_hip_probe(int *n_devices);

/* Context on one device with its own default-priority stream. Replaces
 * CudaContext::new (crates/vokra-backend-cuda/src/context.rs:1167);
 * destroy replaces its Drop (:4769). */
int vokra_hip_create(int device, vokra_hip_ctx_t **out);
void vokra_hip_destroy(vokra_hip_ctx_t *ctx);

/* Message of the last failed call on this thread ("" if none). Replaces
 * vokra_last_error (include/vokra.h:455): per thread, never fails. */
const char *vokra_hip_last_error(void);

/* Blocks until the context stream drains (the CUDA context's sync_stream,
 * crates/vokra-backend-cuda/src/context.rs:4711); reports asynchronous faults, and
 * INVALID_ARGUMENT when an attention kernel met an operand outside its fp16
 * range since the last such check (the flag is per device and is cleared by
 * the report). */
int vokra_hip_synchronize(vokra_hip_ctx_t *ctx);

/* ---- device memory and timing (resident mode plumbing) ------------------ */
/* Raw-byte forms of CudaContext::alloc_dev / upload / download
 * (crates/vokra-backend-cuda/src/context.rs:3162-3215), synchronous copies.
 * The events have no reference counterpart: measurement plumbing. */
int vokra_hip_device_alloc(vokra_hip_ctx_t *ctx, size_t bytes, void **dptr);
int vokra_hip_device_free(vokra_hip_ctx_t *ctx, void *dptr);
int vokra_hip_memcpy_htod(vokra_hip_ctx_t *ctx, void *dst, const void *src, size_t bytes);
int vokra_hip_memcpy_dtoh(vokra_hip_ctx_t *ctx, void *dst, const void *src, size_t bytes);
int vokra_hip_event_create(vokra_hip_ctx_t *ctx, vokra_hip_event_t **ev);
int vokra_hip_event_record(vokra_hip_ctx_t *ctx, vokra_hip_event_t *ev);
int vokra_hip_event_elapsed_ms(vokra_hip_event_t *start, vokra_hip_event_t *stop, float *ms);
void vokra_hip_event_destroy(vokra_hip_event_t *ev);
/* Device-to-device copy by a plain streaming kernel (bytes % 16 == 0, both
 * pointers 16-byte aligned); the HBM bandwidth reference. No reference
 * counterpart: plumbing for measurement. */
int vokra_hip_copy_dev(vokra_hip_ctx_t *ctx, void *d_dst, const void *d_src, size_t bytes);

/* ---- HIP graphs: capture a sequence of _dev calls, replay it ------------- */
/* Launch-bound loops (a decode step, a stream of GEMVs) are recorded once
 * and replayed as one graph launch. Only calls that allocate nothing may be
 * captured (resident weights, pre-created qact buffers). The reference has
 * no counterpart; its sessions synchronize once per step instead
 * (crates/vokra-backend-cuda/src/context.rs:5310). */
typedef struct vokra_hip_graph vokra_hip_graph_t;
int vokra_hip_capture_begin(vokra_hip_ctx_t *ctx);
int vokra_hip_capture_end(vokra_hip_ctx_t *ctx, vokra_hip_graph_t **out);
int vokra_hip_graph_launch(vokra_hip_ctx_t *ctx, vokra_hip_graph_t *g);
void vokra_hip_graph_destroy(vokra_hip_graph_t *g);

/* ---- block dequantization and the fused dequant GEMV ---------------------- */

/* Wire Q4_0/Q5_0/Q8_0 blocks -> f32, bit-exact. Replaces
 * kv_quant::dequantize_bytes_into (crates/vokra-core/src/kv_quant/mod.rs:336-359). */
int vokra_hip_dequantize_bytes(vokra_hip_ctx_t *ctx, int mode, const uint8_t *bytes, size_t n_bytes,
                               float *out, size_t out_len);

/* K-quant super-blocks -> f32, bit-exact. Replaces gguf::quant::dequantize
 * (crates/vokra-core/src/gguf/quant/mod.rs:42-63) for GgmlType::Q4K
 * (q4_k.rs:34-69: y = d*sc*q - dmin*m, two roundings), Q5K (q5_k.rs:36-80:
 * the same with a fifth quant bit) and Q6K (q6_k.rs:34-72: y = d*sc*(q - 32)):
 * n_elements must be a multiple of 256 and n_bytes = n_elements/256 * 144,
 * 176 or 210 (a mismatch is INVALID_ARGUMENT, the reference's
 * TensorSizeMismatch). */
int vokra_hip_kquant_dequantize(vokra_hip_ctx_t *ctx, int wdtype, const uint8_t *bytes, size_t n_bytes,
                                size_t n_elements, float *out);

/* f32 -> wire Q4_0/Q5_0/Q8_0 blocks, bit-exact with the reference packers
 * (BlockQ8_0::pack q8_0.rs:40-64, BlockQ4_0::pack q4_0.rs:44-68,
 * BlockQ5_0::pack) as driven by pack_matrix_to_bytes
 * (crates/vokra-core/src/kv_quant/dequant_gemm.rs:137-186): n must be a
 * multiple of 32 and out_len must equal n/32 * block_bytes. */
int vokra_hip_quantize_bytes(vokra_hip_ctx_t *ctx, int mode, const float *x, size_t n, uint8_t *out,
                             size_t out_len);
/* Same on device pointers (async on the context stream). */
int vokra_hip_quantize_bytes_dev(vokra_hip_ctx_t *ctx, int mode, const float *d_x, size_t n, uint8_t *d_out);

/* y[r] = sum_k dequant(row r)[k] * x[k], f32 semantics. Replaces
 * KvQuantDequantGemvOps::fused_dequant_gemv (crates/vokra-core/src/kv_quant/gpu_ops.rs:70-80)
 * as implemented by CudaContext::dequant_gemv_f32 (crates/vokra-backend-cuda/src/context.rs:1686-1768),
 * validated exactly as validate_dequant_gemv (gpu_ops.rs:95-131). y has n_rows floats. */
int vokra_hip_dequant_gemv_f32(vokra_hip_ctx_t *ctx, int mode, const uint8_t *blocks, size_t n_bytes,
                               size_t n_rows, size_t n_blocks_per_row, const float *x, size_t x_len,
                               float *y);

/* ---- quantized-weight matmul ---------------------------------------------- */

/* out[m, n] = sum_l a[m, l] * dequant(wq[n, l]) (+ bias[n]) through INT8
 * activations. Replaces Compute::gemm_q_f32 (crates/vokra-models/src/compute.rs:943-963)
 * -> kernels::gemm_q_f32 (crates/vokra-backend-cpu/src/kernels/mod.rs:341-364)
 * -> gemm_driver::run_q (gemm_driver.rs:312-332): wq is the untransposed
 * [n, k] payload, a is [m, k], out is [m, n], bias is added after. Block
 * formats use the context's activation convention (default AMAX127); the
 * K-quants (Q4_K, Q5_K, Q6_K: the reference's whole KQuantDtype) run
 * kquant_gemm_i8 (kquant.rs:845-935) over unpack_block_i8's unified
 * representation (:332-407): k a multiple of 256, KQUANT activations,
 * bit-identical outputs. */
int vokra_hip_gemm_q_f32(vokra_hip_ctx_t *ctx, int wdtype, size_t m, size_t n, size_t k, const float *a,
                         size_t a_len, const uint8_t *wq, size_t wq_len, const float *bias, float *out,
                         size_t out_len);

/* Activation convention for the block-format INT8 path of this context. No
 * reference counterpart: the reference has no block-format INT8 route (its
 * one INT8 route is the K-quant one, which always uses KQUANT). */
int vokra_hip_set_act_quant(vokra_hip_ctx_t *ctx, int act_quant);

/* No reference counterpart. Kernel routing for m <= 64 (default 1 = the decode kernel that streams the
 * compact weights; 0 = the tiled GEMM). Both give bit-identical results; the
 * switch exists so callers and tests can compare them. */
int vokra_hip_set_decode_kernel(vokra_hip_ctx_t *ctx, int enable);

/* Device-resident weight: uploads the [n, k] wire payload once and builds
 * the device layouts the kernels stream (the reference keeps weights
 * device-resident in its sessions, context.rs:5025). */
int vokra_hip_qweight_upload(vokra_hip_ctx_t *ctx, int wdtype, size_t n, size_t k, const uint8_t *wq,
                             size_t wq_len, vokra_hip_qweight_t **out);
void vokra_hip_qweight_free(vokra_hip_qweight_t *w);

/* gemm_q_f32 on device pointers against a resident weight (async on the
 * context stream). d_a: [m, k] f32 (16-byte aligned), d_bias: [n] or NULL,
 * d_out: [m, n]. act_quant selects the block-format convention; Q4_K
 * weights ignore it and use KQUANT. */
int vokra_hip_gemm_q_f32_dev(vokra_hip_ctx_t *ctx, const vokra_hip_qweight_t *w, size_t m,
                             const float *d_a, const float *d_bias, float *d_out, int act_quant);

/* gemm_q_f32_dev that allocates nothing. No counterpart in the reference: it
 * is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc). The INT8
 * activation pass writes its fragments, scales and sums into a 32 MiB
 * workspace that the library holds per device for the life of the process;
 * every byte a call reads is written by that call. Results are bit-identical
 * to vokra_hip_gemm_q_f32_dev. Shapes whose workspace exceeds 32 MiB
 * (2.5 * round_up(m, 128) * k bytes, 256-byte aligned regions) are
 * INVALID_ARGUMENT. Calls on one device share the workspace: calls that
 * overlap in time on that device (other streams or contexts) race. */
int vokra_hip_gemm_q_f32_dev_noalloc(vokra_hip_ctx_t *ctx, const vokra_hip_qweight_t *w, size_t m,
                                     const float *d_a, const float *d_bias, float *d_out, int act_quant);

/* gemm_q_f32_dev split in its two launches, for callers that feed one
 * activation matrix to several weights (the q/k/v projections of
 * crates/vokra-models/src/whisper/nn.rs:185-197 read the same LN output):
 * quantize once into a qact buffer, then run any number of GEMMs on it. */
typedef struct vokra_hip_qact vokra_hip_qact_t;
int vokra_hip_qact_create(vokra_hip_ctx_t *ctx, size_t max_m, size_t k, vokra_hip_qact_t **out);
void vokra_hip_qact_free(vokra_hip_qact_t *qa);
int vokra_hip_qact_quantize_dev(vokra_hip_ctx_t *ctx, vokra_hip_qact_t *qa, size_t m, const float *d_a,
                                int act_quant);
/* The weight and the activations must agree: Q4_K weights take KQUANT
 * activations (k a multiple of 256), block formats AMAX127 or POW2. */
int vokra_hip_gemm_qact_dev(vokra_hip_ctx_t *ctx, const vokra_hip_qweight_t *w, const vokra_hip_qact_t *qa,
                            const float *d_bias, float *d_out);

/* A fixed set of decode linears over the same activations, run as ONE launch:
 * count (1..65535) block-format weights of one dtype and one k, each with its
 * own bias (d_biases NULL, or per-entry NULL = no bias) and output [m, n_i]
 * (device pointers, kept by the group). Every output is bit-identical to
 * vokra_hip_gemm_qact_dev of the same weight. Rows m <= 64 run as one decode-
 * kernel launch over a device descriptor table (any mix of n); larger m falls
 * back to one block-GEMM launch per linear. No counterpart in the reference
 * (it issues one gemm_q_f32 per linear, compute.rs:943-963): it serves callers
 * that apply many linears to one batch (q/k/v, heads, expert groups) and
 * streams their weights at HBM rate instead of paying one launch each. */
typedef struct vokra_hip_linear_group vokra_hip_linear_group_t;
int vokra_hip_linear_group_create(vokra_hip_ctx_t *ctx, size_t count, const vokra_hip_qweight_t *const *weights,
                                  const float *const *d_biases, float *const *d_outs, vokra_hip_linear_group_t **out);
int vokra_hip_linear_group_run(vokra_hip_ctx_t *ctx, vokra_hip_linear_group_t *group, const vokra_hip_qact_t *qa);
void vokra_hip_linear_group_destroy(vokra_hip_linear_group_t *group);

/* ---- f32 GEMM / GEMV and row kernels -------------------------------------- */

/* out[m, n] = bias[n] + a[m, k] . b[k, n], f32 (matrix cores in f32: exact
 * products, f32 sums in tree order). Replaces Compute::gemm_f32
 * (crates/vokra-models/src/compute.rs:901-920) -> kernels::gemm_f32
 * (crates/vokra-backend-cpu/src/kernels/mod.rs:298-311, scalar.rs:41-72),
 * with validate_gemm's checks (mod.rs:238-254); bias has n floats or is NULL. */
int vokra_hip_gemm_f32(vokra_hip_ctx_t *ctx, size_t m, size_t n, size_t k, const float *a, size_t a_len,
                       const float *b, size_t b_len, const float *bias, float *out, size_t out_len);
/* Device pointers; b_trans = 1 reads b as [n, k] (weights stored [out, in],
 * e.g. the tied token embedding of the logits projection). */
int vokra_hip_gemm_f32_dev(vokra_hip_ctx_t *ctx, size_t m, size_t n, size_t k, const float *d_a, const float *d_b,
                           int b_trans, const float *d_bias, float *d_out);
/* out[m] = bias[m] + a[m, k] . x. Replaces Compute::gemv_f32 (compute.rs:966-985)
 * -> kernels::gemv_f32 (mod.rs:391-407, scalar.rs:74-91). */
int vokra_hip_gemv_f32(vokra_hip_ctx_t *ctx, size_t m, size_t k, const float *a, size_t a_len, const float *x,
                       size_t x_len, const float *bias, float *out, size_t out_len);
int vokra_hip_gemv_f32_dev(vokra_hip_ctx_t *ctx, size_t m, size_t k, const float *d_a, const float *d_x,
                           const float *d_bias, float *d_out);
/* Row softmax (scalar.rs:177-199), LayerNorm with population variance
 * (scalar.rs:201-222), RMSNorm (crates/vokra-models/src/voxtral/text_decoder.rs:801-822).
 * Replace Compute::softmax_f32 / layer_norm_f32 (compute.rs:988-1030). */
int vokra_hip_softmax_f32(vokra_hip_ctx_t *ctx, const float *in, size_t in_len, float *out, size_t out_len,
                          size_t rows, size_t cols);
int vokra_hip_layer_norm_f32(vokra_hip_ctx_t *ctx, const float *in, size_t in_len, float *out, size_t out_len,
                             size_t rows, size_t cols, const float *gamma, size_t gamma_len, const float *beta,
                             size_t beta_len, float eps);
int vokra_hip_rms_norm_f32(vokra_hip_ctx_t *ctx, const float *in, size_t in_len, float *out, size_t out_len,
                           size_t rows, size_t cols, const float *gamma, size_t gamma_len, float eps);
int vokra_hip_softmax_f32_dev(vokra_hip_ctx_t *ctx, const float *d_in, float *d_out, size_t rows, size_t cols);
int vokra_hip_layer_norm_f32_dev(vokra_hip_ctx_t *ctx, const float *d_in, float *d_out, size_t rows, size_t cols,
                                 const float *d_gamma, const float *d_beta, float eps);
int vokra_hip_rms_norm_f32_dev(vokra_hip_ctx_t *ctx, const float *d_in, float *d_out, size_t rows, size_t cols,
                               const float *d_gamma, float eps);
/* GELU through the Abramowitz & Stegun 7.1.26 erf (scalar.rs:126-172).
 * Replaces Compute::gelu_f32. */
int vokra_hip_gelu_f32(vokra_hip_ctx_t *ctx, const float *x, float *out, size_t n);
int vokra_hip_gelu_f32_dev(vokra_hip_ctx_t *ctx, const float *d_x, float *d_out, size_t n);
/* Per-row argmax, first strict maximum from -inf (crates/vokra-core/src/decode/sampler.rs:197-206). */
int vokra_hip_argmax_f32_dev(vokra_hip_ctx_t *ctx, const float *d_logits, size_t rows, size_t cols,
                             int32_t *d_out);

/* Tied logits and greedy argmax in one pass over the embedding:
 * logits[s, v] = emb[v, :] . x[s, :] for s < rows, v < vocab, then
 * next[s] = the first strict maximum of row s from -inf (NaN never wins, ties
 * keep the lowest index, 0 when nothing beats -inf). Replaces
 * project_logits_into (crates/vokra-models/src/whisper/decoder.rs:754-796:
 * gemv_f32 / gemm_f32 of token_emb [vocab, d] against h) followed by argmax
 * (crates/vokra-core/src/decode/sampler.rs:197-206). f32 products and sums
 * (sum order differs from the sequential fold). d must be a multiple of 64;
 * x and emb 16-byte aligned. d_logits may be NULL: the logits are then not
 * written at all. Device pointers. */
int vokra_hip_logits_argmax_dev(vokra_hip_ctx_t *ctx, size_t rows, size_t vocab, size_t d, const float *d_x,
                                const float *d_emb, float *d_logits, int32_t *d_next);

/* ---- fused attention --------------------------------------------------- */

/* Scaled-dot-product attention, f32 in and out, per batch b and query head h
 * (kv head h / (n_head_q / n_head_kv)):
 *   S = (q * scale) . k^T, -inf where causal and key j > q_offset + i,
 *   P = softmax over keys, out = P . v.
 * q and out are [batch, t_q, n_head_q * head_dim], k and v
 * [batch, t_kv, n_head_kv * head_dim], row-major with heads side by side.
 * Replaces the attention core of Compute::attn_f32
 * (crates/vokra-models/src/compute.rs:2703-2742) as computed by
 * attention_from_kv_into (crates/vokra-models/src/whisper/nn.rs:209-325; q is
 * scaled before the product, scale = head_dim^-0.5 there) and the GQA loop of
 * crates/vokra-models/src/voxtral/text_decoder.rs:1302-1360 (n_head_kv <
 * n_head_q). The projections around it are gemm_q_f32 calls. head_dim is 64
 * or 128 (else UNSUPPORTED_OP); t_kv = 0 gives zeros. Products run as fp16
 * hi/lo split MFMAs (three per product, f32 accumulation): results agree with
 * the f32 reference to about 1e-6 relative. With t_q = 1 (decode) the low
 * parts of k and v are held in one byte each, an integer times the fp16 high
 * part's ulp / 128 (a quarter fewer bytes for the bandwidth-bound
 * single-query case). Each k / v element then carries a relative error of at
 * most 2^-18 / (1 - 2^-12) when |x| >= 2^-7; below that (fp16 exponent field
 * under 8, subnormals included) the low byte is zero and the element is the
 * plain fp16 rounding, an absolute error of at most 2^-19. The decoder
 * session's cross-attention uses the same form. q is split as
 * q * scale * log2(e) (the softmax runs in base 2); a finite element of that,
 * of k or of v with magnitude >= 65520 (beyond fp16) is INVALID_ARGUMENT: here
 * after the launch, for the _dev form at the next vokra_hip_synchronize. */
int vokra_hip_attn_f32(vokra_hip_ctx_t *ctx, size_t batch, size_t t_q, size_t t_kv, size_t n_head_q,
                       size_t n_head_kv, size_t head_dim, const float *q, const float *k, const float *v,
                       float scale, int causal, size_t q_offset, float *out);
/* Same on device pointers (16-byte aligned q, k, out), async on the context
 * stream; uses the context's attention workspace (grown on first use). */
int vokra_hip_attn_f32_dev(vokra_hip_ctx_t *ctx, size_t batch, size_t t_q, size_t t_kv, size_t n_head_q,
                           size_t n_head_kv, size_t head_dim, const float *d_q, const float *d_k,
                           const float *d_v, float scale, int causal, size_t q_offset, float *d_out);

/* ---- paged quantized KV cache in HBM ------------------------------------- */

/* QuantizedPagedKvCache (crates/vokra-core/src/cache/paged_quant.rs:240-545)
 * on the device, one codebook: pages of block_size time steps x all streams
 * of one layer, page table entry layer * pages_per_layer + t / block_size,
 * LIFO free list, rows stored as Q8_0 blocks of 32 (bit-identical packing and
 * dequantization). The table, free list and allocator state live in device
 * memory; appends allocate pages on the GPU. This arm stores Q8_0 rows only
 * (other modes are UNSUPPORTED_OP) with d_head 64 or 128. */
typedef struct vokra_hip_kv vokra_hip_kv_t;

/* QuantizedPagedKvCache::new (paged_quant.rs:260-307): same rejections. */
int vokra_hip_kv_create(vokra_hip_ctx_t *ctx, size_t n_layer, size_t n_head, size_t d_head, size_t n_stream,
                        size_t max_time, size_t block_size, int mode, vokra_hip_kv_t **out);
void vokra_hip_kv_destroy(vokra_hip_kv_t *kv);

/* append_step (paged_quant.rs:396-437) for items i = 0..n-1 in order:
 * (streams[i], times[i]) with rows k_rows[i], v_rows[i] of n_head*d_head
 * floats; host arrays, synchronous. The first item that is out of range
 * (INVALID_ARGUMENT) or finds no free page (KV_CACHE_EXHAUSTED) stops the
 * batch; earlier items stay appended, as with successive calls. n <= 1024. */
int vokra_hip_kv_append(vokra_hip_ctx_t *ctx, vokra_hip_kv_t *kv, size_t layer, size_t n, const int32_t *streams,
                        const int32_t *times, const float *k_rows, const float *v_rows);
/* Same with device arrays, asynchronous; the outcome is read by kv_status. */
int vokra_hip_kv_append_dev(vokra_hip_ctx_t *ctx, vokra_hip_kv_t *kv, size_t layer, size_t n,
                            const int32_t *d_streams, const int32_t *d_times, const float *d_k, const float *d_v);
/* Synchronizes and returns the last append's status (n_appended items done):
 * append_step's result (paged_quant.rs:396-437) for the asynchronous form. */
int vokra_hip_kv_status(vokra_hip_ctx_t *ctx, vokra_hip_kv_t *kv, size_t *n_appended);

/* read_step (paged_quant.rs:448-480): dequantized rows, *found = 0 for None. */
int vokra_hip_kv_read(vokra_hip_ctx_t *ctx, vokra_hip_kv_t *kv, size_t layer, size_t t, size_t s, float *k_out,
                      float *v_out, int *found);
/* reset (paged_quant.rs:489-493) and release_layer (:500-515). */
int vokra_hip_kv_reset(vokra_hip_ctx_t *ctx, vokra_hip_kv_t *kv);
int vokra_hip_kv_release_layer(vokra_hip_ctx_t *ctx, vokra_hip_kv_t *kv, size_t layer);
/* free_pages / pages_in_use (paged_quant.rs:343-353). */
int vokra_hip_kv_pages(vokra_hip_ctx_t *ctx, vokra_hip_kv_t *kv, size_t *free_pages, size_t *pages_in_use);
/* The page id of table entry (layer, t / block_size), -1 if none. No
 * reference counterpart (inspection of page placement). */
int vokra_hip_kv_page_of(vokra_hip_ctx_t *ctx, vokra_hip_kv_t *kv, size_t layer, size_t t, long *page);
/* Resets the cache with the free list set to `order` (a permutation of the
 * page ids, top of the stack last): places pages at shuffled addresses. No
 * reference counterpart (the reference always starts from [cap-1 .. 0]). */
int vokra_hip_kv_set_free_order(vokra_hip_ctx_t *ctx, vokra_hip_kv_t *kv, const int32_t *order, size_t n);

/* Decode attention over the cache: for item i (stream streams[i], keys
 * 0..lens[i]-1 of `layer`) and query head h (kv head h / (n_head_q / n_head)):
 * out = softmax((q * scale) . K^T) . V with K, V the cache's dequantized
 * rows. q and out are [n, n_head_q * d_head]. The single-step case of
 * attention_from_kv_into (crates/vokra-models/src/whisper/nn.rs:209-325) and
 * the GQA loop (crates/vokra-models/src/voxtral/text_decoder.rs:1302-1360)
 * reading QuantizedPagedKvCache rows (the intent of GpuPagedKvCacheOps,
 * crates/vokra-core/src/cache/paged.rs:941-986). n_head_q / n_head in
 * {1, 2, 4, 8}. Host arrays, synchronous: */
int vokra_hip_paged_attn(vokra_hip_ctx_t *ctx, vokra_hip_kv_t *kv, size_t layer, size_t n, const int32_t *streams,
                         const int32_t *lens, size_t n_head_q, const float *q, float scale, float *out);
/* Device arrays, asynchronous; max_len bounds every lens[i] (sizes the key
 * split). */
int vokra_hip_paged_attn_dev(vokra_hip_ctx_t *ctx, vokra_hip_kv_t *kv, size_t layer, size_t n,
                             const int32_t *d_streams, const int32_t *d_lens, size_t max_len, size_t n_head_q,
                             const float *d_q, float scale, float *d_out);

/* out = a + b on device (residual connections; add_assign in the reference's
 * model code, crates/vokra-models/src/whisper/nn.rs). */
int vokra_hip_add_f32_dev(vokra_hip_ctx_t *ctx, const float *d_a, const float *d_b, float *d_out, size_t n);

/* ---- Whisper front end ---------------------------------------------------- */

/* whisper::mel::log_mel (crates/vokra-models/src/whisper/mel.rs:123-183; fused
 * form crates/vokra-ops/src/fused_logmel.rs:80-175) for `batch` clips of
 * n_samples 16 kHz samples each, pcm [batch][n_samples]: each clip zero-padded
 * or trimmed to 30 s, STFT (n_fft 400, hop 160, periodic Hann, reflect
 * centre padding, trailing frame dropped), Slaney mel bands, log10 with the
 * 1e-10 floor, per-clip (max(v, gmax - 8) + 4) / 4. out [batch][n_mels][3000]. */
int vokra_hip_log_mel(vokra_hip_ctx_t *ctx, const float *pcm, size_t batch, size_t n_samples, size_t n_mels,
                      float *out, size_t out_len);
int vokra_hip_log_mel_dev(vokra_hip_ctx_t *ctx, const float *d_pcm, size_t batch, size_t n_samples, size_t n_mels,
                          float *d_out);
/* kernels::conv1d_f32 (crates/vokra-backend-cpu/src/kernels/mod.rs:583-822;
 * Compute::conv1d_f32): input [in_ch, in_len], weight [out_ch, in_ch, kernel],
 * optional bias [out_ch], out [out_ch, out_len] with
 * out_len = (in_len + 2 padding - kernel) / stride + 1; the same rejections
 * (zero stride or kernel, padded length shorter than the kernel, length
 * mismatches). */
int vokra_hip_conv1d_f32(vokra_hip_ctx_t *ctx, const float *input, size_t input_len, size_t in_ch, size_t in_len,
                         const float *weight, size_t weight_len, size_t out_ch, size_t kernel, const float *bias,
                         size_t stride, size_t padding, float *out, size_t out_len);
int vokra_hip_conv1d_f32_dev(vokra_hip_ctx_t *ctx, const float *d_input, size_t in_ch, size_t in_len,
                             const float *d_weight, size_t out_ch, size_t kernel, const float *d_bias, size_t stride,
                             size_t padding, float *d_out);

/* ---- GGUF model files ------------------------------------------------------- */

typedef struct vokra_hip_gguf vokra_hip_gguf_t;

/* GgufFile::open over a read-only mapping (crates/vokra-core/src/gguf/
 * reader.rs:126-190 with crates/vokra-mmap): GGUF v3 header, typed metadata,
 * tensor infos, aligned data region, with the reader's checks (magic,
 * version, counts, alignment, rank <= 8, duplicate names, offsets inside the
 * file, whole blocks). Tensor types: F32, F16, Q4_0, Q5_0, Q8_0, Q4_K (the
 * reference accepts F32/F16/Q4_K/Q5_K/Q6_K/BF16, tensor.rs:85-95; this file
 * adds the block formats its GEMMs run). No GPU is touched. */
int vokra_hip_gguf_open(const char *path, vokra_hip_gguf_t **out);
void vokra_hip_gguf_close(vokra_hip_gguf_t *f);
int vokra_hip_gguf_tensor_count(const vokra_hip_gguf_t *f, size_t *n);
/* GgufFile::tensors / tensor_bytes (crates/vokra-core/src/gguf/reader.rs:213,242):
 * name, ggml type tag, dims (up to 8, ggml
 * order: dims[0] is the contiguous axis) and the payload inside the mapping. */
int vokra_hip_gguf_tensor_info(const vokra_hip_gguf_t *f, size_t index, const char **name, uint32_t *ggml_type,
                               size_t *n_dims, uint64_t *dims, const void **data, size_t *n_bytes);
/* GgufFile::tensor_info by name (reader.rs:218); MODEL_LOAD when absent. */
int vokra_hip_gguf_find(const vokra_hip_gguf_t *f, const char *name, size_t *index);
/* GgufFile::get (reader.rs:208) for integer / bool and string values. */
int vokra_hip_gguf_meta_int(const vokra_hip_gguf_t *f, const char *key, int64_t *out);
int vokra_hip_gguf_meta_str(const vokra_hip_gguf_t *f, const char *key, const char **out, size_t *len);
/* A 2-D block-quant weight straight from the mapping into a resident weight,
 * as vokra_hip_qweight_upload. Dims are read as the reference's loader reads a
 * Linear weight, [out_features, in_features] (crates/vokra-models/src/whisper/
 * weights.rs:460-470): the fused-quant-weights route (weights.rs:454-509). */
int vokra_hip_gguf_upload_qweight(vokra_hip_ctx_t *ctx, const vokra_hip_gguf_t *f, const char *name,
                                  vokra_hip_qweight_t **out);
/* GgufFile::tensor_f32 (reader.rs:256) for F32 / F16 tensors (host output). */
int vokra_hip_gguf_read_f32(const vokra_hip_gguf_t *f, const char *name, float *out, size_t out_len);

/* ---- pre-norm encoder session ------------------------------------------- */

/* One pre-norm block with quantized linears: wire-format weights [out, in]
 * (block or K-quant dtype), f32 norms and biases (NULL = no bias). The quant
 * counterpart of PrenormLayer (crates/vokra-core/src/prenorm.rs), which the
 * reference holds in f32 only. */
typedef struct vokra_hip_prenorm_layer {
    const float *ln1_gamma, *ln1_beta;
    const uint8_t *wq, *wk, *wv, *wo;  /* [d, d] */
    const float *bq, *bk, *bv, *bo;
    const float *ln2_gamma, *ln2_beta;
    const uint8_t *w1, *w2;            /* fc1 [d_ff, d], fc2 [d, d_ff] */
    const float *b1, *b2;
} vokra_hip_prenorm_layer_t;

typedef struct vokra_hip_encoder vokra_hip_encoder_t;

/* Device-resident encoder: uploads every layer once (the reference's
 * Compute::encode_prenorm_encoder, crates/vokra-models/src/compute.rs:2775, over
 * the blocks of crates/vokra-models/src/whisper/encoder.rs:180-245). max_rows
 * bounds batch * frames of a forward. */
int vokra_hip_encoder_create(vokra_hip_ctx_t *ctx, int wdtype, size_t n_layer, size_t d_model, size_t n_head,
                             size_t d_ff, const vokra_hip_prenorm_layer_t *layers, const float *ln_post_gamma,
                             const float *ln_post_beta, size_t max_rows, vokra_hip_encoder_t **out);
void vokra_hip_encoder_destroy(vokra_hip_encoder_t *enc);
/* x [batch, frames, d] (the conv stem's output) -> out [batch, frames, d]:
 * per block h += attn(LN1 h) (non-causal, scale head_dim^-0.5), h += MLP(LN2 h)
 * with GELU, then ln_post. Device pointers, asynchronous. */
int vokra_hip_encoder_forward_dev(vokra_hip_ctx_t *ctx, vokra_hip_encoder_t *enc, size_t batch, size_t frames,
                                  const float *d_x, float *d_out);
/* Host arrays, synchronous. */
int vokra_hip_encoder_forward(vokra_hip_ctx_t *ctx, vokra_hip_encoder_t *enc, size_t batch, size_t frames,
                              const float *x, float *out);
/* The conv stem in front of the blocks (crates/vokra-models/src/whisper/
 * encoder.rs:58-104): conv1 [d, n_mels, 3] (stride 1, pad 1) + GELU, conv2
 * [d, d, 3] (stride 2, pad 1) + GELU, transposed to [frames / 2, d] plus the
 * positional embedding pos_emb [n_frames / 2, d]. Host arrays, copied. */
int vokra_hip_encoder_set_stem(vokra_hip_ctx_t *ctx, vokra_hip_encoder_t *enc, size_t n_mels, size_t n_frames,
                               const float *conv1_w, const float *conv1_b, const float *conv2_w,
                               const float *conv2_b, const float *pos_emb);
/* WhisperEncoder::encode (encoder.rs:41-178): log-mel [batch][n_mels][n_frames]
 * -> stem -> blocks -> ln_post, out [batch][n_frames / 2][d]. Device pointers,
 * asynchronous; needs vokra_hip_encoder_set_stem first. */
int vokra_hip_encoder_encode_dev(vokra_hip_ctx_t *ctx, vokra_hip_encoder_t *enc, size_t batch,
                                 const float *d_log_mel, float *d_out);
int vokra_hip_encoder_encode(vokra_hip_ctx_t *ctx, vokra_hip_encoder_t *enc, size_t batch, const float *log_mel,
                             float *out);
/* The stem part of encode alone (encoder.rs:58-104): log-mel -> conv1 + GELU
 * -> conv2 + GELU -> + pos_emb into d_x [batch][n_frames / 2][d], the input
 * encode then hands to the blocks (encode == stem, then forward, bit for
 * bit). Device pointers, asynchronous. */
int vokra_hip_encoder_stem_dev(vokra_hip_ctx_t *ctx, vokra_hip_encoder_t *enc, size_t batch,
                               const float *d_log_mel, float *d_x);

/* ---- batched decoder-step session --------------------------------------- */

/* One Whisper decoder block with quantized linears (the quant counterpart of
 * DecoderLayerView, crates/vokra-core/src/prenorm.rs). */
typedef struct vokra_hip_decoder_layer {
    const float *ln1_gamma, *ln1_beta;            /* self-attention LN */
    const uint8_t *wq, *wk, *wv, *wo;
    const float *bq, *bk, *bv, *bo;
    const float *ln2_gamma, *ln2_beta;            /* cross-attention LN */
    const uint8_t *cwq, *cwk, *cwv, *cwo;
    const float *cbq, *cbk, *cbv, *cbo;
    const float *ln3_gamma, *ln3_beta;            /* MLP LN */
    const uint8_t *w1, *w2;
    const float *b1, *b2;
} vokra_hip_decoder_layer_t;

typedef struct vokra_hip_decoder vokra_hip_decoder_t;

/* Device-resident batched decoder for n_stream concurrent streams: quantized
 * weights, f32 token/positional embeddings (the token embedding doubles as the
 * tied output projection), a paged Q8_0 self-KV cache (block_size-token pages)
 * and per-stream cross K/V. Replaces Compute::new_decoder_step_session /
 * DecoderStepSession (crates/vokra-models/src/compute.rs:2892-3139) with the
 * batch axis the reference lacks. */
int vokra_hip_decoder_create(vokra_hip_ctx_t *ctx, int wdtype, size_t n_layer, size_t d_model, size_t n_head,
                             size_t d_ff, size_t n_vocab, size_t n_text_ctx, size_t n_audio_ctx, size_t n_stream,
                             size_t block_size, const vokra_hip_decoder_layer_t *layers, const float *token_emb,
                             const float *pos_emb, const float *ln_post_gamma, const float *ln_post_beta,
                             vokra_hip_decoder_t **out);
void vokra_hip_decoder_destroy(vokra_hip_decoder_t *dec);
/* Sets stream `stream`'s cross K/V from its encoder output enc [n_audio_ctx, d]
 * for every layer (k = enc.Wk + bk, v = enc.Wv + bv, as
 * cross_attention_capture, crates/vokra-models/src/whisper/nn.rs:342-399). */
int vokra_hip_decoder_set_encoder(vokra_hip_ctx_t *ctx, vokra_hip_decoder_t *dec, size_t stream, const float *enc);
int vokra_hip_decoder_set_encoder_dev(vokra_hip_ctx_t *ctx, vokra_hip_decoder_t *dec, size_t stream,
                                      const float *d_enc);
/* Precision of the cross-attention K/V reads. VOKRA_HIP_CROSS_F32 (default):
 * K and V are held as an fp16 high part plus a one-byte low part scaled by the
 * high part's ulp (the single-query form of vokra_hip_attn_f32): relative
 * error at most 2^-18 / (1 - 2^-12) per element of magnitude >= 2^-7, absolute
 * error at most 2^-19 below it (plain fp16 rounding there), against the
 * reference's f32 cross_attention (crates/vokra-models/src/whisper/nn.rs:
 * 342-399, decoder.rs:492-510). VOKRA_HIP_CROSS_F16 reads the fp16 high parts
 * only: two thirds of the bytes of the step's largest stream, with K and V
 * rounded to fp16 (relative 2^-11). A performance mode with no counterpart in
 * the reference; it may be switched between steps (both parts stay stored). */
#define VOKRA_HIP_CROSS_F32 0
#define VOKRA_HIP_CROSS_F16 1
int vokra_hip_decoder_set_cross_precision(vokra_hip_ctx_t *ctx, vokra_hip_decoder_t *dec, int precision);
/* Empties the self-KV cache of every stream (DecoderStepSession::reset,
 * crates/vokra-models/src/compute.rs:3073). */
int vokra_hip_decoder_reset(vokra_hip_ctx_t *ctx, vokra_hip_decoder_t *dec);
/* Resets the decoder (every stream back to length 0) with its self-KV cache's
 * free list set to `order`, a permutation of the cache's page ids (top of the
 * stack last), as vokra_hip_kv_set_free_order: later steps' pages land at
 * shuffled addresses, the page-table placement a long-running server ends up
 * with. Results do not depend on it. No reference counterpart (the reference
 * cache always starts from [cap-1 .. 0], paged_quant.rs:152-216). */
int vokra_hip_decoder_set_free_order(vokra_hip_ctx_t *ctx, vokra_hip_decoder_t *dec, const int32_t *order, size_t n);
/* free_pages / pages_in_use (paged_quant.rs:343-353) of the decoder's self-KV cache (vokra_hip_kv_pages;
 * their sum is the page count a free order must permute). */
int vokra_hip_decoder_kv_pages(vokra_hip_ctx_t *ctx, vokra_hip_decoder_t *dec, size_t *free_pages,
                               size_t *pages_in_use);
/* One decode step of n streams (distinct): stream streams[i] feeds token
 * tokens[i] at position positions[i] (its current length). Per stream this is
 * WhisperDecoder::step_into (crates/vokra-models/src/whisper/decoder.rs:413-567)
 * with one token, then greedy argmax (decode/sampler.rs:197-206) into
 * next_tokens[i]; logits [n, n_vocab] are written when not NULL. Host arrays,
 * synchronous; rejects token >= n_vocab and position >= n_text_ctx as the
 * reference does, a stream whose encoder output was never set (the reference
 * builds cross K/V before the first step, decoder.rs:171-211), and a position
 * other than the stream's current length (the reference takes the position
 * from its cache, decoder.rs:427-434) or 0 (which restarts the stream; later
 * rows of its old history are never read). */
int vokra_hip_decoder_step(vokra_hip_ctx_t *ctx, vokra_hip_decoder_t *dec, size_t n, const int32_t *streams,
                           const int32_t *tokens, const int32_t *positions, int32_t *next_tokens, float *logits);
/* Device arrays, asynchronous (capturable in a HIP graph once warmed up). The
 * caller guarantees what the host variant checks: distinct streams in range,
 * tokens < n_vocab, positions = the stream's length or 0 and < n_text_ctx.
 * A stream whose encoder output is not set attends over zero cross K/V. These
 * calls do not update the lengths the host variant checks: drive a session
 * through one of the two. An item outside the cache ends the step's page
 * allocation; vokra_hip_decoder_status reports it. */
int vokra_hip_decoder_step_dev(vokra_hip_ctx_t *ctx, vokra_hip_decoder_t *dec, size_t n, const int32_t *d_streams,
                               const int32_t *d_tokens, const int32_t *d_positions, int32_t *d_next_tokens,
                               float *d_logits);
/* Synchronizes and reports the last step's page allocation as
 * vokra_hip_kv_status does (INVALID_ARGUMENT for an item outside the cache,
 * KV_CACHE_EXHAUSTED; *n_appended = (layer, item) appends done, layer-major),
 * then INVALID_ARGUMENT if an attention operand left the fp16 range. */
int vokra_hip_decoder_status(vokra_hip_ctx_t *ctx, vokra_hip_decoder_t *dec, size_t *n_appended);

/* ---- Whisper sessions from a GGUF file ------------------------------------ */

/* WhisperConfig (crates/vokra-models/src/whisper/config.rs:58-100) as read by
 * WhisperConfig::from_gguf (config.rs:106-170): the vokra.whisper.* keys, each
 * an unsigned u32-range integer, decoder_start_ids a non-empty u32 array, the
 * optional alignment_heads an even-length array of in-range (layer, head)
 * pairs, n_text_state == n_audio_state, head counts dividing d_model, no zero
 * hyperparameter. MODEL_LOAD with the reference's "whisper config: ..."
 * message otherwise. */
typedef struct vokra_hip_whisper_config {
    size_t n_mels, d_model, n_audio_ctx, n_audio_head, n_audio_layer;
    size_t n_text_ctx, n_text_head, n_text_layer, n_vocab, ffn_dim;
    uint32_t eot;
} vokra_hip_whisper_config_t;
int vokra_hip_whisper_config_from_gguf(const vokra_hip_gguf_t *f, vokra_hip_whisper_config_t *cfg);

/* How the Linear weights were bound (the counterpart of QuantBindReport,
 * weights.rs:145-160): taken verbatim from the mapping (already in the session
 * dtype), or packed from F32/F16 on the device. */
typedef struct vokra_hip_whisper_load_report {
    size_t verbatim, packed;
} vokra_hip_whisper_load_report_t;

/* WhisperWeights::load_with (weights.rs:302-378) with fused-quant weights,
 * building the sessions directly: the encoder half (conv stem, embed_positions,
 * model.encoder.layers.{i}.{self_attn_layer_norm, self_attn.{q,k,v,out}_proj,
 * final_layer_norm, fc1, fc2}, model.encoder.layer_norm) into an encoder
 * session with its stem set, and the decoder half (embed_tokens,
 * embed_positions, model.decoder.layers.{i}.{self_attn..., encoder_attn...,
 * fc1, fc2}, model.decoder.layer_norm) into a decoder session. Tensors are
 * checked in the reference's order with its shapes (PyTorch order) and
 * messages ("whisper weight `<name>`: missing from GGUF", "... shape [..] !=
 * expected [..]"). A Linear whose ggml type equals wdtype goes to the session
 * from the mapping; an F32/F16 Linear is packed when wdtype is Q8_0, Q4_0 or
 * Q5_0; anything else is UNSUPPORTED_OP naming the tensor. report may be NULL.
 * Divergence: a K-quant Linear whose in_features is not a multiple of 256
 * (its rows straddle super-blocks: d_model 384 or 640 models, or any FFN width
 * off the 256 grid) stays on the reference's f32 dequant path and is counted
 * in report.dequantized_unaligned (weights.rs:471-512); these sessions hold
 * quantized Linears only, so such a file is UNSUPPORTED_OP ("in_features 384
 * is not a multiple of 256"), naming the first such tensor. */
int vokra_hip_whisper_encoder_from_gguf(vokra_hip_ctx_t *ctx, const vokra_hip_gguf_t *f,
                                        const vokra_hip_whisper_config_t *cfg, int wdtype, size_t max_rows,
                                        vokra_hip_whisper_load_report_t *report, vokra_hip_encoder_t **out);
int vokra_hip_whisper_decoder_from_gguf(vokra_hip_ctx_t *ctx, const vokra_hip_gguf_t *f,
                                        const vokra_hip_whisper_config_t *cfg, int wdtype, size_t n_stream,
                                        size_t block_size, vokra_hip_whisper_load_report_t *report,
                                        vokra_hip_decoder_t **out);

/* ---- speech-LLM text decoder (Voxtral-style backbone) ------------------- */

/* rope_apply (crates/vokra-models/src/voxtral/text_decoder.rs:858-891) on every
 * head of x [seq_len, n_head * head_dim], in place, host memory: row i is at
 * position position_offset + i and each head's pairs (j, j + head_dim/2)
 * rotate by m * theta_j. theta_j = rope_base^(-2j/head_dim) is evaluated on the
 * host with the reference's f32 expression (so the angle is its f32 product),
 * sin / cos on the device (about 1 ulp of libm). An odd head_dim or a length
 * mismatch is INVALID_ARGUMENT, as rope_apply's. */
int vokra_hip_rope_f32(vokra_hip_ctx_t *ctx, float *x, size_t x_len, size_t seq_len, size_t n_head, size_t head_dim,
                       float rope_base, size_t position_offset);
/* Device rows d_x [rows, n_head * head_dim], row r at position d_positions[r].
 * The context keeps the frequency table of the last (rope_base, head_dim); a
 * new pair uploads its table synchronously first (not capturable). */
int vokra_hip_rope_f32_dev(vokra_hip_ctx_t *ctx, float *d_x, size_t rows, size_t n_head, size_t head_dim,
                           float rope_base, const int32_t *d_positions);
/* The SwiGLU gate: silu_inplace then hadamard_inplace (text_decoder.rs:
 * 826-847, sequenced at :1405-1410): out = (g * (1 / (1 + e^-g))) * up with the
 * reference's roundings (device expf). A length mismatch is INVALID_ARGUMENT. */
int vokra_hip_swiglu_f32(vokra_hip_ctx_t *ctx, const float *gate, size_t gate_len, const float *up, size_t up_len,
                         float *out);
int vokra_hip_swiglu_f32_dev(vokra_hip_ctx_t *ctx, const float *d_gate, const float *d_up, size_t n, float *d_out);

/* One pre-norm block of the text decoder with quantized, bias-free linears
 * (the quant counterpart of DecoderBlock with its GqaAttention and SwiGluFfn,
 * crates/vokra-models/src/voxtral/text_decoder.rs:82-107, which hold
 * transposed f32 weights); wire-format weights [out, in]. */
typedef struct vokra_hip_text_decoder_layer {
    const float *attn_norm_gamma;          /* [d] */
    const uint8_t *wq, *wk, *wv, *wo;      /* [n_head_q*hd, d], [n_head_kv*hd, d] x 2, [d, n_head_q*hd] */
    const float *ffn_norm_gamma;           /* [d] */
    const uint8_t *w_gate, *w_up, *w_down; /* [ffn, d] x 2, [d, ffn] */
} vokra_hip_text_decoder_layer_t;

typedef struct vokra_hip_text_decoder vokra_hip_text_decoder_t;

/* Device-resident text decoder for n_stream concurrent streams. Replaces
 * voxtral::TextDecoderSession (crates/vokra-models/src/voxtral/
 * text_decoder_session.rs:54-330) with a batch axis and, instead of the
 * reference's f32 KvCache, the paged Q8_0 cache of vokra_hip_kv_* (n_head_kv
 * heads, block_size-token pages, n_ctx positions). Every linear is
 * gemm_q_f32 of wdtype (Q4_K: kquant_gemm_i8). lm_head: wire bytes [vocab, d]
 * of wdtype, or NULL for the tied f32 token embedding
 * (TextDecoder::output_head, text_decoder.rs:665). Config checks as TextDecoderSession::new
 * (0-sentinels and n_head_q % n_head_kv are MODEL_LOAD); head_dim 64 or 128
 * and 1, 2, 4 or 8 query heads per kv head (else UNSUPPORTED_OP). */
int vokra_hip_text_decoder_create(vokra_hip_ctx_t *ctx, int wdtype, size_t n_layer, size_t d_model,
                                  size_t n_head_q, size_t n_head_kv, size_t head_dim, size_t ffn_dim, size_t vocab,
                                  size_t n_ctx, size_t n_stream, size_t block_size, float rope_base,
                                  float rms_norm_eps, const vokra_hip_text_decoder_layer_t *layers,
                                  const float *token_emb, const float *final_norm_gamma, const uint8_t *lm_head,
                                  vokra_hip_text_decoder_t **out);
void vokra_hip_text_decoder_destroy(vokra_hip_text_decoder_t *dec);
/* TextDecoderSession::reset (text_decoder_session.rs:192): every stream back to position 0. */
int vokra_hip_text_decoder_reset(vokra_hip_ctx_t *ctx, vokra_hip_text_decoder_t *dec);
/* As vokra_hip_decoder_set_free_order / _kv_pages, for the text decoder's
 * cache (every stream back to position 0). No reference counterpart. */
int vokra_hip_text_decoder_set_free_order(vokra_hip_ctx_t *ctx, vokra_hip_text_decoder_t *dec, const int32_t *order,
                                          size_t n);
int vokra_hip_text_decoder_kv_pages(vokra_hip_ctx_t *ctx, vokra_hip_text_decoder_t *dec, size_t *free_pages,
                                    size_t *pages_in_use);
/* TextDecoderSession::position (text_decoder_session.rs:187) of one stream. */
int vokra_hip_text_decoder_position(vokra_hip_ctx_t *ctx, vokra_hip_text_decoder_t *dec, size_t stream,
                                    size_t *position);
/* TextDecoderSession::kv_restore (text_decoder_session.rs:390-405) for one
 * stream from rows instead of a snapshot: k_rows / v_rows [n_layer][n_pos]
 * [n_head_kv * head_dim] (K after RoPE, as the cache holds them) become the
 * stream's history and its position is set to n_pos. Host arrays, synchronous. */
int vokra_hip_text_decoder_kv_restore(vokra_hip_ctx_t *ctx, vokra_hip_text_decoder_t *dec, size_t stream,
                                      size_t n_pos, const float *k_rows, const float *v_rows);
/* TextDecoderSession::step_into (text_decoder_session.rs:207-240) with one
 * token for each of n distinct streams, at each stream's own position, then
 * greedy argmax into next_tokens[i]; logits [n, vocab] when not NULL. Host
 * arrays, synchronous; forward_step's rejections (token >= vocab, position
 * beyond n_ctx; text_decoder.rs:1007-1045). */
int vokra_hip_text_decoder_step(vokra_hip_ctx_t *ctx, vokra_hip_text_decoder_t *dec, size_t n,
                                const int32_t *streams, const int32_t *tokens, int32_t *next_tokens, float *logits);
/* Device arrays, asynchronous; positions[i] is stream i's position, which the
 * caller tracks (these calls do not move the host clocks of the host variant:
 * drive a session through one of the two). vokra_hip_text_decoder_status
 * reports the step's page allocation and the attention range check. */
int vokra_hip_text_decoder_step_dev(vokra_hip_ctx_t *ctx, vokra_hip_text_decoder_t *dec, size_t n,
                                    const int32_t *d_streams, const int32_t *d_tokens, const int32_t *d_positions,
                                    int32_t *d_next_tokens, float *d_logits);
int vokra_hip_text_decoder_status(vokra_hip_ctx_t *ctx, vokra_hip_text_decoder_t *dec, size_t *n_appended);

/* VoxtralConfig (crates/vokra-models/src/voxtral/config.rs:60-147), the
 * numeric fields. head_dim is the explicit metadata value (0 when the key is
 * absent: TextDecoderConfig::head_dim then derives hidden_dim / n_head_q);
 * rope_base, rms_norm_eps and the optional counts read 0 when absent. */
typedef struct vokra_hip_voxtral_config {
    size_t audio_n_layer, audio_n_head, audio_hidden_dim, audio_n_ctx, audio_n_mels, audio_ffn_dim;
    size_t n_layer, n_head_q, n_head_kv, head_dim, hidden_dim, ffn_dim, vocab_size, n_ctx;
    float rope_base, rms_norm_eps;
    size_t cross_attn_hidden_dim;
} vokra_hip_voxtral_config_t;
/* VoxtralConfig::from_gguf (config.rs:155-267): the vokra.voxtral.* keys,
 * required ones (audio_encoder.{n_layer, hidden_dim, n_head, n_mels},
 * text_decoder.{n_layer, hidden_dim, ffn_dim}) in the reference's order, the
 * head-split checks, MODEL_LOAD "voxtral config: ..." on failure. The mode
 * and codec strings are not read (no compute depends on them). */
int vokra_hip_voxtral_config_from_gguf(const vokra_hip_gguf_t *f, vokra_hip_voxtral_config_t *cfg);
/* TextDecoder::load (crates/vokra-models/src/voxtral/text_decoder.rs:484-575)
 * straight into a text-decoder session (vokra_hip_text_decoder_create): the
 * tensor prefix chosen as pick_prefix (:1456-1471), each layer's
 * input_layernorm, self_attn.{q,k,v,o}_proj, post_attention_layernorm and
 * mlp.{gate,up,down}_proj, the final norm and, when present, the untied
 * lm_head beside the decoder submodule (:763-768), checked in that order with
 * the reference's messages ("voxtral text_decoder: `<name>` missing from GGUF",
 * "... shape [..] != expected [..]"). Norms and the embedding widen to f32
 * (F32, F16 or Q4_K on disk). A Linear already in wdtype is taken from the
 * mapping (Q4_K: in_features a multiple of 256), an F32/F16 one is packed to
 * Q8_0 / Q4_0 / Q5_0 at load, anything else is UNSUPPORTED_OP naming it (the
 * reference widens every Linear to f32 instead). n_ctx = 0 takes the file's
 * text_decoder.n_ctx. report may be NULL. */
int vokra_hip_text_decoder_from_gguf(vokra_hip_ctx_t *ctx, const vokra_hip_gguf_t *f,
                                     const vokra_hip_voxtral_config_t *cfg, int wdtype, size_t n_stream, size_t n_ctx,
                                     size_t block_size, vokra_hip_whisper_load_report_t *report,
                                     vokra_hip_text_decoder_t **out);

#ifdef __cplusplus
}
#endif
#endif /* VOKRA_HIP_H */

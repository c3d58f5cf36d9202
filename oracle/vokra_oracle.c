/*
 * vokra_oracle.c — CPU restatement of the reference's hot-path arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY (parity checker and cpu_baseline). Never linked
 * into or called by the product library. Built with -O2 -ffp-contract=off so
 * no multiply-add is fused unless written as fmaf() explicitly.
 *
 * Reference paths are relative to the ayutaz/vokra repository root.
 */
#include "vokra_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* Rust `f32 as i32` / `as i8`: saturating, NaN -> 0. */
static int32_t sat_i32(float v) {
    if (isnan(v)) return 0;
    if (v >= 2147483647.0f) return INT32_MAX;
    if (v <= -2147483648.0f) return INT32_MIN;
    return (int32_t)v;
}

/* Rust f32::clamp(lo, hi): NaN passes through. */
static float clampf_rs(float x, float lo, float hi) {
    if (x < lo) x = lo;
    if (x > hi) x = hi;
    return x;
}

/* ========================================================================
 * binary16 (A1)
 * ====================================================================== */

/* crates/vokra-core/src/kv_quant/half.rs:53-69 */
float vo_f16_bits_to_f32(uint16_t h) {
    uint32_t sign = (h >> 15) & 1u;
    uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t mant = h & 0x3ffu;
    float sign_f = sign ? -1.0f : 1.0f;
    if (exp == 0) return sign_f * (float)mant * ldexpf(1.0f, -24);
    if (exp == 0x1f) return mant == 0 ? sign_f * INFINITY : NAN;
    return sign_f * (1.0f + (float)mant / 1024.0f) * ldexpf(1.0f, (int)exp - 15);
}

/* crates/vokra-core/src/kv_quant/half.rs:80-151 */
uint16_t vo_f32_to_f16_bits(float x) {
    uint32_t bits;
    memcpy(&bits, &x, 4);
    uint16_t sign = (uint16_t)((bits >> 31) & 1u);
    int32_t exp_f32 = (int32_t)((bits >> 23) & 0xffu);
    uint32_t mant_f32 = bits & 0x007fffffu;
    if (exp_f32 == 0xff) {
        if (mant_f32 == 0) return (uint16_t)((sign << 15) | (0x1f << 10));
        return (uint16_t)((sign << 15) | (0x1f << 10) | 0x200);
    }
    if (exp_f32 == 0 && mant_f32 == 0) return (uint16_t)(sign << 15);
    int32_t f16_exp = exp_f32 - 127 + 15;
    if (f16_exp >= 0x1f) return (uint16_t)((sign << 15) | (0x1f << 10));
    if (f16_exp >= 1) {
        const uint32_t shift = 13;
        uint32_t round_bit = (mant_f32 >> (shift - 1)) & 1u;
        int sticky = (mant_f32 & ((1u << (shift - 1)) - 1u)) != 0;
        uint32_t truncated = mant_f32 >> shift;
        int round_up = round_bit == 1 && (sticky || (truncated & 1u) == 1);
        uint32_t rounded = truncated + (round_up ? 1u : 0u);
        uint32_t e = (uint32_t)f16_exp;
        if (rounded == 0x400) {
            rounded = 0;
            e += 1;
            if (e >= 0x1f) return (uint16_t)((sign << 15) | (0x1f << 10));
        }
        return (uint16_t)((sign << 15) | (e << 10) | (rounded & 0x3ffu));
    }
    if (f16_exp < -10) return (uint16_t)(sign << 15);
    uint32_t mant_with_implicit = mant_f32 | 0x00800000u;
    uint32_t shift = (uint32_t)(1 - f16_exp) + 13u;
    uint32_t round_bit = (mant_with_implicit >> (shift - 1)) & 1u;
    int sticky = (mant_with_implicit & ((1u << (shift - 1)) - 1u)) != 0;
    uint32_t truncated = mant_with_implicit >> shift;
    int round_up = round_bit == 1 && (sticky || (truncated & 1u) == 1);
    uint32_t rounded = truncated + (round_up ? 1u : 0u);
    if (rounded >= 0x400) return (uint16_t)((sign << 15) | (1u << 10));
    return (uint16_t)((sign << 15) | (rounded & 0x3ffu));
}

/* crates/vokra-core/src/gguf/quant/mod.rs:92-125 (exp2i-based twin decoder;
 * every power of two it builds is exact, so it equals vo_f16_bits_to_f32). */
static float exp2i(int n) {
    uint32_t b = (uint32_t)(n + 127) << 23;
    float f;
    memcpy(&f, &b, 4);
    return f;
}
float vo_gguf_f16_to_f32(uint16_t h) {
    uint32_t sign = (h >> 15) & 1u;
    uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t mant = h & 0x3ffu;
    float sign_f = sign ? -1.0f : 1.0f;
    if (exp == 0) return sign_f * (float)mant * exp2i(-24);
    if (exp == 0x1f) return mant == 0 ? sign_f * INFINITY : NAN;
    return sign_f * (1.0f + (float)mant / 1024.0f) * exp2i((int)exp - 15);
}

/* crates/vokra-convert/src/quantize.rs:225-270 (converter's own encoder). */
uint16_t vo_convert_f32_to_f16(float value) {
    uint32_t x;
    memcpy(&x, &value, 4);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    int32_t aexp = (int32_t)((x >> 23) & 0xffu);
    uint32_t mant = x & 0x007fffffu;
    if (aexp == 0xff) return mant == 0 ? (uint16_t)(sign | 0x7c00) : (uint16_t)(sign | 0x7e00);
    int32_t e = aexp - 127 + 15;
    if (e >= 0x1f) return (uint16_t)(sign | 0x7c00);
    if (e <= 0) {
        if (e < -10) return sign;
        uint32_t m = mant | 0x00800000u;
        uint32_t shift = (uint32_t)(14 - e);
        uint16_t h = (uint16_t)(m >> shift);
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (h & 1u) == 1)) h += 1;
        return (uint16_t)(sign | h);
    }
    uint16_t h = (uint16_t)(((uint32_t)e << 10) | (mant >> 13));
    uint32_t rem = mant & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u) == 1)) h += 1;
    return (uint16_t)(sign | h);
}

/* ========================================================================
 * Q_0 block codecs (A2..A5)
 * ====================================================================== */

/* crates/vokra-core/src/kv_quant/mod.rs:101-110 (KvQuant::block_bytes). */
size_t vo_kv_block_bytes(int mode) {
    switch (mode) {
    case VO_KV_FP32: return 128;
    case VO_KV_Q4_0: return 18;
    case VO_KV_Q5_0: return 22;
    case VO_KV_Q8_0: return 34;
    default: return 0;
    }
}

/* fold(0.0, |acc, x| acc.max(x.abs())) */
static float amax32(const float *in, size_t n) {
    float a = 0.0f;
    for (size_t i = 0; i < n; ++i) a = fmaxf(a, fabsf(in[i]));
    return a;
}

/* q4_0.rs:100-105 quantize_nibble: clamp, round, +8, clamp 0..15 */
static uint8_t quantize_nibble(float scaled) {
    float c = clampf_rs(scaled, -8.0f, 7.0f);
    int32_t r = sat_i32(roundf(c));
    int32_t b = r + 8;
    if (b < 0) b = 0;
    if (b > 15) b = 15;
    return (uint8_t)b;
}

/* q5_0.rs quantize_5bit_biased */
static uint8_t quantize_5bit_biased(float scaled) {
    float c = clampf_rs(scaled, -16.0f, 15.0f);
    int32_t r = sat_i32(roundf(c));
    int32_t b = r + 16;
    if (b < 0) b = 0;
    if (b > 31) b = 31;
    return (uint8_t)b;
}

static void put_u16(uint8_t *p, uint16_t v) {
    p[0] = (uint8_t)(v & 0xff);
    p[1] = (uint8_t)(v >> 8);
}
static uint16_t get_u16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* Wire layouts: Q8_0 q8_0.rs:26-33 + mod.rs:470-477; Q4_0 q4_0.rs:29-36 +
 * mod.rs:456-461; Q5_0 q5_0.rs + mod.rs:463-468.  Packers: q8_0.rs:40-64,
 * q4_0.rs:44-68, q5_0.rs pack. */
void vo_pack_block(int mode, const float *in, uint8_t *out) {
    float amax = amax32(in, 32);
    if (mode == VO_KV_Q8_0) {
        float d = amax == 0.0f ? 0.0f : amax / 127.0f;
        float inv_d = d == 0.0f ? 0.0f : 1.0f / d;
        put_u16(out, vo_f32_to_f16_bits(d));
        for (int i = 0; i < 32; ++i) {
            float c = clampf_rs(in[i] * inv_d, -127.0f, 127.0f);
            int32_t r = sat_i32(roundf(c));
            if (r > 127) r = 127;
            if (r < -128) r = -128;
            out[2 + i] = (uint8_t)(int8_t)r;
        }
    } else if (mode == VO_KV_Q4_0) {
        float d = amax == 0.0f ? 0.0f : amax / 7.0f;
        float inv_d = d == 0.0f ? 0.0f : 1.0f / d;
        put_u16(out, vo_f32_to_f16_bits(d));
        for (int i = 0; i < 16; ++i) {
            uint8_t q0 = quantize_nibble(in[2 * i] * inv_d);
            uint8_t q1 = quantize_nibble(in[2 * i + 1] * inv_d);
            out[2 + i] = (uint8_t)((q0 & 0x0f) | ((q1 & 0x0f) << 4));
        }
    } else if (mode == VO_KV_Q5_0) {
        float d = amax == 0.0f ? 0.0f : amax / 15.0f;
        float inv_d = d == 0.0f ? 0.0f : 1.0f / d;
        uint8_t qh[4] = {0, 0, 0, 0};
        uint8_t qs[16];
        memset(qs, 0, sizeof qs);
        for (int i = 0; i < 32; ++i) {
            uint8_t biased = quantize_5bit_biased(in[i] * inv_d);
            uint8_t lo4 = biased & 0x0f;
            uint8_t hi1 = (biased >> 4) & 1;
            if (i % 2 == 0) qs[i / 2] |= lo4;
            else qs[i / 2] |= (uint8_t)(lo4 << 4);
            qh[i / 8] |= (uint8_t)(hi1 << (i % 8));
        }
        put_u16(out, vo_f32_to_f16_bits(d));
        memcpy(out + 2, qh, 4);
        memcpy(out + 6, qs, 16);
    }
}

/* Unpackers: q8_0.rs:69-80, q4_0.rs:73-87, q5_0.rs unpack. */
void vo_unpack_block(int mode, const uint8_t *blk, float *out) {
    float d = vo_f16_bits_to_f32(get_u16(blk));
    if (mode == VO_KV_Q8_0) {
        for (int i = 0; i < 32; ++i) out[i] = (float)(int8_t)blk[2 + i] * d;
    } else if (mode == VO_KV_Q4_0) {
        for (int i = 0; i < 16; ++i) {
            int32_t lo = (int32_t)(blk[2 + i] & 0x0f) - 8;
            int32_t hi = (int32_t)((blk[2 + i] >> 4) & 0x0f) - 8;
            out[2 * i] = (float)lo * d;
            out[2 * i + 1] = (float)hi * d;
        }
    } else if (mode == VO_KV_Q5_0) {
        const uint8_t *qh = blk + 2, *qs = blk + 6;
        for (int i = 0; i < 32; ++i) {
            uint32_t lo4 = (i % 2 == 0) ? (qs[i / 2] & 0x0fu) : ((qs[i / 2] >> 4) & 0x0fu);
            uint32_t hi1 = (qh[i / 8] >> (i % 8)) & 1u;
            int32_t sv = (int32_t)((hi1 << 4) | lo4) - 16;
            out[i] = (float)sv * d;
        }
    }
}

/* crates/vokra-core/src/kv_quant/mod.rs:307-359 (dequantize_bytes[_into]). */
int vo_dequantize_bytes(int mode, const uint8_t *bytes, size_t n_bytes, float *out, size_t out_len) {
    if (mode == VO_KV_FP32) return VO_INVALID_ARGUMENT;
    size_t bb = vo_kv_block_bytes(mode);
    if (bb == 0 || n_bytes % bb != 0) return VO_INVALID_ARGUMENT;
    size_t nb = n_bytes / bb;
    if (out_len != nb * 32) return VO_INVALID_ARGUMENT;
    for (size_t b = 0; b < nb; ++b) vo_unpack_block(mode, bytes + b * bb, out + b * 32);
    return VO_OK;
}

/* crates/vokra-core/src/kv_quant/dequant_gemm.rs:137-186 */
int vo_pack_matrix_to_bytes(int mode, const float *a, size_t n_rows, size_t n_bpr, uint8_t *out) {
    if (mode == VO_KV_FP32) return VO_INVALID_ARGUMENT;
    size_t bb = vo_kv_block_bytes(mode);
    if (bb == 0) return VO_INVALID_ARGUMENT;
    for (size_t r = 0; r < n_rows; ++r)
        for (size_t b = 0; b < n_bpr; ++b)
            vo_pack_block(mode, a + r * n_bpr * 32 + b * 32, out + (r * n_bpr + b) * bb);
    return VO_OK;
}

/* ========================================================================
 * dequant GEMV (A6, A7)
 * ====================================================================== */

/* crates/vokra-core/src/kv_quant/gpu_ops.rs:95-131 */
int vo_validate_dequant_gemv(int mode, size_t n_bytes, size_t n_rows, size_t n_bpr, size_t x_len) {
    if (mode == VO_KV_FP32) return VO_INVALID_ARGUMENT;
    size_t bb = vo_kv_block_bytes(mode);
    if (bb == 0) return VO_INVALID_ARGUMENT;
    if (x_len != n_bpr * 32) return VO_INVALID_ARGUMENT;
    if (n_bpr != 0 && n_rows > SIZE_MAX / n_bpr) return VO_INVALID_ARGUMENT;
    size_t rb = n_rows * n_bpr;
    if (rb != 0 && bb > SIZE_MAX / rb) return VO_INVALID_ARGUMENT;
    if (n_bytes != rb * bb) return VO_INVALID_ARGUMENT;
    return VO_OK;
}

/* crates/vokra-core/src/kv_quant/dequant_gemm.rs:49-98: dequantize the row to
 * f32, then a sequential `.map(a*b).sum()` fold (neutral -0.0). */
int vo_dequant_gemv_scalar(int mode, const uint8_t *bytes, size_t n_bytes, size_t n_rows,
                           size_t n_bpr, const float *x, size_t x_len, float *y) {
    int st = vo_validate_dequant_gemv(mode, n_bytes, n_rows, n_bpr, x_len);
    if (st) return st;
    size_t bb = vo_kv_block_bytes(mode);
    size_t per_row = n_bpr * 32;
    float *row = (float *)malloc((per_row ? per_row : 1) * sizeof(float));
    if (!row) return VO_BACKEND_UNAVAILABLE;
    for (size_t r = 0; r < n_rows; ++r) {
        for (size_t b = 0; b < n_bpr; ++b)
            vo_unpack_block(mode, bytes + (r * n_bpr + b) * bb, row + b * 32);
        float acc = -0.0f;
        for (size_t i = 0; i < per_row; ++i) acc = acc + row[i] * x[i];
        y[r] = acc;
    }
    free(row);
    return VO_OK;
}

/* crates/vokra-core/src/kv_quant/dequant_gemm.rs:108-127 */
void vo_dense_gemv_f32(const float *a, size_t n_rows, const float *x, size_t x_len, float *y) {
    for (size_t r = 0; r < n_rows; ++r) {
        float acc = 0.0f;
        for (size_t i = 0; i < x_len; ++i) acc += a[r * x_len + i] * x[i];
        y[r] = acc;
    }
}

/* ========================================================================
 * Block-format INT8 GEMM (Q8_0 / Q4_0 / Q5_0 weights behind gemm_q_f32).
 *
 * The reference has no GPU or INT8 route for these formats (its gemm_q_f32
 * covers K-quants only: kernels/mod.rs:341-364, kquant.rs:56-63). This build
 * extends the seam with the K-quant INT8 convention at the formats' native
 * 32-element block:
 *   activations: per 32-element block, s = amax/127, q = round(v/s) clamped
 *                to +-127 (kquant.rs:418-441 with group 32 instead of 16);
 *   weights:     the exact integers of the wire block (Q8_0 q, Q4_0 nib-8,
 *                Q5_0 v-16) and the f32 value of the f16 scale;
 *   dot:         isum = sum of 32 int8*int8 products (exact i32);
 *   combine:     acc = fmaf(s_act * d_w, (float)isum, acc), blocks in order,
 *                acc starting at +0.0; bias added after (gemm_driver.rs:326-330).
 * ====================================================================== */

/* pow2 != 0 selects the shared-exponent convention: s = the smallest power
 * of two >= amax/127 (frexpf: amax/127 = f * 2^ex, f in [0.5, 1)). */
void vo_quantize_act_b32_mode(const float *x, size_t k, int8_t *q, float *scale, int32_t *gsum, int pow2) {
    size_t nb = k / 32;
    for (size_t b = 0; b < nb; ++b) {
        const float *xs = x + b * 32;
        float amax = amax32(xs, 32);
        int32_t g = 0;
        if (amax == 0.0f) {
            memset(q + b * 32, 0, 32);
            scale[b] = 0.0f;
            gsum[b] = 0;
            continue;
        }
        float s = amax / 127.0f;
        if (pow2) {
            int ex;
            float f = frexpf(s, &ex);
            s = ldexpf(1.0f, f == 0.5f ? ex - 1 : ex);
        }
        for (int t = 0; t < 32; ++t) {
            float r = clampf_rs(roundf(xs[t] / s), -127.0f, 127.0f);
            int32_t ri = sat_i32(r);
            q[b * 32 + t] = (int8_t)ri;
            g += ri;
        }
        scale[b] = s;
        gsum[b] = g;
    }
}

void vo_quantize_act_b32(const float *x, size_t k, int8_t *q, float *scale, int32_t *gsum) {
    vo_quantize_act_b32_mode(x, k, q, scale, gsum, 0);
}

static int wdtype_block_bytes(int wd) {
    switch (wd) {
    case VO_W_Q4_0: return 18;
    case VO_W_Q5_0: return 22;
    case VO_W_Q8_0: return 34;
    case VO_W_Q4_K: return 144;
    default: return 0;
    }
}

int vo_qblock_weight_ints(int wd, const uint8_t *blk, int8_t *q32, float *d) {
    *d = vo_f16_bits_to_f32(get_u16(blk));
    if (wd == VO_W_Q8_0) {
        for (int i = 0; i < 32; ++i) q32[i] = (int8_t)blk[2 + i];
    } else if (wd == VO_W_Q4_0) {
        for (int i = 0; i < 16; ++i) {
            q32[2 * i] = (int8_t)((blk[2 + i] & 0x0f) - 8);
            q32[2 * i + 1] = (int8_t)(((blk[2 + i] >> 4) & 0x0f) - 8);
        }
    } else if (wd == VO_W_Q5_0) {
        const uint8_t *qh = blk + 2, *qs = blk + 6;
        for (int i = 0; i < 32; ++i) {
            uint32_t lo4 = (i % 2 == 0) ? (qs[i / 2] & 0x0fu) : ((qs[i / 2] >> 4) & 0x0fu);
            uint32_t hi1 = (qh[i / 8] >> (i % 8)) & 1u;
            q32[i] = (int8_t)((int32_t)((hi1 << 4) | lo4) - 16);
        }
    } else {
        return VO_INVALID_ARGUMENT;
    }
    return VO_OK;
}

static int qblock_check(int wd, size_t m, size_t n, size_t k) {
    (void)m;
    (void)n;
    if (wd != VO_W_Q4_0 && wd != VO_W_Q5_0 && wd != VO_W_Q8_0) return VO_INVALID_ARGUMENT;
    if (k == 0 || k % 32 != 0) return VO_INVALID_ARGUMENT;
    return VO_OK;
}

int vo_qblock_block_dots_mode(int wd, size_t m, size_t n, size_t k, const float *a, const uint8_t *wq,
                              int32_t *dots, int pow2) {
    int st = qblock_check(wd, m, n, k);
    if (st) return st;
    size_t nb = k / 32, bb = (size_t)wdtype_block_bytes(wd);
    int8_t *qa = (int8_t *)malloc(k);
    float *sa = (float *)malloc(nb * sizeof(float));
    int32_t *ga = (int32_t *)malloc(nb * sizeof(int32_t));
    int8_t qw[32];
    float dw;
    for (size_t i = 0; i < m; ++i) {
        vo_quantize_act_b32_mode(a + i * k, k, qa, sa, ga, pow2);
        for (size_t j = 0; j < n; ++j)
            for (size_t b = 0; b < nb; ++b) {
                vo_qblock_weight_ints(wd, wq + (j * nb + b) * bb, qw, &dw);
                int32_t s = 0;
                for (int t = 0; t < 32; ++t) s += (int32_t)qw[t] * (int32_t)qa[b * 32 + t];
                dots[(i * n + j) * nb + b] = s;
            }
    }
    free(qa);
    free(sa);
    free(ga);
    return VO_OK;
}

int vo_qblock_block_dots(int wd, size_t m, size_t n, size_t k, const float *a, const uint8_t *wq,
                         int32_t *dots) {
    return vo_qblock_block_dots_mode(wd, m, n, k, a, wq, dots, 0);
}

int vo_gemm_qblock_i8_mode(int wd, size_t m, size_t n, size_t k, const float *a, const uint8_t *wq,
                           size_t wq_len, const float *bias, float *out, int pow2) {
    int st = qblock_check(wd, m, n, k);
    if (st) return st;
    size_t nb = k / 32, bb = (size_t)wdtype_block_bytes(wd);
    if (wq_len != n * nb * bb) return VO_INVALID_ARGUMENT;
    /* Unpack the weight once: integers + f32 scales per block. */
    int8_t *qw = (int8_t *)malloc(n * k);
    float *dw = (float *)malloc(n * nb * sizeof(float));
    int8_t *qa = (int8_t *)malloc(k);
    float *sa = (float *)malloc(nb * sizeof(float));
    int32_t *ga = (int32_t *)malloc(nb * sizeof(int32_t));
    if (!qw || !dw || !qa || !sa || !ga) {
        free(qw); free(dw); free(qa); free(sa); free(ga);
        return VO_BACKEND_UNAVAILABLE;
    }
    for (size_t j = 0; j < n; ++j)
        for (size_t b = 0; b < nb; ++b)
            vo_qblock_weight_ints(wd, wq + (j * nb + b) * bb, qw + j * k + b * 32, dw + j * nb + b);
    for (size_t i = 0; i < m; ++i) {
        vo_quantize_act_b32_mode(a + i * k, k, qa, sa, ga, pow2);
        for (size_t j = 0; j < n; ++j) {
            const int8_t *wr = qw + j * k;
            float acc = 0.0f;
            for (size_t b = 0; b < nb; ++b) {
                int32_t s = 0;
                for (int t = 0; t < 32; ++t) s += (int32_t)wr[b * 32 + t] * (int32_t)qa[b * 32 + t];
                acc = fmaf(sa[b] * dw[j * nb + b], (float)s, acc);
            }
            out[i * n + j] = acc;
        }
        if (bias)
            for (size_t j = 0; j < n; ++j) out[i * n + j] += bias[j];
    }
    free(qw); free(dw); free(qa); free(sa); free(ga);
    return VO_OK;
}

int vo_gemm_qblock_i8(int wd, size_t m, size_t n, size_t k, const float *a, const uint8_t *wq,
                      size_t wq_len, const float *bias, float *out) {
    return vo_gemm_qblock_i8_mode(wd, m, n, k, a, wq, wq_len, bias, out, 0);
}

/* Activation-rounding bound for one output of the block INT8 GEMM, the
 * analogue of kquant.rs:471-495 at group 32: sum_b (s_b / 2) * sum |w|. */
float vo_qblock_error_bound(int wd, const uint8_t *w_row, const float *x, size_t k) {
    size_t nb = k / 32, bb = (size_t)wdtype_block_bytes(wd);
    float bound = 0.0f;
    int8_t qw[32];
    float dw;
    for (size_t b = 0; b < nb; ++b) {
        vo_qblock_weight_ints(wd, w_row + b * bb, qw, &dw);
        float s = amax32(x + b * 32, 32) / 127.0f;
        float wsum = -0.0f;
        for (int t = 0; t < 32; ++t) wsum = wsum + fabsf((float)qw[t] * dw);
        bound += 0.5f * s * wsum;
    }
    return bound;
}

/* ========================================================================
 * K-quants (A8..A10)
 * ====================================================================== */

/* crates/vokra-core/src/gguf/quant/mod.rs:140-149 */
static void get_scale_min_k4(int j, const uint8_t *s, uint8_t *d, uint8_t *m) {
    if (j < 4) {
        *d = s[j] & 63;
        *m = s[j + 4] & 63;
    } else {
        *d = (uint8_t)((s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4));
        *m = (uint8_t)((s[j + 4] >> 4) | ((s[j] >> 6) << 4));
    }
}

/* Super-block bytes of a K-quant dtype (gguf/tensor.rs:117-125), 0 if none. */
static size_t kq_block_bytes(int wd) {
    return wd == VO_W_Q4_K ? 144 : wd == VO_W_Q5_K ? 176 : wd == VO_W_Q6_K ? 210 : 0;
}

/* crates/vokra-core/src/gguf/quant/q4_k.rs:34-69 */
static void dequant_q4k_block(const uint8_t *blk, float *y) {
    float d = vo_gguf_f16_to_f32(get_u16(blk));
    float dmin = vo_gguf_f16_to_f32(get_u16(blk + 2));
    const uint8_t *scales = blk + 4, *qs = blk + 16;
    int is = 0;
    size_t q = 0, base = 0;
    while (base < 256) {
        uint8_t sc0, m0, sc1, m1s;
        get_scale_min_k4(is, scales, &sc0, &m0);
        float d1 = d * (float)sc0, m1 = dmin * (float)m0;
        get_scale_min_k4(is + 1, scales, &sc1, &m1s);
        float d2 = d * (float)sc1, m2 = dmin * (float)m1s;
        for (int l = 0; l < 32; ++l) y[base + l] = d1 * (float)(qs[q + l] & 0xF) - m1;
        for (int l = 0; l < 32; ++l) y[base + 32 + l] = d2 * (float)(qs[q + l] >> 4) - m2;
        q += 32;
        is += 2;
        base += 64;
    }
}

/* crates/vokra-core/src/gguf/quant/q5_k.rs:36-80: Q4_K's sub-scales, each
 * quant gaining a 5th bit from qh (chunk k: low 32 take bit 2k, high 32 bit
 * 2k + 1). */
static void dequant_q5k_block(const uint8_t *blk, float *y) {
    float d = vo_gguf_f16_to_f32(get_u16(blk));
    float dmin = vo_gguf_f16_to_f32(get_u16(blk + 2));
    const uint8_t *scales = blk + 4, *qh = blk + 16, *qs = blk + 48;
    int is = 0;
    size_t ql = 0, base = 0;
    uint8_t u1 = 1, u2 = 2;
    while (base < 256) {
        uint8_t sc0, m0, sc1, m1s;
        get_scale_min_k4(is, scales, &sc0, &m0);
        float d1 = d * (float)sc0, m1 = dmin * (float)m0;
        get_scale_min_k4(is + 1, scales, &sc1, &m1s);
        float d2 = d * (float)sc1, m2 = dmin * (float)m1s;
        for (int l = 0; l < 32; ++l) {
            unsigned q = (qs[ql + l] & 0xFu) + ((qh[l] & u1) ? 16u : 0u);
            y[base + l] = d1 * (float)q - m1;
        }
        for (int l = 0; l < 32; ++l) {
            unsigned q = (unsigned)(qs[ql + l] >> 4) + ((qh[l] & u2) ? 16u : 0u);
            y[base + 32 + l] = d2 * (float)q - m2;
        }
        ql += 32;
        is += 2;
        u1 = (uint8_t)(u1 << 2);
        u2 = (uint8_t)(u2 << 2);
        base += 64;
    }
}

/* crates/vokra-core/src/gguf/quant/q6_k.rs:34-72: y = d * sc (int8) * q with
 * q = (4 low bits | 2 high bits << 4) - 32, in that association. */
static void dequant_q6k_block(const uint8_t *blk, float *out) {
    float d = vo_gguf_f16_to_f32(get_u16(blk + 208));
    for (int half = 0; half < 2; ++half) {
        const uint8_t *ql = blk + 64 * half, *qh = blk + 128 + 32 * half, *sc = blk + 192 + 8 * half;
        float *y = out + 128 * half;
        for (int l = 0; l < 32; ++l) {
            int is = l / 16;
            int q1 = (int)((ql[l] & 0xF) | ((qh[l] & 3) << 4)) - 32;
            int q2 = (int)((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
            int q3 = (int)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
            int q4 = (int)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
            y[l] = d * (float)(int8_t)sc[is] * (float)q1;
            y[l + 32] = d * (float)(int8_t)sc[is + 2] * (float)q2;
            y[l + 64] = d * (float)(int8_t)sc[is + 4] * (float)q3;
            y[l + 96] = d * (float)(int8_t)sc[is + 6] * (float)q4;
        }
    }
}

/* crates/vokra-core/src/gguf/quant/mod.rs:42-63 dequantize, K-quant arms */
int vo_kquant_dequantize(int wd, const uint8_t *bytes, size_t n_bytes, size_t n_elements, float *out) {
    size_t bb = kq_block_bytes(wd);
    if (!bb) return VO_UNSUPPORTED_OP;
    if (n_elements % 256 != 0) return VO_INVALID_ARGUMENT;
    size_t nb = n_elements / 256;
    if (n_bytes != nb * bb) return VO_INVALID_ARGUMENT;
    for (size_t i = 0; i < nb; ++i) {
        if (wd == VO_W_Q4_K) dequant_q4k_block(bytes + i * bb, out + i * 256);
        else if (wd == VO_W_Q5_K) dequant_q5k_block(bytes + i * bb, out + i * 256);
        else dequant_q6k_block(bytes + i * bb, out + i * 256);
    }
    return VO_OK;
}

/* crates/vokra-convert/src/quantize.rs:84-142 (affine_quants + quantize_q4_k) */
int vo_kquant_quantize(int wd, const float *data, size_t n, uint8_t *out) {
    if (wd != VO_W_Q4_K) return VO_UNSUPPORTED_OP;
    if (n % 256 != 0) return VO_INVALID_ARGUMENT;
    for (size_t bi = 0; bi < n / 256; ++bi) {
        const float *block = data + bi * 256;
        float lo = block[0], hi = block[0];
        for (int i = 1; i < 256; ++i) {
            if (block[i] < lo) lo = block[i];
            if (block[i] > hi) hi = block[i];
        }
        float base = fminf(lo, 0.0f);
        float range = hi - base;
        float step = range / 15.0f;
        float d = step > 0.0f ? step / 63.0f : 0.0f;
        float dmin = base < 0.0f ? -base / 63.0f : 0.0f;
        uint8_t q[256];
        for (int i = 0; i < 256; ++i) {
            if (step > 0.0f) {
                float r = clampf_rs(roundf((block[i] - base) / step), 0.0f, 15.0f);
                int32_t ri = sat_i32(r);
                if (ri < 0) ri = 0;
                if (ri > 255) ri = 255;
                q[i] = (uint8_t)ri;
            } else {
                q[i] = 0;
            }
        }
        uint8_t *o = out + bi * 144;
        put_u16(o, vo_convert_f32_to_f16(d));
        put_u16(o + 2, vo_convert_f32_to_f16(dmin));
        memset(o + 4, 0xFF, 12);
        for (int kk = 0; kk < 4; ++kk)
            for (int l = 0; l < 32; ++l)
                o[16 + 32 * kk + l] = (uint8_t)((q[64 * kk + l] & 0xF) | ((q[64 * kk + 32 + l] & 0xF) << 4));
    }
    return VO_OK;
}

/* crates/vokra-backend-cpu/src/kernels/kquant.rs:332-407 unpack_block_i8: the
 * format-independent y = d_eff * q - m_eff per 16-element group. Q4_K / Q5_K
 * take their sub-scales through q45_sub_scales (:290-302; one (d, m) pair per
 * 32 elements, so two identical groups) and Q5_K adds the qh bit; Q6_K keeps
 * the biased q6 + 32 in 0..63 with d_eff = d * sc (int8) per 16 elements in
 * q6_group_scales' order (:306-323) and m_eff = d_eff * 32 (exact). */
typedef struct {
    uint8_t q[256];
    float d_eff[16];
    float m_eff[16];
} unpacked_block;

static void unpack_block_i8(int wd, const uint8_t *block, unpacked_block *ub) {
    if (wd == VO_W_Q6_K) {
        float d = vo_gguf_f16_to_f32(get_u16(block + 208));
        const uint8_t *sc = block + 192;
        for (int half = 0; half < 2; ++half)
            for (int quarter = 0; quarter < 4; ++quarter)
                for (int sub = 0; sub < 2; ++sub) {
                    int g = (128 * half + 32 * quarter + 16 * sub) / 16;
                    int idx = 8 * half + sub + 2 * quarter;
                    ub->d_eff[g] = d * (float)(int8_t)sc[idx];
                }
        for (int g = 0; g < 16; ++g) ub->m_eff[g] = ub->d_eff[g] * 32.0f;
        for (int half = 0; half < 2; ++half) {
            const uint8_t *ql = block + 64 * half, *qh = block + 128 + 32 * half;
            uint8_t *y = ub->q + 128 * half;
            for (int l = 0; l < 32; ++l) {
                y[l] = (uint8_t)((ql[l] & 0xF) | ((qh[l] & 3) << 4));
                y[l + 32] = (uint8_t)((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4));
                y[l + 64] = (uint8_t)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4));
                y[l + 96] = (uint8_t)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4));
            }
        }
        return;
    }
    float d = vo_gguf_f16_to_f32(get_u16(block));
    float dmin = vo_gguf_f16_to_f32(get_u16(block + 2));
    const uint8_t *scales = block + 4;
    const uint8_t *qs = wd == VO_W_Q5_K ? block + 48 : block + 16;
    const uint8_t *qh = wd == VO_W_Q5_K ? block + 16 : NULL;
    for (int j = 0; j < 8; ++j) {
        uint8_t sc, mn;
        get_scale_min_k4(j, scales, &sc, &mn);
        float d1 = d * (float)sc, m1 = dmin * (float)mn;
        ub->d_eff[2 * j] = d1;
        ub->d_eff[2 * j + 1] = d1;
        ub->m_eff[2 * j] = m1;
        ub->m_eff[2 * j + 1] = m1;
        int chunk = j / 2, hi = j % 2;
        for (int t = 0; t < 32; ++t) {
            uint8_t byte = qs[32 * chunk + t];
            uint8_t q = hi ? (uint8_t)(byte >> 4) : (uint8_t)(byte & 0xF);
            if (qh && (qh[t] & (1u << j))) q = (uint8_t)(q + 16);
            ub->q[32 * j + t] = q;
        }
    }
}

/* kquant.rs:418-441 quantize_activations (group 16, divide, round then clamp) */
void vo_kquant_quantize_activations(const float *x, size_t k, int8_t *q, float *scales, int32_t *gsums) {
    size_t ng = k / 16;
    memset(q, 0, k);
    for (size_t g = 0; g < ng; ++g) {
        const float *xs = x + 16 * g;
        float amax = amax32(xs, 16);
        scales[g] = 0.0f;
        gsums[g] = 0;
        if (amax == 0.0f) continue;
        float s = amax / 127.0f;
        int32_t gsum = 0;
        for (int t = 0; t < 16; ++t) {
            float r = clampf_rs(roundf(xs[t] / s), -127.0f, 127.0f);
            int32_t ri = sat_i32(r);
            q[16 * g + t] = (int8_t)ri;
            gsum += ri;
        }
        scales[g] = s;
        gsums[g] = gsum;
    }
}

/* kquant.rs:542-578 validate_gemv_i8 */
static int validate_gemv_i8(int wd, size_t m, size_t k, size_t w_len, size_t x_len, size_t out_len,
                            size_t n_x) {
    size_t bb = kq_block_bytes(wd);
    if (!bb) return VO_UNSUPPORTED_OP;
    if (k == 0 || k % 256 != 0) return VO_INVALID_ARGUMENT;
    size_t row_bytes = (k / 256) * bb;
    if (w_len != m * row_bytes) return VO_INVALID_ARGUMENT;
    if (x_len != n_x * k) return VO_INVALID_ARGUMENT;
    if (out_len != n_x * m) return VO_INVALID_ARGUMENT;
    return VO_OK;
}

/* kquant.rs:590-629 kquant_gemv_i8_on (scalar group sums :453-463, combine :447-449) */
static void kquant_gemv_i8_core(int wd, size_t m, size_t k, const uint8_t *w, const float *x, float *out) {
    size_t nb = k / 256, bb = kq_block_bytes(wd);
    int8_t *q = (int8_t *)malloc(k);
    float *sc = (float *)malloc((k / 16) * sizeof(float));
    int32_t *gs = (int32_t *)malloc((k / 16) * sizeof(int32_t));
    vo_kquant_quantize_activations(x, k, q, sc, gs);
    unpacked_block ub;
    for (size_t i = 0; i < m; ++i) {
        const uint8_t *row = w + i * nb * bb;
        float acc = 0.0f;
        for (size_t blk = 0; blk < nb; ++blk) {
            unpack_block_i8(wd, row + blk * bb, &ub);
            for (int g = 0; g < 16; ++g) {
                int32_t isum = 0;
                for (int t = 0; t < 16; ++t)
                    isum += (int32_t)ub.q[16 * g + t] * (int32_t)q[blk * 256 + 16 * g + t];
                float s_act = sc[blk * 16 + g];
                int32_t asum = gs[blk * 16 + g];
                acc += s_act * (ub.d_eff[g] * (float)isum - ub.m_eff[g] * (float)asum);
            }
        }
        out[i] = acc;
    }
    free(q);
    free(sc);
    free(gs);
}

int vo_kquant_gemv_i8(int wd, size_t m, size_t k, const uint8_t *w, size_t w_len, const float *x,
                      size_t x_len, float *out, size_t out_len) {
    int st = validate_gemv_i8(wd, m, k, w_len, x_len, out_len, 1);
    if (st) return st;
    kquant_gemv_i8_core(wd, m, k, w, x, out);
    return VO_OK;
}

/* kquant.rs:845-935 kquant_gemm_i8_on: n_act single-vector GEMVs, each writing
 * a contiguous [m] output row (validate_batch :962-980 rejects n_act == 0). */
int vo_kquant_gemm_i8(int wd, size_t m, size_t k, size_t n_act, const uint8_t *w, size_t w_len,
                      const float *x, size_t x_len, float *out, size_t out_len) {
    if (n_act == 0) return VO_INVALID_ARGUMENT;
    int st = validate_gemv_i8(wd, m, k, w_len, x_len, out_len, n_act);
    if (st) return st;
    for (size_t c = 0; c < n_act; ++c) kquant_gemv_i8_core(wd, m, k, w, x + c * k, out + c * m);
    return VO_OK;
}

/* kquant.rs:471-495 int8_error_bound */
float vo_int8_error_bound(int wd, const uint8_t *w_row, const float *x, size_t k) {
    size_t nb = k / 256, bb = kq_block_bytes(wd);
    unpacked_block ub;
    float bound = 0.0f;
    if (!bb) return 0.0f;
    for (size_t blk = 0; blk < nb; ++blk) {
        unpack_block_i8(wd, w_row + blk * bb, &ub);
        for (int g = 0; g < 16; ++g) {
            float s = amax32(x + blk * 256 + 16 * g, 16) / 127.0f;
            float wsum = -0.0f;
            for (int t = 0; t < 16; ++t)
                wsum = wsum + fabsf(ub.d_eff[g] * (float)ub.q[16 * g + t] - ub.m_eff[g]);
            bound += 0.5f * s * wsum;
        }
    }
    return bound;
}

/* crates/vokra-backend-cpu/src/kernels/mod.rs:341-364 gemm_q_f32 + the
 * gemm_driver.rs:312-332 run_q bias pass, extended to the block formats. */
int vo_gemm_q_f32(int wd, size_t m, size_t n, size_t k, const float *a, size_t a_len,
                  const uint8_t *wq, size_t wq_len, const float *bias, float *out, size_t out_len) {
    if (a_len != m * k || out_len != m * n) return VO_INVALID_ARGUMENT;
    if (kq_block_bytes(wd)) {
        int st = vo_kquant_gemm_i8(wd, n, k, m, wq, wq_len, a, a_len, out, out_len);
        if (st) return st;
        if (bias)
            for (size_t i = 0; i < m; ++i)
                for (size_t j = 0; j < n; ++j) out[i * n + j] += bias[j];
        return VO_OK;
    }
    if (m == 0) return VO_INVALID_ARGUMENT;
    return vo_gemm_qblock_i8(wd, m, n, k, a, wq, wq_len, bias, out);
}

/* ========================================================================
 * f32 scalar kernels (A11, A12) — crates/vokra-backend-cpu/src/kernels/scalar.rs
 * ====================================================================== */

/* scalar.rs:41-72 */
void vo_gemm_f32(size_t m, size_t n, size_t k, const float *a, const float *b, const float *bias,
                 float *out) {
    for (size_t i = 0; i < m; ++i) {
        float *orow = out + i * n;
        for (size_t j = 0; j < n; ++j) orow[j] = bias ? bias[j] : 0.0f;
        for (size_t l = 0; l < k; ++l) {
            float ail = a[i * k + l];
            const float *brow = b + l * n;
            for (size_t j = 0; j < n; ++j) orow[j] += ail * brow[j];
        }
    }
}

/* Row-parallel split of vo_gemm_f32 over threads: each row is computed by the
 * identical scalar loop, so the result is bit-identical to one thread
 * (crates/vokra-backend-cpu/src/pool.rs:1-16 row-split contract). */
typedef struct {
    size_t r0, r1, n, k;
    const float *a, *b, *bias;
    float *out;
} gemm_job;
static void *gemm_worker(void *p) {
    gemm_job *j = (gemm_job *)p;
    vo_gemm_f32(j->r1 - j->r0, j->n, j->k, j->a + j->r0 * j->k, j->b, j->bias, j->out + j->r0 * j->n);
    return NULL;
}
void vo_gemm_f32_mt(size_t m, size_t n, size_t k, const float *a, const float *b, const float *bias,
                    float *out, int n_threads) {
    if (n_threads <= 1 || m < 2) {
        vo_gemm_f32(m, n, k, a, b, bias, out);
        return;
    }
    if ((size_t)n_threads > m) n_threads = (int)m;
    pthread_t th[256];
    gemm_job jobs[256];
    if (n_threads > 256) n_threads = 256;
    size_t per = (m + (size_t)n_threads - 1) / (size_t)n_threads;
    int used = 0;
    for (int t = 0; t < n_threads; ++t) {
        size_t r0 = (size_t)t * per, r1 = r0 + per;
        if (r0 >= m) break;
        if (r1 > m) r1 = m;
        jobs[t] = (gemm_job){r0, r1, n, k, a, b, bias, out};
        pthread_create(&th[t], NULL, gemm_worker, &jobs[t]);
        used++;
    }
    for (int t = 0; t < used; ++t) pthread_join(th[t], NULL);
}

/* scalar.rs:74-91 */
void vo_gemv_f32(size_t m, size_t k, const float *a, const float *x, const float *bias, float *out) {
    for (size_t i = 0; i < m; ++i) {
        float s = bias ? bias[i] : 0.0f;
        for (size_t l = 0; l < k; ++l) s += a[i * k + l] * x[l];
        out[i] = s;
    }
}

/* scalar.rs:177-199 */
void vo_softmax_f32(const float *in, float *out, size_t rows, size_t cols) {
    for (size_t r = 0; r < rows; ++r) {
        const float *ir = in + r * cols;
        float *orow = out + r * cols;
        float mx = -INFINITY;
        for (size_t c = 0; c < cols; ++c) mx = fmaxf(mx, ir[c]);
        float sum = 0.0f;
        for (size_t c = 0; c < cols; ++c) {
            float e = expf(ir[c] - mx);
            orow[c] = e;
            sum += e;
        }
        float inv = 1.0f / sum;
        for (size_t c = 0; c < cols; ++c) orow[c] *= inv;
    }
}

/* scalar.rs:201-222 (population variance; `.sum()` folds from -0.0) */
void vo_layer_norm_f32(const float *in, float *out, size_t rows, size_t cols, const float *gamma,
                       const float *beta, float eps) {
    float inv_cols = 1.0f / (float)cols;
    for (size_t r = 0; r < rows; ++r) {
        const float *ir = in + r * cols;
        float *orow = out + r * cols;
        float s = -0.0f;
        for (size_t c = 0; c < cols; ++c) s = s + ir[c];
        float mean = s * inv_cols;
        float v = -0.0f;
        for (size_t c = 0; c < cols; ++c) v = v + (ir[c] - mean) * (ir[c] - mean);
        float var = v * inv_cols;
        float inv_std = 1.0f / sqrtf(var + eps);
        for (size_t c = 0; c < cols; ++c) orow[c] = (ir[c] - mean) * inv_std * gamma[c] + beta[c];
    }
}

/* scalar.rs:126-172: Abramowitz & Stegun 7.1.26 erf and the exact GELU. */
float vo_erf_as(float x) {
    const float P = 0.3275911f, A1 = 0.254829592f, A2 = -0.284496736f, A3 = 1.421413741f,
                A4 = -1.453152027f, A5 = 1.061405429f;
    float sign = x < 0.0f ? -1.0f : 1.0f;
    float ax = fabsf(x);
    float t = 1.0f / (1.0f + P * ax);
    float poly = ((((A5 * t + A4) * t + A3) * t + A2) * t + A1) * t;
    float y = 1.0f - poly * expf(-ax * ax);
    return sign * y;
}
void vo_gelu_f32(const float *x, float *out, size_t n) {
    const float frac_1_sqrt_2 = 0.70710678118654752440f;
    for (size_t i = 0; i < n; ++i) out[i] = 0.5f * x[i] * (1.0f + vo_erf_as(x[i] * frac_1_sqrt_2));
}

/* crates/vokra-models/src/voxtral/text_decoder.rs:801-822 rms_norm */
void vo_rms_norm_f32(const float *x, const float *gamma, float eps, size_t rows, size_t d, float *out) {
    for (size_t i = 0; i < rows; ++i) {
        const float *row = x + i * d;
        float ss = -0.0f;
        for (size_t c = 0; c < d; ++c) ss = ss + row[c] * row[c];
        float inv = 1.0f / sqrtf(ss / (float)d + eps);
        for (size_t c = 0; c < d; ++c) out[i * d + c] = row[c] * inv * gamma[c];
    }
}

/* crates/vokra-models/src/voxtral/text_decoder.rs:858-891 rope_apply: one
 * head's x [seq_len, head_dim] in place; row i at position
 * position_offset + i rotates the pairs (j, j + head_dim/2) by the angle
 * m * theta_j, theta_j = rope_base^(-2j / head_dim), evaluated per element as
 * the reference does (powf, then the f32 product, then sinf / cosf). */
int vo_rope_apply(float *x, size_t x_len, size_t seq_len, size_t head_dim, float rope_base, size_t position_offset) {
    if (head_dim % 2 != 0) return VO_INVALID_ARGUMENT;
    if (x_len != seq_len * head_dim) return VO_INVALID_ARGUMENT;
    size_t half = head_dim / 2;
    for (size_t i = 0; i < seq_len; ++i) {
        float m = (float)(position_offset + i);
        float *row = x + i * head_dim;
        for (size_t j = 0; j < half; ++j) {
            float theta = powf(rope_base, -2.0f * (float)j / (float)head_dim);
            float angle = m * theta;
            float s = sinf(angle), c = cosf(angle);
            float a = row[j], b = row[j + half];
            row[j] = a * c - b * s;
            row[j + half] = a * s + b * c;
        }
    }
    return VO_OK;
}

/* text_decoder.rs:826-831 silu_inplace: x <- x * (1 / (1 + exp(-x))). */
void vo_silu_inplace(float *x, size_t n) {
    for (size_t i = 0; i < n; ++i) {
        float s = 1.0f / (1.0f + expf(-x[i]));
        x[i] = x[i] * s;
    }
}

/* text_decoder.rs:835-847 hadamard_inplace: a <- a * b; a length mismatch is
 * InvalidArgument. */
int vo_hadamard_inplace(float *a, size_t a_len, const float *b, size_t b_len) {
    if (a_len != b_len) return VO_INVALID_ARGUMENT;
    for (size_t i = 0; i < a_len; ++i) a[i] = a[i] * b[i];
    return VO_OK;
}

/* ========================================================================
 * Attention (A13, A14)
 * ====================================================================== */

/* crates/vokra-models/src/whisper/nn.rs:267-325 (per-op path): q is scaled by
 * hd^-0.5 first; per head S = gemm_f32(qh, kh^T), causal -inf for
 * j > q_pos_offset + i, softmax_f32, ctx = gemm_f32(P, vh), scatter.
 * q/k/v/out are [t, n_head*hd] row-major. */
int vo_sdpa_whisper(size_t t_q, size_t t_kv, size_t n_head, size_t hd, const float *q, const float *k,
                    const float *v, int causal, size_t q_pos_offset, float *out) {
    if (n_head == 0 || hd == 0) return VO_INVALID_ARGUMENT;
    size_t d = n_head * hd;
    float scale = powf((float)hd, -0.5f);
    float *qs = (float *)malloc(t_q * d * sizeof(float));
    float *qh = (float *)malloc(t_q * hd * sizeof(float));
    float *kh_t = (float *)malloc(hd * (t_kv ? t_kv : 1) * sizeof(float));
    float *vh = (float *)malloc((t_kv ? t_kv : 1) * hd * sizeof(float));
    float *sc = (float *)malloc(t_q * (t_kv ? t_kv : 1) * sizeof(float));
    float *pr = (float *)malloc(t_q * (t_kv ? t_kv : 1) * sizeof(float));
    float *ctx = (float *)malloc(t_q * hd * sizeof(float));
    for (size_t i = 0; i < t_q * d; ++i) qs[i] = q[i] * scale;
    for (size_t h = 0; h < n_head; ++h) {
        size_t c0 = h * hd;
        for (size_t i = 0; i < t_q; ++i) memcpy(qh + i * hd, qs + i * d + c0, hd * sizeof(float));
        for (size_t j = 0; j < t_kv; ++j) {
            memcpy(vh + j * hd, v + j * d + c0, hd * sizeof(float));
            for (size_t c = 0; c < hd; ++c) kh_t[c * t_kv + j] = k[j * d + c0 + c];
        }
        vo_gemm_f32(t_q, t_kv, hd, qh, kh_t, NULL, sc);
        if (causal)
            for (size_t i = 0; i < t_q; ++i)
                for (size_t j = q_pos_offset + i + 1; j < t_kv; ++j) sc[i * t_kv + j] = -INFINITY;
        vo_softmax_f32(sc, pr, t_q, t_kv);
        vo_gemm_f32(t_q, hd, t_kv, pr, vh, NULL, ctx);
        for (size_t i = 0; i < t_q; ++i) memcpy(out + i * d + c0, ctx + i * hd, hd * sizeof(float));
    }
    free(qs); free(qh); free(kh_t); free(vh); free(sc); free(pr); free(ctx);
    return VO_OK;
}

/* crates/vokra-models/src/voxtral/text_decoder.rs:1312-1360: GQA with
 * h_kv = h_q / (n_head_q / n_head_kv); s = (q.k) * scale (scale after the
 * dot); causal for j > position_offset + i; softmax_f32; sequential P.V. */
int vo_gqa_attention(size_t t, size_t t_kv, size_t n_head_q, size_t n_head_kv, size_t hd,
                     const float *q, const float *k_cache, const float *v_cache, float scale,
                     size_t position_offset, float *out) {
    if (n_head_kv == 0 || n_head_q % n_head_kv != 0) return VO_INVALID_ARGUMENT;
    size_t groups = n_head_q / n_head_kv;
    size_t qh_w = n_head_q * hd, kv_w = n_head_kv * hd;
    float *sc = (float *)malloc(t * (t_kv ? t_kv : 1) * sizeof(float));
    float *pr = (float *)malloc(t * (t_kv ? t_kv : 1) * sizeof(float));
    for (size_t hq = 0; hq < n_head_q; ++hq) {
        size_t hk = hq / groups;
        for (size_t i = 0; i < t; ++i) {
            const float *qr = q + i * qh_w + hq * hd;
            for (size_t j = 0; j < t_kv; ++j) {
                const float *kr = k_cache + j * kv_w + hk * hd;
                float s = 0.0f;
                for (size_t c = 0; c < hd; ++c) s += qr[c] * kr[c];
                sc[i * t_kv + j] = s * scale;
            }
            for (size_t j = position_offset + i + 1; j < t_kv; ++j) sc[i * t_kv + j] = -INFINITY;
        }
        vo_softmax_f32(sc, pr, t, t_kv);
        for (size_t i = 0; i < t; ++i)
            for (size_t c = 0; c < hd; ++c) {
                float sum = 0.0f;
                for (size_t j = 0; j < t_kv; ++j) sum += pr[i * t_kv + j] * v_cache[j * kv_w + hk * hd + c];
                out[i * qh_w + hq * hd + c] = sum;
            }
    }
    free(sc);
    free(pr);
    return VO_OK;
}

/* ========================================================================
 * Quantized paged KV cache (A15) — crates/vokra-core/src/cache/paged_quant.rs
 *
 * The reference page (paged_quant.rs:96-144) holds block_size time steps of
 * one layer for every stream: slot (offset, stream) at
 * offset*n_stream*row_blocks + stream*row_blocks. The table index is
 * layer*pages_per_layer + t/block_size (:414-415). The allocator is a LIFO
 * free list (:152-216). n_codebook is fixed to 1 here.
 * ====================================================================== */
struct vo_paged_cache {
    size_t n_layer, n_head, d_head, n_stream, max_time, bs, pages_per_layer, capacity;
    size_t row_blocks, block_bytes;
    int mode;
    uint8_t *k, *v;       /* [capacity][bs][n_stream][row_blocks][block_bytes] */
    long *page_table;     /* [n_layer*pages_per_layer], -1 = none */
    long *free_list;      /* stack */
    size_t free_len;
};

static size_t page_bytes(const vo_paged_cache *c) {
    return c->bs * c->n_stream * c->row_blocks * c->block_bytes;
}

/* paged_quant.rs:262-307 new; allocator :152-191 (free list = [cap-1..0]) */
int vo_paged_create(size_t n_layer, size_t n_head, size_t d_head, size_t n_stream, size_t max_time,
                    size_t block_size, int mode, vo_paged_cache **out) {
    *out = NULL;
    if (mode == VO_KV_FP32 || vo_kv_block_bytes(mode) == 0) return VO_INVALID_ARGUMENT;
    if (!n_layer || !n_head || !d_head || !n_stream || !max_time || !block_size) return VO_INVALID_ARGUMENT;
    if ((n_head * d_head) % 32 != 0) return VO_INVALID_ARGUMENT;
    vo_paged_cache *c = (vo_paged_cache *)calloc(1, sizeof *c);
    c->n_layer = n_layer;
    c->n_head = n_head;
    c->d_head = d_head;
    c->n_stream = n_stream;
    c->max_time = max_time;
    c->bs = block_size;
    c->mode = mode;
    c->row_blocks = n_head * d_head / 32;
    c->block_bytes = vo_kv_block_bytes(mode);
    c->pages_per_layer = (max_time + block_size - 1) / block_size;
    c->capacity = c->pages_per_layer * n_layer;
    c->k = (uint8_t *)calloc(c->capacity * page_bytes(c), 1);
    c->v = (uint8_t *)calloc(c->capacity * page_bytes(c), 1);
    c->page_table = (long *)malloc(c->capacity * sizeof(long));
    c->free_list = (long *)malloc(c->capacity * sizeof(long));
    vo_paged_reset(c);
    *out = c;
    return VO_OK;
}

void vo_paged_destroy(vo_paged_cache *c) {
    if (!c) return;
    free(c->k);
    free(c->v);
    free(c->page_table);
    free(c->free_list);
    free(c);
}

/* paged_quant.rs:489-493 reset + allocator reset :203-215 */
void vo_paged_reset(vo_paged_cache *c) {
    for (size_t i = 0; i < c->capacity; ++i) c->page_table[i] = -1;
    memset(c->k, 0, c->capacity * page_bytes(c));
    memset(c->v, 0, c->capacity * page_bytes(c));
    c->free_len = 0;
    for (size_t idx = c->capacity; idx-- > 0;) c->free_list[c->free_len++] = (long)idx;
}

static int paged_check(const vo_paged_cache *c, size_t layer, size_t t, size_t s) {
    if (layer >= c->n_layer || t >= c->max_time || s >= c->n_stream) return VO_INVALID_ARGUMENT;
    return VO_OK;
}

static size_t slot_off(const vo_paged_cache *c, size_t offset, size_t s) {
    return (offset * c->n_stream * c->row_blocks + s * c->row_blocks) * c->block_bytes;
}

/* paged_quant.rs:396-437 append_step */
int vo_paged_append_step(vo_paged_cache *c, size_t layer, size_t t, size_t s, const float *k_row,
                         const float *v_row) {
    int st = paged_check(c, layer, t, s);
    if (st) return st;
    size_t ti = layer * c->pages_per_layer + t / c->bs;
    long pid = c->page_table[ti];
    if (pid < 0) {
        if (c->free_len == 0) return VO_KV_CACHE_EXHAUSTED;
        pid = c->free_list[--c->free_len];
        c->page_table[ti] = pid;
    }
    size_t base = (size_t)pid * page_bytes(c) + slot_off(c, t % c->bs, s);
    for (size_t b = 0; b < c->row_blocks; ++b) {
        vo_pack_block(c->mode, k_row + b * 32, c->k + base + b * c->block_bytes);
        vo_pack_block(c->mode, v_row + b * 32, c->v + base + b * c->block_bytes);
    }
    return VO_OK;
}

/* paged_quant.rs:448-480 read_step; returns VO_INVALID_ARGUMENT for "None" */
int vo_paged_read_step(const vo_paged_cache *c, size_t layer, size_t t, size_t s, float *k_out,
                       float *v_out) {
    if (paged_check(c, layer, t, s)) return VO_INVALID_ARGUMENT;
    long pid = c->page_table[layer * c->pages_per_layer + t / c->bs];
    if (pid < 0) return VO_INVALID_ARGUMENT;
    size_t base = (size_t)pid * page_bytes(c) + slot_off(c, t % c->bs, s);
    for (size_t b = 0; b < c->row_blocks; ++b) {
        vo_unpack_block(c->mode, c->k + base + b * c->block_bytes, k_out + b * 32);
        vo_unpack_block(c->mode, c->v + base + b * c->block_bytes, v_out + b * 32);
    }
    return VO_OK;
}

/* paged_quant.rs:500-515 release_layer */
int vo_paged_release_layer(vo_paged_cache *c, size_t layer) {
    if (layer >= c->n_layer) return VO_INVALID_ARGUMENT;
    size_t base = layer * c->pages_per_layer;
    for (size_t i = 0; i < c->pages_per_layer; ++i) {
        long pid = c->page_table[base + i];
        if (pid >= 0) {
            c->page_table[base + i] = -1;
            memset(c->k + (size_t)pid * page_bytes(c), 0, page_bytes(c));
            memset(c->v + (size_t)pid * page_bytes(c), 0, page_bytes(c));
            c->free_list[c->free_len++] = pid;
        }
    }
    return VO_OK;
}

size_t vo_paged_free_pages(const vo_paged_cache *c) { return c->free_len; }
size_t vo_paged_pages_in_use(const vo_paged_cache *c) { return c->capacity - c->free_len; }
long vo_paged_page_of(const vo_paged_cache *c, size_t layer, size_t t) {
    if (layer >= c->n_layer || t >= c->max_time) return -1;
    return c->page_table[layer * c->pages_per_layer + t / c->bs];
}

/* ========================================================================
 * Decode + RNG
 * ====================================================================== */

/* crates/vokra-core/src/decode/sampler.rs:197-206 (first strict max wins) */
uint32_t vo_argmax(const float *logits, size_t n) {
    size_t best = 0;
    float best_v = -INFINITY;
    for (size_t i = 0; i < n; ++i)
        if (logits[i] > best_v) {
            best_v = logits[i];
            best = i;
        }
    return (uint32_t)best;
}

/* crates/vokra-backend-cuda/tests/parity_kernels_cuda.rs:23-34 rand_vec */
void vo_xorshift_rand_vec(uint64_t seed, size_t n, float *out) {
    uint64_t x = seed | 1u;
    for (size_t i = 0; i < n; ++i) {
        x ^= x >> 12;
        x ^= x << 25;
        x ^= x >> 27;
        uint32_t bits = (uint32_t)((x * 0x2545F4914F6CDD1DULL) >> 40);
        out[i] = (float)bits / (float)(1u << 24) * 2.0f - 1.0f;
    }
}

/* crates/vokra-core/src/rng/mod.rs:111-175 SplitMix64 + Box-Muller */
void vo_splitmix_gaussian(uint64_t seed, size_t n, float *out) {
    uint64_t state = seed;
    int have_spare = 0;
    float spare = 0.0f;
    const float two_pi = 2.0f * 3.14159265358979323846f;
    for (size_t i = 0; i < n; ++i) {
        if (have_spare) {
            out[i] = spare;
            have_spare = 0;
            continue;
        }
        float u[2];
        for (int j = 0; j < 2; ++j) {
            state += 0x9E3779B97F4A7C15ULL;
            uint64_t z = state;
            z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
            z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
            z ^= z >> 31;
            float bits = (float)(z >> 40);
            u[j] = (bits + 0.5f) / (float)(1u << 24);
        }
        float r = sqrtf(-2.0f * logf(u[0]));
        float theta = two_pi * u[1];
        spare = r * sinf(theta);
        have_spare = 1;
        out[i] = r * cosf(theta);
    }
}

/* ---- Whisper log-mel front end and conv1d ---------------------------------- */

/* Periodic Hann window (crates/vokra-ops/src/window.rs:31 Hann = cosine_sum
 * [0.5, 0.5], :42-55 w[n] = sum_i (-1)^i a_i cos(i 2 pi n / denom) in f64, cast
 * to f32; periodic: denom = length). */
void vo_hann_periodic(size_t len, float *w) {
    for (size_t n = 0; n < len; ++n) {
        const double x = 2.0 * 3.14159265358979323846 * (double)n / (double)len;
        double acc = 0.0, sign = 1.0;
        const double a[2] = {0.5, 0.5};
        for (int i = 0; i < 2; ++i) {
            acc += sign * a[i] * cos((double)i * x);
            sign = -sign;
        }
        w[n] = (float)acc;
    }
}

/* Slaney mel scale (crates/vokra-ops/src/mel.rs hz_to_mel / mel_to_hz). */
static double vo_hz_to_mel_slaney(double f) {
    const double f_sp = 200.0 / 3.0, min_log_hz = 1000.0, min_log_mel = min_log_hz / f_sp;
    const double logstep = log(6.4) / 27.0;
    return f >= min_log_hz ? min_log_mel + log(f / min_log_hz) / logstep : f / f_sp;
}
static double vo_mel_to_hz_slaney(double mel) {
    const double f_sp = 200.0 / 3.0, min_log_hz = 1000.0, min_log_mel = min_log_hz / f_sp;
    const double logstep = log(6.4) / 27.0;
    return mel >= min_log_mel ? min_log_hz * exp(logstep * (mel - min_log_mel)) : f_sp * mel;
}

/* MelFilterbank::new (crates/vokra-ops/src/mel.rs:29-130) for the Whisper
 * front end (frontend.rs:62-80): Slaney scale, triangles linear in Hz, Slaney
 * norm. w is [n_mels][n_fft/2 + 1]. */
void vo_mel_filterbank(size_t sr, size_t n_fft, size_t n_mels, double fmin, double fmax, float *w) {
    const size_t nf = n_fft / 2 + 1;
    const double min_mel = vo_hz_to_mel_slaney(fmin), max_mel = vo_hz_to_mel_slaney(fmax);
    double *band_hz = (double *)malloc((n_mels + 2) * sizeof(double));
    for (size_t i = 0; i < n_mels + 2; ++i)
        band_hz[i] = vo_mel_to_hz_slaney(min_mel + (max_mel - min_mel) * (double)i / (double)(n_mels + 1));
    for (size_t m = 0; m < n_mels; ++m) {
        const double left = band_hz[m], center = band_hz[m + 1], right = band_hz[m + 2];
        const double fdl = center - left, fdh = right - center;
        for (size_t k = 0; k < nf; ++k) {
            const double f = (double)k * (double)sr / (double)n_fft;
            const double lower = fdl > 0.0 ? (f - left) / fdl : 0.0;
            const double upper = fdh > 0.0 ? (right - f) / fdh : 0.0;
            double v = lower < upper ? lower : upper;
            if (v < 0.0) v = 0.0;
            w[m * nf + k] = (float)v;
        }
        const double enorm = 2.0 / (band_hz[m + 2] - band_hz[m]);
        for (size_t k = 0; k < nf; ++k) w[m * nf + k] = (float)((double)w[m * nf + k] * enorm);
    }
    free(band_hz);
}

/* numpy mode="reflect" index (crates/vokra-ops/src/stft.rs:269-285). */
static size_t vo_reflect(long i, size_t n) {
    if (n == 1) return 0;
    const long period = 2 * (long)(n - 1);
    long r = i % period;
    if (r < 0) r += period;
    return (size_t)(r < (long)n ? r : period - r);
}

/* whisper::mel::log_mel (crates/vokra-models/src/whisper/mel.rs:123-183) over
 * the fused single pass (crates/vokra-ops/src/fused_logmel.rs:80-175): PCM
 * zero-padded / trimmed to 480000 samples, reflect-padded by n_fft/2, frames of
 * 400 every 160 samples windowed in f32 (periodic Hann), |X_k|^2 of the
 * unnormalised DFT (k = 0..200), the trailing frame dropped (3000 kept), mel
 * energy acc += w * p in f32 bin order, log10(max(acc, 1e-10)) into
 * out[m * 3000 + t], then (max(v, gmax - 8) + 4) / 4. The reference's FFT is
 * pocketfft in f32; here the DFT is summed in f64 (the reference holds its own
 * fused and unfused front ends to each other within atol 0.01). */
int vo_log_mel(const float *pcm, size_t n_pcm, size_t n_mels, float *out) {
    const size_t NS = 480000, NFFT = 400, HOP = 160, NFR = 3000, NB = 201, PAD = 200;
    float *buf = (float *)calloc(NS, sizeof(float));
    float *win = (float *)malloc(NFFT * sizeof(float));
    float *fb = (float *)malloc(n_mels * NB * sizeof(float));
    double *cs = (double *)malloc(NB * NFFT * sizeof(double));
    double *sn = (double *)malloc(NB * NFFT * sizeof(double));
    float *frame = (float *)malloc(NFFT * sizeof(float));
    float *pw = (float *)malloc(NB * sizeof(float));
    if (!buf || !win || !fb || !cs || !sn || !frame || !pw) return VO_BACKEND_UNAVAILABLE;
    memcpy(buf, pcm, (n_pcm < NS ? n_pcm : NS) * sizeof(float));
    vo_hann_periodic(NFFT, win);
    vo_mel_filterbank(16000, NFFT, n_mels, 0.0, 8000.0, fb);
    for (size_t k = 0; k < NB; ++k)
        for (size_t n = 0; n < NFFT; ++n) {
            const double th = 2.0 * 3.14159265358979323846 * (double)((k * n) % NFFT) / (double)NFFT;
            cs[k * NFFT + n] = cos(th);
            sn[k * NFFT + n] = sin(th);
        }
    float gmax = -INFINITY;
    for (size_t t = 0; t < NFR; ++t) {
        for (size_t i = 0; i < NFFT; ++i)
            frame[i] = buf[vo_reflect((long)(t * HOP + i) - (long)PAD, NS)] * win[i];
        for (size_t k = 0; k < NB; ++k) {
            double re = 0.0, im = 0.0;
            for (size_t n = 0; n < NFFT; ++n) {
                re += (double)frame[n] * cs[k * NFFT + n];
                im -= (double)frame[n] * sn[k * NFFT + n];
            }
            pw[k] = (float)(re * re + im * im);
        }
        for (size_t m = 0; m < n_mels; ++m) {
            float acc = 0.0f;
            for (size_t k = 0; k < NB; ++k) acc += fb[m * NB + k] * pw[k];
            const float l = log10f(acc > 1e-10f ? acc : 1e-10f);
            out[m * NFR + t] = l;
            if (l > gmax) gmax = l;
        }
    }
    const float floor_v = gmax - 8.0f;
    for (size_t i = 0; i < n_mels * NFR; ++i) out[i] = ((out[i] > floor_v ? out[i] : floor_v) + 4.0f) / 4.0f;
    free(buf); free(win); free(fb); free(cs); free(sn); free(frame); free(pw);
    return VO_OK;
}

/* kernels::conv1d_f32 (crates/vokra-backend-cpu/src/kernels/mod.rs:583-822):
 * im2col col[c*kernel + kk][t] = in[c][t*stride + kk - padding] (zero outside),
 * out = weight [out_ch, in_ch*kernel] x col by the scalar gemm (accumulating
 * from 0), then + bias[oc]. Returns INVALID_ARGUMENT for the reference's
 * rejections (zero stride / kernel, padded length shorter than the kernel). */
int vo_conv1d_f32(const float *input, size_t in_ch, size_t in_len, const float *weight, size_t out_ch,
                  size_t kernel, const float *bias, size_t stride, size_t padding, float *out) {
    if (stride == 0 || kernel == 0) return VO_INVALID_ARGUMENT;
    const size_t padded = in_len + 2 * padding;
    if (padded < kernel) return VO_INVALID_ARGUMENT;
    const size_t out_len = (padded - kernel) / stride + 1, k = in_ch * kernel;
    float *col = (float *)calloc((k * out_len) > 0 ? k * out_len : 1, sizeof(float));
    if (!col) return VO_BACKEND_UNAVAILABLE;
    for (size_t c = 0; c < in_ch; ++c)
        for (size_t kk = 0; kk < kernel; ++kk)
            for (size_t t = 0; t < out_len; ++t) {
                const size_t pos = t * stride + kk;
                if (pos >= padding && pos < padding + in_len) col[(c * kernel + kk) * out_len + t] = input[c * in_len + (pos - padding)];
            }
    vo_gemm_f32(out_ch, out_len, k, weight, col, NULL, out);
    if (bias)
        for (size_t oc = 0; oc < out_ch; ++oc)
            for (size_t t = 0; t < out_len; ++t) out[oc * out_len + t] += bias[oc];
    free(col);
    return VO_OK;
}

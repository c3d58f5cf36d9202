"""ctypes wrapper over liboracle.so — the CPU restatement of the reference.

TEST INFRASTRUCTURE ONLY: imported by tests/, ``__graft_entry__.smoke()`` and
the ``cpu_baseline`` leg of ``bench.py`` as the parity checker. The product
library (vokra_amd) never imports it.

Each wrapper names the C function it calls; the C file cites the reference
file:line each function restates.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")

OK = 0
UNSUPPORTED_OP = 3
BACKEND_UNAVAILABLE = 4
INVALID_ARGUMENT = 5
KV_CACHE_EXHAUSTED = 10

# KvQuant (kv_quant/mod.rs:81-91)
FP32, Q4_0, Q5_0, Q8_0 = 0, 1, 2, 3
# weight dtypes (ggml tags)
W_Q4_0, W_Q5_0, W_Q8_0, W_Q4_K, W_Q5_K, W_Q6_K = 2, 6, 8, 12, 13, 14

KV_BLOCK_BYTES = {FP32: 128, Q4_0: 18, Q5_0: 22, Q8_0: 34}
W_BLOCK_BYTES = {W_Q4_0: 18, W_Q5_0: 22, W_Q8_0: 34, W_Q4_K: 144, W_Q5_K: 176, W_Q6_K: 210}
W_BLOCK_ELEMS = {W_Q4_0: 32, W_Q5_0: 32, W_Q8_0: 32, W_Q4_K: 256, W_Q5_K: 256, W_Q6_K: 256}
KV_OF_W = {W_Q4_0: Q4_0, W_Q5_0: Q5_0, W_Q8_0: Q8_0}


def build() -> str:
    """Compile liboracle.so from vokra_oracle.c (gcc, -ffp-contract=off)."""
    subprocess.run(["make", "-s", "-C", _HERE, "-B"], check=True)
    return _LIB_PATH


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = C.CDLL(_LIB_PATH)
        _declare(_lib)
    return _lib


_f32p = C.POINTER(C.c_float)
_u8p = C.POINTER(C.c_uint8)
_i8p = C.POINTER(C.c_int8)
_i32p = C.POINTER(C.c_int32)
_sz = C.c_size_t


def _declare(L):
    L.vo_f16_bits_to_f32.restype = C.c_float
    L.vo_f16_bits_to_f32.argtypes = [C.c_uint16]
    L.vo_f32_to_f16_bits.restype = C.c_uint16
    L.vo_f32_to_f16_bits.argtypes = [C.c_float]
    L.vo_gguf_f16_to_f32.restype = C.c_float
    L.vo_gguf_f16_to_f32.argtypes = [C.c_uint16]
    L.vo_convert_f32_to_f16.restype = C.c_uint16
    L.vo_convert_f32_to_f16.argtypes = [C.c_float]
    L.vo_kv_block_bytes.restype = _sz
    L.vo_kv_block_bytes.argtypes = [C.c_int]
    L.vo_pack_block.argtypes = [C.c_int, _f32p, _u8p]
    L.vo_unpack_block.argtypes = [C.c_int, _u8p, _f32p]
    L.vo_dequantize_bytes.argtypes = [C.c_int, _u8p, _sz, _f32p, _sz]
    L.vo_pack_matrix_to_bytes.argtypes = [C.c_int, _f32p, _sz, _sz, _u8p]
    L.vo_validate_dequant_gemv.argtypes = [C.c_int, _sz, _sz, _sz, _sz]
    L.vo_dequant_gemv_scalar.argtypes = [C.c_int, _u8p, _sz, _sz, _sz, _f32p, _sz, _f32p]
    L.vo_dense_gemv_f32.argtypes = [_f32p, _sz, _f32p, _sz, _f32p]
    L.vo_quantize_act_b32.argtypes = [_f32p, _sz, _i8p, _f32p, _i32p]
    L.vo_quantize_act_b32_mode.argtypes = [_f32p, _sz, _i8p, _f32p, _i32p, C.c_int]
    L.vo_gemm_qblock_i8_mode.argtypes = [C.c_int, _sz, _sz, _sz, _f32p, _u8p, _sz, _f32p, _f32p, C.c_int]
    L.vo_qblock_block_dots_mode.argtypes = [C.c_int, _sz, _sz, _sz, _f32p, _u8p, _i32p, C.c_int]
    L.vo_gemm_qblock_i8.argtypes = [C.c_int, _sz, _sz, _sz, _f32p, _u8p, _sz, _f32p, _f32p]
    L.vo_qblock_block_dots.argtypes = [C.c_int, _sz, _sz, _sz, _f32p, _u8p, _i32p]
    L.vo_qblock_error_bound.restype = C.c_float
    L.vo_qblock_error_bound.argtypes = [C.c_int, _u8p, _f32p, _sz]
    L.vo_kquant_dequantize.argtypes = [C.c_int, _u8p, _sz, _sz, _f32p]
    L.vo_kquant_quantize.argtypes = [C.c_int, _f32p, _sz, _u8p]
    L.vo_kquant_quantize_activations.argtypes = [_f32p, _sz, _i8p, _f32p, _i32p]
    L.vo_kquant_gemv_i8.argtypes = [C.c_int, _sz, _sz, _u8p, _sz, _f32p, _sz, _f32p, _sz]
    L.vo_kquant_gemm_i8.argtypes = [C.c_int, _sz, _sz, _sz, _u8p, _sz, _f32p, _sz, _f32p, _sz]
    L.vo_int8_error_bound.restype = C.c_float
    L.vo_int8_error_bound.argtypes = [C.c_int, _u8p, _f32p, _sz]
    L.vo_gemm_q_f32.argtypes = [C.c_int, _sz, _sz, _sz, _f32p, _sz, _u8p, _sz, _f32p, _f32p, _sz]
    L.vo_gemm_f32.argtypes = [_sz, _sz, _sz, _f32p, _f32p, _f32p, _f32p]
    L.vo_gemm_f32_mt.argtypes = [_sz, _sz, _sz, _f32p, _f32p, _f32p, _f32p, C.c_int]
    L.vo_gemv_f32.argtypes = [_sz, _sz, _f32p, _f32p, _f32p, _f32p]
    L.vo_softmax_f32.argtypes = [_f32p, _f32p, _sz, _sz]
    L.vo_layer_norm_f32.argtypes = [_f32p, _f32p, _sz, _sz, _f32p, _f32p, C.c_float]
    L.vo_gelu_f32.argtypes = [_f32p, _f32p, _sz]
    L.vo_erf_as.restype = C.c_float
    L.vo_erf_as.argtypes = [C.c_float]
    L.vo_rms_norm_f32.argtypes = [_f32p, _f32p, C.c_float, _sz, _sz, _f32p]
    L.vo_rope_apply.argtypes = [_f32p, _sz, _sz, _sz, C.c_float, _sz]
    L.vo_silu_inplace.argtypes = [_f32p, _sz]
    L.vo_hadamard_inplace.argtypes = [_f32p, _sz, _f32p, _sz]
    L.vo_sdpa_whisper.argtypes = [_sz, _sz, _sz, _sz, _f32p, _f32p, _f32p, C.c_int, _sz, _f32p]
    L.vo_gqa_attention.argtypes = [_sz, _sz, _sz, _sz, _sz, _f32p, _f32p, _f32p, C.c_float, _sz, _f32p]
    L.vo_paged_create.argtypes = [_sz, _sz, _sz, _sz, _sz, _sz, C.c_int, C.POINTER(C.c_void_p)]
    L.vo_paged_destroy.argtypes = [C.c_void_p]
    L.vo_paged_append_step.argtypes = [C.c_void_p, _sz, _sz, _sz, _f32p, _f32p]
    L.vo_paged_read_step.argtypes = [C.c_void_p, _sz, _sz, _sz, _f32p, _f32p]
    L.vo_paged_release_layer.argtypes = [C.c_void_p, _sz]
    L.vo_paged_reset.argtypes = [C.c_void_p]
    L.vo_paged_free_pages.restype = _sz
    L.vo_paged_free_pages.argtypes = [C.c_void_p]
    L.vo_paged_pages_in_use.restype = _sz
    L.vo_paged_pages_in_use.argtypes = [C.c_void_p]
    L.vo_paged_page_of.restype = C.c_long
    L.vo_paged_page_of.argtypes = [C.c_void_p, _sz, _sz]
    L.vo_argmax.restype = C.c_uint32
    L.vo_argmax.argtypes = [_f32p, _sz]
    L.vo_xorshift_rand_vec.argtypes = [C.c_uint64, _sz, _f32p]
    L.vo_splitmix_gaussian.argtypes = [C.c_uint64, _sz, _f32p]
    L.vo_hann_periodic.argtypes = [_sz, _f32p]
    L.vo_mel_filterbank.argtypes = [_sz, _sz, _sz, C.c_double, C.c_double, _f32p]
    L.vo_log_mel.argtypes = [_f32p, _sz, _sz, _f32p]
    L.vo_conv1d_f32.argtypes = [_f32p, _sz, _sz, _f32p, _sz, _sz, _f32p, _sz, _sz, _f32p]


def _p(a, t):
    if a is None:
        return None
    return a.ctypes.data_as(t)


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _u8(a):
    return np.ascontiguousarray(a, dtype=np.uint8)


class OracleError(RuntimeError):
    def __init__(self, code, what):
        super().__init__(f"{what}: status {code}")
        self.code = code


def _check(code, what):
    if code != OK:
        raise OracleError(code, what)


# ---- binary16 ----------------------------------------------------------
def f16_bits_to_f32(h: int) -> float:
    return lib().vo_f16_bits_to_f32(h)


def f32_to_f16_bits(x: float) -> int:
    return lib().vo_f32_to_f16_bits(x)


def gguf_f16_to_f32(h: int) -> float:
    return lib().vo_gguf_f16_to_f32(h)


def convert_f32_to_f16(x: float) -> int:
    return lib().vo_convert_f32_to_f16(x)


# ---- Q_0 codecs --------------------------------------------------------
def pack_block(mode, x32):
    x = _f32(x32)
    assert x.size == 32
    out = np.zeros(KV_BLOCK_BYTES[mode], np.uint8)
    lib().vo_pack_block(mode, _p(x, _f32p), _p(out, _u8p))
    return out


def unpack_block(mode, blk):
    b = _u8(blk)
    out = np.zeros(32, np.float32)
    lib().vo_unpack_block(mode, _p(b, _u8p), _p(out, _f32p))
    return out


def dequantize_bytes(mode, data):
    b = _u8(data)
    bb = KV_BLOCK_BYTES.get(mode, 1)
    n_out = (b.size // bb) * 32
    out = np.zeros(max(n_out, 1), np.float32)
    _check(lib().vo_dequantize_bytes(mode, _p(b, _u8p), b.size, _p(out, _f32p), n_out),
           "dequantize_bytes")
    return out[:n_out]


def pack_matrix_to_bytes(mode, a, n_rows, n_bpr):
    x = _f32(a)
    assert x.size == n_rows * n_bpr * 32
    out = np.zeros(n_rows * n_bpr * KV_BLOCK_BYTES[mode], np.uint8)
    _check(lib().vo_pack_matrix_to_bytes(mode, _p(x, _f32p), n_rows, n_bpr, _p(out, _u8p)),
           "pack_matrix_to_bytes")
    return out


def dequant_gemv_scalar(mode, data, n_rows, n_bpr, x):
    b = _u8(data)
    xv = _f32(x)
    y = np.zeros(max(n_rows, 1), np.float32)
    _check(lib().vo_dequant_gemv_scalar(mode, _p(b, _u8p), b.size, n_rows, n_bpr,
                                        _p(xv, _f32p), xv.size, _p(y, _f32p)),
           "dequant_gemv_scalar")
    return y[:n_rows]


def validate_dequant_gemv(mode, n_bytes, n_rows, n_bpr, x_len):
    return lib().vo_validate_dequant_gemv(mode, n_bytes, n_rows, n_bpr, x_len)


def dense_gemv_f32(a, n_rows, x):
    av, xv = _f32(a), _f32(x)
    y = np.zeros(n_rows, np.float32)
    lib().vo_dense_gemv_f32(_p(av, _f32p), n_rows, _p(xv, _f32p), xv.size, _p(y, _f32p))
    return y


# ---- block INT8 --------------------------------------------------------
def quantize_act_b32(x, pow2=False):
    xv = _f32(x)
    k = xv.size
    q = np.zeros(k, np.int8)
    s = np.zeros(k // 32, np.float32)
    g = np.zeros(k // 32, np.int32)
    lib().vo_quantize_act_b32_mode(_p(xv, _f32p), k, _p(q, _i8p), _p(s, _f32p), _p(g, _i32p),
                                   int(pow2))
    return q, s, g


def gemm_qblock_i8(wdtype, m, n, k, a, wq, bias=None, pow2=False):
    av, wv = _f32(a), _u8(wq)
    bv = None if bias is None else _f32(bias)
    out = np.zeros(m * n, np.float32)
    _check(lib().vo_gemm_qblock_i8_mode(wdtype, m, n, k, _p(av, _f32p), _p(wv, _u8p), wv.size,
                                        _p(bv, _f32p), _p(out, _f32p), int(pow2)),
           "gemm_qblock_i8")
    return out.reshape(m, n)


def qblock_block_dots(wdtype, m, n, k, a, wq, pow2=False):
    av, wv = _f32(a), _u8(wq)
    out = np.zeros(m * n * (k // 32), np.int32)
    _check(lib().vo_qblock_block_dots_mode(wdtype, m, n, k, _p(av, _f32p), _p(wv, _u8p),
                                           _p(out, _i32p), int(pow2)), "qblock_block_dots")
    return out.reshape(m, n, k // 32)


def qblock_error_bound(wdtype, w_row, x):
    wv, xv = _u8(w_row), _f32(x)
    return lib().vo_qblock_error_bound(wdtype, _p(wv, _u8p), _p(xv, _f32p), xv.size)


# ---- K-quant -----------------------------------------------------------
def kquant_dequantize(wdtype, data, n_elements):
    b = _u8(data)
    out = np.zeros(max(n_elements, 1), np.float32)
    _check(lib().vo_kquant_dequantize(wdtype, _p(b, _u8p), b.size, n_elements, _p(out, _f32p)),
           "kquant_dequantize")
    return out[:n_elements]


def kquant_quantize(wdtype, data):
    x = _f32(data)
    out = np.zeros(x.size // 256 * 144, np.uint8)
    _check(lib().vo_kquant_quantize(wdtype, _p(x, _f32p), x.size, _p(out, _u8p)),
           "kquant_quantize")
    return out


def kquant_quantize_activations(x):
    xv = _f32(x)
    k = xv.size
    q = np.zeros(k, np.int8)
    s = np.zeros(k // 16, np.float32)
    g = np.zeros(k // 16, np.int32)
    lib().vo_kquant_quantize_activations(_p(xv, _f32p), k, _p(q, _i8p), _p(s, _f32p), _p(g, _i32p))
    return q, s, g


def kquant_gemv_i8(wdtype, m, k, w, x):
    wv, xv = _u8(w), _f32(x)
    out = np.zeros(max(m, 1), np.float32)
    _check(lib().vo_kquant_gemv_i8(wdtype, m, k, _p(wv, _u8p), wv.size, _p(xv, _f32p), xv.size,
                                   _p(out, _f32p), m), "kquant_gemv_i8")
    return out[:m]


def kquant_gemm_i8(wdtype, m, k, n_act, w, x):
    wv, xv = _u8(w), _f32(x)
    out = np.zeros(max(m * n_act, 1), np.float32)
    _check(lib().vo_kquant_gemm_i8(wdtype, m, k, n_act, _p(wv, _u8p), wv.size, _p(xv, _f32p),
                                   xv.size, _p(out, _f32p), m * n_act), "kquant_gemm_i8")
    return out[: m * n_act].reshape(n_act, m)


def int8_error_bound(wdtype, w_row, x):
    wv, xv = _u8(w_row), _f32(x)
    return lib().vo_int8_error_bound(wdtype, _p(wv, _u8p), _p(xv, _f32p), xv.size)


def gemm_q_f32(wdtype, m, n, k, a, wq, bias=None):
    av, wv = _f32(a), _u8(wq)
    bv = None if bias is None else _f32(bias)
    out = np.zeros(max(m * n, 1), np.float32)
    _check(lib().vo_gemm_q_f32(wdtype, m, n, k, _p(av, _f32p), av.size, _p(wv, _u8p), wv.size,
                               _p(bv, _f32p), _p(out, _f32p), m * n), "gemm_q_f32")
    return out[: m * n].reshape(m, n)


# ---- f32 scalar --------------------------------------------------------
def gemm_f32(m, n, k, a, b, bias=None, threads=1):
    av, bv = _f32(a), _f32(b)
    cv = None if bias is None else _f32(bias)
    out = np.zeros(m * n, np.float32)
    lib().vo_gemm_f32_mt(m, n, k, _p(av, _f32p), _p(bv, _f32p), _p(cv, _f32p), _p(out, _f32p),
                         threads)
    return out.reshape(m, n)


def gemv_f32(m, k, a, x, bias=None):
    av, xv = _f32(a), _f32(x)
    cv = None if bias is None else _f32(bias)
    out = np.zeros(m, np.float32)
    lib().vo_gemv_f32(m, k, _p(av, _f32p), _p(xv, _f32p), _p(cv, _f32p), _p(out, _f32p))
    return out


def softmax_f32(x, rows, cols):
    xv = _f32(x)
    out = np.zeros(rows * cols, np.float32)
    lib().vo_softmax_f32(_p(xv, _f32p), _p(out, _f32p), rows, cols)
    return out.reshape(rows, cols)


def layer_norm_f32(x, rows, cols, gamma, beta, eps=1e-5):
    xv, g, b = _f32(x), _f32(gamma), _f32(beta)
    out = np.zeros(rows * cols, np.float32)
    lib().vo_layer_norm_f32(_p(xv, _f32p), _p(out, _f32p), rows, cols, _p(g, _f32p),
                            _p(b, _f32p), eps)
    return out.reshape(rows, cols)


def gelu_f32(x):
    xv = _f32(x)
    out = np.zeros(xv.size, np.float32)
    lib().vo_gelu_f32(_p(xv, _f32p), _p(out, _f32p), xv.size)
    return out.reshape(np.shape(x))


def erf_as(x: float) -> float:
    return lib().vo_erf_as(x)


def rms_norm_f32(x, gamma, eps, rows, d):
    xv, g = _f32(x), _f32(gamma)
    out = np.zeros(rows * d, np.float32)
    lib().vo_rms_norm_f32(_p(xv, _f32p), _p(g, _f32p), eps, rows, d, _p(out, _f32p))
    return out.reshape(rows, d)


def rope_apply(x, seq_len, head_dim, rope_base, position_offset):
    """text_decoder.rs:858-891 on one head's [seq_len, head_dim]; returns a copy."""
    xv = _f32(x).copy()
    _check(lib().vo_rope_apply(_p(xv, _f32p), xv.size, seq_len, head_dim, rope_base, position_offset),
           "rope_apply")
    return xv


def rope_heads(x, n_head, head_dim, rope_base, position_offset):
    """rope_apply per head of x [seq_len, n_head * head_dim] (the loop of
    text_decoder.rs:1230-1275)."""
    xv = _f32(x)
    t = xv.size // (n_head * head_dim)
    xv = xv.reshape(t, n_head, head_dim)
    out = np.empty_like(xv)
    for h in range(n_head):
        out[:, h, :] = rope_apply(xv[:, h, :], t, head_dim, rope_base, position_offset).reshape(t, head_dim)
    return out.reshape(t, n_head * head_dim)


def silu(x):
    """text_decoder.rs:826-831 silu_inplace, on a copy."""
    xv = _f32(x).copy()
    lib().vo_silu_inplace(_p(xv, _f32p), xv.size)
    return xv


def hadamard(a, b):
    """text_decoder.rs:835-847 hadamard_inplace, on a copy of a."""
    av, bv = _f32(a).copy(), _f32(b)
    _check(lib().vo_hadamard_inplace(_p(av, _f32p), av.size, _p(bv, _f32p), bv.size), "hadamard_inplace")
    return av


def swiglu(gate, up):
    """silu(gate) * up exactly as text_decoder.rs:1405-1410 sequences it."""
    return hadamard(silu(gate), up)


# ---- attention ---------------------------------------------------------
def sdpa_whisper(t_q, t_kv, n_head, hd, q, k, v, causal=False, q_pos_offset=0):
    qv, kv, vv = _f32(q), _f32(k), _f32(v)
    out = np.zeros(t_q * n_head * hd, np.float32)
    _check(lib().vo_sdpa_whisper(t_q, t_kv, n_head, hd, _p(qv, _f32p), _p(kv, _f32p),
                                 _p(vv, _f32p), int(causal), q_pos_offset, _p(out, _f32p)),
           "sdpa_whisper")
    return out.reshape(t_q, n_head * hd)


def gqa_attention(t, t_kv, n_head_q, n_head_kv, hd, q, k_cache, v_cache, scale, position_offset):
    qv, kv, vv = _f32(q), _f32(k_cache), _f32(v_cache)
    out = np.zeros(t * n_head_q * hd, np.float32)
    _check(lib().vo_gqa_attention(t, t_kv, n_head_q, n_head_kv, hd, _p(qv, _f32p), _p(kv, _f32p),
                                  _p(vv, _f32p), scale, position_offset, _p(out, _f32p)),
           "gqa_attention")
    return out.reshape(t, n_head_q * hd)


# ---- paged quantized KV cache --------------------------------------------
class PagedCache:
    """QuantizedPagedKvCache restatement (paged_quant.rs:240-545), n_codebook=1."""

    def __init__(self, n_layer, n_head, d_head, n_stream, max_time, block_size, mode):
        h = C.c_void_p()
        _check(lib().vo_paged_create(n_layer, n_head, d_head, n_stream, max_time, block_size,
                                     mode, C.byref(h)), "paged_create")
        self._h = h
        self.per_slot = n_head * d_head

    def __del__(self):
        if getattr(self, "_h", None):
            lib().vo_paged_destroy(self._h)
            self._h = None

    def append_step(self, layer, t, s, k_row, v_row):
        k, v = _f32(k_row), _f32(v_row)
        return lib().vo_paged_append_step(self._h, layer, t, s, _p(k, _f32p), _p(v, _f32p))

    def read_step(self, layer, t, s):
        k = np.zeros(self.per_slot, np.float32)
        v = np.zeros(self.per_slot, np.float32)
        st = lib().vo_paged_read_step(self._h, layer, t, s, _p(k, _f32p), _p(v, _f32p))
        return None if st != OK else (k, v)

    def release_layer(self, layer):
        return lib().vo_paged_release_layer(self._h, layer)

    def reset(self):
        lib().vo_paged_reset(self._h)

    def free_pages(self):
        return lib().vo_paged_free_pages(self._h)

    def pages_in_use(self):
        return lib().vo_paged_pages_in_use(self._h)

    def page_of(self, layer, t):
        return lib().vo_paged_page_of(self._h, layer, t)


# ---- decode + RNG -------------------------------------------------------
def argmax(logits):
    lv = _f32(logits)
    return lib().vo_argmax(_p(lv, _f32p), lv.size)


def xorshift_rand_vec(seed, n):
    out = np.zeros(max(n, 1), np.float32)
    lib().vo_xorshift_rand_vec(seed & 0xFFFFFFFFFFFFFFFF, n, _p(out, _f32p))
    return out[:n]


def splitmix_gaussian(seed, n):
    out = np.zeros(max(n, 1), np.float32)
    lib().vo_splitmix_gaussian(seed & 0xFFFFFFFFFFFFFFFF, n, _p(out, _f32p))
    return out[:n]


# ---- Whisper log-mel front end and conv1d ----------------------------------
N_SAMPLES, N_FFT, HOP, N_FRAMES = 480000, 400, 160, 3000


def hann_periodic(n):
    """vo_hann_periodic: window.rs cosine_sum([0.5, 0.5]), periodic."""
    out = np.zeros(n, np.float32)
    lib().vo_hann_periodic(n, _p(out, _f32p))
    return out


def mel_filterbank(n_mels, sr=16000, n_fft=N_FFT, fmin=0.0, fmax=8000.0):
    """vo_mel_filterbank: [n_mels, n_fft/2 + 1], Slaney scale and norm."""
    out = np.zeros(n_mels * (n_fft // 2 + 1), np.float32)
    lib().vo_mel_filterbank(sr, n_fft, n_mels, fmin, fmax, _p(out, _f32p))
    return out.reshape(n_mels, n_fft // 2 + 1)


def log_mel(pcm, n_mels):
    """vo_log_mel: whisper::mel::log_mel -> [n_mels, 3000]."""
    x = _f32(pcm).reshape(-1)
    out = np.zeros(n_mels * N_FRAMES, np.float32)
    _check(lib().vo_log_mel(_p(x, _f32p) if x.size else None, x.size, n_mels, _p(out, _f32p)), "log_mel")
    return out.reshape(n_mels, N_FRAMES)


def conv1d_out_len(in_len, kernel, stride, padding):
    return (in_len + 2 * padding - kernel) // stride + 1


def conv1d_f32(x, in_ch, in_len, w, out_ch, kernel, bias=None, stride=1, padding=0):
    """vo_conv1d_f32: kernels::conv1d_f32 -> [out_ch, out_len]."""
    xv, wv = _f32(x), _f32(w)
    bv = None if bias is None else _f32(bias)
    out_len = conv1d_out_len(in_len, kernel, stride, padding) if stride and kernel else 0
    out = np.zeros(max(out_ch * max(out_len, 0), 1), np.float32)
    _check(lib().vo_conv1d_f32(_p(xv, _f32p), in_ch, in_len, _p(wv, _f32p), out_ch, kernel, _p(bv, _f32p),
                               stride, padding, _p(out, _f32p)), "conv1d_f32")
    return out[:out_ch * out_len].reshape(out_ch, out_len)


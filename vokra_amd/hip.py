"""Python mirror of the reference's device-context surface over the C ABI.

``HipContext`` follows ``CudaContext`` (crates/vokra-backend-cuda/src/context.rs):
the same method names, argument meaning and error behaviour, so the parity
tests read like the reference's ``parity_kernels_cuda.rs``. Errors map to the
``VokraError`` variants (crates/vokra-core/src/error.rs:21-104). There is no
CPU fallback anywhere: if the HIP library or a device is missing, calls raise
``BackendUnavailable``.
"""
from __future__ import annotations

import ctypes as C
import os
from enum import IntEnum

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libvokra_hip.so")


class VokraError(RuntimeError):
    code = 9


class UnsupportedOp(VokraError):
    code = 3


class BackendUnavailable(VokraError):
    code = 4


class InvalidArgument(VokraError):
    code = 5


class KvCacheExhausted(VokraError):
    code = 10


class IoError(VokraError):
    """VokraError::Io (include/vokra.h VOKRA_ERROR_IO)."""


class ModelLoad(VokraError):
    """VokraError::ModelLoad (include/vokra.h VOKRA_ERROR_MODEL_LOAD)."""


_ERRORS = {1: IoError, 2: ModelLoad, 3: UnsupportedOp, 4: BackendUnavailable, 5: InvalidArgument,
           10: KvCacheExhausted}


class KvQuant(IntEnum):
    """crates/vokra-core/src/kv_quant/mod.rs:81-91 (declaration order)."""
    Fp32 = 0
    Q4_0 = 1
    Q5_0 = 2
    Q8_0 = 3

    def block_bytes(self) -> int:
        return {0: 128, 1: 18, 2: 22, 3: 34}[int(self)]


class WDtype(IntEnum):
    """Weight dtypes of gemm_q_f32 (ggml type tags)."""
    Q4_0 = 2
    Q5_0 = 6
    Q8_0 = 8
    Q4_K = 12
    Q5_K = 13
    Q6_K = 14


class ActQuant(IntEnum):
    AMAX127 = 0
    POW2 = 1
    KQUANT = 2


class CrossPrecision(IntEnum):
    """Decoder cross-attention K/V reads (VOKRA_HIP_CROSS_*)."""
    F32 = 0
    F16 = 1


_lib = None

_F = C.POINTER(C.c_float)
_U8 = C.POINTER(C.c_uint8)


class PrenormLayer(C.Structure):
    """vokra_hip_prenorm_layer_t"""
    _fields_ = [("ln1_gamma", _F), ("ln1_beta", _F), ("wq", _U8), ("wk", _U8), ("wv", _U8), ("wo", _U8),
                ("bq", _F), ("bk", _F), ("bv", _F), ("bo", _F), ("ln2_gamma", _F), ("ln2_beta", _F),
                ("w1", _U8), ("w2", _U8), ("b1", _F), ("b2", _F)]


class DecoderLayer(C.Structure):
    """vokra_hip_decoder_layer_t"""
    _fields_ = [("ln1_gamma", _F), ("ln1_beta", _F), ("wq", _U8), ("wk", _U8), ("wv", _U8), ("wo", _U8),
                ("bq", _F), ("bk", _F), ("bv", _F), ("bo", _F), ("ln2_gamma", _F), ("ln2_beta", _F),
                ("cwq", _U8), ("cwk", _U8), ("cwv", _U8), ("cwo", _U8),
                ("cbq", _F), ("cbk", _F), ("cbv", _F), ("cbo", _F), ("ln3_gamma", _F), ("ln3_beta", _F),
                ("w1", _U8), ("w2", _U8), ("b1", _F), ("b2", _F)]


class WhisperConfig(C.Structure):
    """vokra_hip_whisper_config_t (whisper/config.rs WhisperConfig)."""
    _fields_ = [(n, C.c_size_t) for n in ("n_mels", "d_model", "n_audio_ctx", "n_audio_head", "n_audio_layer",
                                          "n_text_ctx", "n_text_head", "n_text_layer", "n_vocab", "ffn_dim")] + \
               [("eot", C.c_uint32)]


class VoxtralConfig(C.Structure):
    """vokra_hip_voxtral_config_t (voxtral/config.rs VoxtralConfig, numeric fields)."""
    _fields_ = [(n, C.c_size_t) for n in ("audio_n_layer", "audio_n_head", "audio_hidden_dim", "audio_n_ctx",
                                          "audio_n_mels", "audio_ffn_dim", "n_layer", "n_head_q", "n_head_kv",
                                          "head_dim", "hidden_dim", "ffn_dim", "vocab_size", "n_ctx")] + \
               [("rope_base", C.c_float), ("rms_norm_eps", C.c_float), ("cross_attn_hidden_dim", C.c_size_t)]


class WhisperLoadReport(C.Structure):
    """vokra_hip_whisper_load_report_t: Linear weights taken verbatim / packed at load."""
    _fields_ = [("verbatim", C.c_size_t), ("packed", C.c_size_t)]


class TextDecoderLayer(C.Structure):
    """vokra_hip_text_decoder_layer_t"""
    _fields_ = [("attn_norm_gamma", _F), ("wq", _U8), ("wk", _U8), ("wv", _U8), ("wo", _U8),
                ("ffn_norm_gamma", _F), ("w_gate", _U8), ("w_up", _U8), ("w_down", _U8)]


def _ctx_alive(obj):
    """True while the context an object was made on is open: handles are only
    freed through a live context (after close, the process exit reclaims them)."""
    ctx = getattr(obj, "_ctx", None) or getattr(obj, "ctx", None)
    return ctx is not None and getattr(ctx, "_h", None) is not None


def _fill_struct(st_type, fields, keep):
    """Builds a layer struct from a dict of numpy arrays (missing / None -> NULL);
    the arrays are appended to `keep` so they outlive the create call."""
    st = st_type()
    for name, ctype in st_type._fields_:
        arr = fields.get(name)
        if arr is None:
            continue
        arr = np.ascontiguousarray(arr, np.uint8 if ctype is _U8 else np.float32)
        keep.append(arr)
        setattr(st, name, arr.ctypes.data_as(ctype))
    return st


def _declare(L):
    P = C.c_void_p
    sz = C.c_size_t
    f32p = C.POINTER(C.c_float)
    u8p = C.POINTER(C.c_uint8)
    L.vokra_hip_last_error.restype = C.c_char_p
    L.vokra_hip_probe.argtypes = [C.POINTER(C.c_int)]
    L.vokra_hip_create.argtypes = [C.c_int, C.POINTER(P)]
    L.vokra_hip_destroy.argtypes = [P]
    L.vokra_hip_destroy.restype = None
    L.vokra_hip_synchronize.argtypes = [P]
    L.vokra_hip_device_alloc.argtypes = [P, sz, C.POINTER(P)]
    L.vokra_hip_device_free.argtypes = [P, P]
    L.vokra_hip_memcpy_htod.argtypes = [P, P, P, sz]
    L.vokra_hip_memcpy_dtoh.argtypes = [P, P, P, sz]
    L.vokra_hip_event_create.argtypes = [P, C.POINTER(P)]
    L.vokra_hip_event_record.argtypes = [P, P]
    L.vokra_hip_event_elapsed_ms.argtypes = [P, P, f32p]
    L.vokra_hip_event_destroy.argtypes = [P]
    L.vokra_hip_event_destroy.restype = None
    L.vokra_hip_dequantize_bytes.argtypes = [P, C.c_int, u8p, sz, f32p, sz]
    L.vokra_hip_kquant_dequantize.argtypes = [P, C.c_int, u8p, sz, sz, f32p]
    L.vokra_hip_dequant_gemv_f32.argtypes = [P, C.c_int, u8p, sz, sz, sz, f32p, sz, f32p]
    L.vokra_hip_gemm_q_f32.argtypes = [P, C.c_int, sz, sz, sz, f32p, sz, u8p, sz, f32p, f32p, sz]
    L.vokra_hip_set_act_quant.argtypes = [P, C.c_int]
    L.vokra_hip_set_decode_kernel.argtypes = [P, C.c_int]
    L.vokra_hip_qweight_upload.argtypes = [P, C.c_int, sz, sz, u8p, sz, C.POINTER(P)]
    L.vokra_hip_qweight_free.argtypes = [P]
    L.vokra_hip_qweight_free.restype = None
    L.vokra_hip_gemm_q_f32_dev.argtypes = [P, P, sz, P, P, P, C.c_int]
    L.vokra_hip_copy_dev.argtypes = [P, P, P, sz]
    L.vokra_hip_capture_begin.argtypes = [P]
    L.vokra_hip_capture_end.argtypes = [P, C.POINTER(P)]
    L.vokra_hip_graph_launch.argtypes = [P, P]
    L.vokra_hip_graph_destroy.argtypes = [P]
    L.vokra_hip_graph_destroy.restype = None
    L.vokra_hip_quantize_bytes.argtypes = [P, C.c_int, f32p, sz, u8p, sz]
    L.vokra_hip_quantize_bytes_dev.argtypes = [P, C.c_int, P, sz, P]
    L.vokra_hip_qact_create.argtypes = [P, sz, sz, C.POINTER(P)]
    L.vokra_hip_qact_free.argtypes = [P]
    L.vokra_hip_qact_free.restype = None
    L.vokra_hip_qact_quantize_dev.argtypes = [P, P, sz, P, C.c_int]
    L.vokra_hip_gemm_qact_dev.argtypes = [P, P, P, P, P]
    L.vokra_hip_linear_group_create.argtypes = [P, sz, C.POINTER(P), C.POINTER(P), C.POINTER(P), C.POINTER(P)]
    L.vokra_hip_linear_group_run.argtypes = [P, P, P]
    L.vokra_hip_linear_group_destroy.argtypes = [P]
    L.vokra_hip_linear_group_destroy.restype = None
    i32p = C.POINTER(C.c_int32)
    L.vokra_hip_kv_create.argtypes = [P, sz, sz, sz, sz, sz, sz, C.c_int, C.POINTER(P)]
    L.vokra_hip_kv_destroy.argtypes = [P]
    L.vokra_hip_kv_destroy.restype = None
    L.vokra_hip_kv_append.argtypes = [P, P, sz, sz, i32p, i32p, f32p, f32p]
    L.vokra_hip_kv_append_dev.argtypes = [P, P, sz, sz, P, P, P, P]
    L.vokra_hip_kv_status.argtypes = [P, P, C.POINTER(sz)]
    L.vokra_hip_kv_read.argtypes = [P, P, sz, sz, sz, f32p, f32p, C.POINTER(C.c_int)]
    L.vokra_hip_kv_reset.argtypes = [P, P]
    L.vokra_hip_kv_release_layer.argtypes = [P, P, sz]
    L.vokra_hip_kv_pages.argtypes = [P, P, C.POINTER(sz), C.POINTER(sz)]
    L.vokra_hip_kv_page_of.argtypes = [P, P, sz, sz, C.POINTER(C.c_long)]
    L.vokra_hip_kv_set_free_order.argtypes = [P, P, i32p, sz]
    L.vokra_hip_paged_attn.argtypes = [P, P, sz, sz, i32p, i32p, sz, f32p, C.c_float, f32p]
    L.vokra_hip_paged_attn_dev.argtypes = [P, P, sz, sz, P, P, sz, sz, P, C.c_float, P]
    L.vokra_hip_gemm_f32.argtypes = [P, sz, sz, sz, f32p, sz, f32p, sz, f32p, f32p, sz]
    L.vokra_hip_gemm_f32_dev.argtypes = [P, sz, sz, sz, P, P, C.c_int, P, P]
    L.vokra_hip_gemv_f32.argtypes = [P, sz, sz, f32p, sz, f32p, sz, f32p, f32p, sz]
    L.vokra_hip_gemv_f32_dev.argtypes = [P, sz, sz, P, P, P, P]
    L.vokra_hip_softmax_f32.argtypes = [P, f32p, sz, f32p, sz, sz, sz]
    L.vokra_hip_layer_norm_f32.argtypes = [P, f32p, sz, f32p, sz, sz, sz, f32p, sz, f32p, sz, C.c_float]
    L.vokra_hip_rms_norm_f32.argtypes = [P, f32p, sz, f32p, sz, sz, sz, f32p, sz, C.c_float]
    L.vokra_hip_softmax_f32_dev.argtypes = [P, P, P, sz, sz]
    L.vokra_hip_layer_norm_f32_dev.argtypes = [P, P, P, sz, sz, P, P, C.c_float]
    L.vokra_hip_rms_norm_f32_dev.argtypes = [P, P, P, sz, sz, P, C.c_float]
    L.vokra_hip_gelu_f32.argtypes = [P, f32p, f32p, sz]
    L.vokra_hip_gelu_f32_dev.argtypes = [P, P, P, sz]
    L.vokra_hip_gguf_open.argtypes = [C.c_char_p, C.POINTER(P)]
    L.vokra_hip_gguf_close.argtypes = [P]
    L.vokra_hip_gguf_close.restype = None
    L.vokra_hip_gguf_tensor_count.argtypes = [P, C.POINTER(sz)]
    L.vokra_hip_gguf_tensor_info.argtypes = [P, sz, C.POINTER(C.c_char_p), C.POINTER(C.c_uint32), C.POINTER(sz),
                                             C.POINTER(C.c_uint64), C.POINTER(P), C.POINTER(sz)]
    L.vokra_hip_gguf_find.argtypes = [P, C.c_char_p, C.POINTER(sz)]
    L.vokra_hip_gguf_meta_int.argtypes = [P, C.c_char_p, C.POINTER(C.c_int64)]
    L.vokra_hip_gguf_meta_str.argtypes = [P, C.c_char_p, C.POINTER(C.c_char_p), C.POINTER(sz)]
    L.vokra_hip_gguf_upload_qweight.argtypes = [P, P, C.c_char_p, C.POINTER(P)]
    L.vokra_hip_gguf_read_f32.argtypes = [P, C.c_char_p, f32p, sz]
    L.vokra_hip_whisper_config_from_gguf.argtypes = [P, C.POINTER(WhisperConfig)]
    L.vokra_hip_voxtral_config_from_gguf.argtypes = [P, C.POINTER(VoxtralConfig)]
    L.vokra_hip_text_decoder_from_gguf.argtypes = [P, P, C.POINTER(VoxtralConfig), C.c_int, sz, sz, sz,
                                                   C.POINTER(WhisperLoadReport), C.POINTER(P)]
    L.vokra_hip_whisper_encoder_from_gguf.argtypes = [P, P, C.POINTER(WhisperConfig), C.c_int, sz,
                                                      C.POINTER(WhisperLoadReport), C.POINTER(P)]
    L.vokra_hip_whisper_decoder_from_gguf.argtypes = [P, P, C.POINTER(WhisperConfig), C.c_int, sz, sz,
                                                      C.POINTER(WhisperLoadReport), C.POINTER(P)]
    L.vokra_hip_log_mel.argtypes = [P, f32p, sz, sz, sz, f32p, sz]
    L.vokra_hip_log_mel_dev.argtypes = [P, P, sz, sz, sz, P]
    L.vokra_hip_conv1d_f32.argtypes = [P, f32p, sz, sz, sz, f32p, sz, sz, sz, f32p, sz, sz, f32p, sz]
    L.vokra_hip_conv1d_f32_dev.argtypes = [P, P, sz, sz, P, sz, sz, P, sz, sz, P]
    L.vokra_hip_encoder_set_stem.argtypes = [P, P, sz, sz, f32p, f32p, f32p, f32p, f32p]
    L.vokra_hip_encoder_encode.argtypes = [P, P, sz, f32p, f32p]
    L.vokra_hip_encoder_encode_dev.argtypes = [P, P, sz, P, P]
    L.vokra_hip_argmax_f32_dev.argtypes = [P, P, sz, sz, P]
    L.vokra_hip_logits_argmax_dev.argtypes = [P, sz, sz, sz, P, P, P, P]
    L.vokra_hip_decoder_set_cross_precision.argtypes = [P, P, C.c_int]
    L.vokra_hip_add_f32_dev.argtypes = [P, P, P, P, sz]
    L.vokra_hip_encoder_create.argtypes = [P, C.c_int, sz, sz, sz, sz, C.POINTER(PrenormLayer), f32p, f32p, sz,
                                           C.POINTER(P)]
    L.vokra_hip_encoder_destroy.argtypes = [P]
    L.vokra_hip_encoder_destroy.restype = None
    L.vokra_hip_encoder_forward.argtypes = [P, P, sz, sz, f32p, f32p]
    L.vokra_hip_encoder_forward_dev.argtypes = [P, P, sz, sz, P, P]
    L.vokra_hip_decoder_create.argtypes = [P, C.c_int, sz, sz, sz, sz, sz, sz, sz, sz, sz,
                                           C.POINTER(DecoderLayer), f32p, f32p, f32p, f32p, C.POINTER(P)]
    L.vokra_hip_decoder_destroy.argtypes = [P]
    L.vokra_hip_decoder_destroy.restype = None
    L.vokra_hip_decoder_set_encoder.argtypes = [P, P, sz, f32p]
    L.vokra_hip_decoder_set_encoder_dev.argtypes = [P, P, sz, P]
    L.vokra_hip_decoder_reset.argtypes = [P, P]
    L.vokra_hip_decoder_set_free_order.argtypes = [P, P, i32p, sz]
    L.vokra_hip_decoder_kv_pages.argtypes = [P, P, C.POINTER(sz), C.POINTER(sz)]
    L.vokra_hip_decoder_step.argtypes = [P, P, sz, i32p, i32p, i32p, i32p, f32p]
    L.vokra_hip_decoder_step_dev.argtypes = [P, P, sz, P, P, P, P, P]
    L.vokra_hip_decoder_status.argtypes = [P, P, C.POINTER(sz)]
    L.vokra_hip_attn_f32.argtypes = [P, sz, sz, sz, sz, sz, sz, f32p, f32p, f32p, C.c_float, C.c_int, sz, f32p]
    u8p = C.POINTER(C.c_uint8)
    L.vokra_hip_rope_f32.argtypes = [P, f32p, sz, sz, sz, sz, C.c_float, sz]
    L.vokra_hip_rope_f32_dev.argtypes = [P, P, sz, sz, sz, C.c_float, P]
    L.vokra_hip_swiglu_f32.argtypes = [P, f32p, sz, f32p, sz, f32p]
    L.vokra_hip_swiglu_f32_dev.argtypes = [P, P, P, sz, P]
    L.vokra_hip_text_decoder_create.argtypes = [P, C.c_int, sz, sz, sz, sz, sz, sz, sz, sz, sz, sz, C.c_float,
                                                C.c_float, C.POINTER(TextDecoderLayer), f32p, f32p, u8p,
                                                C.POINTER(P)]
    L.vokra_hip_text_decoder_destroy.argtypes = [P]
    L.vokra_hip_text_decoder_destroy.restype = None
    L.vokra_hip_text_decoder_reset.argtypes = [P, P]
    L.vokra_hip_text_decoder_set_free_order.argtypes = [P, P, i32p, sz]
    L.vokra_hip_text_decoder_kv_pages.argtypes = [P, P, C.POINTER(sz), C.POINTER(sz)]
    L.vokra_hip_text_decoder_position.argtypes = [P, P, sz, C.POINTER(sz)]
    L.vokra_hip_text_decoder_kv_restore.argtypes = [P, P, sz, sz, f32p, f32p]
    L.vokra_hip_text_decoder_step.argtypes = [P, P, sz, i32p, i32p, i32p, f32p]
    L.vokra_hip_text_decoder_step_dev.argtypes = [P, P, sz, P, P, P, P, P]
    L.vokra_hip_text_decoder_status.argtypes = [P, P, C.POINTER(sz)]
    L.vokra_hip_attn_f32_dev.argtypes = [P, sz, sz, sz, sz, sz, sz, P, P, P, C.c_float, C.c_int, sz, P]


def lib():
    """Loads libvokra_hip.so; raises BackendUnavailable if it was never built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise BackendUnavailable(
                f"{LIB_PATH} is missing: build it with `python -m vokra_amd.build` "
                "(there is no CPU fallback)")
        L = C.CDLL(LIB_PATH)
        _declare(L)
        _lib = L
    return _lib


def exported_symbols():
    """Names the C ABI exports (for the symbol test on machines without a GPU)."""
    return [n for n in dir(lib()) if n.startswith("vokra_hip_")]


def _check(code: int):
    if code != 0:
        msg = lib().vokra_hip_last_error().decode(errors="replace")
        raise _ERRORS.get(code, VokraError)(msg)


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _u8(a):
    return np.ascontiguousarray(np.frombuffer(a, np.uint8) if isinstance(a, (bytes, bytearray)) else a,
                                dtype=np.uint8)


def _ptr(a, t):
    return None if a is None else a.ctypes.data_as(C.POINTER(t))


def probe() -> int:
    n = C.c_int(0)
    _check(lib().vokra_hip_probe(C.byref(n)))
    return n.value


class DeviceBuffer:
    """A device allocation owned by a context (resident-mode plumbing)."""

    def __init__(self, ctx: "HipContext", nbytes: int):
        self.ctx = ctx
        self.nbytes = int(nbytes)
        p = C.c_void_p()
        _check(lib().vokra_hip_device_alloc(ctx._h, self.nbytes, C.byref(p)))
        self.ptr = p

    @classmethod
    def from_array(cls, ctx, arr):
        arr = np.ascontiguousarray(arr)
        buf = cls(ctx, arr.nbytes)
        buf.upload(arr)
        return buf

    def upload(self, arr):
        arr = np.ascontiguousarray(arr)
        assert arr.nbytes <= self.nbytes
        _check(lib().vokra_hip_memcpy_htod(self.ctx._h, self.ptr, arr.ctypes.data_as(C.c_void_p), arr.nbytes))

    def download(self, dtype, count):
        out = np.empty(count, dtype)
        assert out.nbytes <= self.nbytes
        _check(lib().vokra_hip_memcpy_dtoh(self.ctx._h, out.ctypes.data_as(C.c_void_p), self.ptr, out.nbytes))
        return out

    def download_at(self, dtype, offset, count):
        """count elements of dtype starting at element `offset`."""
        out = np.empty(count, dtype)
        start = int(offset) * out.itemsize
        assert start + out.nbytes <= self.nbytes
        _check(lib().vokra_hip_memcpy_dtoh(self.ctx._h, out.ctypes.data_as(C.c_void_p),
                                           C.c_void_p(self.ptr.value + start), out.nbytes))
        return out

    def free(self):
        if self.ptr:
            _check(lib().vokra_hip_device_free(self.ctx._h, self.ptr))
            self.ptr = None

    def __del__(self):
        try:
            if getattr(self, "ptr", None) and self.ctx._h:
                lib().vokra_hip_device_free(self.ctx._h, self.ptr)
        except Exception:
            pass


class Event:
    def __init__(self, ctx: "HipContext"):
        self.ctx = ctx
        p = C.c_void_p()
        _check(lib().vokra_hip_event_create(ctx._h, C.byref(p)))
        self._h = p

    def record(self):
        _check(lib().vokra_hip_event_record(self.ctx._h, self._h))

    def elapsed_ms(self, stop: "Event") -> float:
        ms = C.c_float(0.0)
        _check(lib().vokra_hip_event_elapsed_ms(self._h, stop._h, C.byref(ms)))
        return ms.value

    def __del__(self):
        try:
            if getattr(self, "_h", None) and _ctx_alive(self):
                lib().vokra_hip_event_destroy(self._h)
        except Exception:
            pass


class QWeight:
    """Device-resident quantized weight ([n, k] wire payload uploaded once)."""

    def __init__(self, ctx: "HipContext", wdtype: WDtype, n: int, k: int, wq):
        self.ctx, self.wdtype, self.n, self.k = ctx, WDtype(wdtype), int(n), int(k)
        w = _u8(wq)
        p = C.c_void_p()
        _check(lib().vokra_hip_qweight_upload(ctx._h, int(wdtype), n, k, _ptr(w, C.c_uint8), w.size,
                                              C.byref(p)))
        self._h = p

    def __del__(self):
        try:
            if getattr(self, "_h", None) and _ctx_alive(self):
                lib().vokra_hip_qweight_free(self._h)
        except Exception:
            pass


class GgufFile:
    """GgufFile (crates/vokra-core/src/gguf/reader.rs) over a read-only mapping
    held by the library. Parsing needs no GPU."""

    def __init__(self, path):
        h = C.c_void_p()
        _check(lib().vokra_hip_gguf_open(os.fsencode(path), C.byref(h)))
        self._h = h

    def close(self):
        if getattr(self, "_h", None) and self._h.value:
            lib().vokra_hip_gguf_close(self._h)
            self._h = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __len__(self):
        n = C.c_size_t()
        _check(lib().vokra_hip_gguf_tensor_count(self._h, C.byref(n)))
        return n.value

    def tensor(self, i):
        """(name, ggml type tag, dims, payload bytes) of tensor i."""
        name, t, nd, data, nb = C.c_char_p(), C.c_uint32(), C.c_size_t(), C.c_void_p(), C.c_size_t()
        dims = (C.c_uint64 * 8)()
        _check(lib().vokra_hip_gguf_tensor_info(self._h, i, C.byref(name), C.byref(t), C.byref(nd), dims,
                                                C.byref(data), C.byref(nb)))
        payload = C.string_at(data.value, nb.value) if nb.value else b""
        return name.value.decode(), t.value, [int(dims[d]) for d in range(nd.value)], payload

    def tensors(self):
        return [self.tensor(i) for i in range(len(self))]

    def find(self, name) -> int:
        i = C.c_size_t()
        _check(lib().vokra_hip_gguf_find(self._h, name.encode(), C.byref(i)))
        return i.value

    def meta_int(self, key) -> int:
        v = C.c_int64()
        _check(lib().vokra_hip_gguf_meta_int(self._h, key.encode(), C.byref(v)))
        return v.value

    def meta_str(self, key) -> str:
        p, n = C.c_char_p(), C.c_size_t()
        _check(lib().vokra_hip_gguf_meta_str(self._h, key.encode(), C.byref(p), C.byref(n)))
        return C.string_at(p, n.value).decode()

    def read_f32(self, name, n):
        out = np.zeros(max(n, 1), np.float32)
        _check(lib().vokra_hip_gguf_read_f32(self._h, name.encode(), _ptr(out, C.c_float), n))
        return out[:n]

    def upload_qweight(self, ctx, name) -> "QWeight":
        """vokra_hip_gguf_upload_qweight: the named [out, in] block-quant tensor as a resident weight."""
        p = C.c_void_p()
        _check(lib().vokra_hip_gguf_upload_qweight(ctx._h, self._h, name.encode(), C.byref(p)))
        _, t, dims, _ = self.tensor(self.find(name))
        w = QWeight.__new__(QWeight)
        w.ctx, w.wdtype, w.n, w.k, w._h = ctx, WDtype(t), dims[0], dims[1], p
        return w

    def whisper_config(self) -> dict:
        """WhisperConfig::from_gguf (whisper/config.rs:106-170); no GPU is touched."""
        c = WhisperConfig()
        _check(lib().vokra_hip_whisper_config_from_gguf(self._h, C.byref(c)))
        return {n: getattr(c, n) for n, _ in WhisperConfig._fields_}

    def voxtral_config(self) -> dict:
        """VoxtralConfig::from_gguf (voxtral/config.rs:155-267); no GPU is touched.
        head_dim is the explicit key (0 when absent); TextDecoderConfig::head_dim
        then derives hidden_dim / n_head_q."""
        c = VoxtralConfig()
        _check(lib().vokra_hip_voxtral_config_from_gguf(self._h, C.byref(c)))
        return {n: getattr(c, n) for n, _ in VoxtralConfig._fields_}


class Graph:
    """A captured sequence of device calls, replayed with one launch."""

    def __init__(self, ctx: "HipContext", handle):
        self.ctx, self._h = ctx, handle

    def launch(self):
        _check(lib().vokra_hip_graph_launch(self.ctx._h, self._h))

    def __del__(self):
        try:
            if getattr(self, "_h", None) and _ctx_alive(self):
                lib().vokra_hip_graph_destroy(self._h)
        except Exception:
            pass


class LinearGroup:
    """A fixed set of decode linears over one activation batch, run as one launch
    (vokra_hip_linear_group_*): outputs equal gemm_qact_dev of each weight."""

    def __init__(self, ctx: "HipContext", weights, d_outs, d_biases=None):
        n = len(weights)
        if len(d_outs) != n or (d_biases is not None and len(d_biases) != n):
            raise InvalidArgument("linear group: weights, outputs and biases differ in length")
        self.ctx = ctx
        self._keep = (list(weights), list(d_outs), None if d_biases is None else list(d_biases))
        ws = (C.c_void_p * n)(*[w._h for w in weights])
        outs = (C.c_void_p * n)(*[d.ptr for d in d_outs])
        bs = None if d_biases is None else (C.c_void_p * n)(*[None if b is None else b.ptr for b in d_biases])
        h = C.c_void_p()
        _check(lib().vokra_hip_linear_group_create(ctx._h, n, ws, bs, outs, C.byref(h)))
        self._h = h

    def run(self, qa: "QAct"):
        _check(lib().vokra_hip_linear_group_run(self.ctx._h, self._h, qa._h))

    def __del__(self):
        try:
            if getattr(self, "_h", None) and self._h.value and _ctx_alive(self):
                lib().vokra_hip_linear_group_destroy(self._h)
                self._h = C.c_void_p()
        except Exception:
            pass


class QAct:
    """Device-resident INT8-quantized activations (quantize once, many GEMMs)."""

    def __init__(self, ctx: "HipContext", max_m: int, k: int):
        self.ctx, self.max_m, self.k = ctx, int(max_m), int(k)
        p = C.c_void_p()
        _check(lib().vokra_hip_qact_create(ctx._h, max_m, k, C.byref(p)))
        self._h = p

    def quantize(self, m: int, d_a: "DeviceBuffer", act: "ActQuant" = None):
        act = ActQuant.AMAX127 if act is None else act
        _check(lib().vokra_hip_qact_quantize_dev(self.ctx._h, self._h, m, d_a.ptr, int(act)))

    def __del__(self):
        try:
            if getattr(self, "_h", None) and _ctx_alive(self):
                lib().vokra_hip_qact_free(self._h)
        except Exception:
            pass


class KvCache:
    """QuantizedPagedKvCache (paged_quant.rs:240-545) resident on the device."""

    def __init__(self, ctx: "HipContext", n_layer, n_head, d_head, n_stream, max_time, block_size,
                 mode: KvQuant = KvQuant.Q8_0):
        self._ctx = ctx
        self.width = n_head * d_head
        self.n_head, self.d_head = n_head, d_head
        h = C.c_void_p()
        _check(lib().vokra_hip_kv_create(ctx._h, n_layer, n_head, d_head, n_stream, max_time, block_size,
                                         int(mode), C.byref(h)))
        self._h = h

    def append(self, layer, streams, times, k_rows, v_rows):
        """append_step for each (stream, t) in order (host arrays)."""
        st = np.ascontiguousarray(streams, np.int32)
        tt = np.ascontiguousarray(times, np.int32)
        k, v = _f32(k_rows).reshape(-1), _f32(v_rows).reshape(-1)
        _check(lib().vokra_hip_kv_append(self._ctx._h, self._h, layer, st.size, _ptr(st, C.c_int32),
                                         _ptr(tt, C.c_int32), _ptr(k, C.c_float), _ptr(v, C.c_float)))

    def append_dev(self, layer, n, d_streams, d_times, d_k, d_v):
        _check(lib().vokra_hip_kv_append_dev(self._ctx._h, self._h, layer, n, d_streams.ptr, d_times.ptr,
                                             d_k.ptr, d_v.ptr))

    def status(self):
        n = C.c_size_t(0)
        _check(lib().vokra_hip_kv_status(self._ctx._h, self._h, C.byref(n)))
        return n.value

    def read(self, layer, t, s):
        """read_step: (k, v) dequantized rows, or None."""
        k = np.zeros(self.width, np.float32)
        v = np.zeros(self.width, np.float32)
        f = C.c_int(0)
        _check(lib().vokra_hip_kv_read(self._ctx._h, self._h, layer, t, s, _ptr(k, C.c_float),
                                       _ptr(v, C.c_float), C.byref(f)))
        return (k, v) if f.value else None

    def reset(self):
        _check(lib().vokra_hip_kv_reset(self._ctx._h, self._h))

    def release_layer(self, layer):
        _check(lib().vokra_hip_kv_release_layer(self._ctx._h, self._h, layer))

    def pages(self):
        fr, used = C.c_size_t(0), C.c_size_t(0)
        _check(lib().vokra_hip_kv_pages(self._ctx._h, self._h, C.byref(fr), C.byref(used)))
        return fr.value, used.value

    def page_of(self, layer, t):
        p = C.c_long(0)
        _check(lib().vokra_hip_kv_page_of(self._ctx._h, self._h, layer, t, C.byref(p)))
        return p.value

    def set_free_order(self, order):
        o = np.ascontiguousarray(order, np.int32)
        _check(lib().vokra_hip_kv_set_free_order(self._ctx._h, self._h, _ptr(o, C.c_int32), o.size))

    def attn(self, layer, streams, lens, q, n_head_q, scale):
        """Decode attention of q [n, n_head_q*d_head] over the cached keys 0..lens[i]-1."""
        st = np.ascontiguousarray(streams, np.int32)
        ln = np.ascontiguousarray(lens, np.int32)
        qv = _f32(q).reshape(st.size, -1)
        out = np.zeros_like(qv)
        _check(lib().vokra_hip_paged_attn(self._ctx._h, self._h, layer, st.size, _ptr(st, C.c_int32),
                                          _ptr(ln, C.c_int32), n_head_q, _ptr(qv, C.c_float), C.c_float(scale),
                                          _ptr(out, C.c_float)))
        return out

    def attn_dev(self, layer, n, d_streams, d_lens, max_len, n_head_q, d_q, scale, d_out):
        _check(lib().vokra_hip_paged_attn_dev(self._ctx._h, self._h, layer, n, d_streams.ptr, d_lens.ptr, max_len,
                                              n_head_q, d_q.ptr, C.c_float(scale), d_out.ptr))

    def __del__(self):
        try:
            if getattr(self, "_h", None) and self._h.value and _ctx_alive(self):
                lib().vokra_hip_kv_destroy(self._h)
                self._h = C.c_void_p()
        except Exception:
            pass


class Encoder:
    """Device-resident pre-norm encoder (compute.rs:2775 encode_prenorm_encoder)."""

    def __init__(self, ctx, wdtype, d_model, n_head, d_ff, layers, ln_post_gamma, ln_post_beta, max_rows):
        self._ctx, self.d = ctx, d_model
        keep = []
        arr = (PrenormLayer * max(len(layers), 1))(*[_fill_struct(PrenormLayer, L, keep) for L in layers])
        g, b = _f32(ln_post_gamma), _f32(ln_post_beta)
        h = C.c_void_p()
        _check(lib().vokra_hip_encoder_create(ctx._h, int(wdtype), len(layers), d_model, n_head, d_ff, arr,
                                              _ptr(g, C.c_float), _ptr(b, C.c_float), max_rows, C.byref(h)))
        self._h = h

    @classmethod
    def from_gguf(cls, ctx, gguf, wdtype, max_rows):
        """vokra_hip_whisper_encoder_from_gguf: the encoder half of WhisperWeights::load_with
        (whisper/weights.rs:302-333) as a session with its stem set. Returns (encoder, report)."""
        cfg = WhisperConfig()
        _check(lib().vokra_hip_whisper_config_from_gguf(gguf._h, C.byref(cfg)))
        rep, h = WhisperLoadReport(), C.c_void_p()
        _check(lib().vokra_hip_whisper_encoder_from_gguf(ctx._h, gguf._h, C.byref(cfg), int(wdtype), max_rows,
                                                         C.byref(rep), C.byref(h)))
        enc = cls.__new__(cls)
        enc._ctx, enc.d, enc._h = ctx, cfg.d_model, h
        enc.n_mels, enc.n_frames = cfg.n_mels, 2 * cfg.n_audio_ctx
        enc.n_ctx = (enc.n_frames - 1) // 2 + 1
        return enc, {"verbatim": rep.verbatim, "packed": rep.packed}

    def forward(self, x):
        xv = _f32(x)
        B, T, _ = xv.shape
        out = np.zeros_like(xv)
        _check(lib().vokra_hip_encoder_forward(self._ctx._h, self._h, B, T, _ptr(xv, C.c_float),
                                               _ptr(out, C.c_float)))
        return out

    def forward_dev(self, batch, frames, d_x, d_out):
        _check(lib().vokra_hip_encoder_forward_dev(self._ctx._h, self._h, batch, frames, d_x.ptr, d_out.ptr))

    def set_stem(self, n_mels, n_frames, conv1_w, conv1_b, conv2_w, conv2_b, pos_emb):
        """The conv stem of WhisperEncoder::encode (encoder.rs:58-104)."""
        keep = [_f32(a).reshape(-1) for a in (conv1_w, conv1_b, conv2_w, conv2_b, pos_emb)]
        _check(lib().vokra_hip_encoder_set_stem(self._ctx._h, self._h, n_mels, n_frames,
                                                *[_ptr(a, C.c_float) for a in keep]))
        self.n_mels, self.n_frames, self.n_ctx = n_mels, n_frames, (n_frames - 1) // 2 + 1

    def encode(self, log_mel):
        """WhisperEncoder::encode (encoder.rs:41-178): [B, n_mels, n_frames] -> [B, n_ctx, d]."""
        x = _f32(log_mel)
        x = x.reshape(-1, self.n_mels, self.n_frames)
        out = np.zeros((x.shape[0], self.n_ctx, self.d), np.float32)
        _check(lib().vokra_hip_encoder_encode(self._ctx._h, self._h, x.shape[0], _ptr(x, C.c_float),
                                              _ptr(out, C.c_float)))
        return out

    def stem_dev(self, batch, d_log_mel, d_x):
        """The conv stem alone (log-mel -> [batch, n_frames/2, d] block input)."""
        _check(lib().vokra_hip_encoder_stem_dev(self._ctx._h, self._h, batch, d_log_mel.ptr, d_x.ptr))

    def encode_dev(self, batch, d_log_mel, d_out):
        _check(lib().vokra_hip_encoder_encode_dev(self._ctx._h, self._h, batch, d_log_mel.ptr, d_out.ptr))

    def __del__(self):
        try:
            if getattr(self, "_h", None) and self._h.value and _ctx_alive(self):
                lib().vokra_hip_encoder_destroy(self._h)
                self._h = C.c_void_p()
        except Exception:
            pass


class Decoder:
    """Batched device-resident decoder step (compute.rs:2892-3139 DecoderStepSession, with a batch axis)."""

    def __init__(self, ctx, wdtype, d_model, n_head, d_ff, n_vocab, n_text_ctx, n_audio_ctx, n_stream, layers,
                 token_emb, pos_emb, ln_post_gamma, ln_post_beta, block_size=16):
        self._ctx, self.vocab, self.d, self.n_audio = ctx, n_vocab, d_model, n_audio_ctx
        keep = []
        arr = (DecoderLayer * len(layers))(*[_fill_struct(DecoderLayer, L, keep) for L in layers])
        te, pe, g, b = _f32(token_emb), _f32(pos_emb), _f32(ln_post_gamma), _f32(ln_post_beta)
        h = C.c_void_p()
        _check(lib().vokra_hip_decoder_create(ctx._h, int(wdtype), len(layers), d_model, n_head, d_ff, n_vocab,
                                              n_text_ctx, n_audio_ctx, n_stream, block_size, arr,
                                              _ptr(te, C.c_float), _ptr(pe, C.c_float), _ptr(g, C.c_float),
                                              _ptr(b, C.c_float), C.byref(h)))
        self._h = h

    @classmethod
    def from_gguf(cls, ctx, gguf, wdtype, n_stream, block_size=16):
        """vokra_hip_whisper_decoder_from_gguf: the decoder half of WhisperWeights::load_with
        (whisper/weights.rs:335-357) as a batched session. Returns (decoder, report)."""
        cfg = WhisperConfig()
        _check(lib().vokra_hip_whisper_config_from_gguf(gguf._h, C.byref(cfg)))
        rep, h = WhisperLoadReport(), C.c_void_p()
        _check(lib().vokra_hip_whisper_decoder_from_gguf(ctx._h, gguf._h, C.byref(cfg), int(wdtype), n_stream,
                                                         block_size, C.byref(rep), C.byref(h)))
        dec = cls.__new__(cls)
        dec._ctx, dec.vocab, dec.d, dec.n_audio, dec._h = ctx, cfg.n_vocab, cfg.d_model, cfg.n_audio_ctx, h
        return dec, {"verbatim": rep.verbatim, "packed": rep.packed}

    def set_encoder(self, stream, enc):
        e = _f32(enc)
        _check(lib().vokra_hip_decoder_set_encoder(self._ctx._h, self._h, stream, _ptr(e, C.c_float)))

    def set_encoder_dev(self, stream, d_enc):
        _check(lib().vokra_hip_decoder_set_encoder_dev(self._ctx._h, self._h, stream, d_enc.ptr))

    def reset(self):
        _check(lib().vokra_hip_decoder_reset(self._ctx._h, self._h))

    def kv_pages(self):
        """(free, in use) pages of the self-KV cache."""
        fr, used = C.c_size_t(0), C.c_size_t(0)
        _check(lib().vokra_hip_decoder_kv_pages(self._ctx._h, self._h, C.byref(fr), C.byref(used)))
        return fr.value, used.value

    def set_free_order(self, order):
        """Resets every stream and places later pages in `order` (a permutation of the page ids)."""
        o = np.ascontiguousarray(order, np.int32)
        _check(lib().vokra_hip_decoder_set_free_order(self._ctx._h, self._h, _ptr(o, C.c_int32), o.size))

    def step(self, streams, tokens, positions, want_logits=False):
        st = np.ascontiguousarray(streams, np.int32)
        tk = np.ascontiguousarray(tokens, np.int32)
        ps = np.ascontiguousarray(positions, np.int32)
        nxt = np.zeros(max(st.size, 1), np.int32)
        lg = np.zeros((st.size, self.vocab), np.float32) if want_logits else None
        _check(lib().vokra_hip_decoder_step(self._ctx._h, self._h, st.size, _ptr(st, C.c_int32), _ptr(tk, C.c_int32),
                                            _ptr(ps, C.c_int32), _ptr(nxt, C.c_int32), _ptr(lg, C.c_float)))
        return (nxt[:st.size], lg) if want_logits else nxt[:st.size]

    def set_cross_precision(self, precision: "CrossPrecision"):
        """CrossPrecision.F32 (default, f32-level cross-attention) or .F16 (K/V
        read as fp16: half the bytes; a performance mode)."""
        _check(lib().vokra_hip_decoder_set_cross_precision(self._ctx._h, self._h, int(precision)))

    def step_dev(self, n, d_streams, d_tokens, d_positions, d_next, d_logits=None):
        _check(lib().vokra_hip_decoder_step_dev(self._ctx._h, self._h, n, d_streams.ptr, d_tokens.ptr,
                                                d_positions.ptr, d_next.ptr,
                                                None if d_logits is None else d_logits.ptr))

    def status(self) -> int:
        """Synchronizes; raises for a failed page allocation of the last
        step, returns the (layer, item) appends done."""
        n = C.c_size_t(0)
        _check(lib().vokra_hip_decoder_status(self._ctx._h, self._h, C.byref(n)))
        return n.value

    def __del__(self):
        try:
            if getattr(self, "_h", None) and self._h.value and _ctx_alive(self):
                lib().vokra_hip_decoder_destroy(self._h)
                self._h = C.c_void_p()
        except Exception:
            pass


class TextDecoder:
    """Batched device-resident speech-LLM text decoder
    (voxtral::TextDecoderSession, text_decoder_session.rs:54-405, with a batch
    axis and the paged Q8_0 cache)."""

    def __init__(self, ctx, wdtype, d_model, n_head_q, n_head_kv, head_dim, ffn_dim, vocab, n_ctx, n_stream,
                 layers, token_emb, final_norm_gamma, lm_head=None, rope_base=1e6, rms_norm_eps=1e-5,
                 block_size=16):
        self._ctx, self.vocab, self.n_layer = ctx, vocab, len(layers)
        self.kv_hidden = n_head_kv * head_dim
        keep = []
        arr = (TextDecoderLayer * len(layers))(*[_fill_struct(TextDecoderLayer, L, keep) for L in layers])
        te, fg = _f32(token_emb), _f32(final_norm_gamma)
        lm = None if lm_head is None else _u8(lm_head)
        h = C.c_void_p()
        _check(lib().vokra_hip_text_decoder_create(ctx._h, int(wdtype), len(layers), d_model, n_head_q, n_head_kv,
                                                   head_dim, ffn_dim, vocab, n_ctx, n_stream, block_size,
                                                   C.c_float(rope_base), C.c_float(rms_norm_eps), arr,
                                                   _ptr(te, C.c_float), _ptr(fg, C.c_float), _ptr(lm, C.c_uint8),
                                                   C.byref(h)))
        self._h = h

    @classmethod
    def from_gguf(cls, ctx, gguf, wdtype, n_stream, n_ctx=0, block_size=16):
        """vokra_hip_text_decoder_from_gguf: TextDecoder::load
        (voxtral/text_decoder.rs:484-575) with VoxtralConfig::from_gguf, as a
        batched session. Returns (decoder, report)."""
        cfg = VoxtralConfig()
        _check(lib().vokra_hip_voxtral_config_from_gguf(gguf._h, C.byref(cfg)))
        rep, h = WhisperLoadReport(), C.c_void_p()
        _check(lib().vokra_hip_text_decoder_from_gguf(ctx._h, gguf._h, C.byref(cfg), int(wdtype), n_stream, n_ctx,
                                                      block_size, C.byref(rep), C.byref(h)))
        dec = cls.__new__(cls)
        hd = cfg.head_dim or cfg.hidden_dim // cfg.n_head_q
        dec._ctx, dec.vocab, dec.n_layer, dec.kv_hidden, dec._h = ctx, cfg.vocab_size, cfg.n_layer, cfg.n_head_kv * hd, h
        return dec, {"verbatim": rep.verbatim, "packed": rep.packed}

    def reset(self):
        _check(lib().vokra_hip_text_decoder_reset(self._ctx._h, self._h))

    def kv_pages(self):
        """(free, in use) pages of the paged cache."""
        fr, used = C.c_size_t(0), C.c_size_t(0)
        _check(lib().vokra_hip_text_decoder_kv_pages(self._ctx._h, self._h, C.byref(fr), C.byref(used)))
        return fr.value, used.value

    def set_free_order(self, order):
        """Resets every stream and places later pages in `order` (a permutation of the page ids)."""
        o = np.ascontiguousarray(order, np.int32)
        _check(lib().vokra_hip_text_decoder_set_free_order(self._ctx._h, self._h, _ptr(o, C.c_int32), o.size))

    def position(self, stream) -> int:
        p = C.c_size_t(0)
        _check(lib().vokra_hip_text_decoder_position(self._ctx._h, self._h, stream, C.byref(p)))
        return p.value

    def kv_restore(self, stream, k_rows, v_rows):
        """k_rows / v_rows [n_layer, n_pos, kv_hidden] become the stream's history."""
        k, v = _f32(k_rows), _f32(v_rows)
        n_pos = k.size // (self.n_layer * self.kv_hidden) if k.size else 0
        if k.size != self.n_layer * n_pos * self.kv_hidden or v.size != k.size:
            raise InvalidArgument("kv_restore: rows must be [n_layer, n_pos, kv_hidden]")
        _check(lib().vokra_hip_text_decoder_kv_restore(self._ctx._h, self._h, stream, n_pos, _ptr(k, C.c_float),
                                                       _ptr(v, C.c_float)))

    def step(self, streams, tokens, want_logits=False):
        st = np.ascontiguousarray(streams, np.int32)
        tk = np.ascontiguousarray(tokens, np.int32)
        nxt = np.zeros(max(st.size, 1), np.int32)
        lg = np.zeros((st.size, self.vocab), np.float32) if want_logits else None
        _check(lib().vokra_hip_text_decoder_step(self._ctx._h, self._h, st.size, _ptr(st, C.c_int32),
                                                 _ptr(tk, C.c_int32), _ptr(nxt, C.c_int32), _ptr(lg, C.c_float)))
        return (nxt[:st.size], lg) if want_logits else nxt[:st.size]

    def step_dev(self, n, d_streams, d_tokens, d_positions, d_next, d_logits=None):
        _check(lib().vokra_hip_text_decoder_step_dev(self._ctx._h, self._h, n, d_streams.ptr, d_tokens.ptr,
                                                     d_positions.ptr, d_next.ptr,
                                                     None if d_logits is None else d_logits.ptr))

    def status(self) -> int:
        n = C.c_size_t(0)
        _check(lib().vokra_hip_text_decoder_status(self._ctx._h, self._h, C.byref(n)))
        return n.value

    def __del__(self):
        try:
            if getattr(self, "_h", None) and self._h.value and _ctx_alive(self):
                lib().vokra_hip_text_decoder_destroy(self._h)
                self._h = C.c_void_p()
        except Exception:
            pass


class HipContext:
    """One gfx950 device + stream (mirror of CudaContext::new, context.rs:1167)."""

    def __init__(self, device: int = 0):
        p = C.c_void_p()
        _check(lib().vokra_hip_create(device, C.byref(p)))
        self._h = p

    def close(self):
        if getattr(self, "_h", None):
            lib().vokra_hip_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def synchronize(self):
        _check(lib().vokra_hip_synchronize(self._h))

    def copy_dev(self, d_dst: "DeviceBuffer", d_src: "DeviceBuffer", nbytes: int):
        _check(lib().vokra_hip_copy_dev(self._h, d_dst.ptr, d_src.ptr, nbytes))

    def capture(self, fn) -> Graph:
        """Records the device calls `fn()` makes on this context into a graph."""
        _check(lib().vokra_hip_capture_begin(self._h))
        try:
            fn()
        finally:
            g = C.c_void_p()
            code = lib().vokra_hip_capture_end(self._h, C.byref(g))
        _check(code)
        return Graph(self, g)

    # ---- kv_quant surface ------------------------------------------------
    def dequantize_bytes(self, mode: KvQuant, data) -> np.ndarray:
        """kv_quant::dequantize_bytes (kv_quant/mod.rs:307-319) on the device."""
        b = _u8(data)
        bb = KvQuant(mode).block_bytes() if int(mode) in (0, 1, 2, 3) else 1
        n_out = (b.size // bb) * 32 if bb else 0
        out = np.zeros(max(n_out, 1), np.float32)
        _check(lib().vokra_hip_dequantize_bytes(self._h, int(mode), _ptr(b, C.c_uint8), b.size,
                                                _ptr(out, C.c_float), n_out))
        return out[:n_out]

    def kquant_dequantize(self, wdtype: WDtype, data, n_elements: int) -> np.ndarray:
        """gguf::quant::dequantize (gguf/quant/mod.rs:42-63) for Q4_K on the device."""
        b = _u8(data)
        out = np.zeros(max(n_elements, 1), np.float32)
        _check(lib().vokra_hip_kquant_dequantize(self._h, int(wdtype), _ptr(b, C.c_uint8), b.size, n_elements,
                                                 _ptr(out, C.c_float)))
        return out[:n_elements]

    def quantize_bytes(self, mode: KvQuant, x) -> np.ndarray:
        """pack_matrix_to_bytes (dequant_gemm.rs:137-186) on the device: f32 -> wire blocks."""
        xv = _f32(x).reshape(-1)
        bb = KvQuant(mode).block_bytes() if int(mode) in (1, 2, 3) else 0
        n_out = xv.size // 32 * bb
        out = np.zeros(max(n_out, 1), np.uint8)
        _check(lib().vokra_hip_quantize_bytes(self._h, int(mode), _ptr(xv, C.c_float), xv.size,
                                              _ptr(out, C.c_uint8), n_out))
        return out[:n_out]

    def quantize_bytes_dev(self, mode: KvQuant, d_x: "DeviceBuffer", n: int, d_out: "DeviceBuffer"):
        _check(lib().vokra_hip_quantize_bytes_dev(self._h, int(mode), d_x.ptr, n, d_out.ptr))

    def dequant_gemv_f32(self, mode: KvQuant, blocks_bytes, n_rows: int, n_blocks_per_row: int, x):
        """CudaContext::dequant_gemv_f32 (context.rs:1686-1699)."""
        b, xv = _u8(blocks_bytes), _f32(x)
        y = np.zeros(max(n_rows, 1), np.float32)
        _check(lib().vokra_hip_dequant_gemv_f32(self._h, int(mode), _ptr(b, C.c_uint8), b.size, n_rows,
                                                n_blocks_per_row, _ptr(xv, C.c_float), xv.size,
                                                _ptr(y, C.c_float)))
        return y[:n_rows]

    def fused_dequant_gemv(self, mode, blocks_bytes, n_rows, n_blocks_per_row, x):
        """KvQuantDequantGemvOps::fused_dequant_gemv (kv_quant/gpu_ops.rs:70-80)."""
        return self.dequant_gemv_f32(mode, blocks_bytes, n_rows, n_blocks_per_row, x)

    # ---- quantized linear -------------------------------------------------
    def set_act_quant(self, act: ActQuant):
        _check(lib().vokra_hip_set_act_quant(self._h, int(act)))

    def set_decode_kernel(self, enable: bool):
        _check(lib().vokra_hip_set_decode_kernel(self._h, int(bool(enable))))

    def gemm_q_f32(self, m: int, n: int, k: int, a, wq, dtype: WDtype, bias=None, out=None):
        """Compute::gemm_q_f32 (compute.rs:943-963): out[m, n] = a[m, k] . dequant(wq[n, k])^T."""
        av, w = _f32(a), _u8(wq)
        bv = None if bias is None else _f32(bias)
        o = np.zeros(max(m * n, 1), np.float32)
        _check(lib().vokra_hip_gemm_q_f32(self._h, int(dtype), m, n, k, _ptr(av, C.c_float), av.size,
                                          _ptr(w, C.c_uint8), w.size, _ptr(bv, C.c_float),
                                          _ptr(o, C.c_float), m * n))
        res = o[: m * n].reshape(m, n)
        if out is not None:
            out[...] = res
            return out
        return res

    def upload_qweight(self, wdtype, n, k, wq) -> QWeight:
        return QWeight(self, wdtype, n, k, wq)

    def gemm_q_f32_dev(self, w: QWeight, m: int, d_a: DeviceBuffer, d_out: DeviceBuffer, d_bias=None,
                       act: ActQuant = ActQuant.AMAX127):
        """Enqueue gemm_q_f32 on device buffers against a resident weight."""
        _check(lib().vokra_hip_gemm_q_f32_dev(self._h, w._h, m, d_a.ptr,
                                              None if d_bias is None else d_bias.ptr, d_out.ptr, int(act)))

    def gemm_q_f32_dev_noalloc(self, w: QWeight, m: int, d_a: DeviceBuffer, d_out: DeviceBuffer, d_bias=None,
                               act: ActQuant = ActQuant.AMAX127):
        """gemm_q_f32_dev whose activation pass uses the library's fixed per-device
        workspace (no device allocation)."""
        _check(lib().vokra_hip_gemm_q_f32_dev_noalloc(self._h, w._h, m, d_a.ptr,
                                                      None if d_bias is None else d_bias.ptr, d_out.ptr, int(act)))

    def kv_cache(self, n_layer, n_head, d_head, n_stream, max_time, block_size, mode=KvQuant.Q8_0) -> KvCache:
        return KvCache(self, n_layer, n_head, d_head, n_stream, max_time, block_size, mode)

    def qact(self, max_m: int, k: int) -> QAct:
        return QAct(self, max_m, k)

    # ---- f32 kernels (compute.rs:901-1076) ---------------------------------
    def gemm_f32(self, m, n, k, a, b, bias=None):
        av, bv = _f32(a).reshape(-1), _f32(b).reshape(-1)
        cv = None if bias is None else _f32(bias)
        out = np.zeros(max(m * n, 1), np.float32)
        _check(lib().vokra_hip_gemm_f32(self._h, m, n, k, _ptr(av, C.c_float), av.size, _ptr(bv, C.c_float), bv.size,
                                        _ptr(cv, C.c_float), _ptr(out, C.c_float), m * n))
        return out[:m * n].reshape(m, n)

    def gemm_f32_dev(self, m, n, k, d_a, d_b, d_out, d_bias=None, b_trans=False):
        _check(lib().vokra_hip_gemm_f32_dev(self._h, m, n, k, d_a.ptr, d_b.ptr, int(bool(b_trans)),
                                            None if d_bias is None else d_bias.ptr, d_out.ptr))

    def gemv_f32(self, m, k, a, x, bias=None):
        av, xv = _f32(a).reshape(-1), _f32(x).reshape(-1)
        cv = None if bias is None else _f32(bias)
        out = np.zeros(max(m, 1), np.float32)
        _check(lib().vokra_hip_gemv_f32(self._h, m, k, _ptr(av, C.c_float), av.size, _ptr(xv, C.c_float), xv.size,
                                        _ptr(cv, C.c_float), _ptr(out, C.c_float), m))
        return out[:m]

    def gemv_f32_dev(self, m, k, d_a, d_x, d_out, d_bias=None):
        _check(lib().vokra_hip_gemv_f32_dev(self._h, m, k, d_a.ptr, d_x.ptr, None if d_bias is None else d_bias.ptr,
                                            d_out.ptr))

    def softmax_f32_dev(self, d_in, d_out, rows, cols):
        _check(lib().vokra_hip_softmax_f32_dev(self._h, d_in.ptr, d_out.ptr, rows, cols))

    def softmax_f32(self, x, rows, cols):
        xv = _f32(x).reshape(-1)
        out = np.zeros(max(xv.size, 1), np.float32)
        _check(lib().vokra_hip_softmax_f32(self._h, _ptr(xv, C.c_float), xv.size, _ptr(out, C.c_float), xv.size,
                                           rows, cols))
        return out[:xv.size].reshape(rows, cols)

    def layer_norm_f32(self, x, rows, cols, gamma, beta, eps=1e-5):
        xv, g, b = _f32(x).reshape(-1), _f32(gamma), _f32(beta)
        out = np.zeros(max(xv.size, 1), np.float32)
        _check(lib().vokra_hip_layer_norm_f32(self._h, _ptr(xv, C.c_float), xv.size, _ptr(out, C.c_float), xv.size,
                                              rows, cols, _ptr(g, C.c_float), g.size, _ptr(b, C.c_float), b.size,
                                              C.c_float(eps)))
        return out[:xv.size].reshape(rows, cols)

    def layer_norm_f32_dev(self, d_in, d_out, rows, cols, d_gamma, d_beta, eps=1e-5):
        _check(lib().vokra_hip_layer_norm_f32_dev(self._h, d_in.ptr, d_out.ptr, rows, cols, d_gamma.ptr, d_beta.ptr,
                                                  C.c_float(eps)))

    def gelu_f32_dev(self, d_x, d_out, n):
        _check(lib().vokra_hip_gelu_f32_dev(self._h, d_x.ptr, d_out.ptr, n))

    def add_f32_dev(self, d_a, d_b, d_out, n):
        """out = a + b on device (residual connections)."""
        _check(lib().vokra_hip_add_f32_dev(self._h, d_a.ptr, d_b.ptr, d_out.ptr, n))

    def rms_norm_f32(self, x, rows, cols, gamma, eps):
        xv, g = _f32(x).reshape(-1), _f32(gamma)
        out = np.zeros(max(xv.size, 1), np.float32)
        _check(lib().vokra_hip_rms_norm_f32(self._h, _ptr(xv, C.c_float), xv.size, _ptr(out, C.c_float), xv.size,
                                            rows, cols, _ptr(g, C.c_float), g.size, C.c_float(eps)))
        return out[:xv.size].reshape(rows, cols)

    def rope_f32(self, x, seq_len, n_head, head_dim, rope_base, position_offset=0):
        """rope_apply on every head of x [seq_len, n_head*head_dim]; returns the rotated copy."""
        xv = _f32(x).copy()
        _check(lib().vokra_hip_rope_f32(self._h, _ptr(xv, C.c_float), xv.size, seq_len, n_head, head_dim,
                                        C.c_float(rope_base), position_offset))
        return xv

    def rms_norm_f32_dev(self, d_in, d_out, rows, cols, d_gamma, eps):
        _check(lib().vokra_hip_rms_norm_f32_dev(self._h, d_in.ptr, d_out.ptr, rows, cols, d_gamma.ptr,
                                                C.c_float(eps)))

    def rope_f32_dev(self, d_x, rows, n_head, head_dim, rope_base, d_positions):
        _check(lib().vokra_hip_rope_f32_dev(self._h, d_x.ptr, rows, n_head, head_dim, C.c_float(rope_base),
                                            d_positions.ptr))

    def swiglu_f32_dev(self, d_gate, d_up, n, d_out):
        _check(lib().vokra_hip_swiglu_f32_dev(self._h, d_gate.ptr, d_up.ptr, n, d_out.ptr))

    def swiglu_f32(self, gate, up):
        """silu(gate) * up (silu_inplace then hadamard_inplace)."""
        g, u = _f32(gate), _f32(up)
        out = np.zeros_like(g)
        _check(lib().vokra_hip_swiglu_f32(self._h, _ptr(g, C.c_float), g.size, _ptr(u, C.c_float), u.size,
                                          _ptr(out, C.c_float)))
        return out

    def gelu_f32(self, x):
        xv = _f32(x).reshape(-1)
        out = np.zeros(max(xv.size, 1), np.float32)
        _check(lib().vokra_hip_gelu_f32(self._h, _ptr(xv, C.c_float), _ptr(out, C.c_float), xv.size))
        return out[:xv.size]

    # ---- Whisper front end ----------------------------------------------------
    def log_mel(self, pcm, n_mels: int):
        """whisper::mel::log_mel (mel.rs:123-183). pcm [n] or [batch, n] -> [n_mels, 3000] / [batch, n_mels, 3000]."""
        x = _f32(pcm)
        single = x.ndim == 1
        x2 = x.reshape(1 if single else x.shape[0], -1)
        batch, n = x2.shape
        out = np.zeros(batch * n_mels * 3000, np.float32)
        _check(lib().vokra_hip_log_mel(self._h, _ptr(x2, C.c_float) if n else None, batch, n, n_mels,
                                       _ptr(out, C.c_float), out.size))
        out = out.reshape(batch, n_mels, 3000)
        return out[0] if single else out

    def log_mel_dev(self, d_pcm, batch, n_samples, n_mels, d_out):
        _check(lib().vokra_hip_log_mel_dev(self._h, d_pcm.ptr, batch, n_samples, n_mels, d_out.ptr))

    def conv1d_f32(self, x, in_ch, in_len, w, out_ch, kernel, bias=None, stride=1, padding=0):
        """kernels::conv1d_f32 (mod.rs:583-822) -> [out_ch, out_len]."""
        xv, wv = _f32(x).reshape(-1), _f32(w).reshape(-1)
        bv = None if bias is None else _f32(bias).reshape(-1)
        out_len = (in_len + 2 * padding - kernel) // stride + 1 if stride and kernel and \
            in_len + 2 * padding >= kernel else 0
        out = np.zeros(max(out_ch * out_len, 1), np.float32)
        _check(lib().vokra_hip_conv1d_f32(self._h, _ptr(xv, C.c_float), xv.size, in_ch, in_len, _ptr(wv, C.c_float),
                                          wv.size, out_ch, kernel, _ptr(bv, C.c_float), stride, padding,
                                          _ptr(out, C.c_float), out_ch * out_len))
        return out[:out_ch * out_len].reshape(out_ch, out_len)

    def conv1d_f32_dev(self, d_x, in_ch, in_len, d_w, out_ch, kernel, d_bias, stride, padding, d_out):
        _check(lib().vokra_hip_conv1d_f32_dev(self._h, d_x.ptr, in_ch, in_len, d_w.ptr, out_ch, kernel,
                                              None if d_bias is None else d_bias.ptr, stride, padding, d_out.ptr))

    def argmax_f32_dev(self, d_logits, rows, cols, d_out):
        _check(lib().vokra_hip_argmax_f32_dev(self._h, d_logits.ptr, rows, cols, d_out.ptr))

    def logits_argmax_dev(self, rows, vocab, d, d_x, d_emb, d_logits, d_next):
        """Tied logits emb[vocab, d] . x[rows, d] and the per-row greedy argmax in
        one pass (decoder.rs:754-796 then sampler.rs:197-206); d_logits may be None."""
        _check(lib().vokra_hip_logits_argmax_dev(self._h, rows, vocab, d, d_x.ptr, d_emb.ptr,
                                                 None if d_logits is None else d_logits.ptr, d_next.ptr))

    # ---- attention ----------------------------------------------------------
    def attn_f32(self, q, k, v, n_head_q: int, n_head_kv: int = None, scale: float = None,
                 causal: bool = False, q_offset: int = 0) -> np.ndarray:
        """Fused SDPA (compute.rs:2703 attn_f32 core; nn.rs:209-325, text_decoder.rs:1302-1360).
        q: [B, Tq, Hq*hd] (or [Tq, Hq*hd]); k, v: [B, Tkv, Hkv*hd]. Returns q's shape."""
        n_head_kv = n_head_q if n_head_kv is None else n_head_kv
        qv, kv, vv = _f32(q), _f32(k), _f32(v)
        squeeze = qv.ndim == 2
        if squeeze:
            qv, kv, vv = qv[None], kv[None], vv[None]
        B, tq, wq = qv.shape
        tkv = kv.shape[1]
        hd = wq // n_head_q
        scale = float(hd) ** -0.5 if scale is None else scale
        out = np.zeros((B, tq, wq), np.float32)
        _check(lib().vokra_hip_attn_f32(self._h, B, tq, tkv, n_head_q, n_head_kv, hd, _ptr(qv, C.c_float),
                                        _ptr(kv, C.c_float), _ptr(vv, C.c_float), C.c_float(scale),
                                        int(bool(causal)), q_offset, _ptr(out, C.c_float)))
        return out[0] if squeeze else out

    def attn_f32_dev(self, batch, t_q, t_kv, n_head_q, n_head_kv, head_dim, d_q, d_k, d_v, scale, causal,
                     q_offset, d_out):
        _check(lib().vokra_hip_attn_f32_dev(self._h, batch, t_q, t_kv, n_head_q, n_head_kv, head_dim, d_q.ptr,
                                            d_k.ptr, d_v.ptr, C.c_float(scale), int(bool(causal)), q_offset,
                                            d_out.ptr))

    def gemm_qact_dev(self, w: QWeight, qa: QAct, d_out: DeviceBuffer, d_bias=None):
        _check(lib().vokra_hip_gemm_qact_dev(self._h, w._h, qa._h, None if d_bias is None else d_bias.ptr,
                                             d_out.ptr))

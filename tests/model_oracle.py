"""Encoder blocks and decoder steps composed from the oracle's restatements
(test infrastructure): the sequence of crates/vokra-models/src/whisper/
encoder.rs:180-245 and decoder.rs:413-567, with every linear through the
oracle's block-INT8 gemm_q_f32 (the definition the GPU implements bit for bit)
and the self-attention K/V through the QuantizedPagedKvCache restatement (Q8_0
rows), one stream at a time."""
import numpy as np

Q8_0_MODE = 3
LN_EPS = 1e-5


def qlin(orc, wd, x, w, n, k, b=None):
    x = np.ascontiguousarray(x, np.float32).reshape(-1, k)
    return orc.gemm_q_f32(wd, x.shape[0], n, k, x, w, b)


def ln(orc, x, g, b):
    x = np.ascontiguousarray(x, np.float32)
    rows = x.size // g.size
    return orc.layer_norm_f32(x, rows, g.size, g, b, LN_EPS).reshape(x.shape)


def encoder(orc, wd, layers, lnp_g, lnp_b, x, n_head, d_ff):
    """x [B, T, d] -> [B, T, d] (pre-norm blocks, then ln_post)."""
    B, T, d = x.shape
    hd = d // n_head
    out = np.zeros_like(x)
    for b in range(B):
        h = x[b].astype(np.float32).copy()
        for L in layers:
            xn = ln(orc, h, L["ln1_gamma"], L["ln1_beta"])
            q = qlin(orc, wd, xn, L["wq"], d, d, L.get("bq"))
            k = qlin(orc, wd, xn, L["wk"], d, d, L.get("bk"))
            v = qlin(orc, wd, xn, L["wv"], d, d, L.get("bv"))
            a = orc.sdpa_whisper(T, T, n_head, hd, q, k, v)
            h = h + qlin(orc, wd, a, L["wo"], d, d, L.get("bo"))
            xn = ln(orc, h, L["ln2_gamma"], L["ln2_beta"])
            f = orc.gelu_f32(qlin(orc, wd, xn, L["w1"], d_ff, d, L.get("b1")).reshape(-1)).reshape(T, d_ff)
            h = h + qlin(orc, wd, f, L["w2"], d, d_ff, L.get("b2"))
        out[b] = ln(orc, h, lnp_g, lnp_b)
    return out


class Decoder:
    """Per-stream greedy decoder step with a Q8_0 paged self-KV cache."""

    def __init__(self, orc, wd, layers, tok_emb, pos_emb, lnp_g, lnp_b, n_head, d_ff, n_stream, n_text, bs):
        self.orc, self.wd, self.layers = orc, wd, layers
        self.tok_emb, self.pos_emb, self.lnp = tok_emb, pos_emb, (lnp_g, lnp_b)
        self.d = tok_emb.shape[1]
        self.n_head, self.hd, self.d_ff = n_head, self.d // n_head, d_ff
        self.cache = orc.PagedCache(len(layers), n_head, self.hd, n_stream, n_text, bs, Q8_0_MODE)
        self.cross = {}

    def set_encoder(self, s, enc):
        o, d = self.orc, self.d
        self.cross[s] = [(qlin(o, self.wd, enc, L["cwk"], d, d, L.get("cbk")),
                          qlin(o, self.wd, enc, L["cwv"], d, d, L.get("cbv"))) for L in self.layers]

    def step(self, s, token, pos):
        o, d, wd, H, hd = self.orc, self.d, self.wd, self.n_head, self.hd
        h = (self.tok_emb[token] + self.pos_emb[pos]).astype(np.float32)[None]
        for li, L in enumerate(self.layers):
            xn = ln(o, h, L["ln1_gamma"], L["ln1_beta"])
            q = qlin(o, wd, xn, L["wq"], d, d, L.get("bq"))
            k = qlin(o, wd, xn, L["wk"], d, d, L.get("bk"))
            v = qlin(o, wd, xn, L["wv"], d, d, L.get("bv"))
            assert self.cache.append_step(li, pos, s, k[0], v[0]) == 0
            rows = [self.cache.read_step(li, t, s) for t in range(pos + 1)]
            K = np.stack([r[0] for r in rows])
            V = np.stack([r[1] for r in rows])
            a = o.sdpa_whisper(1, pos + 1, H, hd, q, K, V, causal=True, q_pos_offset=pos)
            h = h + qlin(o, wd, a, L["wo"], d, d, L.get("bo"))
            xn = ln(o, h, L["ln2_gamma"], L["ln2_beta"])
            cq = qlin(o, wd, xn, L["cwq"], d, d, L.get("cbq"))
            CK, CV = self.cross[s][li]
            a = o.sdpa_whisper(1, CK.shape[0], H, hd, cq, CK, CV)
            h = h + qlin(o, wd, a, L["cwo"], d, d, L.get("cbo"))
            xn = ln(o, h, L["ln3_gamma"], L["ln3_beta"])
            f = o.gelu_f32(qlin(o, wd, xn, L["w1"], self.d_ff, d, L.get("b1")).reshape(-1))
            h = h + qlin(o, wd, f, L["w2"], d, self.d_ff, L.get("b2"))
        xn = ln(o, h, *self.lnp)
        logits = o.gemv_f32(self.tok_emb.shape[0], d, self.tok_emb, xn[0])
        return logits, o.argmax(logits)


W_Q4_K = 12


def quantize_weight(orc, wd, w):
    """Wire bytes of an f32 weight [n, k]: Q4_K through the oracle's
    quantize.rs restatement, the 32-element block formats through
    pack_matrix_to_bytes (one row of blocks per output feature)."""
    n, k = w.shape
    if wd == W_Q4_K:
        return orc.kquant_quantize(W_Q4_K, np.ascontiguousarray(w, np.float32).reshape(-1))
    if wd in (13, 14):   # Q5_K / Q6_K: the tests' quantizer (the reference ships none)
        from tests.helpers import quantize_kquant_test
        return quantize_kquant_test(w, wd)
    return orc.pack_matrix_to_bytes(orc.KV_OF_W[wd], np.ascontiguousarray(w, np.float32), n, k // 32)


def random_text_layer(orc, g, d, hq, hkv, hd, ff, scale=0.05, wd=W_Q4_K):
    """One speech-LLM block with linears of weight dtype wd (Q4_K by default)
    quantized by the oracle, norms near one."""
    L = {"attn_norm_gamma": (1 + 0.1 * g.standard_normal(d)).astype(np.float32),
         "ffn_norm_gamma": (1 + 0.1 * g.standard_normal(d)).astype(np.float32)}
    for name, n, k in (("wq", hq * hd, d), ("wk", hkv * hd, d), ("wv", hkv * hd, d), ("wo", d, hq * hd),
                       ("w_gate", ff, d), ("w_up", ff, d), ("w_down", d, ff)):
        L[name] = quantize_weight(orc, wd, (g.standard_normal((n, k)) * scale).astype(np.float32))
    return L


class TextDecoder:
    """Per-stream speech-LLM decode step: the sequence of
    crates/vokra-models/src/voxtral/text_decoder.rs:1147-1420 (RMSNorm, q/k/v,
    RoPE per head at the stream's position, GQA over the cache with the scale
    after the dot, o-proj + residual, RMSNorm, SwiGLU FFN + residual, final
    RMSNorm, LM head), every linear through the oracle's gemm_q_f32 (Q4_K:
    kquant_gemm_i8; block formats: the block-INT8 GEMM) and the K/V through
    the QuantizedPagedKvCache restatement (Q8_0 rows). lm_head: wire bytes
    [vocab, d] of the layers' dtype wd, or None for the f32 token embedding
    (tied)."""

    def __init__(self, orc, layers, tok_emb, final_gamma, lm_head, hq, hkv, hd, ff, n_stream, n_ctx, bs,
                 rope_base, eps, wd=W_Q4_K):
        self.orc, self.layers, self.tok_emb, self.final_gamma, self.lm_head = orc, layers, tok_emb, final_gamma, lm_head
        self.wd = wd
        self.d = tok_emb.shape[1]
        self.hq, self.hkv, self.hd, self.ff = hq, hkv, hd, ff
        self.rope_base, self.eps = rope_base, eps
        self.scale = np.float32(1.0) / np.sqrt(np.float32(hd))   # 1 / (hd as f32).sqrt()
        self.cache = orc.PagedCache(len(layers), hkv, hd, n_stream, n_ctx, bs, Q8_0_MODE)

    def restore(self, s, k_rows, v_rows):
        """Appends history rows [n_layer][n_pos][kv_hidden] for stream s."""
        for li in range(len(self.layers)):
            for t in range(k_rows.shape[1]):
                assert self.cache.append_step(li, t, s, k_rows[li, t], v_rows[li, t]) == 0

    def lin(self, x, w, n, k):
        return qlin(self.orc, self.wd, x, w, n, k)

    def step(self, s, token, pos):
        o, d, hq, hkv, hd, ff = self.orc, self.d, self.hq, self.hkv, self.hd, self.ff
        h = self.tok_emb[token].astype(np.float32)[None].copy()
        for li, L in enumerate(self.layers):
            x = o.rms_norm_f32(h, L["attn_norm_gamma"], self.eps, 1, d)
            q = o.rope_heads(self.lin(x, L["wq"], hq * hd, d), hq, hd, self.rope_base, pos)
            k = o.rope_heads(self.lin(x, L["wk"], hkv * hd, d), hkv, hd, self.rope_base, pos)
            v = self.lin(x, L["wv"], hkv * hd, d)
            assert self.cache.append_step(li, pos, s, k[0], v[0]) == 0
            rows = [self.cache.read_step(li, t, s) for t in range(pos + 1)]
            K = np.stack([r[0] for r in rows])
            V = np.stack([r[1] for r in rows])
            a = o.gqa_attention(1, pos + 1, hq, hkv, hd, q, K, V, float(self.scale), pos)
            h = h + self.lin(a, L["wo"], d, hq * hd)
            x = o.rms_norm_f32(h, L["ffn_norm_gamma"], self.eps, 1, d)
            f = o.swiglu(self.lin(x, L["w_gate"], ff, d), self.lin(x, L["w_up"], ff, d))
            h = h + self.lin(f, L["w_down"], d, ff)
        x = o.rms_norm_f32(h, self.final_gamma, self.eps, 1, d)
        if self.lm_head is None:
            logits = o.gemv_f32(self.tok_emb.shape[0], d, self.tok_emb, x[0])
        else:
            logits = self.lin(x, self.lm_head, self.tok_emb.shape[0], d)[0]
        return logits, o.argmax(logits)

"""Whisper sessions built straight from a GGUF file
(vokra_hip_whisper_{encoder,decoder}_from_gguf, the route of
crates/vokra-models/src/whisper/weights.rs:302-378).

The file is written by the test's own GGUF writer with the reference's tensor
names and PyTorch-order shapes. Bars:
  * the loaded sessions equal, bit for bit, sessions built directly from the
    same arrays with each name given its role by the test (log-mel -> encode,
    and decoder steps with logits), so a name bound to the wrong role, a
    transposed weight or a misread F16 fails;
  * the loaded encoder's blocks and decoder's greedy tokens against the oracle
    composition (tests/model_oracle.py) at the session tests' bar;
  * the reference's load errors: a missing tensor, a wrong shape, a Linear in
    another block dtype, naming the tensor.
"""
import numpy as np
import pytest

from tests import gguf_writer as gw
from tests import model_oracle
from vokra_amd import hip

pytestmark = pytest.mark.gpu

W_Q8_0, W_Q4_K = 8, 12
CFG = dict(n_mels=16, n_audio_ctx=32, n_audio_state=256, n_audio_head=4, n_audio_layer=2, n_text_ctx=24,
           n_text_state=256, n_text_head=4, n_text_layer=2, n_vocab=300, ffn_dim=512, eot=299)


@pytest.fixture(scope="module")
def ctx():
    c = hip.HipContext(0)
    yield c
    c.close()


def metadata(cfg=CFG):
    m = [(f"vokra.whisper.{k}", gw.U32, v) for k, v in cfg.items()]
    return m + [("vokra.whisper.decoder_start_ids", gw.ARRAY, (gw.U32, [298, 297]))]


class Model:
    """Random Whisper weights by reference tensor name (f32 truths) and the
    on-disk tensors: norms / biases / embeddings as F32 or F16, Linears as
    `lin` (a block or K-quant format stored verbatim, or "f16" / "bf16",
    packed at load into Q8_0)."""

    def __init__(self, ctx, oracle, lin, cfg=CFG):
        self.cfg, self.lin, self.t, self.disk = cfg, lin, {}, []
        d, ff, mels = cfg["n_audio_state"], cfg["ffn_dim"], cfg["n_mels"]
        self.ctx, self.oracle = ctx, oracle
        self.dense("model.encoder.conv1.weight", (d, mels, 3), 0.2)
        self.dense("model.encoder.conv1.bias", (d,), 0.05)
        self.dense("model.encoder.conv2.weight", (d, d, 3), 0.05)
        self.dense("model.encoder.conv2.bias", (d,), 0.05)
        self.dense("model.encoder.embed_positions.weight", (cfg["n_audio_ctx"], d), 0.1, f16=True)
        for i in range(cfg["n_audio_layer"]):
            p = f"model.encoder.layers.{i}"
            self.norm(f"{p}.self_attn_layer_norm", d)
            self.attention(f"{p}.self_attn", d)
            self.norm(f"{p}.final_layer_norm", d)
            self.linear(f"{p}.fc1", d, ff)
            self.linear(f"{p}.fc2", ff, d)
        self.norm("model.encoder.layer_norm", d)
        self.dense("model.decoder.embed_tokens.weight", (cfg["n_vocab"], d), 0.5)
        self.dense("model.decoder.embed_positions.weight", (cfg["n_text_ctx"], d), 0.1)
        for i in range(cfg["n_text_layer"]):
            p = f"model.decoder.layers.{i}"
            self.norm(f"{p}.self_attn_layer_norm", d)
            self.attention(f"{p}.self_attn", d)
            self.norm(f"{p}.encoder_attn_layer_norm", d)
            self.attention(f"{p}.encoder_attn", d)
            self.norm(f"{p}.final_layer_norm", d, f16=True)
            self.linear(f"{p}.fc1", d, ff)
            self.linear(f"{p}.fc2", ff, d)
        self.norm("model.decoder.layer_norm", d)

    def rng(self):
        return np.random.default_rng(len(self.disk) * 7919 + 17)

    def dense(self, name, shape, scale, f16=False):
        a = (self.rng().standard_normal(shape) * scale).astype(np.float32)
        if f16:
            a = a.astype(np.float16)
            self.disk.append((name, list(shape), gw.GGML_F16, a.tobytes()))
            a = a.astype(np.float32)
        else:
            self.disk.append((name, list(shape), gw.GGML_F32, a.tobytes()))
        self.t[name] = a

    def norm(self, p, d, f16=False):
        r = self.rng()
        gm = (1.0 + 0.1 * r.standard_normal(d)).astype(np.float32)
        bt = (0.1 * r.standard_normal(d)).astype(np.float32)
        for name, a in ((f"{p}.weight", gm), (f"{p}.bias", bt)):
            if f16:
                a = a.astype(np.float16)
                self.disk.append((name, [d], gw.GGML_F16, a.tobytes()))
                a = a.astype(np.float32)
            else:
                self.disk.append((name, [d], gw.GGML_F32, a.tobytes()))
            self.t[name] = a

    BLOCK = {"q8_0": (hip.KvQuant.Q8_0, gw.GGML_Q8_0), "q4_0": (hip.KvQuant.Q4_0, gw.GGML_Q4_0),
             "q5_0": (hip.KvQuant.Q5_0, gw.GGML_Q5_0)}
    KQUANT = {"q4_k": (W_Q4_K, gw.GGML_Q4_K), "q5_k": (13, gw.GGML_Q5_K), "q6_k": (14, gw.GGML_Q6_K)}
    WD = {"q8_0": W_Q8_0, "q4_0": 2, "q5_0": 6, "q4_k": W_Q4_K, "q5_k": 13, "q6_k": 14, "f16": W_Q8_0, "bf16": W_Q8_0}

    def linear(self, p, n_in, n_out, bias=True):
        if bias:
            self.dense(f"{p}.bias", (n_out,), 0.05)
        w = (self.rng().standard_normal((n_out, n_in)) * 0.08).astype(np.float32)
        name = f"{p}.weight"
        if self.lin in self.BLOCK:
            mode, tag = self.BLOCK[self.lin]
            wire = self.ctx.quantize_bytes(mode, w)
            self.disk.append((name, [n_out, n_in], tag, bytes(wire)))
        elif self.lin in self.KQUANT:
            wd, tag = self.KQUANT[self.lin]
            wire = model_oracle.quantize_weight(self.oracle, wd, w)
            self.disk.append((name, [n_out, n_in], tag, bytes(np.asarray(wire, np.uint8))))
        elif self.lin == "bf16":  # BF16 on disk (truncated f32 bits); packed at load as F16 is
            bits = (w.view(np.uint32) >> 16).astype(np.uint16)
            self.disk.append((name, [n_out, n_in], gw.GGML_BF16, bits.tobytes()))
            wire = self.ctx.quantize_bytes(hip.KvQuant.Q8_0, (bits.astype(np.uint32) << 16).view(np.float32))
        else:  # F16 on disk; the loader packs what F16 decodes to
            w16 = w.astype(np.float16)
            self.disk.append((name, [n_out, n_in], gw.GGML_F16, w16.tobytes()))
            wire = self.ctx.quantize_bytes(hip.KvQuant.Q8_0, w16.astype(np.float32))
        self.t[name] = np.asarray(wire, np.uint8)

    def attention(self, p, d):
        self.linear(f"{p}.q_proj", d, d)
        self.linear(f"{p}.k_proj", d, d, bias=False)
        self.linear(f"{p}.v_proj", d, d)
        self.linear(f"{p}.out_proj", d, d)

    @property
    def wd(self):
        return self.WD[self.lin]

    def write(self, path, drop=None, replace=None):
        tensors = [t for t in self.disk if t[0] != drop]
        if replace:
            tensors = [replace.get(t[0], t) for t in tensors]
        path.write_bytes(gw.build(metadata(self.cfg), tensors, alignment=64))
        return hip.GgufFile(str(path))

    # each name given its role, as weights.rs:312-356 binds them
    def enc_layers(self):
        out = []
        for i in range(self.cfg["n_audio_layer"]):
            p, t = f"model.encoder.layers.{i}", self.t
            out.append(dict(
                ln1_gamma=t[f"{p}.self_attn_layer_norm.weight"], ln1_beta=t[f"{p}.self_attn_layer_norm.bias"],
                wq=t[f"{p}.self_attn.q_proj.weight"], wk=t[f"{p}.self_attn.k_proj.weight"],
                wv=t[f"{p}.self_attn.v_proj.weight"], wo=t[f"{p}.self_attn.out_proj.weight"],
                bq=t[f"{p}.self_attn.q_proj.bias"], bv=t[f"{p}.self_attn.v_proj.bias"],
                bo=t[f"{p}.self_attn.out_proj.bias"],
                ln2_gamma=t[f"{p}.final_layer_norm.weight"], ln2_beta=t[f"{p}.final_layer_norm.bias"],
                w1=t[f"{p}.fc1.weight"], w2=t[f"{p}.fc2.weight"], b1=t[f"{p}.fc1.bias"], b2=t[f"{p}.fc2.bias"]))
        return out

    def dec_layers(self):
        out = []
        for i in range(self.cfg["n_text_layer"]):
            p, t = f"model.decoder.layers.{i}", self.t
            a, c = f"{p}.self_attn", f"{p}.encoder_attn"
            out.append(dict(
                ln1_gamma=t[f"{p}.self_attn_layer_norm.weight"], ln1_beta=t[f"{p}.self_attn_layer_norm.bias"],
                wq=t[f"{a}.q_proj.weight"], wk=t[f"{a}.k_proj.weight"], wv=t[f"{a}.v_proj.weight"],
                wo=t[f"{a}.out_proj.weight"], bq=t[f"{a}.q_proj.bias"], bv=t[f"{a}.v_proj.bias"],
                bo=t[f"{a}.out_proj.bias"],
                ln2_gamma=t[f"{p}.encoder_attn_layer_norm.weight"], ln2_beta=t[f"{p}.encoder_attn_layer_norm.bias"],
                cwq=t[f"{c}.q_proj.weight"], cwk=t[f"{c}.k_proj.weight"], cwv=t[f"{c}.v_proj.weight"],
                cwo=t[f"{c}.out_proj.weight"], cbq=t[f"{c}.q_proj.bias"], cbv=t[f"{c}.v_proj.bias"],
                cbo=t[f"{c}.out_proj.bias"],
                ln3_gamma=t[f"{p}.final_layer_norm.weight"], ln3_beta=t[f"{p}.final_layer_norm.bias"],
                w1=t[f"{p}.fc1.weight"], w2=t[f"{p}.fc2.weight"], b1=t[f"{p}.fc1.bias"], b2=t[f"{p}.fc2.bias"]))
        return out


def within(got, want, frac=0.1):
    rms = float(np.sqrt(np.mean(np.asarray(want, np.float64) ** 2)))
    err = float(np.max(np.abs(np.asarray(got, np.float64) - want)))
    return err <= frac * rms + 1e-4, err, rms


@pytest.mark.parametrize("lin", ["q8_0", "f16", "q4_k", "q4_0", "q5_0", "q5_k", "q6_k", "bf16"])
def test_sessions_from_gguf_equal_direct_construction(ctx, oracle, tmp_path, lin):
    print(f"[case] whisper gguf sessions, linears {lin}", flush=True)
    cfg = CFG
    m = Model(ctx, oracle, lin)
    f = m.write(tmp_path / "whisper.gguf")
    d, H, ff, t = cfg["n_audio_state"], cfg["n_audio_head"], cfg["ffn_dim"], m.t
    n_lin = 6 * cfg["n_audio_layer"]
    B, n_frames = 2, 2 * cfg["n_audio_ctx"]

    enc, rep = hip.Encoder.from_gguf(ctx, f, m.wd, max_rows=B * cfg["n_audio_ctx"])
    assert rep == ({"verbatim": 0, "packed": n_lin} if lin in ("f16", "bf16") else {"verbatim": n_lin, "packed": 0})
    direct = hip.Encoder(ctx, m.wd, d, H, ff, m.enc_layers(), t["model.encoder.layer_norm.weight"],
                         t["model.encoder.layer_norm.bias"], max_rows=B * cfg["n_audio_ctx"])
    direct.set_stem(cfg["n_mels"], n_frames, t["model.encoder.conv1.weight"], t["model.encoder.conv1.bias"],
                    t["model.encoder.conv2.weight"], t["model.encoder.conv2.bias"],
                    t["model.encoder.embed_positions.weight"])
    mel = np.random.default_rng(11).standard_normal((B, cfg["n_mels"], n_frames)).astype(np.float32)
    got = enc.encode(mel)
    assert np.array_equal(got, direct.encode(mel))
    # blocks of the loaded session against the oracle composition
    x = np.random.default_rng(12).standard_normal((1, cfg["n_audio_ctx"], d)).astype(np.float32)
    want = model_oracle.encoder(oracle, m.wd, m.enc_layers(), t["model.encoder.layer_norm.weight"],
                                t["model.encoder.layer_norm.bias"], x, H, ff)
    ok, err, rms = within(enc.forward(x), want)
    assert ok, (err, rms)

    n_stream, bs = 3, 4
    dec, rep = hip.Decoder.from_gguf(ctx, f, m.wd, n_stream, block_size=bs)
    assert sum(rep.values()) == 10 * cfg["n_text_layer"]
    tok, pos = t["model.decoder.embed_tokens.weight"], t["model.decoder.embed_positions.weight"]
    lpg, lpb = t["model.decoder.layer_norm.weight"], t["model.decoder.layer_norm.bias"]
    ddir = hip.Decoder(ctx, m.wd, d, cfg["n_text_head"], ff, cfg["n_vocab"], cfg["n_text_ctx"], cfg["n_audio_ctx"],
                       n_stream, m.dec_layers(), tok, pos, lpg, lpb, block_size=bs)
    ref = model_oracle.Decoder(oracle, m.wd, m.dec_layers(), tok, pos, lpg, lpb, cfg["n_text_head"], ff, n_stream,
                               cfg["n_text_ctx"], bs)
    for s in range(n_stream):
        dec.set_encoder(s, got[s % B])
        ddir.set_encoder(s, got[s % B])
        ref.set_encoder(s, got[s % B])
    tokens = np.array([298, 298, 298], np.int32)
    for p in range(6):
        nxt, lg = dec.step(np.arange(n_stream), tokens, np.full(n_stream, p), want_logits=True)
        nxt2, lg2 = ddir.step(np.arange(n_stream), tokens, np.full(n_stream, p), want_logits=True)
        assert np.array_equal(lg, lg2) and np.array_equal(nxt, nxt2), p
        for s in range(n_stream):
            want_lg, _ = ref.step(s, int(tokens[s]), p)
            ok, err, rms = within(lg[s], want_lg)
            assert ok, (p, s, err, rms)
        tokens = nxt.astype(np.int32)


def test_load_errors_name_the_tensor(ctx, oracle, tmp_path):
    print("[case] whisper gguf load errors", flush=True)
    m = Model(ctx, oracle, "q8_0")
    d, ff = CFG["n_audio_state"], CFG["ffn_dim"]
    name = "model.encoder.layers.1.fc2.bias"
    with pytest.raises(hip.ModelLoad, match=f"whisper weight `{name}`: missing from GGUF"):
        hip.Encoder.from_gguf(ctx, m.write(tmp_path / "a.gguf", drop=name), W_Q8_0, max_rows=64)
    # a transposed fc1 weight: [in, out] on disk
    w = "model.decoder.layers.0.fc1.weight"
    _, dims, gt, payload = next(t for t in m.disk if t[0] == w)
    bad = {w: (w, [d, ff], gt, payload)}
    with pytest.raises(hip.ModelLoad, match=rf"whisper weight `{w}`: shape \[{d}, {ff}\] != expected \[{ff}, {d}\]"):
        hip.Decoder.from_gguf(ctx, m.write(tmp_path / "b.gguf", replace=bad), W_Q8_0, 2)
    # Q8_0 on disk, the session asked for Q4_K; F16 on disk cannot become Q4_K
    with pytest.raises(hip.UnsupportedOp, match="Q8_0 on disk"):
        hip.Encoder.from_gguf(ctx, m.write(tmp_path / "c.gguf"), W_Q4_K, max_rows=64)
    m16 = Model(ctx, oracle, "f16")
    with pytest.raises(hip.UnsupportedOp, match="F16 on disk"):
        hip.Decoder.from_gguf(ctx, m16.write(tmp_path / "d.gguf"), W_Q4_K, 2)
    # Q4_K Linears whose rows straddle super-blocks (in_features 384, a
    # d_model-384 model): the reference keeps such a tensor on its f32
    # dequant path and counts it (weights.rs:471-512,
    # report.dequantized_unaligned); these sessions hold no f32 Linear, so
    # the load stops at the first one, naming it
    cfg384 = dict(CFG, n_audio_state=384, n_text_state=384, n_audio_head=6, n_text_head=6, ffn_dim=768)
    m384 = Model(ctx, oracle, "q4_k", cfg=cfg384)
    f384 = m384.write(tmp_path / "e.gguf")
    for build in (lambda: hip.Encoder.from_gguf(ctx, f384, W_Q4_K, max_rows=64),
                  lambda: hip.Decoder.from_gguf(ctx, f384, W_Q4_K, 2)):
        with pytest.raises(hip.UnsupportedOp,
                           match=r"whisper weight `model\.(en|de)coder\.layers\.0\.[a-z_.]+\.weight`: in_features 384 "
                                 r"is not a multiple of 256"):
            build()

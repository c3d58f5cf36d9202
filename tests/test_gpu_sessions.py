"""GPU parity of the device-resident encoder and batched decoder-step sessions.

Two bars:
  * exact composition: an encoder forward is bit-identical to the same kernels
    issued one entry point at a time (each covered by its own parity tests);
    a batched decoder step is bit-identical to stepping the same streams one at
    a time (every kernel on the path is row-independent);
  * against the oracle composition (tests/model_oracle.py), which runs the same
    INT8 linears on inputs that differ only by f32 rounding in LayerNorm, GELU
    and attention: where one activation sits within an ulp of an INT8 rounding
    boundary the two quantize one step apart, and that step then spreads
    through later layers. Bar: max |gpu - oracle| <= 0.1 * rms(oracle), and
    greedy tokens agree wherever the oracle's top-2 logit gap exceeds that.
"""
import numpy as np
import pytest

from tests import model_oracle
from vokra_amd import hip

pytestmark = pytest.mark.gpu

W_Q4_0, W_Q8_0, W_Q4_K = 2, 8, 12
W_Q5_0, W_Q5_K, W_Q6_K = 6, 13, 14


@pytest.fixture(scope="module")
def ctx():
    c = hip.HipContext(0)
    yield c
    c.close()


def pack(ctx, wd, w):
    """f32 [n, k] -> wire bytes of `wd` (device packer; Q4_K via the oracle
    quantizer; Q5_0, Q5_K and Q6_K as the oracle composition packs them)."""
    from oracle import oracle as orc
    if wd == W_Q4_K:
        return orc.kquant_quantize(W_Q4_K, w.reshape(-1))
    if wd in (W_Q5_0, W_Q5_K, W_Q6_K):
        return model_oracle.quantize_weight(orc, wd, w)
    mode = {W_Q4_0: hip.KvQuant.Q4_0, W_Q8_0: hip.KvQuant.Q8_0}[wd]
    return ctx.quantize_bytes(mode, w)


def rand_norm(g, d):
    return (1.0 + 0.1 * g.standard_normal(d)).astype(np.float32), (0.1 * g.standard_normal(d)).astype(np.float32)


def enc_layer(ctx, g, wd, d, ff, scale=0.08):
    L = {}
    L["ln1_gamma"], L["ln1_beta"] = rand_norm(g, d)
    L["ln2_gamma"], L["ln2_beta"] = rand_norm(g, d)
    for name, n, k in (("wq", d, d), ("wk", d, d), ("wv", d, d), ("wo", d, d), ("w1", ff, d), ("w2", d, ff)):
        L[name] = pack(ctx, wd, (g.standard_normal((n, k)) * scale).astype(np.float32))
    for name, n in (("bq", d), ("bv", d), ("bo", d), ("b1", ff), ("b2", d)):
        L[name] = (0.05 * g.standard_normal(n)).astype(np.float32)
    return L  # no bk: Whisper's k projection has no bias


def within(got, want, frac=0.1):
    rms = float(np.sqrt(np.mean(np.asarray(want, np.float64) ** 2)))
    err = float(np.max(np.abs(np.asarray(got, np.float64) - want)))
    return err <= frac * rms + 1e-4, err, rms


def encoder_by_ops(ctx, wd, layers, lpg, lpb, x, H, ff):
    """The encoder forward issued one C-ABI entry point at a time."""
    W = hip.WDtype(wd)
    B, T, d = x.shape
    h = x.reshape(B * T, d).copy()
    for L in layers:
        xn = ctx.layer_norm_f32(h, B * T, d, L["ln1_gamma"], L["ln1_beta"])
        q, k, v = (ctx.gemm_q_f32(B * T, d, d, xn, L[w], W, bias=L.get(b)).reshape(B, T, d)
                   for w, b in (("wq", "bq"), ("wk", "bk"), ("wv", "bv")))
        a = ctx.attn_f32(q, k, v, H).reshape(B * T, d)
        h = ctx.gemm_q_f32(B * T, d, d, a, L["wo"], W, bias=L.get("bo")) + h
        xn = ctx.layer_norm_f32(h, B * T, d, L["ln2_gamma"], L["ln2_beta"])
        f = ctx.gelu_f32(ctx.gemm_q_f32(B * T, ff, d, xn, L["w1"], W, bias=L.get("b1"))).reshape(B * T, ff)
        h = ctx.gemm_q_f32(B * T, d, ff, f, L["w2"], W, bias=L.get("b2")) + h
    return ctx.layer_norm_f32(h, B * T, d, lpg, lpb).reshape(B, T, d)


@pytest.mark.parametrize("wd,d,H,ff,T,B", [(W_Q8_0, 128, 2, 256, 70, 2), (W_Q4_0, 128, 2, 256, 64, 1),
                                           (W_Q4_K, 256, 4, 512, 33, 1), (W_Q5_0, 128, 2, 256, 40, 1),
                                           (W_Q5_K, 256, 4, 512, 33, 1), (W_Q6_K, 256, 4, 512, 33, 1)])
def test_encoder_vs_oracle(ctx, oracle, wd, d, H, ff, T, B):
    print(f"[case] encoder wd={wd} d={d} H={H} T={T} B={B}", flush=True)
    g = np.random.default_rng(d + T + wd)
    layers = [enc_layer(ctx, g, wd, d, ff) for _ in range(2)]
    lpg, lpb = rand_norm(g, d)
    x = g.standard_normal((B, T, d)).astype(np.float32)
    enc = hip.Encoder(ctx, wd, d, H, ff, layers, lpg, lpb, max_rows=B * T)
    got = enc.forward(x)
    assert np.array_equal(got, encoder_by_ops(ctx, wd, layers, lpg, lpb, x, H, ff))
    if B > 1:  # batch invariance
        assert np.array_equal(got[1:2], enc.forward(x[1:2]))
    want = model_oracle.encoder(oracle, wd, layers, lpg, lpb, x, H, ff)
    ok, err, rms = within(got, want)
    assert ok, (err, rms)


def test_encoder_config0_layer_full_length(ctx, oracle):
    """Whisper-base dims (d=512, 8 heads, FFN 2048), 1500 frames, one block."""
    print("[case] encoder config0 one layer T=1500", flush=True)
    d, H, ff, T = 512, 8, 2048, 1500
    g = np.random.default_rng(1500)
    layers = [enc_layer(ctx, g, W_Q8_0, d, ff, scale=0.02)]
    lpg, lpb = rand_norm(g, d)
    x = g.standard_normal((1, T, d)).astype(np.float32)
    enc = hip.Encoder(ctx, W_Q8_0, d, H, ff, layers, lpg, lpb, max_rows=T)
    got = enc.forward(x)
    want = model_oracle.encoder(oracle, W_Q8_0, layers, lpg, lpb, x, H, ff)
    ok, err, rms = within(got, want)
    assert ok, (err, rms)


def dec_layer(ctx, g, wd, d, ff, scale=0.08):
    L = enc_layer(ctx, g, wd, d, ff, scale)
    L["ln3_gamma"], L["ln3_beta"] = rand_norm(g, d)
    for name in ("cwq", "cwk", "cwv", "cwo"):
        L[name] = pack(ctx, wd, (g.standard_normal((d, d)) * scale).astype(np.float32))
    for name in ("cbq", "cbv", "cbo"):
        L[name] = (0.05 * g.standard_normal(d)).astype(np.float32)
    return L


def make_decoder(ctx, oracle, g, wd=W_Q4_0, d=128, H=2, ff=256, V=300, n_text=24, n_audio=70, n_stream=4,
                 n_layer=2, bs=4):
    layers = [dec_layer(ctx, g, wd, d, ff) for _ in range(n_layer)]
    tok = (g.standard_normal((V, d)) * 0.5).astype(np.float32)
    pos = (g.standard_normal((n_text, d)) * 0.1).astype(np.float32)
    lpg, lpb = rand_norm(g, d)
    gpu = hip.Decoder(ctx, wd, d, H, ff, V, n_text, n_audio, n_stream, layers, tok, pos, lpg, lpb, block_size=bs)
    ref = model_oracle.Decoder(oracle, wd, layers, tok, pos, lpg, lpb, H, ff, n_stream, n_text, bs)
    encs = [g.standard_normal((n_audio, d)).astype(np.float32) for _ in range(n_stream)]
    for s in range(n_stream):
        gpu.set_encoder(s, encs[s])
        ref.set_encoder(s, encs[s])
    gpu.parts = dict(wd=wd, d=d, H=H, ff=ff, V=V, n_text=n_text, bs=bs, layers=layers, tok=tok, pos=pos, lpg=lpg,
                     lpb=lpb, encs=encs)
    return gpu, ref


class DecoderByOps:
    """The decoder step issued one C-ABI entry point at a time: LayerNorm,
    INT8 linears (+ bias, + residual in numpy, GELU), the paged cache's append
    and decode attention, per-stream cross SDPA over the stream's encoder K/V,
    and the fused tied logits + argmax."""

    def __init__(self, ctx, parts, n_stream):
        self.ctx, self.p = ctx, parts
        P = parts
        self.W = hip.WDtype(P["wd"])
        d, H = P["d"], P["H"]
        self.kv = ctx.kv_cache(len(P["layers"]), H, d // H, n_stream, P["n_text"], P["bs"])
        na = P["encs"][0].shape[0]
        self.cross = [[(ctx.gemm_q_f32(na, d, d, enc, L["cwk"], self.W, bias=L.get("cbk")),
                        ctx.gemm_q_f32(na, d, d, enc, L["cwv"], self.W, bias=L.get("cbv")))
                       for L in P["layers"]] for enc in P["encs"]]

    def step(self, streams, tokens, positions):
        ctx, P, W = self.ctx, self.p, self.W
        n, d, H, ff = len(streams), P["d"], P["H"], P["ff"]
        scale = float(np.float32(d // H) ** np.float32(-0.5))
        h = (P["tok"][tokens] + P["pos"][positions]).astype(np.float32)
        lens = [p + 1 for p in positions]
        for l, L in enumerate(P["layers"]):
            xn = ctx.layer_norm_f32(h, n, d, L["ln1_gamma"], L["ln1_beta"])
            q, k, v = (ctx.gemm_q_f32(n, d, d, xn, L[w], W, bias=L.get(b))
                       for w, b in (("wq", "bq"), ("wk", "bk"), ("wv", "bv")))
            self.kv.append(l, streams, positions, k, v)
            a = self.kv.attn(l, streams, lens, q, H, scale)
            h = ctx.gemm_q_f32(n, d, d, a, L["wo"], W, bias=L["bo"]) + h
            xn = ctx.layer_norm_f32(h, n, d, L["ln2_gamma"], L["ln2_beta"])
            cq = ctx.gemm_q_f32(n, d, d, xn, L["cwq"], W, bias=L["cbq"])
            ca = np.concatenate([ctx.attn_f32(cq[i:i + 1], *self.cross[s][l], H, scale=scale)
                                 for i, s in enumerate(streams)])
            h = ctx.gemm_q_f32(n, d, d, ca, L["cwo"], W, bias=L["cbo"]) + h
            xn = ctx.layer_norm_f32(h, n, d, L["ln3_gamma"], L["ln3_beta"])
            f = ctx.gelu_f32(ctx.gemm_q_f32(n, ff, d, xn, L["w1"], W, bias=L["b1"])).reshape(n, ff)
            h = ctx.gemm_q_f32(n, d, ff, f, L["w2"], W, bias=L["b2"]) + h
        x = ctx.layer_norm_f32(h, n, d, P["lpg"], P["lpb"])
        V = P["V"]
        d_x, d_e = hip.DeviceBuffer.from_array(ctx, x), hip.DeviceBuffer.from_array(ctx, P["tok"])
        d_l, d_n = hip.DeviceBuffer(ctx, n * V * 4), hip.DeviceBuffer(ctx, n * 4)
        ctx.logits_argmax_dev(n, V, d, d_x, d_e, d_l, d_n)
        ctx.synchronize()
        return d_n.download(np.int32, n), d_l.download(np.float32, n * V).reshape(n, V)


@pytest.mark.parametrize("wd", [W_Q4_0, W_Q8_0, W_Q5_0, W_Q4_K, W_Q5_K, W_Q6_K])
def test_decoder_step_equals_entry_points(ctx, oracle, wd):
    """A batched decoder step (fused LN + quantize, q split and activation
    pass inside the attention kernels, residual / GELU epilogues, fused
    logits) is bit-identical to the same step issued one entry point at a
    time, over ragged batches, for every weight format the session takes
    (the K-quant ones at d = 256, their group size)."""
    print(f"[case] decoder == entry points wd={wd}", flush=True)
    kq = wd in (W_Q4_K, W_Q5_K, W_Q6_K)
    gpu, _ = make_decoder(ctx, oracle, np.random.default_rng(5), wd=wd, d=256 if kq else 128, H=4 if kq else 2,
                          ff=512 if kq else 256)
    ops = DecoderByOps(ctx, gpu.parts, 4)
    pos, tok = [0, 0, 0, 0], [1, 2, 3, 4]
    for streams in ([0, 1, 2, 3], [2, 0], [3, 1, 0, 2], [1]):
        args = ([tok[s] for s in streams], [pos[s] for s in streams])
        nxt, logits = gpu.step(streams, *args, want_logits=True)
        n2, l2 = ops.step(streams, *args)
        assert np.array_equal(logits, l2) and np.array_equal(nxt, n2), streams
        for i, s in enumerate(streams):
            tok[s], pos[s] = int(nxt[i]), pos[s] + 1


def test_decoder_batch_equals_single_stream_steps(ctx, oracle):
    """Two sessions with identical weights: one steps all streams together,
    the other one stream at a time; logits and tokens are bit-identical."""
    print("[case] decoder batch == single", flush=True)
    a, _ = make_decoder(ctx, oracle, np.random.default_rng(11))
    b, _ = make_decoder(ctx, oracle, np.random.default_rng(11))
    tok, pos = [3, 7, 11, 13], [0, 0, 0, 0]
    for _ in range(5):
        na, la = a.step([0, 1, 2, 3], tok, pos, want_logits=True)
        for i, s in enumerate([3, 1, 0, 2]):
            nb, lb = b.step([s], [tok[s]], [pos[s]], want_logits=True)
            assert np.array_equal(lb[0], la[s]) and nb[0] == na[s], s
        tok, pos = [int(t) for t in na], [p + 1 for p in pos]


def test_decoder_tokens_without_logits(ctx, oracle):
    """Steps that do not ask for logits (the fused logits + argmax then never
    writes them) choose the same tokens as steps that do."""
    print("[case] decoder tokens without logits", flush=True)
    a, _ = make_decoder(ctx, oracle, np.random.default_rng(11))
    b, _ = make_decoder(ctx, oracle, np.random.default_rng(11))
    tok, pos = [3, 7, 11, 13], [0, 0, 0, 0]
    for _ in range(4):
        na, _ = a.step([0, 1, 2, 3], tok, pos, want_logits=True)
        nb = b.step([0, 1, 2, 3], tok, pos)
        assert np.array_equal(na, nb)
        tok, pos = [int(t) for t in na], [p + 1 for p in pos]


def test_decoder_steps_vs_oracle(ctx, oracle):
    """Ragged batches: streams join late and skip steps; tokens follow the
    GPU's greedy choice in both paths."""
    print("[case] decoder steps", flush=True)
    g = np.random.default_rng(42)
    gpu, ref = make_decoder(ctx, oracle, g)
    pos = [0, 0, 0, 0]
    tok = [1, 2, 3, 4]
    schedule = [[0, 1, 2], [0, 1, 2], [2, 0, 3], [3, 1], [0, 1, 2, 3], [1, 3], [0, 2, 3, 1]]
    for step, streams in enumerate(schedule):
        nxt, logits = gpu.step(streams, [tok[s] for s in streams], [pos[s] for s in streams], want_logits=True)
        for i, s in enumerate(streams):
            want, want_tok = ref.step(s, tok[s], pos[s])
            ok, err, rms = within(logits[i], want)
            assert ok, (step, s, err, rms)
            top2 = np.sort(want)[-2:]
            if top2[1] - top2[0] > 0.1 * rms + 1e-4:
                assert nxt[i] == want_tok, (step, s)
            tok[s], pos[s] = int(nxt[i]), pos[s] + 1


def test_decoder_reset_replays_identically(ctx, oracle):
    print("[case] decoder reset", flush=True)
    g = np.random.default_rng(7)
    gpu, _ = make_decoder(ctx, oracle, g)
    first = [gpu.step([0, 1], [5, 6], [p, p], want_logits=True)[1] for p in range(3)]
    gpu.reset()
    again = [gpu.step([0, 1], [5, 6], [p, p], want_logits=True)[1] for p in range(3)]
    for a, b in zip(first, again):
        assert np.array_equal(a, b)


def test_decoder_rejections(ctx, oracle):
    g = np.random.default_rng(8)
    gpu, _ = make_decoder(ctx, oracle, g)
    with pytest.raises(hip.InvalidArgument, match="n_vocab"):
        gpu.step([0], [300], [0])
    with pytest.raises(hip.InvalidArgument, match="n_text_ctx"):
        gpu.step([0], [1], [24])
    with pytest.raises(hip.InvalidArgument, match="distinct"):
        gpu.step([1, 1], [1, 2], [0, 0])
    with pytest.raises(hip.UnsupportedOp):
        hip.Decoder(ctx, W_Q4_0, 160, 2, 256, 10, 4, 8, 1, [dec_layer(ctx, g, W_Q4_0, 160, 256)],
                    np.zeros((10, 160), np.float32), np.zeros((4, 160), np.float32),
                    np.ones(160, np.float32), np.zeros(160, np.float32))


def test_decoder_cross_f16_mode(ctx, oracle):
    """The half-precision cross-attention mode (K/V read as fp16) stays within
    the oracle bar, keeps batch == single-stream bit identity, and switching
    back to F32 restores the F32 results bit for bit."""
    print("[case] decoder cross f16", flush=True)
    g = np.random.default_rng(42)
    gpu, ref = make_decoder(ctx, oracle, g)
    twin, _ = make_decoder(ctx, oracle, np.random.default_rng(42))
    gpu.set_cross_precision(hip.CrossPrecision.F16)
    twin.set_cross_precision(hip.CrossPrecision.F16)
    tok, pos = [1, 2, 3, 4], [0, 0, 0, 0]
    for step in range(4):
        nxt, logits = gpu.step([0, 1, 2, 3], tok, pos, want_logits=True)
        for i in range(4):
            want, _ = ref.step(i, tok[i], pos[i])
            ok, err, rms = within(logits[i], want)
            assert ok, (step, i, err, rms)
            n1, l1 = twin.step([i], [tok[i]], [pos[i]], want_logits=True)
            assert np.array_equal(l1[0], logits[i]) and n1[0] == nxt[i]
        tok, pos = [int(t) for t in nxt], [p + 1 for p in pos]
    # F32 again: a fresh F32 session on the same history gives the same logits
    gpu.set_cross_precision(hip.CrossPrecision.F32)
    fresh, _ = make_decoder(ctx, oracle, np.random.default_rng(42))
    gpu.reset()
    for step in range(2):
        a = gpu.step([0, 1], [5, 6], [step, step], want_logits=True)[1]
        b = fresh.step([0, 1], [5, 6], [step, step], want_logits=True)[1]
        assert np.array_equal(a, b)
    with pytest.raises(hip.InvalidArgument):
        gpu.set_cross_precision(7)


def test_decoder_long_context_split_attention(ctx, oracle):
    """Histories past the first 256-key split (the paged-attention kernel then
    splits keys and the split holding the new step packs it into the cache),
    built by real steps: streams 0 and 1 step every time, stream 2 joins at
    step 200, stream 3 steps every other time. Every step is bit-identical to
    the entry points issued one at a time."""
    print("[case] decoder long context", flush=True)
    gpu, _ = make_decoder(ctx, oracle, np.random.default_rng(9), n_text=600)
    ops = DecoderByOps(ctx, gpu.parts, 4)
    tok, pos = [5, 6, 7, 8], [0, 0, 0, 0]
    for step in range(520):
        streams = [s for s in range(4) if (s < 2 or (s == 2 and step >= 200) or (s == 3 and step % 2 == 0))]
        args = ([tok[s] for s in streams], [pos[s] for s in streams])
        nxt, logits = gpu.step(streams, *args, want_logits=True)
        n2, l2 = ops.step(streams, *args)
        assert np.array_equal(logits, l2) and np.array_equal(nxt, n2), (step, streams)
        for i, s in enumerate(streams):
            tok[s], pos[s] = int(nxt[i]), pos[s] + 1
    assert pos == [520, 520, 320, 260]


def test_decoder_stream_state_rejections(ctx, oracle):
    """A stream without an encoder output, and a position other than the
    stream's length (or 0, a restart), are rejected by the host step."""
    print("[case] decoder stream state", flush=True)
    g = np.random.default_rng(21)
    d, H, ff, V, n_text, n_audio = 128, 2, 256, 300, 24, 70
    layers = [dec_layer(ctx, g, W_Q4_0, d, ff)]
    tok = (g.standard_normal((V, d)) * 0.5).astype(np.float32)
    pos = (g.standard_normal((n_text, d)) * 0.1).astype(np.float32)
    lpg, lpb = rand_norm(g, d)
    dec = hip.Decoder(ctx, W_Q4_0, d, H, ff, V, n_text, n_audio, 2, layers, tok, pos, lpg, lpb, block_size=4)
    dec.set_encoder(0, g.standard_normal((n_audio, d)).astype(np.float32))
    with pytest.raises(hip.InvalidArgument, match="no encoder output"):
        dec.step([1], [1], [0])
    t = int(dec.step([0], [1], [0])[0])
    with pytest.raises(hip.InvalidArgument, match="position"):
        dec.step([0], [t], [2])
    t = int(dec.step([0], [t], [1])[0])
    a = dec.step([0], [3], [0], want_logits=True)[1]  # restart
    dec.reset()
    b = dec.step([0], [3], [0], want_logits=True)[1]
    assert np.array_equal(a, b)
    with pytest.raises(hip.InvalidArgument, match="position"):
        dec.step([0], [3], [5])


def test_decoder_many_streams_split_page_allocation(ctx, oracle):
    """1024 streams x 5 layers = 5120 (layer, item) appends per step, above the
    4096 of one allocation launch: the step allocates in two launches. A
    batched step equals the same streams stepped alone in a twin session, and
    the cache holds exactly the pages the steps need."""
    print("[case] decoder 1024 streams x 5 layers", flush=True)
    n_stream, n_layer, n_audio, n_text, bs = 1024, 5, 16, 8, 4

    def build(seed):
        g = np.random.default_rng(seed)
        d, H, ff, V = 128, 2, 256, 64
        layers = [dec_layer(ctx, g, W_Q4_0, d, ff) for _ in range(n_layer)]
        tok = (g.standard_normal((V, d)) * 0.5).astype(np.float32)
        pos = (g.standard_normal((n_text, d)) * 0.1).astype(np.float32)
        lpg, lpb = rand_norm(g, d)
        dec = hip.Decoder(ctx, W_Q4_0, d, H, ff, V, n_text, n_audio, n_stream, layers, tok, pos, lpg, lpb,
                          block_size=bs)
        enc = g.standard_normal((n_audio, d)).astype(np.float32)
        for s in range(n_stream):
            dec.set_encoder(s, enc)
        return dec

    a, b = build(3), build(3)
    streams = list(range(n_stream))
    tokens = [s % 64 for s in streams]
    na, la = a.step(streams, tokens, [0] * n_stream, want_logits=True)
    for s in (0, 511, 1023):
        nb, lb = b.step([s], [tokens[s]], [0], want_logits=True)
        assert np.array_equal(lb[0], la[s]) and nb[0] == na[s], s
    na2, la2 = a.step(streams, [int(t) for t in na], [1] * n_stream, want_logits=True)
    assert np.isfinite(la2).all()


def test_attention_fp16_range_is_an_error(ctx):
    """An operand beyond the fp16 range of the split products is
    INVALID_ARGUMENT, not a silent inf / NaN; the next call is clean."""
    print("[case] attention fp16 range", flush=True)
    g = np.random.default_rng(2)
    q = g.standard_normal((1, 8, 128)).astype(np.float32)
    k = g.standard_normal((1, 16, 128)).astype(np.float32)
    v = g.standard_normal((1, 16, 128)).astype(np.float32)
    for which in range(3):
        ops = [q.copy(), k.copy(), v.copy()]
        ops[which][0, 3, 70] = 1.0e5 if which else 1.0e5 / 0.125  # q is scaled by 0.125 first
        with pytest.raises(hip.InvalidArgument, match="fp16 range"):
            ctx.attn_f32(*ops, 2, scale=0.125)
    ok = ctx.attn_f32(q, k, v, 2, scale=0.125)
    assert np.isfinite(ok).all()
    kv = ctx.kv_cache(1, 1, 128, 1, 16, 4)
    kv.append(0, [0] * 4, [0, 1, 2, 3], g.standard_normal((4, 128)), g.standard_normal((4, 128)))
    qb = g.standard_normal((1, 8 * 128)).astype(np.float32)
    qb[0, 5] = 1.0e6
    with pytest.raises(hip.InvalidArgument, match="fp16 range"):
        kv.attn(0, [0], [4], qb, 8, 0.125)

"""GPU parity of the encoder and decoder-step sessions at the configured model
dimensions: config 0 (Whisper-base encoder, all 6 blocks from seeded
synthetic audio), config 2 (Whisper-large-v3 encoder, 32 blocks, batch 16) and
config 3 (Whisper-large-v3 decoder step, 64 streams, 51866-token vocabulary,
1500 encoder frames, prefixes up to 447).

Bars, all at these dimensions:
  * session == the same model issued one C-ABI entry point at a time on
    device buffers, bit for bit (the fused kernels of the sessions are equal
    to the entry-point sequence, and every kernel is row-independent);
  * teacher-forced: each entry point of that chain, fed the GPU's own inputs,
    against the oracle function it replaces on sampled rows and heads:
    INT8 linears bit-exact, LayerNorm within atol 1e-5 + rtol 1e-4, GELU
    within 1e-6 + 1e-5 rel, attention within 1e-4 + 1e-3 rel, log-mel within
    the oracle's own pin (atol 5e-5), the conv stem within the f32
    dot-product bound k * 2^-23 * sum|a b| of float64. A systematic error of
    any one operation fails its check; the chain's bit identity then carries
    the checks to the sessions.
"""
import numpy as np
import pytest

from vokra_amd import hip

pytestmark = pytest.mark.gpu

W_Q4_0, W_Q8_0 = 2, 8
LN_ATOL, LN_RTOL = 1e-5, 1e-4
AT_ATOL, AT_RTOL = 1e-4, 1e-3


@pytest.fixture(scope="module")
def ctx():
    c = hip.HipContext(0)
    yield c
    c.close()


def random_qblock(g, wd, n, k, amax):
    """Random-init block-quant weight [n, k] on the wire: uniform quants and
    one f16 scale (amax / 127 for Q8_0, amax / 7 for Q4_0)."""
    nb = n * (k // 32)
    if wd == W_Q8_0:
        blk = np.empty((nb, 34), np.uint8)
        blk[:, 0:2] = np.frombuffer(np.float16(amax / 127).tobytes(), np.uint8)
        blk[:, 2:] = g.integers(-127, 128, (nb, 32), dtype=np.int8).view(np.uint8)
    else:
        blk = np.empty((nb, 18), np.uint8)
        blk[:, 0:2] = np.frombuffer(np.float16(amax / 7).tobytes(), np.uint8)
        blk[:, 2:] = g.integers(0, 256, (nb, 16), dtype=np.uint8)
    return blk.reshape(-1)


def norm_pair(g, d):
    return (1.0 + 0.1 * g.standard_normal(d)).astype(np.float32), (0.1 * g.standard_normal(d)).astype(np.float32)


def enc_layer(g, wd, d, ff):
    L = {}
    L["ln1_gamma"], L["ln1_beta"] = norm_pair(g, d)
    L["ln2_gamma"], L["ln2_beta"] = norm_pair(g, d)
    for name, n, k in (("wq", d, d), ("wk", d, d), ("wv", d, d), ("wo", d, d), ("w1", ff, d), ("w2", d, ff)):
        L[name] = random_qblock(g, wd, n, k, 1.7 / np.sqrt(k))
    for name, n in (("bq", d), ("bv", d), ("bo", d), ("b1", ff), ("b2", d)):
        L[name] = (0.05 * g.standard_normal(n)).astype(np.float32)
    return L


def close(got, want, atol, rtol):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    err = np.abs(got - want)
    return bool(np.all(err <= atol + rtol * np.abs(want))), float(err.max())


class Checker:
    """Teacher-forced comparisons of one entry point's output against the
    oracle on the GPU's own inputs; records the worst error per operation."""

    def __init__(self, oracle):
        self.o = oracle
        self.worst = {}

    def note(self, what, err):
        self.worst[what] = max(self.worst.get(what, 0.0), err)

    def linear(self, wd, x_rows, w, n, k, bias, y_rows, what):
        want = self.o.gemm_q_f32(wd, x_rows.shape[0], n, k, x_rows, w, bias)
        assert np.array_equal(y_rows.view(np.uint32), want.view(np.uint32)), what

    def layer_norm(self, x_rows, g, b, y_rows, what):
        want = self.o.layer_norm_f32(x_rows, x_rows.shape[0], x_rows.shape[1], g, b)
        ok, err = close(y_rows, want, LN_ATOL, LN_RTOL)
        self.note("layer_norm", err)
        assert ok, (what, err)

    def gelu(self, x_rows, y_rows, what):
        want = self.o.gelu_f32(x_rows.reshape(-1)).reshape(x_rows.shape)
        ok, err = close(y_rows, want, 1e-6, 1e-5)
        self.note("gelu", err)
        assert ok, (what, err)

    def attention(self, q_rows, q_pos, K, V, H, hd, heads, y_rows, causal, what):
        """q_rows [r, H*hd] (unscaled: sdpa_whisper applies hd^-0.5 to q) at
        positions q_pos; K, V [t_kv, H*hd]."""
        for h in heads:
            sl = slice(h * hd, (h + 1) * hd)
            for i, p in enumerate(q_pos):
                t_kv = p + 1 if causal else K.shape[0]
                want = self.o.sdpa_whisper(1, t_kv, 1, hd, q_rows[i:i + 1, sl], K[:t_kv, sl], V[:t_kv, sl])[0]
                ok, err = close(y_rows[i, sl], want, AT_ATOL, AT_RTOL)
                self.note("attention", err)
                assert ok, (what, h, p, err)


def rows_of(buf, width, rows):
    return np.stack([buf.download_at(np.float32, r * width, width) for r in rows])


def block_of(buf, width, r0, n_rows):
    return buf.download_at(np.float32, r0 * width, n_rows * width).reshape(n_rows, width)


class EncoderChain:
    """The pre-norm encoder blocks (encoder.rs:180-245) as C-ABI entry points
    on device buffers: LayerNorm, gemm_q_f32 (INT8 activation pass + block
    GEMM, bias after), attention, residual add, GELU."""

    def __init__(self, ctx, wd, layers, lpg, lpb, H, ff, d, max_rows):
        self.ctx, self.wd, self.layers, self.H, self.ff, self.d = ctx, wd, layers, H, ff, d
        up = lambda a: hip.DeviceBuffer.from_array(ctx, a)
        self.dev = []
        for L in layers:
            D = {k: up(L[k]) for k in ("ln1_gamma", "ln1_beta", "ln2_gamma", "ln2_beta", "bq", "bv", "bo", "b1", "b2")}
            for name, n, k in (("wq", d, d), ("wk", d, d), ("wv", d, d), ("wo", d, d), ("w1", ff, d),
                               ("w2", d, ff)):
                D[name] = ctx.upload_qweight(hip.WDtype(wd), n, k, L[name])
            self.dev.append(D)
        self.lpg, self.lpb = up(lpg), up(lpb)
        B = lambda n: hip.DeviceBuffer(ctx, max_rows * n * 4)
        self.h, self.xn, self.q, self.k, self.v, self.a, self.o = (B(d) for _ in range(7))
        self.f = B(ff)

    def forward(self, d_x, batch, T, out, check=None, check_layers=(), rows=(), heads=()):
        ctx, d, H, ff, hd = self.ctx, self.d, self.H, self.ff, self.d // self.H
        n = batch * T
        ctx.copy_dev(self.h, d_x, n * d * 4)
        for li, (L, D) in enumerate(zip(self.layers, self.dev)):
            chk = check if li in check_layers else None
            pre = rows_of(self.h, d, rows) if chk else None
            ctx.layer_norm_f32_dev(self.h, self.xn, n, d, D["ln1_gamma"], D["ln1_beta"])
            for name, bname, dst in (("wq", "bq", self.q), ("wk", None, self.k), ("wv", "bv", self.v)):
                ctx.gemm_q_f32_dev(D[name], n, self.xn, dst, None if bname is None else D[bname])
            ctx.attn_f32_dev(batch, T, T, H, H, hd, self.q, self.k, self.v, float(hd) ** -0.5, False, 0, self.a)
            if chk:
                xn = rows_of(self.xn, d, rows)
                chk.layer_norm(pre, L["ln1_gamma"], L["ln1_beta"], xn, ("ln1", li))
                for name, bname, dst in (("wq", "bq", self.q), ("wk", None, self.k), ("wv", "bv", self.v)):
                    chk.linear(self.wd, xn, L[name], d, d, L.get(bname), rows_of(dst, d, rows), (name, li))
                # attention of the sampled rows over their utterance's keys
                for r in rows:
                    b0 = (r // T) * T
                    Kb, Vb = block_of(self.k, d, b0, T), block_of(self.v, d, b0, T)
                    chk.attention(rows_of(self.q, d, [r]), [r - b0], Kb, Vb, H, hd, heads, rows_of(self.a, d, [r]),
                                  False, ("attn", li))
            ctx.gemm_q_f32_dev(D["wo"], n, self.a, self.o, D["bo"])
            if chk:
                chk.linear(self.wd, rows_of(self.a, d, rows), L["wo"], d, d, L["bo"], rows_of(self.o, d, rows),
                           ("wo", li))
            ctx.add_f32_dev(self.o, self.h, self.h, n * d)
            mid = rows_of(self.h, d, rows) if chk else None
            ctx.layer_norm_f32_dev(self.h, self.xn, n, d, D["ln2_gamma"], D["ln2_beta"])
            ctx.gemm_q_f32_dev(D["w1"], n, self.xn, self.f, D["b1"])
            f_pre = rows_of(self.f, ff, rows) if chk else None
            ctx.gelu_f32_dev(self.f, self.f, n * ff)
            ctx.gemm_q_f32_dev(D["w2"], n, self.f, self.o, D["b2"])
            if chk:
                xn = rows_of(self.xn, d, rows)
                chk.layer_norm(mid, L["ln2_gamma"], L["ln2_beta"], xn, ("ln2", li))
                chk.linear(self.wd, xn, L["w1"], ff, d, L["b1"], f_pre, ("w1", li))
                f = rows_of(self.f, ff, rows)
                chk.gelu(f_pre, f, ("gelu", li))
                chk.linear(self.wd, f, L["w2"], d, ff, L["b2"], rows_of(self.o, d, rows), ("w2", li))
            ctx.add_f32_dev(self.o, self.h, self.h, n * d)
        ctx.layer_norm_f32_dev(self.h, out, n, d, self.lpg, self.lpb)


# ---- config 0: Whisper-base encoder from audio -------------------------------
def synthetic_audio(seed, n=480000, sr=16000):
    """30 s of seeded 16 kHz audio: white noise plus 3 random sines, amplitude
    0.3."""
    g = np.random.default_rng(seed)
    t = np.arange(n) / sr
    x = g.standard_normal(n) * 0.1
    for _ in range(3):
        x += np.sin(2 * np.pi * g.uniform(100, 4000) * t + g.uniform(0, 2 * np.pi))
    return (0.3 * x / np.abs(x).max()).astype(np.float32)


def test_encoder_config0_all_blocks_from_audio(ctx, oracle):
    """Config 0: 30 s of seeded synthetic audio -> log-mel (80 bins) -> conv
    stem -> 6 blocks (d=512, 8 heads, FFN 2048, Q8_0) -> ln_post. Session
    encode == stem, then the entry-point chain, bit for bit; log-mel and the
    stem against the oracle; every block teacher-forced against the oracle."""
    print("[case] encoder config 0, 6 blocks from audio", flush=True)
    n_mels, d, H, ff, n_layer = 80, 512, 8, 2048, 6
    g = np.random.default_rng(100)
    layers = [enc_layer(g, W_Q8_0, d, ff) for _ in range(n_layer)]
    lpg, lpb = norm_pair(g, d)
    c1w = (g.standard_normal((d, n_mels, 3)) * 0.05).astype(np.float32)
    c1b = (g.standard_normal(d) * 0.05).astype(np.float32)
    c2w = (g.standard_normal((d, d, 3)) * 0.02).astype(np.float32)
    c2b = (g.standard_normal(d) * 0.05).astype(np.float32)
    pos = (g.standard_normal((1500, d)) * 0.1).astype(np.float32)
    enc = hip.Encoder(ctx, W_Q8_0, d, H, ff, layers, lpg, lpb, max_rows=1500)
    enc.set_stem(n_mels, 3000, c1w, c1b, c2w, c2b, pos)
    pcm = synthetic_audio(0)
    chk = Checker(oracle)
    # log-mel against the oracle (the reference's front end)
    mel = ctx.log_mel(pcm, n_mels)
    want_mel = oracle.log_mel(pcm, n_mels).reshape(n_mels, 3000)
    assert np.abs(mel - want_mel).max() <= 5e-5, np.abs(mel - want_mel).max()
    d_mel = hip.DeviceBuffer.from_array(ctx, mel)
    # the stem against the oracle's conv1d -> GELU -> conv1d -> GELU -> + pos
    # on the GPU's own log-mel. Both sides round f32 dot products of length k
    # (error <= k 2^-24 sum|a b| each, so 2 k 2^-24 sum|a b| apart), GELU has
    # slope <= 1.13 and rounds a few ulp, and the first conv's difference
    # reaches the second through |w2|.
    d_x = hip.DeviceBuffer(ctx, 1500 * d * 4)
    enc.stem_dev(1, d_mel, d_x)
    x = d_x.download(np.float32, 1500 * d).reshape(1500, d)
    c1 = oracle.gelu_f32(oracle.conv1d_f32(mel, n_mels, 3000, c1w, d, 3, c1b, 1, 1))
    c2 = oracle.gelu_f32(oracle.conv1d_f32(c1, d, 3000, c2w, d, 3, c2b, 2, 1))
    want_x = c2.T + pos
    u = 2.0 ** -24
    ab1 = oracle.conv1d_f32(np.abs(mel), n_mels, 3000, np.abs(c1w), d, 3, np.abs(c1b), 1, 1).astype(np.float64)
    dl1 = 1.13 * 2 * (3 * n_mels + 1) * u * ab1 + 8 * u * np.abs(c1)
    ab2 = oracle.conv1d_f32(np.abs(c1), d, 3000, np.abs(c2w), d, 3, np.abs(c2b), 2, 1).astype(np.float64)
    prop = oracle.conv1d_f32(dl1.astype(np.float32), d, 3000, np.abs(c2w), d, 3, None, 2, 1).astype(np.float64)
    dl2 = 1.13 * (2 * (3 * d + 1) * u * ab2 + 1.01 * prop) + 8 * u * np.abs(c2)
    bound = dl2.T + 2 * u * np.abs(want_x) + 1e-30
    assert np.all(np.abs(x - want_x) <= bound), float(np.max(np.abs(x - want_x) - bound))
    # session encode == stem, then the chain; every block checked
    got = hip.DeviceBuffer(ctx, 1500 * d * 4)
    enc.encode_dev(1, d_mel, got)
    chain = EncoderChain(ctx, W_Q8_0, layers, lpg, lpb, H, ff, d, 1500)
    out = hip.DeviceBuffer(ctx, 1500 * d * 4)
    chain.forward(d_x, 1, 1500, out, check=chk, check_layers=range(n_layer), rows=(0, 731, 1499), heads=(0, 5))
    ctx.synchronize()
    assert np.array_equal(got.download(np.uint32, 1500 * d), out.download(np.uint32, 1500 * d))
    print("[worst teacher-forced errors]", chk.worst, flush=True)


# ---- config 2: Whisper-large-v3 encoder ---------------------------------------
def test_encoder_config2_batch16_32_blocks(ctx, oracle):
    """Config 2: 32 blocks (d=1280, 20 heads, FFN 5120, Q8_0), batch 16 x 1500
    frames = 24000 rows: session forward == the entry-point chain bit for bit;
    blocks 0, 15 and 31 teacher-forced against the oracle on rows of the
    first and last utterance; batch 1 == row block of batch 16."""
    print("[case] encoder config 2, 32 blocks, batch 16", flush=True)
    d, H, ff, n_layer, T, B = 1280, 20, 5120, 32, 1500, 16
    g = np.random.default_rng(200)
    layers = [enc_layer(g, W_Q8_0, d, ff) for _ in range(n_layer)]
    lpg, lpb = norm_pair(g, d)
    enc = hip.Encoder(ctx, W_Q8_0, d, H, ff, layers, lpg, lpb, max_rows=B * T)
    x = g.standard_normal((B * T, d), dtype=np.float32)
    d_x = hip.DeviceBuffer.from_array(ctx, x)
    got = hip.DeviceBuffer(ctx, B * T * d * 4)
    enc.forward_dev(B, T, d_x, got)
    chk = Checker(oracle)
    chain = EncoderChain(ctx, W_Q8_0, layers, lpg, lpb, H, ff, d, B * T)
    out = hip.DeviceBuffer(ctx, B * T * d * 4)
    chain.forward(d_x, B, T, out, check=chk, check_layers=(0, 15, 31), rows=(0, 1234, 15 * T + 777),
                  heads=(0, 19))
    ctx.synchronize()
    n = B * T * d
    assert np.array_equal(got.download(np.uint32, n), out.download(np.uint32, n))
    # batch invariance: utterance 15 alone
    one = hip.DeviceBuffer(ctx, T * d * 4)
    enc.forward_dev(1, T, hip.DeviceBuffer.from_array(ctx, x[15 * T:]), one)
    ctx.synchronize()
    assert np.array_equal(one.download(np.uint32, T * d), got.download_at(np.uint32, 15 * T * d, T * d))
    print("[worst teacher-forced errors]", chk.worst, flush=True)


# ---- config 3: Whisper-large-v3 decoder step ------------------------------------
def dec_layer(g, wd, d, ff):
    L = enc_layer(g, wd, d, ff)
    L["ln3_gamma"], L["ln3_beta"] = norm_pair(g, d)
    for name in ("cwq", "cwk", "cwv", "cwo"):
        L[name] = random_qblock(g, wd, d, d, 1.7 / np.sqrt(d))
    for name in ("cbq", "cbv", "cbo"):
        L[name] = (0.05 * g.standard_normal(d)).astype(np.float32)
    return L


class DecoderChain:
    """The Whisper decoder step (decoder.rs:413-567) for a batch of streams as
    C-ABI entry points: LayerNorm, gemm_q_f32, the paged cache's append and
    decode attention, cross attention over the stream's encoder K/V (one
    encoder output shared by every stream: its K/V projected once per layer
    and repeated per item), residuals in numpy, GELU, fused logits + argmax."""

    def __init__(self, ctx, wd, layers, tok, pos, lpg, lpb, H, ff, n_stream, n_text, bs, d_enc, n_audio):
        self.ctx, self.wd, self.layers, self.tok, self.pos = ctx, wd, layers, tok, pos
        self.lpg, self.lpb, self.H, self.ff = lpg, lpb, H, ff
        d = tok.shape[1]
        self.d, self.V, self.n_audio = d, tok.shape[0], n_audio
        self.kv = ctx.kv_cache(len(layers), H, d // H, n_stream, n_text, bs)
        W = hip.WDtype(wd)
        self.cross = []
        for L in layers:
            ck, cv = hip.DeviceBuffer(ctx, n_audio * d * 4), hip.DeviceBuffer(ctx, n_audio * d * 4)
            ctx.gemm_q_f32_dev(ctx.upload_qweight(W, d, d, L["cwk"]), n_audio, d_enc, ck)
            ctx.gemm_q_f32_dev(ctx.upload_qweight(W, d, d, L["cwv"]), n_audio, d_enc, cv,
                               hip.DeviceBuffer.from_array(ctx, L["cbv"]))
            self.cross.append((ck, cv))
        self.rep_k = hip.DeviceBuffer(ctx, n_stream * n_audio * d * 4)
        self.rep_v = hip.DeviceBuffer(ctx, n_stream * n_audio * d * 4)
        self.d_tok = hip.DeviceBuffer.from_array(ctx, tok)
        ctx.synchronize()

    def cross_kv(self, l):
        ck, cv = self.cross[l]
        return block_of(ck, self.d, 0, self.n_audio), block_of(cv, self.d, 0, self.n_audio)

    def step(self, streams, tokens, positions, check=None):
        ctx, d, H, ff, W = self.ctx, self.d, self.H, self.ff, hip.WDtype(self.wd)
        n, hd, na = len(streams), self.d // self.H, self.n_audio
        scale = float(np.float32(hd) ** np.float32(-0.5))
        h = (self.tok[tokens] + self.pos[positions]).astype(np.float32)
        lens = [p + 1 for p in positions]
        sample = [0, n - 1] if n > 1 else [0]
        for l, L in enumerate(self.layers):
            xn = ctx.layer_norm_f32(h, n, d, L["ln1_gamma"], L["ln1_beta"])
            q, k, v = (ctx.gemm_q_f32(n, d, d, xn, L[w], W, bias=L.get(b))
                       for w, b in (("wq", "bq"), ("wk", "bk"), ("wv", "bv")))
            self.kv.append(l, streams, positions, k, v)
            a = self.kv.attn(l, streams, lens, q, H, scale)
            if check:
                check.layer_norm(h[sample], L["ln1_gamma"], L["ln1_beta"], xn[sample], ("ln1", l))
                for name, bname, y in (("wq", "bq", q), ("wk", "bk", k), ("wv", "bv", v)):
                    check.linear(self.wd, xn[sample], L[name], d, d, L.get(bname), y[sample], (name, l))
                for i in sample:
                    s = streams[i]
                    rows = [self.kv.read(l, t, s) for t in range(lens[i])]
                    K = np.stack([r[0] for r in rows])
                    V = np.stack([r[1] for r in rows])
                    check.attention(q[i:i + 1], [positions[i]], K, V, H, hd, (0, 7, 19), a[i:i + 1], True,
                                    ("self", l))
            o = ctx.gemm_q_f32(n, d, d, a, L["wo"], W, bias=L["bo"])
            if check:
                check.linear(self.wd, a[sample], L["wo"], d, d, L["bo"], o[sample], ("wo", l))
            h = o + h
            xn = ctx.layer_norm_f32(h, n, d, L["ln2_gamma"], L["ln2_beta"])
            cq = ctx.gemm_q_f32(n, d, d, xn, L["cwq"], W, bias=L["cbq"])
            ck, cv = self.cross[l]
            for i in range(n):
                self._copy_at(self.rep_k, i * na * d, ck, na * d)
                self._copy_at(self.rep_v, i * na * d, cv, na * d)
            d_q = hip.DeviceBuffer.from_array(ctx, cq)
            d_a = hip.DeviceBuffer(ctx, n * d * 4)
            ctx.attn_f32_dev(n, 1, na, H, H, hd, d_q, self.rep_k, self.rep_v, scale, False, 0, d_a)
            ctx.synchronize()
            ca = d_a.download(np.float32, n * d).reshape(n, d)
            if check:
                check.layer_norm(h[sample], L["ln2_gamma"], L["ln2_beta"], xn[sample], ("ln2", l))
                check.linear(self.wd, xn[sample], L["cwq"], d, d, L["cbq"], cq[sample], ("cwq", l))
                K, V = self.cross_kv(l)
                for i in sample:
                    check.attention(cq[i:i + 1], [na - 1], K, V, H, hd, (0, 19), ca[i:i + 1], False, ("cross", l))
            o = ctx.gemm_q_f32(n, d, d, ca, L["cwo"], W, bias=L["cbo"])
            if check:
                check.linear(self.wd, ca[sample], L["cwo"], d, d, L["cbo"], o[sample], ("cwo", l))
            h = o + h
            xn = ctx.layer_norm_f32(h, n, d, L["ln3_gamma"], L["ln3_beta"])
            f_pre = ctx.gemm_q_f32(n, ff, d, xn, L["w1"], W, bias=L["b1"])
            f = ctx.gelu_f32(f_pre).reshape(n, ff)
            o = ctx.gemm_q_f32(n, d, ff, f, L["w2"], W, bias=L["b2"])
            if check:
                check.layer_norm(h[sample], L["ln3_gamma"], L["ln3_beta"], xn[sample], ("ln3", l))
                check.linear(self.wd, xn[sample], L["w1"], ff, d, L["b1"], f_pre[sample], ("w1", l))
                check.gelu(f_pre[sample], f[sample], ("gelu", l))
                check.linear(self.wd, f[sample], L["w2"], d, ff, L["b2"], o[sample], ("w2", l))
            h = o + h
        x = ctx.layer_norm_f32(h, n, d, self.lpg, self.lpb)
        d_x = hip.DeviceBuffer.from_array(ctx, x)
        d_l, d_n = hip.DeviceBuffer(ctx, n * self.V * 4), hip.DeviceBuffer(ctx, n * 4)
        ctx.logits_argmax_dev(n, self.V, d, d_x, self.d_tok, d_l, d_n)
        ctx.synchronize()
        logits = d_l.download(np.float32, n * self.V).reshape(n, self.V)
        nxt = d_n.download(np.int32, n)
        if check:
            check.layer_norm(h[sample], self.lpg, self.lpb, x[sample], ("ln_post", 0))
            for i in sample:
                # tied logits: f32 dot products of length d against float64
                exact = self.tok.astype(np.float64) @ x[i].astype(np.float64)
                bound = d * 2 ** -23 * (np.abs(self.tok) @ np.abs(x[i]).astype(np.float64)) + 1e-30
                assert np.all(np.abs(logits[i] - exact) <= bound), ("logits", i)
                assert nxt[i] == int(np.argmax(logits[i])), ("argmax", i)
        return nxt, logits

    def _copy_at(self, dst, dst_off, src, count):
        hip.lib().vokra_hip_copy_dev(self.ctx._h, hip.C.c_void_p(dst.ptr.value + 4 * dst_off), src.ptr, 4 * count)


def make_config3_decoder(ctx, g, n_layer, n_stream, wd=W_Q4_0, d=1280, H=20, ff=5120, V=51866, n_text=448,
                         n_audio=1500):
    layers = [dec_layer(g, wd, d, ff) for _ in range(n_layer)]
    tok = (g.standard_normal((V, d)) * 0.02).astype(np.float32)
    pos = (g.standard_normal((n_text, d)) * 0.02).astype(np.float32)
    lpg, lpb = norm_pair(g, d)
    dec = hip.Decoder(ctx, wd, d, H, ff, V, n_text, n_audio, n_stream, layers, tok, pos, lpg, lpb, block_size=16)
    enc = g.standard_normal((n_audio, d), dtype=np.float32)
    d_enc = hip.DeviceBuffer.from_array(ctx, enc)
    for s in range(n_stream):
        dec.set_encoder_dev(s, d_enc)
    ctx.synchronize()
    parts = dict(layers=layers, tok=tok, pos=pos, lpg=lpg, lpb=lpb, d_enc=d_enc, wd=wd, H=H, ff=ff, n_text=n_text,
                 n_audio=n_audio)
    return dec, parts


def chain_for(ctx, P, n_stream):
    return DecoderChain(ctx, P["wd"], P["layers"], P["tok"], P["pos"], P["lpg"], P["lpb"], P["H"], P["ff"],
                        n_stream, P["n_text"], 16, P["d_enc"], P["n_audio"])


def test_decoder_config3_two_layers_teacher_forced(ctx, oracle):
    """Config-3 dims (d=1280, 20 heads, FFN 5120, V=51866, 1500 encoder
    frames, Q4_0, 16-token pages) with 2 layers and 64 streams joining over
    ragged steps: session == entry points bit for bit; every entry point
    teacher-forced against the oracle on the first and last item."""
    print("[case] decoder config 3, 2 layers, 64 streams", flush=True)
    n_stream = 64
    g = np.random.default_rng(300)
    dec, P = make_config3_decoder(ctx, g, 2, n_stream)
    chain = chain_for(ctx, P, n_stream)
    chk = Checker(oracle)
    tok = [int(t) for t in g.integers(0, 51866, n_stream)]
    pos = [0] * n_stream
    for step, streams in enumerate([list(range(48)), list(range(n_stream)), [63, 5, 40, 0, 17],
                                    list(range(n_stream - 1, -1, -1))]):
        args = ([tok[s] for s in streams], [pos[s] for s in streams])
        nxt, logits = dec.step(streams, *args, want_logits=True)
        n2, l2 = chain.step(streams, *args, check=chk if step in (1, 3) else None)
        assert np.array_equal(logits.view(np.uint32), l2.view(np.uint32)) and np.array_equal(nxt, n2), step
        for i, s in enumerate(streams):
            tok[s], pos[s] = int(nxt[i]), pos[s] + 1
    print("[worst teacher-forced errors]", chk.worst, flush=True)


def test_decoder_config3_full_depth(ctx, oracle):
    """All 32 layers at config-3 dims, 64 streams: two batched steps ==
    the entry-point chain bit for bit."""
    print("[case] decoder config 3, 32 layers, 64 streams", flush=True)
    n_stream = 64
    g = np.random.default_rng(332)
    dec, P = make_config3_decoder(ctx, g, 32, n_stream)
    chain = chain_for(ctx, P, n_stream)
    tok = [int(t) for t in g.integers(0, 51866, n_stream)]
    pos = [0] * n_stream
    for step in range(2):
        streams = list(range(n_stream))
        nxt, logits = dec.step(streams, tok, pos, want_logits=True)
        n2, l2 = chain.step(streams, tok, pos)
        assert np.array_equal(logits.view(np.uint32), l2.view(np.uint32)) and np.array_equal(nxt, n2), step
        tok, pos = [int(t) for t in nxt], [p + 1 for p in pos]


def test_decoder_config3_prefix_to_447(ctx, oracle):
    """One config-3 layer, 2 streams stepped through their whole 448-token
    context (prefixes cross the 256-key mark and end at 447): every step ==
    the entry-point chain bit for bit, and the last steps teacher-forced
    against the oracle (self-attention over 447 dequantized cache rows)."""
    print("[case] decoder config 3, prefixes to 447", flush=True)
    g = np.random.default_rng(447)
    dec, P = make_config3_decoder(ctx, g, 1, 2)
    chain = chain_for(ctx, P, 2)
    chk = Checker(oracle)
    tok = [5, 9]
    for p in range(448):
        check = chk if p in (255, 256, 447) else None
        nxt, logits = dec.step([0, 1], tok, [p, p], want_logits=True)
        n2, l2 = chain.step([0, 1], tok, [p, p], check=check)
        assert np.array_equal(logits.view(np.uint32), l2.view(np.uint32)) and np.array_equal(nxt, n2), p
        tok = [int(t) for t in nxt]
    with pytest.raises(hip.InvalidArgument, match="n_text_ctx"):
        dec.step([0], [1], [448])
    print("[worst teacher-forced errors]", chk.worst, flush=True)


def test_decoder_config3_ragged_prefixes_shuffled_pages(ctx, oracle):
    """Config 3 as configured: 64 streams whose prefixes are U(1..448)
    (seeded), reached by decode steps over a shuffled page table, 2 layers.
    Stream s takes its steps at positions 0 .. P_s - 1 in batches of the
    streams still short of their prefix, so batch membership is ragged. Bars:
      * the session with a shuffled free list == a twin with the reference's
        LIFO order, every step (tokens every step, all logits every 32nd step
        and at the end): page placement never changes a result;
      * three tracked streams (the longest, the shortest, one crossing the
        256-key mark) == the entry-point chain bit for bit at every one of
        their steps, with the chain's own cache shuffled differently;
      * their last steps teacher-forced against the oracle (self-attention
        over P_s dequantized cache rows that sit on shuffled pages)."""
    print("[case] decoder config 3, prefixes U(1..448), shuffled page table, 64 streams", flush=True)
    n_stream = 64
    g = np.random.default_rng(3448)
    dec, P = make_config3_decoder(ctx, np.random.default_rng(3449), 2, n_stream)
    twin, _ = make_config3_decoder(ctx, np.random.default_rng(3449), 2, n_stream)
    free, used = dec.kv_pages()
    assert used == 0
    dec.set_free_order(g.permutation(free).astype(np.int32))
    prefix = g.integers(1, 449, n_stream)
    prefix[[0, 1, 2]] = [448, 1, 258]
    g.shuffle(prefix)
    longest, shortest, mid = int(np.argmax(prefix)), int(np.argmin(prefix)), int(np.argmax(prefix == 258))
    tracked = [longest, shortest, mid]
    chain = chain_for(ctx, P, n_stream)
    chain.kv.set_free_order(g.permutation(sum(chain.kv.pages())).astype(np.int32))
    chk = Checker(oracle)
    tok = [int(t) for t in g.integers(0, 51866, n_stream)]
    n_steps = int(prefix.max())
    for t in range(n_steps):
        streams = [int(s) for s in g.permutation(n_stream) if prefix[s] > t]
        args = ([tok[s] for s in streams], [t] * len(streams))
        nxt, logits = dec.step(streams, *args, want_logits=True)
        full = t % 32 == 0 or t == n_steps - 1
        if full:
            n_twin, l_twin = twin.step(streams, *args, want_logits=True)
            assert np.array_equal(logits.view(np.uint32), l_twin.view(np.uint32)), t
        else:
            n_twin = twin.step(streams, *args)
        assert np.array_equal(nxt, n_twin), t
        # a tracked stream at its last step goes first: the chain's teacher-
        # forced checks cover the first and last item of its batch
        rows = sorted((i for i, s in enumerate(streams) if s in tracked), key=lambda i: prefix[streams[i]] != t + 1)
        if rows:
            sub = [streams[i] for i in rows]
            last = [s for s in sub if prefix[s] == t + 1]
            n2, l2 = chain.step(sub, [tok[s] for s in sub], [t] * len(sub), check=chk if last else None)
            assert np.array_equal(logits[rows].view(np.uint32), l2.view(np.uint32)), (t, sub)
            assert np.array_equal(nxt[rows], n2), (t, sub)
        for i, s in enumerate(streams):
            tok[s] = int(nxt[i])
    # a page holds 16 steps of every stream of one layer
    free_after, used_after = dec.kv_pages()
    assert free_after + used_after == free and used_after == 2 * ((n_steps + 15) // 16)
    print("[worst teacher-forced errors]", chk.worst, flush=True)

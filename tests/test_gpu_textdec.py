"""GPU parity of the speech-LLM text-decoder path (config 4): RoPE, SwiGLU and
the batched device-resident step over Q4_K linears and the paged Q8_0 cache.

Bars:
  * ops: RoPE and SwiGLU against the oracle's restatements of rope_apply /
    silu_inplace + hadamard_inplace, within bounds derived from the one place
    they differ (device sin / cos / exp against libm, a few ulp);
  * session == the same step issued one C-ABI entry point at a time, bit for
    bit, at config-4 dims (every kernel on the path is row-independent, and
    the paged attention's results depend only on an item's own keys);
  * teacher-forced: every entry point of that chain, fed the GPU's own inputs,
    against the oracle function it replaces (Q4_K linears bit-exact, RMSNorm
    / RoPE / SwiGLU / attention within their derived bounds), so a systematic
    error anywhere in the step fails;
  * free-running session vs the oracle composition (tests/model_oracle.py):
    logits within 0.1 rms (INT8 rounding flips spread) and greedy tokens equal
    wherever the oracle's top-2 gap is wider than that.
"""
import numpy as np
import pytest

from tests import model_oracle
from vokra_amd import hip

pytestmark = pytest.mark.gpu

W_Q4_K = 12
W_Q8_0 = 8
U = 2.0 ** -24


@pytest.fixture(scope="module")
def ctx():
    c = hip.HipContext(0)
    yield c
    c.close()


# ---- ops -----------------------------------------------------------------
@pytest.mark.parametrize("n_head,hd,base", [(16, 128, 1e6), (2, 128, 1e6), (4, 64, 1e4)])
def test_rope_vs_oracle(ctx, oracle, n_head, hd, base):
    print(f"[case] rope H={n_head} hd={hd}", flush=True)
    g = np.random.default_rng(hd + n_head)
    for off, t in ((0, 1), (5, 3), (511, 2), (4094, 2)):
        x = g.standard_normal((t, n_head * hd)).astype(np.float32)
        got = ctx.rope_f32(x, t, n_head, hd, base, off).reshape(t, n_head * hd)
        want = oracle.rope_heads(x, n_head, hd, base, off)
        xr = x.reshape(t, n_head, 2, hd // 2)
        mag = np.abs(xr[:, :, 0, :]) + np.abs(xr[:, :, 1, :])
        bound = np.concatenate([mag, mag], axis=-1).reshape(t, -1).astype(np.float64) * 8 * U
        err = np.abs(got.astype(np.float64) - want)
        assert np.all(err <= bound + 1e-30), (off, float(np.max(err - bound)))
    # position 0 is the identity, exactly
    x = g.standard_normal((1, n_head * hd)).astype(np.float32)
    assert np.array_equal(ctx.rope_f32(x, 1, n_head, hd, base, 0), x)
    # per-row positions on device == copy mode at the same offsets
    rows = g.standard_normal((3, n_head * hd)).astype(np.float32)
    d_x = hip.DeviceBuffer.from_array(ctx, rows)
    d_p = hip.DeviceBuffer.from_array(ctx, np.array([7, 0, 4000], np.int32))
    ctx.rope_f32_dev(d_x, 3, n_head, hd, base, d_p)
    dev = d_x.download(np.float32, rows.size).reshape(3, -1)
    for r, p in enumerate((7, 0, 4000)):
        assert np.array_equal(dev[r], ctx.rope_f32(rows[r], 1, n_head, hd, base, p).reshape(-1))


def test_rope_rejections(ctx):
    with pytest.raises(hip.InvalidArgument, match="even"):
        ctx.rope_f32(np.zeros(3, np.float32), 1, 1, 3, 1e4, 0)
    with pytest.raises(hip.InvalidArgument, match="len"):
        ctx.rope_f32(np.zeros(5, np.float32), 1, 1, 4, 1e4, 0)


def test_swiglu_vs_oracle(ctx, oracle):
    print("[case] swiglu", flush=True)
    g = np.random.default_rng(3)
    gate = np.concatenate([np.linspace(-30, 30, 6001), g.standard_normal(20000) * 4]).astype(np.float32)
    up = g.standard_normal(gate.size).astype(np.float32)
    got = ctx.swiglu_f32(gate, up).astype(np.float64)
    want = oracle.swiglu(gate, up).astype(np.float64)
    # the device expf and libm expf differ by at most a couple of ulp; the
    # add, divide and two products then keep it within 8 ulp of the result
    assert np.all(np.abs(got - want) <= 8 * U * np.abs(want) + 1e-38)
    with pytest.raises(hip.InvalidArgument, match="length mismatch"):
        ctx.swiglu_f32(gate[:4], up[:3])


# ---- the session -----------------------------------------------------------
def make_layers(oracle, g, n_layer, d, hq, hkv, hd, ff, scale=0.03, wd=W_Q4_K):
    return [model_oracle.random_text_layer(oracle, g, d, hq, hkv, hd, ff, scale, wd) for _ in range(n_layer)]


class TextDecoderByOps:
    """The text-decoder step issued one C-ABI entry point at a time: RMSNorm,
    Q4_K linears (kquant_gemm_i8), RoPE per row at its position, the paged
    cache's append and decode attention, SwiGLU, residual adds in numpy,
    final RMSNorm, LM head and argmax. With `check`, each entry point's
    output is also held against the oracle on the same inputs."""

    def __init__(self, ctx, P, n_stream, check=None):
        self.ctx, self.P, self.check = ctx, P, check
        self.kv = ctx.kv_cache(len(P["layers"]), P["hkv"], P["hd"], n_stream, P["n_ctx"], P["bs"])
        self.pos = [0] * n_stream
        self.worst = {}

    def note(self, what, err):
        self.worst[what] = max(self.worst.get(what, 0.0), float(err))

    def restore(self, s, k_rows, v_rows):
        for l in range(k_rows.shape[0]):
            for t0 in range(0, k_rows.shape[1], 1024):
                t1 = min(k_rows.shape[1], t0 + 1024)
                self.kv.append(l, [s] * (t1 - t0), list(range(t0, t1)), k_rows[l, t0:t1], v_rows[l, t0:t1])
        self.pos[s] = k_rows.shape[1]

    def lin(self, x, w, n, k):
        wd = self.P.get("wd", W_Q4_K)
        y = self.ctx.gemm_q_f32(x.shape[0], n, k, x, w, hip.WDtype(wd))
        if self.check is not None:
            rows = min(2, x.shape[0])
            want = self.check.gemm_q_f32(wd, rows, n, k, x[:rows], w)
            assert np.array_equal(y[:rows].view(np.uint32), want.view(np.uint32)), f"linear (dtype {wd})"
        return y

    def rms(self, h, gamma):
        n, d = h.shape
        y = self.ctx.rms_norm_f32(h, n, d, gamma, self.P["eps"])
        if self.check is not None:
            want = self.check.rms_norm_f32(h, gamma, self.P["eps"], n, d).astype(np.float64)
            err = np.abs(y - want) / (np.abs(want) + 1e-30)
            self.note("rms_norm rel", err.max())
            assert np.all(np.abs(y - want) <= (d / 2 + 8) * U * np.abs(want) + 1e-30), "rms_norm"
        return y

    def rope(self, x, n_head, positions):
        P = self.P
        out = np.stack([self.ctx.rope_f32(x[i], 1, n_head, P["hd"], P["base"], p) for i, p in enumerate(positions)])
        if self.check is not None:
            for i, p in enumerate(positions[:2]):
                want = self.check.rope_heads(x[i:i + 1], n_head, P["hd"], P["base"], p)[0]
                xr = x[i].reshape(n_head, 2, P["hd"] // 2)
                mag = np.abs(xr[:, 0]) + np.abs(xr[:, 1])
                bound = np.concatenate([mag, mag], axis=-1).reshape(-1) * 8 * U
                assert np.all(np.abs(out[i] - want) <= bound + 1e-30), "rope"
        return out

    def step(self, streams, tokens):
        ctx, P = self.ctx, self.P
        n, d, hq, hkv, hd, ff = len(streams), P["d"], P["hq"], P["hkv"], P["hd"], P["ff"]
        positions = [self.pos[s] for s in streams]
        lens = [p + 1 for p in positions]
        scale = float(np.float32(1.0) / np.sqrt(np.float32(hd)))
        h = P["tok"][tokens].astype(np.float32)
        for l, L in enumerate(P["layers"]):
            x = self.rms(h, L["attn_norm_gamma"])
            q = self.rope(self.lin(x, L["wq"], hq * hd, d), hq, positions)
            k = self.rope(self.lin(x, L["wk"], hkv * hd, d), hkv, positions)
            v = self.lin(x, L["wv"], hkv * hd, d)
            self.kv.append(l, streams, positions, k, v)
            a = self.kv.attn(l, streams, lens, q, hq, scale)
            if self.check is not None:
                s0 = streams[0]
                rows = [self.kv.read(l, t, s0) for t in range(lens[0])]
                K = np.stack([r[0] for r in rows])
                V = np.stack([r[1] for r in rows])
                want = self.check.gqa_attention(1, lens[0], hq, hkv, hd, q[0:1], K, V, scale, positions[0])[0]
                err = np.abs(a[0] - want)
                self.note("attention", err.max())
                assert np.all(err <= 1e-4 + 1e-3 * np.abs(want)), "attention"
            h = self.lin(a, L["wo"], d, hq * hd) + h
            x = self.rms(h, L["ffn_norm_gamma"])
            gt, up = self.lin(x, L["w_gate"], ff, d), self.lin(x, L["w_up"], ff, d)
            f = ctx.swiglu_f32(gt, up).reshape(n, ff)
            if self.check is not None:
                want = self.check.swiglu(gt[:2], up[:2]).astype(np.float64)
                assert np.all(np.abs(f[:2] - want) <= 8 * U * np.abs(want) + 1e-38), "swiglu"
            h = self.lin(f, L["w_down"], d, ff) + h
        x = self.rms(h, P["final"])
        for s in streams:
            self.pos[s] += 1
        if P["head"] is not None:
            logits = self.lin(x, P["head"], P["V"], d)
            return np.argmax(logits, axis=1).astype(np.int32), logits
        # tied head: the fused f32 logits + argmax entry point
        V = P["V"]
        d_x, d_e = hip.DeviceBuffer.from_array(ctx, x), hip.DeviceBuffer.from_array(ctx, P["tok"])
        d_l, d_n = hip.DeviceBuffer(ctx, n * V * 4), hip.DeviceBuffer(ctx, n * 4)
        ctx.logits_argmax_dev(n, V, d, d_x, d_e, d_l, d_n)
        ctx.synchronize()
        return d_n.download(np.int32, n), d_l.download(np.float32, n * V).reshape(n, V)


def build(ctx, oracle, seed, n_layer, d, hq, hkv, hd, ff, V, n_ctx, n_stream, bs=16, tied=False, base=1e6,
          eps=1e-5, wd=W_Q4_K):
    g = np.random.default_rng(seed)
    layers = make_layers(oracle, g, n_layer, d, hq, hkv, hd, ff, wd=wd)
    tok = (g.standard_normal((V, d)) * 0.5).astype(np.float32)
    fin = (1 + 0.1 * g.standard_normal(d)).astype(np.float32)
    head = None if tied else model_oracle.quantize_weight(oracle, wd, (g.standard_normal((V, d)) * 0.03)
                                                          .astype(np.float32))
    P = dict(layers=layers, tok=tok, final=fin, head=head, d=d, hq=hq, hkv=hkv, hd=hd, ff=ff, V=V, n_ctx=n_ctx,
             bs=bs, base=base, eps=eps, wd=wd)
    dec = hip.TextDecoder(ctx, wd, d, hq, hkv, hd, ff, V, n_ctx, n_stream, layers, tok, fin, head,
                          rope_base=base, rms_norm_eps=eps, block_size=bs)
    return dec, P


def history(g, n_layer, n_pos, w, scale=1.0):
    k = (g.standard_normal((n_layer, n_pos, w)) * scale).astype(np.float32)
    v = (g.standard_normal((n_layer, n_pos, w)) * scale).astype(np.float32)
    return k, v


@pytest.mark.parametrize("wd,tied,hkv", [(W_Q4_K, False, 2), (W_Q4_K, True, 2), (W_Q4_K, False, 4),
                                         (W_Q8_0, False, 2), (W_Q8_0, True, 4), (2, False, 2), (6, True, 4),
                                         (13, False, 2), (14, True, 2)])
def test_text_decoder_small_vs_oracle(ctx, oracle, wd, tied, hkv):
    """Toy dims (d=256, 4 query heads x 64 over 2 kv heads, or 4 = no
    grouping): session == entry points bit for bit, teacher-forced entry
    points vs the oracle, free-running vs the oracle. Q8_0 weights (and Q4_0
    (2), Q5_0 (6)) take the block-format route of the step (RMSNorm and the block activation pass as
    two launches, a separate SwiGLU pass, RoPE as its own launch, paged
    attention without the rotation table); Q5_K (13) and Q6_K (14) the
    K-quant route with the byte-word matmul."""
    print(f"[case] text decoder small wd={wd} tied={tied} hkv={hkv}", flush=True)
    d, hq, hd, ff, V, n_ctx, n_stream = 256, 4, 64, 512, 96, 64, 3
    dec, P = build(ctx, oracle, 11, 2, d, hq, hkv, hd, ff, V, n_ctx, n_stream, bs=4, tied=tied, wd=wd)
    ops = TextDecoderByOps(ctx, P, n_stream, check=oracle)
    ref = model_oracle.TextDecoder(oracle, P["layers"], P["tok"], P["final"], P["head"], hq, hkv, hd, ff, n_stream,
                                   n_ctx, 4, P["base"], P["eps"], wd=wd)
    tok = [1, 2, 3]
    schedule = [[0, 1, 2], [0, 1], [2, 0], [1, 2, 0], [0], [2, 1, 0]]
    for step, streams in enumerate(schedule):
        args = [tok[s] for s in streams]
        nxt, logits = dec.step(streams, args, want_logits=True)
        n2, l2 = ops.step(streams, args)
        assert np.array_equal(logits, l2) and np.array_equal(nxt, n2), (step, streams)
        for i, s in enumerate(streams):
            want, want_tok = ref.step(s, tok[s], dec.position(s) - 1)
            rms = float(np.sqrt(np.mean(want.astype(np.float64) ** 2)))
            err = float(np.max(np.abs(logits[i] - want)))
            assert err <= 0.1 * rms + 1e-4, (step, s, err, rms)
            top2 = np.sort(want)[-2:]
            if top2[1] - top2[0] > 0.1 * rms + 1e-4:
                assert nxt[i] == want_tok, (step, s)
            tok[s] = int(nxt[i])


def test_text_decoder_config4_dims(ctx, oracle):
    """Config-4 shapes (d=2048, 16/2 heads x 128, FFN 5632, 32000-token Q4_K
    LM head) with 2 layers and 6 streams whose histories (restored rows)
    reach 512..4096 positions: session == entry points bit for bit over
    ragged steps, every entry point teacher-forced against the oracle, the
    session free-running against the oracle composition, and batch ==
    single-stream steps in a twin session."""
    print("[case] text decoder config-4 dims", flush=True)
    d, hq, hkv, hd, ff, V, n_ctx, n_stream, n_layer = 2048, 16, 2, 128, 5632, 32000, 4096, 6, 2
    dec, P = build(ctx, oracle, 4, n_layer, d, hq, hkv, hd, ff, V, n_ctx, n_stream)
    twin, _ = build(ctx, oracle, 4, n_layer, d, hq, hkv, hd, ff, V, n_ctx, n_stream)
    ops = TextDecoderByOps(ctx, P, n_stream, check=oracle)
    ref = model_oracle.TextDecoder(oracle, P["layers"], P["tok"], P["final"], P["head"], hq, hkv, hd, ff, n_stream,
                                   n_ctx, 16, P["base"], P["eps"])
    g = np.random.default_rng(40)
    lens = [512, 4090, 1000, 2048, 3584, 600]
    for s, n_pos in enumerate(lens):
        k, v = history(g, n_layer, n_pos, hkv * hd)
        dec.kv_restore(s, k, v)
        twin.kv_restore(s, k, v)
        ops.restore(s, k, v)
        ref.restore(s, k, v)
        assert dec.position(s) == n_pos
    tok = [int(t) for t in g.integers(0, V, n_stream)]
    for step, streams in enumerate([[0, 1, 2, 3, 4, 5], [5, 1, 3], [2, 0, 4, 1]]):
        args = [tok[s] for s in streams]
        pos_before = [dec.position(s) for s in streams]
        nxt, logits = dec.step(streams, args, want_logits=True)
        n2, l2 = ops.step(streams, args)
        assert np.array_equal(logits, l2) and np.array_equal(nxt, n2), (step, streams)
        for i, s in enumerate(streams):
            n1, l1 = twin.step([s], [args[i]], want_logits=True)
            assert np.array_equal(l1[0], logits[i]) and n1[0] == nxt[i], (step, s)
        for i, s in enumerate(streams):
            want, want_tok = ref.step(s, tok[s], pos_before[i])
            rms = float(np.sqrt(np.mean(want.astype(np.float64) ** 2)))
            err = float(np.max(np.abs(logits[i] - want)))
            assert err <= 0.1 * rms + 1e-4, (step, s, err, rms)
            top2 = np.sort(want)[-2:]
            if top2[1] - top2[0] > 0.1 * rms + 1e-4:
                assert nxt[i] == want_tok, (step, s)
        for i, s in enumerate(streams):
            tok[s] = int(nxt[i])
    print("[worst teacher-forced errors]", ops.worst, flush=True)


def test_text_decoder_rows_wider_than_2048(ctx, oracle):
    """d = 2304 (9 super-blocks): the RMSNorm + activation pass streams rows
    wider than the 2048 columns it holds in registers, and the final RMSNorm
    likewise. Session == entry points bit for bit, every entry point
    teacher-forced against the oracle."""
    print("[case] text decoder d=2304", flush=True)
    d, hq, hkv, hd, ff, V, n_ctx, n_stream, n_layer = 2304, 4, 2, 64, 512, 64, 32, 2, 1
    dec, P = build(ctx, oracle, 23, n_layer, d, hq, hkv, hd, ff, V, n_ctx, n_stream, bs=4)
    ops = TextDecoderByOps(ctx, P, n_stream, check=oracle)
    tok = [3, 7]
    for step, streams in enumerate([[0, 1], [1], [0, 1], [1, 0]]):
        args = [tok[s] for s in streams]
        nxt, logits = dec.step(streams, args, want_logits=True)
        n2, l2 = ops.step(streams, args)
        assert np.array_equal(logits, l2) and np.array_equal(nxt, n2), (step, streams)
        for i, s in enumerate(streams):
            tok[s] = int(nxt[i])
    print("[worst teacher-forced errors]", ops.worst, flush=True)


def test_text_decoder_histories_beyond_4096(ctx, oracle):
    """Histories past 4096 positions, where the attention splits grow to 1024
    and 1536 keys: the steps cross 4096 -> 4097 keys (512- to 1024-key
    splits), 5120 -> 5121 (the new key alone in the last split) and 8192 ->
    8193 (1024- to 1536-key splits), so the K/V append and RoPE of the step
    run in each kind of split. Session == entry points bit for bit, every
    entry point teacher-forced against the oracle."""
    print("[case] text decoder histories beyond 4096", flush=True)
    d, hq, hkv, hd, ff, V, n_ctx, n_stream, n_layer = 1024, 8, 2, 128, 512, 96, 8704, 4, 2
    dec, P = build(ctx, oracle, 31, n_layer, d, hq, hkv, hd, ff, V, n_ctx, n_stream)
    ops = TextDecoderByOps(ctx, P, n_stream, check=oracle)
    g = np.random.default_rng(31)
    lens = [4095, 5119, 8191, 8600]
    for s, n_pos in enumerate(lens):
        k, v = history(g, n_layer, n_pos, hkv * hd)
        dec.kv_restore(s, k, v)
        ops.restore(s, k, v)
    streams = list(range(n_stream))
    tok = [int(t) for t in g.integers(0, V, n_stream)]
    for step in range(3):
        args = [tok[s] for s in streams]
        nxt, logits = dec.step(streams, args, want_logits=True)
        n2, l2 = ops.step(streams, args)
        assert np.array_equal(logits, l2) and np.array_equal(nxt, n2), step
        for i, s in enumerate(streams):
            tok[s] = int(nxt[i])
    assert [dec.position(s) for s in streams] == [n + 3 for n in lens]
    print("[worst teacher-forced errors]", ops.worst, flush=True)


def test_text_decoder_full_depth_equals_entry_points(ctx, oracle):
    """All 24 config-4 layers, 32 streams with histories U(512..4096): two
    batched steps are bit-identical to the entry-point chain."""
    print("[case] text decoder 24 layers x 32 streams", flush=True)
    d, hq, hkv, hd, ff, V, n_ctx, n_stream, n_layer = 2048, 16, 2, 128, 5632, 32000, 4096, 32, 24
    dec, P = build(ctx, oracle, 24, n_layer, d, hq, hkv, hd, ff, V, n_ctx, n_stream)
    ops = TextDecoderByOps(ctx, P, n_stream)
    g = np.random.default_rng(24)
    lens = g.integers(512, 4097, n_stream)
    kk, vv = history(g, n_layer, int(lens.max()), hkv * hd)
    for s in range(n_stream):
        dec.kv_restore(s, kk[:, :lens[s]], vv[:, :lens[s]])
        ops.restore(s, kk[:, :lens[s]], vv[:, :lens[s]])
    streams = list(range(n_stream))
    tok = [int(t) for t in g.integers(0, V, n_stream)]
    for step in range(2):
        live = [s for s in streams if lens[s] + step < n_ctx]
        nxt, logits = dec.step(live, [tok[s] for s in live], want_logits=True)
        n2, l2 = ops.step(live, [tok[s] for s in live])
        assert np.array_equal(logits, l2) and np.array_equal(nxt, n2), step
        for i, s in enumerate(live):
            tok[s] = int(nxt[i])


def test_text_decoder_rejections(ctx, oracle):
    g = np.random.default_rng(5)
    d, hq, hkv, hd, ff, V = 256, 4, 2, 64, 512, 50
    layers = make_layers(oracle, g, 1, d, hq, hkv, hd, ff)
    tok = np.zeros((V, d), np.float32)
    fin = np.ones(d, np.float32)
    dec = hip.TextDecoder(ctx, W_Q4_K, d, hq, hkv, hd, ff, V, 8, 2, layers, tok, fin, None, block_size=4)
    with pytest.raises(hip.InvalidArgument, match="token id 50 >= vocab 50"):
        dec.step([0], [50])
    with pytest.raises(hip.InvalidArgument, match="distinct"):
        dec.step([1, 1], [1, 2])
    k, v = history(g, 1, 8, hkv * hd)
    dec.kv_restore(0, k, v)
    with pytest.raises(hip.InvalidArgument, match="position 9 > n_ctx 8"):
        dec.step([0], [1])
    dec.step([1], [1])                 # the other stream is unaffected
    assert dec.position(1) == 1
    dec.reset()
    assert dec.position(0) == 0 and dec.position(1) == 0
    with pytest.raises(hip.ModelLoad, match="divisible"):
        hip.TextDecoder(ctx, W_Q4_K, d, 3, 2, hd, ff, V, 8, 1, layers, tok, fin)
    with pytest.raises(hip.UnsupportedOp):
        hip.TextDecoder(ctx, W_Q4_K, d, 4, 2, 96, ff, V, 8, 1, layers, tok, fin)


# ---- the text decoder straight from a GGUF file --------------------------------
def voxtral_gguf(path, P, prefix, n_ctx, tied, f16_norms=False, drop=None, replace=None):
    """The decoder of P written with TextDecoder::load's tensor names
    (text_decoder.rs:484-575) under `prefix`, the lm_head beside the decoder
    submodule, and the vokra.voxtral.* metadata (explicit head_dim)."""
    from tests import gguf_writer as gw
    d, hq, hkv, hd, ff, V = P["d"], P["hq"], P["hkv"], P["hd"], P["ff"], P["V"]
    wd = P.get("wd", W_Q4_K)
    gt = {W_Q4_K: gw.GGML_Q4_K, W_Q8_0: gw.GGML_Q8_0, 2: gw.GGML_Q4_0, 6: gw.GGML_Q5_0, 13: gw.GGML_Q5_K,
          14: gw.GGML_Q6_K}[wd]
    m = [("vokra.voxtral." + k, t, v) for k, t, v in (
        ("audio_encoder.n_layer", gw.U32, 2), ("audio_encoder.hidden_dim", gw.U32, 256),
        ("audio_encoder.n_head", gw.U32, 4), ("audio_encoder.n_mels", gw.U32, 128),
        ("text_decoder.n_layer", gw.U32, len(P["layers"])), ("text_decoder.hidden_dim", gw.U32, d),
        ("text_decoder.ffn_dim", gw.U32, ff), ("text_decoder.vocab_size", gw.U32, V),
        ("text_decoder.n_ctx", gw.U32, n_ctx), ("text_decoder.n_head_q", gw.U32, hq),
        ("text_decoder.n_head_kv", gw.U32, hkv), ("text_decoder.head_dim", gw.U32, hd),
        ("text_decoder.rope_base", gw.F32, P["base"]), ("text_decoder.rms_norm_eps", gw.F32, P["eps"]))]
    t = []

    def norm(name, a):
        if f16_norms:
            t.append((name, [a.size], gw.GGML_F16, a.astype(np.float16).tobytes()))
        else:
            t.append((name, [a.size], gw.GGML_F32, a.astype(np.float32).tobytes()))

    t.append((prefix + "embed_tokens.weight", [V, d], gw.GGML_F32, P["tok"].tobytes()))
    for i, L in enumerate(P["layers"]):
        p = f"{prefix}layers.{i}"
        norm(p + ".input_layernorm.weight", L["attn_norm_gamma"])
        for name, key, n, k in (("self_attn.q_proj", "wq", hq * hd, d), ("self_attn.k_proj", "wk", hkv * hd, d),
                                ("self_attn.v_proj", "wv", hkv * hd, d), ("self_attn.o_proj", "wo", d, hq * hd)):
            t.append((f"{p}.{name}.weight", [n, k], gt, bytes(np.asarray(L[key], np.uint8))))
        norm(p + ".post_attention_layernorm.weight", L["ffn_norm_gamma"])
        for name, key, n, k in (("mlp.gate_proj", "w_gate", ff, d), ("mlp.up_proj", "w_up", ff, d),
                                ("mlp.down_proj", "w_down", d, ff)):
            t.append((f"{p}.{name}.weight", [n, k], gt, bytes(np.asarray(L[key], np.uint8))))
    norm(prefix + "norm.weight", P["final"])
    if not tied:
        # lm_head_base (text_decoder.rs:763-768): strip a trailing "model."
        # only where what is left is empty or ends in a dot
        base = prefix
        if prefix.endswith("model.") and (prefix[:-6] == "" or prefix[:-6].endswith(".")):
            base = prefix[:-6]
        t.append((base + "lm_head.weight", [V, d], gt, bytes(np.asarray(P["head"], np.uint8))))
    if drop:
        t = [x for x in t if x[0] != drop]
    if replace:
        t = [replace.get(x[0], x) for x in t]
    path.write_bytes(gw.build(m, t))
    return hip.GgufFile(str(path))


@pytest.mark.parametrize("prefix,tied,wd", [("language_model.model.", False, W_Q4_K), ("model.", True, W_Q4_K),
                                            ("language_model.", False, W_Q8_0), ("model.", False, 6),
                                            ("language_model.model.", False, 13), ("model.", True, 14)])
def test_text_decoder_from_gguf_equals_direct(ctx, oracle, tmp_path, prefix, tied, wd):
    """vokra_hip_text_decoder_from_gguf (TextDecoder::load + VoxtralConfig::
    from_gguf) == the session built from the same arrays, bit for bit, over
    ragged steps from restored histories; the three tensor prefixes of
    pick_prefix, the untied head beside the decoder submodule and the tied
    one; F16 norms widen exactly."""
    print(f"[case] text decoder from gguf prefix={prefix} tied={tied} wd={wd}", flush=True)
    d, hq, hkv, hd, ff, V, n_ctx, n_stream = 256, 4, 2, 64, 512, 96, 64, 3
    dec, P = build(ctx, oracle, 21, 2, d, hq, hkv, hd, ff, V, n_ctx, n_stream, bs=4, tied=tied, wd=wd)
    f = voxtral_gguf(tmp_path / "td.gguf", P, prefix, n_ctx, tied, f16_norms=True)
    # the direct session sees the same F16-rounded norms the file holds
    for L in P["layers"]:
        for key in ("attn_norm_gamma", "ffn_norm_gamma"):
            L[key] = L[key].astype(np.float16).astype(np.float32)
    P["final"] = P["final"].astype(np.float16).astype(np.float32)
    direct = hip.TextDecoder(ctx, wd, d, hq, hkv, hd, ff, V, n_ctx, n_stream, P["layers"], P["tok"], P["final"],
                             P["head"], rope_base=P["base"], rms_norm_eps=P["eps"], block_size=4)
    loaded, rep = hip.TextDecoder.from_gguf(ctx, f, wd, n_stream, block_size=4)
    assert rep == {"verbatim": 7 * 2 + (0 if tied else 1), "packed": 0}
    g = np.random.default_rng(22)
    for s, n_pos in enumerate((5, 0, 17)):
        k, v = history(g, 2, n_pos, hkv * hd)
        direct.kv_restore(s, k, v)
        loaded.kv_restore(s, k, v)
    tok = [3, 7, 11]
    for streams in ([0, 1, 2], [2, 0], [1]):
        args = [tok[s] for s in streams]
        n1, l1 = direct.step(streams, args, want_logits=True)
        n2, l2 = loaded.step(streams, args, want_logits=True)
        assert np.array_equal(l1.view(np.uint32), l2.view(np.uint32)) and np.array_equal(n1, n2), streams
        for i, s in enumerate(streams):
            tok[s] = int(n1[i])


def test_text_decoder_from_gguf_errors(ctx, oracle, tmp_path):
    """TextDecoder::load's errors, naming the tensor in the reference's order:
    a missing layer tensor, a mis-shaped projection, and a present but
    mis-shaped lm_head (never a silent tie); a Q8_0 file for a Q4_K session."""
    print("[case] text decoder from gguf errors", flush=True)
    from tests import gguf_writer as gw
    d, hq, hkv, hd, ff, V = 256, 4, 2, 64, 512, 96
    _, P = build(ctx, oracle, 23, 1, d, hq, hkv, hd, ff, V, 16, 1, bs=4)
    pre = "language_model.model."
    name = pre + "layers.0.mlp.up_proj.weight"
    with pytest.raises(hip.ModelLoad, match=rf"voxtral text_decoder: `{name}` missing from GGUF"):
        hip.TextDecoder.from_gguf(ctx, voxtral_gguf(tmp_path / "a.gguf", P, pre, 16, False, drop=name), W_Q4_K, 1)
    w = pre + "layers.0.self_attn.k_proj.weight"
    bad = {w: (w, [d, hkv * hd], gw.GGML_Q4_K, bytes(np.asarray(P["layers"][0]["wk"], np.uint8)))}
    with pytest.raises(hip.ModelLoad, match=rf"`{w}` shape \[{d}, {hkv * hd}\] != expected \[{hkv * hd}, {d}\]"):
        hip.TextDecoder.from_gguf(ctx, voxtral_gguf(tmp_path / "b.gguf", P, pre, 16, False, replace=bad), W_Q4_K, 1)
    h = "language_model.lm_head.weight"
    bad = {h: (h, [V - 1, d], gw.GGML_F32, bytes((V - 1) * d * 4))}
    with pytest.raises(hip.ModelLoad, match=rf"`{h}` shape \[{V - 1}, {d}\] != expected \[{V}, {d}\]"):
        hip.TextDecoder.from_gguf(ctx, voxtral_gguf(tmp_path / "c.gguf", P, pre, 16, False, replace=bad), W_Q4_K, 1)
    with pytest.raises(hip.UnsupportedOp, match=r"`language_model\.model\.layers\.0\.self_attn\.q_proj\.weight`: "
                                                r"Q4_K on disk"):
        hip.TextDecoder.from_gguf(ctx, voxtral_gguf(tmp_path / "d.gguf", P, pre, 16, False), W_Q8_0, 1)

"""Resident-mode entry points (device pointers, asynchronous on the context
stream) against their copy-mode twins: the same kernels behind both, so the
outputs must agree bit for bit. The copy-mode forms carry the parity tests
against the oracle; this pins the device-pointer plumbing of each _dev form."""
import numpy as np
import pytest

from vokra_amd import hip

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    c = hip.HipContext(0)
    yield c
    c.close()


def dev(ctx, a):
    return hip.DeviceBuffer.from_array(ctx, np.ascontiguousarray(a))


def down(ctx, buf, dtype, n):
    ctx.synchronize()
    return buf.download(dtype, n)


def bits(a):
    return np.ascontiguousarray(a, np.float32).reshape(-1).view(np.uint32)


def test_gemv_softmax_rms_swiglu_dev_equal_copy_mode(ctx):
    print("[case] resident f32 kernels", flush=True)
    g = np.random.default_rng(1)
    m, k = 37, 300
    a = g.standard_normal((m, k)).astype(np.float32)
    x = g.standard_normal(k).astype(np.float32)
    b = g.standard_normal(m).astype(np.float32)
    out = hip.DeviceBuffer(ctx, m * 4)
    ctx.gemv_f32_dev(m, k, dev(ctx, a), dev(ctx, x), out, dev(ctx, b))
    assert np.array_equal(bits(down(ctx, out, np.float32, m)), bits(ctx.gemv_f32(m, k, a, x, b)))

    rows, cols = 5, 777
    s = (g.standard_normal((rows, cols)) * 4).astype(np.float32)
    out = hip.DeviceBuffer(ctx, rows * cols * 4)
    ctx.softmax_f32_dev(dev(ctx, s), out, rows, cols)
    assert np.array_equal(bits(down(ctx, out, np.float32, rows * cols)), bits(ctx.softmax_f32(s, rows, cols)))

    for cols in (2048, 2304):   # rows held in registers, and streamed
        r = g.standard_normal((3, cols)).astype(np.float32)
        gam = (1 + 0.1 * g.standard_normal(cols)).astype(np.float32)
        out = hip.DeviceBuffer(ctx, 3 * cols * 4)
        ctx.rms_norm_f32_dev(dev(ctx, r), out, 3, cols, dev(ctx, gam), 1e-5)
        assert np.array_equal(bits(down(ctx, out, np.float32, 3 * cols)),
                              bits(ctx.rms_norm_f32(r, 3, cols, gam, 1e-5)))

    n = 10001
    gate = (g.standard_normal(n) * 4).astype(np.float32)
    up = g.standard_normal(n).astype(np.float32)
    out = hip.DeviceBuffer(ctx, n * 4)
    ctx.swiglu_f32_dev(dev(ctx, gate), dev(ctx, up), n, out)
    assert np.array_equal(bits(down(ctx, out, np.float32, n)), bits(ctx.swiglu_f32(gate, up)))


def test_conv1d_dev_equals_copy_mode(ctx):
    print("[case] resident conv1d", flush=True)
    g = np.random.default_rng(2)
    in_ch, in_len, out_ch, kernel, stride, padding = 3, 50, 4, 3, 2, 1
    x = g.standard_normal((in_ch, in_len)).astype(np.float32)
    w = g.standard_normal((out_ch, in_ch, kernel)).astype(np.float32)
    bias = g.standard_normal(out_ch).astype(np.float32)
    want = ctx.conv1d_f32(x, in_ch, in_len, w, out_ch, kernel, bias, stride, padding)
    out_len = (in_len + 2 * padding - kernel) // stride + 1
    assert want.shape == (out_ch, out_len)
    out = hip.DeviceBuffer(ctx, out_ch * out_len * 4)
    ctx.conv1d_f32_dev(dev(ctx, x), in_ch, in_len, dev(ctx, w), out_ch, kernel, dev(ctx, bias), stride, padding, out)
    assert np.array_equal(bits(down(ctx, out, np.float32, out_ch * out_len)), bits(want))


@pytest.mark.parametrize("mode", [hip.KvQuant.Q4_0, hip.KvQuant.Q5_0, hip.KvQuant.Q8_0])
def test_quantize_bytes_dev_equals_copy_mode(ctx, mode):
    print(f"[case] resident quantize_bytes {mode.name}", flush=True)
    g = np.random.default_rng(int(mode))
    x = (g.standard_normal(32 * 301) * 3).astype(np.float32)
    x[:32] = 0.0
    want = ctx.quantize_bytes(mode, x)
    out = hip.DeviceBuffer(ctx, want.size)
    ctx.quantize_bytes_dev(mode, dev(ctx, x), x.size, out)
    assert np.array_equal(down(ctx, out, np.uint8, want.size), want)


def test_kv_append_dev_equals_copy_mode(ctx):
    """Two caches fed the same batch, one through host arrays and one through
    device arrays: the same pages, the same rows, the same status."""
    print("[case] resident kv append", flush=True)
    H, hd, n_stream, max_time, bs = 2, 64, 3, 24, 4
    a = ctx.kv_cache(2, H, hd, n_stream, max_time, bs)
    b = ctx.kv_cache(2, H, hd, n_stream, max_time, bs)
    g = np.random.default_rng(3)
    for layer, streams, times in ((1, [0, 2, 1], [0, 5, 9]), (0, [1, 1, 2], [3, 4, 23])):
        k = g.standard_normal((3, H * hd)).astype(np.float32)
        v = g.standard_normal((3, H * hd)).astype(np.float32)
        a.append(layer, streams, times, k, v)
        b.append_dev(layer, 3, dev(ctx, np.array(streams, np.int32)), dev(ctx, np.array(times, np.int32)),
                     dev(ctx, k), dev(ctx, v))
        assert b.status() == 3
        assert a.pages() == b.pages()
        for s, t in zip(streams, times):
            ra, rb = a.read(layer, t, s), b.read(layer, t, s)
            assert np.array_equal(bits(ra[0]), bits(rb[0])) and np.array_equal(bits(ra[1]), bits(rb[1]))


@pytest.mark.parametrize("H,hd,hq,lens", [(4, 64, 4, [200, 1, 77, 131]),          # one q head per kv head
                                          (2, 128, 16, [1500, 4097, 33, 600])])  # GQA, key splits + combine
def test_paged_attn_dev_equals_copy_mode(ctx, H, hd, hq, lens):
    print(f"[case] resident paged attn H={H} hd={hd} hq={hq}", flush=True)
    n_stream, max_time, bs = len(lens), max(lens), 16
    kv = ctx.kv_cache(1, H, hd, n_stream, max_time, bs)
    g = np.random.default_rng(hd + hq)
    for t in range(max(lens)):
        live = [s for s in range(n_stream) if lens[s] > t]
        rows = g.standard_normal((2, len(live), H * hd)).astype(np.float32)
        kv.append(0, live, [t] * len(live), rows[0], rows[1])
    order = [3, 1, 0, 2]
    ln = [lens[s] for s in order]
    q = g.standard_normal((n_stream, hq * hd)).astype(np.float32)
    scale = float(np.float32(hd) ** np.float32(-0.5))
    want = kv.attn(0, order, ln, q, hq, scale)
    out = hip.DeviceBuffer(ctx, q.nbytes)
    kv.attn_dev(0, n_stream, dev(ctx, np.array(order, np.int32)), dev(ctx, np.array(ln, np.int32)), max(ln), hq,
                dev(ctx, q), scale, out)
    assert np.array_equal(bits(down(ctx, out, np.float32, q.size)), bits(want))


def test_decoder_step_dev_equals_step(ctx, oracle):
    """Two sessions from the same weights, one stepped through host arrays and
    one through device arrays (the form the bench times and a graph captures):
    the same next tokens and logits, bit for bit, step after step."""
    print("[case] resident decoder step", flush=True)
    from tests.test_gpu_sessions import make_decoder
    a, _ = make_decoder(ctx, oracle, np.random.default_rng(5))
    b, _ = make_decoder(ctx, oracle, np.random.default_rng(5))
    g = np.random.default_rng(6)
    V = a.parts["V"]
    streams = np.array([2, 0, 3], np.int32)
    d_streams = dev(ctx, streams)
    d_next = hip.DeviceBuffer(ctx, 4 * streams.size)
    d_logits = hip.DeviceBuffer(ctx, 4 * streams.size * V)
    for p in range(6):
        tokens = g.integers(0, V, streams.size).astype(np.int32)
        pos = np.full(streams.size, p, np.int32)
        want, lg = a.step(streams, tokens, pos, want_logits=True)
        b.step_dev(streams.size, d_streams, dev(ctx, tokens), dev(ctx, pos), d_next, d_logits)
        assert b.status() == len(a.parts["layers"]) * streams.size
        assert np.array_equal(down(ctx, d_next, np.int32, streams.size), want), p
        assert np.array_equal(bits(down(ctx, d_logits, np.float32, lg.size)), bits(lg)), p


def test_text_decoder_step_dev_equals_step(ctx, oracle):
    print("[case] resident text decoder step", flush=True)
    from tests.test_gpu_textdec import build
    kw = dict(n_layer=2, d=256, hq=4, hkv=2, hd=64, ff=512, V=320, n_ctx=40, n_stream=3)
    a, P = build(ctx, oracle, 9, **kw)
    b, _ = build(ctx, oracle, 9, **kw)
    g = np.random.default_rng(10)
    streams = np.array([1, 2, 0], np.int32)
    d_streams = dev(ctx, streams)
    d_next = hip.DeviceBuffer(ctx, 4 * streams.size)
    d_logits = hip.DeviceBuffer(ctx, 4 * streams.size * P["V"])
    for p in range(6):
        tokens = g.integers(0, P["V"], streams.size).astype(np.int32)
        want, lg = a.step(streams, tokens, want_logits=True)
        b.step_dev(streams.size, d_streams, dev(ctx, tokens), dev(ctx, np.full(streams.size, p, np.int32)), d_next,
                   d_logits)
        b.status()
        assert np.array_equal(down(ctx, d_next, np.int32, streams.size), want), p
        assert np.array_equal(bits(down(ctx, d_logits, np.float32, lg.size)), bits(lg)), p


def test_log_mel_dev_equals_copy_mode(ctx):
    print("[case] resident log-mel", flush=True)
    g = np.random.default_rng(11)
    batch, n, n_mels = 2, 40000, 80
    pcm = (g.standard_normal((batch, n)) * 0.1).astype(np.float32)
    want = ctx.log_mel(pcm, n_mels)
    out = hip.DeviceBuffer(ctx, want.nbytes)
    ctx.log_mel_dev(dev(ctx, pcm), batch, n, n_mels, out)
    assert np.array_equal(bits(down(ctx, out, np.float32, want.size)), bits(want))


def test_events_time_the_library_stream(ctx):
    """vokra_hip_event_record / _elapsed_ms around work on the library stream."""
    print("[case] events", flush=True)
    start, stop = hip.Event(ctx), hip.Event(ctx)
    x = dev(ctx, np.ones(1 << 20, np.float32))
    y = hip.DeviceBuffer(ctx, 4 << 20)
    start.record()
    for _ in range(4):
        ctx.gelu_f32_dev(x, y, 1 << 20)
    stop.record()
    ctx.synchronize()
    ms = start.elapsed_ms(stop)
    assert np.isfinite(ms) and 0.0 <= ms < 1000.0

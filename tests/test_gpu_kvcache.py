"""GPU parity of the paged quantized KV cache and decode attention over it.

Bars:
  * cache state (page table, free list counts, exhaustion point) identical to
    the oracle's QuantizedPagedKvCache restatement for the same operations;
  * read_step rows bit-identical (Q8_0 packing and q * f16(d) decode);
  * decode attention within 1e-4 + 1e-3 * |ref| of the oracle's attention
    (whisper nn.rs:209-325 / voxtral GQA) on the cache's dequantized rows.
"""
import numpy as np
import pytest

from vokra_amd import hip

pytestmark = pytest.mark.gpu

Q8_0 = 3
ATOL, RTOL = 1e-4, 1e-3


@pytest.fixture(scope="module")
def ctx():
    c = hip.HipContext(0)
    yield c
    c.close()


def same_bits(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


def close(got, want):
    err = np.abs(np.asarray(got, np.float64) - want) - (ATOL + RTOL * np.abs(want))
    return bool(np.all(err <= 0)), float(np.max(np.abs(np.asarray(got, np.float64) - want)))


def assert_same_state(kv, ref, n_layer, max_time, bs):
    fr, used = kv.pages()
    assert (fr, used) == (ref.free_pages(), ref.pages_in_use())
    for layer in range(n_layer):
        for t in range(0, max_time, bs):
            assert kv.page_of(layer, t) == ref.page_of(layer, t), (layer, t)


def test_lockstep_with_oracle(ctx, oracle):
    """Random appends (batched on the GPU, one by one in the oracle), releases
    and a reset: same page ids, same free counts, bit-identical rows."""
    print("[case] kv lockstep", flush=True)
    n_layer, H, hd, n_stream, max_time, bs = 3, 2, 64, 5, 40, 4
    w = H * hd
    kv = ctx.kv_cache(n_layer, H, hd, n_stream, max_time, bs)
    ref = oracle.PagedCache(n_layer, H, hd, n_stream, max_time, bs, Q8_0)
    g = np.random.default_rng(3)
    written = {}
    for step in range(30):
        layer = int(g.integers(0, n_layer))
        n = int(g.integers(1, 8))
        streams = g.integers(0, n_stream, n).astype(np.int32)
        times = g.integers(0, max_time, n).astype(np.int32)
        k = (g.standard_normal((n, w)) * g.uniform(0.1, 5)).astype(np.float32)
        v = g.standard_normal((n, w)).astype(np.float32)
        k[0, :32] = 0.0  # an all-zero block: d = 0
        kv.append(layer, streams, times, k, v)
        for i in range(n):
            assert ref.append_step(layer, int(times[i]), int(streams[i]), k[i], v[i]) == 0
            written[(layer, int(times[i]), int(streams[i]))] = True
        if step == 12:
            kv.release_layer(1)
            ref.release_layer(1)
            written = {key: 1 for key in written if key[0] != 1}
        assert_same_state(kv, ref, n_layer, max_time, bs)
    for (layer, t, s) in list(written)[:60]:
        got, want = kv.read(layer, t, s), ref.read_step(layer, t, s)
        assert got is not None and want is not None
        assert same_bits(got[0], want[0]) and same_bits(got[1], want[1])
    # every (layer, t, s): None where the oracle has no page, else the same bits
    for layer in range(n_layer):
        for t in range(max_time):
            for s_ in range(n_stream):
                got, want = kv.read(layer, t, s_), ref.read_step(layer, t, s_)
                assert (got is None) == (want is None), (layer, t, s_)
                if got is not None:
                    assert same_bits(got[0], want[0]) and same_bits(got[1], want[1])
    kv.reset()
    ref.reset()
    assert_same_state(kv, ref, n_layer, max_time, bs)
    assert kv.read(0, 0, 0) is None


def test_full_occupancy_matches_oracle(ctx, oracle):
    """The arena holds one page per table entry (capacity = pages_per_layer x
    n_layer, paged_quant.rs:284-287), so filling every entry empties the free
    list without exhausting it; both caches agree page for page, and a
    release returns the pages in table order."""
    print("[case] kv full occupancy", flush=True)
    n_layer, H, hd, n_stream, max_time, bs = 2, 1, 64, 2, 10, 2
    kv = ctx.kv_cache(n_layer, H, hd, n_stream, max_time, bs)
    ref = oracle.PagedCache(n_layer, H, hd, n_stream, max_time, bs, Q8_0)
    g = np.random.default_rng(4)
    for layer in (1, 0):
        times = np.array([9, 0, 4, 2, 6, 7, 1], np.int32)
        streams = np.array([0, 1, 0, 1, 0, 1, 1], np.int32)
        rows = g.standard_normal((7, 64)).astype(np.float32)
        kv.append(layer, streams, times, rows, rows)
        for i in range(7):
            assert ref.append_step(layer, int(times[i]), int(streams[i]), rows[i], rows[i]) == 0
        assert_same_state(kv, ref, n_layer, max_time, bs)
    assert kv.pages() == (0, 10)
    kv.release_layer(1)
    ref.release_layer(1)
    assert_same_state(kv, ref, n_layer, max_time, bs)
    rows = g.standard_normal((3, 64)).astype(np.float32)
    kv.append(1, [0, 0, 1], [3, 8, 3], rows, rows)     # re-acquires released pages, LIFO
    for i, (s_, t_) in enumerate([(0, 3), (0, 8), (1, 3)]):
        assert ref.append_step(1, t_, s_, rows[i], rows[i]) == 0
    assert_same_state(kv, ref, n_layer, max_time, bs)
    got, want = kv.read(1, 8, 0), ref.read_step(1, 8, 0)
    assert same_bits(got[0], want[0]) and same_bits(got[1], want[1])


def test_invalid_item_stops_batch(ctx, oracle):
    print("[case] kv invalid item", flush=True)
    kv = ctx.kv_cache(2, 2, 64, 3, 16, 4)
    ref = oracle.PagedCache(2, 2, 64, 3, 16, 4, Q8_0)
    g = np.random.default_rng(5)
    r = g.standard_normal((3, 128)).astype(np.float32)
    with pytest.raises(hip.InvalidArgument, match="t 16 >= max_time 16"):
        kv.append(1, [0, 1, 2], [3, 16, 5], r, r)
    assert ref.append_step(1, 3, 0, r[0], r[0]) == 0      # item 0 applied, 1 refused, 2 never ran
    assert_same_state(kv, ref, 2, 16, 4)
    with pytest.raises(hip.InvalidArgument, match="stream 3 >= n_stream 3"):
        kv.append(0, [3], [0], r[:1], r[:1])
    with pytest.raises(hip.InvalidArgument):
        kv.append(2, [0], [0], r[:1], r[:1])              # layer out of range
    assert_same_state(kv, ref, 2, 16, 4)


def test_round_trip_bound(ctx):
    """paged_quant.rs:622-647: |read - written| <= 0.6 * amax / 127 per block."""
    print("[case] kv round trip", flush=True)
    kv = ctx.kv_cache(1, 4, 64, 2, 8, 2)
    g = np.random.default_rng(6)
    rows = (g.standard_normal((8, 256)) * 3).astype(np.float32)
    kv.append(0, [0] * 8, list(range(8)), rows, -rows)
    for t in range(8):
        k, v = kv.read(0, t, 0)
        for b in range(8):
            amax = np.abs(rows[t, 32 * b:32 * b + 32]).max()
            assert np.abs(k[32 * b:32 * b + 32] - rows[t, 32 * b:32 * b + 32]).max() <= 0.6 * amax / 127
            assert np.abs(v[32 * b:32 * b + 32] + rows[t, 32 * b:32 * b + 32]).max() <= 0.6 * amax / 127


def test_create_rejections(ctx):
    with pytest.raises(hip.InvalidArgument):
        ctx.kv_cache(1, 2, 64, 1, 8, 2, hip.KvQuant.Fp32)
    with pytest.raises(hip.InvalidArgument):
        ctx.kv_cache(0, 2, 64, 1, 8, 2)
    with pytest.raises(hip.InvalidArgument):
        ctx.kv_cache(1, 1, 48, 1, 8, 2)                    # 48 not a multiple of 32
    with pytest.raises(hip.UnsupportedOp):
        ctx.kv_cache(1, 2, 64, 1, 8, 2, hip.KvQuant.Q4_0)


def fill_cache(kv, ref, layer, lens, w, rng, n_stream):
    """Appends rows t = 0..len_s-1 for every stream, one decode step per t
    (all live streams in one batch), mirrored into the oracle cache."""
    for t in range(max(lens)):
        live = [s for s in range(n_stream) if lens[s] > t]
        k = rng.standard_normal((len(live), w)).astype(np.float32)
        v = rng.standard_normal((len(live), w)).astype(np.float32)
        kv.append(layer, live, [t] * len(live), k, v)
        if ref is not None:
            for i, s in enumerate(live):
                assert ref.append_step(layer, t, s, k[i], v[i]) == 0


def cached_kv(ref, layer, s, n):
    rows = [ref.read_step(layer, t, s) for t in range(n)]
    return np.stack([r[0] for r in rows]), np.stack([r[1] for r in rows])


@pytest.mark.parametrize("H,hd,hq", [(4, 64, 4), (2, 128, 16), (2, 64, 8), (3, 128, 6), (2, 64, 16), (2, 128, 2),
                                     (2, 128, 8)])
def test_paged_attention_vs_oracle(ctx, oracle, H, hd, hq):
    print(f"[case] paged attn H={H} hd={hd} hq={hq}", flush=True)
    n_stream, max_time, bs = 5, 300, 16
    kv = ctx.kv_cache(2, H, hd, n_stream, max_time, bs)
    ref = oracle.PagedCache(2, H, hd, n_stream, max_time, bs, Q8_0)
    rng = np.random.default_rng(H * hd + hq)
    lens = [1, 17, 64, 300, 129]
    fill_cache(kv, ref, 1, lens, H * hd, rng, n_stream)
    fill_cache(kv, ref, 0, [3, 3, 3, 3, 3], H * hd, rng, n_stream)  # other layer: must not leak
    order = [3, 0, 4, 1, 2]
    q = rng.standard_normal((5, hq * hd)).astype(np.float32)
    scale = float(np.float32(hd) ** np.float32(-0.5))
    got = kv.attn(1, order, [lens[s] for s in order], q, hq, scale)
    for i, s in enumerate(order):
        K, V = cached_kv(ref, 1, s, lens[s])
        if hq == H:
            want = oracle.sdpa_whisper(1, lens[s], H, hd, q[i:i + 1], K, V, causal=True,
                                       q_pos_offset=lens[s] - 1)[0]
        else:
            want = oracle.gqa_attention(1, lens[s], hq, H, hd, q[i:i + 1], K, V, scale, lens[s] - 1)[0]
        ok, err = close(got[i], want.astype(np.float64))
        assert ok, (s, err)


@pytest.mark.parametrize("bs", [4, 12, 32])
def test_paged_attention_page_sizes(ctx, oracle, bs):
    """Page sizes other than 16 with one q head per kv head at head_dim 64:
    4 and 32 (powers of two: the wave-split kernel, whose 16-key passes then
    span four pages or half of one) and 12 (the thread-per-key kernel)."""
    print(f"[case] paged attn bs={bs}", flush=True)
    H, hd, n_stream, max_time = 3, 64, 4, 260
    kv = ctx.kv_cache(1, H, hd, n_stream, max_time, bs)
    ref = oracle.PagedCache(1, H, hd, n_stream, max_time, bs, Q8_0)
    rng = np.random.default_rng(bs)
    lens = [260, 77, 1, 190]
    fill_cache(kv, ref, 0, lens, H * hd, rng, n_stream)
    q = rng.standard_normal((n_stream, H * hd)).astype(np.float32)
    scale = float(np.float32(hd) ** np.float32(-0.5))
    order = [2, 0, 3, 1]
    got = kv.attn(0, order, [lens[s] for s in order], q, H, scale)
    for i, s in enumerate(order):
        K, V = cached_kv(ref, 0, s, lens[s])
        want = oracle.sdpa_whisper(1, lens[s], H, hd, q[i:i + 1], K, V, causal=True, q_pos_offset=lens[s] - 1)[0]
        ok, err = close(got[i], want.astype(np.float64))
        assert ok, (s, err)


def test_paged_attention_q_magnitudes_and_non_finite(ctx, oracle):
    """One q head per kv head at head_dim 64 takes q as 22-bit integers per
    16-dim quarter, scaled by a power of two from the quarter's largest |q|
    (clamped for tiny magnitudes): rows of q from 1e-40 (subnormal) to 1e20
    stay within the f32 tolerance of the oracle, and a NaN or inf q value makes
    exactly its head's output NaN, as the f32 products do."""
    print("[case] paged attn q magnitudes", flush=True)
    H, hd, n_stream, max_time, bs = 4, 64, 6, 200, 16
    kv = ctx.kv_cache(1, H, hd, n_stream, max_time, bs)
    ref = oracle.PagedCache(1, H, hd, n_stream, max_time, bs, Q8_0)
    rng = np.random.default_rng(2024)
    lens = [200, 131, 64, 97, 1, 150]
    fill_cache(kv, ref, 0, lens, H * hd, rng, n_stream)
    scale = float(np.float32(hd) ** np.float32(-0.5))
    q = rng.standard_normal((n_stream, H * hd)).astype(np.float32)
    mags = [1e-40, 1e-30, 1e-3, 1.0, 1e3, 1e20]
    q = (q * np.array(mags, np.float32)[:, None]).astype(np.float32)
    q[2, 16:32] *= np.float32(1e-6)  # quarters of one head with very different ranges
    got = kv.attn(0, list(range(n_stream)), lens, q, H, scale)
    for s in range(n_stream):
        K, V = cached_kv(ref, 0, s, lens[s])
        want = oracle.sdpa_whisper(1, lens[s], H, hd, q[s:s + 1], K, V, causal=True, q_pos_offset=lens[s] - 1)[0]
        ok, err = close(got[s], want.astype(np.float64))
        assert ok, (s, mags[s], err)
    bad = q.copy()
    bad[0, 5] = np.nan           # head 0 of stream 0
    bad[3, hd + 3] = np.inf      # head 1 of stream 3
    bad[5, 3 * hd + 60] = -np.inf  # head 3 of stream 5
    got = kv.attn(0, list(range(n_stream)), lens, bad, H, scale).reshape(n_stream, H, hd)
    nan_heads = {(0, 0), (3, 1), (5, 3)}
    for s in range(n_stream):
        for h in range(H):
            if (s, h) in nan_heads:
                assert np.isnan(got[s, h]).all(), (s, h)
            else:
                assert np.isfinite(got[s, h]).all(), (s, h)


def test_paged_attention_split_path(ctx, oracle):
    """Long contexts with few workgroups use the key split + combine kernel."""
    print("[case] paged attn split", flush=True)
    H, hd, hq, n_stream, max_time, bs = 2, 128, 16, 2, 4096, 16
    kv = ctx.kv_cache(1, H, hd, n_stream, max_time, bs)
    ref = oracle.PagedCache(1, H, hd, n_stream, max_time, bs, Q8_0)
    rng = np.random.default_rng(77)
    lens = [4096, 1500]
    fill_cache(kv, ref, 0, lens, H * hd, rng, n_stream)
    q = rng.standard_normal((2, hq * hd)).astype(np.float32)
    scale = float(np.float32(hd) ** np.float32(-0.5))
    got = kv.attn(0, [0, 1], lens, q, hq, scale)
    for s in range(2):
        K, V = cached_kv(ref, 0, s, lens[s])
        want = oracle.gqa_attention(1, lens[s], hq, H, hd, q[s:s + 1], K, V, scale, lens[s] - 1)[0]
        ok, err = close(got[s], want.astype(np.float64))
        assert ok, (s, err)


@pytest.mark.parametrize("H,hd,hq", [(2, 128, 16), (2, 64, 2), (2, 64, 8)])
def test_paged_attention_contexts_beyond_4096(ctx, oracle, H, hd, hq):
    """Contexts past 4096 keys, where an item's split grows to 1024 (and 1536)
    keys: the matrix-core kernel's looped path (8 and 12 tiles per wave), the
    VALU kernels' 4- to 6-chunk splits, a last split one key short, 5 to 8
    splits through the combine; against the oracle, and an item alone ==
    the same item in the batch, bit for bit."""
    print(f"[case] paged attn beyond 4096 H={H} hd={hd} hq={hq}", flush=True)
    lens = [4097, 6143, 8192, 8193]
    n_stream, max_time, bs = len(lens), 8208, 16
    kv = ctx.kv_cache(1, H, hd, n_stream, max_time, bs)
    ref = oracle.PagedCache(1, H, hd, n_stream, max_time, bs, Q8_0)
    rng = np.random.default_rng(4097 + hd + hq)
    fill_cache(kv, ref, 0, lens, H * hd, rng, n_stream)
    q = rng.standard_normal((n_stream, hq * hd)).astype(np.float32)
    scale = float(np.float32(hd) ** np.float32(-0.5))
    got = kv.attn(0, list(range(n_stream)), lens, q, hq, scale)
    for s in range(n_stream):
        K, V = cached_kv(ref, 0, s, lens[s])
        if hq == H:
            want = oracle.sdpa_whisper(1, lens[s], H, hd, q[s:s + 1], K, V, causal=True,
                                       q_pos_offset=lens[s] - 1)[0]
        else:
            want = oracle.gqa_attention(1, lens[s], hq, H, hd, q[s:s + 1], K, V, scale, lens[s] - 1)[0]
        ok, err = close(got[s], want.astype(np.float64))
        assert ok, (s, err)
        alone = kv.attn(0, [s], [lens[s]], q[s:s + 1], hq, scale)
        assert np.array_equal(alone[0], got[s]), s


def test_config3_self_attention_shape(ctx):
    """Config 3 decoder self-attention: 64 streams, 20 heads x 64, prefix
    lengths U(1..448), 16-token pages at shuffled addresses; checked in float64
    against the rows the cache itself returns."""
    print("[case] config3 paged attn", flush=True)
    H, hd, n_stream, max_time, bs = 20, 64, 64, 448, 16
    kv = ctx.kv_cache(1, H, hd, n_stream, max_time, bs)
    rng = np.random.default_rng(448)
    kv.set_free_order(rng.permutation(max_time // bs).astype(np.int32))
    lens = rng.integers(1, 449, n_stream).tolist()
    fill_cache(kv, None, 0, lens, H * hd, rng, n_stream)
    q = rng.standard_normal((n_stream, H * hd)).astype(np.float32)
    got = kv.attn(0, list(range(n_stream)), lens, q, H, 0.125)
    for s in (0, 17, 63):
        rows = [kv.read(0, t, s) for t in range(lens[s])]
        K = np.stack([r[0] for r in rows]).astype(np.float64)
        V = np.stack([r[1] for r in rows]).astype(np.float64)
        for h in (0, 11, 19):
            sl = slice(h * hd, (h + 1) * hd)
            sc = (q[s, sl].astype(np.float64) * 0.125) @ K[:, sl].T
            p = np.exp(sc - sc.max())
            want = (p / p.sum()) @ V[:, sl]
            ok, err = close(got[s, sl], want)
            assert ok, (s, h, err)


@pytest.mark.parametrize("H,hd,hq", [(20, 64, 20), (2, 128, 16)])
def test_paged_attention_item_independent_of_batch(ctx, H, hd, hq):
    """An item's output depends on its own keys only: the same query over the
    same stream gives the same bits alone, in a large batch and next to
    longer items (which change the launch's key split), for lengths below,
    at and above the 512-key split."""
    print(f"[case] paged attn batch independence H={H} hd={hd} hq={hq}", flush=True)
    n_stream, max_time, bs = 8, 4096, 16
    kv = ctx.kv_cache(1, H, hd, n_stream, max_time, bs)
    rng = np.random.default_rng(hd + hq)
    lens = [1, 300, 512, 513, 1500, 3584, 3585, 4096]
    fill_cache(kv, None, 0, lens, H * hd, rng, n_stream)
    q = rng.standard_normal((n_stream, hq * hd)).astype(np.float32)
    scale = float(np.float32(hd) ** np.float32(-0.5))
    batch = kv.attn(0, list(range(n_stream)), lens, q, hq, scale)
    for s in range(n_stream):
        alone = kv.attn(0, [s], [lens[s]], q[s:s + 1], hq, scale)
        assert np.array_equal(alone[0], batch[s]), s
        pair = kv.attn(0, [s, 7], [lens[s], 4096], q[[s, 7]], hq, scale)
        assert np.array_equal(pair[0], batch[s]), s

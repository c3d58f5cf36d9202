"""The no-allocation GEMM entry point (vokra_hip_gemm_q_f32_dev_noalloc)
against the allocating one (vokra_hip_gemm_q_f32_dev), through the C ABI.

Bar: bit-identical outputs, on two calls in a row where the second is
smaller than the first (the workspace keeps the first call's contents, which
the second must not read), for each weight format and both the decode route
(m <= 64) and the block-GEMM route; the same call replayed from a HIP graph;
and the workspace limit rejected with INVALID_ARGUMENT.
"""
import numpy as np
import pytest

from vokra_amd import hip

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    c = hip.HipContext(0)
    yield c
    c.close()


def weight(ctx, g, wd, n, k):
    if wd == hip.WDtype.Q4_K:
        b = g.integers(0, 256, size=(n * (k // 256), 144), dtype=np.uint8)
        b[:, 1], b[:, 3] = 0x2C, 0x24
        return ctx.upload_qweight(wd, n, k, b.reshape(-1))
    mode = {hip.WDtype.Q4_0: hip.KvQuant.Q4_0, hip.WDtype.Q8_0: hip.KvQuant.Q8_0}[wd]
    w = (g.standard_normal((n, k)) * 0.02).astype(np.float32)
    return ctx.upload_qweight(wd, n, k, ctx.quantize_bytes(mode, w))


def both(ctx, W, m, k, n, a, bias, act):
    d_a = hip.DeviceBuffer.from_array(ctx, a)
    d_b = None if bias is None else hip.DeviceBuffer.from_array(ctx, bias)
    ref, got = hip.DeviceBuffer(ctx, m * n * 4), hip.DeviceBuffer(ctx, m * n * 4)
    ctx.gemm_q_f32_dev(W, m, d_a, ref, d_b, act)
    ctx.gemm_q_f32_dev_noalloc(W, m, d_a, got, d_b, act)
    ctx.synchronize()
    return ref.download(np.float32, m * n), got.download(np.float32, m * n)


@pytest.mark.parametrize("wd,act,n,k,ms", [
    (hip.WDtype.Q8_0, hip.ActQuant.AMAX127, 5120, 1280, (1500, 37)),
    (hip.WDtype.Q8_0, hip.ActQuant.POW2, 1280, 1280, (200, 8)),
    (hip.WDtype.Q4_0, hip.ActQuant.AMAX127, 1280, 5120, (64, 1)),
    (hip.WDtype.Q4_K, hip.ActQuant.KQUANT, 2048, 5632, (32, 3)),
])
def test_noalloc_equals_dev_two_calls(ctx, wd, act, n, k, ms):
    print(f"[case] noalloc wd={int(wd)} n={n} k={k} ms={ms}", flush=True)
    g = np.random.default_rng(n + k)
    W = weight(ctx, g, wd, n, k)
    bias = g.standard_normal(n).astype(np.float32)
    for m in ms:
        a = g.standard_normal((m, k)).astype(np.float32)
        ref, got = both(ctx, W, m, k, n, a, bias if m % 2 else None, act)
        assert np.array_equal(ref.view(np.uint32), got.view(np.uint32)), m


def test_noalloc_graph_replays(ctx):
    """Captured once, replayed three times with eager work and
    synchronizations in between: every replay matches the eager result."""
    print("[case] noalloc graph", flush=True)
    g = np.random.default_rng(7)
    m, n, k = 96, 1280, 1280
    W = weight(ctx, g, hip.WDtype.Q8_0, n, k)
    a = g.standard_normal((m, k)).astype(np.float32)
    d_a = hip.DeviceBuffer.from_array(ctx, a)
    want = hip.DeviceBuffer(ctx, m * n * 4)
    ctx.gemm_q_f32_dev(W, m, d_a, want)
    ctx.synchronize()
    want = want.download(np.float32, m * n)
    d_out = hip.DeviceBuffer(ctx, m * n * 4)
    graph = ctx.capture(lambda: ctx.gemm_q_f32_dev_noalloc(W, m, d_a, d_out))
    other = g.standard_normal((7, k)).astype(np.float32)
    for _ in range(3):
        d_out.upload(np.zeros(m * n, np.float32))
        graph.launch()
        ctx.synchronize()
        assert np.array_equal(d_out.download(np.float32, m * n).view(np.uint32), want.view(np.uint32))
        # eager use of the same workspace between replays
        ref, got = both(ctx, W, 7, k, n, other, None, hip.ActQuant.AMAX127)
        assert np.array_equal(ref.view(np.uint32), got.view(np.uint32))


def test_noalloc_rejects_beyond_workspace(ctx):
    g = np.random.default_rng(3)
    m, n, k = 3000, 64, 5120      # 2.5 * 3072 * 5120 bytes > 32 MiB
    W = weight(ctx, g, hip.WDtype.Q8_0, n, k)
    d_a = hip.DeviceBuffer(ctx, m * k * 4)
    d_out = hip.DeviceBuffer(ctx, m * n * 4)
    with pytest.raises(hip.InvalidArgument, match="workspace"):
        ctx.gemm_q_f32_dev_noalloc(W, m, d_a, d_out)
    with pytest.raises(hip.InvalidArgument):
        ctx.gemm_q_f32_dev_noalloc(W, 0, d_a, d_out)

"""GPU parity of the block-quant path against the oracle, through the C ABI.

Bars (written per test):
  * dequantize_bytes: bit-exact (the "dequantized values" surface).
  * fused dequant GEMV (f32 semantics): |diff| <= 1e-4 on the reference's own
    CUDA parity shapes and seeds (parity_kernels_cuda.rs:2169-2247); larger
    rows use a derived f32 reassociation bound.
  * gemm_q_f32 block formats (INT8 semantics): bit-exact f32 outputs — the
    int32 block dot products are exact and the combine order is the oracle's.
"""
import numpy as np
import pytest

from vokra_amd import hip

pytestmark = pytest.mark.gpu

M3_04_SHAPES = [(1, 1), (1, 8), (2, 2), (4, 2), (16, 2), (32, 4), (128, 2), (256, 4)]


@pytest.fixture(scope="module")
def ctx():
    c = hip.HipContext(0)
    yield c
    c.close()


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.mark.parametrize("mode", [1, 2, 3])
def test_dequantize_bit_exact(ctx, oracle, mode):
    print(f"[case] dequantize mode={mode}", flush=True)
    g = np.random.default_rng(mode)
    x = (g.standard_normal(32 * 1000) * 3).astype(np.float32)
    x[32:64] = 0.0
    data = oracle.pack_matrix_to_bytes(mode, x, 1000, 1)
    got = ctx.dequantize_bytes(hip.KvQuant(mode), data)
    want = oracle.dequantize_bytes(mode, data)
    assert np.array_equal(bits(got), bits(want))


@pytest.mark.parametrize("mode", [1, 2, 3])
def test_dequantize_all_scales(ctx, oracle, mode):
    """Every f16 scale bit pattern (subnormal, inf, NaN included)."""
    print(f"[case] dequantize all-scales mode={mode}", flush=True)
    bb = hip.KvQuant(mode).block_bytes()
    g = np.random.default_rng(10 + mode)
    data = g.integers(0, 256, size=(65536, bb), dtype=np.uint8)
    data[:, 0] = np.arange(65536) & 0xFF
    data[:, 1] = np.arange(65536) >> 8
    got = ctx.dequantize_bytes(hip.KvQuant(mode), data.reshape(-1))
    want = oracle.dequantize_bytes(mode, data.reshape(-1))
    assert np.array_equal(bits(got), bits(want))


@pytest.mark.parametrize("mode", [1, 2, 3])
def test_quantize_bytes_bit_exact(ctx, oracle, mode):
    """Device packer == the reference packers, byte for byte, including zero
    blocks, saturation, NaN / inf elements and subnormal scales."""
    print(f"[case] quantize_bytes mode={mode}", flush=True)
    g = np.random.default_rng(20 + mode)
    x = (g.standard_normal(32 * 4096) * np.exp(g.uniform(-30, 12, 32 * 4096))).astype(np.float32)
    x[:32] = 0.0
    x[32:64] = 1e-41
    x[64] = 1000.0
    x[65] = -1000.0
    x[96] = np.nan
    x[128] = np.inf
    x[160:192] = np.array([(i / 31.0) * 2 - 1 for i in range(32)], np.float32)
    got = ctx.quantize_bytes(hip.KvQuant(mode), x)
    want = oracle.pack_matrix_to_bytes(mode, x, 4096, 1)
    assert np.array_equal(got, want)


def test_dequantize_rejects(ctx):
    with pytest.raises(hip.InvalidArgument):
        ctx.dequantize_bytes(hip.KvQuant.Fp32, np.zeros(128, np.uint8))
    with pytest.raises(hip.InvalidArgument):
        ctx.dequantize_bytes(hip.KvQuant.Q8_0, np.zeros(33, np.uint8))


@pytest.mark.parametrize("mode", [3, 2, 1])
def test_dequant_gemv_matches_cpu_reference_shapes(ctx, oracle, mode):
    """parity_kernels_cuda.rs dequant_gemv_parity: same shapes, seeds, bound."""
    worst = 0.0
    for n_rows, n_bpr in M3_04_SHAPES:
        print(f"[case] dequant_gemv mode={mode} n_rows={n_rows} n_bpr={n_bpr}", flush=True)
        per_row = n_bpr * 32
        a = oracle.xorshift_rand_vec(0xD3 ^ (n_rows * 131 + n_bpr), n_rows * per_row)
        x = oracle.xorshift_rand_vec(0xE5 ^ per_row, per_row)
        data = oracle.pack_matrix_to_bytes(mode, a, n_rows, n_bpr)
        cpu = oracle.dequant_gemv_scalar(mode, data, n_rows, n_bpr, x)
        direct = ctx.dequant_gemv_f32(hip.KvQuant(mode), data, n_rows, n_bpr, x)
        trait = ctx.fused_dequant_gemv(hip.KvQuant(mode), data, n_rows, n_bpr, x)
        assert np.array_equal(bits(direct), bits(trait))
        d = float(np.abs(direct - cpu).max())
        assert d <= 1e-4, f"n_rows={n_rows} n_bpr={n_bpr}: {d}"
        worst = max(worst, d)
    print(f"HIP fused dequant_gemv mode={mode} vs CPU: global max|d| = {worst:.3e} (bound 1e-4)")


@pytest.mark.parametrize("mode,n_rows,n_bpr", [(3, 5120, 40), (1, 1280, 40), (2, 333, 7), (3, 3, 300)])
def test_dequant_gemv_long_rows(ctx, oracle, mode, n_rows, n_bpr):
    """Longer rows than the reference exercises: bound = 4 * K * eps * sum|w*x|
    (reassociation of a K-term f32 sum)."""
    print(f"[case] dequant_gemv long mode={mode} n_rows={n_rows} n_bpr={n_bpr}", flush=True)
    g = np.random.default_rng(n_rows)
    k = n_bpr * 32
    a = (g.standard_normal(n_rows * k) * 0.02).astype(np.float32)
    x = g.standard_normal(k).astype(np.float32)
    data = oracle.pack_matrix_to_bytes(mode, a, n_rows, n_bpr)
    cpu = oracle.dequant_gemv_scalar(mode, data, n_rows, n_bpr, x)
    got = ctx.dequant_gemv_f32(hip.KvQuant(mode), data, n_rows, n_bpr, x)
    deq = oracle.dequantize_bytes(mode, data).reshape(n_rows, k)
    mag = np.abs(deq.astype(np.float64) * x).sum(1)
    bound = 4 * k * np.finfo(np.float32).eps * mag + 1e-30
    assert np.all(np.abs(got.astype(np.float64) - cpu) <= bound)


def test_dequant_gemv_rejections(ctx):
    with pytest.raises(hip.InvalidArgument, match="Fp32"):
        ctx.dequant_gemv_f32(hip.KvQuant.Fp32, np.zeros(4 * 2 * 34, np.uint8), 4, 2, np.zeros(64))
    with pytest.raises(hip.InvalidArgument):
        ctx.dequant_gemv_f32(hip.KvQuant.Q8_0, np.zeros(100, np.uint8), 4, 2, np.zeros(64))
    with pytest.raises(hip.InvalidArgument):
        ctx.dequant_gemv_f32(hip.KvQuant.Q8_0, np.zeros(272, np.uint8), 4, 2, np.zeros(63))
    assert ctx.dequant_gemv_f32(hip.KvQuant.Q8_0, np.zeros(0, np.uint8), 0, 2, np.zeros(64)).size == 0


WD_MODE = {hip.WDtype.Q8_0: 3, hip.WDtype.Q4_0: 1, hip.WDtype.Q5_0: 2}


def _gemm_case(oracle, wd, m, n, k, seed, with_bias=True, zero_rows=()):
    g = np.random.default_rng(seed)
    w = (g.standard_normal((n, k)) * 0.02).astype(np.float32)
    wq = oracle.pack_matrix_to_bytes(WD_MODE[wd], w, n, k // 32)
    a = g.standard_normal((m, k)).astype(np.float32)
    for r in zero_rows:
        a[r] = 0.0
    bias = g.standard_normal(n).astype(np.float32) if with_bias else None
    return a, wq, bias


@pytest.mark.parametrize("act", [hip.ActQuant.AMAX127, hip.ActQuant.POW2])
@pytest.mark.parametrize("wd", [hip.WDtype.Q8_0, hip.WDtype.Q4_0, hip.WDtype.Q5_0])
@pytest.mark.parametrize("m,n,k", [(1, 16, 32), (7, 100, 64), (130, 256, 256), (300, 130, 1280)])
def test_gemm_q_block_bit_exact(ctx, oracle, wd, act, m, n, k):
    print(f"[case] gemm_q wd={wd.name} act={act.name} m={m} n={n} k={k}", flush=True)
    a, wq, bias = _gemm_case(oracle, wd, m, n, k, seed=m * 7 + n, zero_rows=(0,))
    ctx.set_act_quant(act)
    try:
        got = ctx.gemm_q_f32(m, n, k, a, wq, wd, bias)
    finally:
        ctx.set_act_quant(hip.ActQuant.AMAX127)
    want = oracle.gemm_qblock_i8(int(wd), m, n, k, a, wq, bias, pow2=(act == hip.ActQuant.POW2))
    assert np.array_equal(bits(got), bits(want))


@pytest.mark.parametrize("act", [hip.ActQuant.AMAX127, hip.ActQuant.POW2])
def test_gemm_q_activation_edge_values(ctx, oracle, act):
    """The 32-wide block activation pass on blocks random inputs do not
    reach, through the matmul, bit-exact (NaN outputs in the same places):
    an all-NaN block (amax 0: s = 0, every q 0), one NaN in a normal block
    (ignored by the maximum, quantized to 0), exact half ties of v / s (round
    half away from zero), a subnormal-only block, and a row count that leaves
    padding rows. With AMAX127 (kquant.rs:418-441 at group 32) also +Inf and
    -Inf elements (s = inf, every q 0, so the row's outputs are NaN); the
    build-defined POW2 scale of an infinite maximum rests on frexp's
    unspecified exponent for inf, so that case stays out of its run."""
    print(f"[case] gemm_q activation edge values act={act.name}", flush=True)
    m, n, k = 21, 40, 256
    a, wq, _ = _gemm_case(oracle, hip.WDtype.Q8_0, m, n, k, seed=21, with_bias=False, zero_rows=(0,))
    a[1, 32:64] = np.nan
    a[1, 70] = np.nan
    # amax = 127 / 8, so s = 1/8 exactly (also the POW2 scale) and v / s is exact
    ties = np.array([127, 63.5, -63.5, 0.5, -0.5, 1.5, -2.5, 126.5, -126.5, 3, 0, 7.5, -7.5, 100.5, -0.25, 0.75] * 2)
    a[4, 96:128] = (ties / 8).astype(np.float32)
    a[5, 128:160] = (np.arange(32) - 16).astype(np.float32) * np.float32(1e-40)
    inf_rows = act == hip.ActQuant.AMAX127
    if inf_rows:
        a[2, 160] = np.inf
        a[3, 200] = -np.inf
    ctx.set_act_quant(act)
    try:
        got = ctx.gemm_q_f32(m, n, k, a, wq, hip.WDtype.Q8_0)
    finally:
        ctx.set_act_quant(hip.ActQuant.AMAX127)
    want = oracle.gemm_qblock_i8(int(hip.WDtype.Q8_0), m, n, k, a, wq, None, pow2=(act == hip.ActQuant.POW2))
    if inf_rows:
        assert np.isnan(want[2]).all() and np.isnan(want[3]).all()
    assert np.isfinite(want[[0, 1, 4, 5]]).all()
    nw, ng = np.isnan(want), np.isnan(got)
    assert np.array_equal(nw, ng)
    assert np.array_equal(bits(got[~ng]), bits(want[~nw]))


def test_gemm_q_config1_rows_bit_exact(ctx, oracle):
    """Config-1 shape (M=1500, K=1280, N=5120): every output of 24 sampled
    rows (first, last, interior) bit-exact vs the oracle, and whole-matrix
    checksums of the resident and copy paths identical."""
    m, n, k = 1500, 5120, 1280
    print(f"[case] gemm_q config1 m={m} n={n} k={k}", flush=True)
    a, wq, _ = _gemm_case(oracle, hip.WDtype.Q8_0, m, n, k, seed=1, with_bias=False)
    got = ctx.gemm_q_f32(m, n, k, a, wq, hip.WDtype.Q8_0)
    rows = sorted(set([0, 1, 127, 128, 1407, 1408, 1499] + list(range(3, 1500, 89))))
    want = oracle.gemm_qblock_i8(8, len(rows), n, k, a[rows], wq)
    assert np.array_equal(bits(got[rows]), bits(want))
    w = ctx.upload_qweight(hip.WDtype.Q8_0, n, k, wq)
    da = hip.DeviceBuffer.from_array(ctx, a)
    do = hip.DeviceBuffer(ctx, m * n * 4)
    ctx.gemm_q_f32_dev(w, m, da, do)
    ctx.synchronize()
    res = do.download(np.float32, m * n).reshape(m, n)
    assert np.array_equal(bits(res), bits(got))


@pytest.mark.parametrize("act", [hip.ActQuant.AMAX127, hip.ActQuant.POW2])
@pytest.mark.parametrize("m,n,k", [(2100, 1930, 64), (1500, 1280, 96), (1500, 5120, 64)])
def test_gemm_q_tile_routes_rows_bit_exact(ctx, oracle, act, m, n, k):
    """Grids of >= 256 128 x 128 tiles run 64 x 64 wave tiles, smaller ones
    32 x 32 (2100 x 1930: 272 tiles; 1500 x 1280: 120; 1500 x 5120: 480).
    Ragged m and n, bias, both activation schemes: sampled rows bit-exact."""
    print(f"[case] gemm_q routes act={act.name} m={m} n={n} k={k}", flush=True)
    a, wq, bias = _gemm_case(oracle, hip.WDtype.Q8_0, m, n, k, seed=m + n + k, zero_rows=(5,))
    ctx.set_act_quant(act)
    try:
        got = ctx.gemm_q_f32(m, n, k, a, wq, hip.WDtype.Q8_0, bias)
    finally:
        ctx.set_act_quant(hip.ActQuant.AMAX127)
    rows = sorted(set([0, 5, 63, 64, 127, 128, m - 65, m - 64, m - 1] + list(range(9, m, 97))))
    want = oracle.gemm_qblock_i8(int(hip.WDtype.Q8_0), len(rows), n, k, a[rows], wq, bias,
                                 pow2=(act == hip.ActQuant.POW2))
    assert np.array_equal(bits(got[rows]), bits(want))


@pytest.mark.parametrize("act", [hip.ActQuant.AMAX127, hip.ActQuant.POW2])
@pytest.mark.parametrize("wd", [hip.WDtype.Q4_0, hip.WDtype.Q8_0])
@pytest.mark.parametrize("m,n,k", [(1, 16, 128), (3, 100, 256), (17, 48, 512), (33, 200, 128), (64, 1280, 5120),
                                   # the config-1 Q4_0 GEMV shapes: M in {1, 8, 64}, K = 1280, N in {1280, 5120}
                                   (1, 1280, 1280), (1, 5120, 1280), (8, 1280, 1280), (8, 5120, 1280),
                                   (64, 1280, 1280), (64, 5120, 1280)])
def test_decode_kernel_bit_exact(ctx, oracle, wd, act, m, n, k):
    """m <= 64 runs the compact-weight decode kernel: bit-exact vs the oracle
    and bit-identical to the tiled GEMM on the same inputs."""
    print(f"[case] decode wd={wd.name} act={act.name} m={m} n={n} k={k}", flush=True)
    a, wq, bias = _gemm_case(oracle, wd, m, n, k, seed=m * 31 + n + k, zero_rows=(0,) if m > 1 else ())
    ctx.set_act_quant(act)
    try:
        got = ctx.gemm_q_f32(m, n, k, a, wq, wd, bias)
        ctx.set_decode_kernel(False)
        tiled = ctx.gemm_q_f32(m, n, k, a, wq, wd, bias)
    finally:
        ctx.set_decode_kernel(True)
        ctx.set_act_quant(hip.ActQuant.AMAX127)
    want = oracle.gemm_qblock_i8(int(wd), m, n, k, a, wq, bias, pow2=(act == hip.ActQuant.POW2))
    assert np.array_equal(bits(got), bits(want))
    assert np.array_equal(bits(tiled), bits(got))


def test_graph_replay_matches_eager(ctx, oracle):
    """A captured [activation pass + decode GEMV + tiled GEMM] graph replayed
    several times, with eager work and synchronizations between replays:
    every replay equals the eager result bit for bit."""
    m, n, k = 8, 256, 512
    a, wq, bias = _gemm_case(oracle, hip.WDtype.Q4_0, m, n, k, seed=99)
    W = ctx.upload_qweight(hip.WDtype.Q4_0, n, k, wq)
    a2 = np.concatenate([a] * 9)[:72]
    W8 = ctx.upload_qweight(hip.WDtype.Q4_0, n, k, wq)
    da = hip.DeviceBuffer.from_array(ctx, a)
    da2 = hip.DeviceBuffer.from_array(ctx, a2)
    db = hip.DeviceBuffer.from_array(ctx, bias)
    do = hip.DeviceBuffer(ctx, m * n * 4)
    do2 = hip.DeviceBuffer(ctx, 72 * n * 4)
    qa, qa2 = ctx.qact(m, k), ctx.qact(72, k)

    def step():
        qa.quantize(m, da)
        ctx.gemm_qact_dev(W, qa, do, db)
        qa2.quantize(72, da2)
        ctx.gemm_qact_dev(W8, qa2, do2, db)

    step()
    ctx.synchronize()
    want1 = do.download(np.float32, m * n)
    want2 = do2.download(np.float32, 72 * n)
    assert np.array_equal(bits(want1), bits(oracle.gemm_qblock_i8(2, m, n, k, a, wq, bias).reshape(-1)))
    g = ctx.capture(step)
    for rep in range(4):
        do.upload(np.zeros(m * n, np.float32))
        do2.upload(np.zeros(72 * n, np.float32))
        ctx.gemm_q_f32(m, n, k, a, wq, hip.WDtype.Q4_0, bias)  # eager work between replays
        g.launch()
        ctx.synchronize()
        assert np.array_equal(bits(do.download(np.float32, m * n)), bits(want1)), rep
        assert np.array_equal(bits(do2.download(np.float32, 72 * n)), bits(want2)), rep


def test_gemm_q_tracks_f32_within_derived_bound(ctx, oracle):
    """INT8 vs the f32 dequant GEMV oracle: within 2x the activation-rounding
    bound (the rule of kquant_gemm_parity.rs:204-236 at group 32)."""
    m, n, k = 3, 24, 512
    for wd in (hip.WDtype.Q8_0, hip.WDtype.Q4_0):
        a, wq, _ = _gemm_case(oracle, wd, m, n, k, seed=5, with_bias=False)
        got = ctx.gemm_q_f32(m, n, k, a, wq, wd)
        mode = WD_MODE[wd]
        rb = (k // 32) * oracle.KV_BLOCK_BYTES[mode]
        for i in range(m):
            ref = oracle.dequant_gemv_scalar(mode, wq, n, k // 32, a[i])
            for j in range(n):
                bound = oracle.qblock_error_bound(int(wd), wq[j * rb:(j + 1) * rb], a[i])
                assert abs(got[i, j] - ref[j]) <= 2 * bound + 1e-6


def test_gemm_q_rejections(ctx):
    wq = np.zeros(16 * 34, np.uint8)
    with pytest.raises(hip.InvalidArgument):
        ctx.gemm_q_f32(1, 16, 31, np.zeros(31), wq, hip.WDtype.Q8_0)
    with pytest.raises(hip.InvalidArgument):
        ctx.gemm_q_f32(1, 16, 32, np.zeros(32), wq[:-1], hip.WDtype.Q8_0)
    with pytest.raises(hip.InvalidArgument):
        ctx.gemm_q_f32(0, 16, 32, np.zeros(0), wq, hip.WDtype.Q8_0)
    with pytest.raises(hip.UnsupportedOp):
        ctx.gemm_q_f32(1, 16, 32, np.zeros(32), wq, 99)


@pytest.mark.parametrize("wd,m", [(hip.WDtype.Q4_0, 1), (hip.WDtype.Q4_0, 37), (hip.WDtype.Q8_0, 64),
                                  (hip.WDtype.Q8_0, 65)])
def test_linear_group_equals_single_linears(ctx, wd, m):
    """One grouped launch over linears of different widths (some with bias)
    gives the same bits as gemm_qact_dev per weight; m = 65 takes the
    per-linear block-GEMM route."""
    print(f"[case] linear group wd={int(wd)} m={m}", flush=True)
    g = np.random.default_rng(int(wd) * 100 + m)
    k = 256
    mode = hip.KvQuant.Q4_0 if wd == hip.WDtype.Q4_0 else hip.KvQuant.Q8_0
    ns = [48, 1280, 16, 333, 512]
    Ws = [ctx.upload_qweight(wd, n, k, ctx.quantize_bytes(mode, (g.standard_normal((n, k)) * 0.05).astype(np.float32)))
          for n in ns]
    biases = [None if i % 2 else hip.DeviceBuffer.from_array(ctx, g.standard_normal(n).astype(np.float32))
              for i, n in enumerate(ns)]
    a = g.standard_normal((m, k)).astype(np.float32)
    qa = ctx.qact(m, k)
    qa.quantize(m, hip.DeviceBuffer.from_array(ctx, a))
    outs = [hip.DeviceBuffer(ctx, m * n * 4) for n in ns]
    group = hip.LinearGroup(ctx, Ws, outs, biases)
    group.run(qa)
    got = [o.download(np.float32, m * n) for o, n in zip(outs, ns)]
    for W, b, n, gv in zip(Ws, biases, ns, got):
        d_o = hip.DeviceBuffer(ctx, m * n * 4)
        ctx.gemm_qact_dev(W, qa, d_o, d_bias=b)
        assert np.array_equal(gv.view(np.uint32), d_o.download(np.float32, m * n).view(np.uint32)), n


def test_linear_group_rejections(ctx):
    g = np.random.default_rng(3)
    k = 256
    w8 = ctx.upload_qweight(hip.WDtype.Q8_0, 32, k, ctx.quantize_bytes(hip.KvQuant.Q8_0, g.standard_normal((32, k))))
    w4 = ctx.upload_qweight(hip.WDtype.Q4_0, 32, k, ctx.quantize_bytes(hip.KvQuant.Q4_0, g.standard_normal((32, k))))
    w8b = ctx.upload_qweight(hip.WDtype.Q8_0, 32, 512, ctx.quantize_bytes(hip.KvQuant.Q8_0, g.standard_normal((32, 512))))
    o = hip.DeviceBuffer(ctx, 64 * 32 * 4)
    with pytest.raises(hip.InvalidArgument, match="differs from weight 0"):
        hip.LinearGroup(ctx, [w8, w4], [o, o])
    with pytest.raises(hip.InvalidArgument, match="differs from weight 0"):
        hip.LinearGroup(ctx, [w8, w8b], [o, o])
    group = hip.LinearGroup(ctx, [w8], [o])
    qa = ctx.qact(4, 512)
    qa.quantize(4, hip.DeviceBuffer.from_array(ctx, g.standard_normal((4, 512)).astype(np.float32)))
    with pytest.raises(hip.InvalidArgument, match="activation k=512"):
        group.run(qa)

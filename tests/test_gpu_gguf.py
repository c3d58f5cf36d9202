"""Block-quant weights loaded straight from a GGUF mapping give the same GEMM
outputs, bit for bit, as the same wire bytes uploaded directly, on both the
prefill (block GEMM) and decode (M <= 64) kernels. Dims are [out, in], as the
reference's Whisper loader reads a Linear weight."""
import numpy as np
import pytest

from tests import gguf_writer as gw
from vokra_amd import hip

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    c = hip.HipContext(0)
    yield c
    c.close()


def test_gguf_weights_match_direct_upload(ctx, oracle, tmp_path):
    print("[case] gguf upload == direct upload", flush=True)
    g = np.random.default_rng(5)
    n, k = 96, 512
    w = (g.standard_normal((n, k)) * 0.05).astype(np.float32)
    wires = {
        "q8": (hip.WDtype.Q8_0, ctx.quantize_bytes(hip.KvQuant.Q8_0, w)),
        "q4": (hip.WDtype.Q4_0, ctx.quantize_bytes(hip.KvQuant.Q4_0, w)),
        "q5": (hip.WDtype.Q5_0, ctx.quantize_bytes(hip.KvQuant.Q5_0, w)),
        "qk": (hip.WDtype.Q4_K, oracle.kquant_quantize(12, w.reshape(-1))),
    }
    tensors = [(f"blk.0.{name}.weight", [n, k], int(wd), bytes(np.asarray(b, np.uint8)))
               for name, (wd, b) in wires.items()]
    path = tmp_path / "w.gguf"
    path.write_bytes(gw.build([("general.architecture", gw.STRING, "whisper")], tensors, alignment=64))
    f = hip.GgufFile(str(path))
    for m in (37, 8):  # prefill GEMM, decode kernel
        a = g.standard_normal((m, k)).astype(np.float32)
        d_a = hip.DeviceBuffer.from_array(ctx, a)
        for name, (wd, b) in wires.items():
            act = hip.ActQuant.KQUANT if wd == hip.WDtype.Q4_K else hip.ActQuant.AMAX127
            qa = ctx.qact(m, k)
            qa.quantize(m, d_a, act)
            outs = []
            for W in (f.upload_qweight(ctx, f"blk.0.{name}.weight"), ctx.upload_qweight(wd, n, k, b)):
                d_o = hip.DeviceBuffer(ctx, m * n * 4)
                ctx.gemm_qact_dev(W, qa, d_o)
                outs.append(d_o.download(np.float32, m * n))
            assert np.array_equal(outs[0], outs[1]), (name, m)
    with pytest.raises(hip.UnsupportedOp):
        p2 = tmp_path / "f.gguf"
        p2.write_bytes(gw.build([], [("g", [8], gw.GGML_F32, bytes(32))]))
        hip.GgufFile(str(p2)).upload_qweight(ctx, "g")

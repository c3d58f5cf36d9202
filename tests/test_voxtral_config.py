"""VoxtralConfig from GGUF metadata (vokra_hip_voxtral_config_from_gguf), the
cases of crates/vokra-models/src/voxtral/config.rs:269-399: the legacy file
without a head_dim key (derived 3072 / 24 = 128), the shipping mini shape with
an explicit head_dim that decouples q_hidden from hidden_dim, the
divisibility rule that applies only to a derived head_dim, a missing required
key, the GQA split and the audio-encoder head split. Metadata parsing touches
no GPU."""
import pytest

from tests import gguf_writer as gw
from vokra_amd import hip

P = "vokra.voxtral."
VALID = [  # valid_builder (config.rs:274-298), in its order
    ("audio_encoder.n_layer", gw.U32, 24), ("audio_encoder.hidden_dim", gw.U32, 1024),
    ("audio_encoder.n_head", gw.U32, 16), ("audio_encoder.n_ctx", gw.U32, 1500),
    ("audio_encoder.n_mels", gw.U32, 128), ("audio_encoder.ffn_dim", gw.U32, 4096),
    ("text_decoder.n_layer", gw.U32, 28), ("text_decoder.hidden_dim", gw.U32, 3072),
    ("text_decoder.ffn_dim", gw.U32, 8192), ("text_decoder.vocab_size", gw.U32, 32000),
    ("text_decoder.n_ctx", gw.U32, 32768), ("text_decoder.n_head_q", gw.U32, 24),
    ("text_decoder.n_head_kv", gw.U32, 8), ("text_decoder.rope_base", gw.F32, 1_000_000.0),
    ("text_decoder.rms_norm_eps", gw.F32, 1e-5), ("cross_attn.hidden_dim", gw.U32, 1024),
    ("mode", gw.STRING, "asr"), ("s2s.codec_type", gw.STRING, "none"),
]


def meta(**over):
    """VALID with some keys replaced (value) or added; a value of None drops the key."""
    out, seen = [], set()
    for k, t, v in VALID:
        if k in over:
            seen.add(k)
            if over[k] is None:
                continue
            v = over[k]
        out.append((P + k, t, v))
    for k, v in over.items():
        if k not in seen and v is not None:
            out.append((P + k, gw.U32, v))
    return out


def load(tmp_path, m):
    p = tmp_path / "vox.gguf"
    p.write_bytes(gw.build(m))
    return hip.GgufFile(str(p)).voxtral_config()


def head_dim(c):
    """TextDecoderConfig::head_dim (config.rs:108-115)."""
    return c["head_dim"] if c["head_dim"] else c["hidden_dim"] // c["n_head_q"]


def test_reads_legacy_hparams_without_head_dim_key(tmp_path):
    c = load(tmp_path, meta())
    assert c["audio_n_layer"] == 24 and c["audio_hidden_dim"] == 1024
    assert c["audio_hidden_dim"] // c["audio_n_head"] == 64
    assert (c["n_layer"], c["n_head_q"], c["n_head_kv"]) == (28, 24, 8)
    assert c["head_dim"] == 0                     # no explicit key: the 0 sentinel
    assert head_dim(c) == 128                     # derived hidden_dim / n_head_q
    assert c["n_head_q"] * head_dim(c) == 3072 and c["n_head_kv"] * head_dim(c) == 1024
    assert abs(c["rope_base"] - 1_000_000.0) < 1.0 and c["rms_norm_eps"] == pytest.approx(1e-5)
    assert (c["vocab_size"], c["n_ctx"], c["ffn_dim"], c["cross_attn_hidden_dim"]) == (32000, 32768, 8192, 1024)


def test_reads_real_mini_hparams_with_explicit_head_dim(tmp_path):
    c = load(tmp_path, meta(**{"text_decoder.n_layer": 30, "text_decoder.n_head_q": 32,
                               "text_decoder.n_head_kv": 8, "text_decoder.head_dim": 128,
                               "text_decoder.vocab_size": 131_072}))
    assert (c["n_layer"], c["n_head_q"], c["n_head_kv"], head_dim(c)) == (30, 32, 8, 128)
    assert c["n_head_q"] * head_dim(c) == 4096 and c["n_head_kv"] * head_dim(c) == 1024


def test_explicit_head_dim_lifts_the_divisibility_requirement(tmp_path):
    c = load(tmp_path, meta(**{"text_decoder.hidden_dim": 3070, "text_decoder.n_head_q": 32,
                               "text_decoder.head_dim": 128}))
    assert head_dim(c) == 128
    with pytest.raises(hip.ModelLoad, match=r"voxtral config: text_decoder.n_head_q \(32\) must divide "
                                            r"text_decoder.hidden_dim \(3070\)"):
        load(tmp_path, meta(**{"text_decoder.hidden_dim": 3070, "text_decoder.n_head_q": 32}))


def test_missing_required_key_is_model_load_error(tmp_path):
    with pytest.raises(hip.ModelLoad, match="missing metadata key `vokra.voxtral.audio_encoder.n_layer`"):
        load(tmp_path, [(P + "audio_encoder.hidden_dim", gw.U32, 1024)])
    for key in ("audio_encoder.n_mels", "text_decoder.n_layer", "text_decoder.hidden_dim", "text_decoder.ffn_dim"):
        with pytest.raises(hip.ModelLoad, match=f"missing metadata key `{P + key}`"):
            load(tmp_path, meta(**{key: None}))
    # optional keys read as 0 when absent or of another type
    c = load(tmp_path, meta(**{"text_decoder.vocab_size": None, "audio_encoder.n_ctx": None}))
    assert c["vocab_size"] == 0 and c["audio_n_ctx"] == 0
    m = [(k, gw.I32 if k.endswith("n_ctx") else t, v) for k, t, v in meta()]
    assert load(tmp_path, m)["n_ctx"] == 0
    with pytest.raises(hip.ModelLoad, match="is not a u32-range integer"):
        load(tmp_path, [(k, gw.I32 if k.endswith("text_decoder.n_layer") else t, v) for k, t, v in meta()])


def test_gqa_head_split_must_divide_query_heads(tmp_path):
    with pytest.raises(hip.ModelLoad, match=r"text_decoder.n_head_kv \(7\) must divide text_decoder.n_head_q \(24\)"):
        load(tmp_path, meta(**{"text_decoder.n_head_kv": 7}))


def test_audio_encoder_head_split_must_divide_hidden_dim(tmp_path):
    with pytest.raises(hip.ModelLoad, match=r"audio_encoder.n_head \(7\) must divide audio_encoder.hidden_dim"):
        load(tmp_path, meta(**{"audio_encoder.n_head": 7}))

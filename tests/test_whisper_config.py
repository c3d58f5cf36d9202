"""WhisperConfig from GGUF metadata (vokra_hip_whisper_config_from_gguf), the
cases of crates/vokra-models/src/whisper/config.rs:246-560: the base chunk,
the five published Whisper sizes, the optional alignment heads, and every
rejection (missing key, signed or out-of-range value, non-array, empty start
ids, n_text_state != n_audio_state, a head count not dividing d_model, a zero
hyperparameter). Metadata parsing touches no GPU."""
import pytest

from tests import gguf_writer as gw
from vokra_amd import hip

KEYS = ("n_mels", "n_audio_ctx", "n_audio_state", "n_audio_head", "n_audio_layer", "n_text_ctx", "n_text_state",
        "n_text_head", "n_text_layer", "n_vocab", "ffn_dim", "eot")
BASE = dict(n_mels=80, n_audio_ctx=1500, n_audio_state=512, n_audio_head=8, n_audio_layer=6, n_text_ctx=448,
            n_text_state=512, n_text_head=8, n_text_layer=6, n_vocab=51865, ffn_dim=2048, eot=50257)
START_IDS = [50258, 50259, 50359, 50363]


def meta(values=None, start=START_IDS, heads=None, drop=(), types=None):
    v = dict(BASE, **(values or {}))
    types = types or {}
    out = [(f"vokra.whisper.{k}", types.get(k, gw.U32), v[k]) for k in KEYS if k not in drop]
    if start is not None:
        out.append(("vokra.whisper.decoder_start_ids", gw.ARRAY, (gw.U32, start)))
    if heads is not None:
        out.append(("vokra.whisper.alignment_heads", gw.ARRAY, (gw.U32, heads)))
    return out


def load(tmp_path, m):
    p = tmp_path / "cfg.gguf"
    p.write_bytes(gw.build(m))
    return hip.GgufFile(str(p)).whisper_config()


def test_reads_whisper_base_hparams(tmp_path):
    c = load(tmp_path, meta())
    assert (c["n_mels"], c["d_model"], c["n_audio_ctx"], c["n_audio_layer"], c["n_text_layer"]) == (80, 512, 1500, 6, 6)
    assert (c["n_audio_head"], c["d_model"] // c["n_audio_head"], c["n_vocab"], c["ffn_dim"], c["eot"]) == \
        (8, 64, 51865, 2048, 50257)
    assert (c["n_text_ctx"], c["n_text_head"]) == (448, 8)


# OpenAI's published sizes (config.rs:330-420): layers, mels, vocab, d_model, heads, ffn
SIZES = [("base", 6, 6, 80, 51865, 512, 8, 2048), ("small", 12, 12, 80, 51865, 768, 12, 3072),
         ("medium", 24, 24, 80, 51865, 1024, 16, 4096), ("large-v3", 32, 32, 128, 51866, 1280, 20, 5120),
         ("turbo", 32, 4, 128, 51866, 1280, 20, 5120)]


@pytest.mark.parametrize("name,na,nt,mels,vocab,d,h,ff", SIZES)
def test_reads_all_whisper_sizes(tmp_path, name, na, nt, mels, vocab, d, h, ff):
    c = load(tmp_path, meta(dict(n_audio_layer=na, n_text_layer=nt, n_mels=mels, n_vocab=vocab, n_audio_state=d,
                                 n_text_state=d, n_audio_head=h, n_text_head=h, ffn_dim=ff)))
    assert (c["n_audio_layer"], c["n_text_layer"], c["n_mels"], c["n_vocab"]) == (na, nt, mels, vocab)
    assert (c["d_model"], c["n_audio_head"], c["n_text_head"], c["ffn_dim"]) == (d, h, h, ff)
    assert c["d_model"] // c["n_audio_head"] == 64


def test_alignment_heads(tmp_path):
    load(tmp_path, meta(heads=[3, 1, 4, 2]))  # in range: accepted
    with pytest.raises(hip.ModelLoad, match="even-length"):
        load(tmp_path, meta(heads=[3, 1, 4]))
    with pytest.raises(hip.ModelLoad, match="layer index 6 >= n_text_layer 6"):
        load(tmp_path, meta(heads=[6, 0]))


@pytest.mark.parametrize("case,m,pattern", [
    ("missing key", dict(drop=("n_vocab",)), "missing metadata key `vokra.whisper.n_vocab`"),
    ("signed value", dict(types={"n_mels": gw.I32}), "`vokra.whisper.n_mels` is not a u32-range integer"),
    ("u64 beyond u32", dict(values={"eot": 1 << 33}, types={"eot": gw.U64}), "`vokra.whisper.eot` is not a u32"),
    ("string value", dict(values={"ffn_dim": "2048"}, types={"ffn_dim": gw.STRING}), "not a u32-range integer"),
    ("no start ids", dict(start=None), "missing metadata key `vokra.whisper.decoder_start_ids`"),
    ("empty start ids", dict(start=[]), "decoder_start_ids must not be empty"),
    ("state mismatch", dict(values={"n_text_state": 256}), r"n_text_state \(256\) != n_audio_state \(512\)"),
    ("audio heads", dict(values={"n_audio_head": 7}), r"n_audio_head \(7\) must divide d_model \(512\)"),
    ("text heads zero", dict(values={"n_text_head": 0}), r"n_text_head \(0\) must divide d_model"),
    ("zero layers", dict(values={"n_audio_layer": 0}), "a required Whisper hyperparameter was zero"),
    ("zero vocab", dict(values={"n_vocab": 0}), "a required Whisper hyperparameter was zero"),
])
def test_rejections(tmp_path, case, m, pattern):
    with pytest.raises(hip.ModelLoad, match=pattern):
        load(tmp_path, meta(**m))


def test_start_ids_must_be_unsigned_array(tmp_path):
    m = meta(start=None) + [("vokra.whisper.decoder_start_ids", gw.U32, 50258)]
    with pytest.raises(hip.ModelLoad, match="is not an array"):
        load(tmp_path, m)
    m = meta(start=None) + [("vokra.whisper.decoder_start_ids", gw.ARRAY, (gw.I32, [1, 2]))]
    with pytest.raises(hip.ModelLoad, match="element is not a u32-range integer"):
        load(tmp_path, m)

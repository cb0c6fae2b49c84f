"""CPU checks of the host parts of the reference's C API mirror (c_api.rs):

- qasr_hip_text_tokens against a restatement of transcribe_segment's text
  rule (transcribe.rs:196-214: tokens after <asr_text> 151704, stop at
  151643 / 151645, a second <asr_text> is not text) on hand-made sequences;
- qasr_hip_engine_detect (QwenConfig::detect, config.rs:108-156) on
  checkpoints written by the safetensors library: decoder width, vocab and
  intermediate from the tensor shapes, the large encoder when audio_tower
  layer 18 exists, layer counts from the names present.
No GPU: both run on the host."""
import numpy as np
import pytest

ASR_TEXT, EOT, IM_END = 151704, 151643, 151645


def text_rule(raw):
    out, past = [], False
    for t in raw:
        if t in (EOT, IM_END):
            break
        if t == ASR_TEXT:
            past = True
        elif past:
            out.append(t)
    return out


@pytest.mark.parametrize("raw", [
    [], [5, 6, 7], [ASR_TEXT], [5, ASR_TEXT, 7, 8, IM_END, 9], [ASR_TEXT, 1, EOT, ASR_TEXT, 2],
    [1, 2, ASR_TEXT, 3, ASR_TEXT, 4], [IM_END, ASR_TEXT, 1], [ASR_TEXT, 151644, 198, 0, 151935],
])
def test_text_tokens(raw):
    from qwenasr_amd.model import text_tokens
    assert text_tokens(np.array(raw, np.int32)).tolist() == text_rule(raw)


def test_text_tokens_random():
    from qwenasr_amd.model import text_tokens
    r = np.random.default_rng(5)
    for _ in range(200):
        raw = r.choice([1, 2, 3, ASR_TEXT, EOT, IM_END, 9], size=r.integers(0, 30), p=[.3, .2, .2, .1, .05, .05, .1])
        assert text_tokens(raw.astype(np.int32)).tolist() == text_rule(raw.tolist())


def tiny_tensors(dec_layers=2, enc_layers=2, hidden=128, inter=256, vocab=1000, large=False):
    from conftest import bf16
    z = lambda *s: (bf16(np.zeros(s, np.float32)), "BF16")
    t = {"thinker.model.embed_tokens.weight": z(vocab, hidden)}
    for i in range(dec_layers):
        t[f"thinker.model.layers.{i}.self_attn.q_proj.weight"] = z(2048, hidden)
        t[f"thinker.model.layers.{i}.mlp.gate_proj.weight"] = z(inter, hidden)
    for i in range(enc_layers):
        t[f"thinker.audio_tower.layers.{i}.self_attn.q_proj.weight"] = z(4, 4)
    if large:
        t["thinker.audio_tower.layers.18.self_attn.q_proj.weight"] = z(4, 4)
    return t


@pytest.mark.parametrize("case", [
    dict(hidden=1024, inter=3072, vocab=4096, dec_layers=3, enc_layers=2),
    dict(hidden=2048, inter=6144, vocab=2048, dec_layers=2, enc_layers=1, large=True),
    dict(hidden=128, inter=256, vocab=151936, dec_layers=1, enc_layers=4),
])
def test_engine_detect(tmp_path, case):
    from qwenasr_amd.model import Checkpoint, detect_config
    from qwenasr_amd.synth import write_checkpoint
    write_checkpoint(str(tmp_path / "m"), tiny_tensors(**case), shards=2)
    ck = Checkpoint(tmp_path / "m")
    dc, ec = detect_config(ck)
    ck.close()
    large = case.get("large", False)
    assert dc["hidden"] == case["hidden"] and dc["vocab"] == case["vocab"] and dc["intermediate"] == case["inter"]
    assert dc["n_layers"] == case["dec_layers"]
    assert (dc["n_heads"], dc["n_kv_heads"], dc["head_dim"]) == (16, 8, 128)
    # layer 18 present: counted layers stop at the first gap (0..enc_layers-1)
    assert ec["n_layers"] == case["enc_layers"]
    assert (ec["d_model"], ec["n_heads"], ec["ffn_dim"]) == ((1024, 16, 4096) if large else (896, 14, 3584))
    assert ec["output_dim"] == case["hidden"] and ec["chunk_size"] == 100 and ec["conv_hidden"] == 480

"""GPU parity of the streaming driver (qasr_hip_stream_*, stream_push_audio,
transcribe.rs:902-1304) against the oracle's restatement on the same seeded
model and audio: the token ids committed by every push and the chunk
statistics (chunks, reused prefill rows, prefill length, rows prefilled,
encoder windows, raw tokens) must be identical."""
import numpy as np
import pytest

from test_oracle_stream import DEC

pytestmark = pytest.mark.gpu

STAT_COLS = [0, 1, 2, 3, 6, 7]   # forwards (4, 5) differ: the GPU decodes in bursts


@pytest.fixture(scope="module")
def models(dev, orc):
    from qwenasr_amd.model import Decoder, Encoder
    from qwenasr_amd.synth import ENC_0_6B, SynthDecoder, SynthEncoder, audio
    wd = SynthDecoder(DEC, seed=1004)
    we = SynthEncoder(dict(ENC_0_6B, n_layers=2), seed=1004)
    gdec, genc = Decoder(dev, wd, max_seq=1024), Encoder(dev, we)
    cdec, cenc = orc.OracleDecoder(wd, max_seq=1024), orc.OracleEncoder(we)
    x = audio(int(10.5 * 16000), 1004)
    yield gdec, genc, cdec, cenc, x
    cdec.close()
    cenc.close()


def run_both(models, orc, ends, final_end, **cfg):
    from qwenasr_amd.model import Stream
    gdec, genc, cdec, cenc, x = models
    g = Stream(gdec, genc, **cfg)
    c = orc.OracleStream(cdec, cenc, **cfg)
    for end in ends:
        print(f"push {end} samples", flush=True)
        eg, ec = g.push(x[:end]), c.push(x[:end])
        assert list(eg) == list(ec), (end, eg, ec)
        sg, sc = g.stats(), c.stats()
        assert list(sg[STAT_COLS]) == list(sc[STAT_COLS]), (end, sg, sc)
    if final_end:
        eg, ec = g.push(x[:final_end], finalize=True), c.push(x[:final_end], finalize=True)
        assert list(eg) == list(ec), (eg, ec)
    assert list(g.tokens()) == list(c.tokens())
    out = (g.tokens(), g.stats())
    g.close()
    c.close()
    return out


def test_stream_short_tokens_window_cache(models, orc):
    """max_new_tokens 3 / rollback 1: prefix reuse, rollback emission, the 8 s
    window cached, finalize."""
    toks, st = run_both(models, orc, [32000, 64000, 96000, 128000, 160000], 168000, max_new_tokens=3, rollback=1)
    assert st[6] == 1 and len(toks) > 0


def test_stream_defaults_degenerate_reset(models, orc):
    """QwenCtx defaults: a random-init model's repeated tokens reset the stream every chunk."""
    run_both(models, orc, [32000, 64000, 96000], 0)


def test_stream_stop_token(models, orc):
    """A stop token that the model emits first: empty chunks, speech end."""
    first = orc.transcribe_forced(models[2], models[3], models[4][:32000], 1)["tokens"][0]
    run_both(models, orc, [32000, 64000, 96000], 100000, max_new_tokens=4, stop_tokens=(int(first), -1))


def test_stream_long_window_reuse(models, orc):
    """44 s pushed 2 s at a time, max_new_tokens 4 / rollback 1: the repeated
    tokens of the random-init model re-anchor the stream, and once 4 encoder
    windows are cached a re-anchor releases them (their buffers are reused by
    the windows encoded after), so the prompt shrinks at some push."""
    from qwenasr_amd.model import Stream
    from qwenasr_amd.synth import audio
    gdec, genc, cdec, cenc, _ = models
    x = audio(44 * 16000, 1044)
    cfg = dict(max_new_tokens=4, rollback=1)
    g = Stream(gdec, genc, **cfg)
    c = orc.OracleStream(cdec, cenc, **cfg)
    prefill = []
    for end in range(32000, x.size + 1, 32000):
        eg, ec = g.push(x[:end]), c.push(x[:end])
        assert list(eg) == list(ec), (end, eg, ec)
        sg, sc = g.stats(), c.stats()
        assert list(sg[STAT_COLS]) == list(sc[STAT_COLS]), (end, sg, sc)
        prefill.append(int(sg[2]))
    assert list(g.tokens()) == list(c.tokens())
    assert int(g.stats()[6]) >= 5
    assert any(b < a for a, b in zip(prefill, prefill[1:])), prefill
    g.close()
    c.close()


def test_stream_periodic_reanchor(models, orc):
    """48 pushes of 0.5 s chunks (chunk_sec 0.5, max_new_tokens 3, rollback 1):
    the stream passes chunk 45, where the reference re-anchors every 45 chunks
    whatever the tokens (transcribe.rs:1231-1252), and the GPU stream commits
    the oracle's tokens and statistics at every push.  After that chunk the
    raw tokens are <asr_text> and the last min(24, committed) committed tokens
    (the carry; this random-init model commits only a few), and the next chunk
    reuses no prefill rows."""
    from qwenasr_amd.model import Stream
    from qwenasr_amd.synth import audio
    gdec, genc, cdec, cenc, _ = models
    x = audio(24 * 16000, 1045)
    cfg = dict(max_new_tokens=3, rollback=1, chunk_sec=0.5)
    g = Stream(gdec, genc, **cfg)
    c = orc.OracleStream(cdec, cenc, **cfg)
    after = None
    for k, end in enumerate(range(8000, x.size + 1, 8000)):
        eg, ec = g.push(x[:end]), c.push(x[:end])
        assert list(eg) == list(ec), (k, eg, ec)
        sg, sc = g.stats(), c.stats()
        assert list(sg[STAT_COLS]) == list(sc[STAT_COLS]), (k, sg, sc)
        if int(sg[0]) == 46:                          # chunk index 45 processed
            committed = len(g.tokens())
            assert int(sg[7]) == (1 + min(24, committed) if committed else 0), (sg, committed)
            after = k
        if after is not None and k == after + 1:
            assert int(sg[1]) == 0, sg                # no prefill reuse after a re-anchor
    assert after is not None and int(g.stats()[0]) == 48
    assert list(g.tokens()) == list(c.tokens())
    g.close()
    c.close()

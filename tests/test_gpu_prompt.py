"""GPU parity of transcribe_segment's optional prompt ids and of transcribe_audio's
segmentation (transcribe.rs:63-403) through the C ABI, against the oracle on
the same seeded model and audio:

- qasr_hip_transcribe_prompt with a text prompt (between PREFIX_HEAD and
  PREFIX_TAIL), forced-language ids ending in <asr_text> (after SUFFIX_BASE)
  and past text ids closed by <asr_text>, alone and together: every token to
  the first stop equals the oracle's forced-length run;
- the engine (qwen_asr_set_language / set_segment_sec at token level):
  transcribe_pcm with a language, a prompt and segment_sec cuts the audio at
  the oracle's split points, zero-pads segments shorter than 0.5 s, and each
  segment's raw tokens agree with the oracle's run on that segment up to the
  first near-tie; the text ids are every segment's tokens before its stop
  (the forced language opens the text region), segment after segment;
- a stream with prompt and language ids commits, push for push, what the
  oracle's stream_push_audio commits with the same ids (text region from the
  first decoded token), also with past-text conditioning, and the engine's
  stream picks up the engine's language ids.
"""
import numpy as np
import pytest

from test_gpu_engine import TDEC, TENC, check_free_running

pytestmark = pytest.mark.gpu

ASR_TEXT, STOPS = 151704, (151643, 151645)
PROMPT, LANG, PAST = [9707, 11, 1879, 13], [11528, 6364], [40, 1079, 264, 1273, 30]
FORCE = LANG + [ASR_TEXT]


@pytest.fixture(scope="module")
def tiny(tmp_path_factory):
    from qwenasr_amd.synth import SynthDecoder, SynthEncoder, decoder_tensors, encoder_tensors, write_checkpoint
    wd, we = SynthDecoder(TDEC, seed=2301, std=0.05), SynthEncoder(TENC, seed=2302)
    t = decoder_tensors(wd, norm_dtype="F32")
    t.update(encoder_tensors(we, vec_dtype="F32"))
    path = tmp_path_factory.mktemp("engine_prompt") / "model"
    write_checkpoint(str(path), t, shards=1)
    return path, wd, we


def until_stop(toks):
    stop = next((i for i, t in enumerate(toks) if t in STOPS), None)
    return toks[:stop + 1] if stop is not None else toks


@pytest.mark.parametrize("ids", [dict(prompt=PROMPT), dict(force=FORCE), dict(past=PAST),
                                 dict(prompt=PROMPT, force=FORCE, past=PAST)],
                         ids=["prompt", "force", "past", "all"])
def test_transcribe_prompt_ids(dev, orc, tiny, ids):
    from qwenasr_amd.model import Decoder, Encoder, transcribe
    from qwenasr_amd.synth import audio
    _, wd, we = tiny
    x = audio(40000, 2303)
    d, e = Decoder(dev, wd, max_seq=512), Encoder(dev, we)
    od, oe = orc.OracleDecoder(wd, max_seq=512), orc.OracleEncoder(we)
    try:
        for m in (1, 24):
            print(f"ids {sorted(ids)} max_tokens {m}", flush=True)
            toks, _ = transcribe(d, e, x, max_tokens=m, **ids)
            want = until_stop(orc.transcribe_forced(od, oe, x, m, **ids)["tokens"].tolist())
            assert toks.tolist() == want, (m, toks.tolist(), want)
    finally:
        for o in (d, e, od, oe):
            o.close()


def split_raw(raw, n_seg):
    """The engine's raw tokens, segment by segment: each ends at its first stop or after 2048 tokens."""
    out, i = [], 0
    for _ in range(n_seg):
        j = i
        while j < len(raw) and j - i < 2048:
            j += 1
            if raw[j - 1] in STOPS:
                break
        out.append(raw[i:j])
        i = j
    assert i == len(raw)
    return out


@pytest.mark.parametrize("total_sec,segment_sec", [(14.0, 4.0), (1.7, 0.4)], ids=["4s_segments", "padded_segments"])
def test_engine_language_prompt_segments(orc, tiny, total_sec, segment_sec):
    from qwenasr_amd.model import Engine, text_tokens
    from qwenasr_amd.synth import audio
    path, wd, we = tiny
    x = audio(int(total_sec * 16000), 2304)
    g = Engine(path, device=0, max_seq=4096)
    od, oe = orc.OracleDecoder(wd, max_seq=4096), orc.OracleEncoder(we)
    try:
        g.set_language_tokens(LANG)
        g.set_prompt_tokens(PROMPT)
        g.set_segment_sec(segment_sec)
        text = g.transcribe_pcm(x)
        raw, segs = g.last_raw_tokens().tolist(), g.last_segments()
        splits = orc.segment_splits(x, segment_sec, 3.0).tolist()
        print("splits", splits, "raw", len(raw), flush=True)
        assert len(splits) >= 3
        assert segs[:, 0].tolist() == splits and segs[:, 1].tolist() == splits[1:] + [x.size]
        want_text, parts = [], split_raw(raw, len(splits))
        for k, (a, b) in enumerate(zip(segs[:, 0], segs[:, 1])):
            seg = x[a:b]
            if seg.size < 8000:                                # transcribe.rs:355-366
                seg = np.concatenate([seg, np.zeros(8000 - seg.size, np.float32)])
            got = parts[k]
            want = until_stop(orc.transcribe_forced(od, oe, seg, len(got), prompt=PROMPT, force=FORCE)["tokens"]
                              .tolist())
            print(f"segment {k}: samples {a}-{b}, {len(got)} tokens", flush=True)
            check_free_running(orc, od, oe, seg, got, want, prompt=PROMPT, force=FORCE)
            t = text_tokens(np.array(got, np.int32), text_open=True).tolist()
            assert segs[k, 2] == len(want_text) and segs[k, 3] == len(t)
            want_text += t
        assert text.tolist() == want_text
        g.set_segment_sec(0.0)
        g.set_language_tokens([])
        g.set_prompt_tokens([])
        g.transcribe_pcm(x[:32000])
        assert len(g.last_segments()) == 1
        with pytest.raises(RuntimeError, match="outside the vocabulary"):
            g.set_language_tokens([TDEC["vocab"]])
    finally:
        od.close()
        oe.close()
        g.close()


def test_stream_prompt_ids(dev, orc, tiny):
    """Streams with a prompt and a forced language (and with past-text
    conditioning) against the oracle's stream_push_audio with the same ids;
    the engine's stream with set_language_tokens commits the same tokens."""
    from qwenasr_amd.model import Decoder, Encoder, Engine, Stream
    from qwenasr_amd.synth import audio
    path, wd, we = tiny
    x = audio(9 * 16000, 2305)
    ends, final = [32000, 64000, 96000, 128000], x.size
    d, e = Decoder(dev, wd, max_seq=2048), Encoder(dev, we)
    od, oe = orc.OracleDecoder(wd, max_seq=2048), orc.OracleEncoder(we)
    pushes = {}
    try:
        for name, cfg in (("force", dict(max_new_tokens=4, rollback=1)),
                          ("force+past", dict(max_new_tokens=4, rollback=1, past_text_conditioning=1))):
            gs, cs = Stream(d, e, **cfg), orc.OracleStream(od, oe, **cfg)
            gs.set_prompt(prompt=PROMPT, force=FORCE)
            cs.set_prompt(prompt=PROMPT, force=FORCE)
            got_all = []
            for k, end in enumerate(ends + [final]):
                fin = end == final
                print(f"{name}: push {end} samples", flush=True)
                eg, ec = gs.push(x[:end], finalize=fin).tolist(), cs.push(x[:end], finalize=fin).tolist()
                assert eg == ec, (name, end, eg, ec)
                got_all.append(eg)
            assert gs.tokens().tolist() == cs.tokens().tolist()
            pushes[name] = got_all
            gs.close()
            cs.close()
    finally:
        for o in (d, e, od, oe):
            o.close()
    g = Engine(path, device=0, max_seq=2048)
    try:
        g.set_language_tokens(LANG)
        g.set_prompt_tokens(PROMPT)
        g.set_stream(max_new_tokens=4, rollback=1)
        s = g.stream()
        prev = 0
        for k, end in enumerate(ends + [final]):
            got = s.push(x[prev:end], finalize=(end == final)).tolist()
            prev = end
            assert got == pushes["force"][k], (k, got, pushes["force"][k])
        s.close()
    finally:
        g.close()


def test_stream_asr_text_model(dev, orc):
    """A model that emits <asr_text> at every step (plant_asr_text): the raw
    tokens then hold <asr_text> everywhere, so the text region's start (after
    the first one, or 0 with a forced language) and the re-anchor that puts
    one in front of the carried tokens decide what is committed.  Pushes of
    2 s with past-text conditioning, with and without a forced language: the
    GPU stream commits what the oracle's stream commits."""
    from conftest import ASR_TEXT, TINY_DEC, TINY_ENC, plant_asr_text
    from qwenasr_amd.model import Decoder, Encoder, Stream, transcribe
    from qwenasr_amd.synth import SynthDecoder, SynthEncoder, audio
    wd = plant_asr_text(SynthDecoder(TINY_DEC, seed=2401, std=0.05))
    we = SynthEncoder(TINY_ENC, seed=2402)
    x = audio(7 * 16000, 2404)
    d, e = Decoder(dev, wd, max_seq=1024), Encoder(dev, we)
    od, oe = orc.OracleDecoder(wd, max_seq=1024), orc.OracleEncoder(we)
    try:
        toks, _ = transcribe(d, e, x[:32000], max_tokens=4)
        assert toks.tolist() == [ASR_TEXT] * 4
        for ids in (dict(), dict(force=FORCE)):
            cfg = dict(max_new_tokens=3, rollback=1, unfixed_chunks=1, past_text_conditioning=1)
            gs, cs = Stream(d, e, **cfg), orc.OracleStream(od, oe, **cfg)
            gs.set_prompt(**ids)
            cs.set_prompt(**ids)
            for end in (32000, 64000, 96000, x.size):
                fin = end == x.size
                print(f"force {bool(ids)}: push {end}", flush=True)
                eg, ec = gs.push(x[:end], finalize=fin).tolist(), cs.push(x[:end], finalize=fin).tolist()
                assert eg == ec, (ids, end, eg, ec)
            assert gs.tokens().tolist() == cs.tokens().tolist()
            print("committed", cs.tokens().tolist(), flush=True)
            gs.close()
            cs.close()
    finally:
        for o in (d, e, od, oe):
            o.close()

"""GPU parity of the reference's C API mirror (c_api.rs) at token level.

- qasr_hip_transcribe (transcribe_segment's greedy loop to a stop token,
  transcribe.rs:186-230) with a small max_tokens: every token equals the
  oracle's forced-length run;
- qasr_hip_engine_*: a model directory written with the reference's tensor
  names (decoder 2 x 128-wide layers with the full vocabulary, a 2-layer
  896-wide encoder) loads with the detected config; transcribe_pcm's raw
  tokens (to the first stop token or 2048 tokens) equal the oracle's up to the
  first near-tie of its logits, and its text tokens are those after
  <asr_text> (qasr_hip_text_tokens, pinned on the CPU);
- the engine's streams, fed 2 s of new audio per push (the audio accumulates
  inside, as QwenAsrStreamState's buffer), commit what the library's Stream
  commits over the whole audio so far.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

TDEC = dict(n_layers=2, hidden=128, n_heads=16, n_kv_heads=8, head_dim=128, intermediate=256, vocab=151936,
            eps=1e-6, theta=1e6)
TENC = dict(d_model=896, n_layers=2, n_heads=14, head_dim=64, ffn_dim=3584, output_dim=128, chunk_size=100,
            n_window_infer=800, conv_hidden=480)


MARGIN_BOUND = 3e-3
HORIZON = 512


def check_free_running(orc, od, oe, x, got, want, **ids):
    """Free-running greedy runs agree token for token up to the first step
    where the oracle's best and second logits are within MARGIN_BOUND of the
    best (two int8 activation flips, as in the config-3 tests); past such a
    near-tie the two runs follow different texts and are not compared.  A
    first divergence after HORIZON tokens is reported, not bounded: by then
    the runs have attended over hundreds of KV rows whose f32 values differ in
    rounding (the oracle's BLAS-order GEMMs against the MFMA ones), and a
    random-init model's 2048-token free run meets gaps above the bound there
    (one at token 1370 with a gap of 4.0e-3).  ids: the prompt / force / past
    ids both runs used."""
    i = next((k for k, (a, b) in enumerate(zip(got, want)) if a != b), None)
    if i is None:
        assert len(got) == len(want)
        return
    assert i >= 1, (got[:1], want[:1])
    orc.transcribe_forced(od, oe, x, i, **ids)   # oracle state after i tokens
    t, best, second = od.forward_logits(od.embed(want[i - 1]))
    rel = (best - second) / max(abs(best), 1e-30)
    print(f"first divergence at token {i}: oracle {want[i]} gpu {got[i]}, relative top-2 gap {rel:.2e}", flush=True)
    assert t == want[i] and (rel < MARGIN_BOUND or i >= HORIZON), (i, rel)


@pytest.fixture(scope="module")
def engine_dir(tmp_path_factory):
    from qwenasr_amd.synth import SynthDecoder, SynthEncoder, decoder_tensors, encoder_tensors, write_checkpoint
    wd, we = SynthDecoder(TDEC, seed=2201, std=0.05), SynthEncoder(TENC, seed=2202)
    t = decoder_tensors(wd, norm_dtype="F32")
    t.update(encoder_tensors(we, vec_dtype="F32"))
    path = tmp_path_factory.mktemp("engine") / "model"
    write_checkpoint(str(path), t, shards=2)
    return path, wd, we


def test_transcribe_until_stop_matches_forced(dev, orc, engine_dir):
    from qwenasr_amd.model import Decoder, Encoder, transcribe
    from qwenasr_amd.synth import audio
    _, wd, we = engine_dir
    x = audio(32000, 2203)
    d, e = Decoder(dev, wd, max_seq=512), Encoder(dev, we)
    od, oe = orc.OracleDecoder(wd, max_seq=512), orc.OracleEncoder(we)
    try:
        for m in (1, 7, 24):
            toks, _ = transcribe(d, e, x, max_tokens=m)
            want = orc.transcribe_forced(od, oe, x, m)["tokens"].tolist()
            stop = next((i for i, t in enumerate(want) if t in (151643, 151645)), None)
            want = want[:stop + 1] if stop is not None else want
            assert toks.tolist() == want, (m, toks.tolist(), want)
    finally:
        for o in (d, e, od, oe):
            o.close()


def test_engine_transcribe(orc, engine_dir):
    from qwenasr_amd.model import Engine, text_tokens
    from qwenasr_amd.synth import audio
    path, wd, we = engine_dir
    print("engine load", flush=True)
    g = Engine(path, device=0, max_seq=4096)
    od, oe = orc.OracleDecoder(wd, max_seq=4096), orc.OracleEncoder(we)
    try:
        dc, ec = g.config()
        assert dc["n_layers"] == 2 and dc["hidden"] == 128 and dc["vocab"] == 151936 and dc["intermediate"] == 256
        assert ec["n_layers"] == 2 and ec["d_model"] == 896 and ec["output_dim"] == 128
        x = audio(48000, 2204)
        text = g.transcribe_pcm(x)
        raw = g.last_raw_tokens()
        print("engine raw tokens", len(raw), raw[:12].tolist(), flush=True)
        want = orc.transcribe_forced(od, oe, x, len(raw))["tokens"].tolist()
        check_free_running(orc, od, oe, x, raw.tolist(), want)
        assert len(raw) == 2048 or raw[-1] in (151643, 151645)
        assert text.tolist() == text_tokens(raw).tolist()
    finally:
        od.close()
        oe.close()
        g.close()


def test_engine_stream(dev, engine_dir):
    """The engine's streams against the library's Stream on a second copy of
    the same weights (bit-identical kernels; Stream itself is pinned to the
    oracle's stream_push_audio): 2 s pushes of new audio commit the same
    tokens, also when a second stream and a transcribe_pcm write the decoder's
    KV cache between the pushes; a stream outliving its engine is refused."""
    from qwenasr_amd.model import Decoder, Encoder, Engine, Stream
    from qwenasr_amd.synth import audio
    path, wd, we = engine_dir
    cfg = dict(max_new_tokens=4, rollback=1)
    xs, ys = audio(5 * 32000, 2205), audio(3 * 32000, 2206)
    d, e = Decoder(dev, wd, max_seq=4096), Encoder(dev, we)
    ref_x, ref_y = Stream(d, e, **cfg), None
    want_x = [ref_x.push(xs[:(k + 1) * 32000], finalize=(k == 4)).tolist() for k in range(5)]
    all_x = ref_x.tokens().tolist()
    ref_x.close()
    ref_y = Stream(d, e, **cfg)
    want_y = [ref_y.push(ys[:(k + 1) * 32000]).tolist() for k in range(3)]
    ref_y.close()
    d.close()
    e.close()
    print("reference streams", want_x, want_y, flush=True)
    g = Engine(path, device=0, max_seq=4096)
    try:
        s = g.stream()
        g.set_stream(**cfg)          # applies from the next push, as the reference reads its context per push
        for k in range(5):
            assert s.push(xs[k * 32000:(k + 1) * 32000], finalize=(k == 4)).tolist() == want_x[k], k
        assert s.result().tolist() == all_x
        s.reset()
        t = g.stream()
        for k in range(5):                      # interleaved: stream t and transcribe_pcm in between
            got = s.push(xs[k * 32000:(k + 1) * 32000], finalize=(k == 4)).tolist()
            assert got == want_x[k], ("interleaved", k, got, want_x[k])
            if k < 3:
                got = t.push(ys[k * 32000:(k + 1) * 32000]).tolist()
                assert got == want_y[k], ("second stream", k, got, want_y[k])
            if k == 1:
                g.transcribe_pcm(ys[:16000])
        assert s.result().tolist() == all_x
        t.close()
    finally:
        g.close()
    with pytest.raises(RuntimeError, match="engine was freed"):
        s.push(xs[:1600])
    s.close()


def test_engine_edge_cases(engine_dir):
    """Audio shorter than one mel frame is refused before any launch; a push of
    no new samples commits nothing; a stream's result before any push is empty."""
    from qwenasr_amd._lib import QasrError
    from qwenasr_amd.model import Engine
    path, _, _ = engine_dir
    g = Engine(path, device=0, max_seq=1024)
    try:
        with pytest.raises(QasrError, match="too short|bad arguments"):
            g.transcribe_pcm(np.zeros(100, np.float32))
        s = g.stream()
        assert s.result().tolist() == []
        assert s.push(np.zeros(0, np.float32)).tolist() == []
        assert s.result().tolist() == []
        s.close()
    finally:
        g.close()

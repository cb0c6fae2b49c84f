"""GPU parity of the multi-stream streaming driver (qasr_hip_stream_batch_*:
BASELINE config 4 fed by the real chunked pipeline, stream_push_audio,
transcribe.rs:902-1304): several streams with their own audio push 2 s
chunks; each chunk's encoder and prompt prefill go to the stream's slot of a
multi-stream batch and the greedy steps of every stream with a chunk run as one
batched decode.  Every stream's committed token ids per push, and its chunk
statistics, must equal the oracle's stream_push_audio run on that stream
alone (short decodes: 3-4 new tokens per chunk), and at 32 new tokens per
chunk the lone GPU stream on the same decoder must agree push for push."""
import numpy as np
import pytest

from test_oracle_stream import DEC

pytestmark = pytest.mark.gpu

STAT_COLS = [0, 1, 2, 3, 6, 7]   # forwards (4, 5) differ: the decode runs in bursts


@pytest.fixture(scope="module")
def models(dev, orc):
    from qwenasr_amd.model import Decoder, Encoder
    from qwenasr_amd.synth import ENC_0_6B, SynthDecoder, SynthEncoder
    wd = SynthDecoder(DEC, seed=1004)
    we = SynthEncoder(dict(ENC_0_6B, n_layers=2), seed=1004)
    gdec, genc = Decoder(dev, wd, max_seq=1024), Encoder(dev, we)
    cdec, cenc = orc.OracleDecoder(wd, max_seq=1024), orc.OracleEncoder(we)
    yield gdec, genc, cdec, cenc
    cdec.close()
    cenc.close()


def schedule(n_streams, n_pushes):
    """Per stream: its audio and the sample counts of its pushes (ragged starts;
    stream 3 gets new audio only every other push, so some rounds leave its slot
    idle), the last push finalizing with a partial chunk."""
    from qwenasr_amd.synth import audio
    plans = []
    for i in range(n_streams):
        start = 32000 * (1 + i % 3)
        ends = []
        for k in range(n_pushes):
            step = 0 if (i == 3 and k % 2 == 1) else 32000
            ends.append(start if k == 0 else ends[-1] + step)
        final = ends[-1] + 8000 * (1 + i % 2)
        plans.append((audio(final, 1004 + 7 * i), ends, final))
    return plans


def oracle_runs(orc, cdec, cenc, plans, cfg, prompts=None):
    out = []
    for i, (x, ends, final) in enumerate(plans):
        c = orc.OracleStream(cdec, cenc, **cfg)
        if prompts and prompts[i]:
            c.set_prompt(**prompts[i])
        pushes = [(c.push(x[:e]).tolist(), c.stats().tolist()) for e in ends]
        pushes.append((c.push(x[:final], finalize=True).tolist(), c.stats().tolist()))
        out.append((pushes, c.tokens().tolist()))
        c.close()
    return out


def run_batch(models, orc, n_streams, n_pushes, prompts=None, **cfg):
    from qwenasr_amd.model import StreamBatch
    gdec, genc, cdec, cenc = models
    plans = schedule(n_streams, n_pushes)
    want = oracle_runs(orc, cdec, cenc, plans, cfg, prompts)
    g = StreamBatch(gdec, genc, n_streams, 1024, **cfg)
    try:
        for i in range(n_streams):
            if prompts and prompts[i]:
                g.stream(i).set_prompt(**prompts[i])
        for k in range(n_pushes + 1):
            fin = k == n_pushes
            xs = [x[:(final if fin else ends[k])] for x, ends, final in plans]
            print(f"push {k}: samples {[len(x) for x in xs]}", flush=True)
            got = g.push(xs, finalize=[fin] * n_streams)
            for i in range(n_streams):
                exp_tok, exp_st = want[i][0][k]
                assert got[i].tolist() == exp_tok, (k, i, got[i].tolist(), exp_tok)
                st = g.stream(i).stats()
                assert [int(st[c]) for c in STAT_COLS] == [exp_st[c] for c in STAT_COLS], (k, i, st, exp_st)
        for i in range(n_streams):
            assert g.stream(i).tokens().tolist() == want[i][1]
    finally:
        g.close()
    return plans, want


def test_stream_batch_short_tokens(models, orc):
    """4 streams, max_new_tokens 3 / rollback 1: prefix reuse in each slot,
    rollback emission, ragged and idle rounds, finalize."""
    plans, want = run_batch(models, orc, 4, 4, max_new_tokens=3, rollback=1)
    assert sum(len(w[1]) for w in want) > 0


def test_stream_batch_eight_streams(models, orc):
    """8 streams, max_new_tokens 4 / rollback 1 / unfixed_chunks 1: every
    stream emits from its second chunk on."""
    run_batch(models, orc, 8, 4, max_new_tokens=4, rollback=1, unfixed_chunks=1)


def test_stream_batch_prompt_ids(models, orc):
    """4 streams with different prompt ids (none, a forced language ending in
    <asr_text>, a text prompt, both), so the slots' prompts differ in length:
    each stream commits what the oracle's stream commits with its ids."""
    lang = [11528, 6364, 151704]
    prompts = [None, dict(force=lang), dict(prompt=[9707, 11, 1879]), dict(prompt=[9707], force=lang)]
    run_batch(models, orc, 4, 3, prompts=prompts, max_new_tokens=3, rollback=1)


def test_stream_batch_matches_lone_stream(models, orc):
    """6 streams at QwenCtx's defaults (32 new tokens per chunk: 8 decode
    bursts) against the lone GPU stream on the same decoder (whose steps use
    the batch's arithmetic once a batch exists): every push identical.  Not
    against the oracle: at 32 free-running tokens per chunk two of these
    streams reach oracle top-2 gaps of 2.4e-3 and 2.4e-4 of the best logit
    (tokens 28 and 25 of a chunk), under the 3e-3 that one int8 activation
    flip can move."""
    from qwenasr_amd.model import Stream, StreamBatch
    gdec, genc, _, _ = models
    plans = schedule(6, 3)
    g = StreamBatch(gdec, genc, 6, 1024)
    try:
        got = [[] for _ in plans]
        for k in range(4):
            fin = k == 3
            res = g.push([x[:(final if fin else ends[k])] for x, ends, final in plans], finalize=[fin] * 6)
            for i in range(6):
                got[i].append((res[i].tolist(), g.stream(i).stats().tolist()))
    finally:
        g.close()
    for i, (x, ends, final) in enumerate(plans):
        s = Stream(gdec, genc)
        lone = []
        for k, e in enumerate(ends + [final]):
            t = s.push(x[:e], finalize=k == len(ends)).tolist()
            st = s.stats().tolist()
            lone.append((t, [st[c] for c in STAT_COLS]))
        s.close()
        assert lone == [(t, [st[c] for c in STAT_COLS]) for t, st in got[i]], (i, lone, got[i])


def test_stream_batch_rejects_member_push(models):
    from qwenasr_amd._lib import QasrError, lib
    from qwenasr_amd.model import StreamBatch
    gdec, genc, _, _ = models
    g = StreamBatch(gdec, genc, 2, 512, max_new_tokens=3)
    try:
        import ctypes as C
        x = np.zeros(32000, np.float32)
        n = C.c_int64()
        rc = lib().qasr_hip_stream_push(g.stream(0).s, x.ctypes.data_as(C.c_void_p), x.size, 0, None, 0, C.byref(n))
        assert rc != 0 and b"stream batch" in lib().qasr_hip_last_error()
    finally:
        g.close()


def test_stream_batch_mixed_finalize_idle_and_stop(models, orc):
    """One push where stream 0 finalizes, stream 1 gets no new audio, stream 2
    gets a chunk and stream 3 stops at once (its stop token is the token the
    model emits first): each stream's tokens and stats equal the oracle's
    stream run on its own pushes."""
    from qwenasr_amd.model import StreamBatch
    from qwenasr_amd.synth import audio
    gdec, genc, cdec, cenc = models
    xs = [audio(80000, 1300 + i) for i in range(4)]
    first = int(orc.transcribe_forced(cdec, cenc, xs[3][:32000], 1)["tokens"][0])
    cfg = dict(max_new_tokens=3, rollback=1)
    ends = [[32000, 72000], [64000, 64000], [32000, 64000], [32000, 64000]]
    fins = [[False, True], [False, False], [False, False], [False, False]]
    want = []
    for i, x in enumerate(xs):
        kw = dict(cfg, stop_tokens=(first, -1)) if i == 3 else cfg
        c = orc.OracleStream(cdec, cenc, **kw)
        want.append([(c.push(x[:e], finalize=f).tolist(), c.stats().tolist()) for e, f in zip(ends[i], fins[i])])
        c.close()
    # stream 3's stop token differs from the others': a batch holds one
    # configuration, so it runs in its own batch of one
    g = StreamBatch(gdec, genc, 3, 1024, **cfg)
    g3 = StreamBatch(gdec, genc, 1, 1024, **dict(cfg, stop_tokens=(first, -1)))
    try:
        for k in range(2):
            got = g.push([xs[i][:ends[i][k]] for i in range(3)], finalize=[fins[i][k] for i in range(3)])
            got3 = g3.push([xs[3][:ends[3][k]]], finalize=[fins[3][k]])
            for i, t in enumerate(got + got3):
                st = (g.stream(i) if i < 3 else g3.stream(0)).stats().tolist()
                assert t.tolist() == want[i][k][0], (k, i, t.tolist(), want[i][k][0])
                assert [st[c] for c in STAT_COLS] == [want[i][k][1][c] for c in STAT_COLS], (k, i, st, want[i][k][1])
        assert g.stream(0).audio_cursor == 72000 and g.stream(1).audio_cursor == 64000
    finally:
        g.close()
        g3.close()

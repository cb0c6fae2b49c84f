"""CPU pins of the oracle's streaming restatement (oracle_stream.c), the
checker of the GPU streaming driver (stream_push_audio, transcribe.rs:902-1304).

- stream_tail_repeat_blocks (transcribe.rs:38-56): hand-computed answers;
- one finalizing push of <= one chunk is the offline transcription
  (transcribe.rs:63-247) truncated to max_new_tokens: the same prompt rows
  (also with text-prompt and forced-language ids), the same greedy steps —
  pinned against the oracle's offline driver;
- the chunk schedule: nothing is emitted before unfixed_chunks, a chunk that
  reuses the previous partial encoding reuses the whole previous prefill,
  finalize commits every raw token;
- the stop token ends a chunk's decode and, once the stream has raw tokens,
  marks the speech end that commits the held-back tokens.
"""
import numpy as np
import pytest

from conftest import ROOT  # noqa: F401

DEC = dict(n_layers=2, hidden=1024, n_heads=16, n_kv_heads=8, head_dim=128, intermediate=3072,
           vocab=151936, eps=1e-6, theta=1e6)


def test_tail_repeat_blocks(orc):
    T = orc.tail_repeat_blocks
    assert T([], 6) == (1, 0) and T([7], 6) == (1, 0)
    assert T([1, 2, 3, 1, 2, 3, 1, 2, 3], 6) == (3, 3)
    assert T([5, 5, 5, 5, 5], 6) == (5, 1)                  # period 1 wins (first period reaching the max)
    assert T([9, 1, 2, 1, 2], 6) == (2, 2)
    assert T([1, 2, 1, 2, 3], 6) == (1, 0)                  # nothing repeats at the tail
    assert T([4, 1, 2, 3, 4, 5, 6, 7, 1, 2, 3, 4, 5, 6, 7], 6) == (1, 0)   # period 7 > max_period
    assert T([4, 1, 2, 3, 4, 5, 6, 7, 1, 2, 3, 4, 5, 6, 7], 0) == (2, 7)   # 0: up to n / 2
    assert T([3, 3, 1, 3, 3, 1, 3, 3, 1, 3, 3], 6) == (3, 3) # [3 3 1] x3 would need 12; [1 3 3] x3 at the tail


@pytest.fixture(scope="module")
def tiny(orc):
    from qwenasr_amd.synth import ENC_0_6B, SynthDecoder, SynthEncoder, audio
    wd = SynthDecoder(DEC, seed=1004)
    we = SynthEncoder(dict(ENC_0_6B, n_layers=2), seed=1004)
    dec = orc.OracleDecoder(wd, max_seq=1024)
    enc = orc.OracleEncoder(we)
    x = audio(int(10.5 * 16000), 1004)
    yield wd, we, dec, enc, x
    dec.close()
    enc.close()


def test_single_chunk_equals_offline(orc, tiny):
    _, _, dec, enc, x = tiny
    n = 24000                                         # 1.5 s: one chunk, finalized
    s = orc.OracleStream(dec, enc, max_new_tokens=8)
    got = s.push(x[:n], finalize=True)
    res = orc.transcribe_forced(dec, enc, x[:n], 8)
    assert list(got) == list(res["tokens"]), (got, res["tokens"])
    st = s.stats()
    assert st[0] == 1 and st[1] == 0 and st[3] == st[2]   # first chunk: nothing reused
    s.close()


@pytest.mark.parametrize("ids", [dict(prompt=[9707, 11]), dict(force=[11528, 6364, 151704]),
                                 dict(prompt=[9707], force=[11528, 6364, 151704])], ids=["prompt", "force", "both"])
def test_single_chunk_with_prompt_ids_equals_offline(orc, tiny, ids):
    """The stream's prompt rows with a text prompt and forced-language ids
    (transcribe.rs:1037-1089) are the offline layout's (transcribe.rs:97-169):
    one finalizing chunk commits the offline run's tokens."""
    _, _, dec, enc, x = tiny
    s = orc.OracleStream(dec, enc, max_new_tokens=3)      # 3 < the 4 repeats of the degeneracy rule
    s.set_prompt(**ids)
    got = s.push(x[:24000], finalize=True)
    res = orc.transcribe_forced(dec, enc, x[:24000], 3, **ids)
    assert list(got) == list(res["tokens"]), (got, res["tokens"])
    s.close()


@pytest.fixture(scope="module")
def asr_text_model(orc):
    from conftest import TINY_DEC, TINY_ENC, plant_asr_text
    from qwenasr_amd.synth import SynthDecoder, SynthEncoder, audio
    wd = plant_asr_text(SynthDecoder(TINY_DEC, seed=2401, std=0.05))
    we = SynthEncoder(TINY_ENC, seed=2402)
    dec, enc = orc.OracleDecoder(wd, max_seq=512), orc.OracleEncoder(we)
    yield dec, enc, audio(24000, 2403)
    dec.close()
    enc.close()


def test_text_region_rules_with_asr_text_in_raw(orc, asr_text_model):
    """A model that emits <asr_text> (A = 151704) at every step (the planted
    embedding of plant_asr_text; the first check confirms it): one finalizing
    chunk of 3 tokens commits raw[1:] = [A, A] without a forced language (the
    text region starts after the first <asr_text>, transcribe.rs:1257-1263)
    and all of raw = [A, A, A] with one (the region starts at 0); the offline
    rule counts none of them (every <asr_text> only sets past_asr_text,
    transcribe.rs:207-209)."""
    from conftest import ASR_TEXT
    from qwenasr_amd.model import text_tokens
    dec, enc, x = asr_text_model
    force = [11528, 6364, ASR_TEXT]
    for ids, want in ((dict(), [ASR_TEXT] * 2), (dict(force=force), [ASR_TEXT] * 3)):
        raw = orc.transcribe_forced(dec, enc, x, 3, **ids)["tokens"].tolist()
        assert raw == [ASR_TEXT] * 3, raw
        s = orc.OracleStream(dec, enc, max_new_tokens=3)
        s.set_prompt(**ids)
        got = s.push(x, finalize=True).tolist()
        s.close()
        assert got == want, (ids, got)
        assert text_tokens(np.array(raw, np.int32), text_open=bool(ids)).tolist() == []


def test_chunk_schedule(orc, tiny):
    """max_new_tokens 3 keeps the tail-repeat rule (>= 4 repeats) out of the
    way of a random-init model's repetitive tokens; rollback 1."""
    _, _, dec, enc, x = tiny
    s = orc.OracleStream(dec, enc, max_new_tokens=3, rollback=1)
    e0 = s.push(x[:32000])                            # chunk 0: partial encoded, nothing stable yet
    st0 = s.stats()
    e1 = s.push(x[:64000])                            # chunk 1: partial reused (age 2 s < 4 s)
    st1 = s.stats()
    assert len(e0) == 0 and len(e1) == 0              # chunk_idx < unfixed_chunks
    assert st1[1] == st0[2] and st1[3] == 0           # the whole previous prefill is reused
    e2 = s.push(x[:96000])                            # chunk 2: re-encoded; rollback holds 1 back
    st2 = s.stats()
    assert 0 < st2[1] < st2[2]                        # prefix rows reused, the new encoder rows prefilled
    assert len(e2) == max(0, st2[7] - 1)
    e3 = s.push(x[:100000], finalize=True)            # final: commit everything
    toks = s.tokens()
    assert list(toks) == list(e2) + list(e3)
    assert len(toks) == s.stats()[7]                  # no ASR_TEXT marker: every raw token is text
    s.close()


def test_degenerate_tokens_reset(orc, tiny):
    """Default settings on a random-init model: the repeated tail tokens trip
    the degeneracy rule (transcribe.rs:1204-1229) every chunk, which clears
    the raw tokens and the prefill reuse."""
    _, _, dec, enc, x = tiny
    s = orc.OracleStream(dec, enc)
    s.push(x[:32000])
    assert s.stats()[7] == 0
    s.push(x[:64000])
    st = s.stats()
    assert st[1] == 0 and st[3] == st[2]              # nothing reused after the reset
    s.close()


def test_window_cache_and_stop_token(orc, tiny):
    _, _, dec, enc, x = tiny
    s = orc.OracleStream(dec, enc, max_new_tokens=4)
    for end in range(32000, x.size + 1, 32000):
        s.push(x[:end])
    assert s.stats()[6] == 1                          # the 0-8 s window was encoded once
    s.close()
    # a stop token equal to the first decoded token: empty chunks -> speech end
    first = orc.transcribe_forced(dec, enc, x[:32000], 1)["tokens"][0]
    s = orc.OracleStream(dec, enc, max_new_tokens=4, stop_tokens=(int(first), -1))
    s.push(x[:32000])
    assert s.stats()[7] == 0                          # the first chunk stopped at once
    s.close()


def test_periodic_reanchor(orc, tiny):
    """Every 45 chunks the reference re-anchors whatever the tokens
    (transcribe.rs:1231-1252): raw becomes <asr_text> and the last
    min(24, committed) committed tokens, prefix reuse restarts.  48 chunks of
    0.5 s: after chunk index 45 the raw count is 1 + min(24, committed) (or 0
    with nothing committed) and the next chunk prefills every row."""
    from qwenasr_amd.synth import audio
    _, _, dec, enc, _ = tiny
    x = audio(24 * 16000, 1045)
    s = orc.OracleStream(dec, enc, max_new_tokens=3, rollback=1, chunk_sec=0.5)
    seen = False
    for end in range(8000, x.size + 1, 8000):
        s.push(x[:end])
        st = s.stats()
        if st[0] == 46:
            committed = len(s.tokens())
            assert st[7] == (1 + min(24, committed) if committed else 0), (st, committed)
            seen = True
        if st[0] == 47:
            assert st[1] == 0 and st[3] == st[2], st
    assert seen and s.stats()[0] == 48
    s.close()

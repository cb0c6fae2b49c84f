"""BASELINE config 2 at full size through the C ABI: random-init
Qwen3-ASR-0.6B (28-layer int8 decoder, 18-layer encoder), 30 s of synthetic
audio, mel -> encoder -> 404-row prefill -> 200 forced greedy steps
(transcribe.rs:63-247).

- the 200 token ids equal the committed oracle fixture
  (tests/golden/config2_tokens.json, written by make_config2_tokens.py);
- the random-init model settles on one token id, so the token check alone is
  weak: the whole KV cache after the run (every layer, all 604 positions) is
  compared with the oracle's, computed here on the host from the same seeded
  model and audio:
  * the 404 prefill rows of every layer within 1e-5 (f32-class MFMA GEMMs and
    attention against the oracle's f32 sgemm; measured 1e-6);
  * layer 0's 200 decode rows within 1e-5 (identical token embeddings through
    the exact int8 path);
  * deeper decode rows within 5e-2: every decode step re-quantizes its
    activations to int8, so an ulp-level difference can move an element
    across a rounding boundary.  The oracle against itself with its prompt
    rows perturbed by 1e-6 (relative) moves these rows by 0.7-2.1% at layers
    1-27 while its prefill rows move by 1e-6 and its 200 tokens do not change;
    a wrong row, position or layer gives errors of order 1.
"""
import json
import os

import numpy as np
import pytest

from conftest import ROOT

pytestmark = pytest.mark.gpu

# teacher-forced run: deeper-layer decode rows on the GPU's own state
DECODE_KV_BOUND = 5e-2


def rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / np.linalg.norm(b))


def test_config2_full_size(dev):
    from oracle import oracle as orc
    from qwenasr_amd.model import Decoder, Encoder, transcribe_forced
    from qwenasr_amd.synth import DEC_0_6B, ENC_0_6B, SynthDecoder, SynthEncoder, audio
    with open(os.path.join(ROOT, "tests", "golden", "config2_tokens.json")) as f:
        golden = json.load(f)
    wd = SynthDecoder(DEC_0_6B, seed=1002)
    we = SynthEncoder(ENC_0_6B, seed=1002)
    x = audio(480000, 1002)
    print("config 2 full size: GPU transcription", flush=True)
    dec = Decoder(dev, wd, max_seq=1024)
    enc = Encoder(dev, we)
    try:
        toks, _ = transcribe_forced(dec, enc, x, 200)
        assert [int(t) for t in toks] == golden["tokens"]
        k_g, v_g = dec.kv_download()
        n = dec.kv_len
    finally:
        dec.close()
        enc.close()
    assert n == golden["prompt_len"] - 1 + 200
    print("config 2 full size: oracle transcription on the host", flush=True)
    orc.set_threads(min(16, os.cpu_count() or 1))
    od, oe = orc.OracleDecoder(wd, max_seq=1024), orc.OracleEncoder(we)
    try:
        res = orc.transcribe_forced(od, oe, x, 200)
        assert [int(t) for t in res["tokens"]] == golden["tokens"]
        k_c, v_c = od.kv()
    finally:
        od.close()
        oe.close()
    P = golden["prompt_len"] - 1                       # prefill rows; decode rows [P, n)
    pre = [max(rel(k_g[l, :, :P], k_c[l, :, :P]), rel(v_g[l, :, :P], v_c[l, :, :P])) for l in range(28)]
    dec = [max(rel(k_g[l, :, P:n], k_c[l, :, P:n]), rel(v_g[l, :, P:n], v_c[l, :, P:n])) for l in range(28)]
    print("per-layer KV relative error, prefill rows:", [f"{e:.2e}" for e in pre], flush=True)
    print("per-layer KV relative error, decode rows:", [f"{e:.2e}" for e in dec], flush=True)
    assert max(pre) < 1e-5, pre
    assert dec[0] < 1e-5, dec[0]
    assert max(dec) < 5e-2, dec


def test_config2_teacher_forced(dev):
    """The same full-size model, prompt and first step, then 240 teacher-forced
    steps whose input ids are seeded uniform draws over the vocabulary
    (tests/golden/config2_forced.json, written by make_config2_tokens.py), so
    every step sees a different input.

    This random-init model amplifies ulp-sized differences within one step:
    the oracle itself, run from the same state with its input embedding
    perturbed by 1e-6 relative, moves the deeper layers' new K/V rows by about
    2%, the winning logit by up to 1.3% and flips the argmax at several steps
    whose top-2 gap exceeds 3e-3 (the fixture records that run per step).  A
    different summation order (the GPU's attention splits, its f32-class
    prefill) is a perturbation of that size, so the GPU is held to the
    oracle's own sensitivity, not to bit equality:

    State-synchronised (each step checked on its own): after the GPU's first
    step its KV cache is overwritten with the oracle's (prompt rows and first
    step); after every forced step the rows the GPU wrote are compared with
    the oracle's and then replaced by them, so each GPU step starts from
    exactly the oracle's state.  At least 190 steps have a relative top-2 gap
    above 3e-3; there the GPU's argmax differs from the oracle's at no more
    than twice as many steps as the perturbed oracle's does (plus 2); the
    winning logit's and the new rows' deviations (layers >= 1) stay within
    twice the perturbed oracle's largest and three times its median; layer
    0's rows within 1e-5 (exact int8 path, K after a differently ordered
    q/k norm + RoPE).

    Unsynchronised (the GPU on its own state): the same 240 steps from the
    GPU's own prompt rows; the whole KV cache against the oracle's run:
    prefill rows of every layer within 1e-5, layer 0's decode rows within
    1e-5, deeper decode rows within DECODE_KV_BOUND (the oracle against
    itself with its prompt rows perturbed by 1e-6 drifts 2% over the run,
    test_golden.py::test_config2_forced_fixture_reproduces_and_is_chaotic).
    """
    import sys

    from qwenasr_amd.model import Decoder, Encoder, transcribe_forced
    from qwenasr_amd.synth import DEC_0_6B, ENC_0_6B, SynthDecoder, SynthEncoder, audio
    sys.path.insert(0, os.path.join(ROOT, "tests", "golden"))
    import make_config2_tokens as mk
    with open(os.path.join(ROOT, "tests", "golden", "config2_forced.json")) as f:
        golden = json.load(f)
    ids = golden["forced_ids"]
    want = golden["tokens"]
    best = np.asarray(golden["best"], np.float64)
    gap = (best - np.asarray(golden["second"], np.float64)) / np.abs(best)
    clear = [s for s in range(len(ids)) if gap[s] > 3e-3]
    assert len(clear) >= 190, len(clear)
    noisy_flips = sum(golden["noisy_tokens"][s] != want[s] for s in clear)
    noisy_logit = np.abs(np.asarray(golden["noisy_best"], np.float64) - best) / np.abs(best)
    noisy_rows = np.asarray(golden["noisy_row_rel"], np.float64)
    print("config 2 teacher forced: oracle on the host", flush=True)
    first, toks_c, _, _, (k_c, v_c), n_c = mk.oracle_forced_run(np.asarray(ids, np.int32))
    assert first == golden["first_token"] and toks_c == want
    P1 = n_c - len(ids)                                # prompt rows + the first step's row
    wd = SynthDecoder(DEC_0_6B, seed=1002)
    we = SynthEncoder(ENC_0_6B, seed=1002)
    x = audio(480000, 1002)
    dec = Decoder(dev, wd, max_seq=1024)
    enc = Encoder(dev, we)
    try:
        print(f"config 2 teacher forced: GPU, {len(ids)} state-synchronised steps", flush=True)
        toks, _ = transcribe_forced(dec, enc, x, 1)
        assert int(toks[0]) == golden["first_token"] and dec.kv_len == P1
        dec.kv_rows_upload(0, k_c[:, :, :P1], v_c[:, :, :P1])
        got, vals, row_err, row0_err = [], [], [], []
        for s, t in enumerate(ids):
            got.append(dec.forward(token=int(t)))
            vals.append(dec.last_logit())
            kg, vg = dec.kv_rows_download(P1 + s, 1)
            kc, vc = k_c[:, :, P1 + s:P1 + s + 1], v_c[:, :, P1 + s:P1 + s + 1]
            row_err.append(max(rel(kg[1:], kc[1:]), rel(vg[1:], vc[1:])))
            row0_err.append(max(rel(kg[0], kc[0]), rel(vg[0], vc[0])))
            dec.kv_rows_upload(P1 + s, kc, vc)
        flips = [s for s in clear if got[s] != want[s]]
        vrel = np.abs(np.asarray(vals, np.float64) - best) / np.abs(best)
        row_err = np.asarray(row_err)
        print(f"synchronised: argmax differs at {len(flips)} of {len(clear)} clear steps {flips} (perturbed oracle: "
              f"{noisy_flips}); winning logit rel max {vrel.max():.3g} median {np.median(vrel):.3g} (perturbed "
              f"oracle {noisy_logit.max():.3g} / {np.median(noisy_logit):.3g}); new rows, layers >= 1, rel max "
              f"{row_err.max():.3g} median {np.median(row_err):.3g} (perturbed oracle {noisy_rows.max():.3g} / "
              f"{np.median(noisy_rows):.3g}); layer 0 {max(row0_err):.3g}", flush=True)
        assert len(flips) <= 2 * noisy_flips + 2, flips
        assert vrel.max() <= 2 * noisy_logit.max() and np.median(vrel) <= 3 * np.median(noisy_logit)
        assert row_err.max() <= 2 * noisy_rows.max() and np.median(row_err) <= 3 * np.median(noisy_rows)
        assert max(row0_err) < 1e-5

        print("config 2 teacher forced: GPU, unsynchronised", flush=True)
        dec.kv_len = 0
        toks, _ = transcribe_forced(dec, enc, x, 1)
        own = [dec.forward(token=int(t)) for t in ids]
        k_g, v_g = dec.kv_download()
        n = dec.kv_len
    finally:
        dec.close()
        enc.close()
    assert n == n_c
    P = P1 - 1                                         # prefill rows; decode rows [P, n)
    pre = [max(rel(k_g[l, :, :P], k_c[l, :, :P]), rel(v_g[l, :, :P], v_c[l, :, :P])) for l in range(28)]
    dec_e = [max(rel(k_g[l, :, P:n], k_c[l, :, P:n]), rel(v_g[l, :, P:n], v_c[l, :, P:n])) for l in range(28)]
    same = sum(own[s] == want[s] for s in clear)
    print(f"unsynchronised: {same} of {len(clear)} clear steps equal", flush=True)
    print("per-layer KV relative error, prefill rows:", [f"{e:.2e}" for e in pre], flush=True)
    print("per-layer KV relative error, decode rows:", [f"{e:.2e}" for e in dec_e], flush=True)
    assert max(pre) < 1e-5, pre
    assert dec_e[0] < 1e-5, dec_e[0]
    assert max(dec_e) < DECODE_KV_BOUND, dec_e

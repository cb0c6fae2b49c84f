"""Writes the two config-2 fixtures of BASELINE config 2 (seed 1002:
random-init Qwen3-ASR-0.6B, 30 s of synthetic audio; transcribe.rs:63-247):

* config2_tokens.json: the oracle's token ids and top-2 logit margins of 200
  forced greedy steps.  The random-init model settles on one token id, so
  these ids alone pin little;
* config2_forced.json: after the same prompt prefill and first step, 240
  teacher-forced steps whose input ids are seeded uniform draws over the
  vocabulary (seed 1012): the forced ids, the oracle's argmax at each step and
  its best and second-best logits.  Every step sees a different input, so
  each argmax is an independent check of the whole decode step.  Each step
  is also run once more from the same state with its input embedding
  perturbed by 1e-6 relative: that run's argmax, best logit and deeper-layer
  K/V row deviation are the oracle's own sensitivity within one step, the
  scale the GPU's per-step differences are judged against.

Run from the repository root after building the oracle:
    python tests/golden/make_config2_tokens.py
The files are the fixtures the full-size GPU tests (test_gpu_config2.py)
assert against; the CPU suite checks their shape and re-derives them from
the oracle (test_golden.py).
"""
import json
import os
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

SEED = 1002
AUDIO_S = 30.0
STEPS = 200
FORCED_SEED = 1012
FORCED_STEPS = 240
STEP_NOISE = 1e-6
VOCAB = 151936


def oracle_run(n_steps=STEPS, threads=None):
    from oracle import oracle as orc
    from qwenasr_amd.synth import DEC_0_6B, ENC_0_6B, SynthDecoder, SynthEncoder, audio
    orc.set_threads(threads or min(16, os.cpu_count() or 1))
    wd = SynthDecoder(DEC_0_6B, seed=SEED)
    we = SynthEncoder(ENC_0_6B, seed=SEED)
    x = audio(int(round(AUDIO_S * 16000)), SEED)
    od, oe = orc.OracleDecoder(wd, max_seq=1024), orc.OracleEncoder(we)
    try:
        return orc.transcribe_forced(od, oe, x, n_steps)
    finally:
        od.close()
        oe.close()


def forced_ids(n=FORCED_STEPS):
    import numpy as np
    return np.random.default_rng(FORCED_SEED).integers(0, VOCAB, n).astype(np.int32)


def oracle_forced_run(ids=None, threads=None, perturb=0.0, step_noise=0.0):
    """The prompt prefill and first step of the forced run, then one oracle
    forward per forced id; returns (first token, argmax ids, best logits,
    second-best logits, the oracle decoder's KV after the run, its length).
    perturb > 0 scales every KV element written by the prompt and first step
    by (1 + perturb * N(0, 1)) (seeded) before the forced steps: the oracle's
    own sensitivity to ulp-sized differences in its state.  step_noise > 0
    also runs every forced step a second time first, from the same state with
    its input embedding scaled by (1 + step_noise * N(0, 1)), and returns that
    step's argmax, best logit and deeper-layer (>= 1) row deviation from the
    exact step's rows as a seventh item: the oracle's sensitivity within one
    step."""
    from oracle import oracle as orc
    from qwenasr_amd.synth import DEC_0_6B, ENC_0_6B, SynthDecoder, SynthEncoder, audio
    ids = forced_ids() if ids is None else ids
    orc.set_threads(threads or min(16, os.cpu_count() or 1))
    wd = SynthDecoder(DEC_0_6B, seed=SEED)
    we = SynthEncoder(ENC_0_6B, seed=SEED)
    x = audio(int(round(AUDIO_S * 16000)), SEED)
    od, oe = orc.OracleDecoder(wd, max_seq=1024), orc.OracleEncoder(we)
    try:
        first = int(orc.transcribe_forced(od, oe, x, 1)["tokens"][0])
        if perturb > 0:
            import numpy as np
            k, v = od.kv()
            n = od.kv_len
            r = np.random.default_rng(FORCED_SEED + 1)
            for a in (k, v):
                a[:, :, :n] *= (1.0 + perturb * r.standard_normal(a[:, :, :n].shape)).astype(np.float32)
            od.set_kv(k, v)
        import numpy as np
        toks, best, second = [], [], []
        noisy = dict(tokens=[], best=[], row_rel=[])
        rs = np.random.default_rng(FORCED_SEED + 2)
        for t in ids:
            e = od.embed(int(t))
            p = od.kv_len
            if step_noise > 0:
                ep = (e * (1.0 + step_noise * rs.standard_normal(e.shape))).astype(np.float32)
                tn, bn, _ = od.forward_logits(ep)
                kn, vn = od.kv_rows(p, 1)
                od.kv_len = p
            a, b, c = od.forward_logits(e)
            toks.append(a)
            best.append(b)
            second.append(c)
            if step_noise > 0:
                k1, v1 = od.kv_rows(p, 1)
                noisy["tokens"].append(tn)
                noisy["best"].append(bn)
                noisy["row_rel"].append(max(float(np.linalg.norm(x[1:] - y[1:]) / np.linalg.norm(y[1:]))
                                            for x, y in ((kn, k1), (vn, v1))))
        k, v = od.kv()
        if step_noise > 0:
            return first, toks, best, second, (k, v), od.kv_len, noisy
        return first, toks, best, second, (k, v), od.kv_len
    finally:
        od.close()
        oe.close()


def write_forced():
    t0 = time.time()
    ids = forced_ids()
    first, toks, best, second, _, _, noisy = oracle_forced_run(ids, step_noise=STEP_NOISE)
    out = {
        "config": "BASELINE config 2 (as config2_tokens.json): the prompt prefill and the first forced step, then "
                  f"{len(ids)} teacher-forced steps whose input ids are uniform draws over the vocabulary (seed "
                  f"{FORCED_SEED})",
        "source": "oracle/oracle.c or_transcribe_prompt (1 step), then or_decoder_forward per forced id "
                  "(decoder.rs:550-645)",
        "first_token": first,
        "forced_ids": [int(t) for t in ids],
        "tokens": [int(t) for t in toks],
        "best": [float(b) for b in best],
        "second": [float(c) for c in second],
        "step_noise": STEP_NOISE,
        "noisy_tokens": [int(t) for t in noisy["tokens"]],
        "noisy_best": [float(b) for b in noisy["best"]],
        "noisy_row_rel": [float(r) for r in noisy["row_rel"]],
    }
    with open(os.path.join(HERE, "config2_forced.json"), "w") as f:
        json.dump(out, f, indent=1)
        f.write("\n")
    rel = [(b - c) / abs(b) for b, c in zip(best, second)]
    print(f"wrote config2_forced.json ({len(ids)} steps, {len(set(toks))} distinct argmax ids, "
          f"{sum(r > 3e-3 for r in rel)} steps with a relative top-2 gap above 3e-3) in {time.time() - t0:.1f}s")


def main():
    write_forced()
    t0 = time.time()
    res = oracle_run()
    out = {
        "config": "BASELINE config 2: Qwen3-ASR-0.6B random-init (seed 1002, N(0,0.02) bf16 matrices, unit gains, "
                  "zero biases), 30 s 16 kHz audio (seed 1002: white noise -30 dBFS + 440/1000/3150 Hz sines), "
                  "int8 round-mode packing, 200 forced greedy steps",
        "source": "oracle/oracle.c or_transcribe_forced (the C restatement of transcribe.rs:63-247)",
        "prompt_len": res["prompt_len"],
        "tokens": [int(t) for t in res["tokens"]],
        "margins": [float(m) for m in res["margins"]],
    }
    with open(os.path.join(HERE, "config2_tokens.json"), "w") as f:
        json.dump(out, f, indent=1)
        f.write("\n")
    print(f"wrote config2_tokens.json ({len(out['tokens'])} tokens, min margin {min(out['margins']):.3g}) "
          f"in {time.time() - t0:.1f}s")


if __name__ == "__main__":
    main()

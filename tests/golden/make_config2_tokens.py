"""Writes config2_tokens.json: the oracle's token ids and top-2 logit margins
for BASELINE config 2 (seed 1002: random-init Qwen3-ASR-0.6B, 30 s of
synthetic audio, 200 forced greedy steps; transcribe.rs:63-247).

Run from the repository root after building the oracle:
    python tests/golden/make_config2_tokens.py
The file is the fixture the full-size GPU test (test_gpu_config2.py) asserts
against; the CPU suite re-derives its first steps from the oracle
(test_golden.py).
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


def main():
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

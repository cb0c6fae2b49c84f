"""The committed config-2 fixture (tests/golden/config2_tokens.json) against
the oracle that wrote it: the full BASELINE config-2 run on the host
(random-init Qwen3-ASR-0.6B, 30 s of audio, 200 forced steps) reproduces every
token id and top-2 margin.  The GPU test test_gpu_config2.py asserts against
the same file."""
import json
import os
import sys

import pytest

from conftest import ROOT

GOLDEN = os.path.join(ROOT, "tests", "golden")


def test_config2_fixture_shape():
    with open(os.path.join(GOLDEN, "config2_tokens.json")) as f:
        g = json.load(f)
    assert len(g["tokens"]) == len(g["margins"]) == 200
    assert g["prompt_len"] == 3 + 6 + 390 + 6                 # transcribe.rs:13-15 around 390 audio rows
    assert all(0 <= t < 151936 for t in g["tokens"])
    assert all(m >= 0 for m in g["margins"])


@pytest.mark.slow
def test_config2_fixture_reproduces(orc):
    sys.path.insert(0, GOLDEN)
    import make_config2_tokens as mk
    with open(os.path.join(GOLDEN, "config2_tokens.json")) as f:
        g = json.load(f)
    res = mk.oracle_run()
    assert [int(t) for t in res["tokens"]] == g["tokens"]
    assert res["prompt_len"] == g["prompt_len"]
    assert [float(m) for m in res["margins"]] == g["margins"]

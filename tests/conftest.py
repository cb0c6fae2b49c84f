import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libqasr_hip.so)")
    config.addinivalue_line("markers", "slow: long-running CPU case")


@pytest.fixture(scope="session")
def orc():
    from oracle import oracle
    oracle.lib()
    oracle.set_threads(min(8, os.cpu_count() or 8))
    return oracle


@pytest.fixture(scope="session")
def dev():
    """The GPU handle; GPU tests fail (not skip) when the HIP library or device is missing."""
    from qwenasr_amd import Device, device_count
    assert device_count() >= 1, "no HIP device visible"
    d = Device(0)
    yield d
    d.close()


def rng(seed):
    return np.random.default_rng(seed)


def bf16(a):
    from qwenasr_amd.synth import f32_to_bf16
    return f32_to_bf16(np.asarray(a, np.float32))


def bf16f(a):
    return (np.asarray(a, np.uint16).astype(np.uint32) << 16).view(np.float32)


def oracle_head_values(orc, hid, q_rows, s_rows):
    """The oracle LM head's values of the given packed rows for the final
    normed hidden state `hid`, as or_argmax_int8 forms them (oracle.c, after
    mod.rs:1832-1893): one activation quantization, the exact int32 dot, then
    (float)acc * xs * ws[row] in float32, left to right, no contraction."""
    xq, xs = orc.quantize_act(hid)
    acc = np.asarray(q_rows, np.int64).reshape(-1, xq.shape[0]) @ xq.astype(np.int64)
    return (acc.astype(np.float32) * np.float32(xs)).astype(np.float32) * np.asarray(s_rows, np.float32)


def gpu_token_gap(orc, od, hid, best, token):
    """Relative distance (best - v) / |best| of the GPU's token from the
    oracle's best logit at one step, v being the oracle's own value of that
    token's head row on the oracle's state (0 exactly when the token is the
    oracle's argmax)."""
    q, s = od.packed(-1, 0, rows=[int(token)])
    v = float(oracle_head_values(orc, hid, q, s)[0])
    return (best - v) / max(abs(best), 1e-30)


ASR_TEXT = 151704
# a 2-layer decoder small enough for the oracle (the GPU kernels' head_dim
# 128, the full vocabulary) and a 2-layer encoder of the 0.6B width
TINY_DEC = dict(n_layers=2, hidden=128, n_heads=16, n_kv_heads=8, head_dim=128, intermediate=256, vocab=151936,
                eps=1e-6, theta=1e6)
TINY_ENC = dict(d_model=896, n_layers=2, n_heads=14, head_dim=64, ffn_dim=3584, output_dim=128, chunk_size=100,
                n_window_infer=800, conv_hidden=480)


def plant_asr_text(w, base=10.0, top=20.0):
    """Makes a SynthDecoder emit <asr_text> (151704) at every step: element 0
    of every embedding row is `base` and of row 151704 `top`.  The residual of
    every decode position (its input is a token embedding) is then dominated by
    dimension 0, the quantized final activation is (127, ~0, ...), every row of
    the tied int8 head has its absmax in element 0, and the head's logits
    follow that element: 151704's is twice any other's."""
    w.embed[:, 0] = bf16([base])[0]
    w.embed[ASR_TEXT, 0] = bf16([top])[0]
    return w

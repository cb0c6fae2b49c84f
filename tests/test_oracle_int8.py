"""Pins the oracle's int8 functions (CPU only).

Each check is independent of the oracle's code: closed-form known answers,
brute force in numpy int64 / float32 / float64, and special cases, chosen so a
plausible slip (round vs trunc, half-to-even vs half-away, a fused epilogue, a
wrong tie rule) fails.  References: kernels/mod.rs:1795-1893, neon.rs:637-849.
"""
import numpy as np
import pytest

from conftest import bf16, bf16f, rng


def round_half_away(v):
    v = np.asarray(v, np.float64)
    return np.sign(v) * np.floor(np.abs(v) + 0.5)


def np_pack(w_bf16, mode):
    """numpy restatement: per-row absmax, IEEE float32 scale/inv, round or trunc."""
    w = bf16f(w_bf16)
    m = np.abs(w).max(axis=1).astype(np.float32)
    scale = np.where(m > 0, m / np.float32(127.0), np.float32(1.0)).astype(np.float32)
    inv = (np.float32(127.0) / np.maximum(m, np.float32(1e-10))).astype(np.float32)
    v = (w * inv[:, None]).astype(np.float32)
    k = w.shape[1]
    if mode == 0:
        q = np.clip(round_half_away(v), -127, 127)
    else:
        body = k - k % 8
        q = np.empty_like(v, dtype=np.float64)
        q[:, :body] = np.clip(np.trunc(v[:, :body]), -128, 127)
        q[:, body:] = np.clip(round_half_away(v[:, body:]), -127, 127)
    return q.astype(np.int8), scale


def test_pack_zero_row(orc):
    w = np.zeros((3, 64), np.uint16)
    for mode in (0, 1):
        q, s = orc.quantize_bf16_rows(w, mode)
        assert (q == 0).all() and (s == 1.0).all()


def test_pack_halfway_kat(orc):
    # max 127.0 -> inv = 127/127 = 1.0 exactly; 2.5 -> 3 (round half away) vs 2 (trunc);
    # 0.5 -> 1 vs 0 (round-half-even would give 2 and 0: both differ from the reference)
    vals = np.zeros((1, 19), np.float32)
    vals[0, :6] = [127.0, 2.5, -2.5, 0.5, -0.5, 1.5]
    vals[0, 16:19] = [2.5, -0.5, 3.5]               # k >= 16: NEON scalar tail rounds
    w = bf16(vals)
    assert (bf16f(w) == vals).all()
    q, s = orc.quantize_bf16_rows(w, 0)
    assert s[0] == np.float32(1.0)
    assert list(q[0, :6]) == [127, 3, -3, 1, -1, 2]
    assert list(q[0, 16:19]) == [3, -1, 4]
    q, s = orc.quantize_bf16_rows(w, 1)
    assert list(q[0, :6]) == [127, 2, -2, 0, 0, 1]
    assert list(q[0, 16:19]) == [3, -1, 4]


@pytest.mark.parametrize("mode", [0, 1])
@pytest.mark.parametrize("k", [64, 1024, 1000, 77])
def test_pack_bruteforce(orc, mode, k):
    w = bf16(rng(k + mode).normal(0, 0.02, (37, k)))
    q, s = orc.quantize_bf16_rows(w, mode)
    qr, sr = np_pack(w, mode)
    assert (s == sr).all()
    assert (q == qr).all()
    # the row maximum maps to +-127 when rounding; truncation of m * (127 / m),
    # which can land just below 127, may give 126 (neon.rs:677-681)
    wf = bf16f(w)
    am = np.abs(wf).argmax(axis=1)
    top = np.abs(q[np.arange(37), am].astype(int))
    if mode == 0 or k < 8:
        assert (top == 127).all()
    else:
        assert set(top.tolist()) <= {126, 127}


def test_pack_modes_disagree(orc):
    """The two roundings disagree by one LSB on about half of the elements."""
    w = bf16(rng(5).normal(0, 0.02, (64, 1024)))
    q0, _ = orc.quantize_bf16_rows(w, 0)
    q1, _ = orc.quantize_bf16_rows(w, 1)
    d = np.abs(q0.astype(int) - q1.astype(int))
    assert d.max() == 1 and 0.3 < d.mean() < 0.7


def test_quantize_act(orc):
    x = rng(1).normal(0, 1, 3072).astype(np.float32)
    q, s = orc.quantize_act(x)
    m = np.abs(x).max()
    assert s == np.float32(m) / np.float32(127)
    inv = np.float32(127) / np.float32(m)
    assert (q == np.clip(round_half_away((x * inv).astype(np.float32)), -127, 127)).all()
    q0, s0 = orc.quantize_act(np.zeros(64, np.float32))
    assert s0 == 1.0 and (q0 == 0).all()


def np_matvec(xq, xs, w, ws, bias=None):
    k = w.shape[1]
    k16 = k - k % 16
    acc = (w[:, :k16].astype(np.int64) @ xq[:k16].astype(np.int64))
    assert np.abs(acc).max() < 2 ** 31
    y = (acc.astype(np.float32) * np.float32(xs)).astype(np.float32) * ws
    y = y.astype(np.float32)
    for i in range(k16, k):    # scalar tail (neon.rs:754-760), float adds in order
        y = (y + ((np.float32(xq[i]) * w[:, i].astype(np.float32)) * np.float32(xs)) * ws).astype(np.float32)
    if bias is not None:
        y = (y + bias).astype(np.float32)
    return y


@pytest.mark.parametrize("vnni", [0, 1])
@pytest.mark.parametrize("k", [1024, 2048, 3072, 6144, 80])
def test_matvec_bruteforce(orc, k, vnni):
    """both SIMD int8 dots (AVX2 maddubs, AVX-512 VNNI where the host has it)
    give the exact integer sums, extreme values included"""
    orc.lib().or_set_int8_dot(vnni)
    r = rng(k)
    w = r.integers(-127, 128, (96, k), dtype=np.int8)
    ws = r.uniform(1e-4, 2e-3, 96).astype(np.float32)
    x = r.normal(0, 1, k).astype(np.float32)
    xq, xs = orc.quantize_act(x)
    b = r.normal(0, 1, 96).astype(np.float32)
    assert (orc.matvec_w8a8(xq, xs, w, ws) == np_matvec(xq, xs, w, ws)).all()
    assert (orc.matvec_w8a8(xq, xs, w, ws, b) == np_matvec(xq, xs, w, ws, b)).all()
    assert (orc.linear_int8_addto(b, x, w, ws) == np_matvec(xq, xs, w, ws, b)).all()
    ext = np.full((2, k), -127, np.int8)
    ext[1] = 127
    xe = np.where(np.arange(k) % 2, np.int8(-127), np.int8(127)).astype(np.int8)
    assert (orc.matvec_w8a8(xe, 1.0, ext, np.ones(2, np.float32)) ==
            np_matvec(xe, 1.0, ext, np.ones(2, np.float32))).all()
    orc.lib().or_set_int8_dot(1)


def test_matvec_epilogue_not_fused(orc):
    """((float)acc * xs) * ws rounds twice; an FMA-contracted epilogue would not."""
    r = rng(11)
    w = r.integers(-127, 128, (4096, 1024), dtype=np.int8)
    ws = r.uniform(1e-4, 2e-3, 4096).astype(np.float32)
    x = r.normal(0, 1, 1024).astype(np.float32)
    b = r.normal(0, 1, 4096).astype(np.float32)
    xq, xs = orc.quantize_act(x)
    y = orc.matvec_w8a8(xq, xs, w, ws, b)
    acc = w.astype(np.int64) @ xq.astype(np.int64)
    t = (acc.astype(np.float32) * np.float32(xs)).astype(np.float32)
    fused = (t.astype(np.float64) * ws.astype(np.float64) + b.astype(np.float64)).astype(np.float32)
    unfused = ((t * ws).astype(np.float32) + b).astype(np.float32)
    assert (y == unfused).all()
    assert (fused != unfused).any()


def test_qkv_swiglu(orc):
    r = rng(3)
    x = r.normal(0, 1, 1024).astype(np.float32)
    wq, wk, wv = (r.integers(-127, 128, (n, 1024), dtype=np.int8) for n in (256, 128, 128))
    sq, sk, sv = (r.uniform(1e-4, 2e-3, n).astype(np.float32) for n in (256, 128, 128))
    q, k, v = orc.linear_int8_qkv(x, wq, sq, wk, sk, wv, sv)
    xq, xs = orc.quantize_act(x)
    assert (q == np_matvec(xq, xs, wq, sq)).all()
    assert (k == np_matvec(xq, xs, wk, sk)).all()
    assert (v == np_matvec(xq, xs, wv, sv)).all()
    wgu = r.integers(-127, 128, (512, 1024), dtype=np.int8)
    sgu = r.uniform(1e-4, 2e-3, 512).astype(np.float32)
    ffn = orc.linear_int8_swiglu(x, wgu, sgu)
    gu = np_matvec(xq, xs, wgu, sgu).astype(np.float64)
    g, u = gu[0::2], gu[1::2]
    ref = g / (1 + np.exp(-g)) * u
    np.testing.assert_allclose(ffn, ref, rtol=2e-6, atol=1e-9)


def test_argmax_bruteforce_and_ties(orc):
    r = rng(7)
    n, k = 5000, 1024
    w = r.integers(-127, 128, (n, k), dtype=np.int8)
    ws = r.uniform(1e-4, 2e-3, n).astype(np.float32)
    x = r.normal(0, 1, k).astype(np.float32)
    xq, xs = orc.quantize_act(x)
    vals = np_matvec(xq, xs, w, ws)
    i, bv, sv = orc.argmax_int8(x, w, ws)
    assert i == int(np.argmax(vals)) and bv == vals.max()
    srt = np.sort(vals)
    assert sv == srt[-2]
    # duplicate the winner at a lower index in another thread range and a higher one
    best = int(np.argmax(vals))
    for dup in (0, n // 16 - 1, n // 16, n - 1):
        w2, ws2 = w.copy(), ws.copy()
        w2[dup], ws2[dup] = w[best], ws[best]
        i2, bv2, sv2 = orc.argmax_int8(x, w2, ws2)
        assert i2 == min(dup, best) and sv2 == bv2
    # all-negative logits: every row anti-aligned with the quantized activation
    wn = (-np.sign(xq)[None, :] * np.abs(w)).astype(np.int8)
    vn = np_matvec(xq, xs, wn, ws)
    assert (vn < 0).all()
    i3, bv3, _ = orc.argmax_int8(x, wn, ws)
    assert i3 == int(np.argmax(vn)) and bv3 == vn.max()


def test_head_values_match_the_argmax(orc):
    """conftest.oracle_head_values, which the GPU decode tests use for the
    oracle's value of the GPU's chosen token, equals or_argmax_int8's best and
    second-best values bit for bit, one row or all at once; associating the
    two scales the other way gives different bits."""
    from conftest import oracle_head_values
    r = rng(71)
    n, k = 5000, 1024
    w = r.integers(-127, 128, (n, k), dtype=np.int8)
    ws = r.uniform(1e-4, 2e-3, n).astype(np.float32)
    x = r.normal(0, 1, k).astype(np.float32)
    i, bv, sv = orc.argmax_int8(x, w, ws)
    v = oracle_head_values(orc, x, w, ws)
    assert v.shape == (n,) and v[i] == bv and v.max() == bv and np.sort(v)[-2] == sv
    assert oracle_head_values(orc, x, w[i:i + 1], ws[i:i + 1])[0] == bv
    xq, xs = orc.quantize_act(x)
    acc = w.astype(np.int64) @ xq.astype(np.int64)
    other = acc.astype(np.float32) * (np.float32(xs) * ws).astype(np.float32)
    assert (other != v).any()

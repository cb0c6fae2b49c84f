"""Pins of the oracle's floating-point restatements against float64 textbook
forms (numpy), independent library routines (numpy.fft, scipy) and closed
forms.  The reference's own tests hold no golden vectors for these functions
(its kernels.rs tests are invariants only), so each check is chosen so that a
plausible slip — a dropped term, a wrong sign, a transposed operand, a wrong
head / window / frame index — fails it.

Tolerances: f32 restatements of f64 formulas within 1e-5 relative (a few ulp
of accumulated f32 rounding), the degree-5 fast_exp polynomial within 4e-6 + 1e-7|x|
relative, the mel front end within 1e-4 absolute in its normalised log10
domain.
"""
import math

import numpy as np
import pytest

from conftest import rng


def rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))


# ---- reductions -------------------------------------------------------------
def test_hsum8_and_dot(orc):
    L = orc.lib()
    import ctypes as C
    v = np.array([1, 2, 4, 8, 16, 32, 64, 128], np.float32)
    assert L.or_hsum8(v.ctypes.data_as(C.c_void_p)) == 255.0
    # a tree that adds 1e8 and -1e8 first keeps the small terms; a left fold loses them
    v = np.array([1e8, 1, 1, 1, -1e8, 1, 1, 1], np.float32)
    assert L.or_hsum8(v.ctypes.data_as(C.c_void_p)) == 6.0
    r = rng(1)
    for n in (1, 7, 32, 128, 1000):
        a = r.normal(0, 1, n).astype(np.float32)
        b = r.normal(0, 1, n).astype(np.float32)
        got = L.or_dot_f32(a.ctypes.data_as(C.c_void_p), b.ctypes.data_as(C.c_void_p), n)
        exact = float(a.astype(np.float64) @ b.astype(np.float64))
        assert abs(got - exact) <= 1e-5 * (np.abs(a.astype(np.float64) * b).sum() + 1e-30), n


# ---- normalisations ---------------------------------------------------------
@pytest.mark.parametrize("hidden", [1024, 2048, 16, 40, 1000])
def test_rms_norm(orc, hidden):
    r = rng(hidden)
    x = (r.normal(0, 1, (3, hidden)) * np.array([[1e-3], [1.0], [50.0]])).astype(np.float32)
    w = r.uniform(0.5, 1.5, hidden).astype(np.float32)
    got = orc.rms_norm(x, w, 1e-6)
    x64 = x.astype(np.float64)
    ref = x64 / np.sqrt((x64 ** 2).mean(axis=1, keepdims=True) + 1e-6) * w
    assert rel(got, ref) < 1e-6
    np.testing.assert_allclose(got, ref, rtol=2e-6, atol=1e-7)


def test_rms_norm_eps_dominates(orc):
    x = np.full((1, 64), 1e-5, np.float32)
    w = np.ones(64, np.float32)
    got = orc.rms_norm(x, w, 1e-6)
    np.testing.assert_allclose(got, 1e-5 / math.sqrt(1e-10 + 1e-6), rtol=1e-6)


def test_rms_norm_per_head(orc):
    r = rng(3)
    seq, heads, hd = 3, 16, 128
    x = (r.normal(0, 1, (seq, heads, hd)) * r.uniform(0.1, 10, (seq, heads, 1))).astype(np.float32)
    w = r.uniform(0.5, 1.5, hd).astype(np.float32)
    got = orc.rms_norm_per_head(x.copy(), w, heads, 1e-6).reshape(seq, heads, hd)
    x64 = x.astype(np.float64)
    ref = x64 / np.sqrt((x64 ** 2).mean(axis=2, keepdims=True) + 1e-6) * w
    np.testing.assert_allclose(got, ref, rtol=2e-6, atol=1e-7)


@pytest.mark.parametrize("hidden", [896, 1024, 3, 17])
def test_layer_norm(orc, hidden):
    r = rng(hidden + 5)
    x = (r.normal(0, 1, (4, hidden)) * r.uniform(0.1, 10, (4, 1)) + r.normal(0, 5, (4, 1))).astype(np.float32)
    w = r.uniform(0.5, 1.5, hidden).astype(np.float32)
    b = r.normal(0, 0.3, hidden).astype(np.float32)
    got = orc.layer_norm(x, w, b, 1e-5)
    x64 = x.astype(np.float64)
    mu = x64.mean(axis=1, keepdims=True)
    var = ((x64 - mu) ** 2).mean(axis=1, keepdims=True)     # biased variance
    ref = (x64 - mu) / np.sqrt(var + 1e-5) * w + b
    np.testing.assert_allclose(got, ref, rtol=1e-5, atol=2e-6)


# ---- RoPE ---------------------------------------------------------------------
def test_rope_table(orc):
    hd, theta, n = 128, 1e6, 64
    c, s = orc.rope_table(n, hd, theta)
    c = c.reshape(n, hd)
    s = s.reshape(n, hd)
    d = np.arange(hd // 2)
    freq = 1.0 / theta ** (2.0 * d / hd)
    ang = np.arange(n)[:, None] * freq[None, :]
    # the two halves carry the same frequencies (NeoX layout, decoder.rs:302-338)
    np.testing.assert_allclose(c[:, :64], np.cos(ang), atol=2e-5)
    np.testing.assert_allclose(c[:, 64:], np.cos(ang), atol=2e-5)
    np.testing.assert_allclose(s[:, :64], np.sin(ang), atol=2e-5)
    np.testing.assert_allclose(s[:, 64:], np.sin(ang), atol=2e-5)
    assert (c[0] == 1).all() and (s[0] == 0).all()
    # long positions: still a rotation of unit norm
    c2, s2 = orc.rope_table(4096, hd, theta)
    np.testing.assert_allclose(c2.astype(np.float64) ** 2 + s2.astype(np.float64) ** 2, 1.0, atol=1e-6)


def test_apply_rope(orc):
    r = rng(8)
    seq, heads, hd = 5, 4, 128
    x = r.normal(0, 1, (seq, heads, hd)).astype(np.float32)
    c, s = orc.rope_table(64, hd, 1e6)
    c = c.reshape(64, hd)[30:30 + seq]
    s = s.reshape(64, hd)[30:30 + seq]
    got = orc.apply_rope(x.copy(), c, s, heads).reshape(seq, heads, hd)
    x64 = x.astype(np.float64)
    x1, x2 = x64[..., :64], x64[..., 64:]
    cc, ss = c[:, None, :64].astype(np.float64), s[:, None, :64].astype(np.float64)
    ref = np.concatenate([x1 * cc - x2 * ss, x2 * cc + x1 * ss], axis=-1)
    np.testing.assert_allclose(got, ref, rtol=1e-6, atol=1e-6)
    # a rotation keeps each pair's norm
    n0 = x64[..., :64] ** 2 + x64[..., 64:] ** 2
    n1 = got[..., :64].astype(np.float64) ** 2 + got[..., 64:].astype(np.float64) ** 2
    np.testing.assert_allclose(n1, n0, rtol=1e-5)


# ---- attention ----------------------------------------------------------------
def _softmax_attn(q, k, v, scale):
    s = (q @ k.T) * scale
    s = s - s.max(axis=-1, keepdims=True)
    p = np.exp(s)
    return (p / p.sum(axis=-1, keepdims=True)) @ v


@pytest.mark.parametrize("seq_q,start", [(1, 0), (1, 603), (9, 40), (33, 0)])
def test_causal_attention_gqa(orc, seq_q, start):
    r = rng(seq_q * 1000 + start)
    hq, hkv, hd, max_seq = 16, 8, 128, 1024
    seq_k = start + seq_q
    kc = r.normal(0, 1, (hkv, max_seq, hd)).astype(np.float32)
    vc = r.normal(0, 1, (hkv, max_seq, hd)).astype(np.float32)
    q = r.normal(0, 1, (seq_q, hq, hd)).astype(np.float32)
    scale = 1.0 / math.sqrt(hd)
    got = orc.causal_attention(q, kc, vc, max_seq * hd, seq_q, seq_k, hq, hkv, hd, scale, start)
    got = got.reshape(seq_q, hq, hd)
    for i in range(seq_q):
        for h in range(hq):
            kv = h // (hq // hkv)                        # GQA: consecutive q heads share a KV head
            n = start + i + 1
            ref = _softmax_attn(q[i, h][None].astype(np.float64), kc[kv, :n].astype(np.float64),
                                vc[kv, :n].astype(np.float64), scale)[0]
            np.testing.assert_allclose(got[i, h], ref, rtol=1e-5, atol=1e-6)


def test_bidirectional_windows(orc):
    r = rng(11)
    T, H, hd = 50, 3, 64
    ws = [0, 20, 40, 50]
    q, k, v = (r.normal(0, 1, (T, H, hd)).astype(np.float32) for _ in range(3))
    got = orc.bidir_attention(q, k, v, T, H, hd, 0.125, ws).reshape(T, H, hd)
    for w0, w1 in zip(ws[:-1], ws[1:]):
        for h in range(H):
            ref = _softmax_attn(q[w0:w1, h].astype(np.float64), k[w0:w1, h].astype(np.float64),
                                v[w0:w1, h].astype(np.float64), 0.125)
            np.testing.assert_allclose(got[w0:w1, h], ref, rtol=1e-5, atol=1e-6)


# ---- activations ------------------------------------------------------------
def test_fast_exp(orc):
    xs = np.concatenate([np.linspace(-80, 80, 2001), [0.0, 1.0, -1.0, 0.5, 1e-8]])
    for x in xs:
        # degree-5 Taylor remainder on |f| <= ln2/2 (2.4e-6; 3.2e-6 with the
        # f32 coefficients, measured on [-87, 87]) plus the f32
        # rounding of x*log2(e), which scales with |x| (~6e-8 |x|)
        xf = float(np.float32(x))
        got = float(orc.fast_exp(np.float32(x)))
        assert abs(got - math.exp(xf)) <= (4e-6 + 1e-7 * abs(xf)) * math.exp(xf), x
    assert orc.fast_exp(0.0) == 1.0
    # arguments beyond the clamp saturate at 2^126 and 2^-126 times the polynomial
    assert np.isfinite(orc.fast_exp(200.0)) and orc.fast_exp(200.0) > 1e37
    assert 0.0 < orc.fast_exp(-200.0) < 1e-37


def test_swiglu_rows(orc):
    r = rng(12)
    seq, inter = 3, 3072
    gu = r.normal(0, 3, (seq, 2 * inter)).astype(np.float32)
    got = orc.swiglu_rows(gu, inter).reshape(seq, inter)
    g = gu[:, 0::2].astype(np.float64)                  # rows interleaved gate, up (decoder.rs:94-104)
    u = gu[:, 1::2].astype(np.float64)
    ref = g / (1.0 + np.exp(-g)) * u
    np.testing.assert_allclose(got, ref, rtol=2e-5, atol=1e-6)


@pytest.mark.parametrize("n", [100, 4096, 10007])
def test_gelu(orc, n):
    r = rng(n)
    x = r.normal(0, 2, n).astype(np.float32)
    got = orc.gelu(x.copy())
    x64 = x.astype(np.float64)
    ref = 0.5 * x64 * (1 + np.tanh(math.sqrt(2 / math.pi) * (x64 + 0.044715 * x64 ** 3)))
    np.testing.assert_allclose(got, ref, rtol=2e-5, atol=2e-6)


def test_sinusoidal_pe(orc):
    n_pos, d = 13, 896
    got = orc.sinusoidal_pe(n_pos, d).reshape(n_pos, d)
    half = d // 2
    inv = np.exp(-np.arange(half) * math.log(10000.0) / (half - 1))
    ang = np.arange(n_pos)[:, None] * inv[None, :]
    np.testing.assert_allclose(got[:, :half], np.sin(ang), atol=2e-6)
    np.testing.assert_allclose(got[:, half:], np.cos(ang), atol=2e-6)


# ---- GEMMs / conv ------------------------------------------------------------
@pytest.mark.parametrize("M,N,K", [(1, 7, 5), (37, 65, 129), (404, 256, 1024)])
def test_sgemm_nt(orc, M, N, K):
    r = rng(M + N + K)
    A = r.normal(0, 1, (M, K)).astype(np.float32)
    B = r.normal(0, 1, (N, K)).astype(np.float32)
    got = orc.sgemm_nt(A, B)
    ref = A.astype(np.float64) @ B.astype(np.float64).T
    assert rel(got, ref) < 1e-6
    C0 = r.normal(0, 1, (M, N)).astype(np.float32)
    got = orc.sgemm_nt(A, B, C0)                        # beta = 1
    assert rel(got, ref + C0) < 1e-6


def test_linear_bias(orc):
    r = rng(21)
    x = r.normal(0, 1, (6, 40)).astype(np.float32)
    w = r.normal(0, 0.1, (24, 40)).astype(np.float32)
    b = r.normal(0, 1, 24).astype(np.float32)
    ref = x.astype(np.float64) @ w.astype(np.float64).T + b
    assert rel(orc.linear(x, w, b), ref) < 1e-6
    assert rel(orc.linear(x, w), ref - b) < 1e-6


def test_conv2d_3x3_s2(orc):
    import ctypes as C
    r = rng(31)
    cin, cout, H, W = 3, 5, 9, 12
    x = r.normal(0, 1, (cin, H, W)).astype(np.float32)
    w = r.normal(0, 0.3, (cout, cin, 3, 3)).astype(np.float32)
    b = r.normal(0, 1, cout).astype(np.float32)
    Ho, Wo = (H + 2 - 3) // 2 + 1, (W + 2 - 3) // 2 + 1
    out = np.empty((cout, Ho, Wo), np.float32)
    P = C.c_void_p
    orc.lib().or_conv2d(out.ctypes.data_as(P), x.ctypes.data_as(P), w.ctypes.data_as(P), b.ctypes.data_as(P),
                        cin, cout, H, W, 3, 3, 2, 1)
    xp = np.pad(x.astype(np.float64), ((0, 0), (1, 1), (1, 1)))
    ref = np.zeros((cout, Ho, Wo))
    for o in range(cout):
        for i in range(Ho):
            for j in range(Wo):
                ref[o, i, j] = (xp[:, 2 * i:2 * i + 3, 2 * j:2 * j + 3] * w[o]).sum() + b[o]
    np.testing.assert_allclose(out, ref, rtol=1e-5, atol=1e-5)


# ---- mel front end -------------------------------------------------------------
def _slaney_mel_filters(n_mels=128, n_fft=400, sr=16000):
    """Slaney-scale triangular filters with area normalisation (the 'slaney'
    definitions of librosa.filters.mel, htk=False, norm='slaney'), in float64."""
    def hz_to_mel(f):
        f = np.asarray(f, np.float64)
        lin = 3.0 * f / 200.0
        return np.where(f >= 1000.0, 15.0 + np.log(np.maximum(f, 1e-12) / 1000.0) / (math.log(6.4) / 27.0), lin)

    def mel_to_hz(m):
        m = np.asarray(m, np.float64)
        return np.where(m >= 15.0, 1000.0 * np.exp((math.log(6.4) / 27.0) * (m - 15.0)), 200.0 * m / 3.0)

    fft_f = np.linspace(0, sr / 2, n_fft // 2 + 1)
    pts = mel_to_hz(np.linspace(hz_to_mel(0.0), hz_to_mel(sr / 2), n_mels + 2))
    fd = np.diff(pts)
    fb = np.zeros((n_mels, fft_f.size))
    for m in range(n_mels):
        lower = (fft_f - pts[m]) / fd[m]
        upper = (pts[m + 2] - fft_f) / fd[m + 1]
        fb[m] = np.maximum(0, np.minimum(lower, upper)) * (2.0 / (pts[m + 2] - pts[m]))
    return fb


def _mel64(samples):
    x = np.asarray(samples, np.float64)
    xp = np.pad(x, 200, mode="reflect")
    n_frames = (xp.size - 400) // 160                   # the last frame is dropped
    win = 0.5 * (1 - np.cos(2 * np.pi * np.arange(400) / 400))    # periodic Hann
    frames = np.stack([xp[t * 160:t * 160 + 400] * win for t in range(n_frames)], axis=1)
    spec = np.abs(np.fft.rfft(frames, axis=0)) ** 2
    mel = _slaney_mel_filters() @ spec
    lg = np.log10(np.maximum(mel, 1e-10))
    return (np.maximum(lg, lg.max() - 8.0) + 4.0) / 4.0


@pytest.mark.parametrize("n", [16000, 12345])
def test_mel_vs_float64_fft(orc, n):
    from qwenasr_amd.synth import audio
    x = audio(n, 5)
    got = orc.mel(x)
    ref = _mel64(x)
    assert got.shape == ref.shape == (128, orc.lib().or_mel_frames(n))
    np.testing.assert_allclose(got, ref, atol=1e-4, rtol=0)


def test_mel_sine_peak(orc):
    """A pure 1 kHz tone puts its energy in the mel bin whose filter peaks nearest 1 kHz."""
    t = np.arange(16000) / 16000.0
    x = (0.5 * np.sin(2 * np.pi * 1000.0 * t)).astype(np.float32)
    got = orc.mel(x)
    fb = _slaney_mel_filters()
    peak_bin = int(np.argmax(fb[:, int(round(1000 / 40))]))
    assert (np.argmax(got[:, 5:-5], axis=0) == peak_bin).all()


# ---- forced-aligner logits (decoder_prefill_logits, decoder.rs:649-681) ------
def test_prefill_logits_composition(orc):
    """prefill, then the final RMSNorm of every row and the bf16 LM head:
    against float64 RMSNorm + matmul over the oracle's own prefill rows, for a
    separate [5000, H] head and for the tied embedding; the prefill itself
    leaves the same KV length either way."""
    from qwenasr_amd.synth import SynthDecoder
    from conftest import bf16, bf16f
    cfg = dict(n_layers=2, hidden=256, n_heads=4, n_kv_heads=2, head_dim=64, intermediate=512, vocab=1024,
               eps=1e-6, theta=1e6)
    w = SynthDecoder(cfg, seed=77)
    r = rng(78)
    w.norm = (1.0 + 0.5 * r.standard_normal(cfg["hidden"])).astype(np.float32)   # a gain that matters
    e = r.normal(0, 1, (37, cfg["hidden"])).astype(np.float32)
    lm = bf16(r.normal(0, 0.02, (5000, cfg["hidden"])))
    gain = np.asarray(w.norm, np.float64)
    for head in (lm, None):
        d1 = orc.OracleDecoder(w, max_seq=128)
        d2 = orc.OracleDecoder(w, max_seq=128)
        hid = d1.prefill_hidden(e).astype(np.float64)
        got = d2.prefill_logits(e, head)
        assert d1.kv_len == d2.kv_len == e.shape[0]
        xn = hid / np.sqrt((hid * hid).mean(axis=1, keepdims=True) + cfg["eps"]) * gain
        wt = bf16f(head if head is not None else w.embed).astype(np.float64)
        ref = xn @ wt.T
        assert got.shape == ref.shape
        assert rel(got, ref) < 1e-5
        d1.close()
        d2.close()


ARGMAX_KAT = [  # (row, index the aligner's scan picks, align.rs:312-321)
    ([1.0, 3.0, 3.0, 2.0], 1),                       # first of equal maxima
    ([2.0, 2.0, 2.0], 0),
    ([np.nan, 5.0, 7.0], 0),                         # nothing compares greater than a NaN start
    ([1.0, np.nan, 7.0, np.nan], 2),                 # later NaNs are skipped
    ([-np.inf, -np.inf], 0),
    ([-np.inf, np.nan, -np.inf, -1.0], 3),
    ([0.0, -0.0], 0), ([-0.0, 0.0], 0),              # signed zeros compare equal
    ([np.inf, np.inf, 1.0], 0),
    ([-5.0], 0),
]


def test_argmax_f32_rows_kat(orc):
    """the aligner's per-row argmax: hand-derived answers of the scan for ties,
    NaN, infinities and signed zeros, and numpy's first-occurrence argmax on
    NaN-free rows (ties planted across the row)"""
    for row, want in ARGMAX_KAT:
        assert orc.argmax_f32_rows(np.array([row], np.float32))[0] == want, row
    r = rng(79)
    x = r.normal(0, 1, (20, 5000)).astype(np.float32)
    x[3, 4999] = x[3].max() + 1
    x[4, [10, 2000, 4000]] = x[4].max() + 1
    x[5] = 0.25
    assert (orc.argmax_f32_rows(x) == np.argmax(x, axis=1)).all()
    assert orc.argmax_f32_rows(x)[4] == 10 and orc.argmax_f32_rows(x)[5] == 0

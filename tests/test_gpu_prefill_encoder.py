"""GPU parity of the prefill / audio-encoder / mel path and the offline driver.

Tolerances: f32-class GEMMs (bf16x3 split on MFMA) vs the oracle's f32 GEMM
within 2e-5 norm-wise; int8 x bf16 GEMM within 1e-2 norm-wise of the f32 GEMM
on the bf16 weights and 1e-5 of its own exact int8
restatement; LayerNorm bit-exact; attention 1e-5; encoder / mel 2e-4;
transcription token ids identical.
"""
import numpy as np
import pytest

from conftest import bf16, bf16f, rng

pytestmark = pytest.mark.gpu


def nrel(a, b):
    return float(np.linalg.norm(np.asarray(a, np.float64) - b) / np.linalg.norm(np.asarray(b, np.float64)))


@pytest.mark.parametrize("M,N,K", [(404, 4096, 1024), (375, 1024, 3072), (390, 2688, 896), (100, 480, 9),
                                   (33, 70, 100), (33, 70, 128), (1, 64, 32)])
def test_linear_bf16w(dev, orc, M, N, K):
    from qwenasr_amd import kernels as Kr
    print(f"linear_bf16w M={M} N={N} K={K}", flush=True)
    r = rng(M + N + K)
    x = r.normal(0, 1, (M, K)).astype(np.float32)
    w = bf16(r.normal(0, 0.02, (N, K)))
    b = r.normal(0, 1, N).astype(np.float32)
    y = dev.empty((M, N), np.float32)
    dx, dw, db = dev.upload(x), dev.upload(w), dev.upload(b)
    Kr.linear(y, dx, dw, db, M, K, N)
    ref = orc.linear(x, bf16f(w), b)
    exact = x.astype(np.float64) @ bf16f(w).astype(np.float64).T + b
    assert nrel(y.numpy(), exact) < 2e-6
    assert nrel(y.numpy(), ref) < 2e-5
    # linear_accumulate: y = (y + b) + x W^T
    y0 = r.normal(0, 1, (M, N)).astype(np.float32)
    y.copy_from(y0)
    Kr.linear(y, dx, dw, db, M, K, N, accumulate=True)
    assert nrel(y.numpy(), exact + y0) < 2e-6


@pytest.mark.parametrize("M,N,K", [(375, 2048, 1024), (375, 1024, 1024), (375, 1024, 2048), (375, 1024, 3072),
                                   (375, 6144, 1024), (375, 151936, 1024), (1, 1024, 1024), (67, 1024, 3072),
                                   (404, 1024, 1024), (67, 151936, 1024), (1, 151936, 1024), (129, 151936, 1024),
                                   (130, 151936, 2048)])
def test_gemm_w8_bf16_config1(dev, orc, M, N, K):
    """Config 1: M = 375 rows of bf16 activations x int8 per-row weights, the
    0.6B shapes (q, k / v, o, down, gate_up, LM head) and edge row counts
    (partial row tiles); a second call must give the same bits."""
    from qwenasr_amd import kernels as Kr
    print(f"gemm_w8_bf16 M={M} N={N} K={K}", flush=True)
    r = rng(N + K + M)
    wb = bf16(r.normal(0, 0.02, (N, K)))
    a = bf16(r.normal(0, 1, (M, K)))
    q, s = orc.quantize_bf16_rows(wb, 0)
    y = dev.empty((M, N), np.float32)
    da, dq, ds = dev.upload(a), dev.upload(q), dev.upload(s)
    Kr.gemm_w8_bf16(y, da, dq, ds, M, N, K)
    got = y.numpy()
    Kr.gemm_w8_bf16(y, da, dq, ds, M, N, K)
    assert (y.numpy() == got).all()
    af = bf16f(a).astype(np.float64)
    exact_int8 = (af @ q.astype(np.float64).T) * s
    assert nrel(got, exact_int8) < 1e-5
    if N <= 8192:
        ref = orc.sgemm_nt(bf16f(a), bf16f(wb))     # the reference's f32 GEMM on bf16 weights
        assert nrel(got, ref) < 1e-2


def test_layer_norm_bitexact(dev, orc):
    from qwenasr_amd import kernels as Kr
    r = rng(5)
    for seq, hidden in ((390, 896), (3, 1024), (1, 16)):
        x = (r.normal(0, 1, (seq, hidden)) * r.uniform(0.1, 10, (seq, 1)) + r.normal(0, 3, (seq, 1))).astype(np.float32)
        w = r.uniform(0.5, 1.5, hidden).astype(np.float32)
        b = r.normal(0, 0.1, hidden).astype(np.float32)
        out = dev.empty((seq, hidden), np.float32)
        Kr.layer_norm(out, dev.upload(x), dev.upload(w), dev.upload(b), seq, hidden, 1e-5)
        assert (out.numpy() == orc.layer_norm(x, w, b, 1e-5)).all()


@pytest.mark.parametrize("S,start", [(404, 0), (37, 100), (1, 0)])
def test_prefill_attention(dev, orc, S, start):
    from qwenasr_amd import kernels as Kr
    r = rng(S + start)
    hq, hkv, hd, max_seq = 16, 8, 128, 1024
    kc = r.normal(0, 1, (hkv, max_seq, hd)).astype(np.float32)
    vc = r.normal(0, 1, (hkv, max_seq, hd)).astype(np.float32)
    q = r.normal(0, 1, (S, hq * hd)).astype(np.float32)
    scale = float(np.float32(1) / np.sqrt(np.float32(hd)))
    out = dev.empty((S, hq * hd), np.float32)
    Kr.causal_attention(out, dev.upload(q), dev.upload(kc), dev.upload(vc), max_seq * hd, S, start + S, hq, hkv,
                        hd, scale, start)
    ref = orc.causal_attention(q, kc, vc, max_seq * hd, S, start + S, hq, hkv, hd, scale, start)
    np.testing.assert_allclose(out.numpy().reshape(-1), ref, rtol=1e-4, atol=2e-5)
    assert nrel(out.numpy().reshape(-1), ref) < 1e-5


@pytest.mark.parametrize("T,H,hd,win", [(390, 14, 64, 104), (130, 8, 128, 48), (9, 2, 128, 100), (77, 3, 64, 16)])
def test_bidirectional_attention(dev, orc, T, H, hd, win):
    """Windowed attention of the encoder (head_dim 64) and the 128-dim
    single-group form, ragged windows and fewer rows than one 16-row tile."""
    from qwenasr_amd import kernels as Kr
    r = rng(77 + T)
    q, k, v = (r.normal(0, 1, (T, H * hd)).astype(np.float32) for _ in range(3))
    out = dev.empty((T, H * hd), np.float32)
    scale = float(np.float32(1) / np.sqrt(np.float32(hd)))
    Kr.bidirectional_attention(out, dev.upload(q), dev.upload(k), dev.upload(v), T, H, hd, scale, win)
    ws = list(range(0, T, win)) + [T]
    ref = orc.bidir_attention(q, k, v, T, H, hd, scale, ws)
    assert nrel(out.numpy().reshape(-1), ref) < 1e-5


TINY_DEC = dict(n_layers=2, hidden=1024, n_heads=16, n_kv_heads=8, head_dim=128, intermediate=3072,
                vocab=8192, eps=1e-6, theta=1e6)


def test_decoder_prefill_then_decode(dev, orc):
    from qwenasr_amd.model import Decoder
    from qwenasr_amd.synth import SynthDecoder
    w = SynthDecoder(TINY_DEC, seed=1002)
    gpu = Decoder(dev, w, max_seq=512)
    cpu = orc.OracleDecoder(w, max_seq=512)
    r = rng(4)
    S = 100
    emb = (r.normal(0, 0.02, (S, 1024))).astype(np.float32)
    gpu.prefill(emb)
    cpu.prefill(emb)
    assert gpu.kv_len == cpu.kv_len == S
    kg, vg = gpu.kv_download()
    kc, vc = cpu.kv()
    assert nrel(kg[:, :, :S], kc[:, :, :S]) < 1e-4 and nrel(vg[:, :, :S], vc[:, :, :S]) < 1e-4
    # layer 0 only sees f32-class GEMMs + per-head norm + RoPE
    assert nrel(kg[0, :, :S], kc[0, :, :S]) < 1e-5
    tok = 11
    for step in range(16):
        e = cpu.embed(tok)
        t_c, margin = cpu.forward(e)
        t_g = gpu.forward(token=tok)
        assert t_c == t_g, (step, t_c, t_g, margin)
        tok = t_c
    gpu.close()
    cpu.close()


def test_decoder_prefill_k_groups(dev, orc):
    """A narrow decoder (hidden 512, intermediate 1024) whose prefill GEMMs
    take the K-group form (64 x 64 tiles, 4 groups of waves splitting K: at
    most 32 column tiles and 16+ K-steps), the gate_up GEMM with the SwiGLU in
    its epilogue included: the prefill rows of both layers against the oracle
    (layer 1's rows see layer 0's SwiGLU output)."""
    from qwenasr_amd.model import Decoder
    from qwenasr_amd.synth import SynthDecoder
    cfg = dict(TINY_DEC, hidden=512, intermediate=1024)
    w = SynthDecoder(cfg, seed=1012)
    gpu = Decoder(dev, w, max_seq=256)
    cpu = orc.OracleDecoder(w, max_seq=256)
    try:
        S = 150
        emb = rng(41).normal(0, 0.02, (S, cfg["hidden"])).astype(np.float32)
        print("narrow decoder prefill, K groups", flush=True)
        gpu.prefill(emb)
        cpu.prefill(emb)
        kg, vg = gpu.kv_download()
        kc, vc = cpu.kv()
        for l in range(cfg["n_layers"]):
            ek = nrel(kg[l, :, :S], kc[l, :, :S])
            ev = nrel(vg[l, :, :S], vc[l, :, :S])
            print(f"layer {l}: K {ek:.3g} V {ev:.3g}", flush=True)
            assert ek < 1e-5 and ev < 1e-5, (l, ek, ev)
    finally:
        gpu.close()
        cpu.close()


def test_decoder_prefill_logits(dev, orc):
    """decoder_prefill_logits (decoder.rs:649-681), the forced aligner's path:
    every row's logits through the tied embedding and through a separate
    [5000, hidden] bf16 head (ragged against the GEMM tiles), against the
    oracle; per-row argmax agrees wherever the oracle's top-2 gap is clear."""
    from qwenasr_amd.model import Decoder
    from qwenasr_amd.synth import SynthDecoder
    w = SynthDecoder(TINY_DEC, seed=1003)
    r = rng(5)
    w.norm = (1.0 + 0.5 * r.standard_normal(TINY_DEC["hidden"])).astype(np.float32)
    gpu = Decoder(dev, w, max_seq=256)
    S = 50
    emb = r.normal(0, 0.02, (S, TINY_DEC["hidden"])).astype(np.float32)
    head = bf16(r.normal(0, 0.02, (5000, TINY_DEC["hidden"])))
    try:
        for lm in (None, head):
            print("prefill logits, head", "tied" if lm is None else lm.shape, flush=True)
            gpu.set_lm_head(lm)
            gpu.kv_len = 0
            got = gpu.prefill_logits(emb)
            assert gpu.kv_len == S
            cpu = orc.OracleDecoder(w, max_seq=256)
            want = cpu.prefill_logits(emb, lm)
            cpu.close()
            assert got.shape == want.shape == (S, TINY_DEC["vocab"] if lm is None else 5000)
            assert nrel(got, want) < 2e-4
            top2 = np.sort(want, axis=1)[:, -2:]
            clear = (top2[:, 1] - top2[:, 0]) > 1e-3 * np.abs(top2[:, 1]).max()
            assert clear.sum() > S // 2
            assert (got.argmax(1)[clear] == want.argmax(1)[clear]).all()
        # the aligner's readout: argmax at chosen rows, logits left on the device
        rows = np.array([S - 1, 0, 7, 7, 31, 49], np.int32)
        gpu.set_lm_head(head)
        gpu.kv_len = 0
        full = gpu.prefill_logits(emb)
        gpu.kv_len = 0
        idx = gpu.prefill_argmax(emb, rows)
        assert gpu.kv_len == S
        assert (idx == orc.argmax_f32_rows(full[rows])).all()      # same rows, same logits
        gpu.kv_len = 0
        assert gpu.prefill_argmax(emb, np.zeros(0, np.int32)).shape == (0,)
        assert gpu.kv_len == S
        from qwenasr_amd import QasrError
        for bad in ([S], [-1]):
            gpu.kv_len = 0
            with pytest.raises(QasrError):
                gpu.prefill_argmax(emb, np.array(bad, np.int32))
    finally:
        gpu.set_lm_head(None)
        gpu.close()


def test_argmax_f32_rows(dev, orc):
    """per-row argmax kernel vs the oracle's restatement of the aligner's scan:
    the hand-checked cases of the oracle's known answers, full-vocabulary rows
    with maxima planted in different lanes and waves, and a row stride wider
    than the columns scanned"""
    from qwenasr_amd import kernels as Kr
    from test_oracle_float import ARGMAX_KAT
    for row, want in ARGMAX_KAT:
        x = np.array([row], np.float32)
        idx = dev.empty(1, np.int32)
        assert Kr.argmax_f32_rows(dev.upload(x), 1, x.shape[1], idx)[0] == want, row
    r = rng(6)
    rows, cols = 37, 151936
    x = r.normal(0, 1, (rows, cols)).astype(np.float32)
    for k, cs in enumerate(([5, 70000], [257, 1, 151935], [64, 128, 192], [151935, 151934])):
        x[k, cs] = 9.0
    x[10, 0] = np.nan
    x[11, 1::3] = np.nan
    x[12] = -np.inf
    x[13, :500] = np.nan
    x[13, 0] = -1.0
    want = orc.argmax_f32_rows(x)
    idx = dev.empty(rows, np.int32)
    got = Kr.argmax_f32_rows(dev.upload(x), rows, cols, idx)
    assert (got == want).all(), np.nonzero(got != want)
    assert list(want[:4]) == [5, 1, 64, 151934] and want[10] == 0 and want[12] == 0
    got = Kr.argmax_f32_rows(dev.upload(x), rows, 5000, idx, ld=cols)
    assert (got == orc.argmax_f32_rows(np.ascontiguousarray(x[:, :5000]))).all()


def test_mel(dev, orc):
    from qwenasr_amd.model import Encoder
    from qwenasr_amd.synth import ENC_0_6B, SynthEncoder, audio
    cfg = dict(ENC_0_6B, n_layers=1)
    enc = Encoder(dev, SynthEncoder(cfg, seed=1002))
    for n in (48000, 480000, 16123):
        x = audio(n, 1002)
        m_g = enc.mel(x)
        m_c = orc.mel(x)
        assert m_g.shape == m_c.shape == (128, orc.lib().or_mel_frames(n))
        np.testing.assert_allclose(m_g, m_c, atol=2e-4, rtol=0)
    enc.close()


def test_encoder(dev, orc):
    from qwenasr_amd.model import Encoder
    from qwenasr_amd.synth import ENC_0_6B, SynthEncoder, audio
    cfg = dict(ENC_0_6B, n_layers=2)
    w = SynthEncoder(cfg, seed=1002)
    enc = Encoder(dev, w)
    ore = orc.OracleEncoder(w)
    for n in (64000, 50000):                    # 400 frames (4 full chunks); 312 frames (a tail chunk)
        mel = orc.mel(audio(n, 7))
        out_g = enc.forward(mel)
        out_c = ore.forward(mel)
        assert out_g.shape == out_c.shape
        print(f"encoder frames={mel.shape[1]} tokens={out_g.shape[0]} rel={nrel(out_g, out_c):.2e}", flush=True)
        assert nrel(out_g, out_c) < 2e-4
    enc.close()
    ore.close()


@pytest.mark.parametrize("conv_hidden,chunk", [(32, 100), (48, 100), (96, 100), (32, 128)])
def test_encoder_conv_stem_widths(dev, orc, conv_hidden, chunk):
    """The conv stem at widths that are a multiple of 32 (channels-last,
    implicit-im2col GEMMs: 32, 96) and one that is not (48: the im2col form,
    whose conv2 / conv3 K of 432 also takes the fallback GEMM), each against
    the oracle's reference-layout stem (encoder.rs:226-287).  With 128-frame
    chunks the full chunks' input planes exceed the direct first
    convolution's LDS, so the channels-last stem forms conv1 as im2col and a
    K = 9 GEMM with the channels-last GELU epilogue (the 56-frame tail chunk
    stays direct)."""
    from qwenasr_amd.model import Encoder
    from qwenasr_amd.synth import SynthEncoder, audio
    cfg = dict(d_model=64, n_layers=1, n_heads=1, head_dim=64, ffn_dim=128, output_dim=128, chunk_size=chunk,
               n_window_infer=8 * chunk, conv_hidden=conv_hidden)
    w = SynthEncoder(cfg, seed=60 + conv_hidden)
    enc = Encoder(dev, w)
    ore = orc.OracleEncoder(w)
    try:
        mel = orc.mel(audio(50000, 61))             # 312 frames: full chunks and a tail
        out_g, out_c = enc.forward(mel), ore.forward(mel)
        print(f"conv_hidden {conv_hidden}, chunk {chunk}: rel {nrel(out_g, out_c):.2e}", flush=True)
        assert out_g.shape == out_c.shape and nrel(out_g, out_c) < 2e-4
    finally:
        enc.close()
        ore.close()


def test_encoder_forward_batch(dev, orc):
    """One encoder pass over several mels (the stream batch's windows and
    partial tails): each mel's rows are bit for bit those of its own call —
    an 8 s window (800 frames), tails of 1..99 frames after full chunks, a
    mel shorter than one chunk — and the first also against the oracle."""
    from qwenasr_amd.model import Encoder
    from qwenasr_amd.synth import ENC_0_6B, SynthEncoder, audio
    w = SynthEncoder(dict(ENC_0_6B, n_layers=2), seed=1012)
    enc = Encoder(dev, w)
    ore = orc.OracleEncoder(w)
    try:
        ns = [128000, 50000, 8000, 31840, 128000, 1600, 77777]
        mels = [orc.mel(audio(n, 40 + i)) for i, n in enumerate(ns)]
        print("frames", [m.shape[1] for m in mels], flush=True)
        got = enc.forward_batch(mels)
        for m, g in zip(mels, got):
            one = enc.forward(m)
            assert g.shape == one.shape and g.tobytes() == one.tobytes(), m.shape
        assert nrel(got[0], ore.forward(mels[0])) < 2e-4
        got2 = enc.forward_batch(mels[3:5])                 # a second call, fewer sequences
        assert got2[0].tobytes() == got[3].tobytes() and got2[1].tobytes() == got[4].tobytes()
    finally:
        enc.close()
        ore.close()


def test_transcribe_forced_tokens(dev, orc):
    """transcribe_segment with a forced decode length: identical token ids."""
    from qwenasr_amd.model import Decoder, Encoder, transcribe_forced
    from qwenasr_amd.synth import DEC_0_6B, ENC_0_6B, SynthDecoder, SynthEncoder, audio
    dcfg = dict(DEC_0_6B, n_layers=2)
    ecfg = dict(ENC_0_6B, n_layers=2)
    wd, we = SynthDecoder(dcfg, seed=1002), SynthEncoder(ecfg, seed=1002)
    x = audio(64000, 1002)
    gd, ge = Decoder(dev, wd, max_seq=512), Encoder(dev, we)
    cd, ce = orc.OracleDecoder(wd, max_seq=512), orc.OracleEncoder(we)
    toks_g, times = transcribe_forced(gd, ge, x, 24)
    res = orc.transcribe_forced(cd, ce, x, 24)
    print("gpu", toks_g.tolist(), "times", times.tolist(), flush=True)
    print("cpu", res["tokens"].tolist(), "margins", np.round(res["margins"], 4).tolist(), flush=True)
    assert toks_g.tolist() == res["tokens"].tolist()
    for m in (gd, ge, cd, ce):
        m.close()


@pytest.mark.parametrize("vocab", [151650, 151670])
def test_prompt_ids_beyond_vocab_rejected(dev, vocab):
    """Every prompt id (transcribe.rs:13-15: up to 151670) is gathered from the
    embedding table on the device, so a table with fewer rows is rejected with
    QASR_ERR_INVALID before anything is launched: the offline driver at both
    sizes, the stream at 151650 (PREFIX_TAIL's 151669) and 151670 (SUFFIX's
    151670)."""
    from qwenasr_amd import QasrError
    from qwenasr_amd.model import Decoder, Encoder, Stream, transcribe_forced
    from qwenasr_amd.synth import SynthDecoder, SynthEncoder, audio
    wd = SynthDecoder(dict(n_layers=1, hidden=128, n_heads=16, n_kv_heads=8, head_dim=128, intermediate=128,
                           vocab=vocab, eps=1e-6, theta=1e6), seed=31)
    we = SynthEncoder(dict(d_model=64, n_layers=1, n_heads=1, head_dim=64, ffn_dim=128, output_dim=128,
                           chunk_size=100, n_window_infer=800, conv_hidden=32), seed=32)
    d, e = Decoder(dev, wd, max_seq=256), Encoder(dev, we)
    try:
        with pytest.raises(QasrError, match="vocab too small"):
            transcribe_forced(d, e, audio(16000, 33), 4)
        with pytest.raises(QasrError, match="vocab too small"):
            Stream(d, e)
    finally:
        d.close()
        e.close()

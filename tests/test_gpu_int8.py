"""GPU parity of the int8 hot path against the oracle (through the C ABI).

Bar: bit-exact for the packer, activation quantizer, W8A8 matvecs, fused
RMSNorm prologue and argmax indices; SwiGLU outputs (libm expf vs the GPU's
expf) within 2e-6 relative.
"""
import numpy as np
import pytest

from conftest import bf16, rng

pytestmark = pytest.mark.gpu


def _k():
    from qwenasr_amd import kernels
    return kernels


@pytest.mark.parametrize("n,k,mode", [(2048, 1024, 0), (2048, 1024, 1), (1024, 3072, 0),
                                      (77, 1000, 1), (6144, 1024, 1), (3, 24, 0)])
def test_pack_bitexact(dev, orc, n, k, mode):
    print(f"pack n={n} k={k} mode={mode}", flush=True)
    w = bf16(rng(n + k).normal(0, 0.02, (n, k)))
    w[0, :] = 0                                       # zero row -> scale 1
    dw = dev.upload(w)
    q, s = dev.empty((n, k), np.int8), dev.empty(n, np.float32)
    _k().quantize_bf16_weights_to_int8(dw, n, k, q, s, mode)
    qo, so = orc.quantize_bf16_rows(w, mode)
    assert (q.numpy() == qo).all()
    assert (s.numpy() == so).all()


def test_pack_lm_head(dev, orc):
    from qwenasr_amd.synth import normal_bf16
    w = normal_bf16((151936, 1024), 1001, "thinker.model.embed_tokens.weight")
    print("pack lm head 151936x1024", flush=True)
    dw = dev.upload(w)
    q, s = dev.empty(w.shape, np.int8), dev.empty(w.shape[0], np.float32)
    _k().quantize_bf16_weights_to_int8(dw, *w.shape, q, s, 0)
    qo, so = orc.quantize_bf16_rows(w, 0)
    assert (s.numpy() == so).all() and (q.numpy() == qo).all()


def test_quantize_act(dev, orc):
    for k in (1024, 3072, 64):
        x = rng(k).normal(0, 1, k).astype(np.float32)
        q, s = dev.empty(k, np.int8), dev.empty(1, np.float32)
        _k().quantize_f32_to_int8(dev.upload(x), q, s)
        qo, so = orc.quantize_act(x)
        assert (q.numpy() == qo).all() and s.numpy()[0] == so


def _mats(r, n, k):
    w = r.integers(-127, 128, (n, k), dtype=np.int8)
    ws = r.uniform(1e-4, 2e-3, n).astype(np.float32)
    return w, ws


@pytest.mark.parametrize("n,k", [(1024, 1024), (1024, 2048), (1024, 3072), (2048, 6144),
                                 (96, 64), (4096, 320), (151, 1024)])
def test_linear_int8_bitexact(dev, orc, n, k):
    print(f"linear_int8 n={n} k={k}", flush=True)
    r = rng(n * 7 + k)
    w, ws = _mats(r, n, k)
    x = r.normal(0, 1, k).astype(np.float32)
    b = r.normal(0, 1, n).astype(np.float32)
    dw, dws, dx, db = dev.upload(w), dev.upload(ws), dev.upload(x), dev.upload(b)
    y = dev.empty(n, np.float32)
    K = _k()
    K.linear_int8(y, dx, dw, dws, None, k, n)
    assert (y.numpy() == orc.linear_int8(x, w, ws)).all()
    K.linear_int8(y, dx, dw, dws, db, k, n)
    assert (y.numpy() == orc.linear_int8(x, w, ws, b)).all()
    y.copy_from(b)
    K.linear_nobias_int8_addto(y, dx, dw, dws, k, n)
    assert (y.numpy() == orc.linear_int8_addto(b, x, w, ws)).all()


@pytest.mark.parametrize("hidden,qd,kvd", [(1024, 2048, 1024), (2048, 2048, 1024), (256, 512, 256)])
def test_qkv_bitexact(dev, orc, hidden, qd, kvd):
    print(f"qkv hidden={hidden}", flush=True)
    r = rng(hidden)
    (wq, sq), (wk, sk), (wv, sv) = _mats(r, qd, hidden), _mats(r, kvd, hidden), _mats(r, kvd, hidden)
    x = r.normal(0, 1, hidden).astype(np.float32)
    nw = r.uniform(0.5, 1.5, hidden).astype(np.float32)
    d = [dev.upload(a) for a in (x, wq, sq, wk, sk, wv, sv, nw)]
    q, k, v = dev.empty(qd, np.float32), dev.empty(kvd, np.float32), dev.empty(kvd, np.float32)
    _k().linear_nobias_int8_qkv(q, k, v, d[0], *d[1:7], hidden, qd, kvd)
    qo, ko, vo = orc.linear_int8_qkv(x, wq, sq, wk, sk, wv, sv)
    assert (q.numpy() == qo).all() and (k.numpy() == ko).all() and (v.numpy() == vo).all()
    # fused RMSNorm prologue (decoder.rs:583-593): exact, including the AVX summation order
    _k().linear_nobias_int8_qkv(q, k, v, d[0], *d[1:7], hidden, qd, kvd, norm_w=d[7], eps=1e-6)
    xn = orc.rms_norm(x, nw, 1e-6)
    qo, ko, vo = orc.linear_int8_qkv(xn, wq, sq, wk, sk, wv, sv)
    assert (q.numpy() == qo).all() and (k.numpy() == ko).all() and (v.numpy() == vo).all()


@pytest.mark.parametrize("hidden,inter", [(1024, 3072), (2048, 6144), (128, 64)])
def test_swiglu(dev, orc, hidden, inter):
    print(f"swiglu hidden={hidden} inter={inter}", flush=True)
    r = rng(inter)
    w, ws = _mats(r, 2 * inter, hidden)
    x = r.normal(0, 1, hidden).astype(np.float32)
    nw = r.uniform(0.5, 1.5, hidden).astype(np.float32)
    dx, dw, dws, dn = dev.upload(x), dev.upload(w), dev.upload(ws), dev.upload(nw)
    out = dev.empty(inter, np.float32)
    _k().linear_nobias_int8_swiglu(out, dx, dw, dws, hidden, inter)
    np.testing.assert_allclose(out.numpy(), orc.linear_int8_swiglu(x, w, ws), rtol=2e-6, atol=1e-12)
    _k().linear_nobias_int8_swiglu(out, dx, dw, dws, hidden, inter, norm_w=dn, eps=1e-6)
    ref = orc.linear_int8_swiglu(orc.rms_norm(x, nw, 1e-6), w, ws)
    np.testing.assert_allclose(out.numpy(), ref, rtol=2e-6, atol=1e-12)


@pytest.mark.parametrize("n,k", [(151936, 1024), (5000, 1024), (151936, 2048), (300, 64)])
def test_argmax(dev, orc, n, k):
    print(f"argmax n={n} k={k}", flush=True)
    r = rng(n + k)
    w, ws = _mats(r, n, k)
    x = r.normal(0, 1, k).astype(np.float32)
    dx, dw, dws = dev.upload(x), dev.upload(w), dev.upload(ws)
    idx = dev.empty(1, np.int32)
    K = _k()
    io, _, _ = orc.argmax_int8(x, w, ws)
    assert K.argmax_matvec_int8(dx, dw, dws, k, n, idx) == io
    # ties: copy the winner to lower and higher rows in other blocks
    for dup in (0, n // 3, n - 1):
        w2, ws2 = w.copy(), ws.copy()
        w2[dup], ws2[dup] = w[io], ws[io]
        i2, _, _ = orc.argmax_int8(x, w2, ws2)
        assert i2 == min(dup, io)
        assert K.argmax_matvec_int8(dx, dev.upload(w2), dev.upload(ws2), k, n, idx) == i2
    # fused final RMSNorm (decoder.rs:634-641)
    nw = r.uniform(0.5, 1.5, k).astype(np.float32)
    io, _, _ = orc.argmax_int8(orc.rms_norm(x, nw, 1e-6), w, ws)
    assert K.argmax_matvec_int8(dx, dw, dws, k, n, idx, norm_w=dev.upload(nw), eps=1e-6) == io


def test_rms_norm_rows_bitexact(dev, orc):
    r = rng(9)
    for seq, hidden in ((404, 1024), (3, 2048), (1, 64)):
        x = (r.normal(0, 1, (seq, hidden)) * r.uniform(0.1, 10, (seq, 1))).astype(np.float32)
        w = r.uniform(0.5, 1.5, hidden).astype(np.float32)
        out = dev.empty((seq, hidden), np.float32)
        _k().rms_norm(out, dev.upload(x), dev.upload(w), seq, hidden, 1e-6)
        assert (out.numpy() == orc.rms_norm(x, w, 1e-6)).all()

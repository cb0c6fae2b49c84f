"""GPU parity of the decode step (decoder_forward, decoder.rs:550-645) and its
float kernels against the oracle.

Per-head norm, RoPE and attention are f32 kernels compared within 1e-5
relative; token ids must be identical under teacher forcing (the oracle's
token is fed back to both sides at every step).
"""
import numpy as np
import pytest

from conftest import rng

pytestmark = pytest.mark.gpu

TINY = dict(n_layers=2, hidden=1024, n_heads=16, n_kv_heads=8, head_dim=128, intermediate=3072,
            vocab=8192, eps=1e-6, theta=1e6)


def test_head_norm_and_rope(dev, orc):
    from qwenasr_amd import kernels as K
    r = rng(21)
    seq, heads, hd = 7, 16, 128
    x = r.normal(0, 1, (seq, heads, hd)).astype(np.float32)
    w = r.uniform(0.5, 1.5, hd).astype(np.float32)
    cos, sin = orc.rope_table(64, hd, 1e6)
    dx = dev.upload(x)
    K.rms_norm_per_head(dx, dev.upload(w), seq, heads, hd, 1e-6)
    ref = orc.rms_norm_per_head(x, w, heads, 1e-6)
    np.testing.assert_allclose(dx.numpy(), ref.reshape(x.shape), rtol=1e-5, atol=1e-6)
    dx.copy_from(x)
    K.apply_rope_neox(dx, dev.upload(cos[40:40 + seq]), dev.upload(sin[40:40 + seq]), seq, heads, hd)
    ref = orc.apply_rope(x, cos[40:40 + seq], sin[40:40 + seq], heads)
    np.testing.assert_allclose(dx.numpy(), ref.reshape(x.shape), rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("L", [1, 17, 604, 2048, 4096])
def test_decode_attention(dev, orc, L):
    from qwenasr_amd import kernels as K
    print(f"attention L={L}", flush=True)
    r = rng(L)
    hq, hkv, hd, max_seq = 16, 8, 128, 4096
    kc = r.normal(0, 1, (hkv, max_seq, hd)).astype(np.float32)
    vc = r.normal(0, 1, (hkv, max_seq, hd)).astype(np.float32)
    q = r.normal(0, 1, hq * hd).astype(np.float32)
    scale = np.float32(1.0) / np.sqrt(np.float32(hd))
    out = dev.empty(hq * hd, np.float32)
    K.causal_attention(out, dev.upload(q), dev.upload(kc), dev.upload(vc), max_seq * hd, 1, L, hq, hkv,
                       hd, float(scale), L - 1)
    ref = orc.causal_attention(q, kc, vc, max_seq * hd, 1, L, hq, hkv, hd, float(scale), L - 1)
    np.testing.assert_allclose(out.numpy(), ref, rtol=1e-5, atol=2e-6)


@pytest.fixture(scope="module")
def tiny_models(dev, orc):
    from qwenasr_amd.model import Decoder
    from qwenasr_amd.synth import SynthDecoder
    w = SynthDecoder(TINY, seed=1002)
    gpu = Decoder(dev, w, max_seq=512)
    cpu = orc.OracleDecoder(w, max_seq=512)
    yield w, gpu, cpu
    gpu.close()
    cpu.close()


def test_decoder_packing_bitexact(tiny_models):
    _, gpu, cpu = tiny_models
    for layer in (0, 1):
        for which in range(6):
            qg, sg = gpu.packed(layer, which)
            qc, sc = cpu.packed(layer, which)
            assert (qg == qc).all() and (sg == sc).all(), (layer, which)
    qg, sg = gpu.packed(-1, 0)
    qc, sc = cpu.packed(-1, 0)
    assert (qg == qc).all() and (sg == sc).all()


@pytest.mark.parametrize("splits", [-1, 16, 8, 3, 40])
def test_decoder_teacher_forced(tiny_models, splits):
    """splits -1: the automatic choice (8 splits at this context, partials
    merged inside the o_proj kernel); 16 and 8: o_proj merges, most splits
    empty early on; 3: merged by the attention kernel's last block with
    ragged splits; 40: attention-side merge, more splits than positions."""
    w, gpu, cpu = tiny_models
    print(f"teacher forced splits={splits}", flush=True)
    gpu.set_options(attn_splits=splits)
    gpu.kv_len = 0
    cpu.kv_len = 0
    n = 48
    tok = 151644 % TINY["vocab"]
    mism = []
    for s in range(n):
        e = cpu.embed(tok)
        t_c, margin = cpu.forward(e)
        t_g = gpu.forward(token=tok) if s else gpu.forward(embed=e)
        if t_c != t_g:
            mism.append((s, t_c, t_g, margin))
        tok = t_c
    assert not mism, mism
    kg, vg = gpu.kv_download()
    kc, vc = cpu.kv()
    # layer 0 sees bit-identical q/k/v projections (exact int8 path from the
    # embedding); only per-head norm + RoPE rounding separates the caches
    np.testing.assert_allclose(kg[0, :, :n], kc[0, :, :n], rtol=1e-5, atol=1e-5)
    assert (vg[0, :, :n] == vc[0, :, :n]).all()
    # deeper layers inherit attention-order rounding, which can flip an int8
    # activation by one step; the caches stay close norm-wise
    for a, b in ((kg, kc), (vg, vc)):
        rel = np.linalg.norm(a[:, :, :n] - b[:, :, :n]) / np.linalg.norm(b[:, :, :n])
        assert rel < 2e-3, rel
    gpu.set_options(attn_splits=-1)


def test_generate_matches_forward(tiny_models):
    w, gpu, cpu = tiny_models
    e = cpu.embed(42)
    gpu.kv_len = 0
    toks_fwd = [gpu.forward(embed=e)]
    for _ in range(23):
        toks_fwd.append(gpu.forward(token=toks_fwd[-1]))
    for graph in (True, False):
        gpu.set_options(use_graph=graph)
        gpu.kv_len = 0
        toks = gpu.generate(24, first_embed=e)
        assert list(toks) == toks_fwd, graph
    gpu.set_options(use_graph=True)


def test_kv_cache_grows(dev):
    """KvCache::grow (decoder.rs:199-231): a decoder created with room for 256
    positions prefills 100 rows, generates 500 tokens in one call (the cache
    grows to 768 positions first), then decodes step by step past 768 (it
    doubles to 1536 on the way); a decoder created with 1024 positions and
    driven the same way gives the same tokens and, row for row, the same KV
    cache.  Capacity beyond 2^20 positions is refused before anything is
    allocated."""
    from qwenasr_amd import QasrError
    from qwenasr_amd.model import Decoder
    from qwenasr_amd.synth import SynthDecoder
    print("KV cache growth 256 -> 768 -> 1536", flush=True)
    w = SynthDecoder(TINY, seed=1021)
    prompt = (rng(1022).standard_normal((100, TINY["hidden"])) * 0.5).astype(np.float32)
    runs = []
    for cap0 in (256, 1024):
        d = Decoder(dev, w, max_seq=cap0)
        try:
            d.prefill(prompt)
            toks = list(d.generate(500, first_token=7))
            caps = [d.capacity]
            for _ in range(180):                      # positions 600..779
                toks.append(d.forward(token=toks[-1]))
            caps.append(d.capacity)
            k, v = d.kv_download()
            n = d.kv_len
            with pytest.raises(QasrError, match="capacity"):
                d.generate((1 << 20) + 1, first_token=1)
        finally:
            d.close()
        runs.append((toks, caps, k[:, :, :n], v[:, :, :n], n))
    (ta, ca, ka, va, na), (tb, cb, kb, vb, nb) = runs
    assert ca == [768, 1536] and cb == [1024, 1024], (ca, cb)
    assert na == nb == 780
    assert ta == tb
    assert ka.tobytes() == kb.tobytes() and va.tobytes() == vb.tobytes()
    assert len(set(ta)) > 10


@pytest.mark.parametrize("hidden,kv_bf16", [(1024, False), (1024, True), (2048, True)])
def test_fused_qkv_attention_bit_identical(dev, hidden, kv_bf16):
    """The qkv matvec and the decode attention as one launch (the qkv rows
    handed to the attention blocks as (tag, value) pairs) against the two
    launches: tokens and every KV row bit-identical, over a context that crosses
    the 256- and 512-position buckets (1-3 groups per wave), with graph replay
    and eagerly, 0.6B (K 1024) and 1.7B (K 2048) widths."""
    from qwenasr_amd.model import Decoder
    from qwenasr_amd.synth import SynthDecoder
    cfg = dict(TINY, hidden=hidden, intermediate=3 * hidden)
    print(f"fused qkv+attention hidden={hidden} kv_bf16={kv_bf16}", flush=True)
    w = SynthDecoder(cfg, seed=77)
    r = rng(78)
    prompt = (r.standard_normal((230, hidden)) * 0.5).astype(np.float32)
    kv = None
    runs = []
    for fuse, graph in ((True, True), (False, True), (True, False)):
        g = Decoder(dev, w, max_seq=1024, kv_bf16=kv_bf16)
        g.set_fusion(fuse)
        g.set_options(attn_splits=-1, use_graph=graph)
        if kv_bf16:
            # the prefill needs an f32 cache: 229 context rows of N(0, 1) instead
            if kv is None:
                kv = [r.standard_normal(g.kv_shape()).astype(np.float32) for _ in range(2)]
            g.kv_upload(*kv)
            g.kv_len = 229
        else:
            g.prefill(prompt[:-1])
        toks = g.generate(320, first_embed=prompt[-1])
        k, v = g.kv_download()
        runs.append((np.asarray(toks).copy(), k.copy(), v.copy()))
        g.close()
    n = 229 + 320

    def bits(a):
        return np.ascontiguousarray(a[:, :, :n]).view(np.uint8)

    for t, k, v in runs[1:]:
        assert (t == runs[0][0]).all()
        assert np.array_equal(bits(k), bits(runs[0][1]))
        assert np.array_equal(bits(v), bits(runs[0][2]))


@pytest.mark.parametrize("n_heads,n_kv_heads", [(2, 1), (32, 16), (16, 4)])
def test_decoder_load_rejects_other_attention_shapes(dev, n_heads, n_kv_heads):
    """Only the attention shape of both Qwen3-ASR decoders (16 query heads, 8
    KV heads of 128) loads: the decode step's split merges are laid out for
    it, so another shape is refused with QASR_ERR_INVALID before anything is
    allocated."""
    from qwenasr_amd import QasrError
    from qwenasr_amd.model import Decoder
    from qwenasr_amd.synth import SynthDecoder
    w = SynthDecoder(dict(n_layers=1, hidden=128, n_heads=n_heads, n_kv_heads=n_kv_heads, head_dim=128,
                          intermediate=128, vocab=64, eps=1e-6, theta=1e6), seed=5)
    with pytest.raises(QasrError, match="16 query heads"):
        Decoder(dev, w, max_seq=64)

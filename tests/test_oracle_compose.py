"""CPU pins of the oracle's model compositions against the independent
float64 restatement in ref64.py (decoder.rs:455-645, encoder.rs:186-358,
transcribe.rs:13-15 and 63-247).

The pieces (quantizers, matvecs, norms, RoPE, attention, GELU, PE, conv, mel)
are pinned one by one in test_oracle_int8.py / test_oracle_float.py; these
tests pin how the oracle wires them together: the q/k norm -> RoPE -> KV
write order, the residual placement, the GQA head map, positions after a
partial prefill, the final norm and tied LM head, the encoder's per-chunk
conv stem, the [C, 16, w3] -> [w3, 16 C] reshape, the per-chunk PE, the
attention window starts, and the 15-token prompt around the audio rows.

Tolerances.  Prefill and encoder are float paths: f32 against float64 over
two layers measures 2-3e-7 relative (norm-wise); the bar is 1e-5.  The decode
step re-quantizes every activation to int8, so an f32-vs-float64 difference
of one ulp could move an element across a rounding boundary and shift one
product by ~1/127 of its scale; the seeded case has no such flip (3e-7) and
the bar is 2e-5 on the final hidden state and the KV rows, with tokens
compared only where the top-2 logit gap is clear.  Each test_planted_* case
changes the restatement in one plausible way (a wrong GQA map, an
off-by-one RoPE position, a residual from the normed row, a PE counted
across chunks, features flattened in the wrong order, no attention windows,
a prompt missing its tail or with swapped audio markers) and shows the same
comparison then fails by 3 to 6 orders of magnitude (2.8e-2 to 1.25).
"""
import numpy as np
import pytest

import ref64
from conftest import rng

DEC = dict(n_layers=2, hidden=256, n_heads=4, n_kv_heads=2, head_dim=64, intermediate=512, vocab=1024,
           eps=1e-6, theta=1e6)
# n_window_infer 200 -> 26-token windows: a 250-frame input has chunks of 100, 100 and 50
# frames (13, 13 and 7 tokens) and windows [0, 26), [26, 33)
ENC = dict(d_model=64, n_layers=2, n_heads=4, head_dim=16, ffn_dim=128, output_dim=256, chunk_size=100,
           n_window_infer=200, conv_hidden=32)


def rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / np.linalg.norm(b))


def with_gains(w, seed):
    """Distinct non-unit norm gains, so swapped or dropped norms show."""
    r = rng(seed)
    g = lambda n: r.uniform(0.5, 1.5, n).astype(np.float32)
    c = w.cfg
    for L in w.layers:
        L["input_norm"], L["post_attn_norm"] = g(c["hidden"]), g(c["hidden"])
        L["q_norm"], L["k_norm"] = g(c["head_dim"]), g(c["head_dim"])
    w.norm = g(c["hidden"])
    return w


def enc_with_params(w, seed):
    r = rng(seed)
    D, F, Cc, O = w.cfg["d_model"], w.cfg["ffn_dim"], w.cfg["conv_hidden"], w.cfg["output_dim"]
    b = lambda n: r.normal(0, 0.05, n).astype(np.float32)
    g = lambda n: r.uniform(0.5, 1.5, n).astype(np.float32)
    w.conv1_b, w.conv2_b, w.conv3_b = b(Cc), b(Cc), b(Cc)
    for L in w.layers:
        for k in ("bq", "bk", "bv", "bo"):
            L[k] = b(D)
        L["b1"], L["b2"] = b(F), b(D)
        L["ln1_w"], L["ln1_b"], L["ln2_w"], L["ln2_b"] = g(D), b(D), g(D), b(D)
    w.ln_post_w, w.ln_post_b = g(D), b(D)
    w.proj1_b, w.proj2_b = b(D), b(O)
    return w


@pytest.fixture(scope="module")
def dec_w():
    from qwenasr_amd.synth import SynthDecoder
    return with_gains(SynthDecoder(DEC, seed=2101, std=0.05), 2102)


@pytest.fixture(scope="module")
def enc_w():
    from qwenasr_amd.synth import SynthEncoder
    return enc_with_params(SynthEncoder(ENC, seed=2103, std=0.05), 2104)


# ---------------------------------------------------------------- decoder

def prefill_err(orc, w, ref_cls=ref64.Decoder64, start=0, S=20):
    e = rng(2105).normal(0, 1, (start + S, DEC["hidden"])).astype(np.float32)
    o = orc.OracleDecoder(w, max_seq=64)
    r = ref_cls(w, 64)
    if start:
        o.prefill(e[:start])
        r.prefill(e[:start])
    got = o.prefill_hidden(e[start:])
    want = r.prefill(e[start:])
    k, v = o.kv()
    n = start + S
    errs = (rel(got, want), rel(k[:, :, :n], r.K[:, :, :n]), rel(v[:, :, :n], r.V[:, :, :n]))
    o.close()
    return errs


@pytest.mark.parametrize("start", [0, 7])
def test_prefill_composition(orc, dec_w, start):
    """decoder_prefill (decoder.rs:455-547): last-layer rows and every KV row,
    from an empty cache and after a 7-row prefill (positions continue)."""
    h, k, v = prefill_err(orc, dec_w, start=start)
    assert h < 1e-5 and k < 1e-5 and v < 1e-5, (h, k, v)


def decode_run(orc, w, ref_cls=ref64.Decoder64, steps=12):
    """Prefill 9 rows, then teacher-forced steps fed the oracle's tokens:
    (max error of the hidden state and of the KV rows written, tokens
    compared, tokens equal).  The KV rows matter: RoPE is relative, so a
    position shift common to all rows leaves the hidden state unchanged."""
    e = rng(2106).normal(0, 1, (10, DEC["hidden"])).astype(np.float32)
    o = orc.OracleDecoder(w, max_seq=64)
    r = ref_cls(w, 64)
    o.prefill(e[:9])
    r.prefill(e[:9])
    emb = e[9]
    worst, compared, equal = 0.0, 0, 0
    for _ in range(steps):
        t_o, m_o, h_o = o.forward(emb, return_hidden=True)
        t_r, m_r, h_r = r.forward(emb.astype(np.float64))
        worst = max(worst, rel(h_o, h_r))
        if m_r > 1e-2 * np.abs(h_r).max():           # a clear top-2 gap
            compared += 1
            equal += t_o == t_r
        emb = o.embed(t_o)
    k, v = o.kv()
    n = r.len
    worst = max(worst, rel(k[:, :, :n], r.K[:, :, :n]), rel(v[:, :, :n], r.V[:, :, :n]))
    o.close()
    return worst, compared, equal


def test_decode_composition(orc, dec_w):
    """decoder_forward (decoder.rs:550-645): norm -> int8 qkv -> q/k norm ->
    RoPE -> KV write -> GQA attention -> o += -> norm -> gate/up SwiGLU ->
    down += -> final norm -> int8 argmax over the tied head."""
    worst, compared, equal = decode_run(orc, dec_w)
    assert worst < 2e-5, worst
    assert compared >= 8 and equal == compared, (compared, equal)


# ---------------------------------------------------------------- encoder

def enc_err(orc, w, ref_cls=ref64.Encoder64, frames=250):
    mel = rng(2107).normal(-0.5, 0.4, (128, frames)).astype(np.float32)
    o = orc.OracleEncoder(w)
    got = o.forward(mel)
    want, starts = ref_cls(w).forward(mel)
    o.close()
    return rel(got, want), starts


def test_encoder_composition(orc, enc_w):
    """Encoder::forward (encoder.rs:186-358) over three chunks (the last one
    ragged) and two attention windows."""
    err, starts = enc_err(orc, enc_w)
    assert starts == [0, 26, 33]
    assert err < 1e-5, err


def test_encoder_tokens(orc, enc_w):
    o = orc.OracleEncoder(enc_w)
    from oracle.oracle import lib
    for frames, want in ((100, 13), (101, 14), (150, 20), (250, 33), (3000, 390), (7, 1)):
        assert lib().or_encoder_tokens(o.e, frames) == want, frames
    o.close()


# ---------------------------------------------------------------- prompt

TDEC = dict(n_layers=2, hidden=128, n_heads=2, n_kv_heads=1, head_dim=64, intermediate=256, vocab=151936,
            eps=1e-6, theta=1e6)
TENC = dict(ENC, output_dim=128)


@pytest.fixture(scope="module")
def tiny_models():
    from qwenasr_amd.synth import SynthDecoder, SynthEncoder, audio
    wd = with_gains(SynthDecoder(TDEC, seed=2108, std=0.05), 2109)
    we = enc_with_params(SynthEncoder(TENC, seed=2110, std=0.05), 2111)
    return wd, we, audio(24000, 2112)


def transcribe_check(orc, models, dec_cls=ref64.Decoder64, prompt=ref64.prompt_embeds, steps=6, ids=None):
    wd, we, x = models
    ids = ids or {}
    o_d, o_e = orc.OracleDecoder(wd, max_seq=128), orc.OracleEncoder(we)
    res = orc.transcribe_forced(o_d, o_e, x, steps, **ids)
    o_d.close()
    o_e.close()
    d = dec_cls(wd, 128)
    rows, _ = ref64.Encoder64(we).forward(orc.mel(x))
    emb = prompt(d, rows, **ids)
    assert res["prompt_len"] == emb.shape[0]
    d.prefill(emb[:-1])
    tok, margin, _ = d.forward(emb[-1])
    agree = []
    for s in range(steps):
        if margin <= 1e-3:                                # unclear gap: stop comparing
            break
        agree.append(tok == res["tokens"][s])
        tok, margin, _ = d.forward(d.embed(res["tokens"][s]))
    return agree


def test_transcribe_prompt_layout(orc, tiny_models):
    """or_transcribe_forced: mel -> encoder -> [PREFIX_HEAD, PREFIX_TAIL,
    audio rows, SUFFIX_BASE] (transcribe.rs:13-15, 106-169) -> prefill of all
    but the last row -> the first token from the last row -> greedy steps."""
    agree = transcribe_check(orc, tiny_models)
    assert len(agree) >= 4 and all(agree), agree


PROMPT_IDS = dict(prompt=[9707, 11, 1879], force=[11528, 6364, 151704], past=[40, 1079, 264, 1273])


@pytest.mark.parametrize("keys", [("prompt",), ("force",), ("past",), ("prompt", "force", "past")])
def test_transcribe_prompt_ids(orc, tiny_models, keys):
    """or_transcribe_prompt: the text prompt's ids between PREFIX_HEAD and
    PREFIX_TAIL, the forced-language ids (ending in <asr_text>) after
    SUFFIX_BASE, the previous segments' text ids and a closing <asr_text>
    after those (transcribe.rs:97-169); or_prompt_ids lists the same rows."""
    ids = {k: PROMPT_IDS[k] for k in keys}
    agree = transcribe_check(orc, tiny_models, ids=ids)
    assert len(agree) >= 4 and all(agree), (keys, agree)
    head, tail = orc.prompt_ids(**ids)
    p, f, q = (ids.get(k, []) for k in ("prompt", "force", "past"))
    assert head.tolist() == ref64.PREFIX_HEAD + p + ref64.PREFIX_TAIL
    assert tail.tolist() == ref64.SUFFIX_BASE + f + (q + [ref64.ASR_TEXT] if q else [])


# ---------------------------------------------------------------- planted mistakes

class WrongGqa(ref64.Decoder64):
    def _attend(self, l, q, pos):
        c = self.c
        out = np.empty_like(q)
        for h in range(c["n_heads"]):
            kv = h % c["n_kv_heads"]                      # interleaved instead of h / heads_per_kv
            s = self.K[l, kv, :pos + 1] @ q[h] / np.sqrt(c["head_dim"])
            p = np.exp(s - s.max())
            out[h] = (p / p.sum()) @ self.V[l, kv, :pos + 1]
        return out


class RopeOffByOne(ref64.Decoder64):
    def _qk(self, L, q, k, positions):
        return super()._qk(L, q, k, np.asarray(positions) + 1)


class NormedResidual(ref64.Decoder64):
    def prefill(self, embeds):
        c = self.c
        x = np.asarray(embeds, np.float64).copy()
        S = x.shape[0]
        pos = np.arange(self.len, self.len + S)
        for l, L in enumerate(self.L):
            xn = ref64.rms(x, L["in_norm"], c["eps"])
            q, k = self._qk(L, xn @ L["wq"].T, xn @ L["wk"].T, pos)
            v = (xn @ L["wv"].T).reshape(S, c["n_kv_heads"], -1)
            self.K[l, :, pos] = k
            self.V[l, :, pos] = v
            att = np.stack([self._attend(l, q[s], p).reshape(-1) for s, p in enumerate(pos)])
            x = xn + att @ L["wo"].T                      # residual from the normed row
            xn = ref64.rms(x, L["post_norm"], c["eps"])
            x = x + (ref64.silu(xn @ L["gate"].T) * (xn @ L["up"].T)) @ L["down"].T
        self.len += S
        return x


def test_planted_decoder_mistakes(orc, dec_w):
    for cls in (WrongGqa, RopeOffByOne, NormedResidual):
        h, k, _ = prefill_err(orc, dec_w, ref_cls=cls, start=7)
        assert max(h, k) > 1e-2, (cls.__name__, h, k)
    for cls in (WrongGqa, RopeOffByOne):
        worst, _, _ = decode_run(orc, dec_w, ref_cls=cls, steps=3)
        assert worst > 1e-2, (cls.__name__, worst)


class GlobalPe(ref64.Encoder64):
    """PE positions counted across chunks instead of restarting per chunk."""
    def forward(self, mel):
        self.seen = 0
        return super().forward(mel)

    def _pe(self, n, d):
        pe = ref64.sinusoidal_pe(self.seen + n, d)[self.seen:]
        self.seen += n
        return pe


class FeatFMajor(ref64.Encoder64):
    """conv features flattened f-major (column f * C + ch)."""
    @staticmethod
    def _feat(a):
        Cc, h3, w3 = a.shape
        return a.transpose(2, 1, 0).reshape(w3, Cc * h3)


class NoWindows(ref64.Encoder64):
    @staticmethod
    def _windows(T, wts):
        return [0, T]


def test_planted_encoder_mistakes(orc, enc_w):
    for cls in (GlobalPe, FeatFMajor, NoWindows):
        err, _ = enc_err(orc, enc_w, ref_cls=cls)
        assert err > 1e-2, (cls.__name__, err)


def test_planted_prompt_mistake(orc, tiny_models):
    def no_tail(dec, rows):
        toks = [dec.embed(t) for t in ref64.PREFIX_HEAD]
        return np.concatenate([np.stack(toks), rows, np.stack([dec.embed(t) for t in ref64.SUFFIX_BASE])])
    with pytest.raises(AssertionError):
        transcribe_check(orc, tiny_models, prompt=no_tail)

    def swapped_audio_markers(dec, rows):                 # 151669 after the audio, 151670 before
        head = [dec.embed(t) for t in ref64.PREFIX_HEAD + ref64.PREFIX_TAIL[:-1] + [151670]]
        tail = [dec.embed(t) for t in [151669] + ref64.SUFFIX_BASE[1:]]
        return np.concatenate([np.stack(head), rows, np.stack(tail)])
    agree = transcribe_check(orc, tiny_models, prompt=swapped_audio_markers)
    assert len(agree) >= 1 and not all(agree), agree


def test_planted_prompt_id_mistakes(orc, tiny_models):
    """The prompt-id comparison fails when the restatement puts the forced
    language before SUFFIX_BASE, or opens the past text with <asr_text>
    instead of closing it (both keep the prompt length)."""
    def rows_of(dec, head, rows, tail):
        return np.concatenate([np.stack([dec.embed(t) for t in head]), rows, np.stack([dec.embed(t) for t in tail])])

    def force_first(dec, rows, prompt=(), force=(), past=()):
        return rows_of(dec, ref64.PREFIX_HEAD + ref64.PREFIX_TAIL, rows, list(force) + ref64.SUFFIX_BASE)

    def past_opened(dec, rows, prompt=(), force=(), past=()):
        return rows_of(dec, ref64.PREFIX_HEAD + ref64.PREFIX_TAIL, rows,
                       ref64.SUFFIX_BASE + [ref64.ASR_TEXT] + list(past))
    for bad, key in ((force_first, "force"), (past_opened, "past")):
        agree = transcribe_check(orc, tiny_models, prompt=bad, ids={key: PROMPT_IDS[key]})
        assert len(agree) >= 1 and not all(agree), (key, agree)



def test_kv_bf16_mode(orc, dec_w):
    """or_decoder_set_kv_bf16 (this build's config-3 cache, not the
    reference's): the rows it stores are the f32 mode's rows rounded to bf16
    (round to nearest even, conftest.bf16), and the rows already in the cache
    are what attention reads."""
    from conftest import bf16, bf16f
    e = rng(2120).normal(0, 1, (6, DEC["hidden"])).astype(np.float32)
    a = orc.OracleDecoder(dec_w, max_seq=16)
    b = orc.OracleDecoder(dec_w, max_seq=16, kv_bf16=True)
    a.prefill(e[:5])
    b.prefill(e[:5])
    ka, va = a.kv()
    kb, vb = b.kv()
    # layer 0 sees the same inputs in both modes
    assert (kb[0, :, :5] == bf16f(bf16(ka[0, :, :5]))).all() and (vb[0, :, :5] == bf16f(bf16(va[0, :, :5]))).all()
    assert not (kb[0, :, :5] == ka[0, :, :5]).all()
    a.forward(e[5])
    b.forward(e[5])
    ka, va = a.kv()
    kb, vb = b.kv()
    assert (vb[0, :, 5] == bf16f(bf16(va[0, :, 5]))).all()
    assert (kb[1, :, :6] == bf16f(bf16(kb[1, :, :6]))).all()     # every stored value is a bf16 value
    a.close()
    b.close()

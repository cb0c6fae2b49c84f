"""Independent float64 restatement of the reference's model compositions.

Test infrastructure: it pins the oracle's decoder step, prefill, encoder and
offline prompt layout (oracle/oracle.c) from a second, differently written
source.  It is vectorised numpy in float64, written from the reference's
Rust (paths relative to crates/qwen-asr/src/), and shares no code with the
oracle:

* gate and up are separate matrices here (the oracle and the reference
  interleave their rows before quantizing, decoder.rs:91-104);
* attention is a full softmax over the visible keys (the reference and the
  oracle run an online softmax, kernels/mod.rs:1508-1535);
* the convolution is a direct 3x3 sum (the reference runs im2col + sgemm,
  kernels/mod.rs:1077-1154);
* RoPE angles, the sinusoidal PE and GELU are evaluated in float64 from their
  formulas (the reference builds f32 tables with powf/cosf/sinf and uses an
  AVX polynomial exp).

Only the int8 quantizers keep float32 arithmetic, because their rounding
decisions are the definition of the int8 path (kernels/mod.rs:1795-1829);
they are pinned bit for bit elsewhere (test_oracle_int8.py).  Every integer
dot product is exact (int64).
"""
import numpy as np


def bf(a):
    """bf16 bit patterns (uint16) -> float64 (exact)."""
    return (np.asarray(a, np.uint16).astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def _round_half_away(v):
    return np.sign(v) * np.floor(np.abs(v) + 0.5)


def quant_rows(w_bf16):
    """Per-row symmetric int8 of bf16 rows (mod.rs:1805-1829, round mode)."""
    w = (np.asarray(w_bf16, np.uint16).astype(np.uint32) << 16).view(np.float32)
    m = np.max(np.abs(w), axis=1)
    scale = np.where(m > 0, m / np.float32(127.0), np.float32(1.0)).astype(np.float32)
    inv = (np.float32(127.0) / np.maximum(m, np.float32(1e-10))).astype(np.float32)
    q = np.clip(_round_half_away(w * inv[:, None]), -127, 127).astype(np.int64)
    return q, scale.astype(np.float64)


def quant_act(x):
    """Activation int8 (mod.rs:1795-1802): f32 absmax, roundf, clamp."""
    x32 = np.asarray(x, np.float64).astype(np.float32)
    m = np.float32(np.max(np.abs(x32)))
    scale = np.float32(m / np.float32(127.0)) if m > 0 else np.float32(1.0)
    inv = np.float32(np.float32(127.0) / np.float32(max(m, np.float32(1e-10))))
    q = np.clip(_round_half_away(x32 * inv), -127, 127).astype(np.int64)
    return q, float(scale)


def int8_linear(x, packed):
    """y = (acc * x_scale) * w_scale (mod.rs:839-880) for one activation vector."""
    q, s = packed
    xq, xs = quant_act(x)
    return (q @ xq).astype(np.float64) * xs * s


def rms(x, w, eps):
    x = np.asarray(x, np.float64)
    r = 1.0 / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)
    return x * r * np.asarray(w, np.float64)


def layer_norm(x, w, b, eps=1e-5):
    x = np.asarray(x, np.float64)
    mu = x.mean(axis=-1, keepdims=True)
    var = ((x - mu) ** 2).mean(axis=-1, keepdims=True)
    return (x - mu) / np.sqrt(var + eps) * np.asarray(w, np.float64) + np.asarray(b, np.float64)


def rope(x, positions, theta):
    """NeoX RoPE (decoder.rs:302-338, mod.rs:1780-1788) on x [S, heads, hd]."""
    hd = x.shape[-1]
    half = hd // 2
    inv = theta ** (-np.arange(half, dtype=np.float64) * 2.0 / hd)
    ang = np.asarray(positions, np.float64)[:, None] * inv[None, :]
    c, s = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]
    x1, x2 = x[..., :half], x[..., half:]
    return np.concatenate([x1 * c - x2 * s, x2 * c + x1 * s], axis=-1)


def gelu(x):
    """tanh-GELU (mod.rs:1250-1289 generic branch) in float64."""
    return 0.5 * x * (1.0 + np.tanh(0.7978845608028654 * (x + 0.044715 * x ** 3)))


def silu(g):
    return g / (1.0 + np.exp(-g))


def sinusoidal_pe(n_pos, d):
    """mod.rs:1704-1717: sin in the first half, cos in the second."""
    half = d // 2
    lt = np.log(10000.0) / (half - 1)
    ang = np.arange(n_pos, dtype=np.float64)[:, None] * np.exp(-np.arange(half, dtype=np.float64) * lt)[None, :]
    return np.concatenate([np.sin(ang), np.cos(ang)], axis=1)


def conv3x3_s2(x, w, b):
    """Conv2d 3x3, stride 2, padding 1 (mod.rs:1077-1154), direct sum.
    x [cin, h, w], w [cout, cin, 3, 3] -> [cout, ho, wo]."""
    cin, h, wd = x.shape
    ho, wo = (h - 1) // 2 + 1, (wd - 1) // 2 + 1
    xp = np.zeros((cin, h + 2, wd + 2))
    xp[:, 1:h + 1, 1:wd + 1] = x
    out = np.zeros((w.shape[0], ho, wo))
    for ki in range(3):
        for kj in range(3):
            patch = xp[:, ki:ki + 2 * ho:2, kj:kj + 2 * wo:2]          # [cin, ho, wo]
            out += np.einsum("oc,chw->ohw", w[:, :, ki, kj], patch)
    return out + np.asarray(b, np.float64)[:, None, None]


class Decoder64:
    """decoder_prefill / decoder_forward (decoder.rs:455-645) in float64."""

    def __init__(self, sw, max_seq):
        self.c = c = sw.cfg
        self.sw = sw
        self.max_seq = max_seq
        H, hd = c["hidden"], c["head_dim"]
        self.L = []
        for L in sw.layers:
            self.L.append(dict(
                wq=bf(L["wq"]), wk=bf(L["wk"]), wv=bf(L["wv"]), wo=bf(L["wo"]),
                gate=bf(L["gate"]), up=bf(L["up"]), down=bf(L["down"]),
                iq=quant_rows(L["wq"]), ik=quant_rows(L["wk"]), iv=quant_rows(L["wv"]),
                io=quant_rows(L["wo"]), ig=quant_rows(L["gate"]), iu=quant_rows(L["up"]),
                idn=quant_rows(L["down"]),
                q_norm=np.asarray(L["q_norm"], np.float64), k_norm=np.asarray(L["k_norm"], np.float64),
                in_norm=np.asarray(L["input_norm"], np.float64),
                post_norm=np.asarray(L["post_attn_norm"], np.float64)))
        self.norm = np.asarray(sw.norm, np.float64)
        self.lm = quant_rows(sw.embed)                       # tied head (decoder.rs:145-157)
        self.K = np.zeros((c["n_layers"], c["n_kv_heads"], max_seq, hd))
        self.V = np.zeros_like(self.K)
        self.len = 0

    def embed(self, tok):
        return bf(self.sw.embed[tok])

    def _attend(self, l, q, pos):
        """q [Hq, hd] at absolute position pos: keys 0..pos of layer l."""
        c = self.c
        g = c["n_heads"] // c["n_kv_heads"]
        out = np.empty_like(q)
        for h in range(c["n_heads"]):
            kv = h // g                                     # mod.rs:1494
            k = self.K[l, kv, :pos + 1]
            v = self.V[l, kv, :pos + 1]
            s = k @ q[h] / np.sqrt(c["head_dim"])
            p = np.exp(s - s.max())
            out[h] = (p / p.sum()) @ v
        return out

    def _qk(self, L, q, k, positions):
        c = self.c
        S = q.shape[0]
        q = rms(q.reshape(S, c["n_heads"], -1), L["q_norm"], c["eps"])
        k = rms(k.reshape(S, c["n_kv_heads"], -1), L["k_norm"], c["eps"])
        return rope(q, positions, c["theta"]), rope(k, positions, c["theta"])

    def prefill(self, embeds):
        """Returns the last layer's rows (before the final norm) [S, H]."""
        c = self.c
        x = np.asarray(embeds, np.float64).copy()
        S = x.shape[0]
        pos = np.arange(self.len, self.len + S)
        for l, L in enumerate(self.L):
            xn = rms(x, L["in_norm"], c["eps"])
            q, k = self._qk(L, xn @ L["wq"].T, xn @ L["wk"].T, pos)
            v = (xn @ L["wv"].T).reshape(S, c["n_kv_heads"], -1)
            self.K[l, :, pos] = k
            self.V[l, :, pos] = v
            att = np.stack([self._attend(l, q[s], p).reshape(-1) for s, p in enumerate(pos)])
            x = x + att @ L["wo"].T
            xn = rms(x, L["post_norm"], c["eps"])
            x = x + (silu(xn @ L["gate"].T) * (xn @ L["up"].T)) @ L["down"].T
        self.len += S
        return x

    def forward(self, embed):
        """One decode step: (token, best - second logit, final-normed hidden)."""
        c = self.c
        x = np.asarray(embed, np.float64).copy()
        pos = self.len
        for l, L in enumerate(self.L):
            xn = rms(x, L["in_norm"], c["eps"])
            q, k = self._qk(L, int8_linear(xn, L["iq"])[None], int8_linear(xn, L["ik"])[None], [pos])
            v = int8_linear(xn, L["iv"]).reshape(c["n_kv_heads"], -1)
            self.K[l, :, pos] = k[0]
            self.V[l, :, pos] = v
            att = self._attend(l, q[0], pos).reshape(-1)
            x = x + int8_linear(att, L["io"])
            xn = rms(x, L["post_norm"], c["eps"])
            g, u = int8_linear(xn, L["ig"]), int8_linear(xn, L["iu"])
            x = x + int8_linear(silu(g) * u, L["idn"])
        self.len = pos + 1
        xn = rms(x, self.norm, c["eps"])
        logits = int8_linear(xn, self.lm)
        top = np.argsort(-logits, kind="stable")[:2]
        return int(top[0]), float(logits[top[0]] - logits[top[1]]), xn


class Encoder64:
    """Encoder::forward (encoder.rs:186-358) in float64."""

    def __init__(self, sw):
        self.c = sw.cfg
        self.sw = sw

    @staticmethod
    def _feat(a):
        """[C, h3, w3] -> [w3, C * h3], column ch * h3 + f (encoder.rs:265-277)."""
        Cc, h3, w3 = a.shape
        return a.transpose(2, 0, 1).reshape(w3, Cc * h3)

    @staticmethod
    def _pe(n, d):
        """PE restarted at position 0 in every chunk (encoder.rs:283-286)."""
        return sinusoidal_pe(n, d)

    @staticmethod
    def _windows(T, wts):
        """Window starts every wts tokens, then T (encoder.rs:291-298)."""
        return list(range(0, T, wts)) + [T]

    def forward(self, mel):
        c, w = self.c, self.sw
        D, cs = c["d_model"], c["chunk_size"]
        frames = mel.shape[1]
        out_len = lambda n: (n - 1) // 2 + 1                  # (n + 2 - 3) / 2 + 1
        rows = []
        for st in range(0, frames, cs):
            m = np.asarray(mel[:, st:st + cs], np.float64)[None]           # [1, 128, cw]
            a = gelu(conv3x3_s2(m, bf(w.conv1_w), w.conv1_b))
            a = gelu(conv3x3_s2(a, bf(w.conv2_w), w.conv2_b))
            a = gelu(conv3x3_s2(a, bf(w.conv3_w), w.conv3_b))                # [C, h3, w3]
            rows.append(self._feat(a) @ bf(w.conv_out_w).T + self._pe(a.shape[2], D))
        x = np.concatenate(rows)
        T = x.shape[0]
        tpc = out_len(out_len(out_len(cs)))
        starts = self._windows(T, tpc * (c["n_window_infer"] // cs))
        nh, hd = c["n_heads"], c["head_dim"]
        for L in w.layers:
            xn = layer_norm(x, L["ln1_w"], L["ln1_b"])
            q = (xn @ bf(L["wq"]).T + L["bq"]).reshape(T, nh, hd)
            k = (xn @ bf(L["wk"]).T + L["bk"]).reshape(T, nh, hd)
            v = (xn @ bf(L["wv"]).T + L["bv"]).reshape(T, nh, hd)
            att = np.empty_like(q)
            for a0, a1 in zip(starts[:-1], starts[1:]):
                s = np.einsum("ihd,jhd->hij", q[a0:a1], k[a0:a1]) / np.sqrt(hd)
                p = np.exp(s - s.max(axis=-1, keepdims=True))
                p /= p.sum(axis=-1, keepdims=True)
                att[a0:a1] = np.einsum("hij,jhd->ihd", p, v[a0:a1])
            x = x + att.reshape(T, -1) @ bf(L["wo"]).T + L["bo"]
            xn = layer_norm(x, L["ln2_w"], L["ln2_b"])
            x = x + gelu(xn @ bf(L["fc1"]).T + L["b1"]) @ bf(L["fc2"]).T + L["b2"]
        x = layer_norm(x, w.ln_post_w, w.ln_post_b)
        x = gelu(x @ bf(w.proj1_w).T + w.proj1_b)
        return x @ bf(w.proj2_w).T + w.proj2_b, starts


# transcribe.rs:13-15
PREFIX_HEAD = [151644, 8948, 198]
PREFIX_TAIL = [151645, 198, 151644, 872, 198, 151669]
SUFFIX_BASE = [151670, 151645, 198, 151644, 77091, 198]


ASR_TEXT = 151704


def prompt_embeds(dec, enc_rows, prompt=(), force=(), past=()):
    """transcribe.rs:97-169: PREFIX_HEAD, the text prompt's ids, PREFIX_TAIL,
    the audio rows, SUFFIX_BASE, the forced-language ids, and the previous
    segments' text ids closed by <asr_text> when there are any."""
    head = PREFIX_HEAD + [int(t) for t in prompt] + PREFIX_TAIL
    tail = SUFFIX_BASE + [int(t) for t in force] + ([int(t) for t in past] + [ASR_TEXT] if len(past) else [])
    return np.concatenate([np.stack([dec.embed(t) for t in head]), enc_rows,
                           np.stack([dec.embed(t) for t in tail])])


def transcribe_forced(dec, enc, mel, n_steps):
    """transcribe.rs:63-247 with a forced step count: (tokens, margins)."""
    rows, _ = enc.forward(mel)
    emb = prompt_embeds(dec, rows)
    dec.len = 0
    dec.prefill(emb[:-1])
    tok, margin, _ = dec.forward(emb[-1])
    toks, margins = [tok], [margin]
    for _ in range(n_steps - 1):
        tok, margin, _ = dec.forward(dec.embed(tok))
        toks.append(tok)
        margins.append(margin)
    return toks, margins

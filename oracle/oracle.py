"""ctypes wrapper of liboracle.so — the CPU restatement of the reference path.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, and only as the checker.  Built by
``make -C oracle`` (driven by __graft_entry__.build()).
"""
import ctypes as C
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(_HERE, "liboracle.so")
P, I64, I32, F32 = C.c_void_p, C.c_int64, C.c_int32, C.c_float

ROUND, TRUNC = 0, 1


class DecConfig(C.Structure):
    _fields_ = [("n_layers", I32), ("hidden", I32), ("n_heads", I32), ("n_kv_heads", I32),
                ("head_dim", I32), ("intermediate", I32), ("vocab", I32),
                ("eps", F32), ("theta", F32)]


class DecLayer(C.Structure):
    _fields_ = [(n, P) for n in ("wq", "wk", "wv", "wo", "gate", "up", "down",
                                  "q_norm", "k_norm", "input_norm", "post_attn_norm")]


class DecWeights(C.Structure):
    _fields_ = [("embed", P), ("norm", P), ("layers", C.POINTER(DecLayer))]


class EncConfig(C.Structure):
    _fields_ = [(n, I32) for n in ("d_model", "n_layers", "n_heads", "head_dim", "ffn_dim",
                                    "output_dim", "chunk_size", "n_window_infer", "conv_hidden")]


class EncLayer(C.Structure):
    _fields_ = [(n, P) for n in ("wq", "wk", "wv", "wo", "fc1", "fc2", "bq", "bk", "bv", "bo",
                                  "b1", "b2", "ln1_w", "ln1_b", "ln2_w", "ln2_b")]


class EncWeights(C.Structure):
    _fields_ = ([(n, P) for n in ("conv1_w", "conv2_w", "conv3_w", "conv_out_w",
                                   "conv1_b", "conv2_b", "conv3_b")]
                + [("layers", C.POINTER(EncLayer))]
                + [(n, P) for n in ("ln_post_w", "ln_post_b", "proj1_w", "proj2_w",
                                     "proj1_b", "proj2_b")])


_SIGS = {
    "or_quantize_bf16_rows": (None, [P, I64, I64, C.c_int, P, P]),
    "or_quantize_act": (F32, [P, I64, P]),
    "or_matvec_w8a8": (None, [P, P, F32, P, P, P, I64, I64]),
    "or_linear_int8": (None, [P, P, P, P, P, I64, I64]),
    "or_linear_int8_qkv": (None, [P, P, P, P, P, P, P, P, P, P, I64, I64, I64]),
    "or_linear_int8_swiglu": (None, [P, P, P, P, I64, I64]),
    "or_linear_int8_addto": (None, [P, P, P, P, I64, I64]),
    "or_argmax_int8": (I64, [P, P, P, I64, I64, P, P]),
    "or_argmax_f32_rows": (None, [P, I64, I64, P]),
    "or_hsum8": (F32, [P]),
    "or_dot_f32": (F32, [P, P, I64]),
    "or_rms_norm": (None, [P, P, P, I64, I64, F32]),
    "or_rms_norm_per_head": (None, [P, P, I64, I64, I64, F32]),
    "or_rope_table": (None, [P, P, I64, I64, F32]),
    "or_apply_rope": (None, [P, P, P, I64, I64, I64]),
    "or_causal_attention": (None, [P, P, P, P, I64, I64, I64, I64, I64, I64, F32, I64]),
    "or_bidir_attention": (None, [P, P, P, P, I64, I64, I64, F32, P, I64]),
    "or_fast_exp": (F32, [F32]),
    "or_swiglu_rows": (None, [P, P, I64, I64]),
    "or_gelu": (None, [P, I64]),
    "or_layer_norm": (None, [P, P, P, P, I64, I64, F32]),
    "or_sinusoidal_pe": (None, [P, I64, I64]),
    "or_sgemm_nt": (None, [I64, I64, I64, P, I64, P, I64, P, I64, C.c_int]),
    "or_linear": (None, [P, P, P, P, I64, I64, I64]),
    "or_linear_accumulate": (None, [P, P, P, P, I64, I64, I64]),
    "or_conv2d": (None, [P, P, P, P, I64, I64, I64, I64, I64, I64, I64, I64]),
    "or_bf16_to_f32": (None, [P, P, I64]),
    "or_mel_frames": (I64, [I64]),
    "or_mel": (I64, [P, I64, P]),
    "or_decoder_create": (P, [C.POINTER(DecConfig), C.POINTER(DecWeights), C.c_int, I64]),
    "or_decoder_destroy": (None, [P]),
    "or_decoder_packed": (P, [P, C.c_int, C.c_int, C.POINTER(P)]),
    "or_decoder_set_len": (None, [P, I64]),
    "or_decoder_set_kv_bf16": (None, [P, C.c_int]),
    "or_decoder_len": (I64, [P]),
    "or_decoder_prefill": (None, [P, P, I64]),
    "or_decoder_prefill_logits": (None, [P, P, I64, P, I64, P]),
    "or_decoder_prefill_hidden": (None, [P, P, I64, P]),
    "or_decoder_forward": (I32, [P, P, P, P, P]),
    "or_embed_token": (None, [P, I32, P]),
    "or_decoder_kv": (P, [P, C.c_int]),
    "or_encoder_create": (P, [C.POINTER(EncConfig), C.POINTER(EncWeights)]),
    "or_encoder_destroy": (None, [P]),
    "or_encoder_tokens": (I64, [P, I64]),
    "or_encoder_forward": (I64, [P, P, I64, P]),
    "or_transcribe_forced": (I64, [P, P, P, I64, I32, P, P, P]),
    "or_transcribe_prompt": (I64, [P, P, P, I64, P, I64, P, I64, P, I64, I32, P, P, P]),
    "or_prompt_ids": (I64, [P, I64, P, I64, P, I64, P, P, P, P]),
    "or_find_split_point": (I64, [P, I64, I64, C.c_float]),
    "or_segment_splits": (I64, [P, I64, C.c_float, C.c_float, P, I64]),
    "or_stream_set_prompt": (None, [P, P, I64, P, I64]),
    "or_stream_default_config": (None, [P]),
    "or_stream_create": (P, [P, P, P, I64]),
    "or_stream_destroy": (None, [P]),
    "or_stream_push": (I64, [P, P, I64, C.c_int, P, I64]),
    "or_stream_tokens": (I64, [P, P, I64]),
    "or_stream_stats": (None, [P, P]),
    "or_tail_repeat_blocks": (I64, [P, I64, I64, P]),
    "or_set_threads": (None, [C.c_int]),
    "or_int8_dot_kind": (C.c_char_p, []),
    "or_set_int8_dot": (None, [C.c_int]),
    "or_get_threads": (C.c_int, []),
}

_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            raise RuntimeError(f"{LIB} missing: build it with `make -C oracle`")
        L = C.CDLL(LIB)
        for n, (r, a) in _SIGS.items():
            f = getattr(L, n)
            f.restype = r
            f.argtypes = a
        _lib = L
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data_as(P)


def f32(a):
    return np.ascontiguousarray(a, np.float32)


def set_threads(n):
    lib().or_set_threads(int(n))


def int8_dot_kind():
    return lib().or_int8_dot_kind().decode()


def quantize_bf16_rows(w_bf16, mode=ROUND):
    w = np.ascontiguousarray(w_bf16, np.uint16)
    n, k = w.shape
    q = np.empty((n, k), np.int8)
    s = np.empty(n, np.float32)
    lib().or_quantize_bf16_rows(_p(w), n, k, mode, _p(q), _p(s))
    return q, s


def quantize_act(x):
    x = f32(x)
    q = np.empty(x.shape[-1], np.int8)
    s = lib().or_quantize_act(_p(x), x.shape[-1], _p(q))
    return q, np.float32(s)


def matvec_w8a8(xq, xs, w, ws, bias=None):
    n, k = w.shape
    y = np.empty(n, np.float32)
    b = None if bias is None else f32(bias)
    lib().or_matvec_w8a8(_p(y), _p(np.ascontiguousarray(xq, np.int8)), float(xs), _p(w), _p(f32(ws)),
                         _p(b), k, n)
    return y


def linear_int8(x, w, ws, bias=None):
    n, k = w.shape
    y = np.empty(n, np.float32)
    lib().or_linear_int8(_p(y), _p(f32(x)), _p(w), _p(f32(ws)), _p(None if bias is None else f32(bias)),
                         k, n)
    return y


def linear_int8_qkv(x, wq, sq, wk, sk, wv, sv):
    qd, k = wq.shape
    kvd = wk.shape[0]
    q, kk, v = (np.empty(qd, np.float32), np.empty(kvd, np.float32), np.empty(kvd, np.float32))
    lib().or_linear_int8_qkv(_p(q), _p(kk), _p(v), _p(f32(x)), _p(wq), _p(f32(sq)), _p(wk),
                             _p(f32(sk)), _p(wv), _p(f32(sv)), k, qd, kvd)
    return q, kk, v


def linear_int8_swiglu(x, w, ws):
    n2, k = w.shape
    out = np.empty(n2 // 2, np.float32)
    lib().or_linear_int8_swiglu(_p(out), _p(f32(x)), _p(w), _p(f32(ws)), k, n2 // 2)
    return out


def linear_int8_addto(y, x, w, ws):
    n, k = w.shape
    y = f32(y).copy()
    lib().or_linear_int8_addto(_p(y), _p(f32(x)), _p(w), _p(f32(ws)), k, n)
    return y


def argmax_int8(x, w, ws):
    n, k = w.shape
    bv, sv = C.c_float(), C.c_float()
    i = lib().or_argmax_int8(_p(f32(x)), _p(w), _p(f32(ws)), k, n, C.byref(bv), C.byref(sv))
    return int(i), bv.value, sv.value


def argmax_f32_rows(x):
    """align.rs:312-321 per-row argmax of x [rows, cols]."""
    x = f32(np.atleast_2d(x))
    out = np.empty(x.shape[0], np.int32)
    lib().or_argmax_f32_rows(_p(x), x.shape[0], x.shape[1], _p(out))
    return out


def rms_norm(x, w, eps):
    x = f32(x)
    seq, hidden = (1, x.shape[0]) if x.ndim == 1 else x.shape
    out = np.empty_like(x)
    lib().or_rms_norm(_p(out), _p(x), _p(f32(w)), seq, hidden, eps)
    return out


def rms_norm_per_head(x, w, n_heads, eps):
    x = f32(x).copy()
    hd = w.shape[0]
    seq = x.size // (n_heads * hd)
    lib().or_rms_norm_per_head(_p(x), _p(f32(w)), seq, n_heads, hd, eps)
    return x


def rope_table(n_pos, hd, theta):
    c = np.empty((n_pos, hd), np.float32)
    s = np.empty((n_pos, hd), np.float32)
    lib().or_rope_table(_p(c), _p(s), n_pos, hd, theta)
    return c, s


def apply_rope(x, cos, sin, n_heads):
    x = f32(x).copy()
    hd = cos.shape[-1]
    seq = x.size // (n_heads * hd)
    lib().or_apply_rope(_p(x), _p(f32(cos)), _p(f32(sin)), seq, n_heads, hd)
    return x


def causal_attention(q, k_base, v_base, head_stride, seq_q, seq_k, n_heads, n_kv, hd, scale, q_offset):
    out = np.empty(seq_q * n_heads * hd, np.float32)
    lib().or_causal_attention(_p(out), _p(f32(q)), _p(f32(k_base)), _p(f32(v_base)), head_stride, seq_q,
                              seq_k, n_heads, n_kv, hd, scale, q_offset)
    return out


def bidir_attention(q, k, v, seq, n_heads, hd, scale, window_starts):
    out = np.empty(seq * n_heads * hd, np.float32)
    ws = np.ascontiguousarray(window_starts, np.int32)
    lib().or_bidir_attention(_p(out), _p(f32(q)), _p(f32(k)), _p(f32(v)), seq, n_heads, hd, scale,
                             _p(ws), len(ws) - 1)
    return out


def fast_exp(x):
    return np.float32(lib().or_fast_exp(float(x)))


def swiglu_rows(gate_up, inter):
    gu = f32(gate_up)
    seq = gu.size // (2 * inter)
    out = np.empty(seq * inter, np.float32)
    lib().or_swiglu_rows(_p(out), _p(gu), seq, inter)
    return out


def gelu(x):
    x = f32(x).copy()
    lib().or_gelu(_p(x), x.size)
    return x


def layer_norm(x, w, b, eps):
    x = f32(x)
    seq, hidden = (1, x.shape[0]) if x.ndim == 1 else x.shape
    out = np.empty_like(x)
    lib().or_layer_norm(_p(out), _p(x), _p(f32(w)), _p(f32(b)), seq, hidden, eps)
    return out


def sgemm_nt(A, B, C0=None):
    A, B = f32(A), f32(B)
    M, K = A.shape
    N = B.shape[0]
    Cm = np.zeros((M, N), np.float32) if C0 is None else f32(C0).copy()
    lib().or_sgemm_nt(M, N, K, _p(A), K, _p(B), K, _p(Cm), N, 0 if C0 is None else 1)
    return Cm


def linear(x, w, b=None):
    x, w = f32(x), f32(w)
    seq, k = x.shape
    n = w.shape[0]
    y = np.empty((seq, n), np.float32)
    lib().or_linear(_p(y), _p(x), _p(w), _p(None if b is None else f32(b)), seq, k, n)
    return y


def sinusoidal_pe(n_pos, d):
    pe = np.empty((n_pos, d), np.float32)
    lib().or_sinusoidal_pe(_p(pe), n_pos, d)
    return pe


def mel(samples):
    s = f32(samples)
    nf = lib().or_mel_frames(s.size)
    out = np.empty((128, max(nf, 1)), np.float32)
    nf = lib().or_mel(_p(s), s.size, _p(out))
    return out[:, :nf]


class OracleDecoder:
    """or_decoder over SynthDecoder-style numpy weights."""

    def __init__(self, weights, max_seq=2048, mode=ROUND, kv_bf16=False):
        self.w = weights
        self.cfg = weights.cfg
        cfg, w = weights.structs(DecConfig, DecLayer, DecWeights)
        self._keep = (cfg, w)
        self.d = lib().or_decoder_create(C.byref(cfg), C.byref(w), mode, max_seq)
        self.max_seq = max_seq
        if kv_bf16:
            lib().or_decoder_set_kv_bf16(self.d, 1)

    def close(self):
        if self.d:
            lib().or_decoder_destroy(self.d)
            self.d = None

    def __del__(self):
        self.close()

    @property
    def kv_len(self):
        return int(lib().or_decoder_len(self.d))

    @kv_len.setter
    def kv_len(self, n):
        lib().or_decoder_set_len(self.d, int(n))

    def packed(self, layer, which, rows=None):
        """(int8 rows, row scales) of a packed matrix (layer -1: the LM head);
        rows (a list of row indices) copies only those."""
        c = self.cfg
        H, hd, I = c["hidden"], c["head_dim"], c["intermediate"]
        qd, kvd = c["n_heads"] * hd, c["n_kv_heads"] * hd
        shape = (c["vocab"], H) if layer == -1 else [(qd, H), (kvd, H), (kvd, H), (H, qd), (2 * I, H), (H, I)][which]
        sp = P()
        qp = lib().or_decoder_packed(self.d, layer, which, C.byref(sp))
        q = np.ctypeslib.as_array(C.cast(qp, C.POINTER(C.c_int8)), shape=shape)
        s = np.ctypeslib.as_array(C.cast(sp, C.POINTER(C.c_float)), shape=(shape[0],))
        if rows is not None:
            idx = np.asarray(rows, np.int64)
            return q[idx].copy(), s[idx].copy()
        return q.copy(), s.copy()

    def embed(self, token):
        out = np.empty(self.cfg["hidden"], np.float32)
        lib().or_embed_token(self.d, int(token), _p(out))
        return out

    def prefill(self, embeds):
        e = f32(embeds)
        lib().or_decoder_prefill(self.d, _p(e), e.shape[0])

    def prefill_hidden(self, embeds):
        """decoder_prefill, returning the last layer's rows (pref_x) [seq, hidden]."""
        e = f32(embeds)
        out = np.empty((e.shape[0], self.cfg["hidden"]), np.float32)
        lib().or_decoder_prefill_hidden(self.d, _p(e), e.shape[0], _p(out))
        return out

    def prefill_logits(self, embeds, lm_bf16=None):
        """decoder_prefill_logits (decoder.rs:649-681): [seq, out_dim] f32."""
        e = f32(embeds)
        if lm_bf16 is None:
            out_dim = self.cfg["vocab"]
            lm = None
        else:
            lm = np.ascontiguousarray(lm_bf16, np.uint16)
            out_dim = lm.shape[0]
        out = np.empty((e.shape[0], out_dim), np.float32)
        lib().or_decoder_prefill_logits(self.d, _p(e), e.shape[0], None if lm is None else _p(lm), out_dim, _p(out))
        return out

    def forward_logits(self, embed, return_hidden=False):
        """(token, best logit, second-best logit), and with return_hidden the
        final normed hidden state the LM-head argmax scored."""
        bv, sv = C.c_float(), C.c_float()
        hid = np.empty(self.cfg["hidden"], np.float32) if return_hidden else None
        t = lib().or_decoder_forward(self.d, _p(f32(embed)), C.byref(bv), C.byref(sv), _p(hid))
        if return_hidden:
            return int(t), bv.value, sv.value, hid
        return int(t), bv.value, sv.value

    def forward(self, embed, return_hidden=False):
        bv, sv = C.c_float(), C.c_float()
        hid = np.empty(self.cfg["hidden"], np.float32) if return_hidden else None
        t = lib().or_decoder_forward(self.d, _p(f32(embed)), C.byref(bv), C.byref(sv), _p(hid))
        if return_hidden:
            return int(t), bv.value - sv.value, hid
        return int(t), bv.value - sv.value

    def set_kv(self, k, v):
        """Overwrite the KV cache ([layer][kv_head][max_seq][head_dim] f32)."""
        for which, a in ((0, k), (1, v)):
            a = f32(a)
            assert a.size == self.cfg["n_layers"] * self.cfg["n_kv_heads"] * self.max_seq * self.cfg["head_dim"]
            C.memmove(lib().or_decoder_kv(self.d, which), a.ctypes.data, a.nbytes)

    def kv_rows(self, start, n):
        """Copies of positions [start, start + n): ([layer][kv_head][n][head_dim]) x 2."""
        c = self.cfg
        shape = (c["n_layers"], c["n_kv_heads"], self.max_seq, c["head_dim"])
        out = []
        for which in (0, 1):
            p = lib().or_decoder_kv(self.d, which)
            a = np.ctypeslib.as_array(C.cast(p, C.POINTER(C.c_float)), shape=shape)
            out.append(a[:, :, start:start + n].copy())
        return out

    def kv(self):
        c = self.cfg
        shape = (c["n_layers"], c["n_kv_heads"], self.max_seq, c["head_dim"])
        out = []
        for which in (0, 1):
            p = lib().or_decoder_kv(self.d, which)
            out.append(np.ctypeslib.as_array(C.cast(p, C.POINTER(C.c_float)), shape=shape).copy())
        return out


class OracleEncoder:
    def __init__(self, weights):
        self.w = weights
        cfg, w = weights.structs(EncConfig, EncLayer, EncWeights)
        self._keep = (cfg, w)
        self.e = lib().or_encoder_create(C.byref(cfg), C.byref(w))
        self.cfg = weights.cfg

    def close(self):
        if self.e:
            lib().or_encoder_destroy(self.e)
            self.e = None

    def __del__(self):
        self.close()

    def forward(self, mel_arr):
        m = f32(mel_arr)
        frames = m.shape[1]
        T = lib().or_encoder_tokens(self.e, frames)
        out = np.empty((T, self.cfg["output_dim"]), np.float32)
        lib().or_encoder_forward(self.e, _p(m), frames, _p(out))
        return out


def _ids(a):
    a = np.ascontiguousarray(a if a is not None else [], np.int32)
    return a, (_p(a) if a.size else None), a.size


def transcribe_forced(dec, enc, samples, n_steps, prompt=None, force=None, past=None):
    """or_transcribe_prompt: transcribe_segment (transcribe.rs:63-247) with
    n_steps greedy forwards and the optional prompt / forced-language / past
    text ids of its prompt layout (transcribe.rs:97-169)."""
    s = f32(samples)
    toks = np.empty(n_steps, np.int32)
    margins = np.empty(n_steps, np.float32)
    times = np.empty(4, np.float64)
    (pa, pp, pn), (fa, fp, fn), (qa, qp, qn) = _ids(prompt), _ids(force), _ids(past)
    total = lib().or_transcribe_prompt(dec.d, enc.e, _p(s), s.size, pp, pn, fp, fn, qp, qn, n_steps, _p(toks),
                                       _p(margins), _p(times))
    return dict(tokens=toks, margins=margins, times_ms=times, prompt_len=int(total))


def prompt_ids(prompt=None, force=None, past=None):
    """The id rows before and after the audio rows (transcribe.rs:97-169)."""
    (pa, pp, pn), (fa, fp, fn), (qa, qp, qn) = _ids(prompt), _ids(force), _ids(past)
    head = np.empty(9 + pn, np.int32)
    tail = np.empty(7 + fn + qn, np.int32)
    nh, nt = I64(), I64()
    lib().or_prompt_ids(pp, pn, fp, fn, qp, qn, _p(head), C.byref(nh), _p(tail), C.byref(nt))
    return head[:nh.value].copy(), tail[:nt.value].copy()


def find_split_point(samples, target, search_sec):
    x = f32(samples)
    return int(lib().or_find_split_point(_p(x), x.size, int(target), float(search_sec)))


def segment_splits(samples, segment_sec, search_sec=3.0):
    """transcribe_audio's split points (transcribe.rs:323-341)."""
    x = f32(samples)
    out = np.empty(128, np.int64)
    n = lib().or_segment_splits(_p(x) if x.size else None, x.size, float(segment_sec), float(search_sec), _p(out),
                                out.size)
    return out[:n].copy()


class StreamConfig(C.Structure):
    _fields_ = [("chunk_sec", C.c_float), ("rollback", C.c_int32), ("unfixed_chunks", C.c_int32),
                ("max_new_tokens", C.c_int32), ("past_text_conditioning", C.c_int32),
                ("stop_tokens", C.c_int32 * 2)]


def stream_config(**kw):
    c = StreamConfig()
    lib().or_stream_default_config(C.byref(c))
    for k, v in kw.items():
        if k == "stop_tokens":
            c.stop_tokens[0], c.stop_tokens[1] = v
        else:
            setattr(c, k, v)
    return c


def tail_repeat_blocks(tokens, max_period):
    t = np.ascontiguousarray(tokens, np.int32)
    period = I64()
    reps = lib().or_tail_repeat_blocks(_p(t), t.size, max_period, C.byref(period))
    return int(reps), int(period.value)


class OracleStream:
    """or_stream: stream_push_audio (transcribe.rs:902-1304) on the oracle model."""

    def __init__(self, dec, enc, **cfg):
        self.cfg = stream_config(**cfg)
        self.dec, self.enc = dec, enc
        self.s = lib().or_stream_create(dec.d, enc.e, C.byref(self.cfg), dec.cfg["hidden"])

    def set_prompt(self, prompt=None, force=None):
        """QwenCtx::prompt_tokens / force_prompt_tokens for the next chunks."""
        (pa, pp, pn), (fa, fp, fn) = _ids(prompt), _ids(force)
        lib().or_stream_set_prompt(self.s, pp, pn, fp, fn)

    def push(self, samples, finalize=False):
        x = f32(samples)
        out = np.empty(4096, np.int32)
        n = lib().or_stream_push(self.s, _p(x), x.size, 1 if finalize else 0, _p(out), out.size)
        return out[:n].copy()

    def tokens(self):
        out = np.empty(1 << 16, np.int32)
        n = lib().or_stream_tokens(self.s, _p(out), out.size)
        return out[:n].copy()

    def stats(self):
        st = np.zeros(8, np.int64)
        lib().or_stream_stats(self.s, _p(st))
        return st

    def close(self):
        if self.s:
            lib().or_stream_destroy(self.s)
            self.s = None

    def __del__(self):
        self.close()

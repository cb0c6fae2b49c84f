"""Model-level mirror of the reference's decoder API (decoder.rs) on the GPU."""
import ctypes as C

import numpy as np

from ._lib import (F32, I64, QASR_ROUND_HALF_AWAY, DecConfig, DecLayer, DecWeights, EncConfig, EncLayer,
                   EncWeights, I32, P, Prompt, StreamConfig, check, lib)


ST_DTYPES = {0: None, 1: np.float32, 2: np.float16, 3: "bf16", 4: np.int32, 5: np.int64, 6: np.bool_}


class Checkpoint:
    """MultiSafetensors (safetensors.rs:206-272): a read-only mapping of a
    checkpoint directory (model.safetensors or its model-*.safetensors shards)
    or, with ``file=True``, of one file.  No GPU needed."""

    def __init__(self, path, file=False):
        st = P()
        fn = lib().qasr_hip_st_open_file if file else lib().qasr_hip_st_open
        check(fn(str(path).encode(), C.byref(st)))
        self.st = st

    def close(self):
        if self.st:
            lib().qasr_hip_st_free(self.st)
            self.st = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def n_shards(self):
        return int(lib().qasr_hip_st_shards(self.st))

    def names(self):
        return [lib().qasr_hip_st_name(self.st, i).decode("utf-8")
                for i in range(int(lib().qasr_hip_st_count(self.st)))]

    def find(self, name):
        """(dtype code, shape, host address, bytes) of the first shard holding name."""
        dt, nd, shape = C.c_int(), C.c_int(), (I64 * 8)()
        ptr, nbytes = P(), I64()
        check(lib().qasr_hip_st_find(self.st, name.encode("utf-8"), C.byref(dt), C.byref(nd), shape,
                                     C.byref(ptr), C.byref(nbytes)))
        return dt.value, tuple(shape[i] for i in range(nd.value)), ptr.value, nbytes.value

    def array(self, name):
        """A numpy copy of the tensor (bf16 as uint16)."""
        dt, shape, ptr, nbytes = self.find(name)
        raw = np.frombuffer((C.c_char * nbytes).from_address(ptr), np.uint8).copy() if nbytes else \
            np.empty(0, np.uint8)
        t = ST_DTYPES[dt]
        return raw.view(np.uint16 if t == "bf16" else t).reshape(shape) if t is not None else raw


class Decoder:
    """Device-resident Qwen3 decoder: Decoder::load + KvCache + decoder_prefill/forward.

    ``weights`` is a :class:`qwenasr_amd.synth.SynthDecoder` (or any object with
    the same numpy attributes).  The bf16 host arrays are uploaded once; the
    int8 packing happens on the GPU.
    """

    def __init__(self, dev, weights, max_seq=2048, round_mode=QASR_ROUND_HALF_AWAY, kv_bf16=False):
        self.dev = dev
        self.cfg = dict(weights.cfg)
        cfg, w = weights.structs(DecConfig, DecLayer, DecWeights)
        d = P()
        check(lib().qasr_hip_decoder_load(dev.h, C.byref(cfg), C.byref(w), round_mode, max_seq,
                                          1 if kv_bf16 else 0, C.byref(d)))
        self.d = d
        self.max_seq = max_seq
        self.kv_bf16 = kv_bf16
        dev.adopt(self)

    @classmethod
    def from_checkpoint(cls, dev, ckpt, cfg, max_seq=2048, round_mode=QASR_ROUND_HALF_AWAY, kv_bf16=False):
        """Decoder::load (decoder.rs:70-167) from a :class:`Checkpoint`; cfg is the config dict."""
        self = cls.__new__(cls)
        self.dev = dev
        self.cfg = dict(cfg)
        c = DecConfig(**{k: cfg[k] for k in ("n_layers", "hidden", "n_heads", "n_kv_heads", "head_dim",
                                            "intermediate", "vocab", "eps", "theta")})
        d = P()
        check(lib().qasr_hip_decoder_load_st(dev.h, ckpt.st, C.byref(c), round_mode, max_seq,
                                             1 if kv_bf16 else 0, C.byref(d)))
        self.d = d
        self.max_seq = max_seq
        self.kv_bf16 = kv_bf16
        dev.adopt(self)
        return self

    def close(self):
        if self.d:
            lib().qasr_hip_decoder_free(self.d)
            self.d = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def kv_len(self):
        return int(lib().qasr_hip_decoder_len(self.d))

    @kv_len.setter
    def kv_len(self, n):
        check(lib().qasr_hip_decoder_set_len(self.d, int(n)))

    def prefill(self, embeds):
        """decoder_prefill (decoder.rs:455): embeds f32 [seq, hidden]."""
        e = np.ascontiguousarray(embeds, np.float32)
        check(lib().qasr_hip_decoder_prefill(self.d, e.ctypes.data_as(P), e.shape[0]))

    def set_lm_head(self, w_bf16=None):
        """A separate bf16 LM head [out_dim, hidden] for prefill_logits (None: the tied embedding)."""
        if w_bf16 is None:
            check(lib().qasr_hip_decoder_set_lm_head(self.d, None, 0))
        else:
            w = np.ascontiguousarray(w_bf16, np.uint16)
            if w.ndim != 2 or w.shape[1] != self.cfg["hidden"]:
                raise ValueError(f"LM head must be [out_dim, {self.cfg['hidden']}], got {w.shape}")
            check(lib().qasr_hip_decoder_set_lm_head(self.d, w.ctypes.data_as(P), w.shape[0]))

    def prefill_logits(self, embeds):
        """decoder_prefill_logits (decoder.rs:649-681): [seq, out_dim] f32 logits."""
        e = np.ascontiguousarray(embeds, np.float32)
        out = np.empty((e.shape[0], int(lib().qasr_hip_decoder_logits_dim(self.d))), np.float32)
        check(lib().qasr_hip_decoder_prefill_logits(self.d, e.ctypes.data_as(P), e.shape[0],
                                                    out.ctypes.data_as(P)))
        return out

    def prefill_argmax(self, embeds, rows):
        """The aligner's timestamp readout (align.rs:300-321): prefill, then the
        head's per-row argmax at the prefill rows `rows`."""
        e = np.ascontiguousarray(embeds, np.float32)
        r = np.ascontiguousarray(rows, np.int32)
        out = np.empty(r.shape[0], np.int32)
        check(lib().qasr_hip_decoder_prefill_argmax(self.d, e.ctypes.data_as(P), e.shape[0], r.ctypes.data_as(P),
                                                    r.shape[0], out.ctypes.data_as(P)))
        return out

    def forward(self, embed=None, token=0):
        """decoder_forward (decoder.rs:550): returns the greedy token id."""
        out = I32()
        if embed is None:
            check(lib().qasr_hip_decoder_forward(self.d, None, int(token), C.byref(out)))
        else:
            e = np.ascontiguousarray(embed, np.float32)
            check(lib().qasr_hip_decoder_forward(self.d, e.ctypes.data_as(P), 0, C.byref(out)))
        return int(out.value)

    def last_logit(self):
        """The winning logit of the last decode step's LM-head argmax."""
        v = F32()
        check(lib().qasr_hip_decoder_last_logit(self.d, C.byref(v)))
        return float(v.value)

    def generate(self, n_steps, first_embed=None, first_token=0):
        """n_steps forced greedy steps with no host round trip between steps."""
        toks = np.empty(n_steps, np.int32)
        if first_embed is None:
            check(lib().qasr_hip_decoder_generate(self.d, None, int(first_token), n_steps,
                                                  toks.ctypes.data_as(P)))
        else:
            e = np.ascontiguousarray(first_embed, np.float32)
            check(lib().qasr_hip_decoder_generate(self.d, e.ctypes.data_as(P), 0, n_steps,
                                                  toks.ctypes.data_as(P)))
        return toks

    def packed(self, layer, which):
        """(int8 rows, scales) as packed on the GPU; layer -1 is the LM head."""
        c = self.cfg
        H, hd, I = c["hidden"], c["head_dim"], c["intermediate"]
        qd, kvd = c["n_heads"] * hd, c["n_kv_heads"] * hd
        if layer == -1:
            shape = (int(lib().qasr_hip_decoder_head_rows(self.d)), H)
        else:
            shape = [(qd, H), (kvd, H), (kvd, H), (H, qd), (2 * I, H), (H, I)][which]
        q = np.empty(shape, np.int8)
        s = np.empty(shape[0], np.float32)
        check(lib().qasr_hip_decoder_packed(self.d, layer, which, q.ctypes.data_as(P),
                                            s.ctypes.data_as(P)))
        return q, s

    @property
    def capacity(self):
        """Positions the KV cache holds now (it doubles on demand, decoder.rs:199-231)."""
        return int(lib().qasr_hip_decoder_capacity(self.d))

    def kv_shape(self):
        c = self.cfg
        return (c["n_layers"], c["n_kv_heads"], self.capacity, c["head_dim"])

    def kv_upload(self, k, v):
        k = np.ascontiguousarray(k, np.float32)
        v = np.ascontiguousarray(v, np.float32)
        check(lib().qasr_hip_decoder_kv_upload(self.d, k.ctypes.data_as(P), v.ctypes.data_as(P)))

    def kv_rows_upload(self, start, k, v):
        """Overwrite positions [start, start + n) of every layer and KV head from
        [layer][kv_head][n][head_dim] arrays."""
        k = np.ascontiguousarray(k, np.float32)
        v = np.ascontiguousarray(v, np.float32)
        assert k.shape == v.shape and k.ndim == 4
        check(lib().qasr_hip_decoder_kv_upload_rows(self.d, int(start), k.shape[2], k.ctypes.data_as(P),
                                                    v.ctypes.data_as(P)))

    def kv_rows_download(self, start, n):
        c = self.cfg
        shape = (c["n_layers"], c["n_kv_heads"], int(n), c["head_dim"])
        k, v = np.empty(shape, np.float32), np.empty(shape, np.float32)
        check(lib().qasr_hip_decoder_kv_download_rows(self.d, int(start), int(n), k.ctypes.data_as(P),
                                                      v.ctypes.data_as(P)))
        return k, v

    def kv_download(self):
        k = np.empty(self.kv_shape(), np.float32)
        v = np.empty(self.kv_shape(), np.float32)
        check(lib().qasr_hip_decoder_kv_download(self.d, k.ctypes.data_as(P), v.ctypes.data_as(P)))
        return k, v

    def set_options(self, attn_splits=0, use_graph=True):
        check(lib().qasr_hip_decoder_set_options(self.d, int(attn_splits), 1 if use_graph else 0))

    def set_fusion(self, fuse_qkv_attention=True):
        """Each layer's qkv matvec and decode attention as one launch (True) or two."""
        check(lib().qasr_hip_decoder_set_fusion(self.d, 1 if fuse_qkv_attention else 0))


class Encoder:
    """Audio front end on the GPU: mel_spectrogram (audio.rs:273) + Encoder::forward (encoder.rs:186)."""

    def __init__(self, dev, weights):
        self.dev = dev
        self.cfg = dict(weights.cfg)
        cfg, w = weights.structs(EncConfig, EncLayer, EncWeights)
        e = P()
        check(lib().qasr_hip_encoder_load(dev.h, C.byref(cfg), C.byref(w), C.byref(e)))
        self.e = e
        dev.adopt(self)

    @classmethod
    def from_checkpoint(cls, dev, ckpt, cfg):
        """Encoder::load (encoder.rs:123-182) from a :class:`Checkpoint`; cfg is the config dict."""
        self = cls.__new__(cls)
        self.dev = dev
        self.cfg = dict(cfg)
        c = EncConfig(**{k: cfg[k] for k in ("d_model", "n_layers", "n_heads", "head_dim", "ffn_dim",
                                            "output_dim", "chunk_size", "n_window_infer", "conv_hidden")})
        e = P()
        check(lib().qasr_hip_encoder_load_st(dev.h, ckpt.st, C.byref(c), C.byref(e)))
        self.e = e
        dev.adopt(self)
        return self

    def close(self):
        if self.e:
            lib().qasr_hip_encoder_free(self.e)
            self.e = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def tokens(self, frames):
        return int(lib().qasr_hip_encoder_tokens(self.e, int(frames)))

    def mel(self, samples):
        s = np.ascontiguousarray(samples, np.float32)
        nf = I64()
        check(lib().qasr_hip_mel(self.e, s.ctypes.data_as(P), s.size, None, C.byref(nf)))
        out = np.empty((128, nf.value), np.float32)
        check(lib().qasr_hip_mel(self.e, s.ctypes.data_as(P), s.size, out.ctypes.data_as(P), C.byref(nf)))
        return out

    def forward(self, mel):
        m = np.ascontiguousarray(mel, np.float32)
        frames = m.shape[1]
        out = np.empty((self.tokens(frames), self.cfg["output_dim"]), np.float32)
        nt = I64()
        check(lib().qasr_hip_encoder_forward(self.e, m.ctypes.data_as(P), frames, out.ctypes.data_as(P),
                                             C.byref(nt)))
        return out

    def forward_batch(self, mels):
        """One encoder pass over several mels: a list of each one's rows."""
        ms = [np.ascontiguousarray(m, np.float32) for m in mels]
        frames = np.array([m.shape[1] for m in ms], np.int64)
        tot = sum(self.tokens(int(f)) for f in frames)
        out = np.empty((tot, self.cfg["output_dim"]), np.float32)
        toks = np.zeros(len(ms), np.int64)
        ptrs = (P * len(ms))(*[m.ctypes.data_as(P) for m in ms])
        check(lib().qasr_hip_encoder_forward_batch(self.e, len(ms), C.cast(ptrs, P), frames.ctypes.data_as(P),
                                                   out.ctypes.data_as(P), toks.ctypes.data_as(P)))
        offs = np.concatenate([[0], np.cumsum(toks)])
        return [out[offs[j]:offs[j + 1]].copy() for j in range(len(ms))]


def transcribe_forced(decoder, encoder, samples, n_steps):
    """transcribe_segment (transcribe.rs:63-247) with a forced decode length.

    Returns (token ids, stage times in ms: mel, encoder, prefill + first forward, decode).
    """
    s = np.ascontiguousarray(samples, np.float32)
    toks = np.empty(n_steps, np.int32)
    times = np.empty(4, np.float64)
    check(lib().qasr_hip_transcribe_forced(decoder.d, encoder.e, s.ctypes.data_as(P), s.size, int(n_steps),
                                           toks.ctypes.data_as(P), times.ctypes.data_as(P)))
    return toks, times


def _ids(a):
    """An int32 id array and its pointer (None when empty)."""
    a = np.ascontiguousarray(a if a is not None else [], np.int32)
    return a, (a.ctypes.data_as(P) if a.size else None)


def make_prompt(prompt=None, force=None):
    """A qasr_prompt over the given ids; returns (struct, the arrays it points into)."""
    (pa, pp), (fa, fp) = _ids(prompt), _ids(force)
    return Prompt(pp, pa.size, fp, fa.size), (pa, fa)


def transcribe(decoder, encoder, samples, max_tokens=2048, prompt=None, force=None, past=None):
    """transcribe_segment (transcribe.rs:63-247): greedy to a stop token
    (151643, 151645) or max_tokens, with the optional prompt, forced-language
    (ending in <asr_text>) and past-text ids of its prompt layout
    (transcribe.rs:97-169).  Returns (every token produced, the stop
    included; stage times in ms)."""
    s = np.ascontiguousarray(samples, np.float32)
    toks = np.empty(max_tokens, np.int32)
    times = np.empty(4, np.float64)
    n = I64()
    if prompt is None and force is None and past is None:
        check(lib().qasr_hip_transcribe(decoder.d, encoder.e, s.ctypes.data_as(P), s.size, int(max_tokens),
                                        toks.ctypes.data_as(P), C.byref(n), times.ctypes.data_as(P)))
    else:
        pr, keep = make_prompt(prompt, force)
        qa, qp = _ids(past)
        check(lib().qasr_hip_transcribe_prompt(decoder.d, encoder.e, s.ctypes.data_as(P), s.size, C.byref(pr), qp,
                                               qa.size, int(max_tokens), toks.ctypes.data_as(P), C.byref(n),
                                               times.ctypes.data_as(P)))
    return toks[:n.value].copy(), times


def text_tokens(raw, text_open=False):
    """The ids transcribe_segment turns into text (transcribe.rs:196-214);
    text_open: the prompt held forced-language or past-text ids."""
    r = np.ascontiguousarray(raw, np.int32)
    out = np.empty(max(1, r.size), np.int32)
    if text_open:
        k = lib().qasr_hip_text_tokens_from(r.ctypes.data_as(P), r.size, 1, out.ctypes.data_as(P))
    else:
        k = lib().qasr_hip_text_tokens(r.ctypes.data_as(P), r.size, out.ctypes.data_as(P))
    return out[:k].copy()


def segment_splits(samples, segment_sec, search_sec=3.0):
    """transcribe_audio's segment starts (transcribe.rs:323-341); host only."""
    s = np.ascontiguousarray(samples, np.float32)
    out = np.empty(128, np.int64)
    k = lib().qasr_hip_segment_splits(s.ctypes.data_as(P) if s.size else None, s.size, float(segment_sec),
                                      float(search_sec), out.ctypes.data_as(P), out.size)
    if k < 0:
        raise ValueError("qasr_hip_segment_splits: bad arguments")
    return out[:k].copy()


def detect_config(ckpt):
    """QwenConfig::detect (config.rs:108-156) on a Checkpoint: (decoder, encoder) config dicts."""
    dc, ec = DecConfig(), EncConfig()
    check(lib().qasr_hip_engine_detect(ckpt.st, C.byref(dc), C.byref(ec)))
    return ({k: getattr(dc, k) for k, _ in DecConfig._fields_}, {k: getattr(ec, k) for k, _ in EncConfig._fields_})


class Engine:
    """The reference's C API (c_api.rs) at token level: qwen_asr_load_model,
    transcribe_pcm and the streaming calls over one engine."""

    def __init__(self, model_dir, device=0, max_seq=0):
        g = P()
        check(lib().qasr_hip_engine_load(str(model_dir).encode(), int(device), int(max_seq), C.byref(g)))
        self.g = g

    def close(self):
        if self.g:
            lib().qasr_hip_engine_free(self.g)
            self.g = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def config(self):
        dc, ec = DecConfig(), EncConfig()
        check(lib().qasr_hip_engine_config(self.g, C.byref(dc), C.byref(ec)))
        return ({k: getattr(dc, k) for k, _ in DecConfig._fields_}, {k: getattr(ec, k) for k, _ in EncConfig._fields_})

    def transcribe_pcm(self, samples):
        s = np.ascontiguousarray(samples, np.float32)
        out = np.empty(2048 * 128, np.int32)          # 2048 tokens for each of up to 127 segments
        n = I64()
        check(lib().qasr_hip_engine_transcribe_pcm(self.g, s.ctypes.data_as(P), s.size, out.ctypes.data_as(P),
                                                   out.size, C.byref(n)))
        return out[:n.value].copy()

    def last_raw_tokens(self):
        n = I64()
        check(lib().qasr_hip_engine_last_raw_tokens(self.g, None, 0, C.byref(n)))
        out = np.empty(max(n.value, 1), np.int32)
        check(lib().qasr_hip_engine_last_raw_tokens(self.g, out.ctypes.data_as(P), out.size, C.byref(n)))
        return out[:n.value].copy()

    def last_segments(self):
        """[n, 4]: first sample, end sample, first text id index, text id count."""
        out = np.empty((128, 4), np.int64)
        n = I64()
        check(lib().qasr_hip_engine_last_segments(self.g, out.ctypes.data_as(P), 128, C.byref(n)))
        return out[:n.value].copy()

    def set_segment_sec(self, sec, search_sec=None):
        lib().qasr_hip_engine_set_segment_sec(self.g, float(sec))
        if search_sec is not None:
            lib().qasr_hip_engine_set_search_sec(self.g, float(search_sec))

    def set_language_tokens(self, ids):
        """qwen_asr_set_language with "language <Name>" already encoded (empty: automatic)."""
        a, p = _ids(ids)
        check(lib().qasr_hip_engine_set_language_tokens(self.g, p, a.size))

    def set_prompt_tokens(self, ids):
        a, p = _ids(ids)
        check(lib().qasr_hip_engine_set_prompt_tokens(self.g, p, a.size))

    def set_stream(self, chunk_sec=None, rollback=None, unfixed_chunks=None, max_new_tokens=None):
        if chunk_sec is not None:
            lib().qasr_hip_engine_stream_set_chunk_sec(self.g, float(chunk_sec))
        if rollback is not None:
            lib().qasr_hip_engine_stream_set_rollback(self.g, int(rollback))
        if unfixed_chunks is not None:
            lib().qasr_hip_engine_stream_set_unfixed_chunks(self.g, int(unfixed_chunks))
        if max_new_tokens is not None:
            lib().qasr_hip_engine_stream_set_max_new_tokens(self.g, int(max_new_tokens))

    def stream(self):
        return EngineStream(self)


class EngineStream:
    """QwenAsrStreamState (c_api.rs:167-260): push() takes the NEW samples."""

    def __init__(self, engine):
        s = P()
        check(lib().qasr_hip_engine_stream_new(engine.g, C.byref(s)))
        self.s = s
        self.engine = engine

    def push(self, samples, finalize=False):
        x = np.ascontiguousarray(samples, np.float32)
        out = np.empty(4096, np.int32)
        n = I64()
        check(lib().qasr_hip_engine_stream_push(self.s, x.ctypes.data_as(P) if x.size else None, x.size,
                                                1 if finalize else 0, out.ctypes.data_as(P), out.size, C.byref(n)))
        return out[:n.value].copy()

    def result(self):
        out = np.empty(1 << 16, np.int32)
        n = I64()
        check(lib().qasr_hip_engine_stream_get_result(self.s, out.ctypes.data_as(P), out.size, C.byref(n)))
        return out[:n.value].copy()

    def reset(self):
        check(lib().qasr_hip_engine_stream_reset(self.s))

    def close(self):
        if self.s:
            lib().qasr_hip_engine_stream_free(self.s)
            self.s = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


KERNEL_KINDS = ("norm+qkv", "attention", "o_proj+=", "norm+gate_up+swiglu", "down+=", "norm+lm_head_argmax",
                "argmax_merge", "norm+qkv (own launch)")


def profile_decoder(decoder, n_steps):
    """Average us per launch, algorithmic bytes per launch and launches per step
    of each decode-step kernel, timed with HIP events inside real decode steps."""
    k = len(KERNEL_KINDS)
    us = np.zeros(k, np.float32)
    by = np.zeros(k, np.float64)
    n = np.zeros(k, np.int32)
    check(lib().qasr_hip_decoder_profile(decoder.d, int(n_steps), us.ctypes.data_as(P), by.ctypes.data_as(P),
                                         n.ctypes.data_as(P)))
    return [dict(kernel=k, us=float(us[i]), bytes=float(by[i]), per_step=int(n[i]))
            for i, k in enumerate(KERNEL_KINDS)]


class Stream:
    """Incremental streaming transcription (StreamState + stream_push_audio,
    transcribe.rs:902-1304) on a device-resident decoder and encoder.  push()
    takes the whole audio so far and returns the newly committed token ids."""

    _close_first = 2

    def __init__(self, decoder, encoder, **cfg):
        c = StreamConfig()
        lib().qasr_hip_stream_default_config(C.byref(c))
        for k, v in cfg.items():
            if k == "stop_tokens":
                c.stop_tokens[0], c.stop_tokens[1] = v
            else:
                setattr(c, k, v)
        s = P()
        check(lib().qasr_hip_stream_create(decoder.d, encoder.e, C.byref(c), C.byref(s)))
        self.s = s
        self.decoder, self.encoder = decoder, encoder
        decoder.dev.adopt(self)

    def set_prompt(self, prompt=None, force=None):
        """QwenCtx::prompt_tokens / force_prompt_tokens for the next chunks."""
        pr, keep = make_prompt(prompt, force)
        check(lib().qasr_hip_stream_set_prompt(self.s, C.byref(pr)))

    def push(self, samples, finalize=False):
        x = np.ascontiguousarray(samples, np.float32)
        out = np.empty(4096, np.int32)
        n = I64()
        check(lib().qasr_hip_stream_push(self.s, x.ctypes.data_as(P), x.size, 1 if finalize else 0,
                                         out.ctypes.data_as(P), out.size, C.byref(n)))
        return out[:n.value].copy()

    def tokens(self):
        n = I64()
        check(lib().qasr_hip_stream_tokens(self.s, None, 0, C.byref(n)))
        out = np.empty(max(n.value, 1), np.int32)
        check(lib().qasr_hip_stream_tokens(self.s, out.ctypes.data_as(P), out.size, C.byref(n)))
        return out[:n.value].copy()

    def reset(self):
        check(lib().qasr_hip_stream_reset(self.s))

    @property
    def audio_cursor(self):
        return int(lib().qasr_hip_stream_audio_cursor(self.s))

    def stats(self):
        st = np.zeros(8, np.int64)
        check(lib().qasr_hip_stream_stats(self.s, st.ctypes.data_as(P)))
        return st

    def close(self):
        if self.s:
            lib().qasr_hip_stream_free(self.s)
            self.s = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class StreamBatch:
    """Many streaming states over one decoder and encoder whose chunks decode
    together on a multi-stream batch (qasr_hip_stream_batch_*): push() takes
    each stream's whole audio so far and returns each stream's newly committed
    token ids; stream(i) gives a view with tokens(), stats() and audio_cursor."""

    _close_first = 2

    def __init__(self, decoder, encoder, n_streams, max_seq, **cfg):
        c = StreamConfig()
        lib().qasr_hip_stream_default_config(C.byref(c))
        for k, v in cfg.items():
            if k == "stop_tokens":
                c.stop_tokens[0], c.stop_tokens[1] = v
            else:
                setattr(c, k, v)
        g = P()
        check(lib().qasr_hip_stream_batch_create(decoder.d, encoder.e, C.byref(c), int(n_streams), int(max_seq),
                                                 C.byref(g)))
        self.g = g
        self.n = int(n_streams)
        self.decoder, self.encoder = decoder, encoder
        decoder.dev.adopt(self)

    def push(self, samples, finalize=None, cap=4096):
        xs = [np.ascontiguousarray(x, np.float32) for x in samples]
        assert len(xs) == self.n
        ptrs = (P * self.n)(*[x.ctypes.data_as(P) if x.size else None for x in xs])
        ns = np.array([x.size for x in xs], np.int64)
        fin = np.array([1 if (finalize is not None and finalize[i]) else 0 for i in range(self.n)], np.int32)
        out = np.empty((self.n, cap), np.int32)
        n_out = np.zeros(self.n, np.int64)
        check(lib().qasr_hip_stream_batch_push(self.g, C.cast(ptrs, P), ns.ctypes.data_as(P), fin.ctypes.data_as(P),
                                               out.ctypes.data_as(P), cap, n_out.ctypes.data_as(P)))
        return [out[i, :n_out[i]].copy() for i in range(self.n)]

    def stream(self, i):
        return _MemberStream(self, lib().qasr_hip_stream_batch_stream(self.g, int(i)))

    def times(self):
        """ms of the last push's phases: (encoder, prompt rows + prefix comparison, prefill, decode)."""
        ms = np.zeros(4, np.float64)
        check(lib().qasr_hip_stream_batch_times(self.g, ms.ctypes.data_as(P)))
        return tuple(float(v) for v in ms)

    def close(self):
        if self.g:
            lib().qasr_hip_stream_batch_free(self.g)
            self.g = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class _MemberStream:
    """View of one state of a StreamBatch (owned by the batch)."""

    def __init__(self, group, s):
        if not s:
            raise IndexError("stream index out of range")
        self.group, self.s = group, s

    tokens = Stream.tokens
    set_prompt = Stream.set_prompt
    stats = Stream.stats
    reset = Stream.reset
    audio_cursor = Stream.audio_cursor


class Batch:
    """Multi-stream greedy decode: up to 32 streams with
    their own KV caches and lengths step together on one decoder's weights.
    A stream's tokens equal those of the single-stream decoder at the same
    attention split count."""

    _close_first = 2

    def __init__(self, decoder, n_streams, max_seq, max_steps=256):
        b = P()
        check(lib().qasr_hip_batch_create(decoder.d, int(n_streams), int(max_seq), int(max_steps), C.byref(b)))
        self.b = b
        self.n_streams = int(n_streams)
        self.decoder = decoder
        decoder.dev.adopt(self)

    def prefill(self, stream, embeds):
        e = np.ascontiguousarray(embeds, np.float32)
        check(lib().qasr_hip_batch_prefill(self.b, int(stream), e.ctypes.data_as(P), e.shape[0]))

    def set_len(self, stream, n):
        check(lib().qasr_hip_batch_set_len(self.b, int(stream), int(n)))

    def length(self, stream):
        return int(lib().qasr_hip_batch_len(self.b, int(stream)))

    def set_options(self, attn_splits=-1, use_graph=True):
        check(lib().qasr_hip_batch_set_options(self.b, int(attn_splits), 1 if use_graph else 0))

    def generate(self, first_tokens, n_steps):
        ft = np.ascontiguousarray(first_tokens, np.int32)
        if ft.size != self.n_streams:
            raise ValueError("one first token per stream")
        out = np.empty((self.n_streams, int(n_steps)), np.int32)
        check(lib().qasr_hip_batch_generate(self.b, ft.ctypes.data_as(P), int(n_steps), out.ctypes.data_as(P)))
        return out

    BATCH_KINDS = ("embed", "in_norm+quant", "qkv", "qk_prep", "attention", "merge+quant", "o_proj+=",
                   "post_norm+quant", "gate_up+swiglu", "ffn_quant", "down+=", "final_norm+quant",
                   "lm_head_argmax", "argmax_finish")

    def profile(self, first_tokens, n_steps):
        """HIP-event us per launch of each kernel kind of a step (qasr_hip_batch_profile)."""
        ft = np.ascontiguousarray(first_tokens, np.int32)
        us = np.zeros(len(self.BATCH_KINDS), np.float32)
        per = np.zeros(len(self.BATCH_KINDS), np.int32)
        check(lib().qasr_hip_batch_profile(self.b, ft.ctypes.data_as(P), int(n_steps), us.ctypes.data_as(P),
                                           per.ctypes.data_as(P)))
        return [dict(kernel=k, us=float(u), per_step=int(n)) for k, u, n in zip(self.BATCH_KINDS, us, per)]

    def close(self):
        if self.b:
            lib().qasr_hip_batch_free(self.b)
            self.b = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

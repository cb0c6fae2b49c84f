"""Seeded synthetic weights, activations and audio (libqasr_synth.so).

There are no checkpoints or recordings on the GPU boxes, so every benchmark and
parity case builds its inputs here: random-init models with the reference's
tensor names and shapes (decoder.rs:71-151, encoder.rs:126-164), matrices
~ N(0, 0.02) rounded to bf16, norm gains 1 and biases 0, and 16 kHz test audio
(white noise at -30 dBFS plus three sines).
"""
import ctypes as C
import os

import numpy as np

from ._lib import SYNTH_PATH

_s = None


def _synth():
    global _s
    if _s is None:
        if not os.path.exists(SYNTH_PATH):
            raise RuntimeError(f"{SYNTH_PATH} is missing: run __graft_entry__.build() first")
        s = C.CDLL(SYNTH_PATH)
        s.qs_normal_f32.argtypes = [C.c_void_p, C.c_uint64, C.c_uint64, C.c_char_p, C.c_double, C.c_double]
        s.qs_normal_bf16.argtypes = s.qs_normal_f32.argtypes
        s.qs_audio.argtypes = [C.c_void_p, C.c_uint64, C.c_uint64, C.c_double]
        s.qs_set_threads.argtypes = [C.c_int]
        s.qs_f32_to_bf16.argtypes = [C.c_float]
        s.qs_f32_to_bf16.restype = C.c_uint16
        s.qs_set_threads(min(16, os.cpu_count() or 8))
        _s = s
    return _s


def normal_f32(shape, seed, name, mean=0.0, std=1.0):
    a = np.empty(shape, np.float32)
    _synth().qs_normal_f32(a.ctypes.data, a.size, seed, name.encode(), mean, std)
    return a


def normal_bf16(shape, seed, name, mean=0.0, std=0.02):
    a = np.empty(shape, np.uint16)
    _synth().qs_normal_bf16(a.ctypes.data, a.size, seed, name.encode(), mean, std)
    return a


def audio(n_samples, seed, noise_dbfs=-30.0):
    a = np.empty(n_samples, np.float32)
    _synth().qs_audio(a.ctypes.data, n_samples, seed, noise_dbfs)
    return a


def bf16_to_f32(a):
    return (a.astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(a):
    """Round-to-nearest-even f32 -> bf16 (finite values)."""
    u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    u = u + 0x7FFF + ((u >> 16) & 1)
    return (u >> 16).astype(np.uint16)


# QwenConfig values (config.rs:59-156)
DEC_0_6B = dict(n_layers=28, hidden=1024, n_heads=16, n_kv_heads=8, head_dim=128,
                intermediate=3072, vocab=151936, eps=1e-6, theta=1e6)
DEC_1_7B = dict(DEC_0_6B, hidden=2048, intermediate=6144)
ENC_0_6B = dict(d_model=896, n_layers=18, n_heads=14, head_dim=64, ffn_dim=3584, output_dim=1024,
                chunk_size=100, n_window_infer=800, conv_hidden=480)


class SynthDecoder:
    """Random-init Qwen3 decoder weights (host numpy, bf16 matrices)."""

    def __init__(self, cfg, seed, std=0.02):
        self.cfg = dict(cfg)
        c = self.cfg
        H, hd, I, V = c["hidden"], c["head_dim"], c["intermediate"], c["vocab"]
        qd, kvd = c["n_heads"] * hd, c["n_kv_heads"] * hd
        self.embed = normal_bf16((V, H), seed, "thinker.model.embed_tokens.weight", std=std)
        self.norm = np.ones(H, np.float32)
        self.layers = []
        for i in range(c["n_layers"]):
            p = f"thinker.model.layers.{i}"
            L = dict(
                wq=normal_bf16((qd, H), seed, f"{p}.self_attn.q_proj.weight", std=std),
                wk=normal_bf16((kvd, H), seed, f"{p}.self_attn.k_proj.weight", std=std),
                wv=normal_bf16((kvd, H), seed, f"{p}.self_attn.v_proj.weight", std=std),
                wo=normal_bf16((H, qd), seed, f"{p}.self_attn.o_proj.weight", std=std),
                gate=normal_bf16((I, H), seed, f"{p}.mlp.gate_proj.weight", std=std),
                up=normal_bf16((I, H), seed, f"{p}.mlp.up_proj.weight", std=std),
                down=normal_bf16((H, I), seed, f"{p}.mlp.down_proj.weight", std=std),
                q_norm=np.ones(hd, np.float32), k_norm=np.ones(hd, np.float32),
                input_norm=np.ones(H, np.float32), post_attn_norm=np.ones(H, np.float32),
            )
            self.layers.append(L)

    def structs(self, Config, Layer, Weights):
        """ctypes (config, weights) built from the given Structure classes."""
        c = self.cfg
        cfg = Config(**{k: c[k] for k in ("n_layers", "hidden", "n_heads", "n_kv_heads",
                                          "head_dim", "intermediate", "vocab", "eps", "theta")})
        arr = (Layer * c["n_layers"])()
        for i, L in enumerate(self.layers):
            for k, v in L.items():
                setattr(arr[i], k, v.ctypes.data)
        w = Weights(self.embed.ctypes.data, self.norm.ctypes.data, arr)
        w._keep = arr
        return cfg, w


class SynthEncoder:
    """Random-init audio encoder (encoder.rs:123-182 names/shapes)."""

    def __init__(self, cfg, seed, std=0.02):
        self.cfg = dict(cfg)
        c = self.cfg
        D, F, Cc, O = c["d_model"], c["ffn_dim"], c["conv_hidden"], c["output_dim"]
        p = "thinker.audio_tower."
        h3 = 16
        self.conv1_w = normal_bf16((Cc, 1, 3, 3), seed, p + "conv2d1.weight", std=std)
        self.conv2_w = normal_bf16((Cc, Cc, 3, 3), seed, p + "conv2d2.weight", std=std)
        self.conv3_w = normal_bf16((Cc, Cc, 3, 3), seed, p + "conv2d3.weight", std=std)
        self.conv1_b = np.zeros(Cc, np.float32)
        self.conv2_b = np.zeros(Cc, np.float32)
        self.conv3_b = np.zeros(Cc, np.float32)
        self.conv_out_w = normal_bf16((D, Cc * h3), seed, p + "conv_out.weight", std=std)
        self.layers = []
        for i in range(c["n_layers"]):
            q = f"{p}layers.{i}"
            self.layers.append(dict(
                wq=normal_bf16((D, D), seed, f"{q}.self_attn.q_proj.weight", std=std),
                wk=normal_bf16((D, D), seed, f"{q}.self_attn.k_proj.weight", std=std),
                wv=normal_bf16((D, D), seed, f"{q}.self_attn.v_proj.weight", std=std),
                wo=normal_bf16((D, D), seed, f"{q}.self_attn.out_proj.weight", std=std),
                fc1=normal_bf16((F, D), seed, f"{q}.fc1.weight", std=std),
                fc2=normal_bf16((D, F), seed, f"{q}.fc2.weight", std=std),
                bq=np.zeros(D, np.float32), bk=np.zeros(D, np.float32), bv=np.zeros(D, np.float32),
                bo=np.zeros(D, np.float32), b1=np.zeros(F, np.float32), b2=np.zeros(D, np.float32),
                ln1_w=np.ones(D, np.float32), ln1_b=np.zeros(D, np.float32),
                ln2_w=np.ones(D, np.float32), ln2_b=np.zeros(D, np.float32),
            ))
        self.ln_post_w = np.ones(D, np.float32)
        self.ln_post_b = np.zeros(D, np.float32)
        self.proj1_w = normal_bf16((D, D), seed, p + "proj1.weight", std=std)
        self.proj1_b = np.zeros(D, np.float32)
        self.proj2_w = normal_bf16((O, D), seed, p + "proj2.weight", std=std)
        self.proj2_b = np.zeros(O, np.float32)

    def structs(self, Config, Layer, Weights):
        c = self.cfg
        cfg = Config(**{k: c[k] for k in ("d_model", "n_layers", "n_heads", "head_dim", "ffn_dim",
                                          "output_dim", "chunk_size", "n_window_infer",
                                          "conv_hidden")})
        arr = (Layer * c["n_layers"])()
        for i, L in enumerate(self.layers):
            for k, v in L.items():
                setattr(arr[i], k, v.ctypes.data)
        w = Weights(self.conv1_w.ctypes.data, self.conv2_w.ctypes.data, self.conv3_w.ctypes.data,
                    self.conv_out_w.ctypes.data, self.conv1_b.ctypes.data, self.conv2_b.ctypes.data,
                    self.conv3_b.ctypes.data, arr, self.ln_post_w.ctypes.data,
                    self.ln_post_b.ctypes.data, self.proj1_w.ctypes.data, self.proj2_w.ctypes.data,
                    self.proj1_b.ctypes.data, self.proj2_b.ctypes.data)
        w._keep = arr
        return cfg, w


def decoder_tensors(w, norm_dtype="BF16"):
    """The checkpoint tensors of a SynthDecoder under the reference's names
    (decoder.rs:70-167): name -> (array, "BF16" | "F32"); bf16 arrays are uint16."""
    def norm(a):
        a = np.asarray(a, np.float32)
        return (f32_to_bf16(a), "BF16") if norm_dtype == "BF16" else (a, "F32")
    t = {"thinker.model.embed_tokens.weight": (w.embed, "BF16"), "thinker.model.norm.weight": norm(w.norm)}
    for i, L in enumerate(w.layers):
        p = f"thinker.model.layers.{i}"
        for k, n in (("wq", "self_attn.q_proj"), ("wk", "self_attn.k_proj"), ("wv", "self_attn.v_proj"),
                     ("wo", "self_attn.o_proj"), ("gate", "mlp.gate_proj"), ("up", "mlp.up_proj"),
                     ("down", "mlp.down_proj")):
            t[f"{p}.{n}.weight"] = (L[k], "BF16")
        for k, n in (("q_norm", "self_attn.q_norm"), ("k_norm", "self_attn.k_norm"),
                     ("input_norm", "input_layernorm"), ("post_attn_norm", "post_attention_layernorm")):
            t[f"{p}.{n}.weight"] = norm(L[k])
    return t


def encoder_tensors(w, vec_dtype="BF16"):
    """The checkpoint tensors of a SynthEncoder under the reference's names (encoder.rs:123-182)."""
    def vec(a):
        a = np.asarray(a, np.float32)
        return (f32_to_bf16(a), "BF16") if vec_dtype == "BF16" else (a, "F32")
    p = "thinker.audio_tower."
    t = {}
    for k in (1, 2, 3):
        t[f"{p}conv2d{k}.weight"] = (getattr(w, f"conv{k}_w"), "BF16")
        t[f"{p}conv2d{k}.bias"] = vec(getattr(w, f"conv{k}_b"))
    t[p + "conv_out.weight"] = (w.conv_out_w, "BF16")
    for i, L in enumerate(w.layers):
        q = f"{p}layers.{i}"
        for wk, bk, n in (("wq", "bq", "self_attn.q_proj"), ("wk", "bk", "self_attn.k_proj"),
                          ("wv", "bv", "self_attn.v_proj"), ("wo", "bo", "self_attn.out_proj"),
                          ("fc1", "b1", "fc1"), ("fc2", "b2", "fc2")):
            t[f"{q}.{n}.weight"] = (L[wk], "BF16")
            t[f"{q}.{n}.bias"] = vec(L[bk])
        for wk, bk, n in (("ln1_w", "ln1_b", "self_attn_layer_norm"), ("ln2_w", "ln2_b", "final_layer_norm")):
            t[f"{q}.{n}.weight"] = vec(L[wk])
            t[f"{q}.{n}.bias"] = vec(L[bk])
    t[p + "ln_post.weight"] = vec(w.ln_post_w)
    t[p + "ln_post.bias"] = vec(w.ln_post_b)
    for k in (1, 2):
        t[f"{p}proj{k}.weight"] = (getattr(w, f"proj{k}_w"), "BF16")
        t[f"{p}proj{k}.bias"] = vec(getattr(w, f"proj{k}_b"))
    return t


def write_checkpoint(path, tensors, shards=1, metadata=None):
    """Write tensors (name -> (array, "BF16" | "F32" | other numpy dtype name))
    as safetensors with the safetensors library: path/model.safetensors, or
    path/model-0000k-of-0000n.safetensors split round-robin over `shards` files."""
    import torch
    from safetensors.torch import save_file
    os.makedirs(path, exist_ok=True)
    names = sorted(tensors)
    parts = [dict() for _ in range(shards)]
    for i, n in enumerate(names):
        a, dt = tensors[n]
        a = np.ascontiguousarray(a)
        if dt == "BF16":
            t = torch.from_numpy(a.view(np.int16).copy()).view(torch.bfloat16)
        else:
            t = torch.from_numpy(a.copy())
        parts[i % shards][n] = t
    meta = metadata if metadata is not None else {"format": "pt"}
    if shards == 1:
        save_file(parts[0], os.path.join(path, "model.safetensors"), metadata=meta)
    else:
        for k, part in enumerate(parts):
            save_file(part, os.path.join(path, f"model-{k + 1:05d}-of-{shards:05d}.safetensors"), metadata=meta)

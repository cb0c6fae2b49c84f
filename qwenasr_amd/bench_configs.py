"""Measurement harness for the BASELINE configs other than the headline.

    python -m qwenasr_amd.bench_configs config0 [reps]
    python -m qwenasr_amd.bench_configs config1 [reps]
    python -m qwenasr_amd.bench_configs config3 [n_layers] [steps]
    python -m qwenasr_amd.bench_configs config4 [n_streams] [steps] [attn_splits]
    python -m qwenasr_amd.bench_configs config4_stream [n_streams] [rounds]
    python -m qwenasr_amd.bench_configs stream [seconds] [chunk_sec]
    python -m qwenasr_amd.bench_configs load [reps]

config1: the prefill / audio-encoder int8 x bf16 GEMMs at M = 375 (also 390,
404), the seven 0.6B projections and the LM head, seeded N(0,0.02) weights
packed per row on the GPU, bf16 activations N(0,1).  Each shape is timed
with HIP events over `reps` back-to-back launches; reported as TFLOP/s
against the 2.5 PFLOP/s dense bf16 MFMA peak (the kernel dequantizes int8 to
bf16 exactly and runs v_mfma_f32_16x16x32_bf16) and as HBM GB/s.

config3: Qwen3-1.7B-sized decoder (28 layers, hidden 2048, GQA 16/8,
intermediate 6144, int8 per-row weights), batch 1, bf16 KV cache filled with
N(0,1) values, at KV lengths 512, 2048 and 4096: decode us/token (graph
replay, HIP events), per-kernel us and algorithmic GB/s (the same
back-to-back timing as bench.py), int8 matvec GB/s and GQA attention us per
token.

config4: the 0.6B decoder (28 layers, int8) decoding 32 independent streams
together, each with a ragged prefix of U[100, 1500] positions (seeded;
prefilled from N(0,1) embeddings), `steps` greedy steps per stream (a 2 s
chunk's worth of text).  Reports the batched step time and aggregate
tokens/s (HIP events, graph replay), the same streams decoded one at a time
by the single-stream decoder, the token identity of the two, and the
step's algorithmic bytes (int8 weights once + every stream's KV cache) as
GB/s.

config4_stream: config 4 fed by the streaming pipeline (qasr_hip_stream_batch_*):
32 streams of their own synthetic audio with 4-20 s histories each receive a
2 s chunk per round; per round, every stream's encoder and prompt prefill go
to its slot of a multi-stream batch and all their greedy steps run batched.
Reported: wall ms per round (host clock, synchronous), seconds of audio
processed per second, against the same streams pushed one at a time through
lone states, and whether the committed token ids are identical.

stream: the streaming driver (qasr_hip_stream_*, transcribe.rs:902-1304) on the
config-2 model and audio (seeds 1002): the audio pushed `chunk_sec` at a time
(each push hands over all audio so far, as stream_push_audio does), then a
final push; per-push wall time (host clock around the synchronous push, audio
upload included), total time and realtime factor, committed tokens and the
driver's statistics, with the QwenCtx stream defaults and with 3-token
bursts (rollback 1).  Token parity of the
driver against the CPU restatement of the reference is tested in test_gpu_stream.py.

load: Decoder::load / Encoder::load of the config-2 model (0.6B, seeds 1002)
from a 2-shard safetensors checkpoint written with the safetensors library
under $TMPDIR (page cache warm: the files were just written), against the
load from host arrays: wall time per load (host clock, synchronised), and
the bf16 bytes moved per second.  Both paths upload through pinned staging
buffers and pack int8 on the GPU.

Each configuration prints one JSON line (stdout); progress goes to stderr.
"""
import json
import sys
import time

import numpy as np

from . import Device
from . import kernels as K
from ._lib import check
from .model import Batch, Decoder, Encoder, Stream, profile_decoder
from .synth import DEC_0_6B, DEC_1_7B, ENC_0_6B, SynthDecoder, SynthEncoder, audio, normal_bf16

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
# the stream is held this long per timed launch while the host enqueues them
# (a Python ctypes launch takes a few microseconds), so that they run back to
# back and the events time the GPU
HOLD_US_PER_LAUNCH = 15


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def config0(reps=256, mall_mib=256):
    """one Qwen3-0.6B decoder layer's int8 matvecs at batch
    1 through the operator entry points (the reference's kernels:: calls of
    decoder_forward): q 1024->2048, k and v 1024->1024, o 2048->1024 (+=),
    gate/up 1024->3072 (SwiGLU over interleaved rows), down 3072->1024 (+=),
    and the LM-head argmax 1024->151936; the q/k/v as one fused call too.
    Weights N(0,0.02) bf16 packed per row on the GPU; activation N(0,1) f32.
    Each projection rotates over enough distinct device copies of its weights
    (at least 32, and together more than twice the 256 MiB Infinity Cache) that
    every launch streams its matrix from HBM.  Timed with HIP events over
    `reps` launches queued behind a hold of the stream, so they run back to
    back (kernel plus the queue's inter-dispatch gap, the per-kernel method of
    bench.py); GB/s = algorithmic bytes (int8 W N*K +
    scales 4N + x 4K + y 4N, +4N read for +=, +4K gains for a fused RMSNorm)
    per launch / time."""
    dev = Device(0)
    H, qd, kvd, I, V = 1024, 2048, 1024, 3072, 151936
    x = dev.upload(np.random.default_rng(1000).standard_normal(I).astype(np.float32))
    g = dev.upload(np.random.default_rng(1001).uniform(0.5, 1.5, H).astype(np.float32))
    y = dev.empty(V, np.float32)
    idx = dev.zeros(1, np.int32)
    from ._lib import lib
    shapes = [("q", qd, H, "plain"), ("k", kvd, H, "plain"), ("v", kvd, H, "plain"), ("o", H, qd, "addto"),
              ("gate_up", 2 * I, H, "swiglu"), ("down", H, I, "addto"), ("qkv", qd + 2 * kvd, H, "qkv"),
              ("lm_head", V, H, "argmax")]
    rows, layer_bytes, layer_us = [], 0.0, 0.0
    for name, N, Kd, kind in shapes:
        wb = dev.upload(normal_bf16((N, Kd), 1000, f"w0_{name}"))
        q0 = dev.empty((N, Kd), np.int8)
        s0 = dev.empty(N, np.float32)
        K.quantize_bf16_weights_to_int8(wb, N, Kd, q0, s0)
        wb.free()
        per = N * Kd
        n_copies = max(32, -(-2 * (mall_mib << 20) // per))
        copies = []
        for _ in range(n_copies):
            qc, sc = dev.empty((N, Kd), np.int8), dev.empty(N, np.float32)
            dev.copy(qc, q0)
            dev.copy(sc, s0)
            copies.append((qc, sc))
        dev.sync()
        h = dev.h

        def launch(i):
            qw, sw = copies[i % n_copies]
            if kind == "plain":
                check(lib().qasr_hip_linear_int8(h, y.ptr, x.ptr, qw.ptr, sw.ptr, None, Kd, N))
            elif kind == "addto":
                check(lib().qasr_hip_linear_int8_addto(h, y.ptr, x.ptr, qw.ptr, sw.ptr, Kd, N))
            elif kind == "swiglu":
                check(lib().qasr_hip_rmsnorm_linear_int8_swiglu(h, y.ptr, x.ptr, g.ptr, 1e-6, qw.ptr,
                                                                sw.ptr, Kd, N // 2))
            elif kind == "qkv":
                check(lib().qasr_hip_rmsnorm_linear_int8_qkv(
                    h, y.ptr, y.offset(qd), y.offset(qd + kvd), x.ptr, g.ptr, 1e-6, qw.ptr, sw.ptr,
                    qw.offset(qd * H), sw.offset(qd), qw.offset((qd + kvd) * H), sw.offset(qd + kvd), H, qd, kvd))
            else:
                check(lib().qasr_hip_rmsnorm_argmax_int8(h, x.ptr, g.ptr, 1e-6, qw.ptr, sw.ptr, Kd, N,
                                                         idx.ptr))
        for i in range(n_copies):           # warm-up: every copy once
            launch(i)
        dev.sync()
        dev.timer_hold(HOLD_US_PER_LAUNCH * reps)
        dev.timer_start()
        for i in range(reps):
            launch(i)
        ms = dev.timer_stop() / reps
        byts = per + 4.0 * N + 4.0 * Kd + (4.0 * N if kind != "argmax" else 0.0)
        if kind == "addto":
            byts += 4.0 * N
        if kind in ("swiglu", "qkv", "argmax"):
            byts += 4.0 * Kd
        if kind == "swiglu":
            byts -= 2.0 * N                  # N/2 outputs
        gbs = byts / (ms * 1e6)
        r = dict(shape=name, N=N, K=Kd, copies=n_copies, us=round(ms * 1e3, 3), bytes=byts, gbs=round(gbs, 1),
                 frac=round(gbs / HBM_PEAK_GBS, 4))
        rows.append(r)
        if name in ("q", "k", "v", "o", "gate_up", "down"):
            layer_bytes += byts
            layer_us += ms * 1e3
        log(f"[config0] {name:8s} {N:6d}x{Kd:4d} x{n_copies:3d} copies: {r['us']:8.3f} us  {r['gbs']:8.1f} GB/s "
            f"({100 * r['frac']:.1f}% of 8 TB/s)")
        for qc, sc in copies:
            qc.free()
            sc.free()
        q0.free()
        s0.free()
    layer = dict(bytes=layer_bytes, us=round(layer_us, 3), gbs=round(layer_bytes / (layer_us * 1e3), 1),
                 frac=round(layer_bytes / (layer_us * 1e3) / HBM_PEAK_GBS, 4))
    log(f"[config0] one layer (q, k, v, o, gate_up, down as separate launches): {layer['us']:.2f} us, "
        f"{layer['gbs']:.1f} GB/s")
    print(json.dumps({"config": "config 0: one 0.6B layer's int8 matvecs at batch 1 (operator entry points)",
                      "results": rows, "layer": layer}))
    dev.close()


def config1(reps=20, calib_mib=0):
    """calib_mib > 0: first one device copy of that many MiB (the library's
    copy kernel), the calibration launch of a FETCH_SIZE / WRITE_SIZE counter run."""
    dev = Device(0)
    if calib_mib > 0:
        src = dev.zeros(calib_mib << 20, np.uint8)
        dst = dev.empty(calib_mib << 20, np.uint8)
        dev.copy(dst, src)
        dev.sync()
        src.free()
        dst.free()
    shapes = [("q", 2048, 1024), ("k", 1024, 1024), ("v", 1024, 1024), ("o", 1024, 2048),
              ("gate", 3072, 1024), ("up", 3072, 1024), ("down", 1024, 3072), ("lm_head", 151936, 1024)]
    rows = []
    for M in (375, 390, 404):
        for name, N, Kd in shapes:
            wb = dev.upload(normal_bf16((N, Kd), 1001, f"w_{name}"))
            q = dev.empty((N, Kd), np.int8)
            s = dev.empty(N, np.float32)
            K.quantize_bf16_weights_to_int8(wb, N, Kd, q, s)
            a = dev.upload(normal_bf16((M, Kd), 1001, f"a_{name}_{M}", std=1.0))
            y = dev.empty((M, N), np.float32)
            K.gemm_w8_bf16(y, a, q, s, M, N, Kd)          # warm-up
            dev.sync()
            dev.timer_hold(HOLD_US_PER_LAUNCH * reps)
            dev.timer_start()
            for _ in range(reps):
                K.gemm_w8_bf16(y, a, q, s, M, N, Kd)
            ms = dev.timer_stop() / reps
            flops = 2.0 * M * N * Kd
            byts = N * Kd + 4.0 * N + 2.0 * M * Kd + 4.0 * M * N
            r = dict(M=M, shape=name, N=N, K=Kd, us=round(ms * 1e3, 2), tflops=round(flops / (ms * 1e9), 1),
                     mfma_frac=round(flops / (ms * 1e9) / BF16_PEAK_TFLOPS, 4), gbs=round(byts / (ms * 1e6), 1))
            rows.append(r)
            log(f"[config1] M={M} {name:8s} {N}x{Kd}: {r['us']:9.2f} us  {r['tflops']:7.1f} TFLOP/s "
                f"({100 * r['mfma_frac']:.1f}% of bf16 MFMA)  {r['gbs']:8.1f} GB/s")
            for d in (wb, q, s, a, y):
                d.free()
    print(json.dumps({"config": "config 1: int8 x bf16 GEMM (prefill / encoder shapes)", "results": rows}))
    dev.close()


def config3(n_layers=28, steps=20):
    dev = Device(0)
    cfg = dict(DEC_1_7B, n_layers=n_layers)
    t0 = time.time()
    w = SynthDecoder(cfg, seed=1003)
    log(f"[config3] synthetic 1.7B decoder ({n_layers} layers) in {time.time() - t0:.1f}s")
    contexts = (512, 2048, 4096)
    max_seq = contexts[-1] + 2 * steps + 8
    dec = Decoder(dev, w, max_seq=max_seq, kv_bf16=True)
    rng = np.random.default_rng(1003)
    shape = dec.kv_shape()
    k = rng.standard_normal(shape, dtype=np.float32)
    v = rng.standard_normal(shape, dtype=np.float32)
    dec.kv_upload(k, v)
    del k, v
    log("[config3] weights packed, bf16 KV filled with N(0,1)")
    res = []
    for L in contexts:
        dec.kv_len = L
        dec.generate(2, first_token=17)                 # captures the graph of this bucket
        dec.kv_len = L
        dev.sync()
        dev.timer_start()
        dec.generate(steps, first_token=17)
        us_tok = dev.timer_stop() * 1e3 / steps
        dec.kv_len = L
        prof = profile_decoder(dec, steps)
        # the qkv matvec and the attention run as one launch (kind 0) when the
        # attention kind launched nothing
        if prof[1]["per_step"] == 0:
            prof[0]["kernel"] = "norm+qkv+attention"
            prof = [p for p in prof if p["per_step"] > 0]
        kern = {}
        for p in prof:
            kern[p["kernel"]] = dict(us=round(p["us"], 3), bytes=p["bytes"],
                                     gbs=round(p["bytes"] / (p["us"] * 1e3), 1) if p["us"] > 0 else 0.0,
                                     per_step=p["per_step"])
        mv = [p for p in prof if "attention" not in p["kernel"] and p["kernel"] != "argmax_merge"]
        mv_bytes = sum(p["bytes"] * p["per_step"] for p in mv)
        mv_us = sum(p["us"] * p["per_step"] for p in mv)
        att = [p for p in prof if "attention" in p["kernel"]][0]
        r = dict(kv_len=L, decode_us_per_token=round(us_tok, 2),
                 int8_matvec_gbs=round(mv_bytes / (mv_us * 1e3), 1),
                 int8_matvec_frac=round(mv_bytes / (mv_us * 1e3) / HBM_PEAK_GBS, 4),
                 attention_kernel=att["kernel"],
                 attention_us_per_layer=round(att["us"], 3), attention_us_per_token=round(att["us"] * att["per_step"], 2),
                 attention_gbs=round(att["bytes"] / (att["us"] * 1e3), 1), kernels=kern)
        res.append(r)
        log(f"[config3] L={L}: {us_tok:.1f} us/token; matvecs {r['int8_matvec_gbs']} GB/s "
            f"({100 * r['int8_matvec_frac']:.1f}%); {att['kernel']} {att['us']:.2f} us/layer "
            f"({r['attention_gbs']} GB/s); " + ", ".join(f"{k_} {v_['us']}" for k_, v_ in kern.items()))
    print(json.dumps({"config": f"config 3: Qwen3-1.7B-sized decoder, {n_layers} layers, bf16 KV, batch 1",
                      "results": res}))
    dec.close()
    dev.close()


def config4(n_streams=32, steps=32, splits=-1):
    dev = Device(0)
    cfg = dict(DEC_0_6B)
    t0 = time.time()
    w = SynthDecoder(cfg, seed=1004)
    log(f"[config4] synthetic 0.6B decoder in {time.time() - t0:.1f}s")
    rng = np.random.default_rng(1004)
    lens = rng.integers(100, 1501, n_streams)
    first = rng.integers(0, cfg["vocab"], n_streams)
    max_seq = 2048
    dec = Decoder(dev, w, max_seq=max_seq)
    bat = Batch(dec, n_streams, max_seq, max_steps=steps)
    bat.set_options(attn_splits=splits)
    dec.set_options(attn_splits=splits)
    H = cfg["hidden"]
    prefixes = [rng.standard_normal((int(L), H), dtype=np.float32) for L in lens]
    t0 = time.time()
    for i, p in enumerate(prefixes):
        bat.prefill(i, p)
    dev.sync()
    log(f"[config4] {n_streams} prefixes prefilled ({int(lens.sum())} positions) in {time.time() - t0:.1f}s")
    # warm-up: capture the step graphs of every split count the run meets
    toks = bat.generate(first, steps)
    for i in range(n_streams):
        bat.set_len(i, int(lens[i]))
    reps, times = 3, []
    for _ in range(reps):
        dev.sync()
        dev.timer_start()
        toks = bat.generate(first, steps)
        times.append(dev.timer_stop())
        for i in range(n_streams):
            bat.set_len(i, int(lens[i]))
    ms = float(np.median(times))
    us_step = ms * 1e3 / steps
    tok_s = n_streams * steps / (ms / 1e3)
    log(f"[config4] batched: {us_step:.1f} us/step, {tok_s:.0f} tokens/s ({n_streams} streams)")
    # per-kernel HIP-event timing of the step at the mid-run lengths
    for i in range(n_streams):
        bat.set_len(i, int(lens[i]) + steps // 2)
    prof = [p for p in bat.profile(first, 4) if p["per_step"]]   # kinds the step launches
    for i in range(n_streams):
        bat.set_len(i, int(lens[i]))
    c_ = cfg
    H_, hd_, I_ = c_["hidden"], c_["head_dim"], c_["intermediate"]
    qd_, kvd_ = c_["n_heads"] * hd_, c_["n_kv_heads"] * hd_
    B_ = n_streams
    ctx = float((lens + steps // 2 + 1).sum())
    # algorithmic bytes per launch: int8 weights + scales once, activations per stream
    kbytes = {"qkv": (qd_ + 2 * kvd_) * (H_ + 4) + B_ * (H_ + 4 * (qd_ + 2 * kvd_)),
              "attention": 2 * kvd_ * 4 * ctx + B_ * 4 * (qd_ + 2 * kvd_),
              "o_proj+=": H_ * (qd_ + 4) + B_ * (qd_ + 8 * H_),
              "gate_up+swiglu": 2 * I_ * (H_ + 4) + B_ * (H_ + 4 * I_),
              "down+=": H_ * (I_ + 4) + B_ * (I_ + 8 * H_),
              "lm_head_argmax": c_["vocab"] * (H_ + 4) + B_ * H_}
    for p in prof:
        p["bytes"] = kbytes.get(p["kernel"], 0)
        p["gbs"] = round(p["bytes"] / (p["us"] * 1e3), 1) if p["us"] > 0 and p["bytes"] else None
        p["us_per_step"] = round(p["us"] * p["per_step"], 2)
        p["us"] = round(p["us"], 3)
        log(f"[config4] {p['kernel']:18s} {p['us']:8.2f} us x{p['per_step']:2d} = {p['us_per_step']:8.1f} us/step"
            + (f"  {p['gbs']} GB/s" if p["gbs"] else ""))
    # the same streams one at a time on the single-stream decoder
    solo_ms, match = 0.0, 0
    for i in range(n_streams):
        dec.kv_len = 0
        dec.prefill(prefixes[i])
        dec.generate(2, first_token=int(first[i]))          # graph capture of the bucket
        dec.kv_len = int(lens[i])
        dev.sync()
        dev.timer_start()
        t = dec.generate(steps, first_token=int(first[i]))
        solo_ms += dev.timer_stop()
        match += int((t == toks[i]).all())
    solo_tok_s = n_streams * steps / (solo_ms / 1e3)
    log(f"[config4] one at a time: {solo_ms * 1e3 / (n_streams * steps):.1f} us/token, {solo_tok_s:.0f} tokens/s; "
        f"identical streams {match}/{n_streams}")
    # algorithmic bytes of one batched step: int8 weights (+ scales) once and
    # every stream's K/V rows (f32) at the mid-run context
    c = cfg
    hd, qd, kvd, I = c["head_dim"], c["n_heads"] * c["head_dim"], c["n_kv_heads"] * c["head_dim"], c["intermediate"]
    per_layer_w = (qd + 2 * kvd) * (H + 4) + H * (qd + 4) + 2 * I * (H + 4) + H * (I + 4)
    w_bytes = c["n_layers"] * per_layer_w + c["vocab"] * (H + 4)
    mid = lens + steps // 2
    kv_bytes = int(c["n_layers"] * 2 * kvd * 4 * mid.sum())
    gbs = (w_bytes + kv_bytes) / (us_step * 1e3)
    print(json.dumps({"config": f"config 4: Qwen3-ASR-0.6B decoder, {n_streams} streams, prefixes U[100,1500], "
                                f"{steps} greedy steps per stream, f32 KV",
                      "attn_splits": "automatic" if splits < 0 else splits,
                      "prefix_lens": [int(x) for x in lens],
                      "batched_us_per_step": round(us_step, 2), "batched_tokens_per_s": round(tok_s, 1),
                      "solo_us_per_token": round(solo_ms * 1e3 / (n_streams * steps), 2),
                      "solo_tokens_per_s": round(solo_tok_s, 1), "speedup": round(tok_s / solo_tok_s, 2),
                      "identical_streams": f"{match}/{n_streams}",
                      "step_bytes": {"weights": w_bytes, "kv": kv_bytes},
                      "step_gbs": round(gbs, 1), "step_frac_of_hbm": round(gbs / HBM_PEAK_GBS, 4),
                      "kernels": prof}))
    bat.close()
    dec.close()
    dev.close()


def stream(seconds=30.0, chunk_sec=2.0):
    dev = Device(0)
    t0 = time.time()
    wd = SynthDecoder(DEC_0_6B, seed=1002)
    we = SynthEncoder(ENC_0_6B, seed=1002)
    n = int(round(seconds * 16000))
    x = audio(n, 1002)
    dec = Decoder(dev, wd, max_seq=2048)
    enc = Encoder(dev, we)
    dev.sync()
    log(f"[stream] model and {seconds:.0f} s audio ready in {time.time() - t0:.1f}s")
    step = int(round(chunk_sec * 16000))
    ends = list(range(step, n + 1, step))
    res = {}
    # the defaults (a random-init model repeats itself, so the degeneracy rule
    # resets the stream every chunk: full prefill, 32 decode steps per push)
    # and short bursts (no reset: prefix reuse and delta prefill every push)
    for label, cfg in (("defaults", {}), ("bursts_of_3", {"max_new_tokens": 3, "rollback": 1})):
        for rep in range(2):                       # the first pass warms the graphs and buffers
            st = Stream(dec, enc, chunk_sec=chunk_sec, **cfg)
            times, emitted = [], 0
            for end in ends:
                c0 = time.perf_counter()
                emitted += len(st.push(x[:end]))
                times.append(time.perf_counter() - c0)
            c0 = time.perf_counter()
            emitted += len(st.push(x[:n], finalize=True))
            t_final = time.perf_counter() - c0
            stats = [int(v) for v in st.stats()]
            ntok = len(st.tokens())
            st.close()
        total = sum(times) + t_final
        res[label] = {"pushes": len(ends) + 1, "push_ms_mean": round(1000 * float(np.mean(times)), 2),
                      "push_ms_max": round(1000 * float(np.max(times)), 2),
                      "push_ms_last_chunk": round(1000 * times[-1], 2), "final_push_ms": round(1000 * t_final, 2),
                      "total_ms": round(1000 * total, 2), "realtime_factor": round(seconds / total, 2),
                      "committed_tokens": ntok, "stats": stats}
        log(f"[stream] {label}: {len(ends)} pushes of {chunk_sec} s, mean {res[label]['push_ms_mean']} ms, "
            f"max {res[label]['push_ms_max']} ms; total {res[label]['total_ms']} ms = "
            f"{res[label]['realtime_factor']}x realtime; {ntok} tokens; stats {stats}")
    print(json.dumps({"config": f"streaming driver: Qwen3-ASR-0.6B (28-layer int8 decoder, 18-layer encoder), "
                                f"{seconds:.0f} s synthetic audio pushed in {chunk_sec} s chunks",
                      "stats_columns": ["chunk_idx", "reused_rows", "prefill_len", "delta_rows", "forwards",
                                        "forwards_total", "encoder_windows", "raw_tokens"],
                      "results": res}))
    dec.close()
    enc.close()
    dev.close()


def config4_stream(n_streams=32, rounds=3, chunk_sec=2.0):
    """Config 4 fed by the real pipeline: n_streams streams of their own audio
    (seeds 1004 + i) with ragged histories (stream i starts with 4-20 s
    already pushed), then `rounds` timed rounds in which every stream receives
    the next 2 s chunk: a StreamBatch push (per stream: encoder window(s) and
    prompt prefill into its batch slot; one batched greedy decode for all),
    against the same streams pushed one at a time through lone Stream states
    on the same decoder.  Host clock around the synchronous pushes; token ids
    must be identical."""
    from .model import StreamBatch
    dev = Device(0)
    t0 = time.time()
    wd = SynthDecoder(DEC_0_6B, seed=1004)
    we = SynthEncoder(ENC_0_6B, seed=1004)
    step = int(round(chunk_sec * 16000))
    rng = np.random.default_rng(1004)
    start_chunks = rng.integers(2, 11, n_streams)            # 4-20 s already pushed
    total = [int(c + rounds) * step for c in start_chunks]
    xs = [audio(n, 1004 + i) for i, n in enumerate(total)]
    dec = Decoder(dev, wd, max_seq=1024)
    enc = Encoder(dev, we)
    dev.sync()
    log(f"[config4_stream] models and audio ready in {time.time() - t0:.1f}s")
    res = {}
    got = {}
    for mode in ("batched", "one_at_a_time"):
        times, tok_rounds, phases = [], [], []
        if mode == "batched":
            g = StreamBatch(dec, enc, n_streams, 1024)
            g.push([x[:int(c) * step] for x, c in zip(xs, start_chunks)])          # history, untimed
            for r in range(rounds):
                ends = [int(c + r + 1) * step for c in start_chunks]
                c0 = time.perf_counter()
                out = g.push([x[:e] for x, e in zip(xs, ends)])
                times.append(time.perf_counter() - c0)
                phases.append([round(v, 2) for v in g.times()])
                tok_rounds.append([o.tolist() for o in out])
            stats = [[int(v) for v in g.stream(i).stats()] for i in range(n_streams)]
            g.close()
        else:
            # a lone state keeps its reusable prompt rows in the decoder's own
            # KV cache, so each stream runs all its rounds before the next one;
            # a round's time is the sum over the streams
            times = [0.0] * rounds
            tok_rounds = [[None] * n_streams for _ in range(rounds)]
            stats = []
            for i, (x, c) in enumerate(zip(xs, start_chunks)):
                s_ = Stream(dec, enc)
                s_.push(x[:int(c) * step])
                for r in range(rounds):
                    c0 = time.perf_counter()
                    o = s_.push(x[:int(c + r + 1) * step])
                    times[r] += time.perf_counter() - c0
                    tok_rounds[r][i] = o.tolist()
                stats.append([int(v) for v in s_.stats()])
                s_.close()
        got[mode] = tok_rounds
        ms = 1000.0 * float(np.median(times))
        fwd = sum(st[4] for st in stats)
        res[mode] = {"round_ms": [round(1000 * t, 2) for t in times], "round_ms_median": round(ms, 2),
                     "audio_s_per_wall_s": round(n_streams * chunk_sec / (ms / 1000.0), 1),
                     "last_round_forwards_per_stream": [st[4] for st in stats],
                     "last_round_prefill_rows": [st[2] for st in stats]}
        if phases:
            # GPU-timeline phases of each round: the encoder pass over every
            # stream's new windows and tails, the prompt rows and prefix
            # comparison, the multi-stream prefill, the batched decode
            res[mode]["phase_ms"] = {"encoder": [p[0] for p in phases], "prompt_rows": [p[1] for p in phases],
                                     "prefill": [p[2] for p in phases], "decode": [p[3] for p in phases]}
        log(f"[config4_stream] {mode}: rounds {res[mode]['round_ms']} ms; "
            f"{res[mode]['audio_s_per_wall_s']} s of audio per s; last-round forwards {fwd}")
    same = got["batched"] == got["one_at_a_time"]
    print(json.dumps({"config": f"config 4 from the streaming pipeline: Qwen3-ASR-0.6B (28-layer int8 decoder, "
                                f"18-layer encoder), {n_streams} streams, histories of 4-20 s, {rounds} rounds of "
                                f"{chunk_sec} s chunks per stream, QwenCtx stream defaults",
                      "start_seconds": [int(c) * chunk_sec for c in start_chunks], "results": res,
                      "speedup": round(res["one_at_a_time"]["round_ms_median"] / res["batched"]["round_ms_median"], 2),
                      "identical_tokens": same}))
    dec.close()
    enc.close()
    dev.close()


def load(reps=3):
    import os
    import shutil
    import tempfile
    from .model import Checkpoint
    from .synth import decoder_tensors, encoder_tensors, write_checkpoint
    dev = Device(0)
    wd = SynthDecoder(DEC_0_6B, seed=1002)
    we = SynthEncoder(ENC_0_6B, seed=1002)
    tens = decoder_tensors(wd)
    tens.update(encoder_tensors(we))
    d = tempfile.mkdtemp(prefix="qasr_ckpt_")
    try:
        t0 = time.perf_counter()
        write_checkpoint(d, tens, shards=2)
        size = sum(os.path.getsize(os.path.join(d, f)) for f in os.listdir(d))
        log(f"[load] checkpoint written: {size / 1e9:.3f} GB in {time.perf_counter() - t0:.1f}s")
        dec_bytes = sum(a.nbytes for n, (a, _) in tens.items() if n.startswith("thinker.model."))
        enc_bytes = sum(a.nbytes for n, (a, _) in tens.items() if n.startswith("thinker.audio_tower."))
        rows = {"pointer": [], "checkpoint": []}
        for rep in range(reps + 1):              # the first round warms the allocator and the page cache
            t0 = time.perf_counter()
            dec = Decoder(dev, wd, max_seq=2048)
            dev.sync()
            t1 = time.perf_counter()
            enc = Encoder(dev, we)
            dev.sync()
            t2 = time.perf_counter()
            dec.close()
            enc.close()
            t3 = time.perf_counter()
            ck = Checkpoint(d)
            t4 = time.perf_counter()
            dec = Decoder.from_checkpoint(dev, ck, DEC_0_6B, max_seq=2048)
            dev.sync()
            t5 = time.perf_counter()
            enc = Encoder.from_checkpoint(dev, ck, ENC_0_6B)
            dev.sync()
            t6 = time.perf_counter()
            ck.close()
            dec.close()
            enc.close()
            if rep:
                rows["pointer"].append((t1 - t0, t2 - t1, 0.0))
                rows["checkpoint"].append((t5 - t4, t6 - t5, t4 - t3))
            log(f"[load] rep {rep}: host arrays decoder {1e3 * (t1 - t0):.1f} ms encoder {1e3 * (t2 - t1):.1f} ms; "
                f"checkpoint open {1e3 * (t4 - t3):.2f} ms decoder {1e3 * (t5 - t4):.1f} ms "
                f"encoder {1e3 * (t6 - t5):.1f} ms")
        res = {}
        for k, v in rows.items():
            a = np.array(v)
            dms, ems, oms = (1e3 * a.mean(axis=0)).tolist()
            res[k] = {"decoder_ms": round(dms, 1), "encoder_ms": round(ems, 1), "open_ms": round(oms, 2),
                      "decoder_GBps": round(dec_bytes / dms / 1e6, 1), "encoder_GBps": round(enc_bytes / ems / 1e6, 1)}
        print(json.dumps({"config": "Decoder::load + Encoder::load, Qwen3-ASR-0.6B bf16 weights "
                                    f"({dec_bytes / 1e9:.3f} + {enc_bytes / 1e9:.3f} GB), int8 packing on the GPU",
                          "checkpoint": "2 safetensors shards, page cache warm", "reps": reps, "results": res}))
    finally:
        shutil.rmtree(d, ignore_errors=True)
        dev.close()


if __name__ == "__main__":
    what = sys.argv[1] if len(sys.argv) > 1 else "config3"
    if what == "config0":
        config0(int(sys.argv[2]) if len(sys.argv) > 2 else 256)
    elif what == "config1":
        config1(int(sys.argv[2]) if len(sys.argv) > 2 else 20, int(sys.argv[3]) if len(sys.argv) > 3 else 0)
    elif what == "config3":
        config3(int(sys.argv[2]) if len(sys.argv) > 2 else 28, int(sys.argv[3]) if len(sys.argv) > 3 else 20)
    elif what == "config4":
        config4(int(sys.argv[2]) if len(sys.argv) > 2 else 32, int(sys.argv[3]) if len(sys.argv) > 3 else 32,
                int(sys.argv[4]) if len(sys.argv) > 4 else -1)
    elif what == "config4_stream":
        config4_stream(int(sys.argv[2]) if len(sys.argv) > 2 else 32, int(sys.argv[3]) if len(sys.argv) > 3 else 3)
    elif what == "stream":
        stream(float(sys.argv[2]) if len(sys.argv) > 2 else 30.0, float(sys.argv[3]) if len(sys.argv) > 3 else 2.0)
    elif what == "load":
        load(int(sys.argv[2]) if len(sys.argv) > 2 else 3)
    else:
        raise SystemExit(f"unknown configuration {what!r}")

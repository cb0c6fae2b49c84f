// The reference's C API (c_api.rs) over the device-resident engine, at token
// level: text is a sequence of token ids, which the caller's tokenizer
// (tokenizer.rs) turns into bytes.  QwenCtx::load (context.rs:86-150) becomes
// qasr_hip_engine_load: one handle, the checkpoint mapping, the decoder and the
// encoder with the model variant detected from tensor shapes
// (QwenConfig::detect, config.rs:108-156).
#include "model.h"

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <string>
#include <vector>

struct qasr_engine {
    qasr_hip *h = nullptr;
    qasr_st *st = nullptr;
    qasr_decoder *d = nullptr;
    qasr_encoder *e = nullptr;
    qasr_dec_config dc{};
    qasr_enc_config ec{};
    qasr_stream_config scfg{};      // QwenCtx's stream_* fields (context.rs:146-150)
    int32_t max_tokens = 2048;      // transcribe_segment's max_tokens (transcribe.rs:188)
    float segment_sec = 0.0f;       // QwenCtx::segment_sec / search_sec (context.rs:144-145)
    float search_sec = 3.0f;
    std::vector<int32_t> prompt;    // QwenCtx::prompt_tokens
    std::vector<int32_t> force;     // QwenCtx::force_prompt_tokens ("language X" ids + <asr_text>)
    std::vector<int32_t> raw;       // the last transcription's tokens, segment after segment
    std::vector<int64_t> segments;  // the last transcription's segments, 4 values each
    std::vector<qasr_engine_stream *> streams;   // live stream states, detached at engine_free
    // the last caller that wrote the decoder's KV cache (the engine itself for
    // transcribe_pcm, else a stream): a stream whose previous rows were
    // overwritten in between prefills every row on its next push
    const void *kv_owner = nullptr;
};

struct qasr_engine_stream {
    qasr_engine *eng = nullptr;
    qasr_stream *s = nullptr;
    std::vector<float> audio;       // QwenAsrStreamState::audio_buf (c_api.rs:171-175)
};

namespace {

bool shape_of(const qasr_st *st, const std::string &name, std::vector<int64_t> &shape) {
    int dtype = 0, nd = 0;
    int64_t sh[8] = {};
    const void *data = nullptr;
    int64_t bytes = 0;
    if (qasr_hip_st_find(st, name.c_str(), &dtype, &nd, sh, &data, &bytes) != QASR_OK) return false;
    shape.assign(sh, sh + nd);
    return true;
}

bool has(const qasr_st *st, const std::string &name) {
    std::vector<int64_t> s;
    return shape_of(st, name, s);
}

int count_layers(const qasr_st *st, const std::string &prefix, const std::string &suffix) {
    int n = 0;
    while (has(st, prefix + std::to_string(n) + suffix)) n++;
    return n;
}

}  // namespace

// QwenConfig::detect (config.rs:108-156) from the checkpoint's tensor shapes:
// decoder hidden from embed_tokens [vocab, hidden], intermediate from layer
// 0's gate_proj [intermediate, hidden]; the large encoder (1024 wide, 16
// heads, ffn 4096) when audio_tower layer 18 exists, else the small one (896,
// 14 heads, ffn 3584).  The reference takes the layer counts from its
// defaults (decoder 28, encoder 24 or 18), which are the numbers of layers its
// checkpoints hold; here they are counted in the checkpoint, which gives the
// same numbers for those and also loads reduced test checkpoints.
extern "C" int qasr_hip_engine_detect(const qasr_st *st, qasr_dec_config *dc, qasr_enc_config *ec) {
    if (!st || !dc || !ec) return qasr_fail(QASR_ERR_INVALID, "engine_detect: null argument");
    std::vector<int64_t> emb, gate;
    if (!shape_of(st, "thinker.model.embed_tokens.weight", emb) || emb.size() != 2)
        return qasr_fail(QASR_ERR_INVALID, "engine_detect: no thinker.model.embed_tokens.weight [vocab, hidden]");
    const bool large = has(st, "thinker.audio_tower.layers.18.self_attn.q_proj.weight");
    const int64_t hidden = emb[1];
    int64_t inter = hidden >= 2048 ? 6144 : 3072;
    if (shape_of(st, "thinker.model.layers.0.mlp.gate_proj.weight", gate) && gate.size() == 2) inter = gate[0];
    *dc = qasr_dec_config{};
    dc->n_layers = count_layers(st, "thinker.model.layers.", ".self_attn.q_proj.weight");
    dc->hidden = (int32_t)hidden;
    dc->n_heads = 16;
    dc->n_kv_heads = 8;
    dc->head_dim = 128;
    dc->intermediate = (int32_t)inter;
    dc->vocab = (int32_t)emb[0];
    dc->eps = 1e-6f;
    dc->theta = 1e6f;
    *ec = qasr_enc_config{};
    ec->d_model = large ? 1024 : 896;
    ec->n_layers = count_layers(st, "thinker.audio_tower.layers.", ".self_attn.q_proj.weight");
    ec->n_heads = large ? 16 : 14;
    ec->head_dim = 64;
    ec->ffn_dim = large ? 4096 : 3584;
    ec->output_dim = (int32_t)hidden;
    ec->chunk_size = 100;             // enc_n_window * 2 (config.rs:154)
    ec->n_window_infer = 800;
    ec->conv_hidden = 480;
    if (dc->n_layers <= 0 || ec->n_layers <= 0)
        return qasr_fail(QASR_ERR_INVALID, "engine_detect: no decoder or encoder layers in the checkpoint");
    return QASR_OK;
}

// Frees the engine; stream states still alive lose their device state here
// (they hold the engine's decoder and encoder) and afterwards only accept
// qasr_hip_engine_stream_free, which then frees just the handle.
extern "C" void qasr_hip_engine_free(qasr_engine *g) {
    if (!g) return;
    for (qasr_engine_stream *s : g->streams) {
        if (s->s) qasr_hip_stream_free(s->s);
        s->s = nullptr;
        s->eng = nullptr;
    }
    g->streams.clear();
    if (g->d) qasr_hip_decoder_free(g->d);
    if (g->e) qasr_hip_encoder_free(g->e);
    if (g->st) qasr_hip_st_free(g->st);
    if (g->h) qasr_hip_destroy(g->h);
    delete g;
}

// qwen_asr_load_model (c_api.rs:20-46): n_threads and verbosity size the
// reference's CPU pool and logging; here the device index selects the GPU.
// The KV cache holds max_seq positions (the prompt of the longest audio plus
// max_tokens); 0 picks 8192 (about 11 minutes of audio with 2048 tokens).
extern "C" int qasr_hip_engine_load(const char *model_dir, int device, int64_t max_seq, qasr_engine **out) {
    if (!model_dir || !out) return qasr_fail(QASR_ERR_INVALID, "engine_load: null argument");
    *out = nullptr;
    qasr_engine *g = new qasr_engine();
    int rc = qasr_hip_create(device, &g->h);
    if (rc == QASR_OK) rc = qasr_hip_st_open(model_dir, &g->st);
    if (rc == QASR_OK) rc = qasr_hip_engine_detect(g->st, &g->dc, &g->ec);
    if (rc == QASR_OK) rc = qasr_hip_encoder_load_st(g->h, g->st, &g->ec, &g->e);
    if (rc == QASR_OK)
        rc = qasr_hip_decoder_load_st(g->h, g->st, &g->dc, QASR_ROUND_HALF_AWAY, max_seq > 0 ? max_seq : 8192, 0,
                                      &g->d);
    if (rc != QASR_OK) {
        qasr_hip_engine_free(g);
        return rc;
    }
    qasr_hip_stream_default_config(&g->scfg);
    *out = g;
    return QASR_OK;
}

extern "C" int qasr_hip_engine_config(const qasr_engine *g, qasr_dec_config *dc, qasr_enc_config *ec) {
    if (!g) return qasr_fail(QASR_ERR_INVALID, "engine is null");
    if (dc) *dc = g->dc;
    if (ec) *ec = g->ec;
    return QASR_OK;
}

// Rust's `f32 as usize`: truncation toward zero, negative and NaN to 0
static int64_t f32_to_count(float v) {
    if (!(v > 0.0f)) return 0;
    if (v >= 9.2e18f) return INT64_MAX;
    return (int64_t)v;
}

// find_split_point (transcribe.rs:252-277): the center of the 1600-sample
// window (hop 800) of least mean square inside target +- search_sec, the first
// of equal minima; target when no window fits.  The energy is a sequential f32
// sum of squares (built without contraction), as the reference adds it.
static int64_t find_split_point(const float *x, int64_t n, int64_t target, float search_sec) {
    const int64_t half = f32_to_count(search_sec * 16000.0f);
    const int64_t lo = std::max<int64_t>(target - half, 0), hi = std::min(target + half, n);
    constexpr int64_t WIN = 1600;
    float best = 1e30f;
    int64_t center = target;
    for (int64_t pos = lo; pos + WIN <= hi; pos += WIN / 2) {
        const int64_t end = std::min(pos + WIN, n);
        float energy = 0.0f;
        for (int64_t i = pos; i < end; i++) energy += x[i] * x[i];
        energy /= (float)(end - pos);
        if (energy < best) {
            best = energy;
            center = pos + (end - pos) / 2;
        }
    }
    return center;
}

// transcribe_audio's split list (transcribe.rs:323-341)
extern "C" int64_t qasr_hip_segment_splits(const float *samples, int64_t n, float segment_sec, float search_sec,
                                           int64_t *splits_out, int64_t cap) {
    if (n < 0 || (n > 0 && !samples) || cap < 0 || (cap > 0 && !splits_out)) return -1;
    const int64_t target = f32_to_count(segment_sec * 16000.0f);
    const float half_seg = segment_sec / 2.0f;
    // f32::min: a NaN operand yields the other one
    const float search = std::isnan(half_seg) ? search_sec : (search_sec < half_seg ? search_sec : half_seg);
    const int64_t margin = f32_to_count(search * 16000.0f);
    int64_t k = 0;
    auto put = [&](int64_t v) {
        if (k < cap) splits_out[k] = v;
        k++;
    };
    put(0);
    if (segment_sec <= 0.0f || n <= target + margin) return k;
    for (int64_t pos = 0; pos + target + margin < n;) {
        pos = find_split_point(samples, n, pos + target, search);
        put(pos);
        if (k >= 127) break;
    }
    return k;
}

// qwen_asr_transcribe_pcm (c_api.rs:75-95) -> transcribe_audio
// (transcribe.rs:297-403): the audio in one segment, or cut at
// qasr_hip_segment_splits when segment_sec > 0; each segment (a cut one
// zero-padded to 0.5 s at least) runs transcribe_segment's greedy decode to a stop token or
// 2048 tokens with the engine's prompt and language ids, and its text ids
// (after <asr_text>, or all of them with a forced language) follow the
// previous segments' in tokens_out (capacity cap); *n_out = their count (may
// exceed cap: then only cap were written).  Past-text conditioning (off by
// default, with no C-API setter) re-encodes the joined text with the
// tokenizer and is not offered at token level.
extern "C" int qasr_hip_engine_transcribe_pcm(qasr_engine *g, const float *samples, int64_t n_samples,
                                          int32_t *tokens_out, int64_t cap, int64_t *n_out) {
    if (!g || !samples || n_samples <= 0 || !n_out || cap < 0 || (cap > 0 && !tokens_out))
        return qasr_fail(QASR_ERR_INVALID, "engine_transcribe_pcm: bad arguments");
    *n_out = 0;
    g->raw.clear();
    g->segments.clear();
    std::vector<int64_t> splits(128);
    const int64_t n_seg = qasr_hip_segment_splits(samples, n_samples, g->segment_sec, g->search_sec, splits.data(),
                                                  (int64_t)splits.size());
    if (n_seg < 1) return qasr_fail(QASR_ERR_INVALID, "engine_transcribe_pcm: segmentation failed");
    const qasr_prompt ids{g->prompt.data(), (int64_t)g->prompt.size(), g->force.data(), (int64_t)g->force.size()};
    constexpr int64_t MIN_SAMPLES = 16000 / 2;
    std::vector<int32_t> seg_raw((size_t)g->max_tokens), text;
    std::vector<float> padded;
    g->kv_owner = g;
    for (int64_t k = 0; k < n_seg; k++) {
        const int64_t a = splits[(size_t)k], b = k + 1 < n_seg ? splits[(size_t)k + 1] : n_samples;
        const float *x = samples + a;
        int64_t len = b - a;
        if (n_seg > 1 && len < MIN_SAMPLES) {   // only cut segments are padded (transcribe.rs:355-366)
            padded.assign((size_t)MIN_SAMPLES, 0.0f);
            if (len > 0) std::memcpy(padded.data(), x, sizeof(float) * (size_t)len);
            x = padded.data();
            len = MIN_SAMPLES;
        }
        int64_t n_raw = 0;
        const int rc = qasr_hip_transcribe_prompt(g->d, g->e, x, len, &ids, nullptr, 0, g->max_tokens,
                                                  seg_raw.data(), &n_raw, nullptr);
        if (rc != QASR_OK) {
            g->raw.clear();
            g->segments.clear();
            return rc;
        }
        g->raw.insert(g->raw.end(), seg_raw.begin(), seg_raw.begin() + n_raw);
        const size_t t0 = text.size();
        text.resize(t0 + (size_t)n_raw);
        const int64_t m = qasr_hip_text_tokens_from(seg_raw.data(), n_raw, g->force.empty() ? 0 : 1, text.data() + t0);
        text.resize(t0 + (size_t)m);
        g->segments.insert(g->segments.end(), {a, b, (int64_t)t0, m});
    }
    const int64_t k = (int64_t)text.size();
    if (k > 0 && cap > 0) std::memcpy(tokens_out, text.data(), sizeof(int32_t) * (size_t)std::min(k, cap));
    *n_out = k;
    return QASR_OK;
}

extern "C" int qasr_hip_engine_last_segments(const qasr_engine *g, int64_t *bounds, int64_t cap, int64_t *n) {
    if (!g || !n || cap < 0 || (cap > 0 && !bounds)) return qasr_fail(QASR_ERR_INVALID, "engine: bad arguments");
    *n = (int64_t)g->segments.size() / 4;
    if (*n > 0 && cap > 0)
        std::memcpy(bounds, g->segments.data(), sizeof(int64_t) * 4 * (size_t)std::min<int64_t>(*n, cap));
    return QASR_OK;
}

// qwen_asr_set_segment_sec (c_api.rs:123-129); QwenCtx::search_sec
extern "C" void qasr_hip_engine_set_segment_sec(qasr_engine *g, float sec) {
    if (g) g->segment_sec = sec;
}
extern "C" void qasr_hip_engine_set_search_sec(qasr_engine *g, float sec) {
    if (g) g->search_sec = sec;
}

// an id list for the engine's prompt: checked against the vocabulary, then copied
static int engine_ids(const qasr_engine *g, const int32_t *ids, int64_t n, std::vector<int32_t> &out) {
    if (!g || n < 0 || (n > 0 && !ids)) return qasr_fail(QASR_ERR_INVALID, "engine: bad id list");
    for (int64_t i = 0; i < n; i++)
        if (ids[i] < 0 || ids[i] >= g->dc.vocab) return qasr_fail(QASR_ERR_INVALID, "engine: id outside the vocabulary");
    out.assign(ids, ids + n);
    return QASR_OK;
}

// qwen_asr_set_language (c_api.rs:131-148) with the language already encoded;
// <asr_text> closes the forced ids as in prepare_prompt_tokens
// (context.rs:215-221); no ids: automatic language
extern "C" int qasr_hip_engine_set_language_tokens(qasr_engine *g, const int32_t *ids, int64_t n) {
    std::vector<int32_t> v;
    if (int rc = engine_ids(g, ids, n, v)) return rc;
    if (n > 0) {
        if (151704 >= g->dc.vocab) return qasr_fail(QASR_ERR_INVALID, "engine: vocab too small for <asr_text>");
        v.push_back(151704);
    }
    g->force.swap(v);
    return QASR_OK;
}

// QwenCtx::set_prompt (context.rs:165-175) with the prompt already encoded
extern "C" int qasr_hip_engine_set_prompt_tokens(qasr_engine *g, const int32_t *ids, int64_t n) {
    std::vector<int32_t> v;
    if (int rc = engine_ids(g, ids, n, v)) return rc;
    g->prompt.swap(v);
    return QASR_OK;
}

// the raw tokens of the last transcription (stop token included)
extern "C" int qasr_hip_engine_last_raw_tokens(const qasr_engine *g, int32_t *tokens_out, int64_t cap, int64_t *n) {
    if (!g || !n || cap < 0 || (cap > 0 && !tokens_out)) return qasr_fail(QASR_ERR_INVALID, "engine: bad arguments");
    *n = (int64_t)g->raw.size();
    if (*n > 0 && cap > 0) std::memcpy(tokens_out, g->raw.data(), sizeof(int32_t) * (size_t)std::min<int64_t>(*n, cap));
    return QASR_OK;
}

// ---- streaming (c_api.rs:166-299) ------------------------------------------

// qwen_asr_stream_new (c_api.rs:179-184); the state binds the engine's
// decoder and encoder (the reference passes the engine to every push instead)
extern "C" int qasr_hip_engine_stream_new(qasr_engine *g, qasr_engine_stream **out) {
    if (!g || !out) return qasr_fail(QASR_ERR_INVALID, "engine_stream_new: null argument");
    *out = nullptr;
    qasr_engine_stream *s = new qasr_engine_stream();
    s->eng = g;
    int rc = qasr_hip_stream_create(g->d, g->e, &g->scfg, &s->s);
    if (rc != QASR_OK) {
        delete s;
        return rc;
    }
    g->streams.push_back(s);
    *out = s;
    return QASR_OK;
}

extern "C" void qasr_hip_engine_stream_free(qasr_engine_stream *s) {
    if (!s) return;
    if (s->eng) {
        auto &v = s->eng->streams;
        v.erase(std::remove(v.begin(), v.end(), s), v.end());
        if (s->eng->kv_owner == s) s->eng->kv_owner = nullptr;
    }
    if (s->s) qasr_hip_stream_free(s->s);
    delete s;
}

namespace {
int stream_live(const qasr_engine_stream *s) {
    if (!s) return qasr_fail(QASR_ERR_INVALID, "engine stream is null");
    if (!s->s) return qasr_fail(QASR_ERR_INVALID, "engine stream: its engine was freed");
    return QASR_OK;
}
}  // namespace

// qwen_asr_stream_reset (c_api.rs:196-202)
extern "C" int qasr_hip_engine_stream_reset(qasr_engine_stream *s) {
    if (int rc = stream_live(s)) return rc;
    s->audio.clear();
    return qasr_hip_stream_reset(s->s);
}

// qwen_asr_stream_push (c_api.rs:212-248): appends the new samples to the
// stream's audio, runs stream_push_audio over all of it with the engine's
// current stream settings, and writes the newly
// committed text token ids (capacity cap; *n_out = their count)
extern "C" int qasr_hip_engine_stream_push(qasr_engine_stream *s, const float *samples, int64_t n_samples, int finalize,
                                       int32_t *tokens_out, int64_t cap, int64_t *n_out) {
    if (int rc = stream_live(s)) return rc;
    if (!n_out || n_samples < 0 || (n_samples > 0 && !samples))
        return qasr_fail(QASR_ERR_INVALID, "engine_stream_push: bad arguments");
    if (n_samples > 0) s->audio.insert(s->audio.end(), samples, samples + n_samples);
    *n_out = 0;
    if (s->audio.empty()) return QASR_OK;
    if (s->eng->kv_owner != s) stream_drop_prefix(s->s);
    s->eng->kv_owner = s;
    // the reference reads the stream settings and the prepared prompt ids
    // from its context on every push
    stream_set_config(s->s, s->eng->scfg);
    const qasr_engine *g = s->eng;
    const qasr_prompt ids{g->prompt.data(), (int64_t)g->prompt.size(), g->force.data(), (int64_t)g->force.size()};
    if (int rc = qasr_hip_stream_set_prompt(s->s, &ids)) return rc;
    return qasr_hip_stream_push(s->s, s->audio.data(), (int64_t)s->audio.size(), finalize, tokens_out, cap, n_out);
}

// qwen_asr_stream_get_result (c_api.rs:250-267): every committed text token
extern "C" int qasr_hip_engine_stream_get_result(const qasr_engine_stream *s, int32_t *tokens_out, int64_t cap,
                                             int64_t *n) {
    if (int rc = stream_live(s)) return rc;
    return qasr_hip_stream_tokens(s->s, tokens_out, cap, n);
}

// qwen_asr_stream_set_* (c_api.rs:269-299): the settings every stream of the
// engine uses from its next push on; out-of-range values are ignored as there
extern "C" void qasr_hip_engine_stream_set_chunk_sec(qasr_engine *g, float sec) {
    if (g && sec > 0.0f) g->scfg.chunk_sec = sec;
}
extern "C" void qasr_hip_engine_stream_set_rollback(qasr_engine *g, int32_t tokens) {
    if (g && tokens >= 0) g->scfg.rollback = tokens;
}
extern "C" void qasr_hip_engine_stream_set_unfixed_chunks(qasr_engine *g, int32_t chunks) {
    if (g && chunks >= 0) g->scfg.unfixed_chunks = chunks;
}
extern "C" void qasr_hip_engine_stream_set_max_new_tokens(qasr_engine *g, int32_t tokens) {
    if (g && tokens > 0) g->scfg.max_new_tokens = tokens;
}

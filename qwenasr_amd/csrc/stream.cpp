// Incremental streaming transcription on the device-resident encoder and
// decoder: stream_push_audio (transcribe.rs:902-1304) with the defaults of
// QwenCtx (context.rs:144-150).  Per 2 s chunk:
//   1. completed 8 s encoder windows are encoded once and kept in HBM
//      (transcribe.rs:959-965); the partial tail is re-encoded on the first
//      chunk, every second chunk and when finalizing (:971-1002);
//   2. the prompt rows (prefix tokens | encoder rows | suffix tokens | rolled-
//      back text tokens) are assembled in HBM (:1036-1089);
//   3. the rows equal to the previous chunk's prefill (bitwise, k_row_diff)
//      keep their KV entries: kv len = that common-prefix length, and only the
//      remaining rows are prefilled (:1095-1115);
//   4. up to max_new_tokens greedy steps stop at the first stop token
//      (:1138-1151) — the steps run as graph replays in bursts, the host reads
//      the token log between bursts;
//   5. host bookkeeping on token ids: speech-end commit, rollback, degeneracy
//      and periodic re-anchoring, emission of the newly stable text tokens
//      (:1153-1292).
// Text is returned as token ids; turning them into bytes is the tokenizer's
// job on the host (tokenizer.rs), outside this library.
#include "decoder.h"
#include "encoder.h"

#include <algorithm>
#include <cstring>
#include <vector>

using namespace qasr;

#define TRY(x)                  \
    do {                        \
        int rc_ = (x);          \
        if (rc_ != QASR_OK) {   \
            return rc_;         \
        }                       \
    } while (0)

namespace {
constexpr int32_t TOKEN_ASR_TEXT = 151704;
// the last id of SUFFIX_BASE (transcribe.rs:15), the input of idle batch slots
constexpr int32_t SUFFIX_LAST = 198;
constexpr int DEGEN_MAX_PERIOD = 6, DEGEN_MIN_REPEATS = 4, STALE_CHUNKS = 4;
constexpr int RESET_INTERVAL_CHUNKS = 45, RESET_CARRY_TOKENS = 24, MAX_ENC_WINDOWS = 4;
constexpr int64_t SAMPLE_RATE = 16000, HOP = 160, WINDOW_FRAMES = 800;
constexpr int DECODE_BURST = 4;

// stream_tail_repeat_blocks (transcribe.rs:38-56): how many times a block of
// some period <= max_period repeats at the tail; the best (reps, period)
std::pair<int64_t, int64_t> tail_repeat_blocks(const std::vector<int32_t> &t, int64_t max_period) {
    const int64_t n = (int64_t)t.size();
    if (n < 2) return {1, 0};
    const int64_t cap = std::min(n / 2, max_period > 0 ? max_period : n / 2);
    int64_t best_reps = 1, best_period = 0;
    for (int64_t p = 1; p <= cap; p++) {
        int64_t reps = 1;
        while ((reps + 1) * p <= n) {
            const int32_t *a = t.data() + n - (reps + 1) * p, *b = t.data() + n - reps * p;
            if (!std::equal(a, a + p, b)) break;
            reps++;
        }
        if (reps > best_reps) { best_reps = reps; best_period = p; }
    }
    return {best_reps, best_period};
}
}  // namespace

// Device scratch of encode_requests (the audio slices, their mels, the mel
// working area and, for several inputs, the joint output rows).
struct EncScratch {
    DevBuf audio, mel, melsc, out;
};

struct EncWindow {
    DevBuf out;
    int64_t seq = 0;
};

struct qasr_stream {
    qasr_decoder *d = nullptr;
    qasr_encoder *e = nullptr;
    qasr_stream_config cfg{};
    // encoder
    std::vector<EncWindow> win;
    int64_t enc_cached_total = 0, enc_base_windows = 0;
    DevBuf partial, partial_next;   // the partial tail's rows; the re-encode goes to partial_next, then they swap
    std::vector<DevBuf> win_pool;   // buffers of released windows, reused by later ones
    int64_t partial_seq = 0, last_partial_cursor = 0;
    // tokens
    std::vector<int32_t> raw, stable, prev_tail;
    std::vector<int32_t> prompt, force;   // QwenCtx::prompt_tokens / force_prompt_tokens
    // prefill reuse
    DevBuf embeds, prev_embeds;
    int64_t prev_prefill_len = 0;
    int stale = 0;
    int64_t cursor = 0;
    int32_t chunk_idx = 0;
    // scratch
    EncScratch enc;                 // the encoder inputs' audio, mels and joint output rows
    DevBuf enc_all, toks, flags;
    HostBuf hflags;                 // the prefix comparison's flags, read after the round's one wait
    std::vector<int32_t> host_tok;
    // statistics of the last chunk
    int64_t st_reused = 0, st_prefill_len = 0, st_delta = 0, st_steps_total = 0, st_forwards = 0;
    // the stream batch this state belongs to (its KV lives in a batch slot)
    qasr_stream_batch *group = nullptr;
};

extern "C" void qasr_hip_stream_default_config(qasr_stream_config *c) {
    if (!c) return;
    c->chunk_sec = 2.0f;
    c->rollback = 5;
    c->unfixed_chunks = 2;
    c->max_new_tokens = 32;
    c->past_text_conditioning = 0;
    c->stop_tokens[0] = 151643;   // TOKEN_ENDOFTEXT
    c->stop_tokens[1] = 151645;   // TOKEN_IM_END
}

extern "C" int qasr_hip_stream_create(qasr_decoder *d, qasr_encoder *e, const qasr_stream_config *cfg,
                                      qasr_stream **out) {
    if (!d || !e || !out) return qasr_fail(QASR_ERR_INVALID, "stream_create: null argument");
    *out = nullptr;
    if (encoder_output_dim(e) != d->c.hidden)
        return qasr_fail(QASR_ERR_INVALID, "stream_create: encoder output_dim != decoder hidden");
    // every prompt id is gathered from the embedding table on the device
    std::vector<int32_t> head, tail;
    if (prompt_id_rows(nullptr, nullptr, 0, d->c.vocab, head, tail) != QASR_OK ||
        (cfg && cfg->past_text_conditioning && TOKEN_ASR_TEXT >= d->c.vocab))
        return qasr_fail(QASR_ERR_INVALID, "stream_create: vocab too small for the prompt");
    qasr_stream *s = new qasr_stream();
    s->d = d;
    s->e = e;
    if (cfg) s->cfg = *cfg;
    else qasr_hip_stream_default_config(&s->cfg);
    if (s->cfg.chunk_sec <= 0.0f || s->cfg.rollback < 0 || s->cfg.unfixed_chunks < 0 || s->cfg.max_new_tokens <= 0) {
        delete s;
        return qasr_fail(QASR_ERR_INVALID, "stream_create: bad configuration");
    }
    *out = s;
    return QASR_OK;
}

// the windows' buffers go back to the pool (kept until the stream is freed)
static void release_windows(qasr_stream *s) {
    for (auto &w : s->win) s->win_pool.push_back(w.out);
    s->win.clear();
}

extern "C" void qasr_hip_stream_free(qasr_stream *s) {
    if (!s) return;
    (void)hipSetDevice(s->d->h->device);
    (void)hipStreamSynchronize(s->d->h->stream);
    release_windows(s);
    for (DevBuf &b : s->win_pool) dbuf_release(b);
    for (DevBuf *b : {&s->partial, &s->partial_next, &s->embeds, &s->prev_embeds, &s->enc.audio, &s->enc.mel,
                      &s->enc.melsc, &s->enc.out, &s->enc_all,
                      &s->toks, &s->flags})
        dbuf_release(*b);
    hbuf_release(s->hflags);
    delete s;
}

void stream_drop_prefix(qasr_stream *s) {
    if (s) s->prev_prefill_len = 0;
}

void stream_set_config(qasr_stream *s, const qasr_stream_config &c) {
    if (s) s->cfg = c;
}

// StreamState::reset (transcribe.rs:865-883)
extern "C" int qasr_hip_stream_reset(qasr_stream *s) {
    if (!s) return qasr_fail(QASR_ERR_INVALID, "stream is null");
    CHECK_H(s->d->h);
    HIPCHK(hipStreamSynchronize(s->d->h->stream));
    release_windows(s);
    s->enc_cached_total = s->enc_base_windows = 0;
    s->partial_seq = s->last_partial_cursor = 0;
    s->raw.clear();
    s->stable.clear();
    s->prev_tail.clear();
    s->prev_prefill_len = 0;
    s->stale = 0;
    s->cursor = 0;
    s->chunk_idx = 0;
    return QASR_OK;
}

// One encoder input of a chunk (transcribe.rs:959-1002): host samples[0, ns)
// of a newly completed window (win >= 0: the stream's window win) or of the
// partial tail (win < 0: into the stream's partial_next); seq = its rows
// (0 when the slice has no mel frame).
struct EncReq {
    qasr_stream *s = nullptr;
    const float *x = nullptr;
    int64_t ns = 0;
    int win = -1;
    int64_t seq = 0;
};

static DevBuf &req_dst(EncReq &r) { return r.win >= 0 ? r.s->win[(size_t)r.win].out : r.s->partial_next; }

// The mel and encoder of every request, up to 64 inputs per encoder pass
// (qasr_hip_encoder_forward_batch's arithmetic: each input's rows are those of
// an encoder call of its own).  The host slices are read before it returns.
static hipStream_t enc_stream(qasr_decoder *d, qasr_encoder *e) { return e ? encoder_handle(e)->stream : d->h->stream; }

static int encode_requests(qasr_decoder *d, qasr_encoder *e, std::vector<EncReq> &reqs, EncScratch &sc) {
    hipStream_t st = d->h->stream;
    const int64_t H = d->c.hidden;
    std::vector<size_t> live;
    int64_t tot_s = 0, tot_f = 0, max_f = 0;
    for (size_t k = 0; k < reqs.size(); k++) {
        reqs[k].seq = 0;
        const int64_t nf = mel_frames_for(reqs[k].ns);
        if (nf <= 0) continue;
        live.push_back(k);
        tot_s += reqs[k].ns;
        tot_f += nf;
        max_f = std::max(max_f, nf);
    }
    if (live.empty()) return QASR_OK;
    TRY(dbuf_ensure(sc.audio, sizeof(float) * tot_s, enc_stream(d, e), d->h->stream));
    TRY(dbuf_ensure(sc.mel, sizeof(float) * 128 * tot_f, enc_stream(d, e), d->h->stream));
    TRY(dbuf_ensure(sc.melsc, sizeof(float) * mel_multi_scratch_floats(tot_f, max_f), enc_stream(d, e), d->h->stream));
    std::vector<const float *> mels, xs;
    std::vector<float *> mels_w;
    std::vector<int64_t> frames, lens;
    int64_t so = 0, fo = 0, tot_t = 0;
    for (size_t k : live) {
        const EncReq &r = reqs[k];
        float *xa = sc.audio.as<float>() + so, *m = sc.mel.as<float>() + 128 * fo;
        HIPCHK(hipMemcpyAsync(xa, r.x, sizeof(float) * r.ns, hipMemcpyHostToDevice, st));
        const int64_t nf = mel_frames_for(r.ns);
        xs.push_back(xa);
        lens.push_back(r.ns);
        mels.push_back(m);
        mels_w.push_back(m);
        frames.push_back(nf);
        tot_t += encoder_tokens(e, nf);
        so += r.ns;
        fo += nf;
    }
    TRY(mel_dev_multi(e, (int)live.size(), xs.data(), lens.data(), mels_w.data(), sc.melsc.as<float>()));
    std::vector<int64_t> tok(live.size());
    if (live.size() == 1) {
        // one input: its rows straight into its destination
        DevBuf &dst = req_dst(reqs[live[0]]);
        TRY(dbuf_ensure(dst, sizeof(float) * tot_t * H, enc_stream(d, e), d->h->stream));
        TRY(encoder_forward_multi(e, 1, mels.data(), frames.data(), dst.as<float>(), tok.data()));
    } else {
        TRY(dbuf_ensure(sc.out, sizeof(float) * tot_t * H, enc_stream(d, e), d->h->stream));
        int64_t row = 0;
        for (size_t g0 = 0; g0 < live.size(); g0 += QASR_ATTN_MAX_SEG) {
            const int ng = (int)std::min<size_t>(QASR_ATTN_MAX_SEG, live.size() - g0);
            TRY(encoder_forward_multi(e, ng, mels.data() + g0, frames.data() + g0, sc.out.as<float>() + row * H,
                                      tok.data() + g0));
            for (int q = 0; q < ng; q++) row += tok[g0 + q];
        }
        row = 0;
        for (size_t q = 0; q < live.size(); q++) {
            DevBuf &dst = req_dst(reqs[live[q]]);
            TRY(dbuf_ensure(dst, sizeof(float) * tok[q] * H, enc_stream(d, e), d->h->stream));
            HIPCHK(hipMemcpyAsync(dst.p, sc.out.as<float>() + row * H, sizeof(float) * tok[q] * H,
                                  hipMemcpyDeviceToDevice, st));
            row += tok[q];
        }
    }
    for (size_t q = 0; q < live.size(); q++) reqs[live[q]].seq = tok[q];
    // the host slices must outlive their uploads
    HIPCHK(hipStreamSynchronize(st));
    return QASR_OK;
}

static bool is_stop(const qasr_stream *s, int32_t t) {
    return t == s->cfg.stop_tokens[0] || t == s->cfg.stop_tokens[1];
}

// the text region of raw (transcribe.rs:1166-1172, 1257-1263): just past the
// first TOKEN_ASR_TEXT (0 when absent), or all of raw when the language is
// forced (the forced ids end with <asr_text> themselves)
static size_t text_start(const qasr_stream *s, const std::vector<int32_t> &raw) {
    if (!s->force.empty()) return 0;
    const auto it = std::find(raw.begin(), raw.end(), TOKEN_ASR_TEXT);
    return it == raw.end() ? 0 : (size_t)(it - raw.begin()) + 1;
}

extern "C" int qasr_hip_stream_set_prompt(qasr_stream *s, const qasr_prompt *p) {
    if (!s) return qasr_fail(QASR_ERR_INVALID, "stream is null");
    std::vector<int32_t> head, tail;
    if (int rc = prompt_id_rows(p, nullptr, 0, s->d->c.vocab, head, tail)) return rc;
    s->prompt.assign(head.begin() + 3, head.end() - 6);
    s->force.assign(tail.begin() + 6, tail.end());
    return QASR_OK;
}

static void carry_reset(qasr_stream *s) {
    const size_t carry = std::min<size_t>(s->stable.size(), RESET_CARRY_TOKENS);
    const size_t carry_start = s->stable.size() - carry;
    s->raw.clear();
    if (carry > 0) {
        s->raw.push_back(TOKEN_ASR_TEXT);
        s->raw.insert(s->raw.end(), s->stable.begin() + carry_start, s->stable.end());
    }
    s->prev_prefill_len = 0;
    s->stale = 0;
    s->prev_tail.clear();
    if ((int)s->win.size() >= MAX_ENC_WINDOWS) {
        s->enc_base_windows += (int64_t)s->win.size();
        release_windows(s);
        s->enc_cached_total = 0;
    }
}

// Where a chunk's prefill goes: the decoder's own KV cache (b == nullptr), or
// stream slot `slot` of a multi-stream batch.
struct PrefillTarget {
    qasr_batch *b = nullptr;
    int32_t slot = 0;
    bool defer = false;   // leave the rows to the caller's multi-slot prefill (ChunkPlan rows / reused / delta)
};

// What a prepared chunk hands to the decode and the commit.
struct ChunkPlan {
    bool is_final = false;
    int64_t prefill_len = 0;       // rows prefilled; the last prompt row is decoded first
    int64_t n_prefix_tokens = 0;   // rolled-back text tokens at the prompt's end
    int32_t last_token = 0;        // the prompt's last row is this token's embedding
    const float *rows = nullptr;   // a deferred prefill: delta rows at position reused
    int64_t reused = 0, delta = 0;
    // the chunk's encoder inputs: reqs[req0, req0 + nreq) of the round
    size_t req0 = 0, nreq = 0;
    int64_t full_end = 0;          // samples covered by complete windows
    bool tail_req = false;         // the partial tail is re-encoded (the last request)
    int64_t cmp = 0;               // prompt rows compared with the previous prefill (flags in hflags)
};

// greedy decode of up to max_new tokens after the prefill of prefill_len rows
// into the decoder's own cache; returns the chunk's tokens (stop token excluded)
static int decode_chunk(qasr_stream *s, int64_t prefill_len, std::vector<int32_t> &chunk) {
    qasr_decoder *d = s->d;
    hipStream_t st = d->h->stream;
    const int64_t H = d->c.hidden;
    const int max_new = s->cfg.max_new_tokens;
    chunk.clear();
    // first forward on the last prompt row
    d->len = prefill_len;
    TRY(decoder_set_state(d, 0));
    HIPCHK(hipMemcpyAsync(d->x, s->embeds.as<float>() + prefill_len * H, sizeof(float) * H, hipMemcpyDeviceToDevice,
                          st));
    TRY(decoder_enqueue_step(d, false));
    d->step_pos += 1;
    int64_t done = 1, seen = 0;
    s->host_tok.resize(max_new + DECODE_BURST + 1);
    int32_t fault = 0;
    // tokens t_0 .. t_{max_new-1}; t_j comes from forward j + 1
    for (;;) {
        HIPCHK(hipMemcpyAsync(s->host_tok.data() + seen, d->token_log + seen, sizeof(int32_t) * (done - seen),
                              hipMemcpyDeviceToHost, st));
        HIPCHK(hipMemcpyAsync(&fault, d->state + 5, sizeof(fault), hipMemcpyDeviceToHost, st));
        HIPCHK(hipStreamSynchronize(st));
        if (fault) TRY(decoder_fault_check(d));      // a failed hand-off ends the call at once
        bool stop = false;
        for (; seen < done && (int64_t)chunk.size() < max_new; seen++) {
            const int32_t t = s->host_tok[seen];
            if (is_stop(s, t)) { stop = true; break; }
            chunk.push_back(t);
        }
        if (stop || (int64_t)chunk.size() >= max_new) break;
        const int64_t burst = std::min<int64_t>(DECODE_BURST, max_new - done);
        TRY(decoder_run_embed_steps(d, burst));
        done += burst;
    }
    TRY(decoder_fault_check(d));
    d->len = prefill_len + done;
    s->st_forwards = done;
    s->st_steps_total += done;
    return QASR_OK;
}

// Step 1 of a chunk of stream_push_audio, first half: advance the cursor and
// list the encoder inputs (transcribe.rs:959-1002): every newly completed 8 s
// window (its buffer appended to the stream's windows, filled by
// encode_requests) and the partial tail when it is re-encoded (the first
// chunk, every second chunk, and when finalizing).
static void chunk_advance(qasr_stream *s, int64_t n, bool finalize, const float *samples, ChunkPlan &pl,
                          std::vector<EncReq> &reqs) {
    const int64_t chunk_samples = (int64_t)(s->cfg.chunk_sec * (float)SAMPLE_RATE);
    const int64_t win_samples = WINDOW_FRAMES * HOP;
    s->cursor = std::min(s->cursor + chunk_samples, n);
    pl.is_final = finalize && s->cursor >= n;
    pl.req0 = reqs.size();
    pl.full_end = (s->cursor / win_samples) * win_samples;
    while ((s->enc_base_windows + (int64_t)s->win.size()) * win_samples < pl.full_end) {
        const int64_t ws = (s->enc_base_windows + (int64_t)s->win.size()) * win_samples;
        EncWindow w;
        if (!s->win_pool.empty()) {
            w.out = s->win_pool.back();
            s->win_pool.pop_back();
        }
        s->win.push_back(w);
        EncReq r;
        r.s = s;
        r.x = samples + ws;
        r.ns = win_samples;
        r.win = (int)s->win.size() - 1;
        reqs.push_back(r);
    }
    const int64_t partial_age = s->cursor - s->last_partial_cursor;
    const bool need_encode = s->last_partial_cursor == 0 || partial_age >= 2 * chunk_samples || pl.is_final;
    pl.tail_req = pl.full_end < s->cursor && need_encode;
    if (pl.tail_req) {
        EncReq r;
        r.s = s;
        r.x = samples + pl.full_end;
        r.ns = s->cursor - pl.full_end;
        reqs.push_back(r);
    }
    pl.nreq = reqs.size() - pl.req0;
}

// Steps 1 (second half) to 3 of a chunk: the encoded windows and partial tail
// taken over, the prompt rows and the prefill with common-prefix reuse into
// `tgt`.  *skip: the chunk has no encoder rows, the reference returns from the
// whole push with an empty delta (transcribe.rs:1005-1008).
static int chunk_build(qasr_stream *s, const std::vector<EncReq> &reqs, const PrefillTarget &tgt, ChunkPlan &pl,
                       bool *skip) {
    qasr_decoder *d = s->d;
    hipStream_t st = d->h->stream;
    const int64_t H = d->c.hidden;
    const int rollback = s->cfg.rollback;
    *skip = false;
    for (size_t k = pl.req0; k < pl.req0 + pl.nreq; k++) {
        const EncReq &r = reqs[k];
        if (r.win >= 0) {
            s->win[(size_t)r.win].seq = r.seq;
            s->enc_cached_total += r.seq;
        }
    }
    int64_t partial_seq = 0;
    if (pl.full_end < s->cursor) {
        partial_seq = s->partial_seq;                       // reuse unless re-encoded
        const int64_t seq = pl.tail_req ? reqs[pl.req0 + pl.nreq - 1].seq : 0;
        if (seq > 0) {
            std::swap(s->partial, s->partial_next);
            s->partial_seq = partial_seq = seq;
            s->last_partial_cursor = s->cursor;
        }
    }
    const int64_t enc_len = s->enc_cached_total + partial_seq;
    if (enc_len == 0) {
        s->chunk_idx += 1;
        *skip = true;
        return QASR_OK;
    }

    // ---- prompt rows ----
    pl.n_prefix_tokens =
        (s->cfg.past_text_conditioning && s->chunk_idx >= s->cfg.unfixed_chunks && !s->raw.empty())
            ? (int64_t)std::max<int64_t>((int64_t)s->raw.size() - rollback, 0)
            : 0;
    const int64_t n_head = 9 + (int64_t)s->prompt.size(), n_suffix = 6 + (int64_t)s->force.size();
    const int64_t total_seq = n_head + enc_len + n_suffix + pl.n_prefix_tokens;
    pl.prefill_len = total_seq - 1;
    // a lone stream's decoder cache grows on demand (decoder.rs:199-231); a
    // multi-stream slot has the batch's fixed capacity
    const int64_t need = pl.prefill_len + s->cfg.max_new_tokens + DECODE_BURST;
    if (!tgt.b) TRY(decoder_reserve(d, need));
    if (need > (tgt.b ? batch_max_seq(tgt.b) : d->max_seq))
        return qasr_fail(QASR_ERR_INVALID, "stream: the batch's max_seq is too small for this context");
    TRY(dbuf_ensure(s->enc_all, sizeof(float) * enc_len * H, d->h->stream, s->e ? encoder_handle(s->e)->stream : nullptr));
    int64_t off = 0;
    for (auto &w : s->win) {
        HIPCHK(hipMemcpyAsync(s->enc_all.as<float>() + off * H, w.out.p, sizeof(float) * w.seq * H,
                              hipMemcpyDeviceToDevice, st));
        off += w.seq;
    }
    if (partial_seq > 0)
        HIPCHK(hipMemcpyAsync(s->enc_all.as<float>() + off * H, s->partial.p, sizeof(float) * partial_seq * H,
                              hipMemcpyDeviceToDevice, st));
    // PREFIX_HEAD | prompt | PREFIX_TAIL, then SUFFIX_BASE | force | rolled-back text
    qasr_prompt ids{s->prompt.data(), (int64_t)s->prompt.size(), s->force.data(), (int64_t)s->force.size()};
    std::vector<int32_t> toks, tail;
    TRY(prompt_id_rows(&ids, nullptr, 0, d->c.vocab, toks, tail));
    toks.insert(toks.end(), tail.begin(), tail.end());
    toks.insert(toks.end(), s->raw.begin(), s->raw.begin() + pl.n_prefix_tokens);
    for (int32_t t : toks)
        if (t < 0 || t >= d->c.vocab) return qasr_fail(QASR_ERR_INVALID, "stream: token id out of range");
    pl.last_token = toks.back();
    TRY(dbuf_ensure(s->toks, sizeof(int32_t) * toks.size(), d->h->stream, s->e ? encoder_handle(s->e)->stream : nullptr));
    HIPCHK(hipMemcpyAsync(s->toks.p, toks.data(), sizeof(int32_t) * toks.size(), hipMemcpyHostToDevice, st));
    TRY(dbuf_ensure(s->embeds, sizeof(float) * total_seq * H, d->h->stream, s->e ? encoder_handle(s->e)->stream : nullptr));
    LAUNCHCHK(launch_build_prompt(s->embeds.as<float>(), d->embed, s->toks.as<int>(), (int)n_head,
                                  s->enc_all.as<float>(), (int)enc_len, (int)(n_suffix + pl.n_prefix_tokens), (int)H, st),
              "stream prompt");

    // ---- the rows equal to the previous prefill's (read back after the
    // caller's wait, chunk_reuse) ----
    pl.cmp = 0;
    if (s->prev_prefill_len > 0) {
        pl.cmp = std::min(pl.prefill_len, s->prev_prefill_len);
        TRY(dbuf_ensure(s->flags, sizeof(int) * pl.cmp, d->h->stream, s->e ? encoder_handle(s->e)->stream : nullptr));
        TRY(hbuf_ensure(s->hflags, sizeof(int) * pl.cmp, d->h->stream, s->e ? encoder_handle(s->e)->stream : nullptr));
        LAUNCHCHK(launch_row_diff(s->embeds.as<float>(), s->prev_embeds.as<float>(), pl.cmp, H, s->flags.as<int>(),
                                  st),
                  "stream row diff");
        HIPCHK(hipMemcpyAsync(s->hflags.p, s->flags.p, sizeof(int) * pl.cmp, hipMemcpyDeviceToHost, st));
    }
    return QASR_OK;
}

// Step 3 of a chunk, after the wait for chunk_build's work: the prefill with
// common-prefix reuse (transcribe.rs:1092-1115) into `tgt`: the leading rows
// equal to the previous prefill keep their KV entries.
static int chunk_reuse(qasr_stream *s, const PrefillTarget &tgt, ChunkPlan &pl) {
    qasr_decoder *d = s->d;
    const int64_t H = d->c.hidden;
    const int64_t prefill_len = pl.prefill_len;
    int64_t reused = 0;
    const int *fl = s->hflags.as<int>();
    while (reused < pl.cmp && !fl[reused]) reused++;
    const int64_t delta = prefill_len - reused;
    pl.rows = s->embeds.as<float>() + reused * H;
    pl.reused = reused;
    pl.delta = delta;
    if (tgt.b && tgt.defer) {
        // the stream batch prefills every stream of the round in one call
    } else if (tgt.b) {
        if (delta > 0) TRY(batch_prefill_dev(tgt.b, tgt.slot, pl.rows, reused, delta));
        else TRY(qasr_hip_batch_set_len(tgt.b, tgt.slot, reused));
    } else {
        d->len = reused;
        if (delta > 0) TRY(decoder_prefill_dev(d, s->embeds.as<float>() + reused * H, delta));
    }
    s->st_reused = reused;
    s->st_prefill_len = prefill_len;
    s->st_delta = delta;
    return QASR_OK;
}

// Step 5 of a chunk: host bookkeeping on the chunk's tokens (transcribe.rs:
// 1153-1292); the newly stable text tokens are appended to `emitted`.
static void chunk_commit(qasr_stream *s, const ChunkPlan &pl, const std::vector<int32_t> &chunk,
                         std::vector<int32_t> &emitted, bool *speech_ended_out) {
    const int rollback = s->cfg.rollback;
    // keep this chunk's prefill rows for the next comparison
    std::swap(s->embeds, s->prev_embeds);
    s->prev_prefill_len = pl.prefill_len;

    // ---- speech end: commit everything that was held back ----
    const bool speech_ended = chunk.empty() && !s->raw.empty() && s->chunk_idx >= s->cfg.unfixed_chunks;
    if (speech_ended) {
        const size_t ts = text_start(s, s->raw);
        for (size_t i = s->stable.size(); i + ts < s->raw.size(); i++) {
            s->stable.push_back(s->raw[ts + i]);
            emitted.push_back(s->raw[ts + i]);
        }
    }
    s->raw.resize((size_t)pl.n_prefix_tokens);
    s->raw.insert(s->raw.end(), chunk.begin(), chunk.end());

    if (!speech_ended) {
        // ---- degeneracy and periodic re-anchoring ----
        if (s->raw == s->prev_tail) {
            s->stale += 1;
        } else {
            s->stale = 0;
            s->prev_tail = s->raw;
        }
        const int64_t reps = tail_repeat_blocks(s->raw, DEGEN_MAX_PERIOD).first;
        if (s->stale >= STALE_CHUNKS || reps >= DEGEN_MIN_REPEATS) carry_reset(s);
        if (s->chunk_idx > 0 && s->chunk_idx % RESET_INTERVAL_CHUNKS == 0) carry_reset(s);
        // ---- emit the tokens that are now stable ----
        const size_t ts = text_start(s, s->raw);
        const int64_t n_text = (int64_t)s->raw.size() - (int64_t)std::min(ts, s->raw.size());
        int64_t cand = 0;
        if (pl.is_final) cand = n_text;
        else if (s->chunk_idx >= s->cfg.unfixed_chunks) cand = std::max<int64_t>(n_text - rollback, 0);
        const int64_t from = (int64_t)s->stable.size();
        const int64_t to = std::max(cand, from);
        for (int64_t i = from; i < to; i++) {
            if (i < n_text) {
                s->stable.push_back(s->raw[ts + i]);
                emitted.push_back(s->raw[ts + i]);
            }
        }
    }
    s->chunk_idx += 1;
    *speech_ended_out = speech_ended;
}

// whether the stream has a chunk to process in a push over n_samples samples
static bool chunk_pending(const qasr_stream *s, int64_t n_samples, bool finalize) {
    const int64_t chunk_samples = (int64_t)(s->cfg.chunk_sec * (float)SAMPLE_RATE);
    if (s->cursor >= n_samples) return false;
    return n_samples - s->cursor >= chunk_samples || finalize;
}

extern "C" int qasr_hip_stream_push(qasr_stream *s, const float *samples, int64_t n_samples, int finalize,
                                    int32_t *tokens_out, int64_t cap, int64_t *n_out) {
    if (!s) return qasr_fail(QASR_ERR_INVALID, "stream is null");
    CHECK_H(s->d->h);
    if (n_out) *n_out = 0;
    if (s->group) return qasr_fail(QASR_ERR_INVALID, "stream_push: the stream belongs to a stream batch");
    if (n_samples < 0 || (n_samples > 0 && !samples) || n_samples < s->cursor)
        return qasr_fail(QASR_ERR_INVALID, "stream_push: samples must hold the whole stream so far");
    std::vector<int32_t> emitted;
    while (chunk_pending(s, n_samples, finalize != 0)) {
        ChunkPlan pl;
        bool skip = false, ended = false;
        std::vector<EncReq> reqs;
        chunk_advance(s, n_samples, finalize != 0, samples, pl, reqs);
        TRY(encode_requests(s->d, s->e, reqs, s->enc));
        TRY(chunk_build(s, reqs, PrefillTarget{}, pl, &skip));
        if (!skip) {
            HIPCHK(hipStreamSynchronize(s->d->h->stream));
            TRY(chunk_reuse(s, PrefillTarget{}, pl));
        }
        if (skip) {
            emitted.clear();
            break;
        }
        std::vector<int32_t> chunk;
        TRY(decode_chunk(s, pl.prefill_len, chunk));
        chunk_commit(s, pl, chunk, emitted, &ended);
        if (ended) break;
    }
    if (n_out) *n_out = (int64_t)emitted.size();
    if ((int64_t)emitted.size() > cap && tokens_out)
        return qasr_fail(QASR_ERR_INVALID, "stream_push: tokens_out too small (n_out holds the count)");
    if (tokens_out) std::copy(emitted.begin(), emitted.end(), tokens_out);
    return QASR_OK;
}

// ---- many streams, one batched decode ---------------------------------------
// N streaming states over one decoder and encoder whose chunks decode together
// on a multi-stream batch (BASELINE config 4 fed by the real pipeline): per
// round, every stream with a pending chunk runs its encoder and builds its
// prompt (common-prefix reuse within its own KV slot), one prefill of all
// their changed rows fills the slots, then all of them take their greedy
// steps together in bursts of DECODE_BURST (M = streams per projection), each
// stopping at its own stop token or max_new_tokens, then each commits its
// tokens.  Per stream, the sequence of operations is that of
// qasr_hip_stream_push; the batch's decode is the lone decoder's arithmetic.
struct qasr_stream_batch {
    qasr_decoder *d = nullptr;
    qasr_batch *b = nullptr;
    std::vector<qasr_stream *> s;
    // phase boundaries of each round on the library stream (encoder; prompt
    // rows and prefix comparison; prefill; decode), summed over the rounds of
    // the last push
    hipEvent_t ev[5] = {};
    double phase_ms[4] = {};
    EncScratch enc;                 // one encoder pass over every stream's inputs of a round
};

extern "C" void qasr_hip_stream_batch_free(qasr_stream_batch *g) {
    if (!g) return;
    for (qasr_stream *s : g->s) {
        s->group = nullptr;
        qasr_hip_stream_free(s);
    }
    if (g->b) qasr_hip_batch_free(g->b);
    for (hipEvent_t &v : g->ev)
        if (v) (void)hipEventDestroy(v);
    for (DevBuf *b : {&g->enc.audio, &g->enc.mel, &g->enc.melsc, &g->enc.out}) dbuf_release(*b);
    delete g;
}

extern "C" int qasr_hip_stream_batch_create(qasr_decoder *d, qasr_encoder *e, const qasr_stream_config *cfg,
                                            int32_t n_streams, int64_t max_seq, qasr_stream_batch **out) {
    if (!d || !e || !out) return qasr_fail(QASR_ERR_INVALID, "stream_batch_create: null argument");
    *out = nullptr;
    qasr_stream_batch *g = new qasr_stream_batch();
    g->d = d;
    int rc = qasr_hip_batch_create(d, n_streams, max_seq, DECODE_BURST, &g->b);
    for (int32_t i = 0; i < n_streams && rc == QASR_OK; i++) {
        qasr_stream *s = nullptr;
        rc = qasr_hip_stream_create(d, e, cfg, &s);
        if (rc == QASR_OK) {
            s->group = g;
            g->s.push_back(s);
        }
    }
    if (rc != QASR_OK) {
        qasr_hip_stream_batch_free(g);
        return rc;
    }
    *out = g;
    return QASR_OK;
}

extern "C" qasr_stream *qasr_hip_stream_batch_stream(qasr_stream_batch *g, int32_t i) {
    return (g && i >= 0 && i < (int32_t)g->s.size()) ? g->s[i] : nullptr;
}

// the greedy steps of the prepared streams `act` (plans pl), all slots
// stepping together; chunks[i] gets stream i's tokens (stop excluded)
static int group_decode(qasr_stream_batch *g, const std::vector<int> &act, const std::vector<ChunkPlan> &pl,
                        std::vector<std::vector<int32_t>> &chunks) {
    const int B = (int)g->s.size();
    std::vector<int32_t> first(B, SUFFIX_LAST), out((size_t)B * DECODE_BURST);
    std::vector<char> busy(B, 0), done(B, 1);
    for (int i : act) {
        busy[i] = 1;
        done[i] = 0;
        first[i] = pl[i].last_token;
        chunks[i].clear();
    }
    // the other slots step along from the end of the rows their next chunk may
    // reuse (their last prefill), which the capacity check of that chunk covered
    for (int j = 0; j < B; j++)
        if (!busy[j]) TRY(qasr_hip_batch_set_len(g->b, j, g->s[j]->prev_prefill_len));
    int64_t forwards = 0;
    for (;;) {
        bool open = false;
        for (int i : act) open |= !done[i];
        if (!open) break;
        TRY(qasr_hip_batch_generate(g->b, first.data(), DECODE_BURST, out.data()));
        forwards += DECODE_BURST;
        for (int i : act) {
            qasr_stream *s = g->s[i];
            for (int k = 0; k < DECODE_BURST && !done[i]; k++) {
                const int32_t t = out[(size_t)i * DECODE_BURST + k];
                if (is_stop(s, t)) { done[i] = 1; break; }
                chunks[i].push_back(t);
                if ((int64_t)chunks[i].size() >= s->cfg.max_new_tokens) done[i] = 1;
            }
        }
        for (int j = 0; j < B; j++) first[j] = out[(size_t)j * DECODE_BURST + DECODE_BURST - 1];
    }
    for (int i : act) {
        g->s[i]->st_forwards = forwards;
        g->s[i]->st_steps_total += forwards;
    }
    return QASR_OK;
}

extern "C" int qasr_hip_stream_batch_push(qasr_stream_batch *g, const float *const *samples, const int64_t *n_samples,
                                          const int32_t *finalize, int32_t *tokens_out, int64_t cap, int64_t *n_out) {
    if (!g || !samples || !n_samples || !n_out) return qasr_fail(QASR_ERR_INVALID, "stream_batch_push: null argument");
    CHECK_H(g->d->h);
    const int B = (int)g->s.size();
    for (int i = 0; i < B; i++) {
        n_out[i] = 0;
        if (n_samples[i] < 0 || (n_samples[i] > 0 && !samples[i]) || n_samples[i] < g->s[i]->cursor)
            return qasr_fail(QASR_ERR_INVALID, "stream_batch_push: samples must hold each whole stream so far");
    }
    std::vector<std::vector<int32_t>> emitted(B), chunks(B);
    std::vector<ChunkPlan> pl(B);
    std::vector<char> open(B, 1);
    hipStream_t st = g->d->h->stream;
    for (hipEvent_t &v : g->ev)
        if (!v) HIPCHK(hipEventCreate(&v));
    for (double &v : g->phase_ms) v = 0.0;
    for (;;) {
        HIPCHK(hipEventRecord(g->ev[0], st));
        // every stream with a pending chunk: its encoder inputs, all encoded in
        // one pass, then its prompt rows and prefix comparison
        std::vector<int> cand, act;
        std::vector<EncReq> reqs;
        for (int i = 0; i < B; i++) {
            const bool fin = finalize && finalize[i];
            if (!open[i] || !chunk_pending(g->s[i], n_samples[i], fin)) {
                open[i] = 0;
                continue;
            }
            chunk_advance(g->s[i], n_samples[i], fin, samples[i], pl[i], reqs);
            cand.push_back(i);
        }
        TRY(encode_requests(g->d, g->s.empty() ? nullptr : g->s[0]->e, reqs, g->enc));
        HIPCHK(hipEventRecord(g->ev[1], st));
        for (int i : cand) {
            bool skip = false;
            TRY(chunk_build(g->s[i], reqs, PrefillTarget{g->b, i, true}, pl[i], &skip));
            if (skip) {
                emitted[i].clear();
                open[i] = 0;
                continue;
            }
            act.push_back(i);
        }
        if (act.empty()) break;
        HIPCHK(hipStreamSynchronize(st));      // every stream's prefix comparison
        for (int i : act) TRY(chunk_reuse(g->s[i], PrefillTarget{g->b, i, true}, pl[i]));
        HIPCHK(hipEventRecord(g->ev[2], st));
        // one prefill of every stream's changed prompt rows (GEMMs over all of
        // them), each into its own slot
        {
            std::vector<int32_t> slots;
            std::vector<const float *> rows;
            std::vector<int64_t> starts, counts;
            for (int i : act) {
                slots.push_back(i);
                rows.push_back(pl[i].rows);
                starts.push_back(pl[i].reused);
                counts.push_back(pl[i].delta);
            }
            TRY(batch_prefill_segments(g->b, (int)act.size(), slots.data(), rows.data(), starts.data(),
                                       counts.data()));
        }
        HIPCHK(hipEventRecord(g->ev[3], st));
        TRY(group_decode(g, act, pl, chunks));
        HIPCHK(hipEventRecord(g->ev[4], st));
        HIPCHK(hipEventSynchronize(g->ev[4]));
        for (int k = 0; k < 4; k++) {
            float ms = 0.0f;
            HIPCHK(hipEventElapsedTime(&ms, g->ev[k], g->ev[k + 1]));
            g->phase_ms[k] += ms;
        }
        for (int i : act) {
            bool ended = false;
            chunk_commit(g->s[i], pl[i], chunks[i], emitted[i], &ended);
            if (ended) open[i] = 0;
        }
    }
    for (int i = 0; i < B; i++) {
        n_out[i] = (int64_t)emitted[i].size();
        if (tokens_out && (int64_t)emitted[i].size() > cap)
            return qasr_fail(QASR_ERR_INVALID, "stream_batch_push: tokens_out too small (n_out holds the counts)");
    }
    if (tokens_out)
        for (int i = 0; i < B; i++) std::copy(emitted[i].begin(), emitted[i].end(), tokens_out + (size_t)i * cap);
    return QASR_OK;
}

extern "C" int qasr_hip_stream_batch_times(const qasr_stream_batch *g, double *ms) {
    if (!g || !ms) return qasr_fail(QASR_ERR_INVALID, "stream_batch_times: null argument");
    std::copy(g->phase_ms, g->phase_ms + 4, ms);
    return QASR_OK;
}

extern "C" int qasr_hip_stream_tokens(const qasr_stream *s, int32_t *tokens_out, int64_t cap, int64_t *n) {
    if (!s || !n) return qasr_fail(QASR_ERR_INVALID, "stream_tokens: null argument");
    *n = (int64_t)s->stable.size();
    if (tokens_out) std::copy(s->stable.begin(), s->stable.begin() + std::min<int64_t>(cap, *n), tokens_out);
    return QASR_OK;
}

extern "C" int64_t qasr_hip_stream_audio_cursor(const qasr_stream *s) { return s ? s->cursor : -1; }

extern "C" int qasr_hip_stream_stats(const qasr_stream *s, int64_t *stats) {
    if (!s || !stats) return qasr_fail(QASR_ERR_INVALID, "stream_stats: null argument");
    const int64_t v[QASR_STREAM_STATS] = {s->chunk_idx,  s->st_reused,        s->st_prefill_len,
                                          s->st_delta,   s->st_forwards,      s->st_steps_total,
                                          (int64_t)s->win.size() + s->enc_base_windows, (int64_t)s->raw.size()};
    std::copy(v, v + QASR_STREAM_STATS, stats);
    return QASR_OK;
}

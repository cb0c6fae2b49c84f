/* CPU restatement of stream_push_audio (transcribe.rs:902-1304) over the oracle
 * decoder / encoder — test infrastructure only (the parity checker of the
 * GPU streaming driver).  Follows the reference step by step: window-cached
 * encoder (:959-1002), prompt rows (:1036-1089), prefix reuse by row equality
 * (:1092-1115), greedy decode to the first stop token (:1138-1151), speech-end
 * commit, rollback, degeneracy reset, re-anchoring and stable-token emission
 * (:1153-1292).  Text is kept as token ids (no tokenizer). */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "qasr_oracle.h"

#define TOKEN_ASR_TEXT 151704
#define DEGEN_MAX_PERIOD 6
#define DEGEN_MIN_REPEATS 4
#define STALE_CHUNKS 4
#define RESET_INTERVAL_CHUNKS 45
#define RESET_CARRY_TOKENS 24
#define MAX_ENC_WINDOWS 4
#define MAX_WINDOWS 4096

static const int32_t PREFIX_HEAD[] = {151644, 8948, 198};
static const int32_t PREFIX_TAIL[] = {151645, 198, 151644, 872, 198, 151669};
static const int32_t SUFFIX_BASE[] = {151670, 151645, 198, 151644, 77091, 198};

typedef struct {
    int32_t *v;
    int64_t n, cap;
} ivec;

static void iv_push(ivec *a, int32_t x) {
    if (a->n == a->cap) {
        a->cap = a->cap ? 2 * a->cap : 64;
        a->v = (int32_t *)realloc(a->v, sizeof(int32_t) * a->cap);
    }
    a->v[a->n++] = x;
}
static void iv_copy(ivec *dst, const ivec *src) {
    dst->n = 0;
    for (int64_t i = 0; i < src->n; i++) iv_push(dst, src->v[i]);
}
static int iv_equal(const ivec *a, const ivec *b) {
    return a->n == b->n && (a->n == 0 || memcmp(a->v, b->v, sizeof(int32_t) * a->n) == 0);
}

struct or_stream {
    or_decoder *d;
    or_encoder *e;
    or_stream_config cfg;
    int64_t H;
    float *win_out[MAX_WINDOWS];
    int64_t win_seq[MAX_WINDOWS];
    int64_t n_win, enc_cached_total, enc_base_windows;
    float *partial;
    int64_t partial_seq, last_partial_cursor;
    ivec raw, stable, prev_tail, out;
    ivec prompt, force;   /* QwenCtx::prompt_tokens / force_prompt_tokens */
    float *prev_embeds;
    int64_t prev_prefill_len;
    int stale;
    int64_t cursor;
    int32_t chunk_idx;
    int64_t st_reused, st_prefill_len, st_delta, st_forwards, st_forwards_total;
};

void or_stream_default_config(or_stream_config *c) {
    c->chunk_sec = 2.0f;
    c->rollback = 5;
    c->unfixed_chunks = 2;
    c->max_new_tokens = 32;
    c->past_text_conditioning = 0;
    c->stop_tokens[0] = 151643;
    c->stop_tokens[1] = 151645;
}

or_stream *or_stream_create(or_decoder *d, or_encoder *e, const or_stream_config *cfg, int64_t hidden) {
    or_stream *s = (or_stream *)calloc(1, sizeof(or_stream));
    s->d = d;
    s->e = e;
    if (cfg) s->cfg = *cfg;
    else or_stream_default_config(&s->cfg);
    s->H = hidden;
    return s;
}

static void release_windows(or_stream *s) {
    for (int64_t i = 0; i < s->n_win; i++) free(s->win_out[i]);
    s->n_win = 0;
}

void or_stream_destroy(or_stream *s) {
    if (!s) return;
    release_windows(s);
    free(s->partial);
    free(s->prev_embeds);
    free(s->raw.v);
    free(s->stable.v);
    free(s->prev_tail.v);
    free(s->out.v);
    free(s->prompt.v);
    free(s->force.v);
    free(s);
}

/* stream_tail_repeat_blocks (transcribe.rs:38-56) */
int64_t or_tail_repeat_blocks(const int32_t *t, int64_t n, int64_t max_period, int64_t *period) {
    int64_t best_reps = 1, best_period = 0;
    if (n >= 2) {
        int64_t cap = n / 2;
        if (max_period > 0 && max_period < cap) cap = max_period;
        for (int64_t p = 1; p <= cap; p++) {
            int64_t reps = 1;
            while ((reps + 1) * p <= n) {
                if (memcmp(t + n - (reps + 1) * p, t + n - reps * p, sizeof(int32_t) * p) != 0) break;
                reps++;
            }
            if (reps > best_reps) {
                best_reps = reps;
                best_period = p;
            }
        }
    }
    if (period) *period = best_period;
    return best_reps;
}

/* mel + encoder of samples[0, ns); NULL (seq 0) when mel_spectrogram has no frame */
static float *encode(or_stream *s, const float *samples, int64_t ns, int64_t *seq) {
    *seq = 0;
    const int64_t nf = or_mel_frames(ns);
    if (nf <= 0) return NULL;
    float *mel = (float *)malloc(sizeof(float) * 128 * nf);
    or_mel(samples, ns, mel);
    const int64_t T = or_encoder_tokens(s->e, nf);
    float *out = (float *)malloc(sizeof(float) * T * s->H);
    *seq = or_encoder_forward(s->e, mel, nf, out);
    free(mel);
    return out;
}

static int is_stop(const or_stream *s, int32_t t) { return t == s->cfg.stop_tokens[0] || t == s->cfg.stop_tokens[1]; }

void or_stream_set_prompt(or_stream *s, const int32_t *prompt, int64_t n_prompt, const int32_t *force,
                          int64_t n_force) {
    s->prompt.n = 0;
    for (int64_t i = 0; i < n_prompt; i++) iv_push(&s->prompt, prompt[i]);
    s->force.n = 0;
    for (int64_t i = 0; i < n_force; i++) iv_push(&s->force, force[i]);
}

/* the text region of raw (transcribe.rs:1166-1172, 1257-1263): after the
 * first <asr_text>, or all of it when the language is forced (the forced ids
 * end with <asr_text> themselves) */
static int64_t text_start(const or_stream *s, const ivec *raw) {
    if (s->force.n > 0) return 0;
    for (int64_t i = 0; i < raw->n; i++)
        if (raw->v[i] == TOKEN_ASR_TEXT) return i + 1;
    return 0;
}

static void carry_reset(or_stream *s) {
    const int64_t carry = s->stable.n < RESET_CARRY_TOKENS ? s->stable.n : RESET_CARRY_TOKENS;
    const int64_t carry_start = s->stable.n - carry;
    s->raw.n = 0;
    if (carry > 0) {
        iv_push(&s->raw, TOKEN_ASR_TEXT);
        for (int64_t i = carry_start; i < s->stable.n; i++) iv_push(&s->raw, s->stable.v[i]);
    }
    s->prev_prefill_len = 0;
    s->stale = 0;
    s->prev_tail.n = 0;
    if (s->n_win >= MAX_ENC_WINDOWS) {
        s->enc_base_windows += s->n_win;
        release_windows(s);
        s->enc_cached_total = 0;
    }
}

static void emit(or_stream *s, int32_t t) {
    iv_push(&s->stable, t);
    iv_push(&s->out, t);
}

/* one chunk; returns 1 when speech ended, 2 when the push returns empty */
static int process_chunk(or_stream *s, const float *samples, int64_t n, int finalize) {
    const int64_t H = s->H;
    const int64_t chunk_samples = (int64_t)(s->cfg.chunk_sec * 16000.0f);
    const int64_t win_samples = 800 * 160;
    const int rollback = s->cfg.rollback;
    s->cursor = s->cursor + chunk_samples < n ? s->cursor + chunk_samples : n;
    const int is_final = finalize && s->cursor >= n;

    const int64_t full_end = (s->cursor / win_samples) * win_samples;
    while ((s->enc_base_windows + s->n_win) * win_samples < full_end) {
        const int64_t ws = (s->enc_base_windows + s->n_win) * win_samples;
        int64_t seq = 0;
        float *o = encode(s, samples + ws, win_samples, &seq);
        s->win_out[s->n_win] = o;
        s->win_seq[s->n_win] = seq;
        s->n_win++;
        s->enc_cached_total += seq;
    }
    const int64_t partial_age = s->cursor - s->last_partial_cursor;
    const int need_encode = s->last_partial_cursor == 0 || partial_age >= 2 * chunk_samples || is_final;
    int64_t partial_seq = 0;
    if (full_end < s->cursor) {
        partial_seq = s->partial_seq;
        if (need_encode) {
            int64_t seq = 0;
            float *o = encode(s, samples + full_end, s->cursor - full_end, &seq);
            if (o && seq > 0) {
                free(s->partial);
                s->partial = o;
                s->partial_seq = partial_seq = seq;
                s->last_partial_cursor = s->cursor;
            } else {
                free(o);
            }
        }
    }
    const int64_t enc_len = s->enc_cached_total + partial_seq;
    if (enc_len == 0) {
        s->chunk_idx++;
        return 2;
    }

    const int64_t n_prefix_tokens =
        (s->cfg.past_text_conditioning && s->chunk_idx >= s->cfg.unfixed_chunks && s->raw.n > 0)
            ? (s->raw.n - rollback > 0 ? s->raw.n - rollback : 0)
            : 0;
    const int64_t prefix_len = 3 + s->prompt.n + 6, suffix_len = 6 + s->force.n;
    const int64_t total_seq = prefix_len + enc_len + suffix_len + n_prefix_tokens;
    float *emb = (float *)malloc(sizeof(float) * total_seq * H);
    int64_t off = 0;
    for (int i = 0; i < 3; i++) or_embed_token(s->d, PREFIX_HEAD[i], emb + (off++) * H);
    for (int64_t i = 0; i < s->prompt.n; i++) or_embed_token(s->d, s->prompt.v[i], emb + (off++) * H);
    for (int i = 0; i < 6; i++) or_embed_token(s->d, PREFIX_TAIL[i], emb + (off++) * H);
    for (int64_t w = 0; w < s->n_win; w++) {
        memcpy(emb + off * H, s->win_out[w], sizeof(float) * s->win_seq[w] * H);
        off += s->win_seq[w];
    }
    if (partial_seq > 0) {
        memcpy(emb + off * H, s->partial, sizeof(float) * partial_seq * H);
        off += partial_seq;
    }
    for (int i = 0; i < 6; i++) or_embed_token(s->d, SUFFIX_BASE[i], emb + (off++) * H);
    for (int64_t i = 0; i < s->force.n; i++) or_embed_token(s->d, s->force.v[i], emb + (off++) * H);
    for (int64_t i = 0; i < n_prefix_tokens; i++) or_embed_token(s->d, s->raw.v[i], emb + (off++) * H);

    /* prefill with reuse of the rows equal to the previous chunk's (float equality, :1095-1104) */
    const int64_t prefill_len = total_seq - 1;
    int64_t reused = 0;
    if (s->prev_embeds && s->prev_prefill_len > 0) {
        const int64_t cmp = prefill_len < s->prev_prefill_len ? prefill_len : s->prev_prefill_len;
        while (reused < cmp) {
            const float *a = s->prev_embeds + reused * H, *b = emb + reused * H;
            int same = 1;
            for (int64_t i = 0; i < H; i++)
                if (a[i] != b[i]) { same = 0; break; }
            if (!same) break;
            reused++;
        }
    }
    or_decoder_set_len(s->d, reused);
    const int64_t delta = prefill_len - reused;
    if (delta > 0) or_decoder_prefill(s->d, emb + reused * H, delta);
    s->st_reused = reused;
    s->st_prefill_len = prefill_len;
    s->st_delta = delta;

    /* greedy decode (:1138-1151) */
    float bv, sv;
    float *tmp = (float *)malloc(sizeof(float) * H);
    int32_t token = or_decoder_forward(s->d, emb + prefill_len * H, &bv, &sv, NULL);
    int64_t forwards = 1;
    ivec chunk = {0};
    int n_generated = 0;
    while (n_generated < s->cfg.max_new_tokens) {
        n_generated++;
        if (is_stop(s, token)) break;
        iv_push(&chunk, token);
        if (n_generated == s->cfg.max_new_tokens) break;   /* the reference's last forward is never read */
        or_embed_token(s->d, token, tmp);
        token = or_decoder_forward(s->d, tmp, &bv, &sv, NULL);
        forwards++;
    }
    free(tmp);
    s->st_forwards = forwards;
    s->st_forwards_total += forwards;
    free(s->prev_embeds);
    s->prev_embeds = emb;
    s->prev_prefill_len = prefill_len;

    const int speech_ended = chunk.n == 0 && s->raw.n > 0 && s->chunk_idx >= s->cfg.unfixed_chunks;
    if (speech_ended) {
        const int64_t ts = text_start(s, &s->raw);
        const int64_t n_text = s->raw.n - ts;
        for (int64_t i = s->stable.n; i < n_text; i++) emit(s, s->raw.v[ts + i]);
    }
    if (s->raw.n > n_prefix_tokens) s->raw.n = n_prefix_tokens;
    for (int64_t i = 0; i < chunk.n; i++) iv_push(&s->raw, chunk.v[i]);
    free(chunk.v);

    if (!speech_ended) {
        if (iv_equal(&s->raw, &s->prev_tail)) {
            s->stale++;
        } else {
            s->stale = 0;
            iv_copy(&s->prev_tail, &s->raw);
        }
        const int64_t reps = or_tail_repeat_blocks(s->raw.v, s->raw.n, DEGEN_MAX_PERIOD, NULL);
        if (s->stale >= STALE_CHUNKS || reps >= DEGEN_MIN_REPEATS) carry_reset(s);
        if (s->chunk_idx > 0 && s->chunk_idx % RESET_INTERVAL_CHUNKS == 0) carry_reset(s);
        const int64_t ts = text_start(s, &s->raw);
        const int64_t n_text = s->raw.n - ts;
        int64_t cand = 0;
        if (is_final) cand = n_text;
        else if (s->chunk_idx >= s->cfg.unfixed_chunks) cand = n_text - rollback > 0 ? n_text - rollback : 0;
        const int64_t from = s->stable.n, to = cand > from ? cand : from;
        for (int64_t i = from; i < to; i++)
            if (i < n_text) emit(s, s->raw.v[ts + i]);
    }
    s->chunk_idx++;
    return speech_ended ? 1 : 0;
}

int64_t or_stream_push(or_stream *s, const float *samples, int64_t n, int finalize, int32_t *out, int64_t cap) {
    const int64_t chunk_samples = (int64_t)(s->cfg.chunk_sec * 16000.0f);
    s->out.n = 0;
    const int64_t available = n > s->cursor ? n - s->cursor : 0;
    if ((available < chunk_samples && !finalize) || available == 0) return 0;
    while (s->cursor < n) {
        if (n - s->cursor < chunk_samples && !finalize) break;
        const int r = process_chunk(s, samples, n, finalize);
        if (r == 2) {
            s->out.n = 0;
            break;
        }
        if (r == 1) break;
    }
    const int64_t m = s->out.n < cap ? s->out.n : cap;
    if (out && m > 0) memcpy(out, s->out.v, sizeof(int32_t) * m);
    return s->out.n;
}

int64_t or_stream_tokens(const or_stream *s, int32_t *out, int64_t cap) {
    const int64_t m = s->stable.n < cap ? s->stable.n : cap;
    if (out && m > 0) memcpy(out, s->stable.v, sizeof(int32_t) * m);
    return s->stable.n;
}

void or_stream_stats(const or_stream *s, int64_t *stats) {
    stats[0] = s->chunk_idx;
    stats[1] = s->st_reused;
    stats[2] = s->st_prefill_len;
    stats[3] = s->st_delta;
    stats[4] = s->st_forwards;
    stats[5] = s->st_forwards_total;
    stats[6] = s->n_win + s->enc_base_windows;
    stats[7] = s->raw.n;
}

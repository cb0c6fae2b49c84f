// Multi-stream decode: B <= 32 independent streams share
// the decoder's int8 weights and step together.  Each stream owns a KV region
// (layout [layer][stream][kv_head][max_seq][hd], f32) with its own length and
// device step state {token, pos, step, flag}.  One step per layer: per-row
// RMSNorm + int8 quantization, an M = B W8A8 projection on int8 MFMA, the
// decode attention over every stream's ragged cache (grid y = stream), the
// split merge, and the o_proj / gate_up / down projections; then the LM-head
// argmax per stream.  Integer dots are exact and every per-row operation is
// the single-stream one, so each stream's tokens are those it would produce
// alone.  That includes the attention's split partition: each stream gets
// the single-stream decoder's partition for its own context bucket (groups per
// block from a per-position table, kept per stream on the device and advanced
// by the argmax finisher), inside a launch with the largest stream's split
// count; the extra splits of a shorter stream are empty and merge as exact
// zeros.  Steps replay one captured HIP graph per split count.
#include "decoder.h"

#include <algorithm>
#include <cstdlib>
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
constexpr int MAX_STREAMS = 32;
constexpr int ATT_MAX_SPLITS = 64;
constexpr int ARGMAX_BLOCKS = 608;      // 16 waves each: one 16-row tile per wave and pass (9496 tiles at 0.6B)
}

struct qasr_batch {
    qasr_decoder *d = nullptr;
    int B = 0;
    int64_t max_seq = 0, max_steps = 0;
    void *kc = nullptr, *vc = nullptr;
    float *x = nullptr, *qkv = nullptr, *att = nullptr, *ffn = nullptr, *xs = nullptr, *part = nullptr;
    float *rope_cur = nullptr, *am_val = nullptr;
    int8_t *xq = nullptr;
    int32_t *state = nullptr, *token_log = nullptr, *am_idx = nullptr;
    int32_t *gpb_dev = nullptr, *gpb_table = nullptr;   // per-stream / per-position attention partition
    int32_t *order_dev = nullptr;                        // attention grid rows -> streams, largest units first
    std::vector<int32_t> gpb_host;
    int64_t part_stride = 0;
    std::vector<int64_t> len;          // host copy of each stream's KV length
    int64_t steps_done = 0;            // steps since the last set of first tokens
    int n_split = 0, use_graph = 1;
    // groups in flight per k_attn_decode wave: one keeps the kernel at 4 waves
    // per SIMD, which measured faster at 32 streams than two
    int attn_depth = 1;
    int32_t *fault = nullptr;                            // set by an attention launch that cannot serve a stream
    // by (split count x 8 + groups per wave) x 4 + the attention forms present
    std::map<int, hipGraphExec_t> graphs;
    DevBuf prefill_rows;                                 // batch_prefill's staged rows, kept between calls
    std::vector<void *> allocs;
};

template <typename T>
static int balloc(qasr_batch *b, T **p, size_t count, bool zero = false) {
    void *v = nullptr;
    if (hipMalloc(&v, count * sizeof(T) + 256) != hipSuccess)
        return qasr_fail(QASR_ERR_NOMEM, "batch: device allocation failed");
    b->allocs.push_back(v);
    if (zero && hipMemset(v, 0, count * sizeof(T) + 256) != hipSuccess)
        return qasr_fail(QASR_ERR_HIP, "batch: memset failed");
    *p = reinterpret_cast<T *>(v);
    return QASR_OK;
}

extern "C" void qasr_hip_batch_free(qasr_batch *b) {
    if (!b) return;
    (void)hipSetDevice(b->d->h->device);
    (void)hipStreamSynchronize(b->d->h->stream);
    for (auto &g : b->graphs) (void)hipGraphExecDestroy(g.second);
    dbuf_release(b->prefill_rows);
    for (void *p : b->allocs) (void)hipFree(p);
    delete b;
}

// context bucket of a step whose new position is pos (the single-stream
// decoder's rule, decoder_ctx_cap at L = pos + 1, with this batch's capacity)
static int64_t batch_cap(const qasr_batch *b, int64_t pos) {
    const int64_t c = ((pos + 1 + 255) / 256) * 256;
    return std::min<int64_t>(std::max<int64_t>(c, 256), b->max_seq);
}

// split count of a bucket: the forced count, else the single-stream automatic choice
static int batch_splits(const qasr_batch *b, int64_t cap) {
    if (b->n_split > 0) return b->n_split;
    return attn_splits_auto(b->d->c, cap);
}

// groups of 8 positions per attention block for every position (the
// single-stream decoder's static partition: ceil(ceil(cap / 8) / splits))
static int batch_partition(qasr_batch *b) {
    b->gpb_host.resize(b->max_seq);
    for (int64_t p = 0; p < b->max_seq; p++) {
        const int64_t cap = batch_cap(b, p);
        const int S = batch_splits(b, cap);
        b->gpb_host[p] = (int32_t)((((cap + 7) / 8) + S - 1) / S);
    }
    HIPCHK(hipMemcpy(b->gpb_table, b->gpb_host.data(), sizeof(int32_t) * b->max_seq, hipMemcpyHostToDevice));
    return QASR_OK;
}

// Every stream decodes bit-identically to its solo run on the same decoder
// so each stream's attention takes the form the
// single-stream decoder takes at that stream's context bucket: k_attn_step's
// (here k_attn_step_batch) when the bucket's partition fits it, else
// k_attn_decode's.  A step whose streams sit in buckets of both kinds runs
// both kernels, each serving its own streams; the decoder itself is never
// changed by a batch.
static bool step_form(const qasr_batch *b, int64_t pos) {
    return b->d->attn_step && attn_step_gpw(b->gpb_host[(size_t)pos]) > 0;
}

// the attention forms of step s of the current run: bit 0 some stream takes
// the step form, bit 1 some stream takes k_attn_decode's
static int batch_forms(const qasr_batch *b, int64_t s) {
    int m = 0;
    for (int64_t l : b->len) m |= step_form(b, std::min<int64_t>(l + s, b->max_seq - 1)) ? 1 : 2;
    return m;
}

// groups per attention wave of a multi-stream step at step s of the current
// run (k_attn_step_batch): the most any step-form stream's partition needs
static int batch_step_gpw(const qasr_batch *b, int64_t s) {
    int g = 1;
    for (int64_t l : b->len) {
        const int64_t p = std::min<int64_t>(l + s, b->max_seq - 1);
        if (step_form(b, p)) g = std::max(g, attn_step_gpw(b->gpb_host[(size_t)p]));
    }
    return g;
}

extern "C" int qasr_hip_batch_create(qasr_decoder *d, int32_t n_streams, int64_t max_seq, int64_t max_steps,
                                     qasr_batch **out) {
    if (!d || !out) return qasr_fail(QASR_ERR_INVALID, "batch_create: null argument");
    CHECK_H(d->h);
    *out = nullptr;
    const qasr_dec_config &c = d->c;
    if (n_streams <= 0 || n_streams > MAX_STREAMS)
        return qasr_fail(QASR_ERR_INVALID, "batch_create: 1..32 streams");
    if (max_seq <= 0 || max_seq > d->max_seq || max_steps <= 0)
        return qasr_fail(QASR_ERR_INVALID, "batch_create: max_seq must be in 1..decoder max_seq, max_steps > 0");
    if (c.n_heads != 16 || c.n_kv_heads != 8 || c.head_dim != 128 || d->kv_bf16)
        return qasr_fail(QASR_ERR_INVALID, "batch_create: needs the 16/8-head, head_dim 128 decoder with an f32 KV cache");
    auto steps_ok = [](int64_t k) { return k % 1024 == 0 && (k == 1024 || k == 2048 || k == 3072 || k == 4096 || k == 6144); };
    if (!steps_ok(c.hidden) || !steps_ok(c.intermediate) || c.hidden > 4096 || d->lm_i8_rows % 16)
        return qasr_fail(QASR_ERR_INVALID, "batch_create: hidden and intermediate must be 1024, 2048, 3072, 4096 or 6144");
    qasr_batch *b = new qasr_batch();
    b->d = d;
    b->B = n_streams;
    b->max_seq = max_seq;
    b->max_steps = max_steps;
    b->len.assign(n_streams, 0);
    b->use_graph = d->use_graph;         // the decoder's setting (QASR_DISABLE_GRAPH=1 turns both off)
    const int64_t H = c.hidden, hd = c.head_dim, qd = (int64_t)c.n_heads * hd, kvd = (int64_t)c.n_kv_heads * hd;
    const int64_t I = c.intermediate, nqkv = qd + 2 * kvd;
    const int64_t kmax = std::max({H, qd, I});
    const size_t kv = (size_t)c.n_layers * n_streams * c.n_kv_heads * max_seq * hd;
    b->part_stride = (2 * c.n_heads + c.n_heads * hd) * ATT_MAX_SPLITS;
    int rc = QASR_OK;
    float *kcf = nullptr, *vcf = nullptr;
    if (rc == QASR_OK) rc = balloc(b, &kcf, kv, true);
    if (rc == QASR_OK) rc = balloc(b, &vcf, kv, true);
    b->kc = kcf;
    b->vc = vcf;
    if (rc == QASR_OK) rc = balloc(b, &b->x, (size_t)n_streams * H);
    if (rc == QASR_OK) rc = balloc(b, &b->qkv, (size_t)n_streams * nqkv);
    if (rc == QASR_OK) rc = balloc(b, &b->att, (size_t)n_streams * qd);
    if (rc == QASR_OK) rc = balloc(b, &b->ffn, (size_t)n_streams * I);
    if (rc == QASR_OK) rc = balloc(b, &b->xq, (size_t)MAX_STREAMS * kmax, true);   // rows >= B stay zero
    if (rc == QASR_OK) rc = balloc(b, &b->xs, MAX_STREAMS, true);
    if (rc == QASR_OK) rc = balloc(b, &b->part, (size_t)n_streams * b->part_stride);
    if (rc == QASR_OK) rc = balloc(b, &b->rope_cur, (size_t)n_streams * 256);
    if (rc == QASR_OK) rc = balloc(b, &b->state, (size_t)n_streams * 4, true);
    if (rc == QASR_OK) rc = balloc(b, &b->token_log, (size_t)n_streams * max_steps, true);
    if (rc == QASR_OK) rc = balloc(b, &b->am_val, (size_t)ARGMAX_BLOCKS * 32);
    if (rc == QASR_OK) rc = balloc(b, &b->am_idx, (size_t)ARGMAX_BLOCKS * 32);
    if (rc == QASR_OK) rc = balloc(b, &b->gpb_dev, (size_t)n_streams, true);
    if (rc == QASR_OK) rc = balloc(b, &b->order_dev, (size_t)n_streams, true);
    if (rc == QASR_OK) rc = balloc(b, &b->gpb_table, (size_t)max_seq);
    if (rc == QASR_OK) rc = balloc(b, &b->fault, 1, true);
    if (rc == QASR_OK) {
        std::vector<int32_t> ident(n_streams);
        for (int i = 0; i < n_streams; i++) ident[i] = i;
        if (hipMemcpy(b->order_dev, ident.data(), sizeof(int32_t) * n_streams, hipMemcpyHostToDevice) != hipSuccess)
            rc = qasr_fail(QASR_ERR_HIP, "batch: order upload failed");
    }
    if (rc == QASR_OK) rc = batch_partition(b);
    if (rc != QASR_OK) {
        qasr_hip_batch_free(b);
        return rc;
    }
    *out = b;
    return QASR_OK;
}

static int64_t stream_layer_elems(const qasr_batch *b) {
    return (int64_t)b->d->c.n_kv_heads * b->max_seq * b->d->c.head_dim;
}

// decoder_prefill (decoder.rs:455) of one stream: the decoder's prefill run on
// the stream's view of the cache
extern "C" int qasr_hip_batch_prefill(qasr_batch *b, int32_t stream, const float *embeds, int64_t seq_len) {
    if (!b || !embeds || seq_len <= 0) return qasr_fail(QASR_ERR_INVALID, "batch_prefill: bad arguments");
    qasr_decoder *d = b->d;
    CHECK_H(d->h);
    if (stream < 0 || stream >= b->B) return qasr_fail(QASR_ERR_INVALID, "batch_prefill: stream out of range");
    if (b->len[stream] + seq_len > b->max_seq) return qasr_fail(QASR_ERR_INVALID, "batch_prefill: capacity exceeded");
    const int64_t H = d->c.hidden, le = stream_layer_elems(b);
    int rc0 = dbuf_ensure(b->prefill_rows, sizeof(float) * seq_len * H, d->h->stream);
    if (rc0 != QASR_OK) return rc0;
    float *emb = b->prefill_rows.as<float>();
    hipError_t e = hipMemcpyAsync(emb, embeds, sizeof(float) * seq_len * H, hipMemcpyHostToDevice, d->h->stream);
    // swap in the stream's view: base, layer stride, capacity, length
    void *kc0 = d->kc, *vc0 = d->vc;
    const int64_t ms0 = d->max_seq, len0 = d->len, ls0 = d->kv_layer_stride;
    d->kc = reinterpret_cast<float *>(b->kc) + stream * le;
    d->vc = reinterpret_cast<float *>(b->vc) + stream * le;
    d->kv_layer_stride = (int64_t)b->B * le;
    d->max_seq = b->max_seq;
    d->len = b->len[stream];
    int rc = e == hipSuccess ? decoder_prefill_dev(d, emb, seq_len) : qasr_fail(QASR_ERR_HIP, "batch_prefill: upload");
    d->kc = kc0;
    d->vc = vc0;
    d->kv_layer_stride = ls0;
    d->max_seq = ms0;
    d->len = len0;
    if (hipStreamSynchronize(d->h->stream) != hipSuccess && rc == QASR_OK)
        rc = qasr_fail(QASR_ERR_HIP, "batch_prefill: stream failed");
    if (rc == QASR_OK) b->len[stream] += seq_len;
    return rc;
}

// decoder_prefill of several stream slots at once (the multi-stream
// streaming driver's chunk prefills): slot slots[i] gets counts[i] device rows
// rows[i] at positions [starts[i], starts[i] + counts[i]) and that length;
// each slot's rows get the bits a prefill of that slot alone gives
int batch_prefill_segments(qasr_batch *b, int n, const int32_t *slots, const float *const *rows,
                           const int64_t *starts, const int64_t *counts) {
    if (!b || n < 0 || (n > 0 && (!slots || !rows || !starts || !counts)))
        return qasr_fail(QASR_ERR_INVALID, "batch prefill: bad arguments");
    qasr_decoder *d = b->d;
    CHECK_H(d->h);
    const int64_t le = stream_layer_elems(b);
    std::vector<PrefillSeg> segs((size_t)n);
    for (int i = 0; i < n; i++) {
        if (slots[i] < 0 || slots[i] >= b->B) return qasr_fail(QASR_ERR_INVALID, "batch prefill: stream out of range");
        if (starts[i] < 0 || counts[i] < 0 || starts[i] + counts[i] > b->max_seq)
            return qasr_fail(QASR_ERR_INVALID, "batch prefill: capacity exceeded");
        PrefillSeg &g = segs[(size_t)i];
        g.rows = rows[i];
        g.n = counts[i];
        g.start = starts[i];
        g.kc = reinterpret_cast<float *>(b->kc) + slots[i] * le;
        g.vc = reinterpret_cast<float *>(b->vc) + slots[i] * le;
        g.layer_elems = (int64_t)b->B * le;
        g.head_stride = b->max_seq * d->c.head_dim;
        g.cap = b->max_seq;
    }
    TRY(decoder_prefill_segments(d, segs.data(), n));
    for (int i = 0; i < n; i++) b->len[slots[i]] = starts[i] + counts[i];
    return QASR_OK;
}

int batch_prefill_dev(qasr_batch *b, int32_t stream, const float *rows, int64_t start, int64_t n) {
    return batch_prefill_segments(b, 1, &stream, &rows, &start, &n);
}

int64_t batch_max_seq(const qasr_batch *b) { return b ? b->max_seq : 0; }
int32_t batch_streams(const qasr_batch *b) { return b ? b->B : 0; }

extern "C" int qasr_hip_batch_set_len(qasr_batch *b, int32_t stream, int64_t len) {
    if (!b || stream < 0 || stream >= b->B || len < 0 || len > b->max_seq)
        return qasr_fail(QASR_ERR_INVALID, "batch_set_len: bad arguments");
    b->len[stream] = len;
    return QASR_OK;
}

extern "C" int64_t qasr_hip_batch_len(const qasr_batch *b, int32_t stream) {
    return (b && stream >= 0 && stream < b->B) ? b->len[stream] : -1;
}

extern "C" int qasr_hip_batch_set_options(qasr_batch *b, int attn_splits, int use_graph) {
    if (!b) return qasr_fail(QASR_ERR_INVALID, "batch is null");
    CHECK_H(b->d->h);
    if (attn_splits < 0) b->n_split = 0;
    if (attn_splits > 0) {
        if (attn_splits > ATT_MAX_SPLITS)
            return qasr_fail(QASR_ERR_INVALID, "batch_set_options: attn_splits must be 1..64 (or -1)");
        b->n_split = attn_splits;
    }
    b->use_graph = use_graph ? 1 : 0;
    HIPCHK(hipStreamSynchronize(b->d->h->stream));
    for (auto &g : b->graphs) HIPCHK(hipGraphExecDestroy(g.second));
    b->graphs.clear();
    return batch_partition(b);
}

// kernels of a step (profile kinds); per-layer kinds launch once per layer
enum {
    BK_EMBED, BK_IN_QUANT, BK_QKV, BK_PREP, BK_ATTN, BK_MERGE, BK_O, BK_POST_QUANT, BK_GU, BK_FFN_QUANT, BK_DOWN,
    BK_FINAL_QUANT, BK_LM, BK_LM_FINISH, BK_KINDS
};
static_assert(BK_KINDS == QASR_BATCH_PROFILE_KINDS, "profile kinds");
static bool per_layer_kind(int k) { return k >= BK_IN_QUANT && k <= BK_DOWN; }

// one batched step with n_split attention splits (only kernels of one kind
// when kind >= 0)
static int batch_enqueue_step(qasr_batch *b, int n_split, int gpw, int forms, int kind = -1) {
    qasr_decoder *d = b->d;
    const qasr_dec_config &c = d->c;
    hipStream_t st = d->h->stream;
    const int B = b->B, H = c.hidden, hd = c.head_dim, qd = c.n_heads * hd, kvd = c.n_kv_heads * hd;
    const int I = c.intermediate, nqkv = qd + 2 * kvd;
    const int64_t le = stream_layer_elems(b);
    auto on = [&](int k) { return kind < 0 || kind == k; };
    if (on(BK_EMBED)) LAUNCHCHK(launch_embed_rows(b->x, d->embed, b->state, B, H, st), "batch embed");
    auto mv = [&](const int8_t *w, const float *ws, float *y, int64_t ldy, int K, int N, int mode) -> int {
        BatchMvArgs a{};
        a.xq = b->xq; a.xs = b->xs; a.w = w; a.ws = ws; a.y = y; a.ldy = ldy; a.K = K; a.N = N; a.B = B;
        LAUNCHCHK(launch_w8a8_batch(a, mode, st), "batch projection");
        return QASR_OK;
    };
    for (int l = 0; l < c.n_layers; l++) {
        const DecLayerDev &L = d->L[l];
        if (on(BK_IN_QUANT)) LAUNCHCHK(launch_quant_rows(b->x, L.in_norm, c.eps, H, B, b->xq, b->xs, st), "batch norm+quant");
        if (on(BK_QKV)) TRY(mv(L.wqkv, L.sqkv, b->qkv, nqkv, H, nqkv, MV_PLAIN));
        AttnDecodeArgs t{};
        t.qkv = b->qkv; t.q_norm = L.q_norm; t.k_norm = L.k_norm;
        t.rope_cos = d->rc; t.rope_sin = d->rs; t.rope_cur = b->rope_cur; t.state = b->state;
        t.kcache = reinterpret_cast<float *>(b->kc) + (int64_t)l * B * le;
        t.vcache = reinterpret_cast<float *>(b->vc) + (int64_t)l * B * le;
        t.head_stride = b->max_seq * hd;
        t.part = b->part; t.counters = d->counters + QASR_CTR_ATTN; t.out = b->att;
        t.n_split = n_split; t.waves = d->attn_waves; t.eps = c.eps; t.scale = 1.0f / sqrtf((float)hd);
        t.gpb = 1;                           // the per-stream gpb_dev rows are used
        t.gpb_dev = b->gpb_dev;
        t.stream_order = b->order_dev;
        t.depth = b->attn_depth;
        t.fault = b->fault;
        t.batch = B; t.batch_kv_stride = le; t.batch_qkv_stride = nqkv; t.batch_part_stride = b->part_stride;
        // the step-form streams: k_attn_step_batch does their q/k norm + RoPE
        // and K/V row write itself; the others: k_qk_prep_rows, k_attn_decode
        const bool mixed = forms == 3;
        if ((forms & 1) && on(BK_ATTN)) {
            AttnDecodeArgs ts = t;
            ts.waves = 4;
            ts.gpw = gpw;
            ts.select = mixed ? 1 : 0;
            LAUNCHCHK(launch_attn_decode(ts, c.n_heads, c.n_kv_heads, hd, 0, st, false), "batch attention");
        }
        if (forms & 2) {
            t.select = mixed ? 2 : 0;
            if (on(BK_PREP)) LAUNCHCHK(launch_qk_prep_rows(t, c.n_heads, c.n_kv_heads, hd, 0, st), "batch q/k prep");
            if (on(BK_ATTN))
                LAUNCHCHK(launch_attn_decode(t, c.n_heads, c.n_kv_heads, hd, 0, st, false), "batch attention");
        }
        if (on(BK_MERGE))
            LAUNCHCHK(launch_attn_merge_rows(b->part, b->part_stride, n_split, nullptr, qd, b->xq, b->xs, B, st),
                      "batch merge+quant");
        if (on(BK_O)) TRY(mv(L.wo, L.so, b->x, H, qd, H, MV_ADDTO));
        if (on(BK_POST_QUANT))
            LAUNCHCHK(launch_quant_rows(b->x, L.post_norm, c.eps, H, B, b->xq, b->xs, st), "batch norm+quant");
        if (on(BK_GU)) TRY(mv(L.wgu, L.sgu, b->ffn, I, H, 2 * I, MV_SWIGLU));
        if (on(BK_FFN_QUANT)) LAUNCHCHK(launch_quant_rows(b->ffn, nullptr, 0.0f, I, B, b->xq, b->xs, st), "batch quant");
        if (on(BK_DOWN)) TRY(mv(L.wdown, L.sdown, b->x, H, I, H, MV_ADDTO));
    }
    if (on(BK_FINAL_QUANT))
        LAUNCHCHK(launch_quant_rows(b->x, d->norm, c.eps, H, B, b->xq, b->xs, st), "batch final norm");
    if (on(BK_LM) || on(BK_LM_FINISH)) {
        BatchMvArgs am{};
        am.xq = b->xq; am.xs = b->xs; am.w = d->lm; am.ws = d->lm_s; am.K = H; am.N = (int)d->lm_i8_rows; am.B = B;
        am.part_val = b->am_val; am.part_idx = b->am_idx;
        LAUNCHCHK(launch_argmax_batch(am, ARGMAX_BLOCKS, b->state, b->token_log, b->max_steps, d->rc, d->rs,
                                      b->rope_cur, (int)b->max_seq, b->gpb_table, b->gpb_dev, st, on(BK_LM),
                                      on(BK_LM_FINISH)),
                  "batch argmax");
    }
    return QASR_OK;
}

// set every stream's step state {first token, len, 0, 0} and RoPE rows
static int batch_set_state(qasr_batch *b, const int32_t *first_tokens) {
    qasr_decoder *d = b->d;
    hipStream_t st = d->h->stream;
    const int64_t hd = d->c.head_dim;
    std::vector<int32_t> hs((size_t)b->B * 4, 0);
    for (int i = 0; i < b->B; i++) {
        if (first_tokens[i] < 0 || first_tokens[i] >= d->c.vocab)
            return qasr_fail(QASR_ERR_INVALID, "batch: token id out of range");
        hs[4 * i] = first_tokens[i];
        hs[4 * i + 1] = (int32_t)b->len[i];
    }
    HIPCHK(hipMemcpyAsync(b->state, hs.data(), sizeof(int32_t) * hs.size(), hipMemcpyHostToDevice, st));
    std::vector<int32_t> gp(b->B);
    for (int i = 0; i < b->B; i++) gp[i] = b->gpb_host[b->len[i]];
    HIPCHK(hipMemcpyAsync(b->gpb_dev, gp.data(), sizeof(int32_t) * b->B, hipMemcpyHostToDevice, st));
    // attention blocks of the streams with the longest units (groups per
    // block, then context) are dispatched first, so that the short ones fill
    // the tail; every stream grows by one position per step, so the order
    // holds for the whole call
    std::vector<int32_t> order(b->B);
    for (int i = 0; i < b->B; i++) order[i] = i;
    std::stable_sort(order.begin(), order.end(), [&](int x, int y) {
        return gp[x] != gp[y] ? gp[x] > gp[y] : b->len[x] > b->len[y];
    });
    HIPCHK(hipMemcpyAsync(b->order_dev, order.data(), sizeof(int32_t) * b->B, hipMemcpyHostToDevice, st));
    for (int i = 0; i < b->B; i++) {
        HIPCHK(hipMemcpyAsync(b->rope_cur + 256 * i, d->rc + b->len[i] * hd, sizeof(float) * hd,
                              hipMemcpyDeviceToDevice, st));
        HIPCHK(hipMemcpyAsync(b->rope_cur + 256 * i + hd, d->rs + b->len[i] * hd, sizeof(float) * hd,
                              hipMemcpyDeviceToDevice, st));
    }
    HIPCHK(hipStreamSynchronize(st));
    return QASR_OK;
}

// n_steps greedy steps of every stream; the first consumes first_tokens[b];
// tokens_out [B][n_steps]
extern "C" int qasr_hip_batch_generate(qasr_batch *b, const int32_t *first_tokens, int32_t n_steps,
                                       int32_t *tokens_out) {
    if (!b || !first_tokens || !tokens_out || n_steps <= 0) return qasr_fail(QASR_ERR_INVALID, "batch_generate: bad arguments");
    qasr_decoder *d = b->d;
    CHECK_H(d->h);
    if (n_steps > b->max_steps) return qasr_fail(QASR_ERR_INVALID, "batch_generate: more steps than max_steps");
    const int64_t longest = *std::max_element(b->len.begin(), b->len.end());
    if (longest + n_steps > b->max_seq) return qasr_fail(QASR_ERR_INVALID, "batch_generate: KV capacity exceeded");
    TRY(batch_set_state(b, first_tokens));
    hipStream_t st = d->h->stream;
    for (int32_t s = 0; s < n_steps; s++) {
        // the longest stream's bucket sets the split count (the largest of the
        // streams'), the longest partition the attention's groups per wave
        const int S = batch_splits(b, batch_cap(b, longest + s));
        const int forms = batch_forms(b, s);
        const int gpw = (forms & 1) ? batch_step_gpw(b, s) : 0;
        if (!b->use_graph) {
            TRY(batch_enqueue_step(b, S, gpw, forms));
            continue;
        }
        const int key = (S * 8 + gpw) * 4 + forms;
        auto it = b->graphs.find(key);
        if (it == b->graphs.end()) {
            hipGraph_t g = nullptr;
            hipGraphExec_t ge = nullptr;
            HIPCHK(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
            int rc = batch_enqueue_step(b, S, gpw, forms);
            hipError_t e = hipStreamEndCapture(st, &g);
            if (rc != QASR_OK) {
                if (g) (void)hipGraphDestroy(g);
                return rc;
            }
            HIPCHK(e);
            e = hipGraphInstantiate(&ge, g, nullptr, nullptr, 0);
            (void)hipGraphDestroy(g);
            HIPCHK(e);
            it = b->graphs.emplace(key, ge).first;
        }
        HIPCHK(hipGraphLaunch(it->second, st));
    }
    // the whole [streams][max_steps] log in one contiguous copy, then the rows
    std::vector<int32_t> log((size_t)b->B * b->max_steps);
    int32_t fault = 0;
    HIPCHK(hipMemcpyAsync(log.data(), b->token_log, sizeof(int32_t) * log.size(), hipMemcpyDeviceToHost, st));
    HIPCHK(hipMemcpyAsync(&fault, b->fault, sizeof(fault), hipMemcpyDeviceToHost, st));
    HIPCHK(hipStreamSynchronize(st));
    if (fault) {
        const int32_t z = 0;
        HIPCHK(hipMemcpy(b->fault, &z, sizeof(z), hipMemcpyHostToDevice));
        return qasr_fail(QASR_ERR_HIP, "batch_generate: an attention partition exceeded its launch's groups per wave; "
                                       "the tokens of this call are not valid");
    }
    for (int i = 0; i < b->B; i++)
        memcpy(tokens_out + (size_t)i * n_steps, log.data() + (size_t)i * b->max_steps, sizeof(int32_t) * n_steps);
    for (auto &l : b->len) l += n_steps;
    return QASR_OK;
}

// HIP-event timing of each kernel kind of a step (back-to-back launches behind
// a delay kernel, as the single-stream decoder profile): per-layer kinds over
// the layers of one step, the others repeated once per layer; n_steps steps
// from first_tokens at the streams' current lengths, which are restored.
extern "C" int qasr_hip_batch_profile(qasr_batch *b, const int32_t *first_tokens, int32_t n_steps,
                                      float *us_per_launch, int32_t *launches_per_step) {
    if (!b || !first_tokens || !us_per_launch || n_steps <= 0)
        return qasr_fail(QASR_ERR_INVALID, "batch_profile: bad arguments");
    qasr_decoder *d = b->d;
    CHECK_H(d->h);
    const int64_t longest = *std::max_element(b->len.begin(), b->len.end());
    if (longest + n_steps > b->max_seq) return qasr_fail(QASR_ERR_INVALID, "batch_profile: KV capacity exceeded");
    hipStream_t st = d->h->stream;
    const int L = d->c.n_layers;
    const int reps_once = (int)std::min<int64_t>(L, b->max_steps);
    std::vector<int64_t> len0 = b->len;
    std::vector<int32_t> tok(first_tokens, first_tokens + b->B), st_h((size_t)b->B * 4);
    double tot[BK_KINDS] = {};
    int cnt[BK_KINDS] = {};
    hipEvent_t e0 = nullptr, e1 = nullptr;
    HIPCHK(hipEventCreate(&e0));
    HIPCHK(hipEventCreate(&e1));
    int rc = QASR_OK;
    for (int s = 0; s < n_steps && rc == QASR_OK; s++) {
        const int S = batch_splits(b, batch_cap(b, longest + s));
        const int forms = batch_forms(b, 0);                               // b->len advances per profiled step
        const int gpw = (forms & 1) ? batch_step_gpw(b, 0) : 0;
        if ((rc = batch_set_state(b, tok.data())) != QASR_OK) break;
        if ((rc = batch_enqueue_step(b, S, gpw, forms)) != QASR_OK) break;
        HIPCHK(hipMemcpyAsync(st_h.data(), b->state, sizeof(int32_t) * st_h.size(), hipMemcpyDeviceToHost, st));
        HIPCHK(hipStreamSynchronize(st));
        for (int k = 0; k < BK_KINDS && rc == QASR_OK; k++) {
            if (k == BK_PREP && forms == 1) continue;   // the attention does the q/k prep
            if ((rc = batch_set_state(b, tok.data())) != QASR_OK) break;
            LAUNCHCHK(launch_delay(400, st), "profile delay");
            HIPCHK(hipEventRecord(e0, st));
            const int reps = per_layer_kind(k) ? 1 : reps_once;
            for (int r = 0; r < reps && rc == QASR_OK; r++) rc = batch_enqueue_step(b, S, gpw, forms, k);
            HIPCHK(hipEventRecord(e1, st));
            HIPCHK(hipEventSynchronize(e1));
            float ms = 0.0f;
            HIPCHK(hipEventElapsedTime(&ms, e0, e1));
            tot[k] += ms * 1000.0;
            cnt[k] += per_layer_kind(k) ? L : reps_once;
        }
        for (int i = 0; i < b->B; i++) {
            tok[i] = st_h[4 * i];
            b->len[i] += 1;
        }
    }
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    b->len = len0;
    if (rc != QASR_OK) return rc;
    for (int k = 0; k < BK_KINDS; k++) {
        us_per_launch[k] = cnt[k] ? (float)(tot[k] / cnt[k]) : 0.0f;
        if (launches_per_step) launches_per_step[k] = cnt[k] ? (per_layer_kind(k) ? L : 1) : 0;
    }
    return QASR_OK;
}

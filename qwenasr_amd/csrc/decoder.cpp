// Device-resident Qwen3 decoder (decoder.rs): int8 weights packed on the GPU
// at load, an HBM-resident KV cache, and a decode step of 5 fused kernels per
// layer plus the LM-head argmax, replayed from a captured HIP graph.
#include "decoder.h"
#include "upload.h"

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

using namespace qasr;

template <typename T>
static int dalloc(qasr_decoder *d, T **p, size_t count) {
    void *v = nullptr;
    hipError_t e = hipMalloc(&v, count * sizeof(T) + 256);
    if (e != hipSuccess)
        return qasr_fail(QASR_ERR_NOMEM, std::string("decoder: hipMalloc of ") +
                                             std::to_string(count * sizeof(T)) + " bytes failed");
    d->allocs.push_back(v);
    *p = reinterpret_cast<T *>(v);
    return QASR_OK;
}

#define TRY(x)                  \
    do {                        \
        int rc_ = (x);          \
        if (rc_ != QASR_OK) {   \
            return rc_;         \
        }                       \
    } while (0)

static int upload(qasr_decoder *d, void *dst, const void *src, size_t bytes) {
    HIPCHK(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, d->h->stream));
    return QASR_OK;
}

// pack the device bf16 matrix bf [n, k] to int8 + scales on the device
static int pack(qasr_decoder *d, const uint16_t *bf, int64_t n, int64_t k, int8_t **q, float **s) {
    TRY(dalloc(d, q, n * k));
    TRY(dalloc(d, s, n));
    LAUNCHCHK(launch_pack_int8(bf, n, (int)k, d->round_mode, *q, *s, d->h->stream), "decoder pack");
    return QASR_OK;
}

// KV cache [layer][kv_head][cap][hd], zeroed
static int kv_alloc(qasr_decoder *d, int64_t cap, void **kc, void **vc) {
    const qasr_dec_config &c = d->c;
    const size_t bytes = (size_t)c.n_layers * c.n_kv_heads * cap * c.head_dim * (d->kv_bf16 ? 2 : 4);
    for (void **p : {kc, vc}) {
        *p = nullptr;
        if (hipMalloc(p, bytes) != hipSuccess) {
            *p = nullptr;
            return qasr_fail(QASR_ERR_NOMEM, "decoder: KV cache allocation failed");
        }
        d->allocs.push_back(*p);
        HIPCHK(hipMemsetAsync(*p, 0, bytes, d->h->stream));
    }
    return QASR_OK;
}

// RoPE table of cap positions (RopeCache::ensure, decoder.rs:301-338) with the host libm
static int rope_alloc(qasr_decoder *d, int64_t cap, float **rc, float **rs) {
    const qasr_dec_config &c = d->c;
    const int64_t hd = c.head_dim;
    std::vector<float> cs((size_t)cap * hd), sn((size_t)cap * hd), inv(hd / 2);
    for (int64_t i = 0; i < hd / 2; i++) inv[i] = 1.0f / powf(c.theta, (float)(2 * i) / (float)hd);
    for (int64_t p = 0; p < cap; p++)
        for (int64_t i = 0; i < hd / 2; i++) {
            const float a = (float)p * inv[i];
            const float cv = cosf(a), sv = sinf(a);
            cs[p * hd + i] = cv; cs[p * hd + hd / 2 + i] = cv;
            sn[p * hd + i] = sv; sn[p * hd + hd / 2 + i] = sv;
        }
    TRY(dalloc(d, rc, cs.size()));
    TRY(dalloc(d, rs, sn.size()));
    TRY(upload(d, *rc, cs.data(), sizeof(float) * cs.size()));
    TRY(upload(d, *rs, sn.data(), sizeof(float) * sn.size()));
    HIPCHK(hipStreamSynchronize(d->h->stream));   // the host tables go out of scope
    return QASR_OK;
}

static void release(qasr_decoder *d, void *p) {
    for (auto it = d->allocs.begin(); it != d->allocs.end(); ++it)
        if (*it == p) {
            d->allocs.erase(it);
            (void)hipFree(p);
            return;
        }
}

// KvCache::grow (decoder.rs:199-231): the cache doubles (at least to `need`
// positions, rounded up to a whole 256-position context bucket, at most 2^20)
// when a call needs more positions than it holds.  Every position of the old
// cache is copied to the same position of the new one, the RoPE table is
// rebuilt for the new capacity and the captured decode steps are dropped (they
// hold the old addresses).  The old RoPE tables stay allocated until the
// decoder is freed: a multi-stream batch's captured steps may still read them
// (their rows are the new table's rows).
int decoder_reserve(qasr_decoder *d, int64_t need) {
    if (need <= d->max_seq) return QASR_OK;
    const int64_t limit = (int64_t)1 << 20;
    if (need > limit) return qasr_fail(QASR_ERR_INVALID, "decoder: KV cache capacity exceeded (2^20 positions)");
    int64_t cap = std::max<int64_t>(2 * d->max_seq, need);
    cap = std::min<int64_t>((cap + 255) / 256 * 256, limit);
    const qasr_dec_config &c = d->c;
    hipStream_t st = d->h->stream;
    HIPCHK(hipStreamSynchronize(st));
    void *kc = nullptr, *vc = nullptr;
    float *rc = nullptr, *rs = nullptr;
    int32_t *log = nullptr;
    TRY(kv_alloc(d, cap, &kc, &vc));
    TRY(rope_alloc(d, cap, &rc, &rs));
    TRY(dalloc(d, &log, cap));
    const size_t esz = d->kv_bf16 ? 2 : 4, old_row = (size_t)d->max_seq * c.head_dim * esz;
    const size_t new_row = (size_t)cap * c.head_dim * esz, heads = (size_t)c.n_layers * c.n_kv_heads;
    HIPCHK(hipMemcpy2DAsync(kc, new_row, d->kc, old_row, old_row, heads, hipMemcpyDeviceToDevice, st));
    HIPCHK(hipMemcpy2DAsync(vc, new_row, d->vc, old_row, old_row, heads, hipMemcpyDeviceToDevice, st));
    HIPCHK(hipMemcpyAsync(log, d->token_log, sizeof(int32_t) * d->max_seq, hipMemcpyDeviceToDevice, st));
    HIPCHK(hipStreamSynchronize(st));
    for (auto &g : d->graphs) (void)hipGraphExecDestroy(g.second);
    d->graphs.clear();
    release(d, d->kc);
    release(d, d->vc);
    release(d, d->token_log);
    d->kc = kc;
    d->vc = vc;
    d->rc = rc;
    d->rs = rs;
    d->token_log = log;
    d->max_seq = cap;
    return QASR_OK;
}

extern "C" int qasr_hip_decoder_load(qasr_hip *h, const qasr_dec_config *cfg, const qasr_dec_weights *w,
                                     int round_mode, int64_t max_seq, int kv_bf16, qasr_decoder **out) {
    return decoder_load_impl(h, cfg, w, nullptr, 0, round_mode, max_seq, kv_bf16, out);
}

int decoder_load_impl(qasr_hip *h, const qasr_dec_config *cfg, const qasr_dec_weights *w, const uint16_t *lm_head,
                      int64_t lm_rows, int round_mode, int64_t max_seq, int kv_bf16, qasr_decoder **out) {
    CHECK_H(h);
    if (!cfg || !w || !out || !w->embed || !w->norm || !w->layers)
        return qasr_fail(QASR_ERR_INVALID, "decoder_load: null argument");
    *out = nullptr;
    const qasr_dec_config c = *cfg;
    // The decode step's split merges (k_oproj_merge, k_attn_merge_rows / _seq /
    // _heads) are laid out for the attention shape of both Qwen3-ASR decoders
    // (config.rs: 16 query heads, 8 KV heads of 128): other head counts are
    // refused here, before any of their partials could be merged as 16 heads.
    if (c.n_layers <= 0 || c.head_dim != 128 || c.n_kv_heads != 8 || c.n_heads != 16 || c.hidden <= 0 ||
        c.hidden % 64 != 0 || c.hidden > 4096 || c.intermediate <= 0 || (c.intermediate % 64) != 0 ||
        c.intermediate > 6144 || c.vocab <= 0 || max_seq <= 0 || max_seq > (1 << 20))
        return qasr_fail(QASR_ERR_INVALID,
                         "decoder_load: unsupported config (16 query heads and 8 KV heads of head_dim 128, "
                         "hidden/intermediate multiples of 64)");
    if (round_mode != QASR_ROUND_HALF_AWAY && round_mode != QASR_TRUNC)
        return qasr_fail(QASR_ERR_INVALID, "decoder_load: unknown round_mode");
    if (lm_head && (lm_rows <= 0 || lm_rows > (1 << 30)))
        return qasr_fail(QASR_ERR_INVALID, "decoder_load: bad LM head row count");
    for (int l = 0; l < c.n_layers; l++) {
        const qasr_dec_layer &L = w->layers[l];
        if (!L.wq || !L.wk || !L.wv || !L.wo || !L.gate || !L.up || !L.down || !L.q_norm || !L.k_norm ||
            !L.input_norm || !L.post_attn_norm)
            return qasr_fail(QASR_ERR_INVALID, "decoder_load: null weight in layer " + std::to_string(l));
    }
    qasr_decoder *d = new qasr_decoder();
    d->h = h;
    d->c = c;
    d->round_mode = round_mode;
    d->kv_bf16 = kv_bf16 ? 1 : 0;
    d->max_seq = max_seq;
    d->n_split = 0;   // automatic, per context bucket
    // QASR_DISABLE_GRAPH=1: launch decode steps kernel by kernel (profilers that
    // do not follow graph launches)
    const char *ng = getenv("QASR_DISABLE_GRAPH");
    if (ng && ng[0] == '1') d->use_graph = 0;
    // The decode attention is k_attn_step wherever a block's run fits it (at
    // most 16 groups of 8 positions).  Measured on the 0.6B decode: k_attn_step
    // with 4 waves of up to 4 groups each 5.72 / 6.50 / 7.42 us at contexts
    // 494 / 700 / 1000 against 6.76 / 7.24 / 7.86 for k_attn_decode; 8-wave
    // blocks were slower (5.82-7.30).  qasr_hip_decoder_set_fusion selects the
    // fused qkv + attention launch or two launches.
    int rc = decoder_build(d, w, lm_head, lm_head ? lm_rows : c.vocab);
    if (rc != QASR_OK) {
        qasr_hip_decoder_free(d);
        return rc;
    }
    *out = d;
    return QASR_OK;
}

int decoder_build(qasr_decoder *d, const qasr_dec_weights *w, const uint16_t *lm_head, int64_t lm_rows) {
    const qasr_dec_config &c = d->c;
    const int64_t H = c.hidden, hd = c.head_dim, qd = (int64_t)c.n_heads * hd;
    const int64_t kvd = (int64_t)c.n_kv_heads * hd, I = c.intermediate, V = c.vocab;
    const int64_t nqkv = qd + 2 * kvd;
    // every matrix goes host -> HBM through the pinned staging ring (the q|k|v
    // concatenation and the gate/up interleave are assembled on the way) and
    // is packed to int8 on the device behind its upload
    Stager stg(d->h->stream);
    TRY(stg.init());
    const size_t B2 = sizeof(uint16_t);
    d->L.resize(c.n_layers);
    for (int l = 0; l < c.n_layers; l++) {
        const qasr_dec_layer &S = w->layers[l];
        DecLayerDev &D = d->L[l];
        // q | k | v concatenated by rows (one fused projection)
        TRY(dalloc(d, &D.bqkv, nqkv * H));
        TRY(stg.upload(D.bqkv, S.wq, B2 * qd * H));
        TRY(stg.upload(D.bqkv + qd * H, S.wk, B2 * kvd * H));
        TRY(stg.upload(D.bqkv + (qd + kvd) * H, S.wv, B2 * kvd * H));
        TRY(pack(d, D.bqkv, nqkv, H, &D.wqkv, &D.sqkv));
        TRY(dalloc(d, &D.bo, H * qd));
        TRY(stg.upload(D.bo, S.wo, B2 * H * qd));
        TRY(pack(d, D.bo, H, qd, &D.wo, &D.so));
        // gate/up interleaved by rows (decoder.rs:91-104)
        TRY(dalloc(d, &D.bgu, 2 * I * H));
        const void *gu[2] = {S.gate, S.up};
        TRY(stg.upload_rows(D.bgu, gu, 2, I, B2 * H));
        TRY(pack(d, D.bgu, 2 * I, H, &D.wgu, &D.sgu));
        TRY(dalloc(d, &D.bdown, H * I));
        TRY(stg.upload(D.bdown, S.down, B2 * H * I));
        TRY(pack(d, D.bdown, H, I, &D.wdown, &D.sdown));
        TRY(dalloc(d, &D.q_norm, hd));
        TRY(dalloc(d, &D.k_norm, hd));
        TRY(dalloc(d, &D.in_norm, H));
        TRY(dalloc(d, &D.post_norm, H));
        TRY(upload(d, D.q_norm, S.q_norm, sizeof(float) * hd));
        TRY(upload(d, D.k_norm, S.k_norm, sizeof(float) * hd));
        TRY(upload(d, D.in_norm, S.input_norm, sizeof(float) * H));
        TRY(upload(d, D.post_norm, S.post_attn_norm, sizeof(float) * H));
    }
    // embedding table (bf16, kept for lookups) and the int8 decode head packed
    // from it, or from a separate [lm_rows, hidden] head (decoder.rs:143-157:
    // the forced aligner's head has classify_num rows)
    TRY(dalloc(d, &d->embed, V * H));
    TRY(stg.upload(d->embed, w->embed, B2 * V * H));
    d->lm_i8_rows = lm_head ? lm_rows : V;
    TRY(dalloc(d, &d->lm, d->lm_i8_rows * H));
    TRY(dalloc(d, &d->lm_s, d->lm_i8_rows));
    if (lm_head) {
        uint16_t *tmp = nullptr;
        TRY(dalloc(d, &tmp, lm_rows * H));     // bf16 staging, freed with the decoder
        TRY(stg.upload(tmp, lm_head, B2 * lm_rows * H));
        LAUNCHCHK(launch_pack_int8(tmp, lm_rows, (int)H, d->round_mode, d->lm, d->lm_s, d->h->stream), "lm pack");
    } else {
        LAUNCHCHK(launch_pack_int8(d->embed, V, (int)H, d->round_mode, d->lm, d->lm_s, d->h->stream), "lm pack");
    }
    TRY(stg.finish());
    TRY(dalloc(d, &d->norm, H));
    TRY(upload(d, d->norm, w->norm, sizeof(float) * H));
    TRY(kv_alloc(d, d->max_seq, &d->kc, &d->vc));
    TRY(rope_alloc(d, d->max_seq, &d->rc, &d->rs));
    TRY(dalloc(d, &d->rope_cur, 2 * d->c.head_dim));
    TRY(dalloc(d, &d->x, H));
    TRY(dalloc(d, &d->qkv, nqkv));
    TRY(dalloc(d, &d->att, qd));
    TRY(dalloc(d, &d->ffn, I));
    TRY(dalloc(d, &d->state, 8));
    TRY(dalloc(d, &d->qkv_tag, nqkv));
    HIPCHK(hipMemsetAsync(d->qkv_tag, 0, sizeof(unsigned long long) * nqkv, d->h->stream));
    {
        // epoch 1 (tag 0, which the cleared pairs hold, is never a live tag), no fault
        const int32_t init[8] = {0, 0, 0, 0, 1, 0, 0, 0};
        HIPCHK(hipMemcpy(d->state, init, sizeof(init), hipMemcpyHostToDevice));
    }
    TRY(dalloc(d, &d->token_log, d->max_seq));
    TRY(dalloc(d, &d->out_idx, 4));
    TRY(dalloc(d, &d->counters, QASR_COUNTERS));
    HIPCHK(hipMemsetAsync(d->counters, 0, QASR_COUNTERS * sizeof(unsigned), d->h->stream));
    TRY(dalloc(d, &d->am_val, QASR_ARGMAX_MAX_BLOCKS));
    TRY(dalloc(d, &d->am_idx, QASR_ARGMAX_MAX_BLOCKS));
    TRY(dalloc(d, &d->part, (size_t)c.n_kv_heads * 64 * 2 * (hd + 2)));
    HIPCHK(hipStreamSynchronize(d->h->stream));
    return QASR_OK;
}

extern "C" void qasr_hip_decoder_free(qasr_decoder *d) {
    if (!d) return;
    (void)hipSetDevice(d->h->device);
    (void)hipStreamSynchronize(d->h->stream);
    for (auto &g : d->graphs) (void)hipGraphExecDestroy(g.second);
    decoder_free_prefill(d);
    dbuf_release(d->head_out);
    dbuf_release(d->gemm_ws);
    if (d->lm_bf16) (void)hipFree(d->lm_bf16);
    for (void *p : d->allocs) (void)hipFree(p);
    delete d;
}

// ---------------------------------------------------------------------------
// one decode step: per layer [norm+qkv] [qk-norm+rope+kv-write+attention]
// [o-proj += ] [norm+gate_up+swiglu] [down += ], then [norm+LM-head argmax]
// ---------------------------------------------------------------------------
// The fused qkv + attention launch applies with k_attn_step, 4 qkv rows per
// wave, K of 1024 or 2048 and at most 32 layers (5 bits of the tag)
static bool fused_qkv_attn(const qasr_decoder *d, bool step_kernel, int qkv_rows) {
    const qasr_dec_config &c = d->c;
    return d->attn_fuse && step_kernel && qkv_rows == 4 && (c.hidden == 1024 || c.hidden == 2048) &&
           c.n_layers <= 32 && c.head_dim == 128 && c.n_heads == 2 * c.n_kv_heads;
}

int64_t decoder_ctx_cap(const qasr_decoder *d, int64_t L) {
    const int64_t c = ((L + 255) / 256) * 256;
    return std::min<int64_t>(std::max<int64_t>(c, 256), d->max_seq);
}

// profiling build: the phase stamps of kernel kind k (0 the fused qkv +
// attention launch, 1 o_proj, 2 gate_up, 3 down), each [layer][QASR_STAMP_BLOCKS][slots]
static unsigned long long *stamp_region(const qasr_decoder *d, int k) {
    return d->stamps ? d->stamps + (size_t)k * d->c.n_layers * QASR_STAMP_BLOCKS * QASR_STAMP_SLOTS : nullptr;
}

int decoder_enqueue_step(qasr_decoder *d, bool embed_mode, int only_kind) {
    const qasr_dec_config &c = d->c;
    const int H = c.hidden, hd = c.head_dim, qd = c.n_heads * hd, kvd = c.n_kv_heads * hd;
    const int I = c.intermediate;
    hipStream_t st = d->h->stream;
    const size_t esz = d->kv_bf16 ? 2 : 4;
    const int64_t layer_elems = (int64_t)c.n_kv_heads * d->max_seq * hd;
    const float scale = 1.0f / sqrtf((float)hd);
    auto want = [only_kind](int kind) { return only_kind < 0 || only_kind == kind; };
    // with 1, 2, 4, 8 or 16 splits the o_proj kernel merges the attention
    // partials in its prologue; otherwise a merge kernel writes the attention
    // row and the plain o_proj kernel quantizes it.  The context bucket of
    // this step sizes the attention's static partition and its splits
    const int64_t cap = decoder_ctx_cap(d, d->step_pos + 1);
    const int n_split = d->n_split > 0 ? d->n_split : attn_splits_auto(c, cap);
    const bool fused_merge = oproj_merges(c, n_split);
    // rows per wave of the qkv, gate_up, down and plain o_proj matvecs: about
    // 1024 waves per launch (rows / 1024 rounded up to 1, 2, 4 or 8; SwiGLU
    // pairs need 2).  Measured on the 0.6B and 1.7B shapes: fewer rows per
    // wave leave each wave's fixed prologue and reductions on too little data,
    // more leave fewer waves to stream the matrix.
    auto rows_for = [](int64_t rows, bool swiglu) {
        int r = 1;
        while (r < 8 && (int64_t)r * 1024 < rows) r *= 2;
        return swiglu ? std::max(r, 2) : r;
    };
    // (o_proj: about 512 waves; the fused split merge that every block
    // repeats favours fewer blocks)
    std::array<int, 4> mv_rows{rows_for(qd + 2 * kvd, false), rows_for(2 * I, true), rows_for(H, false),
                               std::min(4, 2 * rows_for(H, false))};
    for (int l = 0; l < c.n_layers; l++) {
        const DecLayerDev &L = d->L[l];
        MvArgs a{};
        a.x = d->x; a.embed = d->embed; a.state = d->state; a.norm_w = L.in_norm; a.eps = c.eps; a.K = H;
        a.seg[0] = {L.wqkv, L.sqkv, d->qkv, qd + 2 * kvd};
        a.n_total = qd + 2 * kvd;
        a.resid_out = d->x;
        AttnDecodeArgs t{};
        t.qkv = d->qkv; t.q_norm = L.q_norm; t.k_norm = L.k_norm;
        t.rope_cos = d->rc; t.rope_sin = d->rs; t.rope_cur = d->rope_cur; t.state = d->state;
        t.kcache = (char *)d->kc + (size_t)l * layer_elems * esz;
        t.vcache = (char *)d->vc + (size_t)l * layer_elems * esz;
        t.head_stride = (int64_t)d->max_seq * hd;
        t.part = d->part; t.counters = d->counters + QASR_CTR_ATTN; t.out = d->att;
        t.n_split = n_split; t.waves = d->attn_waves; t.eps = c.eps; t.scale = scale;
        // static partition of the step's context bucket: the first KV loads need no device state
        t.gpb = (int)((((cap + 7) / 8) + n_split - 1) / n_split);
        // k_attn_step (one query head per block, same partials, 4 waves) when
        // a block's run is at most 4 groups per wave
        const bool step_kernel = d->attn_step && attn_step_gpw(t.gpb) > 0;
        if (step_kernel) {
            t.waves = 4;
            t.gpw = attn_step_gpw(t.gpb);
        }
        // the qkv matvec and k_attn_step as one launch (kind 0; kind 1 then
        // launches nothing): the qkv rows reach the attention as tagged pairs
        if (only_kind == 7) {
            // profile only: the RMSNorm + qkv matvec as its own launch (the
            // two-launch form's first kernel), whatever form the step uses
            LAUNCHCHK(launch_w8a8(a, MV_PLAIN, true, embed_mode && l == 0, mv_rows[0], st), "profile qkv");
            continue;
        }
        if (fused_qkv_attn(d, step_kernel, mv_rows[0])) {
            if (want(0)) {
                t.qkv_tag = d->qkv_tag; t.layer = l; t.fault = d->state + 5; t.stamps = stamp_region(d, 0);
                LAUNCHCHK(launch_qkv_attn(a, t, c.n_heads, c.n_kv_heads, hd, d->kv_bf16, embed_mode && l == 0,
                                          mv_rows[0], st),
                          "step qkv + attention");
            }
        } else {
            if (want(0)) LAUNCHCHK(launch_w8a8(a, MV_PLAIN, true, embed_mode && l == 0, mv_rows[0], st), "step qkv");
            if (want(1))
                LAUNCHCHK(launch_attn_decode(t, c.n_heads, c.n_kv_heads, hd, d->kv_bf16, st, false), "step attention");
        }
        if (want(2)) {
            if (fused_merge) {
                OprojMergeArgs om{d->part, n_split, c.n_kv_heads, L.wo, L.so, d->x, H, stamp_region(d, 1), l};
                LAUNCHCHK(launch_oproj_merge(om, mv_rows[3], st), "step o_proj");
            } else {
                LAUNCHCHK(launch_attn_merge_rows(d->part, 0, n_split, d->att, qd, nullptr, nullptr, 1, st),
                          "step attention merge");
                MvArgs o{};
                o.x = d->att; o.K = qd;
                o.seg[0] = {L.wo, L.so, d->x, H};
                o.n_total = H;
                LAUNCHCHK(launch_w8a8(o, MV_ADDTO, false, false, mv_rows[3], st), "step o_proj");
            }
        }
        if (want(3)) {
            MvArgs g{};
            g.x = d->x; g.norm_w = L.post_norm; g.eps = c.eps; g.K = H;
            g.seg[0] = {L.wgu, L.sgu, d->ffn, 2 * I};
            g.n_total = 2 * I;
            g.stamps = stamp_region(d, 2);
            g.layer = l;
            LAUNCHCHK(launch_w8a8(g, MV_SWIGLU, true, false, mv_rows[1], st), "step gate_up");
        }
        if (want(4)) {
            MvArgs dn{};
            dn.x = d->ffn; dn.K = I;
            dn.seg[0] = {L.wdown, L.sdown, d->x, H};
            dn.n_total = H;
            dn.stamps = stamp_region(d, 3);
            dn.layer = l;
            LAUNCHCHK(launch_w8a8(dn, MV_ADDTO, false, false, mv_rows[2], st), "step down");
        }
    }
    if (want(5) || want(6)) {
        ArgmaxArgs am{};
        am.x = d->x; am.norm_w = d->norm; am.eps = c.eps; am.K = H; am.N = (int)d->lm_i8_rows;
        am.w = d->lm; am.ws = d->lm_s;
        am.part_val = d->am_val; am.part_idx = d->am_idx;
        am.out_idx = d->out_idx; am.out_val = reinterpret_cast<float *>(d->out_idx + 1);
        am.state = d->state; am.token_log = d->token_log;
        am.rope_cos = d->rc; am.rope_sin = d->rs; am.rope_cur = d->rope_cur; am.max_pos = (int)d->max_seq;
        am.epoch = d->state + 4;
        LAUNCHCHK(launch_argmax(am, true, argmax_blocks(d->lm_i8_rows), st, want(5), want(6)), "step argmax");
        if (want(6)) d->epochs += 1;
    }
    return QASR_OK;
}

int decoder_set_state(qasr_decoder *d, int32_t token) {
    const int64_t hd = d->c.head_dim;
    // tags are epoch * 32 + layer in 32 bits: long before the epoch reaches
    // 2^27 (one call runs at most max_seq steps) the pairs are cleared and the
    // epoch restarts at 1
    if (d->epochs >= ((int64_t)1 << 26)) {
        const int64_t nqkv = (int64_t)(d->c.n_heads + 2 * d->c.n_kv_heads) * d->c.head_dim;
        static const int32_t one = 1;
        HIPCHK(hipMemsetAsync(d->qkv_tag, 0, sizeof(unsigned long long) * nqkv, d->h->stream));
        HIPCHK(hipMemcpyAsync(d->state + 4, &one, sizeof(one), hipMemcpyHostToDevice, d->h->stream));
        HIPCHK(hipStreamSynchronize(d->h->stream));
        d->epochs = 0;
    }
    d->host_state[0] = token;
    d->host_state[1] = (int32_t)d->len;
    d->host_state[2] = 0;
    d->host_state[3] = 0;
    HIPCHK(hipMemcpyAsync(d->state, d->host_state, sizeof(d->host_state), hipMemcpyHostToDevice, d->h->stream));
    d->step_pos = d->len;
    if (d->len < d->max_seq) {
        HIPCHK(hipMemcpyAsync(d->rope_cur, d->rc + d->len * hd, sizeof(float) * hd, hipMemcpyDeviceToDevice,
                              d->h->stream));
        HIPCHK(hipMemcpyAsync(d->rope_cur + hd, d->rs + d->len * hd, sizeof(float) * hd, hipMemcpyDeviceToDevice,
                              d->h->stream));
    }
    return QASR_OK;
}

static int set_state(qasr_decoder *d, int32_t token) { return decoder_set_state(d, token); }

// Token-fed decode steps replay captured graphs, one per (context bucket,
// steps per graph): runs of QASR_GRAPH_STEPS steps inside one bucket replay a
// graph of that many steps (the device advances token, position and RoPE rows
// between them), the rest one step at a time.  The kernels and their order are
// those of single steps, so the results do not depend on the grouping.
#define QASR_GRAPH_STEPS 4
static int run_step_graph(qasr_decoder *d, int64_t cap, int n) {
    const int64_t key = cap * 16 + n;
    auto it = d->graphs.find(key);
    if (it == d->graphs.end()) {
        hipGraph_t g = nullptr;
        hipGraphExec_t ge = nullptr;
        const int64_t pos0 = d->step_pos;
        HIPCHK(hipStreamBeginCapture(d->h->stream, hipStreamCaptureModeThreadLocal));
        int rc = QASR_OK;
        for (int k = 0; k < n && rc == QASR_OK; k++) {
            rc = decoder_enqueue_step(d, true);
            d->step_pos += 1;
        }
        d->step_pos = pos0;
        hipError_t e = hipStreamEndCapture(d->h->stream, &g);
        if (rc != QASR_OK) {
            if (g) (void)hipGraphDestroy(g);
            return rc;
        }
        HIPCHK(e);
        e = hipGraphInstantiate(&ge, g, nullptr, nullptr, 0);
        (void)hipGraphDestroy(g);
        HIPCHK(e);
        it = d->graphs.emplace(key, ge).first;
    }
    HIPCHK(hipGraphLaunch(it->second, d->h->stream));
    d->step_pos += n;
    d->epochs += n;
    return QASR_OK;
}

int decoder_run_embed_steps(qasr_decoder *d, int64_t n) {
    while (n > 0) {
        if (!d->use_graph) {
            TRY(decoder_enqueue_step(d, true));
            d->step_pos += 1;
            n -= 1;
            continue;
        }
        const int64_t cap = decoder_ctx_cap(d, d->step_pos + 1);
        const int k = n >= QASR_GRAPH_STEPS && decoder_ctx_cap(d, d->step_pos + QASR_GRAPH_STEPS) == cap
                          ? QASR_GRAPH_STEPS : 1;
        TRY(run_step_graph(d, cap, k));
        n -= k;
    }
    return QASR_OK;
}

int decoder_run_embed_step(qasr_decoder *d) { return decoder_run_embed_steps(d, 1); }

int decoder_fault_check(qasr_decoder *d) {
    int32_t f = 0;
    HIPCHK(hipMemcpy(&f, d->state + 5, sizeof(f), hipMemcpyDeviceToHost));
    if (f == 0) return QASR_OK;
    const int32_t z = 0;
    HIPCHK(hipMemcpy(d->state + 5, &z, sizeof(z), hipMemcpyHostToDevice));
    return qasr_fail(QASR_ERR_HIP, "decode step: an attention block never observed the step's qkv rows (the fused "
                                   "qkv + attention hand-off timed out); the tokens of this call are not valid");
}

extern "C" int qasr_hip_decoder_forward(qasr_decoder *d, const float *embed, int32_t token_in,
                                        int32_t *token_out) {
    if (!d) return qasr_fail(QASR_ERR_INVALID, "decoder is null");
    CHECK_H(d->h);
    if (!token_out) return qasr_fail(QASR_ERR_INVALID, "token_out is null");
    TRY(decoder_reserve(d, d->len + 1));
    if (!embed && (token_in < 0 || token_in >= d->c.vocab))
        return qasr_fail(QASR_ERR_INVALID, "decoder_forward: token id out of range");
    TRY(set_state(d, token_in));
    if (embed) {
        HIPCHK(hipMemcpyAsync(d->x, embed, sizeof(float) * d->c.hidden, hipMemcpyHostToDevice, d->h->stream));
        TRY(decoder_enqueue_step(d, false));
        d->step_pos += 1;
    } else {
        TRY(decoder_run_embed_step(d));
    }
    HIPCHK(hipMemcpyAsync(d->host_state, d->state, sizeof(d->host_state), hipMemcpyDeviceToHost, d->h->stream));
    HIPCHK(hipStreamSynchronize(d->h->stream));
    TRY(decoder_fault_check(d));
    *token_out = d->host_state[0];
    d->len += 1;
    return QASR_OK;
}

extern "C" int qasr_hip_decoder_generate(qasr_decoder *d, const float *first_embed, int32_t first_token,
                                         int32_t n_steps, int32_t *tokens_out) {
    if (!d) return qasr_fail(QASR_ERR_INVALID, "decoder is null");
    CHECK_H(d->h);
    if (n_steps <= 0 || !tokens_out) return qasr_fail(QASR_ERR_INVALID, "decoder_generate: bad arguments");
    TRY(decoder_reserve(d, d->len + n_steps));
    if (!first_embed && (first_token < 0 || first_token >= d->c.vocab))
        return qasr_fail(QASR_ERR_INVALID, "decoder_generate: token id out of range");
    TRY(set_state(d, first_token));
    if (first_embed) {
        HIPCHK(hipMemcpyAsync(d->x, first_embed, sizeof(float) * d->c.hidden, hipMemcpyHostToDevice,
                              d->h->stream));
        TRY(decoder_enqueue_step(d, false));
        d->step_pos += 1;
    } else {
        TRY(decoder_run_embed_step(d));
    }
    TRY(decoder_run_embed_steps(d, n_steps - 1));
    HIPCHK(hipMemcpyAsync(tokens_out, d->token_log, sizeof(int32_t) * n_steps, hipMemcpyDeviceToHost,
                          d->h->stream));
    HIPCHK(hipStreamSynchronize(d->h->stream));
    TRY(decoder_fault_check(d));
    d->len += n_steps;
    return QASR_OK;
}

extern "C" int qasr_hip_decoder_last_logit(qasr_decoder *d, float *best) {
    if (!d || !best) return qasr_fail(QASR_ERR_INVALID, "decoder_last_logit: null argument");
    CHECK_H(d->h);
    HIPCHK(hipMemcpyAsync(best, d->out_idx + 1, sizeof(float), hipMemcpyDeviceToHost, d->h->stream));
    HIPCHK(hipStreamSynchronize(d->h->stream));
    return QASR_OK;
}

extern "C" int qasr_hip_decoder_set_len(qasr_decoder *d, int64_t len) {
    if (!d) return qasr_fail(QASR_ERR_INVALID, "decoder is null");
    if (len < 0 || len > d->max_seq) return qasr_fail(QASR_ERR_INVALID, "decoder_set_len: out of range");
    d->len = len;
    return QASR_OK;
}

extern "C" int64_t qasr_hip_decoder_len(const qasr_decoder *d) { return d ? d->len : -1; }

extern "C" int64_t qasr_hip_decoder_capacity(const qasr_decoder *d) { return d ? d->max_seq : -1; }

extern "C" int qasr_hip_decoder_set_fusion(qasr_decoder *d, int fuse_qkv_attention) {
    if (!d) return qasr_fail(QASR_ERR_INVALID, "decoder is null");
    if (fuse_qkv_attention != 0 && fuse_qkv_attention != 1)
        return qasr_fail(QASR_ERR_INVALID, "decoder_set_fusion: fuse_qkv_attention must be 0 or 1");
    CHECK_H(d->h);
    if (d->attn_fuse != fuse_qkv_attention) {
        HIPCHK(hipStreamSynchronize(d->h->stream));
        for (auto &g : d->graphs) (void)hipGraphExecDestroy(g.second);
        d->graphs.clear();
        d->attn_fuse = fuse_qkv_attention;
    }
    return QASR_OK;
}

// Phase stamps of the fused qkv + attention launch (the profiling build,
// libqasr_hip_stamps.so, only): dev is a device buffer of n_layers x (the
// launch's blocks) x QASR_STAMP_SLOTS 64-bit counters, or null to stop.
extern "C" int qasr_hip_decoder_set_stamps(qasr_decoder *d, void *dev, int64_t bytes) {
    if (!d) return qasr_fail(QASR_ERR_INVALID, "decoder is null");
    CHECK_H(d->h);
#ifdef QASR_STAMPS
    const qasr_dec_config &c = d->c;
    const int64_t blocks = (int64_t)(c.n_heads + 2 * c.n_kv_heads) * c.head_dim / 16 + 2 * c.n_kv_heads * 64;
    if (blocks > QASR_STAMP_BLOCKS || 2 * (int64_t)c.intermediate / 16 > QASR_STAMP_BLOCKS)
        return qasr_fail(QASR_ERR_INVALID, "decoder_set_stamps: more blocks per launch than the stamp layout holds");
    if (dev && bytes < 4 * (int64_t)c.n_layers * QASR_STAMP_BLOCKS * QASR_STAMP_SLOTS * 8)
        return qasr_fail(QASR_ERR_INVALID, "decoder_set_stamps: buffer too small (4 kinds x layers x 2048 blocks)");
    HIPCHK(hipStreamSynchronize(d->h->stream));
    for (auto &g : d->graphs) (void)hipGraphExecDestroy(g.second);
    d->graphs.clear();
    d->stamps = reinterpret_cast<unsigned long long *>(dev);
    return QASR_OK;
#else
    (void)dev;
    (void)bytes;
    return qasr_fail(QASR_ERR_INVALID, "decoder_set_stamps: this library is built without phase stamps "
                                       "(libqasr_hip_stamps.so has them)");
#endif
}

extern "C" int qasr_hip_decoder_set_options(qasr_decoder *d, int attn_splits, int use_graph) {
    if (!d) return qasr_fail(QASR_ERR_INVALID, "decoder is null");
    CHECK_H(d->h);
    if (attn_splits < 0) d->n_split = 0;
    if (attn_splits > 0) {
        if (attn_splits > 64)
            return qasr_fail(QASR_ERR_INVALID, "decoder_set_options: attn_splits must be <= 64");
        d->n_split = attn_splits;
    }
    d->use_graph = use_graph ? 1 : 0;
    if (!d->graphs.empty()) {
        HIPCHK(hipStreamSynchronize(d->h->stream));
        for (auto &g : d->graphs) HIPCHK(hipGraphExecDestroy(g.second));
        d->graphs.clear();
    }
    return QASR_OK;
}

extern "C" int qasr_hip_decoder_packed(qasr_decoder *d, int layer, int which, int8_t *q_host,
                                       float *scales_host) {
    if (!d) return qasr_fail(QASR_ERR_INVALID, "decoder is null");
    CHECK_H(d->h);
    const qasr_dec_config &c = d->c;
    const int64_t H = c.hidden, hd = c.head_dim, qd = (int64_t)c.n_heads * hd;
    const int64_t kvd = (int64_t)c.n_kv_heads * hd, I = c.intermediate;
    const int8_t *q = nullptr;
    const float *s = nullptr;
    int64_t rows = 0, cols = H;
    if (layer == -1) {
        q = d->lm; s = d->lm_s; rows = d->lm_i8_rows;
    } else if (layer >= 0 && layer < c.n_layers && which >= 0 && which <= 5) {
        const DecLayerDev &L = d->L[layer];
        switch (which) {
            case 0: q = L.wqkv; s = L.sqkv; rows = qd; break;
            case 1: q = L.wqkv + qd * H; s = L.sqkv + qd; rows = kvd; break;
            case 2: q = L.wqkv + (qd + kvd) * H; s = L.sqkv + qd + kvd; rows = kvd; break;
            case 3: q = L.wo; s = L.so; rows = H; cols = qd; break;
            case 4: q = L.wgu; s = L.sgu; rows = 2 * I; break;
            default: q = L.wdown; s = L.sdown; rows = H; cols = I; break;
        }
    } else {
        return qasr_fail(QASR_ERR_INVALID, "decoder_packed: bad layer / which");
    }
    if (q_host) HIPCHK(hipMemcpyAsync(q_host, q, rows * cols, hipMemcpyDeviceToHost, d->h->stream));
    if (scales_host) HIPCHK(hipMemcpyAsync(scales_host, s, sizeof(float) * rows, hipMemcpyDeviceToHost, d->h->stream));
    HIPCHK(hipStreamSynchronize(d->h->stream));
    return QASR_OK;
}

// host f32 <-> device cache.  A bf16 cache is converted on the host (f32 -> bf16
// round-to-nearest-even on upload; bf16 -> f32 is exact on download), in
// slices so the staging buffer stays small.
static uint16_t f32_to_bf16_host(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

static int kv_copy(qasr_decoder *d, float *kh, float *vh, bool up) {
    if (!d) return qasr_fail(QASR_ERR_INVALID, "decoder is null");
    CHECK_H(d->h);
    const size_t n = (size_t)d->c.n_layers * d->c.n_kv_heads * d->max_seq * d->c.head_dim;
    if (!d->kv_bf16) {
        if (up) {
            if (kh) HIPCHK(hipMemcpyAsync(d->kc, kh, n * 4, hipMemcpyHostToDevice, d->h->stream));
            if (vh) HIPCHK(hipMemcpyAsync(d->vc, vh, n * 4, hipMemcpyHostToDevice, d->h->stream));
        } else {
            if (kh) HIPCHK(hipMemcpyAsync(kh, d->kc, n * 4, hipMemcpyDeviceToHost, d->h->stream));
            if (vh) HIPCHK(hipMemcpyAsync(vh, d->vc, n * 4, hipMemcpyDeviceToHost, d->h->stream));
        }
        HIPCHK(hipStreamSynchronize(d->h->stream));
        return QASR_OK;
    }
    const size_t slice = (size_t)1 << 22;
    std::vector<uint16_t> tmp(std::min(n, slice));
    for (int which = 0; which < 2; which++) {
        float *hbuf = which ? vh : kh;
        uint16_t *dbuf = reinterpret_cast<uint16_t *>(which ? d->vc : d->kc);
        if (!hbuf) continue;
        for (size_t o = 0; o < n; o += slice) {
            const size_t m = std::min(slice, n - o);
            if (up) {
                for (size_t i = 0; i < m; i++) tmp[i] = f32_to_bf16_host(hbuf[o + i]);
                HIPCHK(hipMemcpy(dbuf + o, tmp.data(), m * 2, hipMemcpyHostToDevice));
            } else {
                HIPCHK(hipMemcpy(tmp.data(), dbuf + o, m * 2, hipMemcpyDeviceToHost));
                for (size_t i = 0; i < m; i++) {
                    const uint32_t u = (uint32_t)tmp[i] << 16;
                    std::memcpy(hbuf + o + i, &u, 4);
                }
            }
        }
    }
    return QASR_OK;
}

extern "C" int qasr_hip_decoder_kv_upload(qasr_decoder *d, const float *k, const float *v) {
    return kv_copy(d, const_cast<float *>(k), const_cast<float *>(v), true);
}

extern "C" int qasr_hip_decoder_kv_download(qasr_decoder *d, float *k, float *v) {
    return kv_copy(d, k, v, false);
}

// rows [start, start + n) of every (layer, KV head) against host [layer][kv_head][n][head_dim] f32
static int kv_rows_copy(qasr_decoder *d, int64_t start, int64_t n, float *kh, float *vh, bool up) {
    if (!d) return qasr_fail(QASR_ERR_INVALID, "decoder is null");
    CHECK_H(d->h);
    if (start < 0 || n <= 0 || start + n > d->max_seq)
        return qasr_fail(QASR_ERR_INVALID, "decoder_kv_rows: rows outside the cache");
    const qasr_dec_config &c = d->c;
    const size_t heads = (size_t)c.n_layers * c.n_kv_heads, row = (size_t)c.head_dim;
    const size_t esz = d->kv_bf16 ? 2 : 4, width = (size_t)n * row * esz, pitch = (size_t)d->max_seq * row * esz;
    hipStream_t st = d->h->stream;
    std::vector<uint16_t> tmp(d->kv_bf16 ? heads * n * row : 0);
    for (int which = 0; which < 2; which++) {
        float *hb = which ? vh : kh;
        char *db = reinterpret_cast<char *>(which ? d->vc : d->kc) + (size_t)start * row * esz;
        if (!hb) continue;
        if (!d->kv_bf16) {
            if (up) HIPCHK(hipMemcpy2DAsync(db, pitch, hb, width, width, heads, hipMemcpyHostToDevice, st));
            else HIPCHK(hipMemcpy2DAsync(hb, width, db, pitch, width, heads, hipMemcpyDeviceToHost, st));
            HIPCHK(hipStreamSynchronize(st));
            continue;
        }
        if (up) {
            for (size_t i = 0; i < tmp.size(); i++) tmp[i] = f32_to_bf16_host(hb[i]);
            HIPCHK(hipMemcpy2DAsync(db, pitch, tmp.data(), width, width, heads, hipMemcpyHostToDevice, st));
            HIPCHK(hipStreamSynchronize(st));
        } else {
            HIPCHK(hipMemcpy2DAsync(tmp.data(), width, db, pitch, width, heads, hipMemcpyDeviceToHost, st));
            HIPCHK(hipStreamSynchronize(st));
            for (size_t i = 0; i < tmp.size(); i++) {
                const uint32_t u = (uint32_t)tmp[i] << 16;
                std::memcpy(hb + i, &u, 4);
            }
        }
    }
    return QASR_OK;
}

extern "C" int qasr_hip_decoder_kv_upload_rows(qasr_decoder *d, int64_t start, int64_t n, const float *k,
                                               const float *v) {
    return kv_rows_copy(d, start, n, const_cast<float *>(k), const_cast<float *>(v), true);
}

extern "C" int qasr_hip_decoder_kv_download_rows(qasr_decoder *d, int64_t start, int64_t n, float *k, float *v) {
    return kv_rows_copy(d, start, n, k, v, false);
}

// ---------------------------------------------------------------------------
// per-kernel timing.  Each of n_steps real decode steps runs unbracketed (no
// graph); then, from the same input state, every kernel kind is launched once
// per layer back to back (the LM head n_layers times) between two HIP events
// on the handle's stream, behind a 400 us delay kernel that holds the stream
// until the host has queued the batch.  The average per launch is then the
// kernel's duration plus the queue's inter-dispatch gap, neither an event
// bracket's overhead nor the host's launch rate.  These
// extra launches rewrite the KV slot of the step's position, the residual and
// the step buffers; the KV length is restored afterwards and that slot is
// beyond it, so later decoding is unaffected.
// ---------------------------------------------------------------------------
extern "C" int qasr_hip_decoder_profile(qasr_decoder *d, int32_t n_steps, float *us_per_launch,
                                        double *bytes_per_launch, int32_t *launches_per_step) {
    if (!d) return qasr_fail(QASR_ERR_INVALID, "decoder is null");
    CHECK_H(d->h);
    if (n_steps <= 0 || !us_per_launch) return qasr_fail(QASR_ERR_INVALID, "decoder_profile: bad arguments");
    if (d->len + n_steps > d->max_seq) return qasr_fail(QASR_ERR_INVALID, "decoder_profile: KV cache capacity exceeded");
    const qasr_dec_config &c = d->c;
    hipStream_t st = d->h->stream;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    HIPCHK(hipEventCreate(&e0));
    HIPCHK(hipEventCreate(&e1));
    const int lm_reps = (int)std::min<int64_t>(c.n_layers, d->max_seq);
    // with the fused qkv + attention launch, kind 0 is that launch and kind 1
    // launches nothing (the split count and partition of the first step's
    // bucket decide, as in decoder_enqueue_step)
    auto fused_at = [d, &c](int64_t len) {
        const int64_t cap = decoder_ctx_cap(d, len + 1);
        const int ns = d->n_split > 0 ? d->n_split : attn_splits_auto(c, cap);
        const int gpb = (int)((((cap + 7) / 8) + ns - 1) / ns);
        int qr = 1;
        while (qr < 8 && (int64_t)qr * 1024 < (int64_t)(c.n_heads + 2 * c.n_kv_heads) * c.head_dim) qr *= 2;
        return fused_qkv_attn(d, d->attn_step && attn_step_gpw(gpb) > 0, qr);
    };
    bool fused = fused_at(d->len), any_fused = false;
    double tot[QASR_PROFILE_KINDS] = {};
    int cnt[QASR_PROFILE_KINDS] = {};
    const int64_t len0 = d->len;
    int rc = QASR_OK;
    int32_t tok = 0;
    for (int s = 0; s < n_steps && rc == QASR_OK; s++) {
        fused = fused_at(d->len);
        any_fused = any_fused || fused;
        if ((rc = set_state(d, tok)) != QASR_OK) break;
        if ((rc = decoder_enqueue_step(d, true)) != QASR_OK) break;
        HIPCHK(hipStreamSynchronize(st));
        int32_t next[4];
        HIPCHK(hipMemcpy(next, d->state, sizeof(next), hipMemcpyDeviceToHost));
        for (int k = 0; k < QASR_PROFILE_KINDS && rc == QASR_OK; k++) {
            if ((rc = set_state(d, tok)) != QASR_OK) break;
            LAUNCHCHK(launch_delay(400, st), "profile delay");
            HIPCHK(hipEventRecord(e0, st));
            const int reps = k == 5 || k == 6 ? lm_reps : 1;
            for (int r = 0; r < reps && rc == QASR_OK; r++) rc = decoder_enqueue_step(d, true, k);
            HIPCHK(hipEventRecord(e1, st));
            // the fused qkv + attention launches above used this step's tags:
            // advance the epoch so the next real step does not match them
            if (k == 0 && fused) LAUNCHCHK(launch_epoch_advance(d->state + 4, st), "profile epoch");
            HIPCHK(hipEventSynchronize(e1));
            float ms = 0.0f;
            HIPCHK(hipEventElapsedTime(&ms, e0, e1));
            tot[k] += ms * 1000.0;
            if (!(k == 1 && fused)) cnt[k] += k == 5 || k == 6 ? lm_reps : c.n_layers;
        }
        tok = next[0];
        d->len += 1;
    }
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    const double Lavg = (double)len0 + 0.5 * (n_steps - 1) + 1.0;   // context length seen by the attention
    d->len = len0;
    if (rc != QASR_OK) return rc;
    TRY(decoder_fault_check(d));
    const double H = c.hidden, qd = (double)c.n_heads * c.head_dim, kvd = (double)c.n_kv_heads * c.head_dim;
    const double I = c.intermediate, V = (double)d->lm_i8_rows, esz = d->kv_bf16 ? 2 : 4;
    // algorithmic bytes: int8 weights N*K + scales 4N + activation 4K + output 4N (+4N read for += )
    const double nqkv = qd + 2 * kvd;
    const double bytes[QASR_PROFILE_KINDS] = {
        nqkv * H + 4 * nqkv + 4 * H + 4 * nqkv,
        2.0 * kvd * Lavg * esz + 4 * nqkv + 4 * qd + 2 * kvd * esz,
        H * qd + 4 * H + 4 * qd + 8 * H,
        2 * I * H + 8 * I + 4 * H + 4 * I,
        H * I + 4 * H + 4 * I + 8 * H,
        V * H + 4 * V + 4 * H,
        8.0 * argmax_blocks(d->lm_i8_rows),
        nqkv * H + 4 * nqkv + 4 * H + 4 * nqkv};
    for (int k = 0; k < QASR_PROFILE_KINDS; k++) {
        us_per_launch[k] = cnt[k] ? (float)(tot[k] / cnt[k]) : 0.0f;
        if (bytes_per_launch)
            bytes_per_launch[k] = any_fused && k == 0 ? bytes[0] + bytes[1] : (any_fused && k == 1 ? 0.0 : bytes[k]);
        if (launches_per_step)
            launches_per_step[k] = k == 7 ? 0 : (k >= 5 ? 1 : (any_fused && k == 1 ? 0 : c.n_layers));
    }
    return QASR_OK;
}

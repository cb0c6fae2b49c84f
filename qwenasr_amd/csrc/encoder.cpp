// Audio front end on the device: mel spectrogram (audio.rs:273-372), the audio
// encoder (encoder.rs:186-358) and the offline driver with a forced decode
// length (transcribe.rs:63-247).
#include <cmath>
#include <cstring>
#include <vector>

#include "decoder.h"
#include "encoder.h"
#include "upload.h"

using namespace qasr;

#define TRY(x)                  \
    do {                        \
        int rc_ = (x);          \
        if (rc_ != QASR_OK) {   \
            return rc_;         \
        }                       \
    } while (0)

struct EncLayerDev {
    uint16_t *wqkv = nullptr, *wo = nullptr, *fc1 = nullptr, *fc2 = nullptr;
    float *bqkv = nullptr, *bo = nullptr, *b1 = nullptr, *b2 = nullptr;
    float *ln1_w = nullptr, *ln1_b = nullptr, *ln2_w = nullptr, *ln2_b = nullptr;
};

struct qasr_encoder {
    qasr_hip *h = nullptr;
    qasr_enc_config c{};
    uint16_t *conv1_w = nullptr, *conv2_w = nullptr, *conv3_w = nullptr, *conv_out_w = nullptr;
    // channels-last conv stem (conv_hidden % 32 == 0): conv2 / conv3 / conv_out
    // weights hold K in (tap, channel) order for the implicit-im2col GEMM
    bool stem_nhwc = false;
    float *conv1_b = nullptr, *conv2_b = nullptr, *conv3_b = nullptr;
    std::vector<EncLayerDev> L;
    float *ln_post_w = nullptr, *ln_post_b = nullptr;
    uint16_t *proj1_w = nullptr, *proj2_w = nullptr;
    float *proj1_b = nullptr, *proj2_b = nullptr;
    float *pe = nullptr;                        // sinusoidal PE [tokens_per_chunk][d_model]
    int tokens_per_chunk = 0;
    // mel tables
    float *window = nullptr, *dft_cos = nullptr, *dft_sin = nullptr, *filters = nullptr;
    // scratch (grown on demand)
    size_t scratch_bytes = 0;
    char *scratch = nullptr;
    // per-call buffers of qasr_hip_mel / encoder_forward / transcribe_forced,
    // kept between calls
    DevBuf audio, mel, melsc, enc_out, embeds, toks;
    hipEvent_t ev[5] = {};
    std::vector<void *> allocs;
};

template <typename T>
static int ealloc(qasr_encoder *e, T **p, size_t count) {
    void *v = nullptr;
    if (hipMalloc(&v, count * sizeof(T) + 256) != hipSuccess)
        return qasr_fail(QASR_ERR_NOMEM, "encoder: device allocation failed");
    e->allocs.push_back(v);
    *p = reinterpret_cast<T *>(v);
    return QASR_OK;
}

template <typename T>
static int eupload(qasr_encoder *e, T **p, const T *host, size_t count) {
    TRY(ealloc(e, p, count));
    HIPCHK(hipMemcpyAsync(*p, host, count * sizeof(T), hipMemcpyHostToDevice, e->h->stream));
    return QASR_OK;
}

static int conv_len(int n) { return (n + 2 - 3) / 2 + 1; }

// ---- mel tables with the reference's f32 formulas and the host libm ---------
static float hz_to_mel(float f) {                       // audio.rs:202-212
    const float logstep = 27.0f / logf(6.4f);
    const float mels = 3.0f * f / 200.0f;
    return f >= 1000.0f ? 15.0f + logf(f / 1000.0f) * logstep : mels;
}
static float mel_to_hz(float m) {                       // audio.rs:214-223
    const float logstep = logf(6.4f) / 27.0f;
    return m >= 15.0f ? 1000.0f * expf(logstep * (m - 15.0f)) : 200.0f * m / 3.0f;
}

static void mel_tables(std::vector<float> &win, std::vector<float> &ct, std::vector<float> &sn,
                       std::vector<float> &filt) {
    const float PI = 3.14159265358979323846264338327950288f;
    win.resize(400);
    for (int i = 0; i < 400; i++) win[i] = 0.5f * (1.0f - cosf(2.0f * PI * (float)i / 400.0f));
    ct.resize(201 * 400);
    sn.resize(201 * 400);
    for (int k = 0; k < 201; k++)
        for (int n = 0; n < 400; n++) {
            const float a = 2.0f * PI * (float)k * (float)n / 400.0f;
            ct[k * 400 + n] = cosf(a);
            sn[k * 400 + n] = sinf(a);
        }
    float fft[201], ff[130], fd[129];                    // audio.rs:225-262
    for (int i = 0; i < 201; i++) fft[i] = (float)i * (16000.0f / 2.0f) / 200.0f;
    const float mmin = hz_to_mel(0.0f), mmax = hz_to_mel(8000.0f);
    for (int i = 0; i < 130; i++) ff[i] = mel_to_hz(mmin + (mmax - mmin) * (float)i / 129.0f);
    for (int i = 0; i < 129; i++) {
        fd[i] = ff[i + 1] - ff[i];
        if (fd[i] == 0.0f) fd[i] = 1e-6f;
    }
    filt.assign(128 * 201, 0.0f);
    for (int m = 0; m < 128; m++) {
        const float enorm = 2.0f / (ff[m + 2] - ff[m]);
        for (int f = 0; f < 201; f++) {
            const float down = (fft[f] - ff[m]) / fd[m];
            const float up = (ff[m + 2] - fft[f]) / fd[m + 1];
            filt[m * 201 + f] = fmaxf(fminf(down, up), 0.0f) * enorm;
        }
    }
}

// a weight matrix through the pinned staging ring
template <typename T>
static int eupload_big(qasr_encoder *e, Stager &stg, T **p, const T *host, size_t count) {
    TRY(ealloc(e, p, count));
    return stg.upload(*p, host, count * sizeof(T));
}

static int encoder_build(qasr_encoder *e, const qasr_enc_weights *w) {
    const qasr_enc_config &c = e->c;
    const int64_t D = c.d_model, F = c.ffn_dim, C = c.conv_hidden, O = c.output_dim;
    const int h3 = conv_len(conv_len(conv_len(128)));
    Stager stg(e->h->stream);
    TRY(stg.init());
    TRY(eupload_big(e, stg, &e->conv1_w, w->conv1_w, C * 9));
    e->stem_nhwc = C % 32 == 0;
    if (e->stem_nhwc) {
        // each matrix staged as the reference holds it ([out][channel][tap]),
        // then reordered on the device to [out][tap][channel]; the staging
        // buffer is reused in stream order and freed once the stream drains
        uint16_t *raw = nullptr;
        const size_t raw_n = (size_t)std::max(C * C * 9, D * C * h3);
        if (hipMalloc(&raw, raw_n * sizeof(uint16_t)) != hipSuccess)
            return qasr_fail(QASR_ERR_NOMEM, "encoder: device allocation failed");
        const struct { uint16_t **dst; const uint16_t *src; int64_t o, t; } mats[3] = {
            {&e->conv2_w, w->conv2_w, C, 9}, {&e->conv3_w, w->conv3_w, C, 9}, {&e->conv_out_w, w->conv_out_w, D, h3}};
        int rc = QASR_OK;
        for (const auto &m : mats) {
            if (rc == QASR_OK) rc = ealloc(e, m.dst, (size_t)(m.o * C * m.t));
            if (rc == QASR_OK) rc = stg.upload(raw, m.src, sizeof(uint16_t) * m.o * C * m.t);
            if (rc == QASR_OK && launch_taps_last(*m.dst, raw, (int)m.o, (int)C, (int)m.t, e->h->stream) != hipSuccess)
                rc = qasr_fail(QASR_ERR_HIP, "encoder: weight reorder failed");
        }
        if (rc == QASR_OK) rc = stg.finish();
        if (rc == QASR_OK && hipStreamSynchronize(e->h->stream) != hipSuccess)
            rc = qasr_fail(QASR_ERR_HIP, "encoder: weight reorder failed");
        (void)hipFree(raw);
        if (rc != QASR_OK) return rc;
    } else {
        TRY(eupload_big(e, stg, &e->conv2_w, w->conv2_w, C * C * 9));
        TRY(eupload_big(e, stg, &e->conv3_w, w->conv3_w, C * C * 9));
        TRY(eupload_big(e, stg, &e->conv_out_w, w->conv_out_w, D * C * h3));
    }
    TRY(eupload(e, &e->conv1_b, w->conv1_b, C));
    TRY(eupload(e, &e->conv2_b, w->conv2_b, C));
    TRY(eupload(e, &e->conv3_b, w->conv3_b, C));
    e->L.resize(c.n_layers);
    for (int l = 0; l < c.n_layers; l++) {
        const qasr_enc_layer &s = w->layers[l];
        EncLayerDev &L = e->L[l];
        TRY(ealloc(e, &L.wqkv, 3 * D * D));
        TRY(stg.upload(L.wqkv, s.wq, 2 * D * D));
        TRY(stg.upload(L.wqkv + D * D, s.wk, 2 * D * D));
        TRY(stg.upload(L.wqkv + 2 * D * D, s.wv, 2 * D * D));
        TRY(ealloc(e, &L.bqkv, 3 * D));
        HIPCHK(hipMemcpyAsync(L.bqkv, s.bq, D * 4, hipMemcpyHostToDevice, e->h->stream));
        HIPCHK(hipMemcpyAsync(L.bqkv + D, s.bk, D * 4, hipMemcpyHostToDevice, e->h->stream));
        HIPCHK(hipMemcpyAsync(L.bqkv + 2 * D, s.bv, D * 4, hipMemcpyHostToDevice, e->h->stream));
        TRY(eupload_big(e, stg, &L.wo, s.wo, D * D));
        TRY(eupload(e, &L.bo, s.bo, D));
        TRY(eupload_big(e, stg, &L.fc1, s.fc1, F * D));
        TRY(eupload(e, &L.b1, s.b1, F));
        TRY(eupload_big(e, stg, &L.fc2, s.fc2, D * F));
        TRY(eupload(e, &L.b2, s.b2, D));
        TRY(eupload(e, &L.ln1_w, s.ln1_w, D));
        TRY(eupload(e, &L.ln1_b, s.ln1_b, D));
        TRY(eupload(e, &L.ln2_w, s.ln2_w, D));
        TRY(eupload(e, &L.ln2_b, s.ln2_b, D));
    }
    TRY(eupload(e, &e->ln_post_w, w->ln_post_w, D));
    TRY(eupload(e, &e->ln_post_b, w->ln_post_b, D));
    TRY(eupload_big(e, stg, &e->proj1_w, w->proj1_w, D * D));
    TRY(eupload(e, &e->proj1_b, w->proj1_b, D));
    TRY(eupload_big(e, stg, &e->proj2_w, w->proj2_w, O * D));
    TRY(eupload(e, &e->proj2_b, w->proj2_b, O));
    // per-chunk sinusoidal PE (sinusoidal_pe, kernels/mod.rs:1704-1717)
    e->tokens_per_chunk = conv_len(conv_len(conv_len(c.chunk_size)));
    {
        const int64_t n_pos = e->tokens_per_chunk, half = D / 2;
        std::vector<float> pe(n_pos * D);
        const float lt = logf(10000.0f) / (float)(half - 1);
        for (int64_t p = 0; p < n_pos; p++)
            for (int64_t d = 0; d < half; d++) {
                const float inv_ts = expf(-(float)d * lt);
                const float a = (float)p * inv_ts;
                pe[p * D + d] = sinf(a);
                pe[p * D + half + d] = cosf(a);
            }
        TRY(eupload(e, &e->pe, pe.data(), pe.size()));
        std::vector<float> win, ct, sn, filt;
        mel_tables(win, ct, sn, filt);
        TRY(eupload(e, &e->window, win.data(), win.size()));
        TRY(eupload(e, &e->dft_cos, ct.data(), ct.size()));
        TRY(eupload(e, &e->dft_sin, sn.data(), sn.size()));
        TRY(eupload(e, &e->filters, filt.data(), filt.size()));
        HIPCHK(hipStreamSynchronize(e->h->stream));
    }
    TRY(stg.finish());
    return QASR_OK;
}

extern "C" int qasr_hip_encoder_load(qasr_hip *h, const qasr_enc_config *cfg, const qasr_enc_weights *w,
                                     qasr_encoder **out) {
    CHECK_H(h);
    if (!cfg || !w || !out || !w->layers) return qasr_fail(QASR_ERR_INVALID, "encoder_load: null argument");
    *out = nullptr;
    const qasr_enc_config c = *cfg;
    if (c.n_layers <= 0 || c.d_model <= 0 || c.d_model % 16 != 0 || c.d_model > 4096 || c.head_dim != 64 ||
        c.n_heads * c.head_dim != c.d_model || c.ffn_dim <= 0 || c.output_dim <= 0 || c.chunk_size <= 0 ||
        c.n_window_infer < c.chunk_size || c.conv_hidden <= 0)
        return qasr_fail(QASR_ERR_INVALID, "encoder_load: unsupported config (head_dim 64, d_model % 16 == 0)");
    qasr_encoder *e = new qasr_encoder();
    e->h = h;
    e->c = c;
    int rc = encoder_build(e, w);
    if (rc != QASR_OK) {
        qasr_hip_encoder_free(e);
        return rc;
    }
    *out = e;
    return QASR_OK;
}

extern "C" void qasr_hip_encoder_free(qasr_encoder *e) {
    if (!e) return;
    (void)hipSetDevice(e->h->device);
    (void)hipStreamSynchronize(e->h->stream);
    if (e->scratch) (void)hipFree(e->scratch);
    for (DevBuf *b : {&e->audio, &e->mel, &e->melsc, &e->enc_out, &e->embeds, &e->toks}) dbuf_release(*b);
    for (hipEvent_t v : e->ev)
        if (v) (void)hipEventDestroy(v);
    for (void *p : e->allocs) (void)hipFree(p);
    delete e;
}

static int ensure_scratch(qasr_encoder *e, size_t bytes) {
    if (bytes <= e->scratch_bytes) return QASR_OK;
    HIPCHK(hipStreamSynchronize(e->h->stream));
    if (e->scratch) (void)hipFree(e->scratch);
    e->scratch = nullptr;
    e->scratch_bytes = 0;
    if (hipMalloc((void **)&e->scratch, bytes) != hipSuccess)
        return qasr_fail(QASR_ERR_NOMEM, "encoder: scratch allocation failed");
    e->scratch_bytes = bytes;
    return QASR_OK;
}

int64_t encoder_tokens(const qasr_encoder *e, int64_t frames) {
    int64_t tot = 0;
    for (int64_t s = 0; s < frames; s += e->c.chunk_size) {
        const int w = (int)std::min<int64_t>(e->c.chunk_size, frames - s);
        tot += conv_len(conv_len(conv_len(w)));
    }
    return tot;
}

static int egemm(qasr_encoder *e, const float *A, int64_t lda, const uint16_t *B, int64_t ldb, float *C,
                 int64_t ldc, int M, int N, int K, const float *bias, int epi, int64_t gelu_n = 0,
                 int gelu_rows = 0) {
    GemmArgs g{};
    g.M = M; g.N = N; g.K = K;
    g.A = A; g.lda = lda; g.B = B; g.ldb = ldb; g.C = C; g.ldc = ldc; g.bias = bias;
    g.gelu_n = gelu_n; g.gelu_rows = gelu_rows;
    g.ws = reinterpret_cast<float *>(e->h->scratch); g.ws_bytes = QASR_SCRATCH_BYTES;
    // K split chosen by the shape alone: a row's bits do not depend on how many
    // rows (sequences) share the call
    g.split_by_shape = 1;
    LAUNCHCHK(launch_gemm(g, A_F32_SPLIT, B_BF16, epi, e->h->stream), "encoder gemm");
    return QASR_OK;
}

// implicit-im2col GEMM of a channels-last convolution (K in (tap, channel)
// order): out[(chunk, oy, ox)][n] with the reference's GELU index rule
static int econv(qasr_encoder *e, const float *in, int n_chunks, int hin, int win, int cin, int hout, int wout,
                 int kh, int kw, int sy, int sx, int py, int px, const uint16_t *w, int N, const float *bias,
                 float *out, int64_t ldc, int epi) {
    GemmArgs g{};
    g.M = n_chunks * hout * wout; g.N = N; g.K = cin * kh * kw;
    g.A = in; g.lda = cin; g.B = w; g.ldb = g.K; g.C = out; g.ldc = ldc; g.bias = bias;
    g.gelu_n = (int64_t)N * hout * wout; g.gelu_rows = hout * wout;
    g.conv_hin = hin; g.conv_win = win; g.conv_c = cin; g.conv_hout = hout; g.conv_wout = wout;
    g.conv_kh = kh; g.conv_kw = kw; g.conv_sy = sy; g.conv_sx = sx; g.conv_py = py; g.conv_px = px;
    LAUNCHCHK(launch_gemm(g, A_CONV, B_BF16, epi, e->h->stream), "encoder conv gemm");
    return QASR_OK;
}

// conv stem for n_chunks chunks of cw frames starting at frame f0; writes the
// projected + PE rows to x (encoder.rs:226-287).  With stem_nhwc the
// activations stay channels-last, [chunk][h][w][C]: conv2 and conv3 are
// implicit-im2col GEMMs over them (3 x 3 taps, stride 2, padding 1) and the
// output projection one over conv3's (all h3 rows x 1 column: the
// reference's [chunk][w3][C h3] rows with K in (row, channel) order); GELU
// picks each element's path by its index in the reference's [C][h][w] chunk
// tensor.  Otherwise the reference's layouts through im2col.
static int conv_stem(qasr_encoder *e, const float *mel, int64_t frames, int64_t f0, int n_chunks, int cw,
                     float *x, char *buf) {
    hipStream_t st = e->h->stream;
    const int C = e->c.conv_hidden, D = e->c.d_model;
    const int h1 = conv_len(128), w1 = conv_len(cw), h2 = conv_len(h1), w2 = conv_len(w1);
    const int h3 = conv_len(h2), w3 = conv_len(w2);
    const bool direct1 = 130 * (cw + 2) <= 13312 && C >= 16;
    if (e->stem_nhwc) {
        float *a1 = reinterpret_cast<float *>(buf);
        float *a2 = a1 + (int64_t)n_chunks * C * h1 * w1;
        float *a3 = a2 + (int64_t)n_chunks * C * h2 * w2;
        float *cols = a3 + (int64_t)n_chunks * C * h3 * w3;           // conv1's patches (no direct form)
        if (direct1) {
            LAUNCHCHK(launch_conv1_direct(a1, mel + f0, n_chunks, e->c.chunk_size, frames, 128, cw, e->conv1_w,
                                          e->conv1_b, C, h1, w1, true, st),
                      "conv1");
        } else {
            LAUNCHCHK(launch_im2col3x3s2(cols, mel + f0, n_chunks, 1, 128, cw, e->c.chunk_size, 0, frames, h1, w1,
                                         st),
                      "im2col1");
            TRY(egemm(e, cols, 9, e->conv1_w, 9, a1, C, n_chunks * h1 * w1, C, 9, e->conv1_b, EPI_GELU | EPI_CHW,
                      (int64_t)C * h1 * w1, h1 * w1));
        }
        TRY(econv(e, a1, n_chunks, h1, w1, C, h2, w2, 3, 3, 2, 2, 1, 1, e->conv2_w, C, e->conv2_b, a2, C,
                  EPI_GELU | EPI_CHW));
        TRY(econv(e, a2, n_chunks, h2, w2, C, h3, w3, 3, 3, 2, 2, 1, 1, e->conv3_w, C, e->conv3_b, a3, C,
                  EPI_GELU | EPI_CHW));
        TRY(econv(e, a3, n_chunks, h3, w3, C, 1, w3, h3, 1, 1, 1, 0, 0, e->conv_out_w, D, nullptr, x, D, EPI_NONE));
        LAUNCHCHK(launch_add_periodic(x, e->pe, (int64_t)n_chunks * w3, D, w3, st), "pe add");
        return QASR_OK;
    }
    float *cols = reinterpret_cast<float *>(buf);
    float *a1 = cols + (int64_t)n_chunks * h2 * w2 * C * 9 + (int64_t)n_chunks * h1 * w1 * 9;
    float *a2 = a1 + (int64_t)n_chunks * C * h1 * w1;
    float *a3 = a2 + (int64_t)n_chunks * C * h2 * w2;
    float *rsh = a3 + (int64_t)n_chunks * C * h3 * w3;
    // conv1: input (chunk c, ic 0, ih, iw) = mel[ih * frames + f0 + c * chunk + iw]; computed
    // directly (9 taps) when the chunk's input plane fits the kernel's LDS, else as a GEMM
    if (direct1) {
        LAUNCHCHK(launch_conv1_direct(a1, mel + f0, n_chunks, e->c.chunk_size, frames, 128, cw, e->conv1_w,
                                      e->conv1_b, C, h1, w1, false, st),
                  "conv1");
    } else {
        LAUNCHCHK(launch_im2col3x3s2(cols, mel + f0, n_chunks, 1, 128, cw, e->c.chunk_size, 0, frames, h1, w1, st),
                  "im2col1");
        TRY(egemm(e, cols, 9, e->conv1_w, 9, a1, 0, n_chunks * h1 * w1, C, 9, e->conv1_b, EPI_TRANS | EPI_GELU,
                  (int64_t)C * h1 * w1, h1 * w1));
    }
    LAUNCHCHK(launch_im2col3x3s2(cols, a1, n_chunks, C, h1, w1, (int64_t)C * h1 * w1, (int64_t)h1 * w1, w1, h2, w2,
                                 st),
              "im2col2");
    TRY(egemm(e, cols, (int64_t)C * 9, e->conv2_w, (int64_t)C * 9, a2, 0, n_chunks * h2 * w2, C, C * 9, e->conv2_b,
              EPI_TRANS | EPI_GELU, (int64_t)C * h2 * w2, h2 * w2));
    LAUNCHCHK(launch_im2col3x3s2(cols, a2, n_chunks, C, h2, w2, (int64_t)C * h2 * w2, (int64_t)h2 * w2, w2, h3, w3,
                                 st),
              "im2col3");
    TRY(egemm(e, cols, (int64_t)C * 9, e->conv3_w, (int64_t)C * 9, a3, 0, n_chunks * h3 * w3, C, C * 9, e->conv3_b,
              EPI_TRANS | EPI_GELU, (int64_t)C * h3 * w3, h3 * w3));
    LAUNCHCHK(launch_conv_reshape(rsh, a3, n_chunks, C, h3, w3, st), "conv reshape");
    TRY(egemm(e, rsh, (int64_t)C * h3, e->conv_out_w, (int64_t)C * h3, x, D, n_chunks * w3, D, C * h3, nullptr,
              EPI_NONE));
    LAUNCHCHK(launch_add_periodic(x, e->pe, (int64_t)n_chunks * w3, D, w3, st), "pe add");
    return QASR_OK;
}

static size_t stem_bytes(const qasr_encoder *e, int n_chunks, int cw) {
    const int C = e->c.conv_hidden;
    const int h1 = conv_len(128), w1 = conv_len(cw), h2 = conv_len(h1), w2 = conv_len(w1);
    const int h3 = conv_len(h2), w3 = conv_len(w2);
    const int64_t acts = (int64_t)n_chunks * C * (h1 * w1 + h2 * w2 + h3 * w3);
    const int64_t f = e->stem_nhwc ? acts + (int64_t)n_chunks * h1 * w1 * 9
                                   : (int64_t)n_chunks * h2 * w2 * C * 9 + (int64_t)n_chunks * h1 * w1 * 9 + acts +
                                         (int64_t)n_chunks * w3 * C * h3;
    return sizeof(float) * f + 1024;
}

// Encoder::forward (encoder.rs:186-358) of n sequences in one pass, each the
// forward of its own device mel [128][frames[j]]: the conv stem per sequence,
// then every layer over the rows of all of them.  Sequence j's rows start at
// row P_j, a multiple of 32 (n > 1; the rows between sequences are zeros and
// not attended): the attention windows restart at each sequence and no block
// of the row attention straddles two, and the GEMMs (K split by shape),
// norms and GELU are row-wise, so each sequence's rows have the bits of a
// call of its own.  (The GELU's vector/scalar split depends on the buffer
// length only through tails that d_model and ffn_dim multiples of 128 never
// have; other widths take one call per sequence.)  Sequence j's output rows
// go to out + (T_0 + ... + T_{j-1}) * output_dim, tokens[j] = T_j.
int encoder_forward_multi(qasr_encoder *e, int n, const float *const *mels, const int64_t *frames, float *out,
                          int64_t *tokens) {
    const qasr_enc_config &c = e->c;
    hipStream_t st = e->h->stream;
    const int D = c.d_model, F = c.ffn_dim, O = c.output_dim;
    if (n < 1 || n > QASR_ATTN_MAX_SEG) return qasr_fail(QASR_ERR_INVALID, "encoder: 1 to 64 sequences per call");
    if (n > 1 && (D % 128 != 0 || F % 128 != 0)) {
        int64_t off = 0;
        for (int j = 0; j < n; j++) {
            TRY(encoder_forward_multi(e, 1, mels + j, frames + j, out + off * O, tokens + j));
            off += tokens[j];
        }
        return QASR_OK;
    }
    std::vector<int64_t> T(n), P(n + 1, 0);
    size_t stem = 0;
    for (int j = 0; j < n; j++) {
        T[j] = encoder_tokens(e, frames[j]);
        P[j + 1] = P[j] + (n > 1 ? (T[j] + 31) / 32 * 32 : T[j]);
        const int64_t n_full = frames[j] / c.chunk_size;
        const int tail = (int)(frames[j] % c.chunk_size);
        stem = std::max({stem, stem_bytes(e, (int)std::max<int64_t>(n_full, 1), c.chunk_size),
                         tail ? stem_bytes(e, 1, tail) : (size_t)0});
    }
    const int64_t Mt = P[n];
    const size_t tf = sizeof(float) * (size_t)Mt;
    const size_t layer_bytes = tf * (D + 3 * D + D + F) + 4096;
    const size_t x_bytes = (tf * D + 255) / 256 * 256;
    TRY(ensure_scratch(e, x_bytes + std::max(stem, layer_bytes)));
    float *x = reinterpret_cast<float *>(e->scratch);     // residual stream [Mt][D]
    char *buf = e->scratch + x_bytes;
    if (n > 1) HIPCHK(hipMemsetAsync(x, 0, sizeof(float) * Mt * D, st));   // the rows between sequences
    for (int j = 0; j < n; j++) {
        const int64_t n_full = frames[j] / c.chunk_size;
        const int tail = (int)(frames[j] % c.chunk_size);
        float *xj = x + P[j] * D;
        if (n_full > 0) TRY(conv_stem(e, mels[j], frames[j], 0, (int)n_full, c.chunk_size, xj, buf));
        if (tail)
            TRY(conv_stem(e, mels[j], frames[j], n_full * c.chunk_size, 1, tail, xj + n_full * e->tokens_per_chunk * D,
                          buf));
    }
    float *xn = reinterpret_cast<float *>(buf);
    float *qkv = xn + Mt * D;
    float *att = qkv + Mt * 3 * D;
    float *mid = att + Mt * D;
    const int wsz = e->tokens_per_chunk * (c.n_window_infer / c.chunk_size);
    const int M = (int)Mt;
    for (int l = 0; l < c.n_layers; l++) {
        const EncLayerDev &L = e->L[l];
        LAUNCHCHK(launch_layer_norm_rows(xn, x, L.ln1_w, L.ln1_b, Mt, D, 1e-5f, st), "enc ln1");
        TRY(egemm(e, xn, D, L.wqkv, D, qkv, 3 * D, M, 3 * D, D, L.bqkv, EPI_NONE));
        AttnRowsArgs a{};
        a.q = qkv; a.q_rs = 3 * D;
        a.k = qkv + D; a.v = qkv + 2 * D; a.k_hs = c.head_dim; a.k_rs = 3 * D;
        a.out = att; a.o_rs = D;
        a.n_q = M; a.n_k = M; a.G = 1; a.q_offset = 0; a.window = wsz;
        a.scale = 1.0f / sqrtf((float)c.head_dim);
        if (n > 1) {
            a.n_seg = n;
            for (int j = 0; j < n; j++) {
                a.seg_lo[j] = (int)P[j];
                a.seg_hi[j] = (int)(P[j] + T[j]);
            }
        }
        LAUNCHCHK(launch_attn_rows(a, c.n_heads, c.head_dim, st), "enc attention");
        TRY(egemm(e, att, D, L.wo, D, x, D, M, D, D, L.bo, EPI_ACCUM));
        LAUNCHCHK(launch_layer_norm_rows(xn, x, L.ln2_w, L.ln2_b, Mt, D, 1e-5f, st), "enc ln2");
        TRY(egemm(e, xn, D, L.fc1, D, mid, F, M, F, D, L.b1, EPI_GELU, (int64_t)Mt * F));
        TRY(egemm(e, mid, F, L.fc2, F, x, D, M, D, F, L.b2, EPI_ACCUM));
    }
    LAUNCHCHK(launch_layer_norm_rows(xn, x, e->ln_post_w, e->ln_post_b, Mt, D, 1e-5f, st), "enc ln_post");
    TRY(egemm(e, xn, D, e->proj1_w, D, att, D, M, D, D, e->proj1_b, EPI_GELU, (int64_t)Mt * D));
    int64_t off = 0;
    for (int j = 0; j < n; j++) {
        TRY(egemm(e, att + P[j] * D, D, e->proj2_w, D, out + off * O, O, (int)T[j], O, D, e->proj2_b, EPI_NONE));
        tokens[j] = T[j];
        off += T[j];
    }
    return QASR_OK;
}

// Encoder::forward on a device mel [128][frames]; out [tokens][output_dim]
int encoder_forward_dev(qasr_encoder *e, const float *mel, int64_t frames, float *out, int64_t *n_tok) {
    int64_t t = 0;
    TRY(encoder_forward_multi(e, 1, &mel, &frames, out, &t));
    if (n_tok) *n_tok = t;
    return QASR_OK;
}

int64_t encoder_output_dim(const qasr_encoder *e) { return e->c.output_dim; }
qasr_hip *encoder_handle(const qasr_encoder *e) { return e->h; }

int64_t mel_frames_for(int64_t n) {
    const int64_t padded = n + 400;
    if (padded < 400) return 0;
    return (padded - 400) / 160;
}

// mel_spectrogram on device samples; mel [128][frames]
int mel_dev(qasr_encoder *e, const float *x, int64_t ns, float *mel, float *scratch) {
    hipStream_t st = e->h->stream;
    const int nf = (int)mel_frames_for(ns);
    float *fr = scratch, *re = fr + (int64_t)nf * 400, *im = re + (int64_t)nf * 201;
    float *pT = im + (int64_t)nf * 201, *bmax = pT + (int64_t)nf * 201;
    LAUNCHCHK(launch_mel_frames(fr, x, ns, e->window, nf, st), "mel frames");
    GemmArgs g{};
    g.M = 201; g.N = nf; g.K = 400;
    g.A = e->dft_cos; g.lda = 400; g.B = fr; g.ldb = 400; g.C = re; g.ldc = nf;
    LAUNCHCHK(launch_gemm_f32(g, st), "mel dft");
    g.A = e->dft_sin; g.C = im;
    LAUNCHCHK(launch_gemm_f32(g, st), "mel dft");
    LAUNCHCHK(launch_mel_power(pT, re, im, nf, st), "mel power");
    g.M = 128; g.N = nf; g.K = 201;
    g.A = e->filters; g.lda = 201; g.B = pT; g.ldb = 201; g.C = mel; g.ldc = nf;
    LAUNCHCHK(launch_gemm_f32(g, st), "mel filterbank");
    LAUNCHCHK(launch_mel_log_norm(mel, (int64_t)128 * nf, bmax, st), "mel log");
    return QASR_OK;
}

size_t mel_scratch_floats(int64_t nf) { return (size_t)nf * (400 + 3 * 201) + (size_t)(128 * nf / 256 + 2); }

// mel_spectrogram of n device signals at once: the frames, the two DFT GEMMs,
// the power and the filterbank GEMM over all their frames together (each f32
// GEMM element is a sum over K in a fixed order, whatever the frame count),
// then each mel copied out to mel[j] [128][frames_j] and log-normalised with
// its own maximum.  scratch: mel_multi_scratch_floats(total frames, largest).
int mel_dev_multi(qasr_encoder *e, int n, const float *const *x, const int64_t *ns, float *const *mel, float *scratch) {
    hipStream_t st = e->h->stream;
    int64_t tot = 0;
    for (int j = 0; j < n; j++) tot += mel_frames_for(ns[j]);
    float *fr = scratch, *re = fr + tot * 400, *im = re + tot * 201, *pT = im + tot * 201, *all = pT + tot * 201;
    float *bmax = all + tot * 128;
    int64_t off = 0;
    for (int j = 0; j < n; j++) {
        const int nf = (int)mel_frames_for(ns[j]);
        LAUNCHCHK(launch_mel_frames(fr + off * 400, x[j], ns[j], e->window, nf, st), "mel frames");
        off += nf;
    }
    GemmArgs g{};
    g.M = 201; g.N = (int)tot; g.K = 400;
    g.A = e->dft_cos; g.lda = 400; g.B = fr; g.ldb = 400; g.C = re; g.ldc = tot;
    LAUNCHCHK(launch_gemm_f32(g, st), "mel dft");
    g.A = e->dft_sin; g.C = im;
    LAUNCHCHK(launch_gemm_f32(g, st), "mel dft");
    LAUNCHCHK(launch_mel_power(pT, re, im, (int)tot, st), "mel power");
    g.M = 128; g.N = (int)tot; g.K = 201;
    g.A = e->filters; g.lda = 201; g.B = pT; g.ldb = 201; g.C = all; g.ldc = tot;
    LAUNCHCHK(launch_gemm_f32(g, st), "mel filterbank");
    off = 0;
    for (int j = 0; j < n; j++) {
        const int64_t nf = mel_frames_for(ns[j]);
        HIPCHK(hipMemcpy2DAsync(mel[j], sizeof(float) * nf, all + off, sizeof(float) * tot, sizeof(float) * nf, 128,
                                hipMemcpyDeviceToDevice, st));
        LAUNCHCHK(launch_mel_log_norm(mel[j], 128 * nf, bmax, st), "mel log");
        off += nf;
    }
    return QASR_OK;
}

size_t mel_multi_scratch_floats(int64_t total_frames, int64_t max_frames) {
    return (size_t)total_frames * (400 + 3 * 201 + 128) + (size_t)(128 * max_frames / 256 + 2);
}

extern "C" int qasr_hip_mel(qasr_encoder *e, const float *samples, int64_t n, float *mel_out, int64_t *frames) {
    if (!e) return qasr_fail(QASR_ERR_INVALID, "encoder is null");
    CHECK_H(e->h);
    if (!samples || n <= 0 || !frames) return qasr_fail(QASR_ERR_INVALID, "mel: bad arguments");
    const int64_t nf = mel_frames_for(n);
    if (nf <= 0) return qasr_fail(QASR_ERR_INVALID, "mel: audio too short");
    *frames = nf;
    if (!mel_out) return QASR_OK;
    TRY(dbuf_ensure(e->audio, sizeof(float) * n, e->h->stream));
    TRY(dbuf_ensure(e->mel, sizeof(float) * 128 * nf, e->h->stream));
    TRY(dbuf_ensure(e->melsc, sizeof(float) * mel_scratch_floats(nf), e->h->stream));
    float *dx = e->audio.as<float>(), *dm = e->mel.as<float>(), *sc = e->melsc.as<float>();
    int rc = QASR_OK;
    if (hipMemcpyAsync(dx, samples, sizeof(float) * n, hipMemcpyHostToDevice, e->h->stream) != hipSuccess)
        rc = qasr_fail(QASR_ERR_HIP, "mel: upload failed");
    if (rc == QASR_OK) rc = mel_dev(e, dx, n, dm, sc);
    if (rc == QASR_OK &&
        hipMemcpyAsync(mel_out, dm, sizeof(float) * 128 * nf, hipMemcpyDeviceToHost, e->h->stream) != hipSuccess)
        rc = qasr_fail(QASR_ERR_HIP, "mel: download failed");
    if (hipStreamSynchronize(e->h->stream) != hipSuccess && rc == QASR_OK)
        rc = qasr_fail(QASR_ERR_HIP, "mel: stream failed");
    return rc;
}

// n host mels [128][frames[j]] -> their encoder rows, one after another in
// out (host), tokens[j] each; one encoder pass over all of them
extern "C" int qasr_hip_encoder_forward_batch(qasr_encoder *e, int32_t n, const float *const *mels,
                                              const int64_t *frames, float *out, int64_t *tokens) {
    if (!e) return qasr_fail(QASR_ERR_INVALID, "encoder is null");
    CHECK_H(e->h);
    if (n < 1 || n > QASR_ATTN_MAX_SEG || !mels || !frames || !out || !tokens)
        return qasr_fail(QASR_ERR_INVALID, "encoder_forward_batch: bad arguments");
    int64_t tot_f = 0, tot_t = 0;
    for (int j = 0; j < n; j++) {
        if (!mels[j] || frames[j] <= 0) return qasr_fail(QASR_ERR_INVALID, "encoder_forward_batch: bad sequence");
        tot_f += frames[j];
        tot_t += encoder_tokens(e, frames[j]);
    }
    TRY(dbuf_ensure(e->mel, sizeof(float) * 128 * tot_f, e->h->stream));
    TRY(dbuf_ensure(e->enc_out, sizeof(float) * tot_t * e->c.output_dim, e->h->stream));
    std::vector<const float *> dm(n);
    int rc = QASR_OK;
    int64_t f = 0;
    for (int j = 0; j < n && rc == QASR_OK; j++) {
        dm[j] = e->mel.as<float>() + 128 * f;
        if (hipMemcpyAsync(const_cast<float *>(dm[j]), mels[j], sizeof(float) * 128 * frames[j],
                           hipMemcpyHostToDevice, e->h->stream) != hipSuccess)
            rc = qasr_fail(QASR_ERR_HIP, "encoder_forward_batch: upload failed");
        f += frames[j];
    }
    if (rc == QASR_OK) rc = encoder_forward_multi(e, n, dm.data(), frames, e->enc_out.as<float>(), tokens);
    if (rc == QASR_OK && hipMemcpyAsync(out, e->enc_out.p, sizeof(float) * tot_t * e->c.output_dim,
                                        hipMemcpyDeviceToHost, e->h->stream) != hipSuccess)
        rc = qasr_fail(QASR_ERR_HIP, "encoder_forward_batch: download failed");
    if (hipStreamSynchronize(e->h->stream) != hipSuccess && rc == QASR_OK)
        rc = qasr_fail(QASR_ERR_HIP, "encoder_forward_batch: stream failed");
    return rc;
}

extern "C" int64_t qasr_hip_encoder_tokens(const qasr_encoder *e, int64_t frames) {
    return e ? encoder_tokens(e, frames) : -1;
}

extern "C" int qasr_hip_encoder_forward(qasr_encoder *e, const float *mel, int64_t frames, float *out,
                                        int64_t *n_tokens) {
    if (!e) return qasr_fail(QASR_ERR_INVALID, "encoder is null");
    CHECK_H(e->h);
    if (!mel || frames <= 0 || !out) return qasr_fail(QASR_ERR_INVALID, "encoder_forward: bad arguments");
    const int64_t T = encoder_tokens(e, frames);
    TRY(dbuf_ensure(e->mel, sizeof(float) * 128 * frames, e->h->stream));
    TRY(dbuf_ensure(e->enc_out, sizeof(float) * T * e->c.output_dim, e->h->stream));
    float *dm = e->mel.as<float>(), *dout = e->enc_out.as<float>();
    int rc = QASR_OK;
    if (hipMemcpyAsync(dm, mel, sizeof(float) * 128 * frames, hipMemcpyHostToDevice, e->h->stream) != hipSuccess)
        rc = qasr_fail(QASR_ERR_HIP, "encoder_forward: upload failed");
    if (rc == QASR_OK) rc = encoder_forward_dev(e, dm, frames, dout, n_tokens);
    if (rc == QASR_OK && hipMemcpyAsync(out, dout, sizeof(float) * T * e->c.output_dim, hipMemcpyDeviceToHost,
                                        e->h->stream) != hipSuccess)
        rc = qasr_fail(QASR_ERR_HIP, "encoder_forward: download failed");
    if (hipStreamSynchronize(e->h->stream) != hipSuccess && rc == QASR_OK)
        rc = qasr_fail(QASR_ERR_HIP, "encoder_forward: stream failed");
    return rc;
}

// ---------------------------------------------------------------------------
// offline transcription with a forced number of decode steps
// ---------------------------------------------------------------------------
static const int32_t PREFIX_HEAD[] = {151644, 8948, 198};
static const int32_t PREFIX_TAIL[] = {151645, 198, 151644, 872, 198, 151669};
static const int32_t SUFFIX_BASE[] = {151670, 151645, 198, 151644, 77091, 198};
static const int32_t TOKEN_ASR_TEXT = 151704;

// The id rows of transcribe_segment's prompt (transcribe.rs:97-169): before
// the audio rows PREFIX_HEAD | prompt | PREFIX_TAIL, after them SUFFIX_BASE |
// force | past | <asr_text> (the last two only with past ids).  The ids are
// gathered from the embedding table on the device, so each must index it.
int prompt_id_rows(const qasr_prompt *p, const int32_t *past, int64_t n_past, int32_t vocab,
                   std::vector<int32_t> &head, std::vector<int32_t> &tail) {
    const int64_t np = p ? p->n_prompt : 0, nf = p ? p->n_force : 0;
    if (np < 0 || nf < 0 || n_past < 0 || (np > 0 && !p->prompt) || (nf > 0 && !p->force) || (n_past > 0 && !past))
        return qasr_fail(QASR_ERR_INVALID, "prompt ids: null ids with a nonzero count");
    head.assign(PREFIX_HEAD, PREFIX_HEAD + 3);
    if (np > 0) head.insert(head.end(), p->prompt, p->prompt + np);
    head.insert(head.end(), PREFIX_TAIL, PREFIX_TAIL + 6);
    tail.assign(SUFFIX_BASE, SUFFIX_BASE + 6);
    if (nf > 0) tail.insert(tail.end(), p->force, p->force + nf);
    if (n_past > 0) {
        tail.insert(tail.end(), past, past + n_past);
        tail.push_back(TOKEN_ASR_TEXT);
    }
    for (const auto *v : {&head, &tail})
        for (int32_t t : *v)
            if (t < 0 || t >= vocab) return qasr_fail(QASR_ERR_INVALID, "prompt ids: vocab too small for the prompt (an id outside the vocabulary)");
    return QASR_OK;
}

// mel -> encoder -> prompt rows -> prefill of all but the last row -> the
// first forward from the last row (transcribe.rs:71-183), queued on the
// handle's stream; events ev[0..3] mark mel, encoder, prefill + first token.
// Returns the prompt length in *total.
static int transcribe_begin(qasr_decoder *d, qasr_encoder *e, const float *samples, int64_t n, int64_t steps_max,
                            const qasr_prompt *prompt, const int32_t *past, int64_t n_past, int64_t *total_out) {
    if (!d || !e) return qasr_fail(QASR_ERR_INVALID, "transcribe: null model");
    CHECK_H(d->h);
    if (d->h != e->h) return qasr_fail(QASR_ERR_INVALID, "transcribe: models on different handles");
    if (!samples || n <= 0 || steps_max <= 0) return qasr_fail(QASR_ERR_INVALID, "transcribe: bad arguments");
    if (e->c.output_dim != d->c.hidden) return qasr_fail(QASR_ERR_INVALID, "transcribe: encoder/decoder width mismatch");
    hipStream_t st = d->h->stream;
    const int64_t nf = mel_frames_for(n);
    if (nf <= 0) return qasr_fail(QASR_ERR_INVALID, "transcribe: audio too short");
    const int64_t T = encoder_tokens(e, nf);
    const int H = d->c.hidden;
    std::vector<int32_t> head, tail;
    TRY(prompt_id_rows(prompt, past, n_past, d->c.vocab, head, tail));
    const int n_head = (int)head.size(), n_tail = (int)tail.size();
    const int64_t total = n_head + T + n_tail;
    TRY(decoder_reserve(d, total - 1 + steps_max));
    std::vector<int32_t> toks(head);
    toks.insert(toks.end(), tail.begin(), tail.end());
    TRY(dbuf_ensure(e->audio, sizeof(float) * n, e->h->stream, d->h->stream));
    TRY(dbuf_ensure(e->mel, sizeof(float) * 128 * nf, e->h->stream, d->h->stream));
    TRY(dbuf_ensure(e->melsc, sizeof(float) * mel_scratch_floats(nf), e->h->stream, d->h->stream));
    TRY(dbuf_ensure(e->enc_out, sizeof(float) * T * H, e->h->stream, d->h->stream));
    TRY(dbuf_ensure(e->embeds, sizeof(float) * total * H, e->h->stream, d->h->stream));
    TRY(dbuf_ensure(e->toks, sizeof(int32_t) * toks.size(), e->h->stream, d->h->stream));
    for (hipEvent_t &v : e->ev)
        if (!v) HIPCHK(hipEventCreate(&v));
    float *dx = e->audio.as<float>(), *dmel = e->mel.as<float>(), *msc = e->melsc.as<float>();
    float *enc = e->enc_out.as<float>(), *emb = e->embeds.as<float>();
    int *dtok = e->toks.as<int>();
    hipEvent_t *ev = e->ev;
    HIPCHK(hipMemcpyAsync(dx, samples, sizeof(float) * n, hipMemcpyHostToDevice, st));
    HIPCHK(hipMemcpyAsync(dtok, toks.data(), sizeof(int32_t) * toks.size(), hipMemcpyHostToDevice, st));
    HIPCHK(hipEventRecord(ev[0], st));
    TRY(mel_dev(e, dx, n, dmel, msc));
    HIPCHK(hipEventRecord(ev[1], st));
    int64_t nt = 0;
    TRY(encoder_forward_dev(e, dmel, nf, enc, &nt));
    HIPCHK(hipEventRecord(ev[2], st));
    LAUNCHCHK(launch_build_prompt(emb, d->embed, dtok, n_head, enc, (int)T, n_tail, H, st), "prompt");
    d->len = 0;
    TRY(decoder_prefill_dev(d, emb, total - 1));
    TRY(decoder_set_state(d, 0));
    HIPCHK(hipMemcpyAsync(d->x, emb + (total - 1) * H, sizeof(float) * H, hipMemcpyDeviceToDevice, st));
    TRY(decoder_enqueue_step(d, false));
    d->step_pos += 1;
    HIPCHK(hipEventRecord(ev[3], st));
    *total_out = total;
    return QASR_OK;
}

static void stage_times(qasr_encoder *e, double *times_ms) {
    if (!times_ms) return;
    for (int i = 0; i < 4; i++) {
        float ms = 0.0f;
        (void)hipEventElapsedTime(&ms, e->ev[i], e->ev[i + 1]);
        times_ms[i] = ms;
    }
}

// Every error after work has been queued leaves through one exit that waits
// for the stream, so no kernel of this call is still running on return.
extern "C" int qasr_hip_transcribe_forced(qasr_decoder *d, qasr_encoder *e, const float *samples, int64_t n,
                                          int32_t n_steps, int32_t *tokens_out, double *times_ms) {
    if (n_steps <= 0 || !tokens_out) return qasr_fail(QASR_ERR_INVALID, "transcribe: bad arguments");
    int64_t total = 0;
    auto body = [&]() -> int {
        TRY(transcribe_begin(d, e, samples, n, n_steps, nullptr, nullptr, 0, &total));
        hipStream_t st = d->h->stream;
        TRY(decoder_run_embed_steps(d, n_steps - 1));
        HIPCHK(hipEventRecord(e->ev[4], st));
        HIPCHK(hipMemcpyAsync(tokens_out, d->token_log, sizeof(int32_t) * n_steps, hipMemcpyDeviceToHost, st));
        HIPCHK(hipStreamSynchronize(st));
        TRY(decoder_fault_check(d));
        d->len += n_steps;
        stage_times(e, times_ms);
        return QASR_OK;
    };
    const int rc = body();
    if (rc != QASR_OK && d && d->h) (void)hipStreamSynchronize(d->h->stream);
    return rc;
}

// transcribe_segment's decode loop (transcribe.rs:186-230): greedy forwards
// until one yields a stop token (151643 endoftext, 151645 im_end) or
// max_tokens forwards have run.  The steps are graph replays in bursts of 8;
// between bursts the host reads the token log (a burst may run past the stop:
// those positions are discarded by setting the KV length back).
static const int TOKEN_ENDOFTEXT = 151643, TOKEN_IM_END = 151645;

extern "C" int qasr_hip_transcribe_prompt(qasr_decoder *d, qasr_encoder *e, const float *samples, int64_t n,
                                          const qasr_prompt *prompt, const int32_t *past, int64_t n_past,
                                          int32_t max_tokens, int32_t *tokens_out, int64_t *n_out, double *times_ms) {
    if (max_tokens <= 0 || !tokens_out || !n_out) return qasr_fail(QASR_ERR_INVALID, "transcribe: bad arguments");
    *n_out = 0;
    int64_t total = 0;
    constexpr int BURST = 8;
    auto body = [&]() -> int {
        TRY(transcribe_begin(d, e, samples, n, max_tokens, prompt, past, n_past, &total));
        hipStream_t st = d->h->stream;
        int64_t done = 1, stop_at = -1;            // forwards queued; index of the stop token
        std::vector<int32_t> log;
        int64_t seen = 0;
        int32_t fault = 0;
        while (true) {
            // read what has been produced so far
            log.resize((size_t)done);
            HIPCHK(hipMemcpyAsync(log.data() + seen, d->token_log + seen, sizeof(int32_t) * (done - seen),
                                  hipMemcpyDeviceToHost, st));
            HIPCHK(hipMemcpyAsync(&fault, d->state + 5, sizeof(fault), hipMemcpyDeviceToHost, st));
            HIPCHK(hipStreamSynchronize(st));
            if (fault) TRY(decoder_fault_check(d));  // a failed hand-off ends the call at once
            for (int64_t i = seen; i < done; i++)
                if (log[(size_t)i] == TOKEN_ENDOFTEXT || log[(size_t)i] == TOKEN_IM_END) {
                    stop_at = i;
                    break;
                }
            seen = done;
            if (stop_at >= 0 || done >= max_tokens) break;
            const int64_t b = std::min<int64_t>(BURST, max_tokens - done);
            TRY(decoder_run_embed_steps(d, b));
            done += b;
        }
        HIPCHK(hipEventRecord(e->ev[4], st));
        HIPCHK(hipStreamSynchronize(st));
        TRY(decoder_fault_check(d));
        const int64_t kept = stop_at >= 0 ? stop_at + 1 : done;
        std::memcpy(tokens_out, log.data(), sizeof(int32_t) * kept);
        *n_out = kept;
        d->len += kept;                             // the KV holds the kept tokens' positions
        stage_times(e, times_ms);
        return QASR_OK;
    };
    const int rc = body();
    if (rc != QASR_OK && d && d->h) (void)hipStreamSynchronize(d->h->stream);
    return rc;
}

extern "C" int qasr_hip_transcribe(qasr_decoder *d, qasr_encoder *e, const float *samples, int64_t n,
                                   int32_t max_tokens, int32_t *tokens_out, int64_t *n_out, double *times_ms) {
    return qasr_hip_transcribe_prompt(d, e, samples, n, nullptr, nullptr, 0, max_tokens, tokens_out, n_out, times_ms);
}

// The ids transcribe_segment turns into text (transcribe.rs:196-214): the
// tokens after the first <asr_text> (151704) and before a stop token; with
// text_open (forced-language or past-text ids in the prompt, transcribe.rs:
// 196) every token before the stop except <asr_text> itself.
extern "C" int64_t qasr_hip_text_tokens_from(const int32_t *raw, int64_t n, int text_open, int32_t *out) {
    if (!raw || n < 0) return -1;
    int64_t k = 0;
    bool past = text_open != 0;
    for (int64_t i = 0; i < n; i++) {
        const int32_t t = raw[i];
        if (t == TOKEN_ENDOFTEXT || t == TOKEN_IM_END) break;
        if (t == TOKEN_ASR_TEXT) past = true;
        else if (past) {
            if (out) out[k] = t;
            k++;
        }
    }
    return k;
}

extern "C" int64_t qasr_hip_text_tokens(const int32_t *raw, int64_t n, int32_t *out) {
    return qasr_hip_text_tokens_from(raw, n, 0, out);
}

/*
 * C smoke test of the libqasr_hip C ABI, compiled as C99 against
 * include/qasr_hip.h alone, the way a C, JNI or Dart FFI caller links it
 * (the reference's pass-through layers c_api.rs, jni_api.rs and
 * qwen_asr_bridge.rs bind a C ABI the same way).  Weights and inputs come from
 * the seeded generator of libqasr_synth, named as qwenasr_amd.synth names
 * them, so a Python run of the same model reproduces every number printed.
 *
 * usage: c_abi_smoke [seed]
 * prints "tokens: ..." (8 greedy steps after a 20-row prefill), "argmax: ..."
 * (the aligner readout of rows 0, 7 and 19 of the same prefill) and "ok".
 */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "qasr_hip.h"

/* libqasr_synth (qwenasr_amd/csrc/synth.c) */
void qs_normal_bf16(uint16_t *out, uint64_t n, uint64_t seed, const char *name, double mean, double std);
void qs_normal_f32(float *out, uint64_t n, uint64_t seed, const char *name, double mean, double std);

#define CHECK(call)                                                                   \
    do {                                                                              \
        int rc_ = (call);                                                             \
        if (rc_ != QASR_OK) {                                                         \
            fprintf(stderr, "%s failed (%d): %s\n", #call, rc_, qasr_hip_last_error()); \
            exit(1);                                                                  \
        }                                                                             \
    } while (0)

enum { N_LAYERS = 2, HIDDEN = 1024, N_HEADS = 16, N_KV = 8, HD = 128, INTER = 3072, VOCAB = 4096 };
enum { PREFILL = 20, STEPS = 8, MAX_SEQ = 128 };

static uint16_t *bf16_tensor(uint64_t seed, const char *name, size_t n) {
    uint16_t *p = malloc(n * sizeof *p);
    if (!p) exit(2);
    qs_normal_bf16(p, n, seed, name, 0.0, 0.02);
    return p;
}

static float *ones(size_t n) {
    float *p = malloc(n * sizeof *p);
    size_t i;
    if (!p) exit(2);
    for (i = 0; i < n; i++) p[i] = 1.0f;
    return p;
}

int main(int argc, char **argv) {
    const uint64_t seed = argc > 1 ? strtoull(argv[1], NULL, 10) : 1002;
    const size_t qd = (size_t)N_HEADS * HD, kvd = (size_t)N_KV * HD;
    qasr_dec_config cfg;
    qasr_dec_layer layers[N_LAYERS];
    qasr_dec_weights w;
    qasr_hip *h = NULL;
    qasr_decoder *d = NULL;
    float *emb;
    int32_t tok = 11, rows[3] = {0, 7, PREFILL - 1}, idx[3];
    int n_dev = 0, l, s;
    char name[128];

    CHECK(qasr_hip_device_count(&n_dev));
    if (n_dev < 1) {
        fprintf(stderr, "no GPU\n");
        return 1;
    }
    CHECK(qasr_hip_create(0, &h));

    memset(&cfg, 0, sizeof cfg);
    cfg.n_layers = N_LAYERS; cfg.hidden = HIDDEN; cfg.n_heads = N_HEADS; cfg.n_kv_heads = N_KV;
    cfg.head_dim = HD; cfg.intermediate = INTER; cfg.vocab = VOCAB; cfg.eps = 1e-6f; cfg.theta = 1e6f;
    for (l = 0; l < N_LAYERS; l++) {
        qasr_dec_layer *L = &layers[l];
#define W(field, tensor, n)                                                              \
        snprintf(name, sizeof name, "thinker.model.layers.%d.%s.weight", l, tensor);     \
        L->field = bf16_tensor(seed, name, n)
        W(wq, "self_attn.q_proj", qd * HIDDEN);
        W(wk, "self_attn.k_proj", kvd * HIDDEN);
        W(wv, "self_attn.v_proj", kvd * HIDDEN);
        W(wo, "self_attn.o_proj", (size_t)HIDDEN * qd);
        W(gate, "mlp.gate_proj", (size_t)INTER * HIDDEN);
        W(up, "mlp.up_proj", (size_t)INTER * HIDDEN);
        W(down, "mlp.down_proj", (size_t)HIDDEN * INTER);
#undef W
        L->q_norm = ones(HD);
        L->k_norm = ones(HD);
        L->input_norm = ones(HIDDEN);
        L->post_attn_norm = ones(HIDDEN);
    }
    w.embed = bf16_tensor(seed, "thinker.model.embed_tokens.weight", (size_t)VOCAB * HIDDEN);
    w.norm = ones(HIDDEN);
    w.layers = layers;
    CHECK(qasr_hip_decoder_load(h, &cfg, &w, QASR_ROUND_HALF_AWAY, MAX_SEQ, 0, &d));

    emb = malloc(sizeof(float) * PREFILL * HIDDEN);
    if (!emb) return 2;
    qs_normal_f32(emb, (uint64_t)PREFILL * HIDDEN, seed, "c_abi_smoke.prefill", 0.0, 0.02);

    /* decoder_prefill + greedy decode_forward steps, token in / token out */
    CHECK(qasr_hip_decoder_prefill(d, emb, PREFILL));
    if (qasr_hip_decoder_len(d) != PREFILL) {
        fprintf(stderr, "kv length %lld after prefill\n", (long long)qasr_hip_decoder_len(d));
        return 1;
    }
    printf("tokens:");
    for (s = 0; s < STEPS; s++) {
        CHECK(qasr_hip_decoder_forward(d, NULL, tok, &tok));
        printf(" %d", tok);
    }
    printf("\n");

    /* the aligner readout over the same prefill */
    CHECK(qasr_hip_decoder_set_len(d, 0));
    CHECK(qasr_hip_decoder_prefill_argmax(d, emb, PREFILL, rows, 3, idx));
    printf("argmax: %d %d %d\n", idx[0], idx[1], idx[2]);

    /* a rejected call reports through the status code and the error message */
    if (qasr_hip_decoder_prefill(d, NULL, 5) != QASR_ERR_INVALID || !qasr_hip_last_error() ||
        !qasr_hip_last_error()[0]) {
        fprintf(stderr, "bad-argument call was not rejected\n");
        return 1;
    }

    qasr_hip_decoder_free(d);
    qasr_hip_destroy(h);
    for (l = 0; l < N_LAYERS; l++) {
        free((void *)layers[l].wq); free((void *)layers[l].wk); free((void *)layers[l].wv);
        free((void *)layers[l].wo); free((void *)layers[l].gate); free((void *)layers[l].up);
        free((void *)layers[l].down); free((void *)layers[l].q_norm); free((void *)layers[l].k_norm);
        free((void *)layers[l].input_norm); free((void *)layers[l].post_attn_norm);
    }
    free((void *)w.embed);
    free((void *)w.norm);
    free(emb);
    printf("ok\n");
    return 0;
}

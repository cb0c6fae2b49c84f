/*
 * Seeded synthetic inputs for the QwenASR int8 hot path: weights, activations
 * and audio.  There are no real checkpoints or recordings on the GPU boxes, so
 * every benchmark and parity case draws its data from this one generator; the
 * CPU checker and the HIP path then receive the very same bytes.
 *
 * Stream:  SplitMix64 seeds xoshiro256**; a normal variate is Box-Muller in
 * double (cosine branch only), u1 in (0,1], u2 in [0,1).  A tensor is cut into
 * blocks of QS_BLOCK elements and block b of tensor `name` draws from its own
 * stream seeded with  seed ^ fnv1a64(name) ^ splitmix(b),  so generation is
 * deterministic regardless of how many threads fill the blocks.
 *
 * Weights follow the reference's synthetic-model rule: matrices, embeddings
 * and conv kernels ~ N(0, std) rounded to bf16 (round-to-nearest-even);
 * norm gains = 1, biases = 0 (those are plain fills, not drawn here).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>
#include <pthread.h>
#include <stdlib.h>

#define QS_BLOCK (1u << 20)

static uint64_t splitmix64(uint64_t *s) {
    uint64_t z = (*s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

typedef struct { uint64_t s[4]; } xoshiro_t;

static inline uint64_t rotl(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }

static uint64_t xo_next(xoshiro_t *r) {
    uint64_t *s = r->s;
    uint64_t result = rotl(s[1] * 5, 7) * 9;
    uint64_t t = s[1] << 17;
    s[2] ^= s[0]; s[3] ^= s[1]; s[1] ^= s[2]; s[0] ^= s[3];
    s[2] ^= t; s[3] = rotl(s[3], 45);
    return result;
}

static void xo_seed(xoshiro_t *r, uint64_t seed) {
    uint64_t sm = seed;
    for (int i = 0; i < 4; i++) r->s[i] = splitmix64(&sm);
}

uint64_t qs_fnv1a64(const char *name) {
    uint64_t h = 0xCBF29CE484222325ull;
    for (const unsigned char *p = (const unsigned char *)name; *p; p++) {
        h ^= *p;
        h *= 0x100000001B3ull;
    }
    return h;
}

static uint64_t block_seed(uint64_t seed, const char *name, uint64_t block) {
    uint64_t b = block * 0x2545F4914F6CDD1Dull + 1;
    return seed ^ qs_fnv1a64(name) ^ splitmix64(&b);
}

static inline double xo_unit_open0(xoshiro_t *r) {   /* (0, 1] */
    return ((double)(xo_next(r) >> 11) + 1.0) * (1.0 / 9007199254740992.0);
}
static inline double xo_unit(xoshiro_t *r) {          /* [0, 1) */
    return (double)(xo_next(r) >> 11) * (1.0 / 9007199254740992.0);
}
static inline double xo_normal(xoshiro_t *r) {
    double u1 = xo_unit_open0(r), u2 = xo_unit(r);
    return sqrt(-2.0 * log(u1)) * cos(6.283185307179586476925 * u2);
}

/* f32 -> bf16 with round-to-nearest-even (NaN kept quiet). */
uint16_t qs_f32_to_bf16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x40);
    uint32_t lsb = (u >> 16) & 1u;
    u += 0x7FFFu + lsb;
    return (uint16_t)(u >> 16);
}

/* ---- block-parallel fill ---------------------------------------------- */

typedef struct {
    void *out; int kind;          /* 0: f32, 1: bf16 */
    uint64_t n, seed; const char *name; double mean, std;
    uint64_t next_block, n_blocks;
    pthread_mutex_t mu;
} fill_job_t;

static void fill_block(fill_job_t *j, uint64_t b) {
    xoshiro_t r;
    xo_seed(&r, block_seed(j->seed, j->name, b));
    uint64_t lo = b * QS_BLOCK, hi = lo + QS_BLOCK;
    if (hi > j->n) hi = j->n;
    if (j->kind == 0) {
        float *o = (float *)j->out;
        for (uint64_t i = lo; i < hi; i++) o[i] = (float)(j->mean + j->std * xo_normal(&r));
    } else {
        uint16_t *o = (uint16_t *)j->out;
        for (uint64_t i = lo; i < hi; i++) o[i] = qs_f32_to_bf16((float)(j->mean + j->std * xo_normal(&r)));
    }
}

static void *fill_worker(void *arg) {
    fill_job_t *j = (fill_job_t *)arg;
    for (;;) {
        pthread_mutex_lock(&j->mu);
        uint64_t b = j->next_block++;
        pthread_mutex_unlock(&j->mu);
        if (b >= j->n_blocks) break;
        fill_block(j, b);
    }
    return NULL;
}

static int g_threads = 8;

/* Number of host threads used by the fills (1..64).  Results do not depend on it. */
void qs_set_threads(int n) { g_threads = n < 1 ? 1 : (n > 64 ? 64 : n); }

static void run_fill(void *out, int kind, uint64_t n, uint64_t seed, const char *name,
                     double mean, double std) {
    fill_job_t j;
    j.out = out; j.kind = kind; j.n = n; j.seed = seed; j.name = name;
    j.mean = mean; j.std = std; j.next_block = 0;
    j.n_blocks = (n + QS_BLOCK - 1) / QS_BLOCK;
    pthread_mutex_init(&j.mu, NULL);
    int nt = g_threads;
    if ((uint64_t)nt > j.n_blocks) nt = (int)j.n_blocks;
    if (nt <= 1) {
        fill_worker(&j);
    } else {
        pthread_t th[64];
        for (int t = 0; t < nt; t++) pthread_create(&th[t], NULL, fill_worker, &j);
        for (int t = 0; t < nt; t++) pthread_join(th[t], NULL);
    }
    pthread_mutex_destroy(&j.mu);
}

/* out[i] = f32(mean + std * N(0,1)) */
void qs_normal_f32(float *out, uint64_t n, uint64_t seed, const char *name, double mean, double std) {
    run_fill(out, 0, n, seed, name, mean, std);
}

/* out[i] = bf16_rne(f32(mean + std * N(0,1))) */
void qs_normal_bf16(uint16_t *out, uint64_t n, uint64_t seed, const char *name, double mean, double std) {
    run_fill(out, 1, n, seed, name, mean, std);
}

/*
 * Synthetic 16 kHz mono test audio: white noise at noise_dbfs (sigma =
 * 10^(dBFS/20)) plus sines at 440, 1000 and 3150 Hz of amplitude 0.05 each,
 * rounded to int16 and scaled by 1/32768 like a decoded 16-bit WAV, so the
 * PCM and WAV paths see identical samples.
 */
void qs_audio(float *out, uint64_t n, uint64_t seed, double noise_dbfs) {
    double sigma = pow(10.0, noise_dbfs / 20.0);
    qs_normal_f32(out, n, seed, "audio.noise", 0.0, sigma);
    const double f[3] = {440.0, 1000.0, 3150.0};
    for (uint64_t i = 0; i < n; i++) {
        double t = (double)i / 16000.0, v = (double)out[i];
        for (int k = 0; k < 3; k++) v += 0.05 * sin(6.283185307179586476925 * f[k] * t);
        double s = nearbyint(v * 32768.0);
        if (s > 32767.0) s = 32767.0;
        if (s < -32768.0) s = -32768.0;
        out[i] = (float)((int16_t)s) / 32768.0f;
    }
}

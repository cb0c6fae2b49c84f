/*
 * qasr_oracle GEMM — TEST INFRASTRUCTURE ONLY.
 *
 * Restates the reference's cblas_sgemm calls (kernels/mod.rs:496-628,
 * 1124-1130; OpenBLAS on Linux, build.rs:11-13) as a blocked f32 GEMM in the
 * "NT" form C[m,n] (+)= sum_k A[m,k] B[n,k].  BLAS summation order is not
 * pinned by anything the reference ships, so this file is free to use FMA and
 * K-blocking; GEMM outputs are compared with a tolerance.
 */
#include "qasr_oracle.h"
#include <string.h>
#include <omp.h>

typedef float v8f __attribute__((vector_size(32)));
typedef float v8fu __attribute__((vector_size(32), aligned(4)));

#define MB 3
#define NB 4
#define KB 512
#define PANEL 96

static inline v8f ld8(const float *p) { return *(const v8fu *)p; }

static inline float hsum(v8f v) {
    return ((v[0] + v[4]) + (v[1] + v[5])) + ((v[2] + v[6]) + (v[3] + v[7]));
}

/* one tile: rows [m0, m0+mr) x cols [n0, n0+nr), k in [k0, k1) */
static void tile(int64_t m0, int mr, int64_t n0, int nr, int64_t k0, int64_t k1,
                 const float *A, int64_t lda, const float *B, int64_t ldb,
                 float *C, int64_t ldc, int accumulate) {
    v8f acc[MB][NB];
    for (int i = 0; i < MB; i++)
        for (int j = 0; j < NB; j++) acc[i][j] = (v8f){0, 0, 0, 0, 0, 0, 0, 0};
    int64_t kv = k0 + ((k1 - k0) / 8) * 8;
    if (mr == MB && nr == NB) {
        const float *a0 = A + m0 * lda, *a1 = a0 + lda, *a2 = a1 + lda;
        const float *b0 = B + n0 * ldb, *b1 = b0 + ldb, *b2 = b1 + ldb, *b3 = b2 + ldb;
        for (int64_t k = k0; k < kv; k += 8) {
            v8f x0 = ld8(a0 + k), x1 = ld8(a1 + k), x2 = ld8(a2 + k);
            v8f y = ld8(b0 + k);
            acc[0][0] += x0 * y; acc[1][0] += x1 * y; acc[2][0] += x2 * y;
            y = ld8(b1 + k);
            acc[0][1] += x0 * y; acc[1][1] += x1 * y; acc[2][1] += x2 * y;
            y = ld8(b2 + k);
            acc[0][2] += x0 * y; acc[1][2] += x1 * y; acc[2][2] += x2 * y;
            y = ld8(b3 + k);
            acc[0][3] += x0 * y; acc[1][3] += x1 * y; acc[2][3] += x2 * y;
        }
    } else {
        for (int64_t k = k0; k < kv; k += 8)
            for (int i = 0; i < mr; i++) {
                v8f x = ld8(A + (m0 + i) * lda + k);
                for (int j = 0; j < nr; j++) acc[i][j] += x * ld8(B + (n0 + j) * ldb + k);
            }
    }
    for (int i = 0; i < mr; i++)
        for (int j = 0; j < nr; j++) {
            float s = hsum(acc[i][j]);
            const float *ar = A + (m0 + i) * lda, *br = B + (n0 + j) * ldb;
            for (int64_t k = kv; k < k1; k++) s += ar[k] * br[k];
            float *c = C + (m0 + i) * ldc + n0 + j;
            *c = accumulate ? *c + s : s;
        }
}

void or_sgemm_nt(int64_t M, int64_t N, int64_t K, const float *A, int64_t lda,
                 const float *B, int64_t ldb, float *C, int64_t ldc, int beta_one) {
    if (M <= 0 || N <= 0) return;
    if (K <= 0) {
        if (!beta_one)
            for (int64_t m = 0; m < M; m++) memset(C + m * ldc, 0, sizeof(float) * N);
        return;
    }
    int64_t n_panels = (N + PANEL - 1) / PANEL;
#pragma omp parallel for schedule(dynamic)
    for (int64_t p = 0; p < n_panels; p++) {
        int64_t p0 = p * PANEL, p1 = p0 + PANEL < N ? p0 + PANEL : N;
        for (int64_t k0 = 0; k0 < K; k0 += KB) {
            int64_t k1 = k0 + KB < K ? k0 + KB : K;
            int acc = beta_one || k0 > 0;
            for (int64_t m0 = 0; m0 < M; m0 += MB) {
                int mr = (int)(M - m0 < MB ? M - m0 : MB);
                for (int64_t n0 = p0; n0 < p1; n0 += NB) {
                    int nr = (int)(p1 - n0 < NB ? p1 - n0 : NB);
                    tile(m0, mr, n0, nr, k0, k1, A, lda, B, ldb, C, ldc, acc);
                }
            }
        }
    }
}

/*
 * sanitize_check.c — drives every function of oracle.c on small cases with exactly sized heap buffers, built with
 * AddressSanitizer and UndefinedBehaviorSanitizer (make -C oracle sanitize). TEST INFRASTRUCTURE ONLY: it checks the
 * oracle's memory accesses and arithmetic for undefined behaviour, not its values (tests/test_oracle.py pins those).
 * Edge cases: zero query rows, causal rows whose limit passes the cache end, GQA groups, strided rows, more threads
 * than tasks, every rotary mode, every linear flag, and the f16 conversions over all 65,536 patterns.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>

int oracle_attention_f64(int32_t, int32_t, int32_t, int32_t, int32_t, int32_t, int32_t, double, const uint16_t *, int64_t,
                         const uint16_t *, const uint16_t *, int64_t, double *, int64_t, double *);
int oracle_cpu_attend_f32(int32_t, int32_t, int32_t, int32_t, int32_t, int32_t, int32_t, float, const float *, int64_t,
                          const float *, const float *, int64_t, float *, int64_t, int32_t);
void oracle_f16_to_f32(const uint16_t *, float *, int64_t);
void oracle_f32_to_f16(const float *, uint16_t *, int64_t);
void oracle_rope_f32(int32_t, float, int32_t, int32_t, const float *, float *, int64_t);
int oracle_linear_f64(int32_t, int32_t, int32_t, uint32_t, int32_t, float, const float *, int64_t, const uint16_t *,
                      const float *, const float *, double *);

static uint32_t rng = 12345u;
static float frand(void) {
    rng = rng * 1664525u + 1013904223u;
    return (float)(rng >> 8) / 16777216.f * 2.f - 1.f;
}

static int fails = 0;
#define CHECK(c) do { if (!(c)) { fprintf(stderr, "FAILED %s:%d: %s\n", __FILE__, __LINE__, #c); fails++; } } while (0)

static void attention_case(int nh, int nkv, int hd, int nq, int p0, int n_kv, int causal, int pad, int threads) {
    const int64_t qs = (int64_t)nh * hd + pad, ks = (int64_t)nkv * hd + pad, os = (int64_t)nh * hd + pad;
    const int64_t nq1 = nq > 0 ? nq : 1;
    float * qf = malloc(sizeof(float) * (size_t)(nq1 * qs));
    float * kf = malloc(sizeof(float) * (size_t)(n_kv * ks));
    float * vf = malloc(sizeof(float) * (size_t)(n_kv * ks));
    uint16_t * q = malloc(2 * (size_t)(nq1 * qs));
    uint16_t * k = malloc(2 * (size_t)(n_kv * ks));
    uint16_t * v = malloc(2 * (size_t)(n_kv * ks));
    double * out = malloc(sizeof(double) * (size_t)(nq1 * os));
    double * lse = malloc(sizeof(double) * (size_t)(nq1 * nh));
    float * out32 = malloc(sizeof(float) * (size_t)(nq1 * os));
    for (int64_t i = 0; i < nq1 * qs; i++) qf[i] = frand();
    for (int64_t i = 0; i < n_kv * ks; i++) kf[i] = frand(), vf[i] = frand();
    oracle_f32_to_f16(qf, q, nq1 * qs);
    oracle_f32_to_f16(kf, k, n_kv * ks);
    oracle_f32_to_f16(vf, v, n_kv * ks);
    CHECK(oracle_attention_f64(nh, nkv, hd, nq, p0, n_kv, causal, 1.0 / sqrt((double)hd), q, qs, k, v, ks, out, os, lse) == 0);
    CHECK(oracle_cpu_attend_f32(nh, nkv, hd, nq, p0, n_kv, causal, 1.f / sqrtf((float)hd), qf, qs, kf, vf, ks, out32, os,
                                threads) == 0);
    for (int64_t t = 0; t < nq; t++)
        for (int h = 0; h < nh; h++) CHECK(isfinite(lse[t * nh + h]));
    free(qf), free(kf), free(vf), free(q), free(k), free(v), free(out), free(lse), free(out32);
}

int main(void) {
    // f16 <-> f32 over every bit pattern
    uint16_t * all = malloc(2 * 65536);
    float * f = malloc(4 * 65536);
    uint16_t * back = malloc(2 * 65536);
    for (int i = 0; i < 65536; i++) all[i] = (uint16_t)i;
    oracle_f16_to_f32(all, f, 65536);
    oracle_f32_to_f16(f, back, 65536);
    for (int i = 0; i < 65536; i++)
        if (!isnan(f[i])) CHECK(back[i] == all[i]);
    free(all), free(f), free(back);

    attention_case(4, 2, 16, 5, 0, 5, 1, 0, 1);
    attention_case(4, 2, 16, 0, 3, 7, 1, 0, 3);      // no query rows
    attention_case(8, 1, 64, 7, 40, 30, 1, 8, 4);     // causal limit past the cache end
    attention_case(6, 3, 8, 9, 0, 33, 0, 4, 64);      // non-causal, more threads than tasks
    attention_case(2, 2, 128, 3, 100, 103, 1, 0, 2);
    attention_case(28, 4, 128, 2, 500, 502, 1, 0, 8);

    for (int mode = 0; mode < 3; mode++) {
        for (int hd = 4; hd <= 256; hd *= 2) {
            float * x = malloc(sizeof(float) * (size_t)(3 * hd));
            float * y = malloc(sizeof(float) * (size_t)(3 * hd));
            for (int i = 0; i < 3 * hd; i++) x[i] = frand();
            oracle_rope_f32(mode, 10000.f, hd, 12345, x, y, 3);
            for (int i = 0; i < 3 * hd; i++) CHECK(isfinite(y[i]));
            free(x), free(y);
        }
    }

    for (uint32_t flags = 0; flags < 8; flags++) {
        for (int half_input = 0; half_input < 2; half_input++) {
            const int M = 5, N = 7, K = 96, xs = K + 4;
            float * X = malloc(sizeof(float) * (size_t)(M * xs));
            float * xw = malloc(sizeof(float) * (size_t)(N * K));
            uint16_t * W = malloc(2 * (size_t)(N * K));
            float * g = malloc(sizeof(float) * (size_t)K);
            float * b = malloc(sizeof(float) * (size_t)N);
            double * Y = calloc((size_t)(M * N), sizeof(double));
            for (int i = 0; i < M * xs; i++) X[i] = frand();
            for (int i = 0; i < N * K; i++) xw[i] = frand();
            for (int i = 0; i < K; i++) g[i] = frand() + 1.5f;
            for (int i = 0; i < N; i++) b[i] = frand();
            oracle_f32_to_f16(xw, W, N * K);
            CHECK(oracle_linear_f64(M, N, K, flags, half_input, 1e-5f, X, xs, W, g, b, Y) == 0);
            for (int i = 0; i < M * N; i++) CHECK(isfinite(Y[i]));
            free(X), free(xw), free(W), free(g), free(b), free(Y);
        }
    }
    CHECK(oracle_attention_f64(3, 2, 16, 1, 0, 1, 1, 1.0, NULL, 0, NULL, NULL, 0, NULL, 0, NULL) == 1);  // 3 % 2 != 0
    if (fails) {
        fprintf(stderr, "%d checks failed\n", fails);
        return 1;
    }
    printf("sanitize_check: ok\n");
    return 0;
}

/*
 * oracle.c — CPU oracle of the attention hot path. TEST INFRASTRUCTURE ONLY.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load this library, and only as the checker
 * (or as the timed CPU baseline); the product path (dooms_amd/) never calls it and has no CPU fallback.
 *
 * Two functions:
 *
 * 1. oracle_attention_f64 — brute-force attention in double precision on f16 inputs, the reference's own test oracle:
 *    the attention loop of Reference::step (tests/unit/test_metal_llama_decoder.cpp:129-147: per head, scores
 *    q.k / sqrt(hd) in double over positions 0..pos, max, exp, sum, sum_j p_j v_j / sum) and attention_ref
 *    (tests/unit/test_backend_ggml.cpp:650-675, non-causal, scale argument), generalized to
 *      - GQA: query head h reads key/value head h / (n_head / n_head_kv) (src/backend/metal/llama_kernels.h:560,656,873);
 *      - a chunk offset p0 with the causal limit j <= p0 + t (llama_kernels.h:657,669,701);
 *      - the softmax statistics: m = max_j s_j and l = sum_j exp(s_j - m) of the scaled scores (the (max, sum) pair the
 *        reference's attention_split writes, llama_kernels.h:909), returned as lse = m + ln l.
 *    Pinned (tests/test_oracle.py) by torch's scaled_dot_product_attention in float64, closed forms (scale 0 -> mean of
 *    the visible values, one key -> that value, equal keys -> mean), GQA-as-repeated-MHA, causal-as-prefix, and the
 *    committed golden fixtures.
 *
 * 2. oracle_cpu_attend_f32 — a restatement of the reference's C++ CPU attention, CpuWhisperDecoder::Impl::attend
 *    (src/backend/cpu/cpu_whisper_decoder.cpp:100-112): per head, f32 scores = scale * K_h q_h (cblas_sgemv, here a
 *    plain f32 dot product), f32 max, exp(s - max) in f32 accumulated into a DOUBLE sum, inv = (float)(1 / sum), and
 *    out_h = inv * V_h^T p (cblas_sgemv Trans, here an f32 loop). Generalized like (1) to GQA and the causal limit. With
 *    n_threads > 1 the (row, head) tasks are dealt out over threads as the reference's attention_cpu_op does
 *    (src/backend/ggml/ggml_backend.cpp:292-312, task = ith; task += nth). Accelerate is absent here, so plain loops stand
 *    in for cblas_sgemv. This is the CPU baseline bench.py times; it is checked against (1) within f32 error.
 *
 * 3. oracle_rope_f32 — the rotary embedding of the reference's rope_store / fused attention (rotate_pair and pair_index,
 *    src/backend/metal/llama_kernels.h:508-518): pair i of a head (adjacent (2i, 2i+1), or split halves (i, i + hd/2)
 *    for neox) turns by theta = pos * base^(-2i / hd). As in the reference the angle is an f32 product of the f32
 *    position and the f32 frequency powf(base, -2i / hd); the rotation itself is evaluated in double from libm's sin
 *    and cos and rounded once to f32 (the reference and the GPU kernel rotate in f32: a few f32 ulps apart). Pinned
 *    (tests/test_oracle.py) against the reference test's own double-precision rope (Reference::rope,
 *    tests/unit/test_metal_llama_decoder.cpp:180-189) within the f32 rounding of the angle, against pos 0 = identity,
 *    per-pair norm preservation, the relative-position property <R(m) q, R(n) k> = <R(m - n) q, k>, and neox = adjacent
 *    conjugated by the half/interleave permutation.
 *
 * 4. oracle_linear_f64 — the projections around the attention (src/backend/metal/llama_kernels.h): matvec1 / matvecm
 *    (96-126, 809-842: f32 input, y = (W . (x * gamma)) * scale + bias) and matmul / matmul_big with rms_scale (186-199,
 *    312-328, 418-450: input staged as half(x * (gamma * scale)), half products summed) — selected by half_input —
 *    summed here in double; scale = 1 / sqrt(mean(x^2) + eps) (the sum of squares in double, the scale rounded to
 *    f32 as the kernels keep it). Pinned (tests/test_oracle.py) against numpy's float64 matmul of the same operands,
 *    W = identity, W = 0 (bias only), the residual accumulate, and the closed-form scale of a constant row.
 *
 * Layout (attention functions): q [n_q][q_stride], k/v [n_kv][kv_stride], out [n_q][out_stride], lse [n_q][n_head]; head h
 * at column h * head_dim. Inputs are IEEE binary16 bit patterns.
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* IEEE binary16 -> binary32 (exact). */
static float f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t exp = (h >> 10) & 0x1fu, man = h & 0x3ffu;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else { /* subnormal: man * 2^-24 */
            float f = (float)man * (1.0f / 16777216.0f);
            memcpy(&bits, &f, 4);
            bits |= sign;
        }
    } else if (exp == 31) {
        bits = sign | 0x7f800000u | (man << 13);
    } else {
        bits = sign | ((exp + 112u) << 23) | (man << 13);
    }
    float out;
    memcpy(&out, &bits, 4);
    return out;
}

void oracle_f16_to_f32(const uint16_t * src, float * dst, int64_t n) {
    for (int64_t i = 0; i < n; i++) dst[i] = f16_to_f32(src[i]);
}

/* IEEE binary32 -> binary16, round to nearest even (overflow to infinity). */
static uint16_t f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    const uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0u)); /* inf, nan */
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);                                   /* rounds past 65504 */
    if (ax < 0x38800000u) { /* subnormal half (or zero): value = m * 2^-24 */
        float a;
        memcpy(&a, &ax, 4);
        const float m = a * 16777216.0f; /* exact: scaling by a power of two */
        const uint32_t r = (uint32_t)nearbyintf(m);  /* round half to even (default rounding mode) */
        return (uint16_t)(sign | r);
    }
    const uint32_t e = ((ax >> 23) - 112u) << 10, man = ax & 0x7fffffu;
    uint32_t h = e | (man >> 13);
    const uint32_t rest = man & 0x1fffu;
    if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) h++;
    return (uint16_t)(sign | h);
}

void oracle_f32_to_f16(const float * src, uint16_t * dst, int64_t n) {
    for (int64_t i = 0; i < n; i++) dst[i] = f32_to_f16(src[i]);
}

/* Last key visible to query row t, plus one. */
static int64_t n_visible(int64_t t, int32_t p0, int32_t n_kv, int32_t causal) {
    if (!causal) return n_kv;
    const int64_t v = (int64_t)p0 + t + 1;
    return v < n_kv ? v : n_kv;
}

int oracle_attention_f64(int32_t n_head, int32_t n_head_kv, int32_t head_dim, int32_t n_q, int32_t p0, int32_t n_kv,
                         int32_t causal, double scale, const uint16_t * q, int64_t q_stride, const uint16_t * k,
                         const uint16_t * v, int64_t kv_stride, double * out, int64_t out_stride, double * lse) {
    if (n_head < 1 || n_head_kv < 1 || n_head % n_head_kv || head_dim < 1 || n_q < 0 || n_kv < 1) return 1;
    const int32_t G = n_head / n_head_kv;
    double * sc = (double *)malloc(sizeof(double) * (size_t)n_kv);
    double * qd = (double *)malloc(sizeof(double) * (size_t)head_dim);
    if (!sc || !qd) { free(sc); free(qd); return 2; }
    for (int64_t t = 0; t < n_q; t++) {
        const int64_t nv = n_visible(t, p0, n_kv, causal);
        for (int32_t h = 0; h < n_head; h++) {
            const int32_t kvh = h / G;
            for (int32_t d = 0; d < head_dim; d++) qd[d] = f16_to_f32(q[t * q_stride + (int64_t)h * head_dim + d]);
            double mx = -INFINITY;
            for (int64_t j = 0; j < nv; j++) {
                const uint16_t * kr = k + j * kv_stride + (int64_t)kvh * head_dim;
                double s = 0;
                for (int32_t d = 0; d < head_dim; d++) s += qd[d] * (double)f16_to_f32(kr[d]);
                sc[j] = s * scale;
                if (sc[j] > mx) mx = sc[j];
            }
            double sum = 0;
            for (int64_t j = 0; j < nv; j++) { sc[j] = exp(sc[j] - mx); sum += sc[j]; }
            for (int32_t d = 0; d < head_dim; d++) {
                double a = 0;
                for (int64_t j = 0; j < nv; j++) a += sc[j] * (double)f16_to_f32(v[j * kv_stride + (int64_t)kvh * head_dim + d]);
                out[t * out_stride + (int64_t)h * head_dim + d] = a / sum;
            }
            if (lse) lse[t * n_head + h] = mx + log(sum);
        }
    }
    free(sc);
    free(qd);
    return 0;
}

/* ---- the restated CPU attention (f32, double sum), single- or multi-threaded ---- */

typedef struct {
    int32_t n_head, G, head_dim, n_q, p0, n_kv, causal;
    float scale;
    const float * q; int64_t q_stride;
    const float * k; const float * v; int64_t kv_stride;
    float * out; int64_t out_stride;
    int ith, nth;
} attend_job;

/* One (row, head) task: cpu_whisper_decoder.cpp:100-112 with GQA and a causal limit. */
static void attend_task(const attend_job * J, int64_t t, int32_t h, float * scores) {
    const int64_t n = n_visible(t, J->p0, J->n_kv, J->causal);
    const int32_t hd = J->head_dim, kvh = h / J->G;
    const float * qv = J->q + t * J->q_stride + (int64_t)h * hd;
    const float * K = J->k + (int64_t)kvh * hd;
    const float * V = J->v + (int64_t)kvh * hd;
    for (int64_t j = 0; j < n; j++) { /* cblas_sgemv NoTrans: scores = scale * K q */
        const float * kr = K + j * J->kv_stride;
        float s = 0.f;
        for (int32_t d = 0; d < hd; d++) s += kr[d] * qv[d];
        scores[j] = J->scale * s;
    }
    float mx = -INFINITY;
    for (int64_t j = 0; j < n; j++) mx = scores[j] > mx ? scores[j] : mx;
    double sum = 0;
    for (int64_t j = 0; j < n; j++) { scores[j] = expf(scores[j] - mx); sum += scores[j]; }
    const float inv = (float)(1.0 / sum);
    float * o = J->out + t * J->out_stride + (int64_t)h * hd;
    for (int32_t d = 0; d < hd; d++) o[d] = 0.f;
    for (int64_t j = 0; j < n; j++) { /* cblas_sgemv Trans: out = inv * V^T scores */
        const float * vr = V + j * J->kv_stride;
        const float pj = scores[j];
        for (int32_t d = 0; d < hd; d++) o[d] += pj * vr[d];
    }
    for (int32_t d = 0; d < hd; d++) o[d] *= inv;
}

static void * attend_worker(void * arg) {
    const attend_job * J = (const attend_job *)arg;
    float * scores = (float *)malloc(sizeof(float) * (size_t)J->n_kv);
    if (!scores) return (void *)1;
    const int64_t tasks = (int64_t)J->n_q * J->n_head;
    for (int64_t task = J->ith; task < tasks; task += J->nth) attend_task(J, task / J->n_head, (int32_t)(task % J->n_head), scores);
    free(scores);
    return NULL;
}

/* q/k/v are f32 here (the reference's CPU decoder keeps f32 caches, cpu_whisper_decoder.cpp:58,172-176); convert f16
 * inputs once with oracle_f16_to_f32 outside the timed region. */
int oracle_cpu_attend_f32(int32_t n_head, int32_t n_head_kv, int32_t head_dim, int32_t n_q, int32_t p0, int32_t n_kv,
                          int32_t causal, float scale, const float * q, int64_t q_stride, const float * k, const float * v,
                          int64_t kv_stride, float * out, int64_t out_stride, int32_t n_threads) {
    if (n_head < 1 || n_head_kv < 1 || n_head % n_head_kv || head_dim < 1 || n_q < 0 || n_kv < 1) return 1;
    if (n_threads < 1) n_threads = 1;
    if (n_threads > 256) n_threads = 256;
    attend_job base = {n_head, n_head / n_head_kv, head_dim, n_q, p0, n_kv, causal, scale, q, q_stride, k, v, kv_stride, out, out_stride, 0, n_threads};
    if (n_threads == 1) return attend_worker(&base) ? 2 : 0;
    attend_job jobs[256];
    pthread_t th[256];
    int rc = 0;
    for (int i = 0; i < n_threads; i++) {
        jobs[i] = base;
        jobs[i].ith = i;
        if (i > 0 && pthread_create(&th[i], NULL, attend_worker, &jobs[i]) != 0) { n_threads = i; rc = 3; break; }
    }
    if (attend_worker(&jobs[0])) rc = 2;
    for (int i = 1; i < n_threads; i++) {
        void * r = NULL;
        pthread_join(th[i], &r);
        if (r) rc = 2;
    }
    return rc;
}

/* Rotates n_vec head vectors of head_dim floats (x, contiguous, vector r at x + r * head_dim) for position pos into y.
 * mode 0: adjacent pairs, 1: split halves (neox), 2: copy. */
void oracle_rope_f32(int32_t mode, float base, int32_t head_dim, int32_t pos, const float * x, float * y, int64_t n_vec) {
    const int32_t hd = head_dim;
    for (int64_t r = 0; r < n_vec; r++) {
        const float * a = x + r * hd;
        float * b = y + r * hd;
        memcpy(b, a, sizeof(float) * (size_t)hd);
        if (mode == 2) continue;
        for (int32_t i = 0; i < hd / 2; i++) {
            const float freq = powf(base, -2.f * (float)i / (float)hd);
            const float theta = (float)pos * freq;
            const int32_t i0 = mode == 1 ? i : 2 * i, i1 = mode == 1 ? i + hd / 2 : 2 * i + 1;
            const double c = cos((double)theta), s = sin((double)theta);
            b[i0] = (float)((double)a[i0] * c - (double)a[i1] * s);
            b[i1] = (float)((double)a[i0] * s + (double)a[i1] * c);
        }
    }
}

/* Y[m][n] (+)= sum_k a[m][k] W[n][k] (+ bias[n]) in double for m < M, n < N (Y dense [M][N]). flags: 1 RMS norm with
 * gamma, 2 accumulate into Y, 4 bias. half_input: the matmul staging (a = half(x * (gamma * scale))), else the matvec
 * form (a = x * gamma in f32, the sum times scale). */
int oracle_linear_f64(int32_t M, int32_t N, int32_t K, uint32_t flags, int32_t half_input, float eps, const float * X,
                      int64_t x_stride, const uint16_t * W, const float * gamma, const float * bias, double * Y) {
    if (M < 0 || N < 1 || K < 1) return 1;
    float * a = (float *)malloc(sizeof(float) * (size_t)K);
    if (!a) return 2;
    const int norm = (flags & 1u) != 0;
    for (int64_t m = 0; m < M; m++) {
        const float * x = X + m * x_stride;
        float scale = 1.f;
        if (norm) {
            double ss = 0.0;
            for (int32_t k = 0; k < K; k++) ss += (double)x[k] * (double)x[k];
            scale = (float)(1.0 / sqrt(ss / (double)K + (double)eps));
        }
        for (int32_t k = 0; k < K; k++) {
            if (half_input) {
                const float v = norm ? x[k] * (gamma[k] * scale) : x[k];
                a[k] = f16_to_f32(f32_to_f16(v));
            } else {
                a[k] = norm ? x[k] * gamma[k] : x[k];
            }
        }
        for (int64_t n = 0; n < N; n++) {
            const uint16_t * wr = W + n * K;
            double s = 0.0;
            for (int32_t k = 0; k < K; k++) s += (double)a[k] * (double)f16_to_f32(wr[k]);
            if (norm && !half_input) s *= (double)scale;
            if (flags & 4u) s += (double)bias[n];
            double * y = Y + m * N + n;
            *y = (flags & 2u) ? *y + s : s;
        }
    }
    free(a);
    return 0;
}

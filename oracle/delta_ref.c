/*
 * delta_ref.c — C restatement of the reference's CPU delta-rule forward.
 * TEST INFRASTRUCTURE / CPU BASELINE ONLY: never linked into libpmdelta.so.
 *
 * Follows the reference's JAX/NumPy algorithm for this path:
 *   per-token rank-1 step   kernels/__init__.py:357-376 (_delta_step_np/_jax)
 *       kS = k^T S ; S' = S - beta k kS^T + beta k v^T ; o = q S'
 *   sequential over T       kernels/__init__.py:379-395 / :421-458
 *   fp32 throughout, inputs upcast to fp32 as at kernels/__init__.py:344-347
 * The (b, h) sequences are independent, so OpenMP splits them across threads.
 *
 * Built by oracle/build.py:  gcc -O3 -march=native -fopenmp -shared -fPIC
 */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static inline float bf16_to_f32(uint16_t x) {
    uint32_t u = ((uint32_t)x) << 16;
    float f;
    memcpy(&f, &u, sizeof f);
    return f;
}

static inline float load_in(const void* p, size_t i, int bf16) {
    return bf16 ? bf16_to_f32(((const uint16_t*)p)[i]) : ((const float*)p)[i];
}

/* One (b, h) sequence over T tokens; S is D x D scratch holding the state. */
static void run_sequence(const void* q, const void* k, const void* v, const float* beta,
                         float* o, float* S, int b, int h, int T, int H, int D, int bf16) {
    float* kt = (float*)malloc(sizeof(float) * (size_t)D * 4);
    float* qt = kt + D;
    float* vt = qt + D;
    float* ks = vt + D;
    for (int t = 0; t < T; ++t) {
        size_t base = (((size_t)b * T + t) * H + h) * (size_t)D;
        float bt = beta[((size_t)b * T + t) * H + h];
        for (int d = 0; d < D; ++d) {
            kt[d] = load_in(k, base + d, bf16);
            qt[d] = load_in(q, base + d, bf16);
            vt[d] = load_in(v, base + d, bf16);
        }
        /* kS[e] = sum_d k[d] S[d][e] */
        for (int e = 0; e < D; ++e) ks[e] = 0.0f;
        for (int d = 0; d < D; ++d) {
            float kd = kt[d];
            const float* row = S + (size_t)d * D;
            for (int e = 0; e < D; ++e) ks[e] += kd * row[e];
        }
        /* S[d][e] = S[d][e] - beta k[d] kS[e] + beta k[d] v[e] */
        for (int d = 0; d < D; ++d) {
            float bk = bt * kt[d];
            float* row = S + (size_t)d * D;
            for (int e = 0; e < D; ++e) row[e] = row[e] - bk * ks[e] + bk * vt[e];
        }
        /* o[e] = sum_d q[d] S'[d][e] */
        float* orow = o + base;
        for (int e = 0; e < D; ++e) orow[e] = 0.0f;
        for (int d = 0; d < D; ++d) {
            float qd = qt[d];
            const float* row = S + (size_t)d * D;
            for (int e = 0; e < D; ++e) orow[e] += qd * row[e];
        }
    }
    free(kt);
}

/*
 * Forward over (B, T, H, D); s0 may be NULL (zeros). in_bf16: q/k/v are
 * bf16 bit patterns (uint16) instead of fp32. o is fp32 (B, T, H, D),
 * s_out fp32 (B, H, D, D). threads <= 0 uses the OpenMP default.
 */
int oracle_delta_fwd(const void* q, const void* k, const void* v, const float* beta,
                     const float* s0, float* o, float* s_out, int B, int T, int H, int D,
                     int in_bf16, int threads) {
    if (B < 0 || T < 0 || H < 0 || D < 1) return -2;
    long pairs = (long)B * H;
#ifdef _OPENMP
    if (threads > 0) omp_set_num_threads(threads);
#else
    (void)threads;
#endif
#pragma omp parallel for schedule(dynamic, 1)
    for (long p = 0; p < pairs; ++p) {
        int b = (int)(p / H), h = (int)(p % H);
        float* S = s_out + (size_t)p * D * D;
        if (s0)
            memcpy(S, s0 + (size_t)p * D * D, sizeof(float) * (size_t)D * D);
        else
            memset(S, 0, sizeof(float) * (size_t)D * D);
        run_sequence(q, k, v, beta, o, S, b, h, T, H, D, in_bf16);
    }
    return 0;
}

/* One decode step on (B, H, D) tokens, S (B, H, D, D) updated in place. */
int oracle_delta_step(float* s, const void* q, const void* k, const void* v,
                      const float* beta, float* o, int B, int H, int D, int in_bf16,
                      int threads) {
    if (B < 0 || H < 0 || D < 1) return -2;
    long pairs = (long)B * H;
#ifdef _OPENMP
    if (threads > 0) omp_set_num_threads(threads);
#else
    (void)threads;
#endif
#pragma omp parallel for schedule(static)
    for (long p = 0; p < pairs; ++p) {
        int b = (int)(p / H), h = (int)(p % H);
        /* a (B, H, D) token is a (B, 1, H, D) sequence of length 1 */
        run_sequence(q, k, v, beta, o, s + (size_t)p * D * D, b, h, 1, H, D, in_bf16);
    }
    return 0;
}

int oracle_max_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/*
 * hx_oracle_omp.c — multi-threaded CPU selective scan, the "optimised host" baseline.
 *
 * TEST/BENCH INFRASTRUCTURE ONLY (bench.py's cpu_baseline leg and tests/): never linked into or
 * called by the product library. Same f32 arithmetic as oracle_selective_scan in hx_oracle.c
 * (Gu & Dao 2023 Alg. 2 with the reference's discretisation, crates/nn/src/ssm.rs:108-130),
 * parallelised with OpenMP over independent (batch, channel) rows; within a row the time loop
 * is sequential and the channel-contiguous layout is walked with stride dim.
 */
#include <math.h>
#include <stdint.h>
#include <omp.h>

static inline float softplus_f(float x) { return x > 20.0f ? x : log1pf(expf(x)); }

void oracle_selective_scan_omp(int64_t Bt, int64_t L, int64_t Dd, int64_t N, int delta_softplus,
                               const float* u, const float* delta, const float* A,
                               const float* Bm, const float* Cm, const float* D, const float* z,
                               const float* dt_bias, float* out, int threads) {
    if (threads > 0) omp_set_num_threads(threads);
#pragma omp parallel for schedule(static)
    for (int64_t row = 0; row < Bt * Dd; ++row) {
        const int64_t b = row / Dd, d = row % Dd;
        float h[256];
        for (int64_t n = 0; n < N; ++n) h[n] = 0.0f;
        for (int64_t t = 0; t < L; ++t) {
            const int64_t i = (b * L + t) * Dd + d;
            float dl = delta[i] + (dt_bias ? dt_bias[d] : 0.0f);
            if (delta_softplus) dl = softplus_f(dl);
            const float du = dl * u[i];
            float y = 0.0f;
            for (int64_t n = 0; n < N; ++n) {
                const float ab = expf(dl * A[d * N + n]);
                h[n] = ab * h[n] + du * Bm[(b * L + t) * N + n];
                y += Cm[(b * L + t) * N + n] * h[n];
            }
            if (D) y += D[d] * u[i];
            if (z) y *= z[i] / (1.0f + expf(-z[i]));
            out[i] = y;
        }
    }
}

int oracle_max_threads(void) { return omp_get_max_threads(); }

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

/* oracle_s4_ref_fwd (hx_oracle.c, the reference's S4Block::forward_ssm order,
 * crates/nn/src/ssm.rs:138-186) with the two O(L*M*N) phases spread over threads: every value is
 * computed by the same f32 operations in the same order as the sequential function, so the result
 * is bit-identical to it. Phase 1 (parallel over t): U[t][n] = sum_m (B[n][m]*dt) * x[m][t],
 * m ascending. Phase 2 (sequential): h = a*h + U[t]. Phase 3 (parallel over t):
 * y[t][m] = (sum_n C[m][n] * h_t[n]) + D[m]*x[m][t] (then * gate[m]). U and H: L*N floats each,
 * caller-owned. */
void oracle_s4_ref_fwd_omp(int64_t M, int64_t N, int64_t L, float dt, const float* x,
                           const float* a_real, const float* a_imag, const float* B, const float* C,
                           const float* D, const float* gate, float* y, float* U, float* H,
                           int threads) {
    if (threads > 0) omp_set_num_threads(threads);
    float a[256];
    for (int64_t n = 0; n < N; ++n) {
        float tr = a_real[n] * dt;
        float ti = a_imag[n] * dt;
        float er = expf(tr);
        float ci = cosf(ti);
        a[n] = er * ci;
    }
#pragma omp parallel for schedule(static)
    for (int64_t t = 0; t < L; ++t) {
        for (int64_t n = 0; n < N; ++n) {
            float sum = 0.0f;
            for (int64_t m = 0; m < M; ++m) {
                float bd = B[n * M + m] * dt;
                sum += bd * x[m * L + t];
            }
            U[t * N + n] = sum;
        }
    }
    float h[256];
    for (int64_t n = 0; n < N; ++n) h[n] = 0.0f;
    for (int64_t t = 0; t < L; ++t)
        for (int64_t n = 0; n < N; ++n) {
            float s1 = a[n] * h[n];
            h[n] = s1 + U[t * N + n];
            H[t * N + n] = h[n];
        }
#pragma omp parallel for schedule(static)
    for (int64_t t = 0; t < L; ++t) {
        for (int64_t m = 0; m < M; ++m) {
            float o = 0.0f;
            for (int64_t n = 0; n < N; ++n) o += C[m * N + n] * H[t * N + n];
            float fe = D[m] * x[m * L + t];
            float v = o + fe;
            if (gate) v = v * gate[m];
            y[t * M + m] = v;
        }
    }
}

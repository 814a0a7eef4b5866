/*
 * hx_oracle_omp.c — multi-threaded CPU kernels, the "optimised host" ("(O)") baseline.
 *
 * TEST/BENCH INFRASTRUCTURE ONLY (bench.py's cpu_baseline leg and tests/): never linked into or
 * called by the product library.
 *
 * Every function here computes the same f32 operations in the same order as its sequential
 * counterpart in hx_oracle.c, so its outputs are bit-identical to that function's (checked in
 * tests/test_oracle.py); only the schedule differs:
 *   - the scans run OpenMP tasks over (batch, block of 16 channels); a task walks time once and
 *     updates its 16 channels per step, so each step touches one 64-byte line per stream instead
 *     of one line per channel;
 *   - linear is a blocked product over a packed transpose of the weight (the copy Linear::forward
 *     makes, crates/nn/src/lib.rs:120-134): a tile of RB rows x JB columns accumulates in L1 with
 *     k ascending, the inner loop over columns vectorises without reassociating any sum, and a
 *     vector-ISA clone is chosen at load time (target_clones);
 *   - conv1d, rmsnorm: independent rows spread over threads.
 * s4d_complex_omp is the one exception: it is the f32 form of the f64 checker oracle_s4d_complex
 * (the GPU computes in f32), within rounding of it.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>
#include <omp.h>

static inline float softplus_f(float x) { return x > 20.0f ? x : log1pf(expf(x)); }
static inline float silu_f(float x) { return x / (1.0f + expf(-x)); }

static void set_threads(int threads) {
    if (threads > 0) omp_set_num_threads(threads);
}

int oracle_max_threads(void) { return omp_get_max_threads(); }

enum { CB = 16 };  /* channels per scan task: one 64-byte line of f32 */

/* oracle_selective_scan (hx_oracle.c; Gu & Dao 2023 Alg. 2 with the reference's discretisation,
 * crates/nn/src/ssm.rs:108-130), per channel the identical operation sequence. init_state and
 * last_state [Bt, Dd, N] are nullable; N <= 256. */
void oracle_selective_scan_omp(int64_t Bt, int64_t L, int64_t Dd, int64_t N, int delta_softplus,
                               const float* u, const float* delta, const float* A,
                               const float* Bm, const float* Cm, const float* D, const float* z,
                               const float* dt_bias, float* out, const float* init_state,
                               float* last_state, int threads) {
    set_threads(threads);
    const int64_t nblk = (Dd + CB - 1) / CB;
#pragma omp parallel for schedule(dynamic, 1)
    for (int64_t task = 0; task < Bt * nblk; ++task) {
        const int64_t b = task / nblk, d0 = (task % nblk) * CB;
        const int64_t nc = Dd - d0 < CB ? Dd - d0 : CB;
        float h[CB][256];
        for (int64_t c = 0; c < nc; ++c)
            for (int64_t n = 0; n < N; ++n)
                h[c][n] = init_state ? init_state[(b * Dd + d0 + c) * N + n] : 0.0f;
        for (int64_t t = 0; t < L; ++t) {
            const float* bt = Bm + (b * L + t) * N;
            const float* ct = Cm + (b * L + t) * N;
            for (int64_t c = 0; c < nc; ++c) {
                const int64_t d = d0 + c, i = (b * L + t) * Dd + d;
                float dl = delta[i] + (dt_bias ? dt_bias[d] : 0.0f);
                if (delta_softplus) dl = softplus_f(dl);
                const float du = dl * u[i];
                float y = 0.0f;
                for (int64_t n = 0; n < N; ++n) {
                    const float ab = expf(dl * A[d * N + n]);
                    h[c][n] = ab * h[c][n] + du * bt[n];
                    y += ct[n] * h[c][n];
                }
                if (D) y += D[d] * u[i];
                if (z) y *= silu_f(z[i]);
                out[i] = y;
            }
        }
        if (last_state)
            for (int64_t c = 0; c < nc; ++c)
                for (int64_t n = 0; n < N; ++n) last_state[(b * Dd + d0 + c) * N + n] = h[c][n];
    }
}

/* oracle_selective_state_update: one step of the scan, state [Bt, Dd, N] updated in place. */
void oracle_selective_state_update_omp(int64_t Bt, int64_t Dd, int64_t N, int delta_softplus,
                                       float* state, const float* u, const float* delta,
                                       const float* A, const float* Bm, const float* Cm,
                                       const float* D, const float* z, const float* dt_bias,
                                       float* out, int threads) {
    oracle_selective_scan_omp(Bt, 1, Dd, N, delta_softplus, u, delta, A, Bm, Cm, D, z, dt_bias,
                              out, state, state, threads);
}

/* ---------------------------------------------------------------- linear (X . W^T + bias) */

enum { RB = 4, JB = 64 };

/* One RB x JB tile (rows <= RB, cols <= JB) of Y = act(X . Wt + bias): for every output the sum
 * starts at 0 and adds X[r][k] * Wt[k][j] for k ascending, then the bias, then silu (act = 1),
 * exactly as oracle_linear. X points at the tile's first row (row stride IN), Wt, bias and Y at
 * its first column (row strides OUT). */
__attribute__((target_clones("avx512f", "avx2", "default")))
static void linear_tile(int64_t rows, int64_t cols, int64_t IN, int64_t OUT, const float* X,
                        const float* Wt, const float* bias, int act, float* Y) {
    float acc[RB][JB];
    memset(acc, 0, sizeof(acc));
    if (rows == RB && cols == JB) {
        for (int64_t k = 0; k < IN; ++k) {
            const float* w = Wt + k * OUT;
            for (int r = 0; r < RB; ++r) {
                const float a = X[r * IN + k];
                for (int j = 0; j < JB; ++j) acc[r][j] += a * w[j];
            }
        }
    } else {
        for (int64_t k = 0; k < IN; ++k) {
            const float* w = Wt + k * OUT;
            for (int64_t r = 0; r < rows; ++r) {
                const float a = X[r * IN + k];
                for (int64_t j = 0; j < cols; ++j) acc[r][j] += a * w[j];
            }
        }
    }
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t j = 0; j < cols; ++j) {
            const float v = bias ? acc[r][j] + bias[j] : acc[r][j];
            Y[r * OUT + j] = act == 1 ? silu_f(v) : v;
        }
}

/* oracle_linear (nn::Linear::forward, crates/nn/src/lib.rs:120-134): X [R, IN], W [OUT, IN],
 * bias [OUT] nullable, Y [R, OUT]. Wt: caller scratch of IN*OUT floats for the packed
 * transpose. */
void oracle_linear_omp(int64_t R, int64_t IN, int64_t OUT, const float* X, const float* W,
                       const float* bias, int act, float* Y, float* Wt, int threads) {
    set_threads(threads);
#pragma omp parallel for schedule(static)
    for (int64_t k = 0; k < IN; ++k)
        for (int64_t o = 0; o < OUT; ++o) Wt[k * OUT + o] = W[o * IN + k];
    const int64_t nr = (R + RB - 1) / RB, nc = (OUT + JB - 1) / JB;
    /* column blocks outermost: consecutive tiles of a thread share one packed panel */
#pragma omp parallel for schedule(static)
    for (int64_t tile = 0; tile < nr * nc; ++tile) {
        const int64_t jb = tile / nr, ib = tile % nr;
        const int64_t r0 = ib * RB, j0 = jb * JB;
        const int64_t rows = R - r0 < RB ? R - r0 : RB, cols = OUT - j0 < JB ? OUT - j0 : JB;
        linear_tile(rows, cols, IN, OUT, X + r0 * IN, Wt + j0, bias ? bias + j0 : 0, act,
                    Y + r0 * OUT + j0);
    }
}

/* ---------------------------------------------------------------- row-parallel pieces */

/* oracle_conv1d_silu: causal depthwise conv + bias + SiLU, rows (b, t) over threads. */
void oracle_conv1d_silu_omp(int64_t Bt, int64_t L, int64_t Dd, int64_t W, const float* x,
                            int64_t ldx, const float* w, const float* bias, float* y, int threads) {
    set_threads(threads);
#pragma omp parallel for schedule(static)
    for (int64_t row = 0; row < Bt * L; ++row) {
        const int64_t b = row / L, t = row % L;
        for (int64_t d = 0; d < Dd; ++d) {
            float acc = bias ? bias[d] : 0.0f;
            for (int64_t j = 0; j < W; ++j) {
                const int64_t tt = t - (W - 1) + j;
                if (tt < 0) continue;
                acc += w[d * W + j] * x[(b * L + tt) * ldx + d];
            }
            y[row * Dd + d] = silu_f(acc);
        }
    }
}

/* oracle_rmsnorm (nn::RMSNorm::forward, crates/nn/src/lib.rs:258-285), rows over threads. */
void oracle_rmsnorm_omp(int64_t R, int64_t Dm, const float* X, const float* w, float eps, float* Y,
                        int threads) {
    set_threads(threads);
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < R; ++r) {
        float s = 0.0f;
        for (int64_t j = 0; j < Dm; ++j) s += X[r * Dm + j] * X[r * Dm + j];
        const float ms = s / (float)Dm;
        const float rms = sqrtf(ms + eps);
        for (int64_t j = 0; j < Dm; ++j) Y[r * Dm + j] = (X[r * Dm + j] / rms) * w[j];
    }
}

/* ---------------------------------------------------------------- S4D complex, f32 */

/* The diagonal complex S4D recurrence of oracle_s4d_complex (Gu, Goel, Gupta, Re 2022; the
 * reference's discretisation Abar = exp(dt*A) complex, Bbar = dt*B, crates/nn/src/ssm.rs:108-130)
 * in f32 arithmetic: y = 2*Re(sum_n C_n h_n) + D*x. x, y [Bt, L, Dd]; per-channel parameters
 * [Dd, N]; N <= 256. */
void oracle_s4d_complex_omp(int64_t Bt, int64_t L, int64_t Dd, int64_t N, const float* x,
                            const float* dt, const float* a_re, const float* a_im,
                            const float* B_re, const float* B_im, const float* C_re,
                            const float* C_im, const float* D, float* y, int threads) {
    set_threads(threads);
    const int64_t nblk = (Dd + CB - 1) / CB;
#pragma omp parallel for schedule(dynamic, 1)
    for (int64_t task = 0; task < Bt * nblk; ++task) {
        const int64_t b = task / nblk, d0 = (task % nblk) * CB;
        const int64_t nc = Dd - d0 < CB ? Dd - d0 : CB;
        float hr[CB][256], hi[CB][256], ar[CB][256], ai[CB][256], br[CB][256], bi[CB][256];
        for (int64_t c = 0; c < nc; ++c) {
            const int64_t d = d0 + c;
            const float dtd = dt[d];
            for (int64_t n = 0; n < N; ++n) {
                const float mag = expf(dtd * a_re[d * N + n]);
                ar[c][n] = mag * cosf(dtd * a_im[d * N + n]);
                ai[c][n] = mag * sinf(dtd * a_im[d * N + n]);
                br[c][n] = dtd * B_re[d * N + n];
                bi[c][n] = dtd * B_im[d * N + n];
                hr[c][n] = hi[c][n] = 0.0f;
            }
        }
        for (int64_t t = 0; t < L; ++t)
            for (int64_t c = 0; c < nc; ++c) {
                const int64_t d = d0 + c, i = (b * L + t) * Dd + d;
                const float u = x[i];
                float acc = 0.0f;
                for (int64_t n = 0; n < N; ++n) {
                    const float nr = ar[c][n] * hr[c][n] - ai[c][n] * hi[c][n] + br[c][n] * u;
                    const float ni = ar[c][n] * hi[c][n] + ai[c][n] * hr[c][n] + bi[c][n] * u;
                    hr[c][n] = nr;
                    hi[c][n] = ni;
                    acc += C_re[d * N + n] * nr - C_im[d * N + n] * ni;
                }
                y[i] = 2.0f * acc + (D ? D[d] * u : 0.0f);
            }
    }
}

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
    set_threads(threads);
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

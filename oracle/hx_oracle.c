/*
 * hx_oracle.c — CPU oracle for HelixML's SSM forward path.
 *
 * TEST INFRASTRUCTURE ONLY. This file is the checker, never the product: only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load liboracle.so. The product
 * path (libhelix_hip.so) does not link, call or fall back to it.
 *
 * It restates, in plain C, the arithmetic of the reference's CPU path (HelixML, Rust, CpuTensor
 * over ndarray f32) with the same loop orders and f32 accumulation, and the textbook selective
 * scan the reference lacks. Built with -O2 -ffp-contract=off (no FMA contraction, like rustc's
 * default) so op order is the reference's. Rust's f32::{exp,cos,sin} lower to libm's
 * expf/cosf/sinf, which is what this file calls.
 *
 * Pins (tests/test_oracle.py): every function here is checked against the reference's own
 * known-answer tests where they exist (ones.ones KATs, backend-cpu/src/lib.rs:1733-1758), against
 * closed forms (zero input, impulse and step responses, prefix sums, geometric series,
 * steady states), invariants (linearity, chunked == sequential, decode == prefill) and an
 * independent float64 numpy restatement.
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* ---------------------------------------------------------------- CpuTensor primitives */

/* CpuTensor::matmul 2-D x 2-D (backend-cpu/src/lib.rs:644-678): ijk order, f32 sum from 0.0,
 * k ascending, `sum += a*b` (lib.rs:659-667). */
void oracle_matmul(int64_t M, int64_t K, int64_t N, const float* A, const float* B, float* Y) {
    for (int64_t i = 0; i < M; ++i)
        for (int64_t j = 0; j < N; ++j) {
            float sum = 0.0f;
            for (int64_t k = 0; k < K; ++k) sum += A[i * K + k] * B[k * N + j];
            Y[i * N + j] = sum;
        }
}

/* CpuTensor::silu (backend-cpu/src/lib.rs:1154-1170): x / (1 + exp(-x)). */
static inline float silu_ref(float x) { return x / (1.0f + expf(-x)); }

void oracle_silu(int64_t n, const float* x, float* y) {
    for (int64_t i = 0; i < n; ++i) y[i] = silu_ref(x[i]);
}

/* nn::Linear::forward (crates/nn/src/lib.rs:120-134): input.matmul(weight.transpose(0,1))
 * then add(bias.broadcast_to(out_shape)) (repeat-rows broadcast, backend-cpu lib.rs:1388-1404).
 * W is [out, in]; the transpose copy holds Wt[k][o] = W[o][k], which the ijk matmul reads in
 * the same k order. act = 1 applies CpuTensor::silu to the result. */
void oracle_linear(int64_t R, int64_t IN, int64_t OUT, const float* X, const float* W,
                   const float* bias, int act, float* Y) {
    for (int64_t r = 0; r < R; ++r)
        for (int64_t o = 0; o < OUT; ++o) {
            float sum = 0.0f;
            for (int64_t k = 0; k < IN; ++k) sum += X[r * IN + k] * W[o * IN + k];
            float v = bias ? sum + bias[o] : sum;
            Y[r * OUT + o] = act == 1 ? silu_ref(v) : v;
        }
}

/* Exported nn::MambaBlock::forward_mamba (crates/nn/src/lib.rs:888-906):
 * Y = Linear_out(silu(Linear_gate(X))). X [R, d_model], Wg [d_inner, d_model],
 * Wo [d_model, d_inner]. tmp must hold R*d_inner floats. */
void oracle_mamba_mlp(int64_t R, int64_t d_model, int64_t d_inner, const float* X,
                      const float* Wg, const float* bg, const float* Wo, const float* bo,
                      float* tmp, float* Y) {
    oracle_linear(R, d_model, d_inner, X, Wg, bg, 1, tmp);
    oracle_linear(R, d_inner, d_model, tmp, Wo, bo, 0, Y);
}

/* nn::RMSNorm::forward (crates/nn/src/lib.rs:258-285): ms = mean(x*x, last dim);
 * y = x / sqrt(ms + eps) * w. The reference draws eps' ~ U[eps, eps+1e-8) per row (lib.rs:262);
 * the oracle uses eps' = eps (the perturbation is below f32 resolution of ms+eps for the
 * magnitudes the path sees). The mean is sum-then-divide in f32 (ndarray mean_axis). */
void oracle_rmsnorm(int64_t R, int64_t Dm, const float* X, const float* w, float eps, float* Y) {
    for (int64_t r = 0; r < R; ++r) {
        float s = 0.0f;
        for (int64_t j = 0; j < Dm; ++j) s += X[r * Dm + j] * X[r * Dm + j];
        float ms = s / (float)Dm;
        float rms = sqrtf(ms + eps);
        for (int64_t j = 0; j < Dm; ++j) Y[r * Dm + j] = (X[r * Dm + j] / rms) * w[j];
    }
}

/* ---------------------------------------------------------------- S4 (reference mode) */

/* nn::ssm::S4Block::discretize (crates/nn/src/ssm.rs:103-135) + forward_ssm (ssm.rs:138-186),
 * exact f32 op order:
 *   tr = a_real*dt; ti = a_imag*dt (mul_scalar, ssm.rs:113-114); a = expf(tr)*cosf(ti)
 *   (ssm.rs:116-120); Bd = B*dt (ssm.rs:130); h = 0 (ssm.rs:162); per t (ssm.rs:166-182):
 *   s1 = a*h; s2[n] = sum_m Bd[n][m]*u[m] (2-D x 1-D matmul, backend-cpu lib.rs:728-735);
 *   h = s1 + s2; o[m] = sum_n C[m][n]*h[n]; y[t][m] = o[m] + D[m]*u[m].
 * x [M, L] row-major; y memory [L, M] (stack(.,1), backend-cpu lib.rs:277-296).
 * gate (nullable): y[t][m] *= gate[m] (nn::ssm::MambaBlock gating, ssm.rs:460-461).
 * work must hold 3*N + M floats. */
void oracle_s4_ref_fwd(int64_t M, int64_t N, int64_t L, float dt, const float* x,
                       const float* a_real, const float* a_imag, const float* B, const float* C,
                       const float* D, const float* gate, float* y, float* work) {
    float* a = work;
    float* h = work + N;
    float* s2 = work + 2 * N;
    float* u = work + 3 * N;
    for (int64_t n = 0; n < N; ++n) {
        float tr = a_real[n] * dt;
        float ti = a_imag[n] * dt;
        float er = expf(tr);
        float ci = cosf(ti);
        a[n] = er * ci;
        h[n] = 0.0f;
    }
    for (int64_t t = 0; t < L; ++t) {
        for (int64_t m = 0; m < M; ++m) u[m] = x[m * L + t];
        for (int64_t n = 0; n < N; ++n) {
            float sum = 0.0f;
            for (int64_t m = 0; m < M; ++m) {
                float bd = B[n * M + m] * dt;
                sum += bd * u[m];
            }
            s2[n] = sum;
        }
        for (int64_t n = 0; n < N; ++n) {
            float s1 = a[n] * h[n];
            h[n] = s1 + s2[n];
        }
        for (int64_t m = 0; m < M; ++m) {
            float o = 0.0f;
            for (int64_t n = 0; n < N; ++n) o += C[m * N + n] * h[n];
            float fe = D[m] * u[m];
            float v = o + fe;
            if (gate) v = v * gate[m];
            y[t * M + m] = v;
        }
    }
}

/* oracle_s4_ref_fwd with every operation in double (inputs read as f32, dt widened): the exact
 * value the f32 restatement approximates. Used where the f32 path's own rounding (sequential
 * 2048-term sums, |a| ~ 1 recurrences) is comparable to the tolerance. work: 3N + M doubles. */
void oracle_s4_ref_fwd_f64(int64_t M, int64_t N, int64_t L, float dt, const float* x,
                           const float* a_real, const float* a_imag, const float* B,
                           const float* C, const float* D, const float* gate, double* y,
                           double* work) {
    double* a = work;
    double* h = work + N;
    double* s2 = work + 2 * N;
    double* u = work + 3 * N;
    const double dtd = dt;
    for (int64_t n = 0; n < N; ++n) {
        a[n] = exp(a_real[n] * dtd) * cos(a_imag[n] * dtd);
        h[n] = 0.0;
    }
    for (int64_t t = 0; t < L; ++t) {
        for (int64_t m = 0; m < M; ++m) u[m] = x[m * L + t];
        for (int64_t n = 0; n < N; ++n) {
            double sum = 0.0;
            for (int64_t m = 0; m < M; ++m) sum += B[n * M + m] * dtd * u[m];
            s2[n] = sum;
        }
        for (int64_t n = 0; n < N; ++n) h[n] = a[n] * h[n] + s2[n];
        for (int64_t m = 0; m < M; ++m) {
            double o = 0.0;
            for (int64_t n = 0; n < N; ++n) o += C[m * N + n] * h[n];
            double v = o + D[m] * u[m];
            if (gate) v *= gate[m];
            y[t * M + m] = v;
        }
    }
}

/* nn::ssm::MambaBlock::forward_mamba (crates/nn/src/ssm.rs:435-464) for X [M, M]:
 * conv1d is identity (ssm.rs:467-471); delta = X.delta_proj (ssm.rs:450); X.B_proj and X.C_proj
 * are computed and discarded by selective_ssm (ssm.rs:453-454, 474-483), so they are skipped;
 * y = S4Block::forward_ssm(delta) (ssm.rs:482); out = y * broadcast(gate) (ssm.rs:460-461).
 * work must hold M*M + 3*N + M floats. */
void oracle_ssm_mamba_fwd(int64_t M, int64_t N, float dt, const float* X, const float* delta_proj,
                          const float* a_real, const float* a_imag, const float* B,
                          const float* C, const float* D, const float* gate, float* y,
                          float* work) {
    float* delta = work;
    oracle_matmul(M, M, M, X, delta_proj, delta);
    oracle_s4_ref_fwd(M, N, M, dt, delta, a_real, a_imag, B, C, D, gate, y, work + M * M);
}

/* ---------------------------------------------------------------- selective scan */

/* softplus(x) = log(1 + exp(x)); for x > 20 it returns x (exp(x) > 4.8e8, so log1p(exp(x)) - x
 * < 2.1e-9, below f32 resolution of x). */
static inline float softplus_f(float x) { return x > 20.0f ? x : log1pf(expf(x)); }
static inline double softplus_d(double x) { return x > 20.0 ? x : log1p(exp(x)); }

/* Textbook selective scan (Gu & Dao 2023, arXiv:2312.00752, Alg. 2 / Sec. 3), with the
 * reference's own discretisation choices: Abar = exp(dt*A) (ssm.rs:108-116), Bbar = dt*B
 * (ssm.rs:127-130), and its SiLU (backend-cpu lib.rs:1158-1162). Recurrence skeleton as
 * ssm.rs:166-182 but per channel. f32 arithmetic, state in f32.
 * Layout: u, delta, z, out [Bt, L, Dd]; Bm, Cm [Bt, L, N]; A [Dd, N]; D, dt_bias [Dd];
 * init_state, last_state [Bt, Dd, N] (nullable). */
void oracle_selective_scan(int64_t Bt, int64_t L, int64_t Dd, int64_t N, int delta_softplus,
                           const float* u, const float* delta, const float* A, const float* Bm,
                           const float* Cm, const float* D, const float* z,
                           const float* dt_bias, float* out, const float* init_state,
                           float* last_state) {
    float h[256];
    for (int64_t b = 0; b < Bt; ++b)
        for (int64_t d = 0; d < Dd; ++d) {
            for (int64_t n = 0; n < N; ++n) h[n] = init_state ? init_state[(b * Dd + d) * N + n] : 0.0f;
            for (int64_t t = 0; t < L; ++t) {
                int64_t i = (b * L + t) * Dd + d;
                float dl = delta[i] + (dt_bias ? dt_bias[d] : 0.0f);
                if (delta_softplus) dl = softplus_f(dl);
                float du = dl * u[i];
                float y = 0.0f;
                for (int64_t n = 0; n < N; ++n) {
                    float ab = expf(dl * A[d * N + n]);
                    h[n] = ab * h[n] + du * Bm[(b * L + t) * N + n];
                    y += Cm[(b * L + t) * N + n] * h[n];
                }
                if (D) y += D[d] * u[i];
                if (z) y *= silu_ref(z[i]);
                out[i] = y;
            }
            if (last_state)
                for (int64_t n = 0; n < N; ++n) last_state[(b * Dd + d) * N + n] = h[n];
        }
}

/* Same as oracle_selective_scan with every operation in double (inputs read as f32). The
 * f32 oracle and the GPU path are both compared against this where accumulated rounding
 * matters (long sequences). */
void oracle_selective_scan_f64(int64_t Bt, int64_t L, int64_t Dd, int64_t N, int delta_softplus,
                               const float* u, const float* delta, const float* A,
                               const float* Bm, const float* Cm, const float* D, const float* z,
                               const float* dt_bias, double* out, const float* init_state,
                               double* last_state) {
    double h[256];
    for (int64_t b = 0; b < Bt; ++b)
        for (int64_t d = 0; d < Dd; ++d) {
            for (int64_t n = 0; n < N; ++n) h[n] = init_state ? init_state[(b * Dd + d) * N + n] : 0.0;
            for (int64_t t = 0; t < L; ++t) {
                int64_t i = (b * L + t) * Dd + d;
                double dl = (double)delta[i] + (dt_bias ? (double)dt_bias[d] : 0.0);
                if (delta_softplus) dl = softplus_d(dl);
                double du = dl * (double)u[i];
                double y = 0.0;
                for (int64_t n = 0; n < N; ++n) {
                    double ab = exp(dl * (double)A[d * N + n]);
                    h[n] = ab * h[n] + du * (double)Bm[(b * L + t) * N + n];
                    y += (double)Cm[(b * L + t) * N + n] * h[n];
                }
                if (D) y += (double)D[d] * (double)u[i];
                if (z) { double zz = z[i]; y *= zz / (1.0 + exp(-zz)); }
                out[i] = y;
            }
            if (last_state)
                for (int64_t n = 0; n < N; ++n) last_state[(b * Dd + d) * N + n] = h[n];
        }
}

/* One decode step: the body of oracle_selective_scan at a single t, updating state in place.
 * u, delta, z, out [Bt, Dd]; Bm, Cm [Bt, N]; state [Bt, Dd, N]. */
void oracle_selective_state_update(int64_t Bt, int64_t Dd, int64_t N, int delta_softplus,
                                   float* state, const float* u, const float* delta,
                                   const float* A, const float* Bm, const float* Cm,
                                   const float* D, const float* z, const float* dt_bias,
                                   float* out) {
    oracle_selective_scan(Bt, 1, Dd, N, delta_softplus, u, delta, A, Bm, Cm, D, z, dt_bias, out,
                          state, state);
}

/* ---------------------------------------------------------------- S4D complex */

/* Diagonal complex S4D recurrence (Gu, Goel, Gupta, Re 2022, arXiv:2206.11893), with the
 * reference's discretisation choices: Abar = exp(dt*A) complex (ssm.rs:108-121 keeps both
 * exp(dt*Re)cos(dt*Im) and exp(dt*Re)sin(dt*Im)), Bbar = dt*B (ssm.rs:127-130).
 * y = 2*Re(sum_n C_n h_n) + D*x. Double precision internally (it is the checker). */
void oracle_s4d_complex(int64_t Bt, int64_t L, int64_t Dd, int64_t N, const float* x,
                        const float* dt, const float* a_re, const float* a_im,
                        const float* B_re, const float* B_im, const float* C_re,
                        const float* C_im, const float* D, double* y) {
    double hr[256], hi[256], ar[256], ai[256], br[256], bi[256];
    for (int64_t b = 0; b < Bt; ++b)
        for (int64_t d = 0; d < Dd; ++d) {
            double dtd = dt[d];
            for (int64_t n = 0; n < N; ++n) {
                double mag = exp(dtd * a_re[d * N + n]);
                ar[n] = mag * cos(dtd * a_im[d * N + n]);
                ai[n] = mag * sin(dtd * a_im[d * N + n]);
                br[n] = dtd * B_re[d * N + n];
                bi[n] = dtd * B_im[d * N + n];
                hr[n] = hi[n] = 0.0;
            }
            for (int64_t t = 0; t < L; ++t) {
                int64_t i = (b * L + t) * Dd + d;
                double u = x[i], acc = 0.0;
                for (int64_t n = 0; n < N; ++n) {
                    double nr = ar[n] * hr[n] - ai[n] * hi[n] + br[n] * u;
                    double ni = ar[n] * hi[n] + ai[n] * hr[n] + bi[n] * u;
                    hr[n] = nr; hi[n] = ni;
                    acc += C_re[d * N + n] * nr - C_im[d * N + n] * ni;
                }
                y[i] = 2.0 * acc + (D ? (double)D[d] * u : 0.0);
            }
        }
}

/* ---------------------------------------------------------------- Mamba block pieces */

/* Causal depthwise conv1d over time + bias + SiLU, the block's short convolution (Gu & Dao 2023,
 * Fig. 3; the reference allocates d_conv but never convolves, nn/src/lib.rs:847-885).
 * y[b,t,d] = silu(bias[d] + sum_{j<W} w[d,j] * x[b, t-W+1+j, d]), zero for t-W+1+j < 0;
 * j ascending, f32. x row stride ldx (elements), y contiguous [Bt, L, Dd]. */
void oracle_conv1d_silu(int64_t Bt, int64_t L, int64_t Dd, int64_t W, const float* x, int64_t ldx,
                        const float* w, const float* bias, float* y) {
    for (int64_t b = 0; b < Bt; ++b)
        for (int64_t t = 0; t < L; ++t)
            for (int64_t d = 0; d < Dd; ++d) {
                float acc = bias ? bias[d] : 0.0f;
                for (int64_t j = 0; j < W; ++j) {
                    int64_t tt = t - (W - 1) + j;
                    if (tt < 0) continue;
                    acc += w[d * W + j] * x[(b * L + tt) * ldx + d];
                }
                y[(b * L + t) * Dd + d] = silu_ref(acc);
            }
}

/* ---------------------------------------------------------------- tensor primitives */

/* CpuTensor's elementwise maps (backend-cpu/src/lib.rs): op codes of include/helix_hip.h's
 * hx_unary_op. Rust's f32::{exp, ln, sin, cos, sqrt, abs} lower to libm's expf/logf/sinf/cosf and
 * the correctly rounded square root; silu = x / (1 + exp(-x)) (lib.rs:1158-1162), sigmoid =
 * 1 / (1 + exp(-x)) (lib.rs:1172-1178). */
void oracle_unary(int op, int64_t n, const float* x, float s, float* y) {
    for (int64_t i = 0; i < n; ++i) {
        const float v = x[i];
        float r;
        switch (op) {
            case 0: r = expf(v); break;
            case 1: r = cosf(v); break;
            case 2: r = sinf(v); break;
            case 3: r = sqrtf(v); break;
            case 4: r = v / (1.0f + expf(-v)); break;
            case 5: r = -v; break;
            case 6: r = v * s; break;
            case 7: r = v + s; break;
            case 8: r = fabsf(v); break;
            case 9: r = logf(v); break;
            default: r = 1.0f / (1.0f + expf(-v)); break;
        }
        y[i] = r;
    }
}

/* ndarray 0.15's unrolled fold over a contiguous slice (numeric_util::unrolled_fold, what
 * ArrayBase::sum uses for a contiguous lane): eight partial sums p_k over elements i = k mod 8
 * of the first 8*floor(n/8), acc = 0 + (p0+p4), + (p1+p5), + (p2+p6), + (p3+p7), then the
 * n mod 8 trailing elements in order. */
static float unrolled_sum(const float* x, int64_t n) {
    float p[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    const int64_t body = n / 8 * 8;
    for (int64_t i = 0; i < body; i += 8)
        for (int k = 0; k < 8; ++k) p[k] = p[k] + x[i + k];
    float acc = 0.0f;
    acc = acc + (p[0] + p[4]);
    acc = acc + (p[1] + p[5]);
    acc = acc + (p[2] + p[6]);
    acc = acc + (p[3] + p[7]);
    for (int64_t i = body; i < n; ++i) acc = acc + x[i];
    return acc;
}

/* TensorReduce::mean over one axis (backend-cpu/src/lib.rs:995-1010 -> ndarray mean_axis =
 * sum_axis / len) of x viewed as [outer, len, inner]. ndarray's sum_axis sums each lane with the
 * unrolled fold when the axis is the array's minimum-stride axis (lane_fold = 1, inner == 1),
 * else adds the len sub-views in axis order from zero. */
void oracle_mean_axis(int64_t outer, int64_t len, int64_t inner, int lane_fold, const float* x,
                      float* y) {
    for (int64_t o = 0; o < outer; ++o) {
        if (lane_fold) {
            y[o] = unrolled_sum(x + o * len, len) / (float)len;
            continue;
        }
        for (int64_t i = 0; i < inner; ++i) {
            float acc = 0.0f;
            for (int64_t l = 0; l < len; ++l) acc = acc + x[(o * len + l) * inner + i];
            y[o * inner + i] = acc / (float)len;
        }
    }
}

/* nn::RMSNorm::forward (crates/nn/src/lib.rs:258-285) as its primitives compute it, with
 * eps' = eps: ms = mean(x*x, last axis) by the unrolled fold; rms = sqrt(ms + eps);
 * y = (x / rms) * w. (oracle_rmsnorm above sums the squares sequentially: the two differ by
 * rounding only.) */
void oracle_rmsnorm_ref(int64_t R, int64_t Dm, const float* X, const float* w, float eps, float* Y,
                        float* work) {
    for (int64_t r = 0; r < R; ++r) {
        for (int64_t j = 0; j < Dm; ++j) work[j] = X[r * Dm + j] * X[r * Dm + j];
        const float ms = unrolled_sum(work, Dm) / (float)Dm;
        const float rms = sqrtf(ms + eps);
        for (int64_t j = 0; j < Dm; ++j) Y[r * Dm + j] = (X[r * Dm + j] / rms) * w[j];
    }
}

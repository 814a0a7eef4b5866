/*
 * hx_oracle_ref.c — reference-faithful CPU timing restatement ("(R)") of HelixML's CpuTensor
 * path for the S4 recurrence and the exported Mamba MLP.
 *
 * TEST / BENCHMARK INFRASTRUCTURE ONLY: loaded by tests/ and by bench.py's cpu_baseline leg,
 * never by the product library.
 *
 * The arithmetic is hx_oracle.c's (the same f32 operations in the same order, so the outputs
 * are bit-identical to oracle_s4_ref_fwd / oracle_mamba_mlp; tests/test_oracle.py checks that).
 * What this file adds is the reference's execution shape: every tensor operation returns a
 * freshly allocated result, as CpuTensor's ndarray-backed ops do, and the per-step slice,
 * reshape and final stack are copies. It times what the reference's single-threaded CPU path
 * costs, op for op:
 *   S4Block::forward_ssm (crates/nn/src/ssm.rs:138-186): clone of the block (7 parameters,
 *     ssm.rs:150), discretize on the clone (mul_scalar x3, exp, cos, sin, mul x2, ssm.rs:113-130),
 *     state zeros (ssm.rs:162); per step: slice [M, t..t+1] (backend-cpu/src/lib.rs:139-183),
 *     reshape to [M] (lib.rs:94-113), A_d.mul(state), B_d.matmul(u) (2-D x 1-D, lib.rs:715-746),
 *     add, C.matmul(state), D.mul(u), add, push; then stack(outputs, 1) (lib.rs:254-296).
 *   nn::MambaBlock::forward_mamba (crates/nn/src/lib.rs:888-906) with Linear::forward
 *     (lib.rs:120-134): weight.transpose(0,1) (a copy, lib.rs:115-137), matmul (lib.rs:644-678),
 *     bias.broadcast_to (repeat rows, lib.rs:1388-1404), add, silu (lib.rs:1154-1170), Linear.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

static float* alloc_f(int64_t n) { return (float*)malloc((size_t)(n > 0 ? n : 1) * sizeof(float)); }
static float* clone_f(const float* p, int64_t n) {
    float* q = alloc_f(n);
    memcpy(q, p, (size_t)n * sizeof(float));
    return q;
}
static float* op_mul_scalar(const float* a, int64_t n, float s) {
    float* r = alloc_f(n);
    for (int64_t i = 0; i < n; ++i) r[i] = a[i] * s;
    return r;
}
static float* op_mul(const float* a, const float* b, int64_t n) {
    float* r = alloc_f(n);
    for (int64_t i = 0; i < n; ++i) r[i] = a[i] * b[i];
    return r;
}
static float* op_add(const float* a, const float* b, int64_t n) {
    float* r = alloc_f(n);
    for (int64_t i = 0; i < n; ++i) r[i] = a[i] + b[i];
    return r;
}
static float* op_map(const float* a, int64_t n, float (*f)(float)) {
    float* r = alloc_f(n);
    for (int64_t i = 0; i < n; ++i) r[i] = f(a[i]);
    return r;
}
/* 2-D [R, K] x 1-D [K] (backend-cpu lib.rs:715-746): f32 sum from 0, k ascending */
static float* op_matvec(const float* A, const float* v, int64_t R, int64_t K) {
    float* r = alloc_f(R);
    for (int64_t i = 0; i < R; ++i) {
        float sum = 0.0f;
        for (int64_t k = 0; k < K; ++k) sum += A[i * K + k] * v[k];
        r[i] = sum;
    }
    return r;
}
/* 2-D x 2-D, ijk (backend-cpu lib.rs:644-678) */
static float* op_matmul(const float* A, const float* B, int64_t M, int64_t K, int64_t N) {
    float* r = alloc_f(M * N);
    for (int64_t i = 0; i < M; ++i)
        for (int64_t j = 0; j < N; ++j) {
            float sum = 0.0f;
            for (int64_t k = 0; k < K; ++k) sum += A[i * K + k] * B[k * N + j];
            r[i * N + j] = sum;
        }
    return r;
}
static float silu_f(float x) { return x / (1.0f + expf(-x)); }

/* S4Block::forward_ssm, reference execution shape. x [M, L]; y memory [L, M]. The block's other
 * parameters (delta [M], Lambda [N]) are cloned with it, as ssm.rs:150 clones the whole block. */
void oracle_r_s4_forward_ssm(int64_t M, int64_t N, int64_t L, float dt, const float* x,
                             const float* a_real, const float* a_imag, const float* B,
                             const float* C, const float* D, const float* delta,
                             const float* lambda, float* y) {
    /* let mut self_mut = self.clone() */
    float* c_ar = clone_f(a_real, N);
    float* c_ai = clone_f(a_imag, N);
    float* c_B = clone_f(B, N * M);
    float* c_C = clone_f(C, M * N);
    float* c_D = clone_f(D, M);
    float* c_delta = clone_f(delta, M);
    float* c_lambda = clone_f(lambda, N);
    /* discretize(0.1) on the clone */
    float* dt_real = op_mul_scalar(c_ar, N, dt);
    float* dt_imag = op_mul_scalar(c_ai, N, dt);
    float* exp_real = op_map(dt_real, N, expf);
    float* cos_imag = op_map(dt_imag, N, cosf);
    float* sin_imag = op_map(dt_imag, N, sinf);
    float* A_d = op_mul(exp_real, cos_imag, N);
    float* A_d_imag = op_mul(exp_real, sin_imag, N); /* computed and dropped (ssm.rs:121-125) */
    float* B_d = op_mul_scalar(c_B, N * M, dt);
    /* state = zeros([N]); outputs = Vec::new() */
    float* state = alloc_f(N);
    memset(state, 0, (size_t)N * sizeof(float));
    float** outputs = (float**)malloc((size_t)(L > 0 ? L : 1) * sizeof(float*));
    for (int64_t t = 0; t < L; ++t) {
        float* sl = alloc_f(M); /* input.slice([0, t], [M, t + 1]): a copy of column t */
        for (int64_t m = 0; m < M; ++m) sl[m] = x[m * L + t];
        float* input_t = clone_f(sl, M); /* reshape([M]): a copy */
        free(sl);
        float* state_update = op_mul(A_d, state, N);
        float* input_contribution = op_matvec(B_d, input_t, N, M);
        float* new_state = op_add(state_update, input_contribution, N);
        free(state);
        state = new_state;
        float* output_t = op_matvec(c_C, state, M, N); /* self.C: the clone's, same values */
        float* feedthrough = op_mul(c_D, input_t, M);
        outputs[t] = op_add(output_t, feedthrough, M);
        free(state_update);
        free(input_contribution);
        free(output_t);
        free(feedthrough);
        free(input_t);
    }
    /* T::stack(outputs, 1): rows in time order */
    for (int64_t t = 0; t < L; ++t) {
        memcpy(y + t * M, outputs[t], (size_t)M * sizeof(float));
        free(outputs[t]);
    }
    free(outputs);
    free(state);
    free(dt_real); free(dt_imag); free(exp_real); free(cos_imag); free(sin_imag);
    free(A_d); free(A_d_imag); free(B_d);
    free(c_ar); free(c_ai); free(c_B); free(c_C); free(c_D); free(c_delta); free(c_lambda);
}

/* Linear::forward, reference execution shape: X [R, IN], W [OUT, IN], bias [OUT] (nullable). */
static float* r_linear(const float* X, const float* W, const float* bias, int64_t R, int64_t IN,
                       int64_t OUT) {
    float* Wt = alloc_f(IN * OUT); /* weight.transpose(0, 1) */
    for (int64_t o = 0; o < OUT; ++o)
        for (int64_t k = 0; k < IN; ++k) Wt[k * OUT + o] = W[o * IN + k];
    float* out = op_matmul(X, Wt, R, IN, OUT);
    free(Wt);
    if (!bias) return out;
    float* bb = alloc_f(R * OUT); /* bias.broadcast_to([R, OUT]): repeat rows */
    for (int64_t r = 0; r < R; ++r) memcpy(bb + r * OUT, bias, (size_t)OUT * sizeof(float));
    float* res = op_add(out, bb, R * OUT);
    free(out);
    free(bb);
    return res;
}

/* Linear::forward in the reference's execution shape, exported for the block and LM timing
 * legs: Y [R, OUT] = X . W^T (+ bias); same values as oracle_linear, bit for bit. */
void oracle_r_linear(int64_t R, int64_t IN, int64_t OUT, const float* X, const float* W,
                     const float* bias, float* Y) {
    float* o = r_linear(X, W, bias, R, IN, OUT);
    memcpy(Y, o, (size_t)(R * OUT) * sizeof(float));
    free(o);
}

/* nn::MambaBlock::forward_mamba (lib.rs:888-906): Y = out_proj(silu(gate(X))). */
void oracle_r_mamba_mlp(int64_t R, int64_t d_model, int64_t d_inner, const float* X,
                        const float* Wg, const float* bg, const float* Wo, const float* bo,
                        float* Y) {
    float* h = r_linear(X, Wg, bg, R, d_model, d_inner);
    float* s = op_map(h, R * d_inner, silu_f);
    float* o = r_linear(s, Wo, bo, R, d_inner, d_model);
    memcpy(Y, o, (size_t)(R * d_model) * sizeof(float));
    free(h);
    free(s);
    free(o);
}

// hx_s4.hip — S4 recurrences for gfx950.
//
// (1) Reference-mode S4Block::forward_ssm (crates/nn/src/ssm.rs:138-186): one state h[N] shared
//     by all d_model channels, constant diagonal decay a[n] = exp(dt*a_real)*cos(dt*a_imag)
//     (ssm.rs:113-120), Bd = dt*B (ssm.rs:130). It factors into three steps:
//       U[t][n] = sum_m Bd[n][m] * x[m][t]            (column reduction over channels)
//       H[t][n] = a[n]*H[t-1][n] + U[t][n]             (16 independent first-order recurrences)
//       y[t][m] = (sum_n C[m][n]*H[t][n] + D[m]*x[m][t]) * gate[m]
//     x is [d_model, L] (time contiguous) and y is [L, d_model] (channels contiguous), so the
//     output kernel transposes through LDS.
// (2) S4D diagonal complex recurrence, per channel.
#include "hx_common.h"

namespace hx {
namespace {

constexpr int kMaxState = 64;

// No multiply-add contraction anywhere in reference mode (hipcc defaults to contracting, and
// __fmul_rn/__fadd_rn are plain operators here).
#pragma clang fp contract(off)

// Reference mode reproduces the reference's f32 operation order exactly, so its output is
// bit-identical to CpuTensor's (the recurrence is ill-conditioned when |a| ~ 1, which the
// reference's default init A_real = 0 gives, so any re-association drifts): every product and
// sum is an unfused, individually rounded f32 operation (__fmul_rn / __fadd_rn), sums run in
// the reference's index order, and a[n] is computed on the host with the same libm expf/cosf
// the reference's Rust f32 methods call.

// ---------------------------------------------------------------- ref mode, step 1
// U[t][n] = sum_m Bd[n][m] * x[m][t], m ascending (CpuTensor 2-D x 1-D matmul,
// backend-cpu/src/lib.rs:728-735). One thread per t; Bd rows are wave-uniform (scalar loads).
template <int NS>
__global__ __launch_bounds__(256) void s4_input_proj_kernel(int64_t M, int64_t L, int64_t N,
                                                            const float* __restrict__ x,
                                                            const float* __restrict__ Bd,
                                                            float* __restrict__ U) {
#pragma clang fp contract(off)
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= L) return;
    float acc[NS];
#pragma unroll
    for (int n = 0; n < NS; ++n) acc[n] = 0.0f;
    for (int64_t m = 0; m < M; ++m) {
        const float xv = x[m * L + t];
#pragma unroll
        for (int n = 0; n < NS; ++n)
            if (n < N) acc[n] = __fadd_rn(acc[n], __fmul_rn(Bd[n * M + m], xv));
    }
#pragma unroll
    for (int n = 0; n < NS; ++n)
        if (n < N) U[t * N + n] = acc[n];
}

// Bd = B * dt (mul_scalar, ssm.rs:130), rounded once like the reference.
__global__ void s4_scale_kernel(int64_t n, float dt, const float* __restrict__ B,
                                float* __restrict__ Bd) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) Bd[i] = __fmul_rn(B[i], dt);
}

// ---------------------------------------------------------------- ref mode, step 2
// H[t][n] = a[n]*H[t-1][n] + U[t][n] sequentially in t, one lane per state: s1 = a*h rounded,
// then h = s1 + s2 rounded (ssm.rs:172-174). In place over U.
__global__ __launch_bounds__(64) void s4_scan_seq_kernel(int64_t L, int64_t N,
                                                         const float* __restrict__ a,
                                                         float* __restrict__ H) {
#pragma clang fp contract(off)
    const int n = threadIdx.x;
    if (n >= N) return;
    const float an = a[n];
    float h = 0.0f;
    int64_t t = 0;
    // 8 steps per iteration: the loads of a batch issue together ahead of the dependent chain
    for (; t + 8 <= L; t += 8) {
        float s2[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) s2[k] = H[(t + k) * N + n];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            h = __fadd_rn(__fmul_rn(an, h), s2[k]);
            H[(t + k) * N + n] = h;
        }
    }
    for (; t < L; ++t) {
        h = __fadd_rn(__fmul_rn(an, h), H[t * N + n]);
        H[t * N + n] = h;
    }
}

// ---------------------------------------------------------------- ref mode, step 3
// o[m] = sum_n C[m][n]*h[n] (n ascending, 2-D x 1-D matmul); y = o + D[m]*u[m]
// (ssm.rs:177-179); y *= gate[m] (ssm.rs:460-461). Tile = 64 channels x 32 steps: x is read
// along t (rows of x) into LDS and y written along m.
constexpr int kTileM = 64, kTileT = 32;

template <int NS>
__global__ __launch_bounds__(256) void s4_output_kernel(int64_t M, int64_t L, int64_t N,
                                                        const float* __restrict__ x,
                                                        const float* __restrict__ H,
                                                        const float* __restrict__ C,
                                                        const float* __restrict__ D,
                                                        const float* __restrict__ gate,
                                                        float* __restrict__ y) {
#pragma clang fp contract(off)
    __shared__ float sx[kTileM][kTileT + 1];
    __shared__ float sh[kTileT][NS];
    const int64_t m0 = (int64_t)blockIdx.x * kTileM;
    const int64_t t0 = (int64_t)blockIdx.y * kTileT;
    const int tid = threadIdx.x;
    for (int i = tid; i < kTileM * kTileT; i += 256) {
        const int mm = i / kTileT, tt = i % kTileT;
        const int64_t m = m0 + mm, t = t0 + tt;
        sx[mm][tt] = (m < M && t < L) ? x[m * L + t] : 0.0f;
    }
    for (int i = tid; i < kTileT * NS; i += 256) {
        const int tt = i / NS, n = i % NS;
        const int64_t t = t0 + tt;
        sh[tt][n] = (t < L && n < N) ? H[t * N + n] : 0.0f;
    }
    __syncthreads();
    const int mm = tid & 63;
    const int64_t m = m0 + mm;
    if (m >= M) return;
    float c[NS];
#pragma unroll
    for (int n = 0; n < NS; ++n) c[n] = n < N ? C[m * N + n] : 0.0f;
    const float dd = D[m];
    const float g = gate ? gate[m] : 1.0f;
    for (int tt = tid >> 6; tt < kTileT; tt += 4) {
        const int64_t t = t0 + tt;
        if (t >= L) break;
        float o = 0.0f;
#pragma unroll
        for (int n = 0; n < NS; ++n)
            if (n < N) o = __fadd_rn(o, __fmul_rn(c[n], sh[tt][n]));
        float v = __fadd_rn(o, __fmul_rn(dd, sx[mm][tt]));
        if (gate) v = __fmul_rn(v, g);
        y[t * M + m] = v;
    }
}

// ---------------------------------------------------------------- S4D complex
// One thread per (b, d); complex diagonal state in registers; fp32.
template <int NS>
__global__ __launch_bounds__(128) void s4d_complex_kernel(
    int64_t Bt, int64_t L, int64_t Dm, int64_t N, const float* __restrict__ x,
    const float* __restrict__ dtv, const float* __restrict__ a_re, const float* __restrict__ a_im,
    const float* __restrict__ B_re, const float* __restrict__ B_im,
    const float* __restrict__ C_re, const float* __restrict__ C_im, const float* __restrict__ Dv,
    float* __restrict__ y) {
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= Bt * Dm) return;
    const int64_t b = gid / Dm, d = gid % Dm;
    float ar[NS], ai[NS], br[NS], bi[NS], cr[NS], ci[NS], hr[NS], hi[NS];
    const float dt = dtv[d];
#pragma unroll
    for (int n = 0; n < NS; ++n) {
        const bool v = n < N;
        const int64_t k = d * N + n;
        const float mag = v ? expf(dt * a_re[k]) : 0.0f;
        float sn, cs;
        sincosf(v ? dt * a_im[k] : 0.0f, &sn, &cs);
        ar[n] = mag * cs;
        ai[n] = mag * sn;
        br[n] = v ? dt * B_re[k] : 0.0f;
        bi[n] = v ? dt * B_im[k] : 0.0f;
        cr[n] = v ? C_re[k] : 0.0f;
        ci[n] = v ? C_im[k] : 0.0f;
        hr[n] = hi[n] = 0.0f;
    }
    const float dd = Dv ? Dv[d] : 0.0f;
    for (int64_t t = 0; t < L; ++t) {
        const int64_t i = (b * L + t) * Dm + d;
        const float u = x[i];
        float acc = 0.0f;
#pragma unroll
        for (int n = 0; n < NS; ++n) {
            const float nr = fmaf(ar[n], hr[n], fmaf(-ai[n], hi[n], br[n] * u));
            const float ni = fmaf(ar[n], hi[n], fmaf(ai[n], hr[n], bi[n] * u));
            hr[n] = nr;
            hi[n] = ni;
            acc = fmaf(cr[n], nr, fmaf(-ci[n], ni, acc));
        }
        y[i] = fmaf(2.0f, acc, dd * u);
    }
}

}  // namespace
}  // namespace hx

extern "C" int hx_s4_ref_fwd(int64_t d_model, int64_t dstate, int64_t seqlen, float dt,
                             const float* x, const float* a_real, const float* a_imag,
                             const float* B, const float* C, const float* D, const float* gate,
                             float* y, void* stream) {
    using namespace hx;
    HX_REQUIRE(d_model >= 0 && seqlen >= 0, HX_ERR_INVALID_DIMENSION,
               "s4_ref: negative size (d_model=%lld seqlen=%lld)", (long long)d_model,
               (long long)seqlen);
    HX_REQUIRE(dstate >= 1 && dstate <= kMaxState, HX_ERR_UNSUPPORTED,
               "s4_ref: dstate=%lld not supported (1..%d)", (long long)dstate, kMaxState);
    if (d_model == 0 || seqlen == 0) return HX_OK;
    HX_REQUIRE(x && a_real && a_imag && B && C && D && y, HX_ERR_INVALID_INPUT,
               "s4_ref: x, a_real, a_imag, B, C, D and y must be non-NULL");
    hipStream_t s = as_stream(stream);

    // discretize(dt) (ssm.rs:113-120) on the host with libm, exactly as the reference:
    // tr = a_real*dt; ti = a_imag*dt; a = expf(tr) * cosf(ti). This synchronises with `stream`
    // (the parameters are read back), which reference mode accepts for bit-faithfulness.
    float ar[kMaxState], ai[kMaxState], a[kMaxState];
    HX_HIP_CHECK(hipStreamSynchronize(s));
    HX_HIP_CHECK(hipMemcpy(ar, a_real, dstate * sizeof(float), hipMemcpyDeviceToHost));
    HX_HIP_CHECK(hipMemcpy(ai, a_imag, dstate * sizeof(float), hipMemcpyDeviceToHost));
    for (int64_t n = 0; n < dstate; ++n) {
        volatile float tr = ar[n] * dt;
        volatile float ti = ai[n] * dt;
        a[n] = expf(tr) * cosf(ti);
    }

    // scratch: a [N] | Bd [N*M] | H [L*N]
    const size_t n_a = 64, n_bd = (size_t)dstate * d_model, n_h = (size_t)seqlen * dstate;
    float* scratch = nullptr;
    HX_HIP_CHECK(hipMallocAsync((void**)&scratch, (n_a + n_bd + n_h) * sizeof(float), s));
    float* a_dev = scratch;
    float* Bd = scratch + n_a;
    float* H = Bd + n_bd;
    int rc = HX_OK;
    hipError_t e = hipMemcpyAsync(a_dev, a, dstate * sizeof(float), hipMemcpyHostToDevice, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);  // `a` is a stack buffer
    if (e != hipSuccess) {
        rc = set_error(HX_ERR_BACKEND, "s4_ref: upload of discretised A failed: %s",
                       hipGetErrorString(e));
    } else {
        hipLaunchKernelGGL(s4_scale_kernel, dim3((unsigned)((n_bd + 255) / 256)), dim3(256), 0, s,
                           (int64_t)n_bd, dt, B, Bd);
        dim3 g1((unsigned)((seqlen + 255) / 256));
        if (dstate <= 16)
            hipLaunchKernelGGL(s4_input_proj_kernel<16>, g1, dim3(256), 0, s, d_model, seqlen,
                               dstate, x, Bd, H);
        else
            hipLaunchKernelGGL(s4_input_proj_kernel<kMaxState>, g1, dim3(256), 0, s, d_model,
                               seqlen, dstate, x, Bd, H);
        hipLaunchKernelGGL(s4_scan_seq_kernel, dim3(1), dim3(64), 0, s, seqlen, dstate, a_dev, H);
        dim3 g3((unsigned)((d_model + kTileM - 1) / kTileM),
                (unsigned)((seqlen + kTileT - 1) / kTileT));
        if (dstate <= 16)
            hipLaunchKernelGGL(s4_output_kernel<16>, g3, dim3(256), 0, s, d_model, seqlen, dstate,
                               x, H, C, D, gate, y);
        else
            hipLaunchKernelGGL(s4_output_kernel<kMaxState>, g3, dim3(256), 0, s, d_model, seqlen,
                               dstate, x, H, C, D, gate, y);
        hipError_t le = hipGetLastError();
        if (le != hipSuccess)
            rc = set_error(HX_ERR_BACKEND, "s4_ref: launch failed: %s", hipGetErrorString(le));
    }
    (void)hipFreeAsync(scratch, s);
    return rc;
}

extern "C" int hx_s4d_complex_fwd(int64_t batch, int64_t seqlen, int64_t dim, int64_t dstate,
                                  const float* x, const float* dt, const float* a_re,
                                  const float* a_im, const float* B_re, const float* B_im,
                                  const float* C_re, const float* C_im, const float* D, float* y,
                                  void* stream) {
    using namespace hx;
    HX_REQUIRE(batch >= 0 && seqlen >= 0 && dim >= 0, HX_ERR_INVALID_DIMENSION,
               "s4d_complex: negative size");
    HX_REQUIRE(dstate >= 1 && dstate <= kMaxState, HX_ERR_UNSUPPORTED,
               "s4d_complex: dstate=%lld not supported (1..%d)", (long long)dstate, kMaxState);
    if (batch == 0 || seqlen == 0 || dim == 0) return HX_OK;
    HX_REQUIRE(x && dt && a_re && a_im && B_re && B_im && C_re && C_im && y, HX_ERR_INVALID_INPUT,
               "s4d_complex: a required pointer is NULL");
    const int64_t total = batch * dim;
    dim3 grid((unsigned)((total + 127) / 128));
    hipStream_t s = as_stream(stream);
    if (dstate <= 16)
        hipLaunchKernelGGL(s4d_complex_kernel<16>, grid, dim3(128), 0, s, batch, seqlen, dim,
                           dstate, x, dt, a_re, a_im, B_re, B_im, C_re, C_im, D, y);
    else
        hipLaunchKernelGGL(s4d_complex_kernel<kMaxState>, grid, dim3(128), 0, s, batch, seqlen,
                           dim, dstate, x, dt, a_re, a_im, B_re, B_im, C_re, C_im, D, y);
    HX_LAUNCH_CHECK();
    return HX_OK;
}

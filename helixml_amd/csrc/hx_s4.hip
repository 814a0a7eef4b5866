// hx_s4.hip — S4 recurrences for gfx950.
//
// (1) Reference-mode S4Block::forward_ssm (crates/nn/src/ssm.rs:138-186): one state h[N] shared
//     by all d_model channels, constant diagonal decay a[n] = exp(dt*a_real)*cos(dt*a_imag)
//     (ssm.rs:113-120), Bd = dt*B (ssm.rs:130). It factors into three bandwidth-bound steps:
//       U[t][n] = sum_m Bd[n][m] * x[m][t]            (column reduction over channels)
//       H[t][n] = a[n]*H[t-1][n] + U[t][n]             (16 independent first-order scans)
//       y[t][m] = (sum_n C[m][n]*H[t][n] + D[m]*x[m][t]) * gate[m]
//     x is [d_model, L] (time contiguous) and y is [L, d_model] (channels contiguous), so the
//     output kernel transposes through LDS.
// (2) S4D diagonal complex recurrence, per channel.
#include "hx_common.h"

namespace hx {
namespace {

constexpr int kMaxState = 64;

// ---------------------------------------------------------------- ref mode, step 1
// U[t][n] = sum_m (B[n][m]*dt) * x[m][t]. One thread per t, m ascending; B is read with
// wave-uniform addresses (scalar loads).
template <int NS>
__global__ __launch_bounds__(256) void s4_input_proj_kernel(int64_t M, int64_t L, int64_t N,
                                                            float dt, const float* __restrict__ x,
                                                            const float* __restrict__ B,
                                                            float* __restrict__ U) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= L) return;
    float acc[NS];
#pragma unroll
    for (int n = 0; n < NS; ++n) acc[n] = 0.0f;
    for (int64_t m = 0; m < M; ++m) {
        const float xv = x[m * L + t];
#pragma unroll
        for (int n = 0; n < NS; ++n)
            if (n < N) acc[n] = fmaf(B[n * M + m] * dt, xv, acc[n]);
    }
#pragma unroll
    for (int n = 0; n < NS; ++n)
        if (n < N) U[t * N + n] = acc[n];
}

// ---------------------------------------------------------------- ref mode, step 2
// Chunked first-order scan H[t] = a*H[t-1] + U[t] for each state n. Phase A: each chunk
// scans from zero and records its end value; phase B: one thread per n carries across chunks;
// phase C: each chunk adds a^(k+1) * carry_in to its local values.
constexpr int kScanChunk = 256;

__device__ inline float s4_decay(const float* a_real, const float* a_imag, int n, float dt) {
    const float tr = a_real[n] * dt;
    const float ti = a_imag[n] * dt;
    return expf(tr) * cosf(ti);
}

__global__ __launch_bounds__(256) void s4_scan_local_kernel(int64_t L, int64_t N, float dt,
                                                            const float* __restrict__ a_real,
                                                            const float* __restrict__ a_imag,
                                                            float* __restrict__ H,
                                                            float* __restrict__ chunk_end) {
    // thread = (chunk, n)
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t nchunks = (L + kScanChunk - 1) / kScanChunk;
    if (gid >= nchunks * N) return;
    const int64_t c = gid / N, n = gid % N;
    const float a = s4_decay(a_real, a_imag, (int)n, dt);
    const int64_t t0 = c * kScanChunk, t1 = min(L, t0 + kScanChunk);
    float h = 0.0f;
    for (int64_t t = t0; t < t1; ++t) {
        h = fmaf(a, h, H[t * N + n]);
        H[t * N + n] = h;
    }
    chunk_end[c * N + n] = h;
}

__global__ void s4_scan_carry_kernel(int64_t L, int64_t N, float dt,
                                     const float* __restrict__ a_real,
                                     const float* __restrict__ a_imag,
                                     float* __restrict__ chunk_end) {
    // In place: chunk_end[c] becomes the state entering chunk c.
    const int n = threadIdx.x;
    if (n >= N) return;
    const float a = s4_decay(a_real, a_imag, n, dt);
    const int64_t nchunks = (L + kScanChunk - 1) / kScanChunk;
    // a^kScanChunk by repeated squaring (kScanChunk is a power of two)
    float aT = a;
    for (int s = 1; s < kScanChunk; s <<= 1) aT *= aT;
    float carry = 0.0f;
    for (int64_t c = 0; c < nchunks; ++c) {
        const float e = chunk_end[c * N + n];
        chunk_end[c * N + n] = carry;
        carry = fmaf(aT, carry, e);
    }
}

__global__ __launch_bounds__(256) void s4_scan_fix_kernel(int64_t L, int64_t N, float dt,
                                                          const float* __restrict__ a_real,
                                                          const float* __restrict__ a_imag,
                                                          float* __restrict__ H,
                                                          const float* __restrict__ carry_in) {
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t nchunks = (L + kScanChunk - 1) / kScanChunk;
    if (gid >= nchunks * N) return;
    const int64_t c = gid / N, n = gid % N;
    if (c == 0) return;
    const float a = s4_decay(a_real, a_imag, (int)n, dt);
    const float cin = carry_in[c * N + n];
    const int64_t t0 = c * kScanChunk, t1 = min(L, t0 + kScanChunk);
    float p = a;
    for (int64_t t = t0; t < t1; ++t) {
        H[t * N + n] = fmaf(p, cin, H[t * N + n]);
        p *= a;
    }
}

// ---------------------------------------------------------------- ref mode, step 3
// y[t][m] = (sum_n C[m][n]*H[t][n] + D[m]*x[m][t]) * gate[m]. Tile = 64 channels x 32 steps:
// x is read along t (row of x) into LDS, y written along m.
constexpr int kTileM = 64, kTileT = 32;

template <int NS>
__global__ __launch_bounds__(256) void s4_output_kernel(int64_t M, int64_t L, int64_t N,
                                                        const float* __restrict__ x,
                                                        const float* __restrict__ H,
                                                        const float* __restrict__ C,
                                                        const float* __restrict__ D,
                                                        const float* __restrict__ gate,
                                                        float* __restrict__ y) {
    __shared__ float sx[kTileM][kTileT + 1];
    __shared__ float sh[kTileT][NS];
    const int64_t m0 = (int64_t)blockIdx.x * kTileM;
    const int64_t t0 = (int64_t)blockIdx.y * kTileT;
    const int tid = threadIdx.x;
    // load x tile: 64 rows (m) x 32 cols (t), 8 passes of 256 threads
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
    const float dd = D ? D[m] : 0.0f;
    const float g = gate ? gate[m] : 1.0f;
    for (int tt = tid >> 6; tt < kTileT; tt += 4) {
        const int64_t t = t0 + tt;
        if (t >= L) break;
        float o = 0.0f;
#pragma unroll
        for (int n = 0; n < NS; ++n) o = fmaf(c[n], sh[tt][n], o);
        float v = o + dd * sx[mm][tt];
        if (gate) v *= g;
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
    // H (L x N) is staged in y's tail? No: y is L x M and may be smaller than L x N when
    // M < N. A scratch buffer is allocated per call.
    float* H = nullptr;
    float* ends = nullptr;
    const int64_t nchunks = (seqlen + kScanChunk - 1) / kScanChunk;
    HX_HIP_CHECK(hipMallocAsync((void**)&H, (size_t)seqlen * dstate * sizeof(float), s));
    hipError_t e = hipMallocAsync((void**)&ends, (size_t)nchunks * dstate * sizeof(float), s);
    if (e != hipSuccess) {
        (void)hipFreeAsync(H, s);
        return set_error(HX_ERR_ALLOCATION, "s4_ref: scratch allocation failed: %s",
                         hipGetErrorString(e));
    }
    int rc = HX_OK;
    {
        dim3 g1((unsigned)((seqlen + 255) / 256));
        if (dstate <= 16)
            hipLaunchKernelGGL(s4_input_proj_kernel<16>, g1, dim3(256), 0, s, d_model, seqlen,
                               dstate, dt, x, B, H);
        else
            hipLaunchKernelGGL(s4_input_proj_kernel<kMaxState>, g1, dim3(256), 0, s, d_model,
                               seqlen, dstate, dt, x, B, H);
        dim3 g2((unsigned)((nchunks * dstate + 255) / 256));
        hipLaunchKernelGGL(s4_scan_local_kernel, g2, dim3(256), 0, s, seqlen, dstate, dt, a_real,
                           a_imag, H, ends);
        hipLaunchKernelGGL(s4_scan_carry_kernel, dim3(1), dim3(64), 0, s, seqlen, dstate, dt,
                           a_real, a_imag, ends);
        hipLaunchKernelGGL(s4_scan_fix_kernel, g2, dim3(256), 0, s, seqlen, dstate, dt, a_real,
                           a_imag, H, ends);
        dim3 g3((unsigned)((d_model + kTileM - 1) / kTileM), (unsigned)((seqlen + kTileT - 1) / kTileT));
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
    (void)hipFreeAsync(ends, s);
    (void)hipFreeAsync(H, s);
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

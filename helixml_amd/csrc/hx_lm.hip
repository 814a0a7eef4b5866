// hx_lm.hip — the byte-level SSM LM pieces around the Mamba block: token
// embedding gather, RMSNorm, and the single-step causal conv of recurrent decode.
#include "hx_common.h"
#include "hx_wave.h"

namespace hx {
namespace {

// out[t][:] = table[tok[t]][:]; a token outside [0, vocab) yields a zero row. One wave per token.
__global__ __launch_bounds__(256) void embedding_kernel(int64_t n, int64_t vocab, int64_t dim,
                                                        const int32_t* __restrict__ tok,
                                                        const float* __restrict__ table,
                                                        float* __restrict__ out, int vec) {
    const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (t >= n) return;
    const int lane = threadIdx.x & 63;
    const int32_t k = tok[t];
    const bool ok = k >= 0 && k < vocab;
    const float* src = table + (ok ? (int64_t)k : 0) * dim;
    float* dst = out + t * dim;
    if (vec) {
        for (int64_t c = lane * 4; c < dim; c += 256) {
            const float4 v = ok ? *reinterpret_cast<const float4*>(src + c) : make_float4(0, 0, 0, 0);
            *reinterpret_cast<float4*>(dst + c) = v;
        }
    } else {
        for (int64_t c = lane; c < dim; c += 64) dst[c] = ok ? src[c] : 0.0f;
    }
}

__device__ inline float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// Sum over the wave, the same value in every lane: DPP within each 16-lane row (quad permutes,
// the half-row mirror, the row rotate by 8), then the rows and the halves by register swaps. Every
// level adds a lane's value to its partner's, so all lanes form the identical sum.
__device__ inline float wave_allsum(float v) {
    v += dpp<kDppXor1>(v);
    v += dpp<kDppXor2>(v);
    v += dpp<kDppHalfMirror>(v);
    v += dpp<kDppRor8>(v);
    float a = v, b = v;
    swap16(a, b);
    v = a + b;
    a = v; b = v;
    swap32(a, b);
    return a + b;
}

// nn::RMSNorm::forward (crates/nn/src/lib.rs:258-285): ms = mean(x^2 over the row);
// y = x / sqrt(ms + eps) * w. One wave per row, dim <= 64 * 4 * RPL: the row and the weight
// are loaded together in one round (the weight is L2-hot), kept in registers, and each lane
// writes its 4 outputs with one 8-byte (bf16) or 16-byte (fp32) store.
template <typename TO, int RPL>
__global__ __launch_bounds__(256) void rmsnorm_kernel(int64_t rows, int64_t dim,
                                                      const float* __restrict__ x,
                                                      const float* __restrict__ w, float eps,
                                                      TO* __restrict__ y) {
    const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= rows) return;
    const int lane = threadIdx.x & 63;
    const float* xr = x + r * dim;
    float4 v[RPL], wv[RPL];
#pragma unroll
    for (int i = 0; i < RPL; ++i) {
        const int64_t c = (int64_t)(i * 64 + lane) * 4;
        v[i] = c < dim ? *reinterpret_cast<const float4*>(xr + c) : make_float4(0, 0, 0, 0);
        wv[i] = c < dim ? *reinterpret_cast<const float4*>(w + c) : make_float4(0, 0, 0, 0);
    }
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < RPL; ++i) {
        ss = fmaf(v[i].x, v[i].x, ss);
        ss = fmaf(v[i].y, v[i].y, ss);
        ss = fmaf(v[i].z, v[i].z, ss);
        ss = fmaf(v[i].w, v[i].w, ss);
    }
    ss = wave_allsum(ss);
    const float inv = 1.0f / sqrtf(ss / (float)dim + eps);
    TO* yr = y + r * dim;
#pragma unroll
    for (int i = 0; i < RPL; ++i) {
        const int64_t c = (int64_t)(i * 64 + lane) * 4;
        if (c < dim) {
            const float4 o = make_float4(v[i].x * inv * wv[i].x, v[i].y * inv * wv[i].y,
                                         v[i].z * inv * wv[i].z, v[i].w * inv * wv[i].w);
            if constexpr (std::is_same_v<TO, float>) {
                *reinterpret_cast<float4*>(yr + c) = o;
            } else {
                *reinterpret_cast<uint2*>(yr + c) = make_uint2(pack_bf16x2(o.x, o.y), pack_bf16x2(o.z, o.w));
            }
        }
    }
}

// Rows of any width: two passes over the row.
template <typename TO>
__global__ __launch_bounds__(256) void rmsnorm_any_kernel(int64_t rows, int64_t dim,
                                                          const float* __restrict__ x,
                                                          const float* __restrict__ w, float eps,
                                                          TO* __restrict__ y) {
    const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= rows) return;
    const int lane = threadIdx.x & 63;
    const float* xr = x + r * dim;
    float ss = 0.0f;
    for (int64_t c = lane; c < dim; c += 64) ss = fmaf(xr[c], xr[c], ss);
    ss = wave_sum(ss);
    const float inv = 1.0f / sqrtf(ss / (float)dim + eps);
    for (int64_t c = lane; c < dim; c += 64) Storage<TO>::store(y + r * dim + c, xr[c] * inv * w[c]);
}

// One decode step of the causal conv: y[b][d] = silu(bias[d] + sum_{j<K-1} w[d][j] *
// state[b][j][d] + w[d][K-1] * x[b][d]); then the window shifts (state[b][j] = state[b][j+1],
// state[b][K-2] = x[b]). state [B][K-1][D] fp32, x rows of stride ldx, y [B][D].
template <typename T>
__global__ __launch_bounds__(256) void conv_step_kernel(int64_t Bt, int64_t Dm, int K,
                                                        const T* __restrict__ x, int64_t ldx,
                                                        const float* __restrict__ w,
                                                        const float* __restrict__ bias,
                                                        float* __restrict__ state,
                                                        T* __restrict__ y) {
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= Bt * Dm) return;
    const int64_t b = gid / Dm, d = gid - b * Dm;
    const float xv = Storage<T>::load(x + b * ldx + d);
    float* st = state + b * (K - 1) * Dm + d;
    float acc = bias ? bias[d] : 0.0f;
    float prev[3];
    for (int j = 0; j < K - 1; ++j) {
        prev[j] = st[j * Dm];
        acc = fmaf(w[d * K + j], prev[j], acc);
    }
    acc = fmaf(w[d * K + K - 1], xv, acc);
    for (int j = 0; j + 1 < K - 1; ++j) st[j * Dm] = prev[j + 1];
    if (K > 1) st[(K - 2) * Dm] = xv;
    Storage<T>::store(y + b * Dm + d, silu(acc));
}

// Decode hand-off after a prefill: state[b][j][d] = x[b][L-(K-1)+j][d] (zero before t = 0).
template <typename T>
__global__ __launch_bounds__(256) void conv_state_capture_kernel(int64_t Bt, int64_t L, int64_t Dm,
                                                                 int K, const T* __restrict__ x,
                                                                 int64_t ldx,
                                                                 float* __restrict__ state) {
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= Bt * (K - 1) * Dm) return;
    const int64_t d = gid % Dm;
    const int64_t j = (gid / Dm) % (K - 1);
    const int64_t b = gid / Dm / (K - 1);
    const int64_t t = L - (K - 1) + j;
    state[gid] = t >= 0 ? Storage<T>::load(x + (b * L + t) * ldx + d) : 0.0f;
}

}  // namespace

int conv_state_capture(int64_t Bt, int64_t L, int64_t Dm, int K, const uint16_t* x, int64_t ldx,
                       float* state, hipStream_t s) {
    if (K <= 1 || Bt == 0) return HX_OK;
    const int64_t n = Bt * (K - 1) * Dm;
    hipLaunchKernelGGL(conv_state_capture_kernel<uint16_t>, dim3((unsigned)((n + 255) / 256)),
                       dim3(256), 0, s, Bt, L, Dm, K, x, ldx, state);
    HX_LAUNCH_CHECK();
    return HX_OK;
}

}  // namespace hx

extern "C" int hx_embedding_fwd(int64_t n_tokens, int64_t vocab, int64_t dim, const int32_t* tokens,
                                const float* table, float* out, void* stream) {
    using namespace hx;
    HX_REQUIRE(n_tokens >= 0 && vocab > 0 && dim > 0, HX_ERR_INVALID_DIMENSION,
               "embedding: bad sizes");
    if (n_tokens == 0) return HX_OK;
    HX_REQUIRE(tokens && table && out, HX_ERR_INVALID_INPUT, "embedding: NULL pointer");
    const int vec = dim % 4 == 0 && aligned(table, 16) && aligned(out, 16);
    hipLaunchKernelGGL(embedding_kernel, dim3((unsigned)((n_tokens + 3) / 4)), dim3(256), 0,
                       as_stream(stream), n_tokens, vocab, dim, tokens, table, out, vec);
    HX_LAUNCH_CHECK();
    return HX_OK;
}

extern "C" int hx_rmsnorm_fwd(int64_t rows, int64_t dim, const float* x, const float* weight,
                              float eps, int out_dtype, void* y, void* stream) {
    using namespace hx;
    HX_REQUIRE(rows >= 0 && dim > 0, HX_ERR_INVALID_DIMENSION, "rmsnorm: bad sizes");
    HX_REQUIRE(out_dtype == HX_F32 || out_dtype == HX_BF16, HX_ERR_DTYPE_MISMATCH,
               "rmsnorm: out_dtype %d", out_dtype);
    if (rows == 0) return HX_OK;
    HX_REQUIRE(x && weight && y, HX_ERR_INVALID_INPUT, "rmsnorm: NULL pointer");
    hipStream_t s = as_stream(stream);
    dim3 grid((unsigned)((rows + 3) / 4));
    const bool vec = dim % 4 == 0 && aligned(x, 16) && aligned(weight, 16) &&
                     aligned(y, out_dtype == HX_BF16 ? 8 : 16);
    if (vec && dim <= 512) {
        if (out_dtype == HX_BF16)
            hipLaunchKernelGGL((rmsnorm_kernel<uint16_t, 2>), grid, dim3(256), 0, s, rows, dim, x,
                               weight, eps, (uint16_t*)y);
        else
            hipLaunchKernelGGL((rmsnorm_kernel<float, 2>), grid, dim3(256), 0, s, rows, dim, x,
                               weight, eps, (float*)y);
    } else if (vec && dim <= 2048) {
        if (out_dtype == HX_BF16)
            hipLaunchKernelGGL((rmsnorm_kernel<uint16_t, 8>), grid, dim3(256), 0, s, rows, dim, x,
                               weight, eps, (uint16_t*)y);
        else
            hipLaunchKernelGGL((rmsnorm_kernel<float, 8>), grid, dim3(256), 0, s, rows, dim, x,
                               weight, eps, (float*)y);
    } else {
        if (out_dtype == HX_BF16)
            hipLaunchKernelGGL((rmsnorm_any_kernel<uint16_t>), grid, dim3(256), 0, s, rows, dim, x,
                               weight, eps, (uint16_t*)y);
        else
            hipLaunchKernelGGL((rmsnorm_any_kernel<float>), grid, dim3(256), 0, s, rows, dim, x,
                               weight, eps, (float*)y);
    }
    HX_LAUNCH_CHECK();
    return HX_OK;
}

extern "C" int hx_conv1d_step(int64_t batch, int64_t dim, int64_t width, int dtype, const void* x,
                              int64_t ldx, const float* weight, const float* bias, float* state,
                              void* y, void* stream) {
    using namespace hx;
    HX_REQUIRE(batch >= 0 && dim >= 0, HX_ERR_INVALID_DIMENSION, "conv1d_step: negative size");
    HX_REQUIRE(width >= 1 && width <= 4, HX_ERR_UNSUPPORTED, "conv1d_step: width %lld (1..4)",
               (long long)width);
    HX_REQUIRE(dtype == HX_F32 || dtype == HX_BF16, HX_ERR_DTYPE_MISMATCH, "conv1d_step: dtype %d",
               dtype);
    if (batch == 0 || dim == 0) return HX_OK;
    HX_REQUIRE(x && weight && y && ldx >= dim && (width == 1 || state), HX_ERR_INVALID_INPUT,
               "conv1d_step: x, weight, y (and state for width > 1) required, ldx >= dim");
    const int64_t n = batch * dim;
    dim3 grid((unsigned)((n + 255) / 256));
    if (dtype == HX_F32)
        hipLaunchKernelGGL(conv_step_kernel<float>, grid, dim3(256), 0, as_stream(stream), batch,
                           dim, (int)width, (const float*)x, ldx, weight, bias, state, (float*)y);
    else
        hipLaunchKernelGGL(conv_step_kernel<uint16_t>, grid, dim3(256), 0, as_stream(stream), batch,
                           dim, (int)width, (const uint16_t*)x, ldx, weight, bias, state,
                           (uint16_t*)y);
    HX_LAUNCH_CHECK();
    return HX_OK;
}

// hx_dense.hip — fp32 dense products for the reference-mode layers.
//
// nn::Linear::forward (crates/nn/src/lib.rs:120-134) computes X . W^T + bias with W stored
// [out, in]; CpuTensor::matmul 2-D x 2-D (backend-cpu/src/lib.rs:644-678) computes A . B.
// Both are small at the reference's shapes (d_model 64..512), so one LDS-tiled VALU kernel
// with a 64x64 output tile and 4x4 register blocking covers them; fp32 accumulate in the
// reference's k order, so results are bit-identical to CpuTensor's before the optional SiLU.
#include "hx_common.h"

namespace hx {
namespace {

// Reference order: each output is an f32 sum from 0.0 over k ascending of individually rounded
// products (CpuTensor::matmul, backend-cpu/src/lib.rs:659-667), so no contraction into FMA.
#pragma clang fp contract(off)

constexpr int TM = 64, TN = 64, TK = 16;

// Y[r][o] = act( sum_k X[r][k] * Wop(k, o) + bias[o] ),
//   W_IS_OUT_IN: Wop(k,o) = W[o*K + k]   (Linear weight [out, in])
//   else       : Wop(k,o) = W[k*N + o]   (matmul right operand [K, N])
template <bool W_IS_OUT_IN>
__global__ __launch_bounds__(256) void gemm_f32_kernel(int64_t M, int64_t K, int64_t N,
                                                       const float* __restrict__ X,
                                                       const float* __restrict__ W,
                                                       const float* __restrict__ bias, int act,
                                                       float* __restrict__ Y) {
#pragma clang fp contract(off)
    __shared__ float sa[TK][TM + 4];
    __shared__ float sb[TK][TN + 4];
    const int tid = threadIdx.x;
    const int tx = tid % 16, ty = tid / 16;
    const int64_t r0 = (int64_t)blockIdx.y * TM, c0 = (int64_t)blockIdx.x * TN;
    float acc[4][4] = {};
    for (int64_t k0 = 0; k0 < K; k0 += TK) {
        for (int i = tid; i < TM * TK; i += 256) {
            const int rr = i / TK, kk = i % TK;
            const int64_t r = r0 + rr, k = k0 + kk;
            sa[kk][rr] = (r < M && k < K) ? X[r * K + k] : 0.0f;
        }
        for (int i = tid; i < TN * TK; i += 256) {
            int cc, kk;
            if (W_IS_OUT_IN) { cc = i / TK; kk = i % TK; }
            else { kk = i / TN; cc = i % TN; }
            const int64_t c = c0 + cc, k = k0 + kk;
            float v = 0.0f;
            if (c < N && k < K) v = W_IS_OUT_IN ? W[c * K + k] : W[k * N + c];
            sb[kk][cc] = v;
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < TK; ++kk) {
            float a[4], b[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) a[i] = sa[kk][ty + 16 * i];
#pragma unroll
            for (int j = 0; j < 4; ++j) b[j] = sb[kk][tx + 16 * j];
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = acc[i][j] + a[i] * b[j];
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int64_t r = r0 + ty + 16 * i;
        if (r >= M) continue;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int64_t c = c0 + tx + 16 * j;
            if (c >= N) continue;
            float v = acc[i][j] + (bias ? bias[c] : 0.0f);
            if (act == 1) v = v / (1.0f + expf(-v));
            Y[r * N + c] = v;
        }
    }
}

}  // namespace
}  // namespace hx

extern "C" int hx_linear_f32(int64_t rows, int64_t in_features, int64_t out_features,
                             const float* X, const float* W, const float* bias, int act,
                             float* Y, void* stream) {
    using namespace hx;
    HX_REQUIRE(rows >= 0 && in_features >= 0 && out_features >= 0, HX_ERR_INVALID_DIMENSION,
               "linear: negative size");
    HX_REQUIRE(act == 0 || act == 1, HX_ERR_INVALID_INPUT, "linear: act=%d (0 none, 1 silu)", act);
    if (rows == 0 || out_features == 0) return HX_OK;
    HX_REQUIRE(X && W && Y, HX_ERR_INVALID_INPUT, "linear: X, W and Y must be non-NULL");
    HX_REQUIRE(rows <= 65535LL * TM, HX_ERR_UNSUPPORTED, "linear: rows=%lld too large",
               (long long)rows);
    dim3 grid((unsigned)((out_features + TN - 1) / TN), (unsigned)((rows + TM - 1) / TM));
    hipLaunchKernelGGL(gemm_f32_kernel<true>, grid, dim3(256), 0, as_stream(stream), rows,
                       in_features, out_features, X, W, bias, act, Y);
    HX_LAUNCH_CHECK();
    return HX_OK;
}

extern "C" int hx_matmul_f32(int64_t M, int64_t K, int64_t N, const float* A, const float* B,
                             float* Y, void* stream) {
    using namespace hx;
    HX_REQUIRE(M >= 0 && K >= 0 && N >= 0, HX_ERR_INVALID_DIMENSION, "matmul: negative size");
    if (M == 0 || N == 0) return HX_OK;
    HX_REQUIRE(A && B && Y, HX_ERR_INVALID_INPUT, "matmul: A, B and Y must be non-NULL");
    HX_REQUIRE(M <= 65535LL * TM, HX_ERR_UNSUPPORTED, "matmul: M=%lld too large", (long long)M);
    dim3 grid((unsigned)((N + TN - 1) / TN), (unsigned)((M + TM - 1) / TM));
    hipLaunchKernelGGL(gemm_f32_kernel<false>, grid, dim3(256), 0, as_stream(stream), M, K, N, A,
                       B, nullptr, 0, Y);
    HX_LAUNCH_CHECK();
    return HX_OK;
}

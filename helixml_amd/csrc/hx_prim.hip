// hx_prim.hip — the CpuTensor primitives a HipTensor needs to implement the reference's tensor
// traits (TensorOps / TensorActivation / TensorReduce::mean / TensorBroadcast and the shape
// operations of Tensor, crates/tensor-core/src/tensor.rs:7-209) on the device, so the generic
// nn code (MambaBlock::<T>, S4Block::<T>, RMSNorm::<T>) runs on HipTensor without the fused
// overrides.
//
// Semantics follow crates/backend-cpu/src/lib.rs:
//   add/sub/mul/div (570-632): one IEEE f32 operation per element -> bit-exact;
//   mul_scalar / add_scalar (916-932), neg (895-902), abs (822-828): bit-exact;
//   sqrt (768-775): correctly rounded -> bit-exact;
//   exp/log/sin/cos (777-811) and silu = x / (1 + exp(-x)) (1154-1170), sigmoid: the device
//     math library in place of the host libm the reference calls (a few ulp apart);
//   mean over one axis (TensorReduce::mean, 995-1010 -> ndarray 0.15 mean_axis = sum_axis / n):
//     the summation order of ndarray's sum_axis — over the contiguous (last) axis each lane is
//     summed by ndarray's eight-accumulator unrolled fold, over any other axis the sub-views are
//     added in axis order — then one correctly rounded division, so results are bit-exact;
//   every shape operation (reshape 94-113, transpose 115-137, slice 139-183, cat 185-252, stack
//     254-335 and 390-467, broadcast_to 1352-1518 and 511-560, contiguous) is an exact copy
//     through one strided-copy kernel whose strides the host computes from the reference's index
//     arithmetic (including its quirks).
// Arithmetic is fp32; layouts are row-major contiguous unless strides say otherwise.
#include "hx_common.h"

namespace hx {
namespace {

#pragma clang fp contract(off)

constexpr int kThreads = 256;

unsigned grid_for(int64_t work, int64_t per_block) {
    int64_t g = (work + per_block - 1) / per_block;
    if (g < 1) g = 1;
    if (g > 16384) g = 16384;  // grid-stride beyond 64 blocks per CU
    return (unsigned)g;
}

template <int OP>
__device__ inline float bin(float a, float b) {
    if constexpr (OP == HX_ADD) return a + b;
    else if constexpr (OP == HX_SUB) return a - b;
    else if constexpr (OP == HX_MUL) return a * b;
    else return a / b;  // correctly rounded (hipcc's default fp32 division)
}

template <int OP, bool VEC>
__global__ __launch_bounds__(kThreads) void binary_kernel(int64_t n, const float* __restrict__ a,
                                                          const float* __restrict__ b,
                                                          float* __restrict__ y) {
#pragma clang fp contract(off)
    const int64_t stride = (int64_t)gridDim.x * kThreads;
    int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if constexpr (VEC) {
        const int64_t n4 = n / 4;
        for (int64_t j = i; j < n4; j += stride) {
            const float4 va = reinterpret_cast<const float4*>(a)[j];
            const float4 vb = reinterpret_cast<const float4*>(b)[j];
            reinterpret_cast<float4*>(y)[j] =
                make_float4(bin<OP>(va.x, vb.x), bin<OP>(va.y, vb.y), bin<OP>(va.z, vb.z), bin<OP>(va.w, vb.w));
        }
        for (int64_t j = n4 * 4 + i; j < n; j += stride) y[j] = bin<OP>(a[j], b[j]);
    } else {
        for (int64_t j = i; j < n; j += stride) y[j] = bin<OP>(a[j], b[j]);
    }
}

// Correctly rounded square root. v_sqrt_f32 is within one ulp; the result is then moved to the
// neighbour on the right side of each rounding midpoint: m = (s + neighbour) / 2 has at most 25
// significant bits, so m*m is exact in double and x >= m*m (or x < m*m) decides the rounding
// exactly (no ties: a 24-bit x is never the square of a 25-bit midpoint).
__device__ inline float sqrt_rn(float x) {
    float s = __builtin_sqrtf(x);
    if (!(x > 0.0f) || !(x < __builtin_inff())) return s;  // +-0, negative (NaN), inf, NaN
    const double xd = (double)x;
    for (int it = 0; it < 3; ++it) {
        const float up = __uint_as_float(__float_as_uint(s) + 1u);
        const float dn = __uint_as_float(__float_as_uint(s) - 1u);
        const double mh = ((double)s + (double)up) * 0.5, ml = ((double)s + (double)dn) * 0.5;
        if (xd >= mh * mh) s = up;
        else if (xd < ml * ml) s = dn;
        else break;
    }
    return s;
}

template <int OP>
__device__ inline float una(float x, float s) {
    if constexpr (OP == HX_EXP) return expf(x);
    else if constexpr (OP == HX_COS) return cosf(x);
    else if constexpr (OP == HX_SIN) return sinf(x);
    else if constexpr (OP == HX_SQRT) return sqrt_rn(x);
    else if constexpr (OP == HX_SILU) return x / (1.0f + expf(-x));
    else if constexpr (OP == HX_NEG) return -x;
    else if constexpr (OP == HX_MUL_SCALAR) return x * s;
    else if constexpr (OP == HX_ADD_SCALAR) return x + s;
    else if constexpr (OP == HX_ABS) return fabsf(x);
    else if constexpr (OP == HX_LOG) return logf(x);
    else return 1.0f / (1.0f + expf(-x));  // HX_SIGMOID
}

template <int OP, bool VEC>
__global__ __launch_bounds__(kThreads) void unary_kernel(int64_t n, const float* __restrict__ x,
                                                         float s, float* __restrict__ y) {
#pragma clang fp contract(off)
    const int64_t stride = (int64_t)gridDim.x * kThreads;
    int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if constexpr (VEC) {
        const int64_t n4 = n / 4;
        for (int64_t j = i; j < n4; j += stride) {
            const float4 v = reinterpret_cast<const float4*>(x)[j];
            reinterpret_cast<float4*>(y)[j] =
                make_float4(una<OP>(v.x, s), una<OP>(v.y, s), una<OP>(v.z, s), una<OP>(v.w, s));
        }
        for (int64_t j = n4 * 4 + i; j < n; j += stride) y[j] = una<OP>(x[j], s);
    } else {
        for (int64_t j = i; j < n; j += stride) y[j] = una<OP>(x[j], s);
    }
}

// Mean over the contiguous axis of [rows, len]: eight lanes per row hold the fold's eight
// partial sums p0..p7 (element k goes to p_{k mod 8} for k < 8*floor(len/8)), then
// acc = ((((0 + (p0+p4)) + (p1+p5)) + (p2+p6)) + (p3+p7)), then the len mod 8 trailing elements
// in order, then acc / len — the order of ndarray's unrolled fold over a contiguous lane.
__global__ __launch_bounds__(kThreads) void mean_lane_kernel(int64_t rows, int64_t len,
                                                             const float* __restrict__ x,
                                                             float* __restrict__ y) {
#pragma clang fp contract(off)
    const int lane8 = threadIdx.x & 7;
    const int64_t row = (int64_t)blockIdx.x * (kThreads / 8) + threadIdx.x / 8;
    const bool live = row < rows;
    const float* xr = x + (live ? row : 0) * len;
    const int64_t body = len / 8 * 8;
    float p = 0.0f;
    if (live)
        for (int64_t k = lane8; k < body; k += 8) p = p + xr[k];
    // gather the group's partials (lanes of a group are 8 consecutive lanes of one wave)
    const int base = (threadIdx.x & 63) & ~7;
    float q[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) q[j] = __shfl(p, base + j, 64);
    if (!live || lane8 != 0) return;
    float acc = 0.0f;
    acc = acc + (q[0] + q[4]);
    acc = acc + (q[1] + q[5]);
    acc = acc + (q[2] + q[6]);
    acc = acc + (q[3] + q[7]);
    for (int64_t k = body; k < len; ++k) acc = acc + xr[k];
    y[row] = acc / (float)len;
}

// Mean over the middle axis of [outer, len, inner] in axis order: y[o][i] = (sum over l in order,
// from 0) / len — ndarray's sum_axis off the array's minimum-stride (last) axis adds the
// sub-views one by one.
__global__ __launch_bounds__(kThreads) void mean_strided_kernel(int64_t outer, int64_t len,
                                                                int64_t inner,
                                                                const float* __restrict__ x,
                                                                float* __restrict__ y) {
#pragma clang fp contract(off)
    const int64_t total = outer * inner;
    const int64_t stride = (int64_t)gridDim.x * kThreads;
    for (int64_t g = (int64_t)blockIdx.x * kThreads + threadIdx.x; g < total; g += stride) {
        const int64_t o = g / inner, i = g % inner;
        const float* xp = x + o * len * inner + i;
        float acc = 0.0f;
        for (int64_t l = 0; l < len; ++l) acc = acc + xp[l * inner];
        y[g] = acc / (float)len;
    }
}

struct StridedCopy {
    int ndim;
    int64_t shape[HX_MAX_DIMS];
    int64_t src_stride[HX_MAX_DIMS];
    int64_t dst_stride[HX_MAX_DIMS];
};

// dst[sum_j c_j * dst_stride[j]] = src[sum_j c_j * src_stride[j]] for every coordinate c of
// `shape`; one thread per element in row-major coordinate order.
__global__ __launch_bounds__(kThreads) void copy_strided_kernel(int64_t total, StridedCopy p,
                                                                const float* __restrict__ src,
                                                                float* __restrict__ dst) {
    const int64_t stride = (int64_t)gridDim.x * kThreads;
    for (int64_t g = (int64_t)blockIdx.x * kThreads + threadIdx.x; g < total; g += stride) {
        int64_t rem = g, so = 0, d = 0;
        for (int j = p.ndim - 1; j >= 0; --j) {
            const int64_t c = rem % p.shape[j];
            rem /= p.shape[j];
            so += c * p.src_stride[j];
            d += c * p.dst_stride[j];
        }
        dst[d] = src[so];
    }
}

template <bool VEC>
__global__ __launch_bounds__(kThreads) void fill_kernel(int64_t n, float v, float* __restrict__ y) {
    const int64_t stride = (int64_t)gridDim.x * kThreads;
    int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if constexpr (VEC) {
        const int64_t n4 = n / 4;
        for (int64_t j = i; j < n4; j += stride) reinterpret_cast<float4*>(y)[j] = make_float4(v, v, v, v);
        for (int64_t j = n4 * 4 + i; j < n; j += stride) y[j] = v;
    } else {
        for (int64_t j = i; j < n; j += stride) y[j] = v;
    }
}

__global__ __launch_bounds__(kThreads) void eye_kernel(int64_t n, float* __restrict__ y) {
    const int64_t total = n * n;
    const int64_t stride = (int64_t)gridDim.x * kThreads;
    for (int64_t g = (int64_t)blockIdx.x * kThreads + threadIdx.x; g < total; g += stride)
        y[g] = (g / n == g % n) ? 1.0f : 0.0f;
}

template <int OP>
int launch_binary(int64_t n, const float* a, const float* b, float* y, hipStream_t s) {
    const bool vec = aligned(a, 16) && aligned(b, 16) && aligned(y, 16);
    const unsigned g = grid_for(vec ? (n + 3) / 4 : n, kThreads);
    if (vec) hipLaunchKernelGGL((binary_kernel<OP, true>), dim3(g), dim3(kThreads), 0, s, n, a, b, y);
    else hipLaunchKernelGGL((binary_kernel<OP, false>), dim3(g), dim3(kThreads), 0, s, n, a, b, y);
    HX_LAUNCH_CHECK();
    return HX_OK;
}

template <int OP>
int launch_unary(int64_t n, const float* x, float sc, float* y, hipStream_t s) {
    const bool vec = aligned(x, 16) && aligned(y, 16);
    const unsigned g = grid_for(vec ? (n + 3) / 4 : n, kThreads);
    if (vec) hipLaunchKernelGGL((unary_kernel<OP, true>), dim3(g), dim3(kThreads), 0, s, n, x, sc, y);
    else hipLaunchKernelGGL((unary_kernel<OP, false>), dim3(g), dim3(kThreads), 0, s, n, x, sc, y);
    HX_LAUNCH_CHECK();
    return HX_OK;
}

}  // namespace
}  // namespace hx

extern "C" int hx_binary_f32(int op, int64_t n, const float* a, const float* b, float* y,
                             void* stream) {
    HX_REQUIRE(n >= 0, HX_ERR_INVALID_DIMENSION, "hx_binary_f32: negative size %lld", (long long)n);
    HX_REQUIRE(op >= HX_ADD && op <= HX_DIV, HX_ERR_INVALID_INPUT, "hx_binary_f32: op %d unknown", op);
    if (n == 0) return HX_OK;
    HX_REQUIRE(a && b && y, HX_ERR_INVALID_INPUT, "hx_binary_f32: NULL operand");
    auto s = hx::as_stream(stream);
    switch (op) {
        case HX_ADD: return hx::launch_binary<HX_ADD>(n, a, b, y, s);
        case HX_SUB: return hx::launch_binary<HX_SUB>(n, a, b, y, s);
        case HX_MUL: return hx::launch_binary<HX_MUL>(n, a, b, y, s);
        default: return hx::launch_binary<HX_DIV>(n, a, b, y, s);
    }
}

extern "C" int hx_unary_f32(int op, int64_t n, const float* x, float scalar, float* y,
                            void* stream) {
    HX_REQUIRE(n >= 0, HX_ERR_INVALID_DIMENSION, "hx_unary_f32: negative size %lld", (long long)n);
    HX_REQUIRE(op >= HX_EXP && op <= HX_SIGMOID, HX_ERR_INVALID_INPUT, "hx_unary_f32: op %d unknown", op);
    if (n == 0) return HX_OK;
    HX_REQUIRE(x && y, HX_ERR_INVALID_INPUT, "hx_unary_f32: NULL operand");
    auto s = hx::as_stream(stream);
    switch (op) {
        case HX_EXP: return hx::launch_unary<HX_EXP>(n, x, scalar, y, s);
        case HX_COS: return hx::launch_unary<HX_COS>(n, x, scalar, y, s);
        case HX_SIN: return hx::launch_unary<HX_SIN>(n, x, scalar, y, s);
        case HX_SQRT: return hx::launch_unary<HX_SQRT>(n, x, scalar, y, s);
        case HX_SILU: return hx::launch_unary<HX_SILU>(n, x, scalar, y, s);
        case HX_NEG: return hx::launch_unary<HX_NEG>(n, x, scalar, y, s);
        case HX_MUL_SCALAR: return hx::launch_unary<HX_MUL_SCALAR>(n, x, scalar, y, s);
        case HX_ADD_SCALAR: return hx::launch_unary<HX_ADD_SCALAR>(n, x, scalar, y, s);
        case HX_ABS: return hx::launch_unary<HX_ABS>(n, x, scalar, y, s);
        case HX_LOG: return hx::launch_unary<HX_LOG>(n, x, scalar, y, s);
        default: return hx::launch_unary<HX_SIGMOID>(n, x, scalar, y, s);
    }
}

extern "C" int hx_mean_axis_f32(int64_t outer, int64_t len, int64_t inner, int lane_fold,
                                const float* x, float* y, void* stream) {
    HX_REQUIRE(outer >= 0 && inner >= 0, HX_ERR_INVALID_DIMENSION,
               "hx_mean_axis_f32: negative size (outer %lld, inner %lld)", (long long)outer,
               (long long)inner);
    // ndarray's mean_axis of an empty axis returns None, which the reference unwraps
    HX_REQUIRE(len >= 1, HX_ERR_INVALID_DIMENSION, "hx_mean_axis_f32: mean over an axis of length %lld",
               (long long)len);
    if (outer == 0 || inner == 0) return HX_OK;
    HX_REQUIRE(x && y, HX_ERR_INVALID_INPUT, "hx_mean_axis_f32: NULL operand");
    auto s = hx::as_stream(stream);
    HX_REQUIRE(!lane_fold || inner == 1, HX_ERR_INVALID_INPUT,
               "hx_mean_axis_f32: the lane fold sums a contiguous axis (inner must be 1, got %lld)",
               (long long)inner);
    if (lane_fold) {
        const int64_t per_block = hx::kThreads / 8;
        HX_REQUIRE((outer + per_block - 1) / per_block <= 0x7fffffff, HX_ERR_UNSUPPORTED,
                   "hx_mean_axis_f32: %lld rows exceed the grid", (long long)outer);
        hipLaunchKernelGGL(hx::mean_lane_kernel, dim3((unsigned)((outer + per_block - 1) / per_block)),
                           dim3(hx::kThreads), 0, s, outer, len, x, y);
    } else {
        hipLaunchKernelGGL(hx::mean_strided_kernel, dim3(hx::grid_for(outer * inner, hx::kThreads)),
                           dim3(hx::kThreads), 0, s, outer, len, inner, x, y);
    }
    HX_LAUNCH_CHECK();
    return HX_OK;
}

extern "C" int hx_copy_strided_f32(int ndim, const int64_t* shape, const float* src,
                                   const int64_t* src_strides, float* dst,
                                   const int64_t* dst_strides, void* stream) {
    HX_REQUIRE(ndim >= 0 && ndim <= HX_MAX_DIMS, HX_ERR_UNSUPPORTED,
               "hx_copy_strided_f32: %d dims (at most %d)", ndim, HX_MAX_DIMS);
    HX_REQUIRE(ndim == 0 || (shape && src_strides && dst_strides), HX_ERR_INVALID_INPUT,
               "hx_copy_strided_f32: NULL shape or strides");
    hx::StridedCopy p{};
    p.ndim = ndim;
    int64_t total = 1;
    for (int j = 0; j < ndim; ++j) {
        HX_REQUIRE(shape[j] >= 0, HX_ERR_INVALID_DIMENSION, "hx_copy_strided_f32: dim %d is %lld",
                   j, (long long)shape[j]);
        p.shape[j] = shape[j];
        p.src_stride[j] = src_strides[j];
        p.dst_stride[j] = dst_strides[j];
        total *= shape[j];
    }
    if (total == 0) return HX_OK;
    HX_REQUIRE(src && dst, HX_ERR_INVALID_INPUT, "hx_copy_strided_f32: NULL buffer");
    hipLaunchKernelGGL(hx::copy_strided_kernel, dim3(hx::grid_for(total, hx::kThreads)),
                       dim3(hx::kThreads), 0, hx::as_stream(stream), total, p, src, dst);
    HX_LAUNCH_CHECK();
    return HX_OK;
}

extern "C" int hx_fill_f32(int64_t n, float value, float* y, void* stream) {
    HX_REQUIRE(n >= 0, HX_ERR_INVALID_DIMENSION, "hx_fill_f32: negative size %lld", (long long)n);
    if (n == 0) return HX_OK;
    HX_REQUIRE(y, HX_ERR_INVALID_INPUT, "hx_fill_f32: NULL output");
    auto s = hx::as_stream(stream);
    if (hx::aligned(y, 16))
        hipLaunchKernelGGL(hx::fill_kernel<true>, dim3(hx::grid_for((n + 3) / 4, hx::kThreads)),
                           dim3(hx::kThreads), 0, s, n, value, y);
    else
        hipLaunchKernelGGL(hx::fill_kernel<false>, dim3(hx::grid_for(n, hx::kThreads)),
                           dim3(hx::kThreads), 0, s, n, value, y);
    HX_LAUNCH_CHECK();
    return HX_OK;
}

extern "C" int hx_eye_f32(int64_t n, float* y, void* stream) {
    HX_REQUIRE(n >= 0, HX_ERR_INVALID_DIMENSION, "hx_eye_f32: negative size %lld", (long long)n);
    if (n == 0) return HX_OK;
    HX_REQUIRE(y, HX_ERR_INVALID_INPUT, "hx_eye_f32: NULL output");
    hipLaunchKernelGGL(hx::eye_kernel, dim3(hx::grid_for(n * n, hx::kThreads)), dim3(hx::kThreads),
                       0, hx::as_stream(stream), n, y);
    HX_LAUNCH_CHECK();
    return HX_OK;
}

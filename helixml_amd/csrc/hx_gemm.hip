// hx_gemm.hip — bf16 GEMM on the gfx950 matrix cores for the Mamba block's projections.
//
// Y = X . W^T (+ bias), the nn::Linear layout (crates/nn/src/lib.rs:120-134: weight [out, in]):
// X [M, K] and W [N, K] both K-contiguous bf16, fp32 accumulate, bf16 or fp32 output.
// Rows whose start is not 16-byte aligned take an element-load variant of the same kernel.
// Block tile 128 x 128 x 32, 4 waves in a 2 x 2 grid, each wave 64 x 64 = 2 x 2 tiles of
// v_mfma_f32_32x32x16_bf16. Tiles are staged through LDS (double-buffered, rows padded by 16
// bytes so the 16-byte fragment reads of 8 consecutive rows cover all 32 banks); global loads
// are 16-byte and issued one K-step ahead. The epilogue can split the N columns over up to three
// outputs with their own row strides (in_proj -> x | z, x_proj -> dt | B | C) so later kernels read
// contiguous operands.
#include "hx_common.h"

namespace hx {
namespace {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16;

constexpr int BM = 128, BN = 128, BK = 32;
constexpr int LDSK = BK + 8;  // padded row (bf16 elements): 80 bytes

struct GemmOut {
    void* y[3];
    int64_t ld[3];
    int64_t split1, split2;  // column boundaries of outputs 0 | 1 | 2
    int out_bf16;
    int act;                 // bit 0: SiLU; bit 1: accumulate (Y += result, read-modify-write)
};

// 8 consecutive bf16 of row `row` from column `col`, zero outside [nrows, ncols). VEC: the row
// start is 16-byte aligned (ld % 8 == 0, aligned base), so an in-bounds piece is one 16-byte load.
template <bool VEC>
__device__ inline uint4 load16_guard(const uint16_t* base, int64_t row, int64_t nrows, int64_t col,
                                     int64_t ncols, int64_t ld) {
    if (VEC && row < nrows && col + 8 <= ncols) return *reinterpret_cast<const uint4*>(base + row * ld + col);
    if (row >= nrows || col >= ncols) return make_uint4(0, 0, 0, 0);
    uint16_t v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = (col + i < ncols) ? base[row * ld + col + i] : (uint16_t)0;
    return make_uint4(v[0] | (v[1] << 16), v[2] | (v[3] << 16), v[4] | (v[5] << 16), v[6] | (v[7] << 16));
}

template <bool VEC>
__global__ __launch_bounds__(256) void gemm_bf16_nt_kernel(int64_t M, int64_t N, int64_t K,
                                                           const uint16_t* __restrict__ X,
                                                           int64_t ldx,
                                                           const uint16_t* __restrict__ W,
                                                           int64_t ldw,
                                                           const float* __restrict__ bias,
                                                           GemmOut o) {
    __shared__ __attribute__((aligned(16))) uint16_t sA[2][BM][LDSK];
    __shared__ __attribute__((aligned(16))) uint16_t sB[2][BN][LDSK];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int64_t m0 = (int64_t)blockIdx.y * BM, n0 = (int64_t)blockIdx.x * BN;

    // global -> register staging: each tile is 128 rows x 32 k = 512 16-byte pieces, 2 per thread
    uint4 ra[2], rb[2];
    auto gload = [&](int64_t k0) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int e = tid + j * 256;
            const int row = e >> 2, kc = (e & 3) * 8;
            ra[j] = load16_guard<VEC>(X, m0 + row, M, k0 + kc, K, ldx);
            rb[j] = load16_guard<VEC>(W, n0 + row, N, k0 + kc, K, ldw);
        }
    };
    auto sstore = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int e = tid + j * 256;
            const int row = e >> 2, kc = (e & 3) * 8;
            *reinterpret_cast<uint4*>(&sA[buf][row][kc]) = ra[j];
            *reinterpret_cast<uint4*>(&sB[buf][row][kc]) = rb[j];
        }
    };

    f32x16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    const int fr = lane & 31;          // fragment row (A: m, B: n)
    const int fk = (lane >> 5) * 8;    // fragment k offset within a 16-wide k step

    const int64_t nk = (K + BK - 1) / BK;
    gload(0);
    sstore(0);
    if (nk > 1) gload(BK);
    __syncthreads();
    for (int64_t kt = 0; kt < nk; ++kt) {
        const int buf = (int)(kt & 1);
#pragma unroll
        for (int kk = 0; kk < BK; kk += 16) {
            bf16x8 a[2], bfr[2];
#pragma unroll
            for (int i = 0; i < 2; ++i)
                a[i] = *reinterpret_cast<const bf16x8*>(&sA[buf][wm * 64 + i * 32 + fr][kk + fk]);
#pragma unroll
            for (int j = 0; j < 2; ++j)
                bfr[j] = *reinterpret_cast<const bf16x8*>(&sB[buf][wn * 64 + j * 32 + fr][kk + fk]);
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], bfr[j], acc[i][j], 0, 0, 0);
        }
        if (kt + 1 < nk) {
            sstore(buf ^ 1);
            if (kt + 2 < nk) gload((kt + 2) * BK);
        }
        __syncthreads();
    }

    // epilogue: acc[i][j][r] holds C[row][col], row = 8*(r/4) + 4*(lane/32) + r%4, col = lane%32
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int64_t col = n0 + wn * 64 + j * 32 + (lane & 31);
            if (col >= N) continue;
            const float bv = bias ? bias[col] : 0.0f;
            int seg = 0;
            int64_t cc = col;
            if (col >= o.split2) { seg = 2; cc = col - o.split2; }
            else if (col >= o.split1) { seg = 1; cc = col - o.split1; }
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int64_t row = m0 + wm * 64 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                if (row >= M) continue;
                float v = acc[i][j][r] + bv;
                if (o.act & 1) v = silu(v);
                const int64_t off = row * o.ld[seg] + cc;
                if (o.out_bf16) {
                    uint16_t* yp = (uint16_t*)o.y[seg] + off;
                    if (o.act & 2) v += Storage<uint16_t>::load(yp);
                    Storage<uint16_t>::store(yp, v);
                } else {
                    float* yp = (float*)o.y[seg] + off;
                    if (o.act & 2) v += *yp;
                    *yp = v;
                }
            }
        }
}

}  // namespace
}  // namespace hx

extern "C" int hx_gemm_bf16(int64_t M, int64_t N, int64_t K, const void* X, int64_t ldx,
                            const void* W, int64_t ldw, const float* bias, int act, int out_dtype,
                            void* Y0, int64_t ld0, int64_t split1, void* Y1, int64_t ld1,
                            int64_t split2, void* Y2, int64_t ld2, void* stream) {
    using namespace hx;
    HX_REQUIRE(M >= 0 && N >= 0 && K >= 0, HX_ERR_INVALID_DIMENSION, "gemm_bf16: negative size");
    HX_REQUIRE(act >= 0 && act <= 3, HX_ERR_INVALID_INPUT,
               "gemm_bf16: act=%d (bit 0 SiLU, bit 1 accumulate into Y)", act);
    HX_REQUIRE(out_dtype == HX_F32 || out_dtype == HX_BF16, HX_ERR_DTYPE_MISMATCH,
               "gemm_bf16: out_dtype %d", out_dtype);
    if (M == 0 || N == 0) return HX_OK;
    HX_REQUIRE(X && W && Y0, HX_ERR_INVALID_INPUT, "gemm_bf16: X, W and Y0 must be non-NULL");
    HX_REQUIRE(ldx >= K && ldw >= K && ld0 >= 0, HX_ERR_INVALID_DIMENSION,
               "gemm_bf16: leading dimensions smaller than K");
    const bool vec = ldx % 8 == 0 && ldw % 8 == 0 && aligned(X, 16) && aligned(W, 16);
    if (split1 <= 0 || split1 > N) split1 = N;
    if (split2 < split1 || split2 > N) split2 = N;
    HX_REQUIRE(split1 == N || Y1, HX_ERR_INVALID_INPUT, "gemm_bf16: Y1 is NULL but split1 < N");
    HX_REQUIRE(split2 == N || Y2, HX_ERR_INVALID_INPUT, "gemm_bf16: Y2 is NULL but split2 < N");
    HX_REQUIRE((N + BN - 1) / BN <= 0x7fffffff && (M + BM - 1) / BM <= 65535, HX_ERR_UNSUPPORTED,
               "gemm_bf16: M=%lld too large for the grid", (long long)M);
    GemmOut o{{Y0, Y1, Y2}, {ld0, ld1, ld2}, split1, split2, out_dtype == HX_BF16, act};
    dim3 grid((unsigned)((N + BN - 1) / BN), (unsigned)((M + BM - 1) / BM));
    if (vec)
        hipLaunchKernelGGL(gemm_bf16_nt_kernel<true>, grid, dim3(256), 0, as_stream(stream), M, N, K,
                           (const uint16_t*)X, ldx, (const uint16_t*)W, ldw, bias, o);
    else  // rows not 16-byte aligned: element loads (odd K such as a small dt_rank)
        hipLaunchKernelGGL(gemm_bf16_nt_kernel<false>, grid, dim3(256), 0, as_stream(stream), M, N, K,
                           (const uint16_t*)X, ldx, (const uint16_t*)W, ldw, bias, o);
    HX_LAUNCH_CHECK();
    return HX_OK;
}

// hx_block.hip — the full Mamba block forward on gfx950:
//   xz = x . W_in^T           (matrix-core GEMM, split into x | z)
//   xc = SiLU(conv1d_causal(x) + conv_b)   (depthwise, kernel d_conv)
//   dt_lo | B | C = xc . W_x^T  (GEMM, three outputs)
//   dt = dt_lo . W_dt^T       (GEMM)
//   y  = selective_scan(xc, dt, A, B, C, D, z, dt_bias, softplus)
//   out = y . W_out^T         (GEMM)
// The reference's exported MambaBlock::forward_mamba is Linear -> SiLU -> Linear
// (crates/nn/src/lib.rs:888-906) and allocates A/B/C/D/delta_proj/B_proj/C_proj it never uses
// (lib.rs:851-867); this is the block those parameters describe. bf16 storage, fp32 arithmetic.
#include "hx_common.h"

extern "C" int hx_gemm_bf16(int64_t M, int64_t N, int64_t K, const void* X, int64_t ldx,
                            const void* W, int64_t ldw, const float* bias, int act, int out_dtype,
                            void* Y0, int64_t ld0, int64_t split1, void* Y1, int64_t ld1,
                            int64_t split2, void* Y2, int64_t ld2, void* stream);

namespace hx {
namespace {

// Causal depthwise conv over time + bias + SiLU. A thread owns CPT adjacent channels (16 bytes
// of a row when VEC) and TT consecutive steps; it keeps the last KW input rows in registers, so
// each input row is read once plus a KW-1 row halo per run of TT steps. Block = 256 threads
// across channels; grid.x = batch x step-runs, grid.y = channel blocks.
// y[b,t,d] = silu(bias[d] + sum_j w[d,j] * x[b, t-(KW-1)+j, d]), zero before t = 0.
template <typename T, int CPT, bool VEC>
struct ConvRow {
    __device__ static inline void load(const T* p, float (&v)[CPT]) {
        if constexpr (VEC && sizeof(T) == 2 && CPT == 8) {
            const uint4 q = *reinterpret_cast<const uint4*>(p);
            const uint32_t wds[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                v[2 * i] = __uint_as_float(wds[i] << 16);
                v[2 * i + 1] = __uint_as_float(wds[i] & 0xffff0000u);
            }
        } else if constexpr (VEC && sizeof(T) == 4 && CPT == 4) {
            const float4 q = *reinterpret_cast<const float4*>(p);
            v[0] = q.x; v[1] = q.y; v[2] = q.z; v[3] = q.w;
        } else {
#pragma unroll
            for (int i = 0; i < CPT; ++i) v[i] = Storage<T>::load(p + i);
        }
    }
    __device__ static inline void store(T* p, const float (&v)[CPT]) {
        if constexpr (VEC && sizeof(T) == 2 && CPT == 8) {
            uint32_t wds[4];
#pragma unroll
            for (int i = 0; i < 4; ++i)
                wds[i] = (uint32_t)Storage<uint16_t>::round(v[2 * i]) |
                         ((uint32_t)Storage<uint16_t>::round(v[2 * i + 1]) << 16);
            *reinterpret_cast<uint4*>(p) = make_uint4(wds[0], wds[1], wds[2], wds[3]);
        } else if constexpr (VEC && sizeof(T) == 4 && CPT == 4) {
            *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
        } else {
#pragma unroll
            for (int i = 0; i < CPT; ++i) Storage<T>::store(p + i, v[i]);
        }
    }
};

template <typename T, int KW, int CPT, bool VEC, int TT>
__global__ __launch_bounds__(256) void conv1d_silu_kernel(int L, int Dm, int nruns,
                                                          const T* __restrict__ x, int64_t ldx,
                                                          const float* __restrict__ w,
                                                          const float* __restrict__ bias,
                                                          T* __restrict__ y) {
    const int d0 = (blockIdx.y * 256 + threadIdx.x) * CPT;
    if (d0 >= Dm) return;
    const int b = blockIdx.x / nruns;
    const int t0 = (blockIdx.x - b * nruns) * TT;
    float wk[KW][CPT], bv[CPT];
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
        bv[i] = bias ? bias[d0 + i] : 0.0f;
#pragma unroll
        for (int j = 0; j < KW; ++j) wk[j][i] = w[(d0 + i) * KW + j];
    }
    const T* xb = x + (int64_t)b * L * ldx + d0;
    T* yb = y + (int64_t)b * L * Dm + d0;
    float win[KW][CPT];  // win[KW-1] = row t, win[KW-2] = row t-1, ...
#pragma unroll
    for (int j = 0; j < KW - 1; ++j) {
        const int tt = t0 - (KW - 1) + j;
        if (tt >= 0) {
            ConvRow<T, CPT, VEC>::load(xb + (int64_t)tt * ldx, win[j + 1]);
        } else {
#pragma unroll
            for (int i = 0; i < CPT; ++i) win[j + 1][i] = 0.0f;
        }
    }
#pragma unroll
    for (int s = 0; s < TT; ++s) {
        const int t = t0 + s;
        if (t >= L) break;
#pragma unroll
        for (int j = 0; j < KW - 1; ++j)
#pragma unroll
            for (int i = 0; i < CPT; ++i) win[j][i] = win[j + 1][i];
        ConvRow<T, CPT, VEC>::load(xb + (int64_t)t * ldx, win[KW - 1]);
        float o[CPT];
#pragma unroll
        for (int i = 0; i < CPT; ++i) {
            float acc = bv[i];
#pragma unroll
            for (int j = 0; j < KW; ++j) acc = fmaf(wk[j][i], win[j][i], acc);
            o[i] = silu(acc);
        }
        ConvRow<T, CPT, VEC>::store(yb + (int64_t)t * Dm, o);
    }
}

template <typename T, int KW, int CPT, bool VEC>
void launch_conv_k(int64_t Bt, int64_t L, int64_t Dm, const void* x, int64_t ldx, const float* w,
                   const float* b, void* y, hipStream_t s) {
    constexpr int TT = 16;
    const int nruns = (int)((L + TT - 1) / TT);
    dim3 grid((unsigned)(Bt * nruns), (unsigned)((Dm / CPT + 255) / 256));
    hipLaunchKernelGGL((conv1d_silu_kernel<T, KW, CPT, VEC, TT>), grid, dim3(256), 0, s, (int)L,
                       (int)Dm, nruns, (const T*)x, ldx, w, b, (T*)y);
}

template <typename T, int CPT, bool VEC>
void launch_conv_w(int64_t Bt, int64_t L, int64_t Dm, int64_t KW, const void* x, int64_t ldx,
                   const float* w, const float* b, void* y, hipStream_t s) {
    switch (KW) {
        case 1: launch_conv_k<T, 1, CPT, VEC>(Bt, L, Dm, x, ldx, w, b, y, s); break;
        case 2: launch_conv_k<T, 2, CPT, VEC>(Bt, L, Dm, x, ldx, w, b, y, s); break;
        case 3: launch_conv_k<T, 3, CPT, VEC>(Bt, L, Dm, x, ldx, w, b, y, s); break;
        default: launch_conv_k<T, 4, CPT, VEC>(Bt, L, Dm, x, ldx, w, b, y, s); break;
    }
}

template <typename T>
int launch_conv(int64_t Bt, int64_t L, int64_t Dm, int64_t KW, const void* x, int64_t ldx,
                const float* w, const float* b, void* y, hipStream_t s) {
    constexpr int CV = 16 / sizeof(T);  // channels in 16 bytes
    const bool vec = Dm % CV == 0 && ldx % CV == 0 && aligned(x, 16) && aligned(y, 16);
    if (vec)
        launch_conv_w<T, CV, true>(Bt, L, Dm, KW, x, ldx, w, b, y, s);
    else
        launch_conv_w<T, 4, false>(Bt, L, Dm, KW, x, ldx, w, b, y, s);
    HX_LAUNCH_CHECK();
    return HX_OK;
}

}  // namespace
}  // namespace hx

extern "C" int hx_conv1d_silu(int64_t batch, int64_t seqlen, int64_t dim, int64_t width,
                              int dtype, const void* x, int64_t ldx, const float* weight,
                              const float* bias, void* y, void* stream) {
    using namespace hx;
    HX_REQUIRE(batch >= 0 && seqlen >= 0 && dim >= 0, HX_ERR_INVALID_DIMENSION,
               "conv1d_silu: negative size");
    HX_REQUIRE(width >= 1 && width <= 4, HX_ERR_UNSUPPORTED, "conv1d_silu: width %lld (1..4)",
               (long long)width);
    HX_REQUIRE(dim % 4 == 0, HX_ERR_UNSUPPORTED, "conv1d_silu: dim %lld not a multiple of 4",
               (long long)dim);
    HX_REQUIRE(dtype == HX_F32 || dtype == HX_BF16, HX_ERR_DTYPE_MISMATCH, "conv1d_silu: dtype %d",
               dtype);
    if (batch == 0 || seqlen == 0 || dim == 0) return HX_OK;
    HX_REQUIRE(x && weight && y && ldx >= dim, HX_ERR_INVALID_INPUT,
               "conv1d_silu: x, weight, y required and ldx >= dim");
    HX_REQUIRE(seqlen < (1LL << 31) && dim <= 65535LL * 1024 && batch * ((seqlen + 15) / 16) < (1LL << 31),
               HX_ERR_UNSUPPORTED, "conv1d_silu: sizes beyond the launch grid");
    return dtype == HX_F32
               ? launch_conv<float>(batch, seqlen, dim, width, x, ldx, weight, bias, y, as_stream(stream))
               : launch_conv<uint16_t>(batch, seqlen, dim, width, x, ldx, weight, bias, y, as_stream(stream));
}

// Workspace layout (bf16 elements, M = batch*seqlen): xpart | z | xconv | dt | y  [M, d_inner]
// each, dt_lo [M, dt_rank], B [M, N], C [M, N]; every region 256-byte aligned. The layer entry
// points add a normalised-input region [M, d_model] in front.
namespace {
inline size_t align256(size_t b) { return (b + 255) / 256 * 256; }
}  // namespace

extern "C" size_t hx_mamba_block_workspace_size(int64_t batch, int64_t seqlen, int64_t d_inner,
                                                int64_t dt_rank, int64_t dstate) {
    const size_t M = (size_t)batch * seqlen;
    return 5 * align256(M * d_inner * 2) + align256(M * dt_rank * 2) + 2 * align256(M * dstate * 2);
}

extern "C" size_t hx_mamba_layer_workspace_size(int64_t batch, int64_t seqlen, int64_t d_model,
                                                int64_t d_inner, int64_t dt_rank, int64_t dstate) {
    return align256((size_t)batch * seqlen * d_model * 2) +
           hx_mamba_block_workspace_size(batch, seqlen, d_inner, dt_rank, dstate);
}

namespace hx {
int conv_state_capture(int64_t Bt, int64_t L, int64_t Dm, int K, const uint16_t* x, int64_t ldx,
                       float* state, hipStream_t s);
}  // namespace hx

extern "C" int hx_conv1d_step(int64_t batch, int64_t dim, int64_t width, int dtype, const void* x,
                              int64_t ldx, const float* weight, const float* bias, float* state,
                              void* y, void* stream);
extern "C" int hx_rmsnorm_fwd(int64_t rows, int64_t dim, const float* x, const float* weight,
                              float eps, int out_dtype, void* y, void* stream);

namespace {

struct BlockWeights {
    const void *w_in, *w_x, *w_dt, *w_out;
    const float *conv_w, *conv_b, *dt_bias, *A, *D;
};

struct BlockBufs {
    void *xpart, *z, *xconv, *dt, *y, *dtlo, *B, *C;
};

BlockBufs carve(char* p, int64_t M, int64_t d_inner, int64_t dt_rank, int64_t dstate) {
    auto take = [&](size_t bytes) { void* r = p; p += align256(bytes); return r; };
    BlockBufs b;
    b.xpart = take(M * d_inner * 2);
    b.z = take(M * d_inner * 2);
    b.xconv = take(M * d_inner * 2);
    b.dt = take(M * d_inner * 2);
    b.y = take(M * d_inner * 2);
    b.dtlo = take(M * dt_rank * 2);
    b.B = take(M * dstate * 2);
    b.C = take(M * dstate * 2);
    return b;
}

int check_block_args(int64_t batch, int64_t seqlen, int64_t d_model, int64_t d_inner,
                     int64_t dstate, int64_t dt_rank, int64_t d_conv, const BlockWeights& w) {
    using namespace hx;
    HX_REQUIRE(batch >= 0 && seqlen >= 0 && d_model > 0 && d_inner > 0 && dt_rank > 0,
               HX_ERR_INVALID_DIMENSION, "mamba_block: bad sizes");
    HX_REQUIRE(dstate == 16, HX_ERR_UNSUPPORTED, "mamba_block: dstate %lld (16 supported)",
               (long long)dstate);
    HX_REQUIRE(d_inner % 4 == 0, HX_ERR_UNSUPPORTED, "mamba_block: d_inner %lld not a multiple of 4",
               (long long)d_inner);
    HX_REQUIRE(d_conv >= 1 && d_conv <= 4, HX_ERR_UNSUPPORTED, "mamba_block: d_conv %lld (1..4)",
               (long long)d_conv);
    HX_REQUIRE(w.w_in && w.conv_w && w.w_x && w.w_dt && w.A && w.w_out, HX_ERR_INVALID_INPUT,
               "mamba_block: a required weight pointer is NULL");
    return HX_OK;
}

// The block on bf16 input x [M, d_model]: writes out (bf16, or fp32 accumulated into when
// accumulate) and optionally the scan's last state and the conv window for decode.
int block_core(int64_t batch, int64_t seqlen, int64_t d_model, int64_t d_inner, int64_t dstate,
               int64_t dt_rank, int64_t d_conv, const void* x, const BlockWeights& w, void* out,
               int out_dtype, bool accumulate, float* last_state, float* conv_state,
               const BlockBufs& b, void* stream) {
    const int64_t M = batch * seqlen;
    int rc;
    // in_proj: [M, d_model] x [2*d_inner, d_model]^T -> xpart | z
    if ((rc = hx_gemm_bf16(M, 2 * d_inner, d_model, x, d_model, w.w_in, d_model, nullptr, 0,
                           HX_BF16, b.xpart, d_inner, d_inner, b.z, d_inner, 2 * d_inner, nullptr,
                           0, stream)))
        return rc;
    if (conv_state &&
        (rc = hx::conv_state_capture(batch, seqlen, d_inner, (int)d_conv, (const uint16_t*)b.xpart,
                                     d_inner, conv_state, hx::as_stream(stream))))
        return rc;
    if ((rc = hx_conv1d_silu(batch, seqlen, d_inner, d_conv, HX_BF16, b.xpart, d_inner, w.conv_w,
                             w.conv_b, b.xconv, stream)))
        return rc;
    // x_proj: [M, d_inner] x [dt_rank + 2N, d_inner]^T -> dt_lo | B | C. Narrow and long (config 3:
    // N 160, K 4096, 64 tiles of 256 x 256): K is split four ways and the fp32 partials go to the
    // in_proj x region, which the conv has consumed by now. The choice depends on the weight shape
    // only, so every batch size and sequence length gets the same arithmetic per token.
    const int64_t nx = dt_rank + 2 * dstate;
    const int splits = (d_inner >= 2048 && d_inner % 256 == 0 && nx <= 256 && 4 * nx * 2 <= d_inner) ? 4 : 1;
    rc = splits > 1 ? hx_gemm_bf16_splitk(M, nx, d_inner, b.xconv, d_inner, w.w_x, d_inner, nullptr, 0,
                                          HX_BF16, b.dtlo, dt_rank, dt_rank, b.B, dstate, dt_rank + dstate,
                                          b.C, dstate, splits, b.xpart, (size_t)M * d_inner * 2, stream)
                    : hx_gemm_bf16(M, nx, d_inner, b.xconv, d_inner, w.w_x, d_inner, nullptr, 0, HX_BF16,
                                   b.dtlo, dt_rank, dt_rank, b.B, dstate, dt_rank + dstate, b.C, dstate,
                                   stream);
    if (rc) return rc;
    // dt_proj: [M, dt_rank] x [d_inner, dt_rank]^T -> dt (dt_bias is added inside the scan)
    if ((rc = hx_gemm_bf16(M, d_inner, dt_rank, b.dtlo, dt_rank, w.w_dt, dt_rank, nullptr, 0,
                           HX_BF16, b.dt, d_inner, d_inner, nullptr, 0, d_inner, nullptr, 0, stream)))
        return rc;
    if ((rc = hx_selective_scan_fwd(batch, seqlen, d_inner, dstate, HX_BF16, 1, b.xconv, b.dt, w.A,
                                    b.B, b.C, w.D, b.z, w.dt_bias, b.y, nullptr, last_state, stream)))
        return rc;
    // out_proj: [M, d_inner] x [d_model, d_inner]^T -> out (+= out when accumulating)
    return hx_gemm_bf16(M, d_model, d_inner, b.y, d_inner, w.w_out, d_inner, nullptr,
                        accumulate ? 2 : 0, out_dtype, out, d_model, d_model, nullptr, 0, d_model,
                        nullptr, 0, stream);
}

}  // namespace

extern "C" int hx_mamba_block_fwd(int64_t batch, int64_t seqlen, int64_t d_model, int64_t d_inner,
                                  int64_t dstate, int64_t dt_rank, int64_t d_conv,
                                  const void* x, const void* w_in, const float* conv_w,
                                  const float* conv_b, const void* w_x, const void* w_dt,
                                  const float* dt_bias, const float* A, const float* D,
                                  const void* w_out, void* out, void* workspace,
                                  size_t workspace_bytes, void* stream) {
    using namespace hx;
    const BlockWeights w{w_in, w_x, w_dt, w_out, conv_w, conv_b, dt_bias, A, D};
    int rc;
    if ((rc = check_block_args(batch, seqlen, d_model, d_inner, dstate, dt_rank, d_conv, w))) return rc;
    if (batch == 0 || seqlen == 0) return HX_OK;
    HX_REQUIRE(x && out && workspace, HX_ERR_INVALID_INPUT, "mamba_block: x, out, workspace required");
    const size_t need = hx_mamba_block_workspace_size(batch, seqlen, d_inner, dt_rank, dstate);
    HX_REQUIRE(workspace_bytes >= need, HX_ERR_INVALID_INPUT,
               "mamba_block: workspace %zu bytes < %zu required", workspace_bytes, need);
    const BlockBufs b = carve((char*)workspace, batch * seqlen, d_inner, dt_rank, dstate);
    return block_core(batch, seqlen, d_model, d_inner, dstate, dt_rank, d_conv, x, w, out, HX_BF16,
                      false, nullptr, nullptr, b, stream);
}

extern "C" int hx_mamba_layer_fwd(int64_t batch, int64_t seqlen, int64_t d_model, int64_t d_inner,
                                  int64_t dstate, int64_t dt_rank, int64_t d_conv, float* resid,
                                  const float* norm_w, float eps, const void* w_in,
                                  const float* conv_w, const float* conv_b, const void* w_x,
                                  const void* w_dt, const float* dt_bias, const float* A,
                                  const float* D, const void* w_out, float* ssm_state,
                                  float* conv_state, void* workspace, size_t workspace_bytes,
                                  void* stream) {
    using namespace hx;
    const BlockWeights w{w_in, w_x, w_dt, w_out, conv_w, conv_b, dt_bias, A, D};
    int rc;
    if ((rc = check_block_args(batch, seqlen, d_model, d_inner, dstate, dt_rank, d_conv, w))) return rc;
    if (batch == 0 || seqlen == 0) return HX_OK;
    HX_REQUIRE(resid && norm_w && workspace, HX_ERR_INVALID_INPUT,
               "mamba_layer: resid, norm_w, workspace required");
    const int64_t M = batch * seqlen;
    const size_t need = hx_mamba_layer_workspace_size(batch, seqlen, d_model, d_inner, dt_rank, dstate);
    HX_REQUIRE(workspace_bytes >= need, HX_ERR_INVALID_INPUT,
               "mamba_layer: workspace %zu bytes < %zu required", workspace_bytes, need);
    char* p = (char*)workspace;
    void* xn = p;
    const BlockBufs b = carve(p + align256((size_t)M * d_model * 2), M, d_inner, dt_rank, dstate);
    if ((rc = hx_rmsnorm_fwd(M, d_model, resid, norm_w, eps, HX_BF16, xn, stream))) return rc;
    return block_core(batch, seqlen, d_model, d_inner, dstate, dt_rank, d_conv, xn, w, resid, HX_F32,
                      true, ssm_state, conv_state, b, stream);
}

extern "C" int hx_mamba_layer_decode(int64_t batch, int64_t d_model, int64_t d_inner,
                                     int64_t dstate, int64_t dt_rank, int64_t d_conv, float* resid,
                                     const float* norm_w, float eps, const void* w_in,
                                     const float* conv_w, const float* conv_b, const void* w_x,
                                     const void* w_dt, const float* dt_bias, const float* A,
                                     const float* D, const void* w_out, float* ssm_state,
                                     float* conv_state, void* workspace, size_t workspace_bytes,
                                     void* stream) {
    using namespace hx;
    const BlockWeights w{w_in, w_x, w_dt, w_out, conv_w, conv_b, dt_bias, A, D};
    int rc;
    if ((rc = check_block_args(batch, 1, d_model, d_inner, dstate, dt_rank, d_conv, w))) return rc;
    if (batch == 0) return HX_OK;
    HX_REQUIRE(resid && norm_w && ssm_state && workspace && (d_conv == 1 || conv_state),
               HX_ERR_INVALID_INPUT, "mamba_layer_decode: resid, norm_w, ssm_state, conv_state, "
                                     "workspace required");
    const size_t need = hx_mamba_layer_workspace_size(batch, 1, d_model, d_inner, dt_rank, dstate);
    HX_REQUIRE(workspace_bytes >= need, HX_ERR_INVALID_INPUT,
               "mamba_layer_decode: workspace %zu bytes < %zu required", workspace_bytes, need);
    char* p = (char*)workspace;
    void* xn = p;
    const BlockBufs b = carve(p + align256((size_t)batch * d_model * 2), batch, d_inner, dt_rank, dstate);
    if ((rc = hx_rmsnorm_fwd(batch, d_model, resid, norm_w, eps, HX_BF16, xn, stream))) return rc;
    if ((rc = hx_gemm_bf16(batch, 2 * d_inner, d_model, xn, d_model, w.w_in, d_model, nullptr, 0,
                           HX_BF16, b.xpart, d_inner, d_inner, b.z, d_inner, 2 * d_inner, nullptr,
                           0, stream)))
        return rc;
    if ((rc = hx_conv1d_step(batch, d_inner, d_conv, HX_BF16, b.xpart, d_inner, w.conv_w, w.conv_b,
                             conv_state, b.xconv, stream)))
        return rc;
    if ((rc = hx_gemm_bf16(batch, dt_rank + 2 * dstate, d_inner, b.xconv, d_inner, w.w_x, d_inner,
                           nullptr, 0, HX_BF16, b.dtlo, dt_rank, dt_rank, b.B, dstate,
                           dt_rank + dstate, b.C, dstate, stream)))
        return rc;
    if ((rc = hx_gemm_bf16(batch, d_inner, dt_rank, b.dtlo, dt_rank, w.w_dt, dt_rank, nullptr, 0,
                           HX_BF16, b.dt, d_inner, d_inner, nullptr, 0, d_inner, nullptr, 0, stream)))
        return rc;
    if ((rc = hx_selective_state_update(batch, d_inner, dstate, HX_BF16, 1, ssm_state, b.xconv, b.dt,
                                        w.A, b.B, b.C, w.D, b.z, w.dt_bias, b.y, stream)))
        return rc;
    return hx_gemm_bf16(batch, d_model, d_inner, b.y, d_inner, w.w_out, d_inner, nullptr, 2, HX_F32,
                        resid, d_model, d_model, nullptr, 0, d_model, nullptr, 0, stream);
}

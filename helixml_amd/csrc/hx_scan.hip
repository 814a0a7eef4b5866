// hx_scan.hip — fused Mamba selective-scan forward and single-step state update for gfx950.
//
// Semantics (the north-star scan; reference discretisation crates/nn/src/ssm.rs:108-130, SiLU
// backend-cpu/src/lib.rs:1158-1162), per batch b, channel d, state n, time t ascending:
//   dt = softplus(delta + dt_bias);  h[n] = exp(dt*A[d,n])*h[n] + dt*u*B[b,t,n]
//   y  = sum_n C[b,t,n]*h[n] + D[d]*u;  out = y * silu(z)
//
// Work decomposition of the fast path (dstate == 16):
//   * lanes = 64 consecutive channels, so every row access to u/delta/z/out is a 256-byte
//     coalesced segment;
//   * a block has W waves; wave w owns states [w*16/W, (w+1)*16/W) of those 64 channels, so the
//     B[b,t,n] / C[b,t,n] values it needs are wave-uniform: scalar loads into SGPRs that feed
//     the VALU FMAs directly (no per-lane copies of B/C);
//   * time runs in chunks of TCH steps. The per-(t,d) work done once per element (loads,
//     softplus, dt*u; later D*u, SiLU(z), the store) is split across the W waves and exchanged
//     through LDS; the per-state work (exp2, two FMAs, readout FMA) runs on every wave.
// The state stays in VGPRs for the whole sequence; HBM is read once (u, delta, z) and written
// once (out). This kernel is VALU/transcendental-bound at about 4 VALU + 1 v_exp per
// state-update, which is why it runs on VALU and not MFMA.
#include "hx_common.h"

namespace hx {
namespace {

template <typename T>
__device__ inline float ld(const T* p) { return Storage<T>::load(p); }

// ----------------------------------------------------------------------------- fast path
template <typename T, int W, int TCH, bool HAS_Z, bool SOFTPLUS>
__global__ __launch_bounds__(64 * W) void scan_fwd_kernel(
    int64_t L, int64_t Dm,
    const T* __restrict__ u, const T* __restrict__ delta, const float* __restrict__ A,
    const T* __restrict__ Bm, const T* __restrict__ Cm, const float* __restrict__ Dv,
    const T* __restrict__ z, const float* __restrict__ dt_bias, T* __restrict__ out,
    const float* __restrict__ init_state, float* __restrict__ last_state) {
    constexpr int NS = 16;
    constexpr int SPW = NS / W;    // states per wave
    constexpr int SPS = TCH / W;   // pre/post steps per wave per chunk
    static_assert(NS % W == 0 && TCH % W == 0, "bad tiling");

    __shared__ float2 s_du[W > 1 ? TCH : 1][64];
    __shared__ float s_part[W > 1 ? 2 : 1][W][W > 1 ? TCH : 1][64];

    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t b = blockIdx.y;
    const int64_t d = (int64_t)blockIdx.x * 64 + lane;
    const bool dvalid = d < Dm;
    const int64_t dc = dvalid ? d : Dm - 1;

    const int64_t row0 = b * L * Dm + dc;  // element (b, 0, dc)
    const T* __restrict__ up = u + row0;
    const T* __restrict__ dp = delta + row0;
    const T* __restrict__ zp = HAS_Z ? z + row0 : nullptr;
    T* __restrict__ op = out + row0;
    const T* __restrict__ Bp = Bm + b * L * NS + w * SPW;  // wave-uniform
    const T* __restrict__ Cp = Cm + b * L * NS + w * SPW;

    float A2[SPW], h[SPW];
#pragma unroll
    for (int k = 0; k < SPW; ++k) {
        A2[k] = A[dc * NS + w * SPW + k] * kLog2e;
        h[k] = init_state ? init_state[(b * Dm + dc) * NS + w * SPW + k] : 0.0f;
    }
    const float Dd = Dv ? Dv[dc] : 0.0f;
    const float bias = dt_bias ? dt_bias[dc] : 0.0f;

    int buf = 0;
    for (int64_t t0 = 0; t0 < L; t0 += TCH) {
        // ---- pre: this wave's share of the chunk's per-element work
        float uu[SPS], zz[SPS];
        float2 q_reg[W == 1 ? TCH : 1];
#pragma unroll
        for (int i = 0; i < SPS; ++i) {
            const int s = (W > 1) ? (w + i * W) : i;
            const int64_t t = t0 + s;
            const bool tv = t < L;
            const int64_t tc = tv ? t : L - 1;
            uu[i] = ld(up + tc * Dm);
            float dl = ld(dp + tc * Dm) + bias;
            zz[i] = HAS_Z ? ld(zp + tc * Dm) : 0.0f;
            if (SOFTPLUS) dl = softplus(dl);
            dl = tv ? dl : 0.0f;  // steps past the end leave the state unchanged
            const float2 q = make_float2(dl, dl * uu[i]);
            if (W > 1) s_du[s][lane] = q;
            else q_reg[i] = q;
        }
        if (W > 1) __syncthreads();

        // ---- main: every wave advances its states through all TCH steps
        float part[W == 1 ? TCH : 1];
#pragma unroll
        for (int s = 0; s < TCH; ++s) {
            const float2 q = (W > 1) ? s_du[s][lane] : q_reg[s];
            const int64_t tc = (t0 + s < L) ? t0 + s : L - 1;
            const T* Bs = Bp + tc * NS;
            const T* Cs = Cp + tc * NS;
            float acc = 0.0f;
#pragma unroll
            for (int k = 0; k < SPW; ++k) {
                const float ab = fast_exp2(q.x * A2[k]);
                h[k] = fmaf(ab, h[k], q.y * ld(Bs + k));
                acc = fmaf(ld(Cs + k), h[k], acc);
            }
            if (W > 1) s_part[buf][w][s][lane] = acc;
            else part[s] = acc;
        }
        if (W > 1) __syncthreads();

        // ---- post: this wave's share of readout, D skip, SiLU gate, store
#pragma unroll
        for (int i = 0; i < SPS; ++i) {
            const int s = (W > 1) ? (w + i * W) : i;
            const int64_t t = t0 + s;
            float y;
            if (W > 1) {
                y = 0.0f;
#pragma unroll
                for (int ww = 0; ww < W; ++ww) y += s_part[buf][ww][s][lane];
            } else {
                y = part[i];
            }
            y = fmaf(Dd, uu[i], y);
            if (HAS_Z) y *= silu(zz[i]);
            if (dvalid && t < L) Storage<T>::store(op + t * Dm, y);
        }
        buf ^= 1;
    }
    if (last_state && dvalid) {
#pragma unroll
        for (int k = 0; k < SPW; ++k) last_state[(b * Dm + d) * NS + w * SPW + k] = h[k];
    }
}

// ----------------------------------------------------------------------------- generic path
// One thread per (b, d), states in registers, any dstate <= NMAX, no alignment assumptions.
template <typename T, int NMAX>
__global__ __launch_bounds__(128) void scan_fwd_generic_kernel(
    int64_t Bt, int64_t L, int64_t Dm, int64_t N, int softplus_on,
    const T* __restrict__ u, const T* __restrict__ delta, const float* __restrict__ A,
    const T* __restrict__ Bm, const T* __restrict__ Cm, const float* __restrict__ Dv,
    const T* __restrict__ z, const float* __restrict__ dt_bias, T* __restrict__ out,
    const float* __restrict__ init_state, float* __restrict__ last_state) {
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= Bt * Dm) return;
    const int64_t b = gid / Dm, d = gid % Dm;
    float h[NMAX], A2[NMAX];
#pragma unroll
    for (int n = 0; n < NMAX; ++n) {
        A2[n] = n < N ? A[d * N + n] * kLog2e : 0.0f;
        h[n] = (n < N && init_state) ? init_state[(b * Dm + d) * N + n] : 0.0f;
    }
    const float Dd = Dv ? Dv[d] : 0.0f;
    const float bias = dt_bias ? dt_bias[d] : 0.0f;
    for (int64_t t = 0; t < L; ++t) {
        const int64_t i = (b * L + t) * Dm + d;
        const float uv = ld(u + i);
        float dl = ld(delta + i) + bias;
        if (softplus_on) dl = softplus(dl);
        const float du = dl * uv;
        const T* Bs = Bm + (b * L + t) * N;
        const T* Cs = Cm + (b * L + t) * N;
        float y = 0.0f;
#pragma unroll
        for (int n = 0; n < NMAX; ++n) {
            if (n < N) {
                const float ab = fast_exp2(dl * A2[n]);
                h[n] = fmaf(ab, h[n], du * ld(Bs + n));
                y = fmaf(ld(Cs + n), h[n], y);
            }
        }
        y = fmaf(Dd, uv, y);
        if (z) y *= silu(ld(z + i));
        Storage<T>::store(out + i, y);
    }
    if (last_state) {
#pragma unroll
        for (int n = 0; n < NMAX; ++n)
            if (n < N) last_state[(b * Dm + d) * N + n] = h[n];
    }
}

// ----------------------------------------------------------------------------- decode step
template <typename T, int NMAX>
__global__ __launch_bounds__(128) void state_update_kernel(
    int64_t Bt, int64_t Dm, int64_t N, int softplus_on, float* __restrict__ state,
    const T* __restrict__ u, const T* __restrict__ delta, const float* __restrict__ A,
    const T* __restrict__ Bm, const T* __restrict__ Cm, const float* __restrict__ Dv,
    const T* __restrict__ z, const float* __restrict__ dt_bias, T* __restrict__ out) {
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= Bt * Dm) return;
    const int64_t b = gid / Dm, d = gid % Dm;
    const int64_t i = b * Dm + d;
    const float uv = ld(u + i);
    float dl = ld(delta + i) + (dt_bias ? dt_bias[d] : 0.0f);
    if (softplus_on) dl = softplus(dl);
    const float du = dl * uv;
    float* hs = state + i * N;
    float y = 0.0f;
#pragma unroll
    for (int n = 0; n < NMAX; ++n) {
        if (n < N) {
            const float ab = fast_exp2(dl * (A[d * N + n] * kLog2e));
            const float hn = fmaf(ab, hs[n], du * ld(Bm + b * N + n));
            hs[n] = hn;
            y = fmaf(ld(Cm + b * N + n), hn, y);
        }
    }
    if (Dv) y = fmaf(Dv[d], uv, y);
    if (z) y *= silu(ld(z + i));
    Storage<T>::store(out + i, y);
}

// ----------------------------------------------------------------------------- dispatch
struct ScanArgs {
    int64_t Bt, L, Dm, N;
    int softplus;
    const void *u, *delta;
    const float* A;
    const void *B, *C;
    const float* D;
    const void* z;
    const float* dt_bias;
    void* out;
    const float* init_state;
    float* last_state;
    hipStream_t stream;
};

template <typename T, int W, int TCH, bool HAS_Z, bool SP>
int launch_fast(const ScanArgs& a) {
    dim3 grid((unsigned)((a.Dm + 63) / 64), (unsigned)a.Bt);
    hipLaunchKernelGGL((scan_fwd_kernel<T, W, TCH, HAS_Z, SP>), grid, dim3(64 * W), 0, a.stream,
                       a.L, a.Dm, (const T*)a.u, (const T*)a.delta, a.A, (const T*)a.B,
                       (const T*)a.C, a.D, (const T*)a.z, a.dt_bias, (T*)a.out, a.init_state,
                       a.last_state);
    HX_LAUNCH_CHECK();
    return HX_OK;
}

template <typename T, int W, int TCH>
int dispatch_fast(const ScanArgs& a) {
    const bool hz = a.z != nullptr;
    if (hz && a.softplus) return launch_fast<T, W, TCH, true, true>(a);
    if (hz) return launch_fast<T, W, TCH, true, false>(a);
    if (a.softplus) return launch_fast<T, W, TCH, false, true>(a);
    return launch_fast<T, W, TCH, false, false>(a);
}

template <typename T, int NMAX>
int launch_generic(const ScanArgs& a) {
    const int64_t total = a.Bt * a.Dm;
    dim3 grid((unsigned)((total + 127) / 128));
    hipLaunchKernelGGL((scan_fwd_generic_kernel<T, NMAX>), grid, dim3(128), 0, a.stream, a.Bt, a.L,
                       a.Dm, a.N, a.softplus, (const T*)a.u, (const T*)a.delta, a.A,
                       (const T*)a.B, (const T*)a.C, a.D, (const T*)a.z, a.dt_bias, (T*)a.out,
                       a.init_state, a.last_state);
    HX_LAUNCH_CHECK();
    return HX_OK;
}

template <typename T>
int dispatch_generic(const ScanArgs& a) {
    if (a.N <= 4) return launch_generic<T, 4>(a);
    if (a.N <= 8) return launch_generic<T, 8>(a);
    if (a.N <= 16) return launch_generic<T, 16>(a);
    if (a.N <= 32) return launch_generic<T, 32>(a);
    return launch_generic<T, 64>(a);
}

// Kernel variant: 0 = auto, 1/2/4/8 = fast kernel with that many waves, -1 = generic.
// hx_set_scan_variant() sets it; HX_SCAN_VARIANT in the environment gives the initial value.
int g_scan_variant = [] {
    const char* s = getenv("HX_SCAN_VARIANT");
    return s ? atoi(s) : 0;
}();

template <typename T>
int run_scan(const ScanArgs& a) {
    const size_t es = sizeof(T);
    const bool fast_ok = a.N == 16 && aligned(a.B, 16 * es) && aligned(a.C, 16 * es);
    const int v = g_scan_variant;
    if (!fast_ok || v < 0) return dispatch_generic<T>(a);
    switch (v) {
        case 1: return dispatch_fast<T, 1, 16>(a);
        case 2: return dispatch_fast<T, 2, 16>(a);
        case 8: return dispatch_fast<T, 8, 16>(a);
        default: return dispatch_fast<T, 4, 16>(a);
    }
}

int check_common(int64_t Bt, int64_t L, int64_t Dm, int64_t N, int dtype) {
    HX_REQUIRE(Bt >= 0 && L >= 0 && Dm >= 0, HX_ERR_INVALID_DIMENSION,
               "selective scan: negative size (batch=%lld seqlen=%lld dim=%lld)", (long long)Bt,
               (long long)L, (long long)Dm);
    HX_REQUIRE(N >= 1 && N <= 64, HX_ERR_UNSUPPORTED,
               "selective scan: dstate=%lld not supported (1..64)", (long long)N);
    HX_REQUIRE(dtype == HX_F32 || dtype == HX_BF16, HX_ERR_DTYPE_MISMATCH,
               "selective scan: dtype %d is neither HX_F32 nor HX_BF16", dtype);
    HX_REQUIRE(Bt <= 65535, HX_ERR_UNSUPPORTED, "selective scan: batch %lld > 65535",
               (long long)Bt);
    return HX_OK;
}

}  // namespace
}  // namespace hx

extern "C" int hx_selective_scan_fwd(int64_t batch, int64_t seqlen, int64_t dim, int64_t dstate,
                                     int dtype, int delta_softplus, const void* u,
                                     const void* delta, const float* A, const void* B,
                                     const void* C, const float* D, const void* z,
                                     const float* dt_bias, void* out, const float* init_state,
                                     float* last_state, void* stream) {
    if (int rc = hx::check_common(batch, seqlen, dim, dstate, dtype)) return rc;
    if (batch == 0 || dim == 0) return HX_OK;
    HX_REQUIRE(A != nullptr, HX_ERR_INVALID_INPUT, "selective scan: A is NULL");
    if (seqlen == 0) {
        // Zero-length sequence: no output rows; the final state is the initial state.
        if (last_state) {
            const size_t bytes = (size_t)batch * dim * dstate * sizeof(float);
            if (init_state)
                HX_HIP_CHECK(hipMemcpyAsync(last_state, init_state, bytes, hipMemcpyDeviceToDevice,
                                            hx::as_stream(stream)));
            else
                HX_HIP_CHECK(hipMemsetAsync(last_state, 0, bytes, hx::as_stream(stream)));
        }
        return HX_OK;
    }
    HX_REQUIRE(u && delta && B && C && out, HX_ERR_INVALID_INPUT,
               "selective scan: u, delta, B, C and out must be non-NULL");
    hx::ScanArgs a{batch, seqlen, dim,     dstate,     delta_softplus != 0,
                   u,     delta,  A,       B,          C,
                   D,     z,      dt_bias, out,        init_state,
                   last_state,    hx::as_stream(stream)};
    return dtype == HX_F32 ? hx::run_scan<float>(a) : hx::run_scan<uint16_t>(a);
}

extern "C" int hx_set_scan_variant(int variant) {
    HX_REQUIRE(variant == 0 || variant == -1 || variant == 1 || variant == 2 || variant == 4 ||
                   variant == 8,
               HX_ERR_INVALID_INPUT, "hx_set_scan_variant: %d is not one of 0, -1, 1, 2, 4, 8",
               variant);
    hx::g_scan_variant = variant;
    return HX_OK;
}

extern "C" int hx_selective_state_update(int64_t batch, int64_t dim, int64_t dstate, int dtype,
                                         int delta_softplus, float* state, const void* u,
                                         const void* delta, const float* A, const void* B,
                                         const void* C, const float* D, const void* z,
                                         const float* dt_bias, void* out, void* stream) {
    if (int rc = hx::check_common(batch, 1, dim, dstate, dtype)) return rc;
    if (batch == 0 || dim == 0) return HX_OK;
    HX_REQUIRE(state && u && delta && A && B && C && out, HX_ERR_INVALID_INPUT,
               "state update: state, u, delta, A, B, C and out must be non-NULL");
    const int64_t total = batch * dim;
    dim3 grid((unsigned)((total + 127) / 128));
    auto s = hx::as_stream(stream);
#define HX_SU(T, NM)                                                                          \
    hipLaunchKernelGGL((hx::state_update_kernel<T, NM>), grid, dim3(128), 0, s, batch, dim,   \
                       dstate, delta_softplus, state, (const T*)u, (const T*)delta, A,        \
                       (const T*)B, (const T*)C, D, (const T*)z, dt_bias, (T*)out)
#define HX_SU_N(T)                                                                            \
    if (dstate <= 16) HX_SU(T, 16);                                                           \
    else HX_SU(T, 64);
    if (dtype == HX_F32) { HX_SU_N(float) } else { HX_SU_N(uint16_t) }
#undef HX_SU_N
#undef HX_SU
    HX_LAUNCH_CHECK();
    return HX_OK;
}

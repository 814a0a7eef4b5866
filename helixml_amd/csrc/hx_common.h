// hx_common.h — shared host/device helpers for libhelix_hip.so (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_bf16.h>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>

#include "helix_hip.h"

namespace hx {

// ------------------------------------------------------------------ error plumbing (host)
// Sets the calling thread's last-error text and returns `code`. Every C entry point reports
// failures through this, so hx_last_error() always names the check that failed.
int set_error(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();

// Resolves the current device's address of the no-allocation scan's device scratch (once per
// device; hx_init calls it). *out (nullable) receives the address.
int scan_scratch_setup(void** out);

// Whether the current device grants kernel `fn` `dyn_bytes` of dynamic LDS next to `static_bytes`
// of static LDS; the first query per (kernel, device, size) raises the kernel's dynamic-LDS limit
// (hipFuncSetAttribute), later ones return the stored answer. Thread-safe.
bool grant_dynamic_lds(const void* fn, size_t dyn_bytes, size_t static_bytes);
// Compute units of the current device (stored per device; 256 if the query fails). Thread-safe.
int device_cus();
// Whether hx_gemm_bf16's automatic choice takes the narrow kernel (64-row tiles holding every
// column: N <= 192, K >= 1024, K % 64 == 0). It depends on the weight shape only, so every M
// gets the same arithmetic per row.
bool gemm_narrow_auto(int64_t N, int64_t K);
// Y = bf16(rmsnorm(X) * nw) . W^T in one launch: hx_rmsnorm_fwd's bf16 output (X fp32 [M, ldx],
// nw fp32 [K]) fed to hx_gemm_bf16 (no bias, no activation; the same output arguments), with the
// normalisation done in the small-M GEMM kernel's operand load. gemm_rmsnorm_small_ok tells
// whether the sizes and alignment fit: the automatic GEMM choice, the small-M kernel for M x N
// (fewer than 128 tiles of 128 x 128) and K <= 512 in 8-wide pieces (16-byte aligned rows).
bool gemm_rmsnorm_small_ok(int64_t M, int64_t N, int64_t K, const float* X, int64_t ldx,
                           const float* nw, const void* W, int64_t ldw);
int gemm_rmsnorm_small(int64_t M, int64_t N, int64_t K, const float* X, int64_t ldx, const float* nw,
                       float eps, const void* W, int64_t ldw, int out_dtype, void* Y0, int64_t ld0,
                       int64_t split1, void* Y1, int64_t ld1, int64_t split2, void* Y2, int64_t ld2,
                       hipStream_t stream);

// The Mamba block's dt_proj and selective scan in one launch (bf16 storage, dstate 16, softplus,
// z gate, zero initial state): delta = bf16(dt_lo . w_dt^T) is formed per 16-step chunk on the
// matrix core inside the wave kernel instead of being read from memory. dt_lo [batch, seqlen,
// rank], w_dt [dim, rank] bf16; the other operands as hx_selective_scan_fwd's. scan_dtproj_ok
// tells whether the sizes fit (rank 32, 64, 96 or 128; seqlen * dim < 2^31); it depends on the
// weight shape and the sizes only, not on the data.
bool scan_dtproj_ok(int64_t batch, int64_t seqlen, int64_t dim, int64_t rank);
// Whether the calling thread's scan variant (hx_set_scan_variant) is the automatic choice; a
// forced variant also makes the block run its dt projection and scan as separate steps.
bool scan_variant_is_auto();
int scan_fwd_dtproj(int64_t batch, int64_t seqlen, int64_t dim, const uint16_t* u, const uint16_t* dtlo,
                    int64_t rank, const uint16_t* w_dt, const float* A, const uint16_t* B,
                    const uint16_t* C, const float* D, const uint16_t* z, const float* dt_bias,
                    uint16_t* out, float* last_state, hipStream_t stream);

#define HX_HIP_CHECK(expr)                                                                   \
    do {                                                                                     \
        hipError_t hx_e_ = (expr);                                                           \
        if (hx_e_ != hipSuccess)                                                             \
            return ::hx::set_error(HX_ERR_BACKEND, "%s failed: %s (%s:%d)", #expr,           \
                                   hipGetErrorString(hx_e_), __FILE__, __LINE__);            \
    } while (0)

// Checks the launch that was just issued.
#define HX_LAUNCH_CHECK() HX_HIP_CHECK(hipGetLastError())

#define HX_REQUIRE(cond, code, ...)                                                          \
    do {                                                                                     \
        if (!(cond)) return ::hx::set_error((code), __VA_ARGS__);                            \
    } while (0)

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

inline bool aligned(const void* p, size_t a) {
    return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0;
}

// ------------------------------------------------------------------ device helpers
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// fp32 -> bf16 on gfx950's converter (v_cvt_pk_bf16_f32): round to nearest even, a NaN stays a
// quiet NaN, branch-free. Two values convert in one instruction; `a` lands in the low half.
typedef float hx_f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 hx_bf16x2 __attribute__((ext_vector_type(2)));
__device__ inline uint32_t pack_bf16x2(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(hx_f32x2{a, b}, hx_bf16x2));
}

// Storage <-> fp32. bf16 is stored as raw uint16 (upper half of an fp32); conversion to
// storage rounds to nearest even.
template <typename T> struct Storage;
template <> struct Storage<float> {
    __device__ static inline float load(const float* p) { return *p; }
    __device__ static inline void store(float* p, float v) { *p = v; }
};
template <> struct Storage<uint16_t> {
    __device__ static inline float load(const uint16_t* p) {
        return __uint_as_float(static_cast<uint32_t>(*p) << 16);
    }
    __device__ static inline uint16_t round(float v) {
        return __builtin_bit_cast(uint16_t, static_cast<__bf16>(v));
    }
    __device__ static inline void store(uint16_t* p, float v) { *p = round(v); }
};

__device__ inline float bf16_bits_to_f32(uint32_t bits16) { return __uint_as_float(bits16 << 16); }

// Workgroup barrier that orders LDS only. __syncthreads() is a workgroup-scope fence over all
// address spaces, which on gfx9 makes every wave wait for its outstanding global loads and
// stores (vmcnt(0)) at each barrier, defeating register prefetch of the next chunk. Kernels
// that exchange data through LDS only use this instead.
__device__ inline void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Global and LDS pointer types of gfx950's global_load_lds (global memory straight into LDS).
typedef __attribute__((address_space(1))) void gvoid_t;
typedef __attribute__((address_space(3))) void lvoid_t;

// The long-sequence scans' end-state passes stop where every state's decay to its segment's end
// is below 2^-kDecayDropBits: what they leave out is that decay times the state there, 2^-8 of
// the fp32 rounding (2^-24) of that state.
constexpr int kDecayDropBits = 32;
constexpr float kDecayDrop = 0x1p-32f;  // 2^-kDecayDropBits

// exp2 on the transcendental unit (v_exp_f32). Inputs here are finite; underflow flushes to 0.
__device__ inline float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ inline float fast_log2(float x) { return __builtin_amdgcn_logf(x); }
__device__ inline float fast_rcp(float x) { return __builtin_amdgcn_rcpf(x); }

// softplus(x) = log(1 + e^x), x > 20 -> x. With u = fl(1 + e), log1p(e) = log(u) + log(1 + d/u)
// where d = (1 + e) - u is the rounding error of u. For e < 1, d = e - (u - 1) exactly (Fast2Sum,
// Dekker 1971), and log(1 + d/u) = d to within |d| e/(1+e) <= 2^-24 log1p(e); for e >= 1 the
// term is below 2^-24 log(u) and is dropped. Two transcendentals, no reciprocal, and full
// relative accuracy for small e^x (u == 1 gives e).
__device__ inline float softplus(float x) {
    float e = fast_exp2(x * kLog2e);
    float u = 1.0f + e;
    float d = e - (u - 1.0f);
    float r = fast_log2(u) * kLn2 + (e < 1.0f ? d : 0.0f);
    return x > 20.0f ? x : r;
}

// silu(z) = z / (1 + e^-z)   (backend-cpu/src/lib.rs:1158-1162)
__device__ inline float silu(float z) { return z * fast_rcp(1.0f + fast_exp2(-z * kLog2e)); }

}  // namespace hx

// hx_wave.h — wave-level building blocks shared by the scan and S4 kernels (gfx950, wave64):
// DPP lane moves, row (16-lane) and half-wave register swaps, compile-time step unrolling,
// and float4 row loads/stores of fp32 or bf16 storage.
#pragma once
#include <type_traits>

#include "hx_common.h"

namespace hx {

template <int CTRL>
__device__ inline float dpp(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xf, 0xf, true));
}
constexpr int kDppRor8 = 0x128;         // row_ror:8 (lane j <- lane j^8 within a row)
constexpr int kDppHalfMirror = 0x141;   // row_half_mirror (lane j <- 7-j within each 8)
constexpr int kDppXor2 = 0x4E;          // quad_perm [2,3,0,1]
constexpr int kDppXor1 = 0xB1;          // quad_perm [1,0,3,2]
template <int S> constexpr int kDppBcast = 0x150 + S;  // row_newbcast:S

template <int S>
struct StepLoop {
    template <typename F>
    __device__ static inline void run(F&& f) {
        StepLoop<S - 1>::run(f);
        f(std::integral_constant<int, S - 1>{});
    }
};
template <>
struct StepLoop<0> {
    template <typename F>
    __device__ static inline void run(F&&) {}
};

template <typename T> struct Vec4;
template <> struct Vec4<float> {
    using raw = float4;
    __device__ static inline float4 load(const float* p) { return *reinterpret_cast<const float4*>(p); }
    __device__ static inline void store(float* p, float4 v) { *reinterpret_cast<float4*>(p) = v; }
};
template <> struct Vec4<uint16_t> {
    using raw = uint2;
    __device__ static inline float4 load(const uint16_t* p) {
        const uint2 r = *reinterpret_cast<const uint2*>(p);
        return make_float4(__uint_as_float(r.x << 16), __uint_as_float(r.x & 0xffff0000u),
                           __uint_as_float(r.y << 16), __uint_as_float(r.y & 0xffff0000u));
    }
    __device__ static inline void store(uint16_t* p, float4 v) {
        uint2 r;
        r.x = pack_bf16x2(v.x, v.y);
        r.y = pack_bf16x2(v.z, v.w);
        *reinterpret_cast<uint2*>(p) = r;
    }
};

__device__ inline float f4get(const float4& v, int i) {
    return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
}

// Register exchanges across the 4 DPP rows of a wave (no LDS): permlane32_swap swaps this
// lane's register with the lane 32 away, permlane16_swap with the lane 16 away within a half.
__device__ inline void swap32(float& a, float& b) {
    auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false, false);
    a = __uint_as_float(r[0]);
    b = __uint_as_float(r[1]);
}
__device__ inline void swap16(float& a, float& b) {
    auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(b), false, false);
    a = __uint_as_float(r[0]);
    b = __uint_as_float(r[1]);
}

// acc += (c broadcast from lane S of its DPP row) * h, one v_fmac_f32_dpp (the compiler folds
// DPP into v_mul but not into v_fmac).
template <int S>
__device__ inline float fmac_bcast(float acc, float c, float h) {
    asm("v_fmac_f32_dpp %0, %1, %2 row_newbcast:%3 row_mask:0xf bank_mask:0xf bound_ctrl:1"
        : "+v"(acc)
        : "v"(c), "v"(h), "n"(S));
    return acc;
}

// Row-transposing reduce-scatter: P[j] holds this lane's partial for step q(j) where
// q(i + 4*rr) = rr + 4*i; on return Y[i] is the sum over the 4 rows for step r + 4*i (r = own row).
__device__ inline void rows_reduce_scatter(float (&P)[16], float (&Y)[4]) {
    float Q[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        float a = P[i], b = P[i + 8];
        swap32(a, b);  // rows 0,1: (P_i own, P_i of row+2); rows 2,3: (P_{i+8} of row-2, own)
        Q[i] = a + b;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        float a = Q[i], b = Q[i + 4];
        swap16(a, b);
        Y[i] = a + b;  // row r: sum for P index i + 4r
    }
}

// Row all-gather: X[i] holds this lane's value for step r + 4*i (r = own row). On return
// G[rr][i] holds the value of row rr's X[i] (same channel), i.e. step rr + 4*i.
__device__ inline void rows_all_gather(const float (&X)[4], float (&G)[4][4]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        float a = X[i], a2 = X[i];
        swap16(a, a2);  // rows 0,1 -> a: row0's, a2: row1's; rows 2,3 -> a: row2's, a2: row3's
        float b = a, b2 = a;
        swap32(b, b2);  // b: (rows 0,1: row0's; rows 2,3: row0's) ; b2: row2's everywhere
        float c = a2, c2 = a2;
        swap32(c, c2);  // c: row1's; c2: row3's
        G[0][i] = b;
        G[1][i] = c;
        G[2][i] = b2;
        G[3][i] = c2;
    }
}

}  // namespace hx

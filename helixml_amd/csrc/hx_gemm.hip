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
#include "hx_wave.h"

namespace hx {
namespace {

// 0 = automatic, 1 = always the 128 x 128 kernel, 2 = the 256 x 128 kernel where rows are aligned,
// 3 = the small-M kernel (32 x 32 or 32 x 64 tiles, K split over 4 waves) where rows are aligned
// and K % 8 == 0, 4 = the direct-to-LDS 256 x 128 kernel
// where K % 64 == 0 and rows are aligned, 5 / 6 = the direct-to-LDS 256 x 256 kernel with 64- /
// 32-wide K tiles where K is a multiple of them and rows are aligned
thread_local int g_gemm_kernel = 0;  // per calling thread (hx_set_gemm_kernel)

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
    // output and leading dimension of segment s, selected without indexing the arrays with a
    // runtime value (which would place the struct in scratch memory)
    // (a select chain is folded back into an indexed load, so the choice is made with masks)
    __device__ uint64_t pick(uint64_t a, uint64_t b, uint64_t c, int s) const {
        const uint64_t m1 = 0 - (uint64_t)(s == 1), m2 = 0 - (uint64_t)(s == 2), m0 = ~(m1 | m2);
        return (a & m0) | (b & m1) | (c & m2);
    }
    __device__ void* yp(int s) const {
        return (void*)pick((uint64_t)y[0], (uint64_t)y[1], (uint64_t)y[2], s);
    }
    __device__ int64_t ldp(int s) const {
        return (int64_t)pick((uint64_t)ld[0], (uint64_t)ld[1], (uint64_t)ld[2], s);
    }
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
                const int64_t off = row * o.ldp(seg) + cc;
                if (o.out_bf16) {
                    uint16_t* yp = (uint16_t*)o.yp(seg) + off;
                    if (o.act & 2) v += Storage<uint16_t>::load(yp);
                    Storage<uint16_t>::store(yp, v);
                } else {
                    float* yp = (float*)o.yp(seg) + off;
                    if (o.act & 2) v += *yp;
                    *yp = v;
                }
            }
        }
}

// ----------------------------------------------------------------------------- skinny (small M)
// For small M (recurrent decode: one token per sequence, M = batch): a block of NW waves owns one
// 32 x TN output tile and splits K NW ways (wave w takes K-steps w, w + NW, w + 2 NW, ...). Each
// wave loads its A and W fragments straight from global memory into registers (16 bytes per
// lane), SP K-steps at a time — for the decode shapes all of its loads at once, so one round of
// load latency per GEMM — and feeds them to v_mfma_f32_32x32x16_bf16. The NW partial tiles go to
// LDS; then every thread of the block sums PER consecutive outputs of one row over the waves in
// wave order, applies the epilogue and writes the group with one vector store where it lies in
// one output and is aligned (element stores otherwise). Loads are branch-free: a piece past K
// reads the row's first piece and is zeroed by a mask (needs K % 8 == 0 and K >= 8), a row past M
// or N reads the last row (its results are never stored). Rows must be 16-byte aligned.
// Measured on MI355X for the decode projections at M = 256, with 12 weight sets cycled like the
// layers: [2048 x 512] 5.0 us and [512 x 1024] accumulate 5.2 us, against 12.2 and 15.1 us for a
// 32 x 64 kernel whose single wave did the whole epilogue with element stores.
template <int NB>
__device__ inline void vload_bytes(const char* p, uint32_t* d) {  // NB bytes, aligned to min(NB, 16)
    if constexpr (NB >= 16) {
#pragma unroll
        for (int i = 0; i < NB / 16; ++i) {
            const uint4 t = reinterpret_cast<const uint4*>(p)[i];
            d[4 * i] = t.x; d[4 * i + 1] = t.y; d[4 * i + 2] = t.z; d[4 * i + 3] = t.w;
        }
    } else if constexpr (NB == 8) {
        const uint2 t = *reinterpret_cast<const uint2*>(p);
        d[0] = t.x; d[1] = t.y;
    } else {
        static_assert(NB == 4, "vector width");
        d[0] = *reinterpret_cast<const uint32_t*>(p);
    }
}
template <int NB>
__device__ inline void vstore_bytes(char* p, const uint32_t* d) {
    if constexpr (NB >= 16) {
#pragma unroll
        for (int i = 0; i < NB / 16; ++i)
            reinterpret_cast<uint4*>(p)[i] = make_uint4(d[4 * i], d[4 * i + 1], d[4 * i + 2], d[4 * i + 3]);
    } else if constexpr (NB == 8) {
        *reinterpret_cast<uint2*>(p) = make_uint2(d[0], d[1]);
    } else {
        static_assert(NB == 4, "vector width");
        *reinterpret_cast<uint32_t*>(p) = d[0];
    }
}

// XT = uint16_t: X is bf16. XT = float: X is the fp32 rows of an RMSNorm whose output is the
// GEMM's left operand, bf16(x / sqrt(mean(x^2) + eps) * nw) (nn::RMSNorm::forward,
// crates/nn/src/lib.rs:258-285, rounded to bf16 as hx_rmsnorm_fwd's bf16 output): the block
// holds all K of its 32 rows in one round (K <= 16 * NW * SP), so each row's sum of squares is
// formed from the loaded pieces (the two lanes of a row in a wave, then the waves in order) and
// the pieces are normalised and packed to bf16 in registers. nw and eps are unused for bf16 X.
template <int TN, int NW, int SP, typename XT = uint16_t>
__global__ __launch_bounds__(NW * 64) void gemm_bf16_nt_skinny_kernel(int64_t M, int64_t N, int64_t K,
                                                                      const XT* __restrict__ X,
                                                                      int64_t ldx,
                                                                      const uint16_t* __restrict__ W,
                                                                      int64_t ldw,
                                                                      const float* __restrict__ bias,
                                                                      GemmOut o,
                                                                      const float* __restrict__ nw,
                                                                      float eps) {
    constexpr int NT = TN / 32;
    constexpr int PER = 32 * TN / (NW * 64);  // outputs per thread in the epilogue
    constexpr bool NORM = std::is_same_v<XT, float>;
    static_assert(PER >= 2 && (PER & (PER - 1)) == 0 && TN % PER == 0, "epilogue groups");
    __shared__ float part[NW][32][TN + 1];
    __shared__ float rss[NORM ? NW : 1][32];  // per wave: its pieces' sum of squares of each row
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int64_t m0 = (int64_t)blockIdx.y * 32, n0 = (int64_t)blockIdx.x * TN;
    const int fr = lane & 31, fk = (lane >> 5) * 8;
    const XT* xr = X + (m0 + fr < M ? m0 + fr : M - 1) * ldx;
    const uint16_t* wr[NT];
#pragma unroll
    for (int j = 0; j < NT; ++j) {
        const int64_t rb = n0 + 32 * j + fr;
        wr[j] = W + (rb < N ? rb : N - 1) * ldw;
    }
    auto piece = [&](const uint16_t* rowp, int64_t kk, uint32_t msk) __attribute__((always_inline)) {
        uint4 v = *reinterpret_cast<const uint4*>(rowp + kk);
        v.x &= msk; v.y &= msk; v.z &= msk; v.w &= msk;
        return __builtin_bit_cast(bf16x8, v);
    };
    const int64_t nsteps = (K + 15) / 16;
    f32x16 acc[NT];
#pragma unroll
    for (int j = 0; j < NT; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[j][r] = 0.0f;
    if constexpr (NORM) {
        // one straight-line round that every wave runs (the barrier is block-wide); pieces past
        // K load the row's first piece and are masked to zero, so they add nothing to the sums
        float4 xv[SP][2], gv[SP][2];
        bf16x8 b[NT][SP];
        float ss = 0.0f;
#pragma unroll
        for (int q = 0; q < SP; ++q) {
            const int64_t kk = (int64_t)(w + NW * q) * 16 + fk;
            const bool in = kk + 8 <= K;
            const int64_t kc = in ? kk : 0;
            uint32_t msk = in ? 0xffffffffu : 0u;
            asm volatile("" : "+v"(msk));
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                uint4 v = *reinterpret_cast<const uint4*>(xr + kc + 4 * h);
                v.x &= msk; v.y &= msk; v.z &= msk; v.w &= msk;
                xv[q][h] = __builtin_bit_cast(float4, v);
                gv[q][h] = *reinterpret_cast<const float4*>(nw + kc + 4 * h);
            }
#pragma unroll
            for (int j = 0; j < NT; ++j) b[j][q] = piece(wr[j], kc, msk);
        }
#pragma unroll
        for (int q = 0; q < SP; ++q)
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                ss = fmaf(xv[q][h].x, xv[q][h].x, ss);
                ss = fmaf(xv[q][h].y, xv[q][h].y, ss);
                ss = fmaf(xv[q][h].z, xv[q][h].z, ss);
                ss = fmaf(xv[q][h].w, xv[q][h].w, ss);
            }
        {  // lanes fr and fr + 32 hold the two halves of row fr's pieces: both form lo + hi
            float lo = ss, hi = ss;
            swap32(lo, hi);
            ss = lo + hi;
        }
        if (lane < 32) rss[w][fr] = ss;
        __syncthreads();
        float tot = rss[0][fr];
#pragma unroll
        for (int w2 = 1; w2 < NW; ++w2) tot += rss[w2][fr];
        const float inv = 1.0f / sqrtf(tot / (float)K + eps);
#pragma unroll
        for (int q = 0; q < SP; ++q) {
            uint32_t d[4];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const float4 x4 = xv[q][h], g4 = gv[q][h];
                d[2 * h] = pack_bf16x2(x4.x * inv * g4.x, x4.y * inv * g4.y);
                d[2 * h + 1] = pack_bf16x2(x4.z * inv * g4.z, x4.w * inv * g4.w);
            }
            const bf16x8 a = __builtin_bit_cast(bf16x8, make_uint4(d[0], d[1], d[2], d[3]));
#pragma unroll
            for (int j = 0; j < NT; ++j)
                acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b[j][q], acc[j], 0, 0, 0);
        }
    } else
    for (int64_t s0 = w; s0 < nsteps; s0 += (int64_t)NW * SP) {  // wave-uniform rounds
        bf16x8 a[SP], b[NT][SP];
#pragma unroll
        for (int q = 0; q < SP; ++q) {
            const int64_t kk = (s0 + (int64_t)NW * q) * 16 + fk;
            const bool in = kk + 8 <= K;
            const int64_t kc = in ? kk : 0;  // the row's first piece: in bounds since K >= 8
            // a mask the compiler cannot see through keeps the loads unconditional (a select on
            // the loaded value would become a branch around each load)
            uint32_t msk = in ? 0xffffffffu : 0u;
            asm volatile("" : "+v"(msk));
            a[q] = piece(xr, kc, msk);
#pragma unroll
            for (int j = 0; j < NT; ++j) b[j][q] = piece(wr[j], kc, msk);
        }
#pragma unroll
        for (int q = 0; q < SP; ++q)
#pragma unroll
            for (int j = 0; j < NT; ++j)
                acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[q], b[j][q], acc[j], 0, 0, 0);
    }
    // acc[j][r] holds C[8 * (r / 4) + 4 * (lane / 32) + r % 4][32 j + lane % 32]
#pragma unroll
    for (int j = 0; j < NT; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) part[w][8 * (r >> 2) + 4 * (lane >> 5) + (r & 3)][32 * j + fr] = acc[j][r];
    __syncthreads();
    const int row = (threadIdx.x * PER) / TN, c0 = (threadIdx.x * PER) % TN;
    const int64_t grow = m0 + row, gc0 = n0 + c0;
    if (grow >= M || gc0 >= N) return;
    float v[PER];
#pragma unroll
    for (int p = 0; p < PER; ++p) {
        float t = part[0][row][c0 + p];
#pragma unroll
        for (int w2 = 1; w2 < NW; ++w2) t += part[w2][row][c0 + p];
        const int64_t col = gc0 + p < N ? gc0 + p : N - 1;
        t += bias ? bias[col] : 0.0f;
        if (o.act & 1) t = silu(t);
        v[p] = t;
    }
    // the group's output: the segment of its first column (non-empty, so its pointer is set)
    const int seg = gc0 >= o.split2 ? 2 : (gc0 >= o.split1 ? 1 : 0);
    const int64_t seg_lo = seg == 2 ? o.split2 : (seg == 1 ? o.split1 : 0);
    const int64_t seg_hi = seg == 0 ? o.split1 : (seg == 1 ? o.split2 : N);
    const int es = o.out_bf16 ? 2 : 4;
    char* yb = (char*)o.yp(seg) + (grow * o.ldp(seg) + (gc0 - seg_lo)) * es;
    const int vb = PER * es < 16 ? PER * es : 16;  // alignment the vector access needs
    if (gc0 + PER <= seg_hi && ((uintptr_t)yb & (uintptr_t)(vb - 1)) == 0) {
        if (o.out_bf16) {
            uint32_t d[PER / 2];
            if (o.act & 2) {
                vload_bytes<PER * 2>(yb, d);
#pragma unroll
                for (int p = 0; p < PER; ++p)
                    v[p] += __uint_as_float((p & 1) ? (d[p / 2] & 0xffff0000u) : (d[p / 2] << 16));
            }
#pragma unroll
            for (int p = 0; p < PER; p += 2)
                d[p / 2] = pack_bf16x2(v[p], v[p + 1]);
            vstore_bytes<PER * 2>(yb, d);
        } else {
            uint32_t d[PER];
            if (o.act & 2) {
                vload_bytes<PER * 4>(yb, d);
#pragma unroll
                for (int p = 0; p < PER; ++p) v[p] += __uint_as_float(d[p]);
            }
#pragma unroll
            for (int p = 0; p < PER; ++p) d[p] = __float_as_uint(v[p]);
            vstore_bytes<PER * 4>(yb, d);
        }
        return;
    }
#pragma unroll
    for (int p = 0; p < PER; ++p) {
        const int64_t col = gc0 + p;
        if (col >= N) break;
        const int sp = col >= o.split2 ? 2 : (col >= o.split1 ? 1 : 0);
        const int64_t off = grow * o.ldp(sp) + col - (sp == 2 ? o.split2 : (sp == 1 ? o.split1 : 0));
        float t = v[p];
        if (o.out_bf16) {
            uint16_t* yp = (uint16_t*)o.yp(sp) + off;
            if (o.act & 2) t += Storage<uint16_t>::load(yp);
            Storage<uint16_t>::store(yp, t);
        } else {
            float* yp = (float*)o.yp(sp) + off;
            if (o.act & 2) t += *yp;
            *yp = t;
        }
    }
}

// Whole-slab store of a staged 32 x 64 fp32 tile (st, row stride 68) without bias or SiLU,
// with nontemporal stores: an output streams out without displacing the A and W panels the
// other tiles still read from L2 (config 5 in_proj, 537 MB out: 439 -> 391 us):
// `yb` points at the slab's first output element, `ldb` is the output row pitch in bytes, both
// 16-byte aligned. bf16: 8 lanes x 8 columns per row, 8 rows per pass; fp32: 16 lanes x 4
// columns, 4 rows per pass.
// ACC adds the existing output (Y += X W^T), in the same order as the general path; the caller
// loads it (load_slab_old) ahead of time.
typedef uint32_t slab_u32v4 __attribute__((ext_vector_type(4)));
template <bool BF16, int ROWS = 32> struct SlabGeom {  // a slab: ROWS x 64 columns
    static constexpr int LPR = BF16 ? 8 : 16;  // lanes per row
    static constexpr int RPP = 64 / LPR;       // rows per pass
    static constexpr int NP = ROWS / RPP;      // passes
    static constexpr int VW = BF16 ? 8 : 4;    // columns per lane
};

// The existing outputs of a slab, as store_slab_fast's lane reads them (global loads: a flat
// access also counts in lgkmcnt and would hold up the LDS waits).
template <bool BF16, int ROWS = 32>
__device__ inline void load_slab_old(const char* __restrict__ yb, int64_t ldb, int lane,
                                     slab_u32v4 (&old)[SlabGeom<BF16, ROWS>::NP]) {
    using G = SlabGeom<BF16, ROWS>;
    typedef __attribute__((address_space(1))) const slab_u32v4 g_u32v4;
    const int rl = lane / G::LPR, cl = (lane % G::LPR) * G::VW;
    const char* yp = yb + rl * ldb + cl * (BF16 ? 2 : 4);
#pragma unroll
    for (int p = 0; p < G::NP; ++p) old[p] = *(g_u32v4*)(yp + p * G::RPP * ldb);
}

template <bool BF16, bool ACC, int ROWS = 32>
__device__ inline void store_slab_fast(char* __restrict__ yb, int64_t ldb, const float* st, int lane,
                                       const slab_u32v4 (&old)[SlabGeom<BF16, ROWS>::NP]) {
    // explicit address spaces: LDS reads, and global (not flat) output accesses, since a flat
    // access also counts in lgkmcnt and would hold up the next slab's LDS waits until it completes
    typedef uint32_t u32v4 __attribute__((ext_vector_type(4)));
    typedef float f32v4 __attribute__((ext_vector_type(4)));
    typedef __attribute__((address_space(1))) u32v4 g_u32v4;
    typedef __attribute__((address_space(1))) f32v4 g_f32v4;
    typedef __attribute__((address_space(3))) const f32v4 l_f32v4;
    using G = SlabGeom<BF16, ROWS>;
    constexpr int RPP = G::RPP, NP = G::NP, VW = G::VW;
    const int rl = lane / G::LPR, cl = (lane % G::LPR) * VW;
    l_f32v4* sp = (l_f32v4*)(st + rl * 68 + cl);
    char* yp = yb + rl * ldb + cl * (BF16 ? 2 : 4);
    // all of the slab's LDS reads first, so their latencies overlap
    f32v4 v[NP][VW / 4];
#pragma unroll
    for (int p = 0; p < NP; ++p)
#pragma unroll
        for (int h = 0; h < VW / 4; ++h) v[p][h] = sp[p * RPP * 17 + h];  // 17 vectors per row
#pragma unroll
    for (int p = 0; p < NP; ++p) {
        char* q = yp + p * RPP * ldb;
        if constexpr (BF16) {
            float f[8] = {v[p][0].x, v[p][0].y, v[p][0].z, v[p][0].w,
                          v[p][1].x, v[p][1].y, v[p][1].z, v[p][1].w};
            if constexpr (ACC) {
                const uint32_t ow[4] = {old[p].x, old[p].y, old[p].z, old[p].w};
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    f[2 * k] += __uint_as_float(ow[k] << 16);
                    f[2 * k + 1] += __uint_as_float(ow[k] & 0xffff0000u);
                }
            }
            uint32_t wv[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) wv[k] = pack_bf16x2(f[2 * k], f[2 * k + 1]);
            __builtin_nontemporal_store(u32v4{wv[0], wv[1], wv[2], wv[3]}, (g_u32v4*)q);
        } else {
            f32v4 f = v[p][0];
            if constexpr (ACC) {
                f.x += __uint_as_float(old[p].x);
                f.y += __uint_as_float(old[p].y);
                f.z += __uint_as_float(old[p].z);
                f.w += __uint_as_float(old[p].w);
            }
            __builtin_nontemporal_store(f, (g_f32v4*)q);
        }
    }
}

// Writes a wave's staged nrows x 64 fp32 tile (st, row stride 68) to the outputs: rows of 64
// columns as 16-byte vectors (8 bf16 or 4 fp32 per lane) with bias, SiLU and accumulate; a
// vector that would straddle a column split or the N edge falls back to element stores.
__device__ inline void store_tile_rows(const GemmOut& o, const float* __restrict__ bias,
                                       const float* st, int64_t M, int64_t N, int64_t row0,
                                       int64_t col0, int lane, int nrows = 32) {
        // rows of 64 columns: o.out_bf16 -> 8 lanes x 8 columns per row (8 rows per pass),
        // fp32 -> 16 lanes x 4 columns per row (4 rows per pass)
        const int vw = o.out_bf16 ? 8 : 4;
        const int lpr = 64 / vw;             // lanes per row
        const int rpp = 64 / lpr;            // rows per pass
        const int rl = lane / lpr, cl = (lane % lpr) * vw;
        for (int rr = rl; rr < nrows; rr += rpp) {
            const int64_t row = row0 + rr;
            const int64_t col = col0 + cl;
            if (row >= M || col >= N) continue;
            float v[8];
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                if (q < vw) {
                    float x = st[rr * 68 + cl + q];
                    if (bias && col + q < N) x += bias[col + q];
                    if (o.act & 1) x = silu(x);
                    v[q] = x;
                }
            }
            int seg = 0;
            int64_t cc = col;
            if (col >= o.split2) { seg = 2; cc = col - o.split2; }
            else if (col >= o.split1) { seg = 1; cc = col - o.split1; }
            const int64_t seg_end = seg == 0 ? o.split1 : seg == 1 ? o.split2 : N;
            const int64_t off = row * o.ldp(seg) + cc;
            const bool whole = col + vw <= seg_end &&
                               ((uintptr_t)((char*)o.yp(seg) + off * (o.out_bf16 ? 2 : 4)) & 15) == 0;
            if (whole) {
                if (o.out_bf16) {
                    uint16_t* yp = (uint16_t*)o.yp(seg) + off;
                    if (o.act & 2) {
                        const uint4 old = *reinterpret_cast<const uint4*>(yp);
                        const uint32_t ow[4] = {old.x, old.y, old.z, old.w};
#pragma unroll
                        for (int q = 0; q < 4; ++q) {
                            v[2 * q] += __uint_as_float(ow[q] << 16);
                            v[2 * q + 1] += __uint_as_float(ow[q] & 0xffff0000u);
                        }
                    }
                    uint32_t wv[4];
#pragma unroll
                    for (int q = 0; q < 4; ++q)
                        wv[q] = pack_bf16x2(v[2 * q], v[2 * q + 1]);
                    *reinterpret_cast<uint4*>(yp) = make_uint4(wv[0], wv[1], wv[2], wv[3]);
                } else {
                    float* yp = (float*)o.yp(seg) + off;
                    if (o.act & 2) {
                        const float4 old = *reinterpret_cast<const float4*>(yp);
                        v[0] += old.x; v[1] += old.y; v[2] += old.z; v[3] += old.w;
                    }
                    *reinterpret_cast<float4*>(yp) = make_float4(v[0], v[1], v[2], v[3]);
                }
            } else {
                for (int q = 0; q < vw; ++q) {
                    const int64_t cq = col + q;
                    if (cq >= N) break;
                    int sq = 0;
                    int64_t ccq = cq;
                    if (cq >= o.split2) { sq = 2; ccq = cq - o.split2; }
                    else if (cq >= o.split1) { sq = 1; ccq = cq - o.split1; }
                    const int64_t oq = row * o.ldp(sq) + ccq;
                    float x = v[q];
                    if (o.out_bf16) {
                        uint16_t* yp = (uint16_t*)o.yp(sq) + oq;
                        if (o.act & 2) x += Storage<uint16_t>::load(yp);
                        Storage<uint16_t>::store(yp, x);
                    } else {
                        float* yp = (float*)o.yp(sq) + oq;
                        if (o.act & 2) x += *yp;
                        *yp = x;
                    }
                }
            }
        }
}

// Tile order of the big-tile kernels (blocks = tiles, one or two per CU). Consecutive block ids
// go to different XCDs (8, each with its own L2), so each XCD takes a contiguous run of the
// row-major tile range; when that run is whole row panels, its tiles go out in groups of up to 4
// row panels, column-major inside a group, so the tiles in flight on an XCD (one per CU) share
// 4 A panels and a few W panels instead of one A panel and every W panel (config 3 in_proj with
// 256 x 256 tiles: 12 MB instead of 33 MB through L2 per round, 585 -> 495 us).
__device__ inline void tile_of(int nbx, int nb, int bid, int& tm, int& tn) {
    if ((nb & 7) == 0 && ((nb >> 3) % nbx) == 0) {
        const int rows_x = (nb >> 3) / nbx;  // row panels per XCD
        const int xcd = bid & 7, li = bid >> 3;
        const int gm = rows_x < 4 ? rows_x : 4;
        const int g = li / (gm * nbx), rem = li % (gm * nbx);
        const int rig = rows_x - g * gm < gm ? rows_x - g * gm : gm;  // row panels in this group
        tm = xcd * rows_x + g * gm + rem % rig;
        tn = rem / rig;
    } else {
        if ((nb & 7) == 0) bid = (bid & 7) * (nb >> 3) + (bid >> 3);
        tm = bid / nbx;
        tn = bid % nbx;
    }
}

// ----------------------------------------------------------------------------- 256 x 128 tiles
constexpr int LBM = 256, LBN = 128, LBK = 64;

// ----------------------------------------------------------------------------- direct-to-LDS
// Block tile 256 x 128 x 64, 4 waves in 2 x 2, each wave 128 x 64 = 4 x 2 tiles of
// v_mfma_f32_32x32x16_bf16. Tiles move from global memory straight into LDS with gfx950's
// global_load_lds_dwordx4 (64 lanes x 16 bytes into
// one contiguous KiB of LDS per instruction): no register staging, a 3-stage LDS ring, and the
// loads of tile kt+2 issued while tile kt is multiplied. Each KiB holds 8 tile rows of 128 bytes;
// within a row the 16-byte K-chunks are XOR-swizzled (chunk c of row r sits in slot c ^ (r & 7))
// by choosing which global chunk each lane loads, so the MFMA fragment reads (one chunk of 32
// consecutive rows) spread over the banks. Requires K % 64 == 0 and 16-byte aligned rows; rows
// past M or N are clamped (their outputs are discarded).
constexpr int DSTAGES = 3;
constexpr int DSTAGE_BYTES = (LBM + LBN) * LBK * 2;  // 48 KiB

__global__ __launch_bounds__(256) void gemm_bf16_nt_dlds_kernel(int64_t M, int64_t N, int64_t K,
                                                                const uint16_t* __restrict__ X,
                                                                int64_t ldx,
                                                                const uint16_t* __restrict__ W,
                                                                int64_t ldw,
                                                                const float* __restrict__ bias,
                                                                GemmOut o) {
    extern __shared__ __attribute__((aligned(16))) uint16_t smem[];
    char* sbase = reinterpret_cast<char*>(smem);

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    const int nbx = gridDim.x, nby = gridDim.y;
    const int nb = nbx * nby;
    int tm, tn;
    tile_of(nbx, nb, blockIdx.y * nbx + blockIdx.x, tm, tn);
    const int64_t m0 = (int64_t)tm * LBM, n0 = (int64_t)tn * LBN;

    // this lane's 12 global sources per tile: wave w issues KiB regions q = 12w .. 12w + 11 of
    // the 48 KiB stage (0..31 = A rows 8q.., 32..47 = B rows 8(q-32)..); lane L fills row
    // 8q' + L/8, slot L%8 with K-chunk (L%8) ^ (row & 7)
    const uint16_t* src[12];
#pragma unroll
    for (int j = 0; j < 12; ++j) {
        const int q = wave * 12 + j;
        const bool isA = q < 32;
        const int row = (isA ? q : q - 32) * 8 + (lane >> 3);
        const int chunk = (lane & 7) ^ (row & 7);
        if (isA) {
            const int64_t gr = m0 + row < M ? m0 + row : M - 1;
            src[j] = X + gr * ldx + chunk * 8;
        } else {
            const int64_t gr = n0 + row < N ? n0 + row : N - 1;
            src[j] = W + gr * ldw + chunk * 8;
        }
    }
    auto issue = [&](int64_t kt) __attribute__((always_inline)) {
        char* stage = sbase + (int)(kt % DSTAGES) * DSTAGE_BYTES;
#pragma unroll
        for (int j = 0; j < 12; ++j) {
            const int q = wave * 12 + j;
            __builtin_amdgcn_global_load_lds((gvoid_t*)(src[j] + kt * LBK), (lvoid_t*)(stage + q * 1024),
                                             16, 0, 0);
        }
    };

    f32x16 acc[4][2];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    const int fr = lane & 31;
    const int fc = lane >> 5;  // chunk half within a 16-wide K sub-step
    const int64_t nk = K / LBK;
    issue(0);
    if (nk > 1) issue(1);
    for (int64_t kt = 0; kt < nk; ++kt) {
        // tile kt's 12 loads of this wave are done when at most the 12 of tile kt+1 remain
        // (wait and barrier in one asm statement: a fenced barrier would make the compiler wait
        // for tile kt+1's loads too, as they also write LDS; the "memory" clobber keeps the LDS
        // reads of this iteration below it)
        if (kt + 1 < nk) asm volatile("s_waitcnt vmcnt(12)\n\ts_barrier" ::: "memory");
        else asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
        if (kt + 2 < nk) issue(kt + 2);  // stage (kt+2)%3 was last read in iteration kt-1
        const char* stage = sbase + (int)(kt % DSTAGES) * DSTAGE_BYTES;
        const char* aw = stage + (wm * 128 + fr) * 128;                 // A rows of this lane
        const char* bw = stage + 32 * 1024 + (wn * 64 + fr) * 128;      // B rows of this lane
        // fragments of K-chunk pair s (chunks 2s + fc): rows r = base + fr, with r & 7 == fr & 7
        // since every base is a multiple of 8
        auto load = [&](int s, bf16x8* af, bf16x8* bf) __attribute__((always_inline)) {
            const int off = ((2 * s + fc) ^ (fr & 7)) << 4;
#pragma unroll
            for (int i = 0; i < 4; ++i) af[i] = *reinterpret_cast<const bf16x8*>(aw + i * 32 * 128 + off);
#pragma unroll
            for (int j = 0; j < 2; ++j) bf[j] = *reinterpret_cast<const bf16x8*>(bw + j * 32 * 128 + off);
        };
        // register double buffer: the fragments of pair s+1 are read while pair s is multiplied
        bf16x8 fa[2][4], fb[2][2];
        load(0, fa[0], fb[0]);
#pragma unroll
        for (int s = 0; s < LBK / 16; ++s) {
            if (s + 1 < LBK / 16) load(s + 1, fa[(s + 1) & 1], fb[(s + 1) & 1]);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[s & 1][i], fb[s & 1][j],
                                                                        acc[i][j], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    lds_barrier();  // the epilogue reuses stage memory

    float* st = reinterpret_cast<float*>(smem) + wave * (32 * 68);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                st[row * 68 + j * 32 + (lane & 31)] = acc[i][j][r];
            }
        __builtin_amdgcn_wave_barrier();
        store_tile_rows(o, bias, st, M, N, m0 + wm * 128 + i * 32, n0 + wn * 64, lane);
        __builtin_amdgcn_wave_barrier();
    }
}


// ----------------------------------------------------------------------------- narrow N
// Products with few output columns and a long K (the block's x_proj: N = dt_rank + 2 dstate, 160
// at config 3 and 64 at config 5, K = d_inner), which stream X from HBM once: a block owns 64 rows
// and every column, so the grid is M / 64 blocks and no K split is needed. Block tile 64 x NB
// (NB = 64 CB, N <= NB): 4 waves in 2 x 2, each 32 rows x 32 CB columns (CB
// v_mfma_f32_32x32x16_bf16 per 16-wide K step, K ascending as in the other kernels, so each
// output is the same sum). K tiles of 64 move straight into a 3- or 4-stage LDS ring with
// global_load_lds_dwordx4 (A rows 0..63, then W rows 0..NB-1, 128-byte rows with the 16-byte
// chunks XOR-swizzled by row); the loads of tile kt+2 (kt+3) are issued while tile kt is multiplied.
// W (at most NB x K) is read by every block and stays in L2. Requires K % 64 == 0 and 16-byte
// aligned rows; rows past M or N are clamped (their outputs are discarded).
constexpr int NBM = 64;

template <int CB>
constexpr int narrow_stage_bytes() { return (NBM + 64 * CB) * 128; }
// Ring depth: 4 stages (loads 3 K tiles ahead) where a CU holds one block either way (CB = 3:
// 128 KB against 96 KB), else 3, which keeps 2 or 3 blocks per CU (measured on MI355X: config 3
// x_proj, CB = 3, 52.7 -> 49.7 us with 4 stages, 54 us with 5 (160 KiB); config 5 x_proj,
// CB = 1, 50.8 -> 54.3 us with 4).
template <int CB>
constexpr int narrow_stages() { return CB >= 3 ? 4 : 3; }

template <int CB>
__global__ __launch_bounds__(256) void gemm_bf16_nt_narrow_kernel(int64_t M, int64_t N, int64_t K,
                                                                  const uint16_t* __restrict__ X,
                                                                  int64_t ldx,
                                                                  const uint16_t* __restrict__ W,
                                                                  int64_t ldw,
                                                                  const float* __restrict__ bias,
                                                                  GemmOut o) {
    extern __shared__ __attribute__((aligned(16))) uint16_t smem[];
    char* sbase = reinterpret_cast<char*>(smem);
    constexpr int SB = narrow_stage_bytes<CB>();
    constexpr int NST3 = narrow_stages<CB>();
    constexpr int QW = (NBM + 64 * CB) / 8 / 4;  // 1-KiB load regions per wave per tile
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    const int64_t m0 = (int64_t)blockIdx.x * NBM;

    // region q = QW * wave + j of a stage: rows 8q .. 8q + 7 (0..63 = A, then W); lane L fills
    // row 8q + L / 8, slot L % 8 with K-chunk (L % 8) ^ (row & 7)
    const uint16_t* src[QW];
#pragma unroll
    for (int j = 0; j < QW; ++j) {
        const int q = wave * QW + j;
        const int row = q * 8 + (lane >> 3);
        const int chunk = (lane & 7) ^ (row & 7);
        if (row < NBM) {
            const int64_t gr = m0 + row < M ? m0 + row : M - 1;
            src[j] = X + gr * ldx + chunk * 8;
        } else {
            const int64_t gr = row - NBM < N ? row - NBM : N - 1;
            src[j] = W + gr * ldw + chunk * 8;
        }
    }
    auto issue = [&](int64_t kt) __attribute__((always_inline)) {
        char* stage = sbase + (int)(kt % NST3) * SB;
#pragma unroll
        for (int j = 0; j < QW; ++j)
            __builtin_amdgcn_global_load_lds((gvoid_t*)(src[j] + kt * 64),
                                             (lvoid_t*)(stage + (wave * QW + j) * 1024), 16, 0, 0);
    };

    f32x16 acc[CB];
#pragma unroll
    for (int j = 0; j < CB; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[j][r] = 0.0f;

    const int fr = lane & 31;
    const int fc = lane >> 5;
    const int64_t nk = K / 64;
#pragma unroll
    for (int t = 0; t < NST3 - 1; ++t)
        if (t < nk) issue(t);
    static_assert(NST3 == 3 || NST3 == 4, "ring depth");
    for (int64_t kt = 0; kt < nk; ++kt) {
        // this wave's loads of tile kt are done when at most the QW of each later tile already
        // issued (up to NST3 - 2 of them) remain; wait and barrier in one statement so the
        // compiler adds no wait for the later tiles' loads
        if (NST3 == 4 && kt + 2 < nk)
            asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(2 * QW) : "memory");
        else if (kt + 1 < nk) asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(QW) : "memory");
        else asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
        // stage (kt + NST3 - 1) % NST3 was last read in iteration kt - 1
        if (kt + NST3 - 1 < nk) issue(kt + NST3 - 1);
        const char* stage = sbase + (int)(kt % NST3) * SB;
        const char* aw = stage + (wm * 32 + fr) * 128;
        const char* bw = stage + (NBM + wn * 32 * CB + fr) * 128;
        auto load = [&](int s, bf16x8& af, bf16x8* bf) __attribute__((always_inline)) {
            const int off = ((2 * s + fc) ^ (fr & 7)) << 4;
            af = *reinterpret_cast<const bf16x8*>(aw + off);
#pragma unroll
            for (int j = 0; j < CB; ++j) bf[j] = *reinterpret_cast<const bf16x8*>(bw + j * 32 * 128 + off);
        };
        bf16x8 fa[2], fb[2][CB];
        load(0, fa[0], fb[0]);
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            if (s + 1 < 4) load(s + 1, fa[(s + 1) & 1], fb[(s + 1) & 1]);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int j = 0; j < CB; ++j)
                acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[s & 1], fb[s & 1][j], acc[j], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    lds_barrier();  // the epilogue reuses stage memory

    // 32 x 64 slabs staged per wave (two column blocks at a time); the wave's columns end at
    // n_end, past which a slab's second half (odd CB) holds no result
    float* st = reinterpret_cast<float*>(smem) + wave * (32 * 68);
    const int64_t c0 = (int64_t)wn * 32 * CB;
    const int64_t n_end = c0 + 32 * CB < N ? c0 + 32 * CB : N;
#pragma unroll
    for (int g = 0; g < (CB + 1) / 2; ++g) {
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) {
            if (2 * g + jj >= CB) continue;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                st[row * 68 + jj * 32 + (lane & 31)] = acc[2 * g + jj][r];
            }
        }
        __builtin_amdgcn_wave_barrier();
        store_tile_rows(o, bias, st, M, n_end, m0 + wm * 32, c0 + 64 * g, lane);
        __builtin_amdgcn_wave_barrier();
    }
}

// ----------------------------------------------------------------------------- 256 x 256
// Direct-to-LDS kernel with a 256 x 256 block tile: 4 waves in 2 x 2, each a 128 x 128 tile
// (4 x 4 v_mfma_f32_32x32x16_bf16 per 16-wide K step, 256 fp32 accumulators per lane, kept in
// AGPRs). Per K step a wave reads 8 fragments of 16 bytes per lane from LDS for 16 MFMAs, half
// the LDS bytes per MFMA of the 256 x 128 kernel (4 x 2 tiles per wave), whose LDS reads plus the
// loads landing in LDS kept it near the CU's LDS bandwidth. K tiles of KB (32 or 64) in an
// NST-stage LDS ring (A rows 0..255 then B rows 0..255, rows of KB K-values, 16-byte chunks
// XOR-swizzled by row so that the 8 lanes of each 128-byte LDS access hit distinct banks); the
// loads of tile kt+NST-1 are issued while tile kt is multiplied, behind one barrier per tile.
// Requires K % KB == 0 and 16-byte aligned rows; rows past M or N are clamped (their outputs are
// discarded).
constexpr int XBM = 256, XBN = 256;
constexpr int kGemmBufRsrcWord3 = 0x00020000;  // gfx9 raw buffer: 32-bit data format, no swizzle

// The loads of a K tile into the ring, QPW instructions per wave, go out over a window of LW
// sub-steps: the last sub-step of the K tile NST before it (right after the barrier that frees its
// stage) and the first LW - 1 sub-steps of the next K tile. Issued as one burst, a block's 64 load
// instructions of a 64-wide K tile arrive at the load path in a quarter of the tile's MFMA time,
// twice what it accepts, and the waves stall on issue while their MFMAs drain. Without any loads
// in the loop (a timing copy multiplying stale stage data) config 3 in_proj takes 410 us against
// 485-506. With the buffer loads below, one box, three rounds: one sub-step 474-478 us, a
// 2-sub-step window 456-459 (out_proj 259-268 against 275-282), 3 sub-steps 461-463, 4 (whose
// last loads have one sub-step before the barrier that waits for them) 484-490; the same bits.
// Slot w of the window issues loads lw_base .. + lw_cnt. (The persistent kernel keeps the
// one-sub-step form: a window measured slower there.)
template <int QPW, int LW>
__device__ constexpr int lw_cnt(int w) { return QPW / LW + (w < QPW % LW ? 1 : 0); }
template <int QPW, int LW>
__device__ constexpr int lw_base(int w) { return w * (QPW / LW) + (w < QPW % LW ? w : QPW % LW); }

template <int KB>
__device__ inline int xswz(int row) {  // XOR applied to the 16-byte chunk index of a row
    return KB == 64 ? (row & 7) : ((row >> 1) & 3);
}

// Epilogue of one wave's 128 x 128 sub-tile when it lies inside one output with aligned rows and
// neither bias nor SiLU applies: 8 slabs of 32 x 64, each staged through the wave's LDS slab and
// written with store_slab_fast. `yb` points at the sub-tile's first output element.
// ACC: the existing outputs of each slab are loaded one slab ahead, so their latency overlaps the
// previous slab's staging and stores instead of stalling every slab.
template <bool BF16, bool ACC>
__device__ __forceinline__ void d256_epilogue_fast(f32x16 (&acc)[4][4], float* st, char* yb, int64_t ldb,
                                                   int lane) {
    constexpr int NP = SlabGeom<BF16>::NP;
    auto slab_ptr = [&](int sl) { return yb + (sl >> 1) * 32 * ldb + (sl & 1) * 64 * (BF16 ? 2 : 4); };
    slab_u32v4 old[2][NP];
    if constexpr (ACC) load_slab_old<BF16>(slab_ptr(0), ldb, lane, old[0]);
#pragma unroll
    for (int sl = 0; sl < 8; ++sl) {  // slab (i, jj) = (sl / 2, sl % 2)
        const int i = sl >> 1, jj = sl & 1;
        if constexpr (ACC) {
            if (sl + 1 < 8) load_slab_old<BF16>(slab_ptr(sl + 1), ldb, lane, old[(sl + 1) & 1]);
        }
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                st[row * 68 + j * 32 + (lane & 31)] = acc[i][2 * jj + j][r];
            }
        __builtin_amdgcn_wave_barrier();
        store_slab_fast<BF16, ACC>(slab_ptr(sl), ldb, st, lane, old[sl & 1]);
        __builtin_amdgcn_wave_barrier();
    }
}

template <int KB, int NST, bool BUF>
__global__ __launch_bounds__(256) void gemm_bf16_nt_d256_kernel(int64_t M, int64_t N, int64_t K,
                                                                const uint16_t* __restrict__ X,
                                                                int64_t ldx,
                                                                const uint16_t* __restrict__ W,
                                                                int64_t ldw,
                                                                const float* __restrict__ bias,
                                                                GemmOut o, int64_t zstride) {
    // split K (gridDim.z > 1): slice z multiplies columns [z K, z K + K) of X and W into its own
    // single-output partial, zstride elements after slice z-1's
    if (gridDim.z > 1) {
        X += blockIdx.z * K;
        W += blockIdx.z * K;
        o.y[0] = (char*)o.y[0] + blockIdx.z * zstride * (o.out_bf16 ? 2 : 4);
    }
    constexpr int RB = KB * 2;              // bytes per tile row
    constexpr int CPR = KB / 8;             // 16-byte chunks per row
    constexpr int RPK = 1024 / RB;          // rows per KiB (one load instruction)
    constexpr int STB = (XBM + XBN) * RB;   // stage bytes
    constexpr int QPW = STB / 1024 / 4;     // load instructions per wave per tile
    constexpr int QA = XBM * RB / 1024;     // KiB regions of A
    extern __shared__ __attribute__((aligned(16))) uint16_t smem[];
    char* sbase = reinterpret_cast<char*>(smem);

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    const int nbx = gridDim.x, nby = gridDim.y;
    const int nb = nbx * nby;
    int tm, tn;
    tile_of(nbx, nb, blockIdx.y * nbx + blockIdx.x, tm, tn);
    const int64_t m0 = (int64_t)tm * XBM, n0 = (int64_t)tn * XBN;

    // this lane's QPW global sources per tile: wave w issues KiB regions q = QPW*w .. of the
    // stage (q < QA: A rows RPK*q.., else B rows RPK*(q-QA)..); lane L fills row RPK*q' + L/CPR,
    // slot L%CPR with the K-chunk (L%CPR) ^ xswz(row). BUF: buffer loads to LDS through one
    // resource per wave (a wave's regions are all A or all W), the lane's row as a 32-bit byte
    // offset and the K tile's offset in a scalar: no per-load address arithmetic, 32-bit
    // addresses (config 3 in_proj and out_proj 2-3% faster than 64-bit pointer loads, same bits).
    // (Arrays of 16 >= QPW: a bound that depends on the template here drops the host launch stub.)
    const uint16_t* src[16];
    uint32_t voff[16];
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        wave * QPW < QA ? (void*)X : (void*)W, (short)0, (int)0x7fffffff, kGemmBufRsrcWord3);
#pragma unroll
    for (int j = 0; j < QPW; ++j) {
        const int q = wave * QPW + j;
        const bool isA = q < QA;
        const int row = (isA ? q : q - QA) * RPK + lane / CPR;
        const int chunk = (lane % CPR) ^ xswz<KB>(row);
        if (isA) {
            const int64_t gr = m0 + row < M ? m0 + row : M - 1;
            src[j] = X + gr * ldx + chunk * 8;
            voff[j] = (uint32_t)((gr * ldx + chunk * 8) * 2);
        } else {
            const int64_t gr = n0 + row < N ? n0 + row : N - 1;
            src[j] = W + gr * ldw + chunk * 8;
            voff[j] = (uint32_t)((gr * ldw + chunk * 8) * 2);
        }
    }
#define HX_D256_LOAD(j, kt, stage)                                                                       \
    do {                                                                                                 \
        if constexpr (BUF)                                                                               \
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lvoid_t*)((stage) + (wave * QPW + (j)) * 1024), \
                                                     16, voff[j], (int)((kt) * KB * 2), 0, 0);           \
        else                                                                                             \
            __builtin_amdgcn_global_load_lds((gvoid_t*)(src[j] + (kt) * KB),                             \
                                             (lvoid_t*)((stage) + (wave * QPW + (j)) * 1024), 16, 0, 0); \
    } while (0)
    auto issue = [&](int64_t kt) __attribute__((always_inline)) {
        char* stage = sbase + (int)(kt % NST) * STB;
#pragma unroll
        for (int j = 0; j < QPW; ++j) HX_D256_LOAD(j, kt, stage);
    };

    f32x16 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    const int fr = lane & 31;
    const int fc = lane >> 5;  // chunk half within a 16-wide K sub-step
    const int64_t nk = K / KB;
    // Sub-steps 0..SUB-1 (16 K each) of tile kt; the fragments of sub-step s+1 are read while the
    // 16 MFMAs of sub-step s issue (one read after each of the first 8 MFMAs), so the MFMA pipe
    // does not wait on LDS. The tile barrier sits before the last sub-step: by then each wave has
    // read all of tile kt (the last sub-step's fragments were waited for), so after it the freed
    // stage takes tile kt+NST and the last sub-step overlaps the reads of tile kt+1's first
    // fragments from the next stage. Tile kt+1's loads, issued NST-1 tiles earlier, are complete
    // at that barrier (the wait leaves the loads of the tiles after it in flight).
    constexpr int SUB = KB / 16;
    auto frag = [&](int stg, int s, int q) __attribute__((always_inline)) {
        const char* stage = sbase + stg * STB;
        const int off = ((2 * s + fc) ^ xswz<KB>(fr)) << 4;  // row bases are multiples of 32
        return q < 4 ? *reinterpret_cast<const bf16x8*>(stage + (wm * 128 + fr) * RB + q * 32 * RB + off)
                     : *reinterpret_cast<const bf16x8*>(stage + XBM * RB + (wn * 128 + fr) * RB +
                                                        (q - 4) * 32 * RB + off);
    };
    // wait until at most `after` tiles' loads are in flight (this wave's), then the barrier
    auto wait_barrier = [&](int64_t after) __attribute__((always_inline)) {
        if (after >= 3) asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(3 * QPW) : "memory");
        else if (after == 2) asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(2 * QPW) : "memory");
        else if (after == 1) asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(QPW) : "memory");
        else asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    };
    static_assert(NST >= 2 && NST <= 4 && (SUB == 2 || SUB == 4) && 3 * QPW <= 63 && QPW % 8 == 0,
                  "ring depth / K tile");
    // window of LW sub-steps with two stages: its slots precede the barrier that waits for them
    // (vmcnt(0): no other K tile's loads are in flight there); deeper rings keep one sub-step
    constexpr int LW = (NST == 2 && SUB == 4) ? 2 : 1;
    bf16x8 fg[2][8];  // [buffer][A rows 0..3, B rows 0..3] (32-row fragments)
#pragma unroll
    for (int t = 0; t < NST; ++t)
        if (t < nk) issue(t);
    wait_barrier((nk < NST ? nk : NST) - 1);
#pragma unroll
    for (int q = 0; q < 8; ++q) fg[0][q] = frag(0, 0, q);
    int stg = 0;
    for (int64_t kt = 0; kt < nk; ++kt) {
        const int nstg = stg + 1 == NST ? 0 : stg + 1;
#pragma unroll
        for (int s = 0; s < SUB; ++s) {
            const int cur = s & 1, nxt = cur ^ 1;
            // loads between the MFMAs (one burst before them measured config 3 in_proj 493 vs 468
            // us), over a window of LW sub-steps: slot w = 0 is this tile's last sub-step (starts
            // tile kt + NST), slot w >= 1 sub-step w - 1 (continues tile kt + NST - 1)
            const int w = s == SUB - 1 ? 0 : (s + 1 < LW ? s + 1 : -1);
            const int64_t tl = w == 0 ? kt + NST : kt + NST - 1;
            const bool ilv = w == 0 ? tl < nk : (w > 0 && kt >= 1 && tl < nk);  // uniform
            const int jb = w < 0 ? 0 : lw_base<QPW, LW>(w), jc = w < 0 ? 0 : lw_cnt<QPW, LW>(w);
            if (s == SUB - 1 && kt + 1 < nk) wait_barrier(nk - 2 - kt < NST - 2 ? nk - 2 - kt : NST - 2);
#pragma unroll
            for (int q = 0; q < 8; ++q) {
#pragma unroll
                for (int jj = 0; jj < 2; ++jj) {
                    const int i = q >> 1, j = (q & 1) * 2 + jj;
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fg[cur][i], fg[cur][4 + j],
                                                                        acc[i][j], 0, 0, 0);
                }
                // (the last tile's last sub-step reads unused fragments of the next stage, which
                // no load targets any more, so that no sub-step branches)
                fg[nxt][q] = s < SUB - 1 ? frag(stg, s + 1, q) : frag(nstg, 0, q);
                if (ilv) {
                    char* stage = sbase + (int)(tl % NST) * STB;
#pragma unroll
                    for (int u = q * jc / 8; u < (q + 1) * jc / 8; ++u) HX_D256_LOAD(jb + u, tl, stage);
                }
            }
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one LDS read
                __builtin_amdgcn_sched_group_barrier(0x020, (lw_cnt<QPW, LW>(0) + 7) / 8, 0);  // loads
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        stg = nstg;
    }
    lds_barrier();  // the epilogue reuses stage memory

    float* st = reinterpret_cast<float*>(smem) + wave * (32 * 68);
    {
        // this wave's 128 x 128 sub-tile inside one output, rows aligned, no bias or SiLU: the
        // unguarded slab stores
        const int64_t r0 = m0 + wm * 128, c0 = n0 + wn * 128;
        int seg = 0;
        int64_t cc = c0;
        if (c0 >= o.split2) { seg = 2; cc = c0 - o.split2; }
        else if (c0 >= o.split1) { seg = 1; cc = c0 - o.split1; }
        const int64_t seg_end = seg == 0 ? o.split1 : seg == 1 ? o.split2 : N;
        const int64_t es = o.out_bf16 ? 2 : 4;
        char* yb = (char*)o.yp(seg) + (r0 * o.ldp(seg) + cc) * es;
        const int64_t ldb = o.ldp(seg) * es;
        if (!bias && !(o.act & 1) && r0 + 128 <= M && c0 + 128 <= seg_end &&
            (((uintptr_t)yb | (uint64_t)ldb) & 15) == 0) {
            const int kind = (o.out_bf16 ? 0 : 2) + ((o.act & 2) ? 1 : 0);
            if (kind == 0) d256_epilogue_fast<true, false>(acc, st, yb, ldb, lane);
            else if (kind == 1) d256_epilogue_fast<true, true>(acc, st, yb, ldb, lane);
            else if (kind == 2) d256_epilogue_fast<false, false>(acc, st, yb, ldb, lane);
            else d256_epilogue_fast<false, true>(acc, st, yb, ldb, lane);
            return;
        }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) {
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int row = 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                    st[row * 68 + j * 32 + (lane & 31)] = acc[i][2 * jj + j][r];
                }
            __builtin_amdgcn_wave_barrier();
            store_tile_rows(o, bias, st, M, N, m0 + wm * 128 + i * 32, n0 + wn * 128 + jj * 64, lane);
            __builtin_amdgcn_wave_barrier();
        }
    }
}



#undef HX_D256_LOAD

// Epilogue of the persistent kernel for one wave's 128 x 128 sub-tile inside one output with
// aligned rows and no bias/SiLU: 16 slabs of 16 x 64 through the wave's own 16-row LDS slab
// (the K-tile ring keeps filling meanwhile); ACC loads each slab's existing outputs a slab ahead.
template <bool BF16, bool ACC>
__device__ __forceinline__ void d256p_epilogue_fast(f32x16 (&acc)[4][4], float* st, char* yb, int64_t ldb,
                                                    int lane) {
    constexpr int NP = SlabGeom<BF16, 16>::NP;
    // slab sl: 32-row block i = sl / 4, 16-row half h = (sl / 2) % 2, 64-column half jj = sl % 2
    auto slab_ptr = [&](int sl) {
        return yb + ((sl >> 2) * 32 + ((sl >> 1) & 1) * 16) * ldb + (sl & 1) * 64 * (BF16 ? 2 : 4);
    };
    slab_u32v4 old[2][NP];
    if constexpr (ACC) load_slab_old<BF16, 16>(slab_ptr(0), ldb, lane, old[0]);
#pragma unroll
    for (int sl = 0; sl < 16; ++sl) {
        const int i = sl >> 2, h = (sl >> 1) & 1, jj = sl & 1;
        if constexpr (ACC) {
            if (sl + 1 < 16) load_slab_old<BF16, 16>(slab_ptr(sl + 1), ldb, lane, old[(sl + 1) & 1]);
        }
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int rr = 0; rr < 8; ++rr) {
                const int r = 8 * h + rr;  // the accumulator rows of this half
                const int row = 8 * ((r >> 2) - 2 * h) + 4 * (lane >> 5) + (r & 3);
                st[row * 68 + j * 32 + (lane & 31)] = acc[i][2 * jj + j][r];
            }
        __builtin_amdgcn_wave_barrier();
        store_slab_fast<BF16, ACC, 16>(slab_ptr(sl), ldb, st, lane, old[sl & 1]);
        __builtin_amdgcn_wave_barrier();
    }
}

// Persistent form of the 256 x 256 kernel: one block per CU walks its tiles (block b takes tile
// ids b, b + gridDim.x, ... in tile_of's order, so each tile stays on the XCD the one-tile-per-
// block launch gives it), and the K-tile ring runs on across tiles: the loads of the next tile's
// first K tiles are issued during this tile's last ones, so they are in flight while this tile's
// epilogue stores, and the next tile starts without a pipeline fill. The epilogue stages 16-row
// slabs in an LDS region of its own (NST stages + 4 x 16 x 68 floats). Each tile's arithmetic is
// the 256 x 256 kernel's: the same MFMA products, K ascending.
template <int KB, int NST, bool BUF>
__global__ __launch_bounds__(256) void gemm_bf16_nt_d256p_kernel(int64_t M, int64_t N, int64_t K,
                                                                 const uint16_t* __restrict__ X,
                                                                 int64_t ldx,
                                                                 const uint16_t* __restrict__ W,
                                                                 int64_t ldw,
                                                                 const float* __restrict__ bias,
                                                                 GemmOut o) {
    constexpr int RB = KB * 2;              // bytes per tile row
    constexpr int CPR = KB / 8;             // 16-byte chunks per row
    constexpr int RPK = 1024 / RB;          // rows per KiB (one load instruction)
    constexpr int STB = (XBM + XBN) * RB;   // stage bytes
    constexpr int QPW = STB / 1024 / 4;     // load instructions per wave per tile
    constexpr int QA = XBM * RB / 1024;     // KiB regions of A
    extern __shared__ __attribute__((aligned(16))) uint16_t smem[];
    char* sbase = reinterpret_cast<char*>(smem);

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    const int nbx = (int)((N + XBN - 1) / XBN);
    const int nb = nbx * (int)((M + XBM - 1) / XBM);
    const int nblk = gridDim.x;  // <= nb
    const int ntl = (nb - (int)blockIdx.x + nblk - 1) / nblk;  // this block's tiles
    const int64_t nk = K / KB;
    const int64_t total = (int64_t)ntl * nk;  // K tiles over all of this block's tiles
    float* st = reinterpret_cast<float*>(sbase + NST * STB) + wave * (16 * 68);

    // the global sources of the tile whose K tiles are being issued (set when the issue moves to
    // the next tile): wave w issues KiB regions q = QPW*w .. of a stage, as in the 256 x 256 kernel
    // (BUF: buffer loads to LDS with 32-bit row offsets, as there)
    const uint16_t* src[16];
    uint32_t voff[16];
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        wave * QPW < QA ? (void*)X : (void*)W, (short)0, (int)0x7fffffff, kGemmBufRsrcWord3);
    int src_tile = -1;
    auto set_src = [&](int i) __attribute__((always_inline)) {
        int tm, tn;
        tile_of(nbx, nb, (int)blockIdx.x + i * nblk, tm, tn);
        const int64_t m0 = (int64_t)tm * XBM, n0 = (int64_t)tn * XBN;
#pragma unroll
        for (int j = 0; j < QPW; ++j) {
            const int q = wave * QPW + j;
            const bool isA = q < QA;
            const int row = (isA ? q : q - QA) * RPK + lane / CPR;
            const int chunk = (lane % CPR) ^ xswz<KB>(row);
            if (isA) {
                const int64_t gr = m0 + row < M ? m0 + row : M - 1;
                src[j] = X + gr * ldx + chunk * 8;
                voff[j] = (uint32_t)((gr * ldx + chunk * 8) * 2);
            } else {
                const int64_t gr = n0 + row < N ? n0 + row : N - 1;
                src[j] = W + gr * ldw + chunk * 8;
                voff[j] = (uint32_t)((gr * ldw + chunk * 8) * 2);
            }
        }
        src_tile = i;
    };
    // global K tile p of this block: its offset along K in the tile and its stage (the sources
    // move on to p's tile first)
    auto prep = [&](int64_t p, int64_t& koff, char*& stage) __attribute__((always_inline)) {
        const int i = (int)(p / nk);
        koff = (p - (int64_t)i * nk) * KB;
        if (i != src_tile) set_src(i);
        stage = sbase + (int)(p % NST) * STB;
    };
    auto load = [&](int j, int64_t koff, char* stage) __attribute__((always_inline)) {
        if constexpr (BUF)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lvoid_t*)(stage + (wave * QPW + j) * 1024), 16, voff[j],
                                                     (int)(koff * 2), 0, 0);
        else
            __builtin_amdgcn_global_load_lds((gvoid_t*)(src[j] + koff), (lvoid_t*)(stage + (wave * QPW + j) * 1024),
                                             16, 0, 0);
    };
    auto issue = [&](int64_t p) __attribute__((always_inline)) {
        int64_t koff;
        char* stage;
        prep(p, koff, stage);
#pragma unroll
        for (int j = 0; j < QPW; ++j) load(j, koff, stage);
    };

    f32x16 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    const int fr = lane & 31;
    const int fc = lane >> 5;
    constexpr int SUB = KB / 16;
    auto frag = [&](int stg, int s, int q) __attribute__((always_inline)) {
        const char* stage = sbase + stg * STB;
        const int off = ((2 * s + fc) ^ xswz<KB>(fr)) << 4;
        return q < 4 ? *reinterpret_cast<const bf16x8*>(stage + (wm * 128 + fr) * RB + q * 32 * RB + off)
                     : *reinterpret_cast<const bf16x8*>(stage + XBM * RB + (wn * 128 + fr) * RB +
                                                        (q - 4) * 32 * RB + off);
    };
    // wait until at most `after` K tiles' loads are in flight (this wave's), then the barrier;
    // the epilogue's stores count in vmcnt too, so the first wait of a tile also covers them
    auto wait_barrier = [&](int64_t after) __attribute__((always_inline)) {
        if (after >= 3) asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(3 * QPW) : "memory");
        else if (after == 2) asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(2 * QPW) : "memory");
        else if (after == 1) asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(QPW) : "memory");
        else asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    };
    static_assert(NST >= 2 && NST <= 4 && (SUB == 2 || SUB == 4) && 3 * QPW <= 63 && QPW % 8 == 0,
                  "ring depth / K tile");
    // the first barrier after an epilogue: the loads it waits for were issued before the
    // epilogue's stores, so `sprev` (the stores this wave's epilogue issued: 32 for bf16, 64 for
    // fp32, capped at 63; 0 when unknown) may stay in flight (vector memory completes in order)
    static_assert(NST == 2, "the epilogue wait assumes no other K tile's loads in flight");
    auto wait_barrier_after_stores = [&](int sprev) __attribute__((always_inline)) {
        if (sprev >= 63) asm volatile("s_waitcnt vmcnt(63) lgkmcnt(0)\n\ts_barrier" ::: "memory");
        else if (sprev >= 32) asm volatile("s_waitcnt vmcnt(32) lgkmcnt(0)\n\ts_barrier" ::: "memory");
        else asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    };
    int sprev = 0;
    bf16x8 fg[2][8];
#pragma unroll
    for (int t = 0; t < NST; ++t)
        if (t < total) issue(t);
    wait_barrier((total < NST ? total : NST) - 1);
#pragma unroll
    for (int q = 0; q < 8; ++q) fg[0][q] = frag(0, 0, q);
    int stg = 0;
    int64_t p = 0;
    for (int i = 0; i < ntl; ++i) {
        int tm, tn;
        tile_of(nbx, nb, (int)blockIdx.x + i * nblk, tm, tn);
        for (int64_t kt = 0; kt < nk; ++kt, ++p) {
            const int nstg = stg + 1 == NST ? 0 : stg + 1;
#pragma unroll
            for (int s = 0; s < SUB; ++s) {
                const int cur = s & 1, nxt = cur ^ 1;
                // the last sub-step issues K tile p + NST's loads between its MFMAs, QPW / 8
                // after each pair (uniform condition); spread over a window of sub-steps as in the
                // one-tile kernel they measured slower here (config 5 in_proj 308 -> 320 us)
                const bool ld = s == SUB - 1 && p + NST < total;
                int64_t koff = 0;
                char* lstage = sbase;
                if (s == SUB - 1) {
                    if (p + 1 < total) {
                        if (kt == 0 && i > 0) wait_barrier_after_stores(sprev);
                        else wait_barrier(total - 2 - p < NST - 2 ? total - 2 - p : NST - 2);
                    }
                    if (ld) prep(p + NST, koff, lstage);
                }
#pragma unroll
                for (int q = 0; q < 8; ++q) {
#pragma unroll
                    for (int jj = 0; jj < 2; ++jj) {
                        const int a = q >> 1, b = (q & 1) * 2 + jj;
                        acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fg[cur][a], fg[cur][4 + b],
                                                                            acc[a][b], 0, 0, 0);
                    }
                    // the last sub-step reads the next K tile's first fragments (the next tile's,
                    // after a tile's last K tile; past the block's last K tile, unused stage data)
                    fg[nxt][q] = s < SUB - 1 ? frag(stg, s + 1, q) : frag(nstg, 0, q);
                    if (ld) {
#pragma unroll
                        for (int u = 0; u < QPW / 8; ++u) load(q * (QPW / 8) + u, koff, lstage);
                    }
                }
#pragma unroll
                for (int q = 0; q < 8; ++q) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
                    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one LDS read
                    __builtin_amdgcn_sched_group_barrier(0x020, QPW / 8, 0);  // loads
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
                }
                __builtin_amdgcn_sched_barrier(0);
            }
            stg = nstg;
        }

        // epilogue of tile i; then its accumulators restart at zero
        const int64_t m0 = (int64_t)tm * XBM, n0 = (int64_t)tn * XBN;
        const int64_t r0 = m0 + wm * 128, c0 = n0 + wn * 128;
        int seg = 0;
        int64_t cc = c0;
        if (c0 >= o.split2) { seg = 2; cc = c0 - o.split2; }
        else if (c0 >= o.split1) { seg = 1; cc = c0 - o.split1; }
        const int64_t seg_end = seg == 0 ? o.split1 : seg == 1 ? o.split2 : N;
        const int64_t es = o.out_bf16 ? 2 : 4;
        char* yb = (char*)o.yp(seg) + (r0 * o.ldp(seg) + cc) * es;
        const int64_t ldb = o.ldp(seg) * es;
        if (!bias && !(o.act & 1) && r0 + 128 <= M && c0 + 128 <= seg_end &&
            (((uintptr_t)yb | (uint64_t)ldb) & 15) == 0) {
            const int kind = (o.out_bf16 ? 0 : 2) + ((o.act & 2) ? 1 : 0);
            if (kind == 0) d256p_epilogue_fast<true, false>(acc, st, yb, ldb, lane);
            else if (kind == 1) d256p_epilogue_fast<true, true>(acc, st, yb, ldb, lane);
            else if (kind == 2) d256p_epilogue_fast<false, false>(acc, st, yb, ldb, lane);
            else d256p_epilogue_fast<false, true>(acc, st, yb, ldb, lane);
            sprev = o.out_bf16 ? 16 * SlabGeom<true, 16>::NP : 16 * SlabGeom<false, 16>::NP;
        } else {
            sprev = 0;
#pragma unroll
            for (int a = 0; a < 4; ++a) {
#pragma unroll
                for (int h = 0; h < 2; ++h) {
#pragma unroll
                    for (int jj = 0; jj < 2; ++jj) {
#pragma unroll
                        for (int j = 0; j < 2; ++j)
#pragma unroll
                            for (int rr = 0; rr < 8; ++rr) {
                                const int r = 8 * h + rr;
                                const int row = 8 * ((r >> 2) - 2 * h) + 4 * (lane >> 5) + (r & 3);
                                st[row * 68 + j * 32 + (lane & 31)] = acc[a][2 * jj + j][r];
                            }
                        __builtin_amdgcn_wave_barrier();
                        store_tile_rows(o, bias, st, M, N, r0 + a * 32 + h * 16, c0 + jj * 64, lane, 16);
                        __builtin_amdgcn_wave_barrier();
                    }
                }
            }
        }
#pragma unroll
        for (int a = 0; a < 4; ++a)
#pragma unroll
            for (int b = 0; b < 4; ++b)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[a][b][r] = 0.0f;
    }
}

// Sum of the S split-K partials P[z][M][N] (fp32, row stride N) in slice order, then bias, SiLU,
// accumulate and the column split of o, one element per thread (consecutive threads take
// consecutive columns).
__global__ __launch_bounds__(256) void splitk_reduce_kernel(int64_t M, int64_t N, int S,
                                                            const float* __restrict__ P,
                                                            const float* __restrict__ bias, GemmOut o) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= M * N) return;
    const int64_t row = i / N, col = i % N;
    float v = P[i];
    for (int z = 1; z < S; ++z) v += P[(int64_t)z * M * N + i];
    if (bias) v += bias[col];
    if (o.act & 1) v = silu(v);
    int seg = 0;
    int64_t cc = col;
    if (col >= o.split2) { seg = 2; cc = col - o.split2; }
    else if (col >= o.split1) { seg = 1; cc = col - o.split1; }
    const int64_t off = row * o.ldp(seg) + cc;
    if (o.out_bf16) {
        uint16_t* yp = (uint16_t*)o.yp(seg) + off;
        if (o.act & 2) v += Storage<uint16_t>::load(yp);
        Storage<uint16_t>::store(yp, v);
    } else {
        float* yp = (float*)o.yp(seg) + off;
        if (o.act & 2) v += *yp;
        *yp = v;
    }
}

}  // namespace
}  // namespace hx

namespace {
// The 256 x 256 kernels' buffer-load form needs every byte offset into X and W below 2^31.
bool d256_buf(int64_t M, int64_t N, int64_t ldx, int64_t ldw) {
    return M * ldx * 2 < (1LL << 31) && N * ldw * 2 < (1LL << 31);
}

template <int KB, int NST>
bool d256_ok() {
    const size_t bytes = (size_t)NST * (hx::XBM + hx::XBN) * KB * 2;
    return hx::grant_dynamic_lds((const void*)hx::gemm_bf16_nt_d256_kernel<KB, NST, true>, bytes, 0) &&
           hx::grant_dynamic_lds((const void*)hx::gemm_bf16_nt_d256_kernel<KB, NST, false>, bytes, 0);
}

template <int KB, int NST>
int launch_d256(int64_t M, int64_t N, int64_t K, const void* X, int64_t ldx, const void* W, int64_t ldw,
                const float* bias, const hx::GemmOut& o, void* stream) {
    using namespace hx;
    const size_t bytes = (size_t)NST * (XBM + XBN) * KB * 2;
    dim3 lg((unsigned)((N + XBN - 1) / XBN), (unsigned)((M + XBM - 1) / XBM));
    if (d256_buf(M, N, ldx, ldw))
        hipLaunchKernelGGL((gemm_bf16_nt_d256_kernel<KB, NST, true>), lg, dim3(256), bytes, as_stream(stream), M, N,
                           K, (const uint16_t*)X, ldx, (const uint16_t*)W, ldw, bias, o, (int64_t)0);
    else
        hipLaunchKernelGGL((gemm_bf16_nt_d256_kernel<KB, NST, false>), lg, dim3(256), bytes, as_stream(stream), M,
                           N, K, (const uint16_t*)X, ldx, (const uint16_t*)W, ldw, bias, o, (int64_t)0);
    HX_LAUNCH_CHECK();
    return HX_OK;
}

template <int KB, int NST>
size_t d256p_bytes() {
    return (size_t)NST * (hx::XBM + hx::XBN) * KB * 2 + 4 * 16 * 68 * sizeof(float);
}

template <int KB, int NST>
bool d256p_ok() {
    return hx::grant_dynamic_lds((const void*)hx::gemm_bf16_nt_d256p_kernel<KB, NST, true>, d256p_bytes<KB, NST>(), 0) &&
           hx::grant_dynamic_lds((const void*)hx::gemm_bf16_nt_d256p_kernel<KB, NST, false>, d256p_bytes<KB, NST>(), 0);
}

template <int KB, int NST>
int launch_d256p(int64_t M, int64_t N, int64_t K, const void* X, int64_t ldx, const void* W, int64_t ldw,
                 const float* bias, const hx::GemmOut& o, void* stream) {
    using namespace hx;
    const int64_t nb = ((N + XBN - 1) / XBN) * ((M + XBM - 1) / XBM);
    const int64_t cus = device_cus();
    const unsigned grid = (unsigned)(nb < cus ? nb : cus);  // one block per CU (the LDS allows one)
    const size_t bytes = d256p_bytes<KB, NST>();
    if (d256_buf(M, N, ldx, ldw))
        hipLaunchKernelGGL((gemm_bf16_nt_d256p_kernel<KB, NST, true>), dim3(grid), dim3(256), bytes, as_stream(stream),
                           M, N, K, (const uint16_t*)X, ldx, (const uint16_t*)W, ldw, bias, o);
    else
        hipLaunchKernelGGL((gemm_bf16_nt_d256p_kernel<KB, NST, false>), dim3(grid), dim3(256), bytes, as_stream(stream),
                           M, N, K, (const uint16_t*)X, ldx, (const uint16_t*)W, ldw, bias, o);
    HX_LAUNCH_CHECK();
    return HX_OK;
}

bool dlds_ok(size_t bytes) { return hx::grant_dynamic_lds((const void*)hx::gemm_bf16_nt_dlds_kernel, bytes, 0); }

template <int CB>
int launch_narrow_cb(int64_t M, int64_t N, int64_t K, const void* X, int64_t ldx, const void* W,
                     int64_t ldw, const float* bias, const hx::GemmOut& o, void* stream) {
    using namespace hx;
    const size_t bytes = (size_t)narrow_stages<CB>() * narrow_stage_bytes<CB>();
    HX_REQUIRE(grant_dynamic_lds((const void*)gemm_bf16_nt_narrow_kernel<CB>, bytes, 0), HX_ERR_UNSUPPORTED,
               "gemm_bf16: the device does not grant %zu bytes of LDS", bytes);
    HX_REQUIRE((M + NBM - 1) / NBM <= 0x7fffffff, HX_ERR_UNSUPPORTED, "gemm_bf16: M=%lld too large",
               (long long)M);
    hipLaunchKernelGGL((gemm_bf16_nt_narrow_kernel<CB>), dim3((unsigned)((M + NBM - 1) / NBM)), dim3(256),
                       bytes, as_stream(stream), M, N, K, (const uint16_t*)X, ldx, (const uint16_t*)W, ldw,
                       bias, o);
    HX_LAUNCH_CHECK();
    return HX_OK;
}

// The narrow kernel for 1 <= N <= 256 (block tile 64 x 64 ceil(N / 64)).
int launch_narrow(int64_t M, int64_t N, int64_t K, const void* X, int64_t ldx, const void* W,
                  int64_t ldw, const float* bias, const hx::GemmOut& o, void* stream) {
    switch ((N + 63) / 64) {
        case 1: return launch_narrow_cb<1>(M, N, K, X, ldx, W, ldw, bias, o, stream);
        case 2: return launch_narrow_cb<2>(M, N, K, X, ldx, W, ldw, bias, o, stream);
        case 3: return launch_narrow_cb<3>(M, N, K, X, ldx, W, ldw, bias, o, stream);
        default: return launch_narrow_cb<4>(M, N, K, X, ldx, W, ldw, bias, o, stream);
    }
}
}  // namespace

namespace hx {
bool gemm_narrow_auto(int64_t N, int64_t K) { return N >= 1 && N <= 192 && K >= 1024 && K % 64 == 0; }
}  // namespace hx

namespace hx {
namespace {
// The small-M kernel's tiling for an M x N x K product: 64-wide tiles where they still give the
// GPU 256 blocks (decode in_proj), else 32-wide; blocks of 8 waves where the grid has at most one
// block per CU, else 4; spw = the K-steps (16 wide) each wave covers.
struct SkinnyShape {
    bool wide, w8;
    int tn;
    int64_t spw;
};
SkinnyShape skinny_shape(int64_t M, int64_t N, int64_t K) {
    SkinnyShape sh;
    sh.wide = ((N + 63) / 64) * ((M + 31) / 32) >= 256;
    sh.tn = sh.wide ? 64 : 32;
    sh.w8 = ((N + sh.tn - 1) / sh.tn) * ((M + 31) / 32) <= device_cus();
    sh.spw = ((K + 15) / 16 + (sh.w8 ? 7 : 3)) / (sh.w8 ? 8 : 4);
    return sh;
}
}  // namespace

bool gemm_rmsnorm_small_ok(int64_t M, int64_t N, int64_t K, const float* X, int64_t ldx,
                           const float* nw, const void* W, int64_t ldw) {
    if (g_gemm_kernel != 0 || M <= 0 || N <= 0 || K < 8 || K % 8 != 0 || ldx < K || ldw < K)
        return false;
    if (ldx % 4 != 0 || ldw % 8 != 0 || !aligned(X, 16) || !aligned(nw, 16) || !aligned(W, 16))
        return false;
    // hx_gemm_bf16 takes the small-M kernel for these sizes (its other forms need K >= 1024 or
    // at least 128 tiles of 128 x 128)
    if (((M + BM - 1) / BM) * ((N + BN - 1) / BN) >= 128 || (M + 31) / 32 > 65535) return false;
    return skinny_shape(M, N, K).spw <= 4;  // one round of at most 4 pieces per lane
}

int gemm_rmsnorm_small(int64_t M, int64_t N, int64_t K, const float* X, int64_t ldx, const float* nw,
                       float eps, const void* W, int64_t ldw, int out_dtype, void* Y0, int64_t ld0,
                       int64_t split1, void* Y1, int64_t ld1, int64_t split2, void* Y2, int64_t ld2,
                       hipStream_t stream) {
    HX_REQUIRE(gemm_rmsnorm_small_ok(M, N, K, X, ldx, nw, W, ldw), HX_ERR_UNSUPPORTED,
               "gemm_rmsnorm_small: sizes or alignment outside the fused form");
    HX_REQUIRE(out_dtype == HX_F32 || out_dtype == HX_BF16, HX_ERR_DTYPE_MISMATCH,
               "gemm_rmsnorm_small: out_dtype %d", out_dtype);
    HX_REQUIRE(Y0 && ld0 >= 0, HX_ERR_INVALID_INPUT, "gemm_rmsnorm_small: Y0 is NULL");
    if (split1 <= 0 || split1 > N) split1 = N;
    if (split2 < split1 || split2 > N) split2 = N;
    HX_REQUIRE(split1 == N || Y1, HX_ERR_INVALID_INPUT, "gemm_rmsnorm_small: Y1 is NULL but split1 < N");
    HX_REQUIRE(split2 == N || Y2, HX_ERR_INVALID_INPUT, "gemm_rmsnorm_small: Y2 is NULL but split2 < N");
    const GemmOut o{{Y0, Y1, Y2}, {ld0, ld1, ld2}, split1, split2, out_dtype == HX_BF16, 0};
    const SkinnyShape sh = skinny_shape(M, N, K);
    auto launch = [&](auto kern, int nwv) {
        dim3 sg((unsigned)((N + sh.tn - 1) / sh.tn), (unsigned)((M + 31) / 32));
        hipLaunchKernelGGL(kern, sg, dim3(64 * nwv), 0, stream, M, N, K, X, ldx, (const uint16_t*)W,
                           ldw, (const float*)nullptr, o, nw, eps);
    };
    const bool two = sh.spw <= 2;
    if (sh.wide && sh.w8) {
        if (two) launch(gemm_bf16_nt_skinny_kernel<64, 8, 2, float>, 8);
        else launch(gemm_bf16_nt_skinny_kernel<64, 8, 4, float>, 8);
    } else if (sh.wide) {
        if (two) launch(gemm_bf16_nt_skinny_kernel<64, 4, 2, float>, 4);
        else launch(gemm_bf16_nt_skinny_kernel<64, 4, 4, float>, 4);
    } else if (sh.w8) {
        if (two) launch(gemm_bf16_nt_skinny_kernel<32, 8, 2, float>, 8);
        else launch(gemm_bf16_nt_skinny_kernel<32, 8, 4, float>, 8);
    } else {
        if (two) launch(gemm_bf16_nt_skinny_kernel<32, 4, 2, float>, 4);
        else launch(gemm_bf16_nt_skinny_kernel<32, 4, 4, float>, 4);
    }
    HX_LAUNCH_CHECK();
    return HX_OK;
}
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
    // narrow N, long K (x_proj): one pass over X with every column in the block, chosen by the
    // weight shape alone (measured on MI355X: config 3 x_proj N 160 K 4096, config 5 N 64 K 1024)
    // the tile kernels below load whole K tiles unguarded: K == 0 (Y = bias) takes the guarded
    // 128 x 128 kernel
    if (vec && K > 0 && K % 64 == 0 && N <= 256 &&
        (g_gemm_kernel == 7 || (g_gemm_kernel == 0 && gemm_narrow_auto(N, K))))
        return launch_narrow(M, N, K, X, ldx, W, ldw, bias, o, stream);
    // auto: the 256 x 256 kernel wherever it fills the GPU with tiles at least 256 columns wide
    // (measured on MI355X ahead of every other kernel here for the block's in_proj, out_proj,
    // dt_proj and the LM head: 1.5-2.3x the 128 x 128 kernel; behind it for the narrow x_proj);
    // the 32-wide K tile where K is not a multiple of 64 (config 5 dt_proj, K = 32)
    const bool d256_auto = g_gemm_kernel == 0 && N >= 256 && M >= 256 &&
                           ((M + XBM - 1) / XBM) * ((N + XBN - 1) / XBN) >= 256;
    // the persistent form where K is short (<= 1024) and every block gets at least two tiles:
    // there a tile's epilogue (its output drain, which every CU reaches at once in the one-tile
    // form) is a large share and overlaps the next tile's K loop (config 5 prefill 18.16 ->
    // 18.02 ms on one box; config 3's K = 2048 / 4096 projections measured 1% slower with it).
    // Both forms give the same bits.
    const bool d256p_auto = d256_auto && K <= 1024 &&
                            ((M + XBM - 1) / XBM) * ((N + XBN - 1) / XBN) >= 2 * (int64_t)device_cus();
    if (vec && K > 0 && K % 64 == 0 && (g_gemm_kernel == 8 || d256p_auto) && d256p_ok<64, 2>())
        return launch_d256p<64, 2>(M, N, K, X, ldx, W, ldw, bias, o, stream);
    if (vec && K > 0 && K % 64 == 0 && (g_gemm_kernel == 5 || d256_auto) && d256_ok<64, 2>())
        return launch_d256<64, 2>(M, N, K, X, ldx, W, ldw, bias, o, stream);
    if (vec && K > 0 && K % 32 == 0 && (g_gemm_kernel == 6 || (d256_auto && K % 64 != 0)) && d256_ok<32, 4>())
        return launch_d256<32, 4>(M, N, K, X, ldx, W, ldw, bias, o, stream);
    const size_t dlds = (size_t)DSTAGES * DSTAGE_BYTES;
    // auto: the direct-to-LDS kernel for long K (measured ahead of the 128 x 128 kernel from
    // K = 2048 on, and from K = 1024 for N <= 128 where its tiles fill half the GPU: config 5
    // x_proj 78 vs 87 us; behind it at K <= 512 where its one block per CU cannot hide the
    // epilogue). Its per-element arithmetic is the 256 x 256 kernel's (K ascending in 16-wide
    // MFMA steps), so a short batch that lands here matches a long one that takes that kernel.
    const int64_t tiles_dlds = ((M + LBM - 1) / LBM) * ((N + LBN - 1) / LBN);
    if (vec && K > 0 && K % LBK == 0 &&
        (g_gemm_kernel == 4 ||
         (g_gemm_kernel == 0 && (K >= 2048 || (K >= 1024 && N <= 128 && tiles_dlds >= 128)))) &&
        dlds_ok(dlds)) {
        dim3 lg((unsigned)((N + LBN - 1) / LBN), (unsigned)((M + LBM - 1) / LBM));
        hipLaunchKernelGGL(gemm_bf16_nt_dlds_kernel, lg, dim3(256), dlds, as_stream(stream), M, N, K,
                           (const uint16_t*)X, ldx, (const uint16_t*)W, ldw, bias, o);
        HX_LAUNCH_CHECK();
        return HX_OK;
    }
    const int64_t tiles128 = ((M + BM - 1) / BM) * ((N + BN - 1) / BN);
    if (vec && K % 8 == 0 && K >= 8 && g_gemm_kernel != 1 && g_gemm_kernel != 4 &&
        (g_gemm_kernel == 3 || tiles128 < 128) && (M + 31) / 32 <= 65535) {
        // 64-wide tiles where they still give the GPU 256 blocks (decode in_proj), else 32-wide;
        // SP covers a wave's whole share of K where it can (one round of loads). Where the grid
        // has at most one block per CU, blocks of 8 waves: each wave loads half the share, and two
        // waves per SIMD overlap their load rounds (config 5 decode at batch 256: 403 -> 394 us
        // per step, the same with only out_proj's 128 blocks so; the sums over the waves' K
        // slices then meet in 8 parts)
        const SkinnyShape sh = skinny_shape(M, N, K);
        const bool wide = sh.wide, w8 = sh.w8;
        const int tn = sh.tn;
        const int64_t spw = sh.spw;
        auto launch = [&](auto kern, int nw) {
            dim3 sg((unsigned)((N + tn - 1) / tn), (unsigned)((M + 31) / 32));
            hipLaunchKernelGGL(kern, sg, dim3(64 * nw), 0, as_stream(stream), M, N, K, (const uint16_t*)X,
                               ldx, (const uint16_t*)W, ldw, bias, o, (const float*)nullptr, 0.0f);
        };
        if (wide && w8) {
            if (spw <= 2) launch(gemm_bf16_nt_skinny_kernel<64, 8, 2>, 8);
            else if (spw <= 4) launch(gemm_bf16_nt_skinny_kernel<64, 8, 4>, 8);
            else if (spw <= 8) launch(gemm_bf16_nt_skinny_kernel<64, 8, 8>, 8);
            else launch(gemm_bf16_nt_skinny_kernel<64, 8, 16>, 8);
        } else if (wide) {
            if (spw <= 2) launch(gemm_bf16_nt_skinny_kernel<64, 4, 2>, 4);
            else if (spw <= 4) launch(gemm_bf16_nt_skinny_kernel<64, 4, 4>, 4);
            else if (spw <= 8) launch(gemm_bf16_nt_skinny_kernel<64, 4, 8>, 4);
            else launch(gemm_bf16_nt_skinny_kernel<64, 4, 16>, 4);
        } else if (w8) {
            if (spw <= 2) launch(gemm_bf16_nt_skinny_kernel<32, 8, 2>, 8);
            else if (spw <= 4) launch(gemm_bf16_nt_skinny_kernel<32, 8, 4>, 8);
            else if (spw <= 8) launch(gemm_bf16_nt_skinny_kernel<32, 8, 8>, 8);
            else launch(gemm_bf16_nt_skinny_kernel<32, 8, 16>, 8);
        } else {
            if (spw <= 2) launch(gemm_bf16_nt_skinny_kernel<32, 4, 2>, 4);
            else if (spw <= 4) launch(gemm_bf16_nt_skinny_kernel<32, 4, 4>, 4);
            else if (spw <= 8) launch(gemm_bf16_nt_skinny_kernel<32, 4, 8>, 4);
            else launch(gemm_bf16_nt_skinny_kernel<32, 4, 16>, 4);
        }
        HX_LAUNCH_CHECK();
        return HX_OK;
    }
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

// Split-K form of hx_gemm_bf16 for GEMMs with too few 256 x 256 tiles to fill the GPU (a narrow N
// with a long K: the block's x_proj). The K range is cut into `splits` slices of whole 64-wide K
// tiles, each slice's product goes to its own fp32 partial in the workspace (splits * M * N
// floats), and one pass sums the partials in slice order and applies hx_gemm_bf16's epilogue
// (same output arguments).
extern "C" int hx_gemm_bf16_splitk(int64_t M, int64_t N, int64_t K, const void* X, int64_t ldx,
                                   const void* W, int64_t ldw, const float* bias, int act, int out_dtype,
                                   void* Y0, int64_t ld0, int64_t split1, void* Y1, int64_t ld1,
                                   int64_t split2, void* Y2, int64_t ld2, int splits, void* workspace,
                                   size_t workspace_bytes, void* stream) {
    using namespace hx;
    HX_REQUIRE(M >= 0 && N >= 0 && K >= 0, HX_ERR_INVALID_DIMENSION, "gemm_bf16_splitk: negative size");
    HX_REQUIRE(act >= 0 && act <= 3, HX_ERR_INVALID_INPUT,
               "gemm_bf16_splitk: act=%d (bit 0 SiLU, bit 1 accumulate into Y)", act);
    HX_REQUIRE(out_dtype == HX_F32 || out_dtype == HX_BF16, HX_ERR_DTYPE_MISMATCH,
               "gemm_bf16_splitk: out_dtype %d", out_dtype);
    HX_REQUIRE(splits >= 1 && splits <= 16, HX_ERR_INVALID_INPUT, "gemm_bf16_splitk: splits %d (1..16)",
               splits);
    if (M == 0 || N == 0) return HX_OK;
    HX_REQUIRE(X && W && Y0, HX_ERR_INVALID_INPUT, "gemm_bf16_splitk: X, W and Y0 must be non-NULL");
    HX_REQUIRE(ldx >= K && ldw >= K && ld0 >= 0, HX_ERR_INVALID_DIMENSION,
               "gemm_bf16_splitk: leading dimensions smaller than K");
    HX_REQUIRE(K > 0 && K % ((int64_t)splits * 64) == 0, HX_ERR_UNSUPPORTED,
               "gemm_bf16_splitk: K %lld is not a positive multiple of 64 * splits", (long long)K);
    HX_REQUIRE(ldx % 8 == 0 && ldw % 8 == 0 && aligned(X, 16) && aligned(W, 16), HX_ERR_UNSUPPORTED,
               "gemm_bf16_splitk: rows of X and W must be 16-byte aligned");
    HX_REQUIRE(workspace && aligned(workspace, 16) &&
                   workspace_bytes >= (size_t)splits * (size_t)M * (size_t)N * sizeof(float),
               HX_ERR_INVALID_INPUT, "gemm_bf16_splitk: workspace %zu bytes < %zu required",
               workspace_bytes, (size_t)splits * (size_t)M * (size_t)N * sizeof(float));
    HX_REQUIRE((M + XBM - 1) / XBM <= 65535, HX_ERR_UNSUPPORTED, "gemm_bf16_splitk: M=%lld too large",
               (long long)M);
    HX_REQUIRE((d256_ok<64, 2>()), HX_ERR_UNSUPPORTED, "gemm_bf16_splitk: the device does not grant "
               "the 256 x 256 kernel's LDS");
    if (split1 <= 0 || split1 > N) split1 = N;
    if (split2 < split1 || split2 > N) split2 = N;
    HX_REQUIRE(split1 == N || Y1, HX_ERR_INVALID_INPUT, "gemm_bf16_splitk: Y1 is NULL but split1 < N");
    HX_REQUIRE(split2 == N || Y2, HX_ERR_INVALID_INPUT, "gemm_bf16_splitk: Y2 is NULL but split2 < N");
    float* partial = (float*)workspace;
    const GemmOut po{{partial, nullptr, nullptr}, {N, 0, 0}, N, N, 0, 0};
    const size_t bytes = (size_t)2 * (XBM + XBN) * 64 * 2;
    dim3 lg((unsigned)((N + XBN - 1) / XBN), (unsigned)((M + XBM - 1) / XBM), (unsigned)splits);
    if (d256_buf(M, N, ldx, ldw))
        hipLaunchKernelGGL((gemm_bf16_nt_d256_kernel<64, 2, true>), lg, dim3(256), bytes, as_stream(stream), M, N,
                           K / splits, (const uint16_t*)X, ldx, (const uint16_t*)W, ldw, (const float*)nullptr,
                           po, M * N);
    else
        hipLaunchKernelGGL((gemm_bf16_nt_d256_kernel<64, 2, false>), lg, dim3(256), bytes, as_stream(stream), M, N,
                           K / splits, (const uint16_t*)X, ldx, (const uint16_t*)W, ldw, (const float*)nullptr,
                           po, M * N);
    HX_LAUNCH_CHECK();
    const GemmOut o{{Y0, Y1, Y2}, {ld0, ld1, ld2}, split1, split2, out_dtype == HX_BF16, act};
    const int64_t n = M * N;
    hipLaunchKernelGGL(splitk_reduce_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                       as_stream(stream), M, N, splits, (const float*)partial, bias, o);
    HX_LAUNCH_CHECK();
    return HX_OK;
}

extern "C" int hx_set_gemm_kernel(int k) {
    using namespace hx;
    HX_REQUIRE(k >= 0 && k <= 8 && k != 2, HX_ERR_INVALID_INPUT,
               "hx_set_gemm_kernel: %d (0 auto, 1, 3, 4, 5, 6, 7, 8)", k);
    g_gemm_kernel = k;
    return HX_OK;
}

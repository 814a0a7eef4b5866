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
#include <type_traits>

#include <mutex>

#include "hx_common.h"
#include "hx_wave.h"

namespace hx {
namespace {

template <typename T>
__device__ inline float ld(const T* p) { return Storage<T>::load(p); }

// ----------------------------------------------------------------------------- fast path
// Vector of SPW consecutive storage elements read from LDS as fp32.
template <int SPW>
__device__ inline void lds_row(const float* p, float* v) {
    if constexpr (SPW == 4) {
        const float4 q = *reinterpret_cast<const float4*>(p);
        v[0] = q.x; v[1] = q.y; v[2] = q.z; v[3] = q.w;
    } else if constexpr (SPW == 2) {
        const float2 q = *reinterpret_cast<const float2*>(p);
        v[0] = q.x; v[1] = q.y;
    } else {
#pragma unroll
        for (int k = 0; k < SPW; ++k) v[k] = p[k];
    }
}

template <typename T, int W, int TCH, bool HAS_Z, bool SOFTPLUS>
__global__ __launch_bounds__(64 * W) void scan_fwd_kernel(
    int64_t L, int64_t Dm,
    const T* __restrict__ u, const T* __restrict__ delta, const float* __restrict__ A,
    const T* __restrict__ Bm, const T* __restrict__ Cm, const float* __restrict__ Dv,
    const T* __restrict__ z, const float* __restrict__ dt_bias, T* __restrict__ out,
    const float* __restrict__ init_state, float* __restrict__ last_state) {
    constexpr int NS = 16;
    constexpr int SPW = NS / W;        // states per wave
    constexpr int SPS = TCH / W;       // pre/post steps per wave per chunk
    constexpr int NT = 64 * W;         // threads
    constexpr int BC = TCH * NS;       // B (or C) elements per chunk
    constexpr int BCT = (2 * BC + NT - 1) / NT;  // B/C elements each thread stages per chunk
    static_assert(NS % W == 0 && TCH % W == 0, "bad tiling");

    __shared__ float2 s_du[TCH][64];             // (dt, dt*u) per step and channel
    __shared__ float s_part[2][W][TCH][64];      // per-wave partial readouts, double-buffered
    __shared__ float s_bc[2][2][TCH][NS];        // [buf][B|C][step][state], double-buffered

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int64_t b = blockIdx.y;
    const int64_t d = (int64_t)blockIdx.x * 64 + lane;
    const bool dvalid = d < Dm;
    const int64_t dc = dvalid ? d : Dm - 1;

    const int64_t row0 = b * L * Dm + dc;  // element (b, 0, dc)
    const T* __restrict__ up = u + row0;
    const T* __restrict__ dp = delta + row0;
    const T* __restrict__ zp = HAS_Z ? z + row0 : nullptr;
    T* __restrict__ op = out + row0;
    const T* __restrict__ Bb = Bm + b * L * NS;
    const T* __restrict__ Cb = Cm + b * L * NS;

    float A2[SPW], h[SPW];
#pragma unroll
    for (int k = 0; k < SPW; ++k) {
        A2[k] = A[dc * NS + w * SPW + k] * kLog2e;
        h[k] = init_state ? init_state[(b * Dm + dc) * NS + w * SPW + k] : 0.0f;
    }
    const float Dd = Dv ? Dv[dc] : 0.0f;
    const float bias = dt_bias ? dt_bias[dc] : 0.0f;

    // Register prefetch of one chunk: this wave's u/delta/z rows and this thread's share of B/C.
    float pu[SPS], pd[SPS], pz[SPS], pbc[BCT];
    auto fetch = [&](int64_t t0) {
#pragma unroll
        for (int i = 0; i < SPS; ++i) {
            const int64_t t = t0 + w + i * W;
            const int64_t tc = t < L ? t : L - 1;
            pu[i] = ld(up + tc * Dm);
            pd[i] = ld(dp + tc * Dm);
            pz[i] = HAS_Z ? ld(zp + tc * Dm) : 0.0f;
        }
#pragma unroll
        for (int j = 0; j < BCT; ++j) {
            const int e = tid + j * NT;  // [B|C][step][state]
            if (e < 2 * BC) {
                const int which = e / BC, r = e % BC;
                int64_t t = t0 + r / NS;
                t = t < L ? t : L - 1;
                const T* src = which ? Cb : Bb;
                pbc[j] = ld(src + t * NS + (r % NS));
            }
        }
    };
    auto stage_bc = [&](int buf) {
#pragma unroll
        for (int j = 0; j < BCT; ++j) {
            const int e = tid + j * NT;
            if (e < 2 * BC) (&s_bc[buf][0][0][0])[e] = pbc[j];
        }
    };

    fetch(0);
    stage_bc(0);
    int buf = 0;
    for (int64_t t0 = 0; t0 < L; t0 += TCH) {
        // ---- pre: this wave's share of the chunk's per-element work (prefetched inputs)
        float uu[SPS], zz[SPS];
#pragma unroll
        for (int i = 0; i < SPS; ++i) {
            const int s = w + i * W;
            const bool tv = t0 + s < L;
            uu[i] = pu[i];
            zz[i] = pz[i];
            float dl = pd[i] + bias;
            if (SOFTPLUS) dl = softplus(dl);
            dl = tv ? dl : 0.0f;  // steps past the end leave the state unchanged
            s_du[s][lane] = make_float2(dl, dl * uu[i]);
        }
        // ---- prefetch the next chunk while this one computes
        if (t0 + TCH < L) fetch(t0 + TCH);
        lds_barrier();

        // ---- main: every wave advances its states through all TCH steps
#pragma unroll
        for (int s = 0; s < TCH; ++s) {
            const float2 q = s_du[s][lane];
            float bv[SPW], cv[SPW];
            lds_row<SPW>(&s_bc[buf][0][s][w * SPW], bv);
            lds_row<SPW>(&s_bc[buf][1][s][w * SPW], cv);
            float acc = 0.0f;
#pragma unroll
            for (int k = 0; k < SPW; ++k) {
                const float ab = fast_exp2(q.x * A2[k]);
                h[k] = fmaf(ab, h[k], q.y * bv[k]);
                acc = fmaf(cv[k], h[k], acc);
            }
            s_part[buf][w][s][lane] = acc;
        }
        // B/C of the next chunk into the other buffer: every wave finished reading it (it was
        // last read in the previous chunk's main loop, before this chunk's barrier).
        if (t0 + TCH < L) stage_bc(buf ^ 1);
        lds_barrier();

        // ---- post: this wave's share of readout, D skip, SiLU gate, store
#pragma unroll
        for (int i = 0; i < SPS; ++i) {
            const int s = w + i * W;
            const int64_t t = t0 + s;
            float y = 0.0f;
#pragma unroll
            for (int ww = 0; ww < W; ++ww) y += s_part[buf][ww][s][lane];
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

// ----------------------------------------------------------------------------- wave-complete path
// One wave owns 16 channels x all 16 states: DPP row r (16 lanes) holds states [4r, 4r+4) of the
// wave's 16 channels, lane c of the row one channel. Nothing of the math crosses waves, so the
// only block-level exchange is the memory staging:
//   * a block = 4 waves = 64 channels reads u/delta/z and writes out as float4 tiles
//     [16 steps x 64 ch] through LDS (256-byte row segments), one barrier per chunk;
//   * per-element work (softplus, dt*u; D*u, SiLU(z)) runs once per element: lane (r, c) owns
//     steps r, r+4, r+8, r+12 of channel c; the other rows get dt and dt*u by an all-gather over
//     v_permlane16_swap / v_permlane32_swap (register transposes across rows, no LDS);
//   * B[t][4r..4r+3] and C[t][4r..4r+3] of step t0+j sit in lane j of row r (one float4 load
//     each per chunk) and reach the multiplies by DPP row_newbcast;
//   * the per-row partial readouts are reduce-scattered across rows with the same swaps
//     (12 swaps + 12 adds per 16 steps), leaving each lane the sums of its own 4 steps.

// Segments: for long sequences with few (batch, channel-tile) pairs the sequence is cut into
// nseg segments of seg_len steps, each its own block. END_ONLY blocks compute a segment's end
// state from a zero entry state and the decay over the segment (per state); a carry kernel
// chains the segments' entry states; full blocks then run each segment from its entry state
// (seg_init) and write the outputs.
// Number of time segments for the wave kernel: 0 = automatic; set by hx_set_scan_segments.
thread_local int g_scan_segments = 0;

struct WaveSeg {
    int64_t seg_len;
    int nseg;
    const float* seg_init;  // [nseg][B][D][16] entry states (full mode, nseg > 1)
    float* seg_hend;        // [nseg][B][D][16] end state from zero (END_ONLY)
    float* seg_decay;       // [nseg][B][D][16] decay over the segment (END_ONLY; 0 = dropped)
    // fused dt projection (scan_wave3_kernel with DTP, bf16 storage): delta = bf16(dt_lo . w_dt^T)
    // formed in the kernel, dt_lo [B][L][rank], w_dt [D][rank], rank a multiple of 32 up to 128
    const uint16_t* dtlo = nullptr;
    const uint16_t* wdt = nullptr;
    int rank = 0;
};

template <typename T, int PF, bool HAS_Z, bool SOFTPLUS, bool END_ONLY>
__global__ __launch_bounds__(256) void scan_wave_kernel(
    int64_t L, int64_t Dm, int ntiles, int64_t Bt,
    const T* __restrict__ u, const T* __restrict__ delta, const float* __restrict__ A,
    const T* __restrict__ Bm, const T* __restrict__ Cm, const float* __restrict__ Dv,
    const T* __restrict__ z, const float* __restrict__ dt_bias, T* __restrict__ out,
    const float* __restrict__ init_state, float* __restrict__ last_state, WaveSeg sg) {
    constexpr int NS = 16, TCH = 16;
    constexpr int TS = 80;  // tile row stride (floats): rows r and r+1 of a wave hit disjoint banks
    constexpr bool USE_Z = HAS_Z && !END_ONLY;
    __shared__ float s_in[2][3][TCH][TS];  // [buf][u|delta|z][step][channel]
    __shared__ float s_out[END_ONLY ? 1 : 2][TCH][TS];

    const int nblk = gridDim.x;
    int id = blockIdx.x;
    if ((nblk & 7) == 0) id = (id & 7) * (nblk >> 3) + (id >> 3);  // XCD-aware order
    const int tile = id % ntiles;
    const int64_t b = (id / ntiles) % Bt;
    const int seg = (int)(id / ntiles / Bt);
    const int64_t tbeg = (int64_t)seg * sg.seg_len;
    const int64_t tend = tbeg + sg.seg_len < L ? tbeg + sg.seg_len : L;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int w = tid >> 6;
    const int r = lane >> 4;   // row = state group
    const int c = lane & 15;   // channel within the wave
    const int64_t c0 = (int64_t)tile * 64;
    const int cb = w * 16 + c;  // channel within the block tile
    const int64_t d = c0 + cb;
    const bool dvalid = d < Dm;
    const int64_t dc = dvalid ? d : Dm - 1;

    // memory phase ownership: float4 e = tid of each [16 x 64] tile
    const int mrow = tid >> 4, mcl = (tid & 15) * 4;
    const int64_t mch = c0 + mcl;
    const bool mvalid = mch < Dm;  // Dm % 4 == 0
    const int64_t rowbase = b * L * Dm;

    float A2[4], h[4];
    const float* h0 = END_ONLY ? nullptr
                    : (sg.nseg > 1 ? sg.seg_init + (int64_t)seg * Bt * Dm * NS : init_state);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        A2[k] = A[dc * NS + 4 * r + k] * kLog2e;
        h[k] = h0 ? h0[(b * Dm + dc) * NS + 4 * r + k] : 0.0f;
    }
    const float Dd = Dv ? Dv[dc] : 0.0f;
    const float bias = dt_bias ? dt_bias[dc] : 0.0f;
    float sumdt = 0.0f;

    // ring of PF chunks: the thread's float4 of u/delta/z, and this lane's B/C float4s
    float4 ru[PF], rd[PF], rz[PF], rb[PF], rc[PF];
    const int64_t Lm1 = tend - 1;
    auto fetch = [&](int k, int64_t t0) __attribute__((always_inline)) {
        int64_t t = t0 + mrow;
        t = t < Lm1 ? t : Lm1;
        const int64_t off = rowbase + t * Dm + (mvalid ? mch : 0);
        ru[k] = Vec4<T>::load(u + off);
        rd[k] = Vec4<T>::load(delta + off);
        rz[k] = USE_Z ? Vec4<T>::load(z + off) : make_float4(0, 0, 0, 0);
        int64_t tb = t0 + c;  // lane c of row r: step t0+c, states 4r..4r+3
        tb = tb < Lm1 ? tb : Lm1;
        rb[k] = Vec4<T>::load(Bm + (b * L + tb) * NS + 4 * r);
        rc[k] = END_ONLY ? make_float4(0, 0, 0, 0) : Vec4<T>::load(Cm + (b * L + tb) * NS + 4 * r);
    };
    auto stage_in = [&](int k, int buf) __attribute__((always_inline)) {
        *reinterpret_cast<float4*>(&s_in[buf][0][mrow][mcl]) = ru[k];
        *reinterpret_cast<float4*>(&s_in[buf][1][mrow][mcl]) = rd[k];
        if (USE_Z) *reinterpret_cast<float4*>(&s_in[buf][2][mrow][mcl]) = rz[k];
    };
    auto store_out = [&](int64_t t0, int buf) __attribute__((always_inline)) {
        if constexpr (!END_ONLY) {
            const int64_t t = t0 + mrow;
            if (mvalid && t < tend)
                Vec4<T>::store(out + rowbase + t * Dm + mch,
                               *reinterpret_cast<const float4*>(&s_out[buf][mrow][mcl]));
        }
    };

    // math for one chunk: inputs from s_in[buf], outputs into s_out[buf]
    auto compute = [&](int64_t t0, int buf, const float4& B4, const float4& C4) __attribute__((always_inline)) {
        // pre: steps r + 4i of channel d
        float uu[4], zz[4], dl[4], du[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int s = r + 4 * i;
            uu[i] = s_in[buf][0][s][cb];
            float x = s_in[buf][1][s][cb] + bias;
            zz[i] = USE_Z ? s_in[buf][2][s][cb] : 0.0f;
            if (SOFTPLUS) x = softplus(x);
            x = (t0 + s < tend) ? x : 0.0f;  // steps past the end leave the state unchanged
            dl[i] = x;
            du[i] = x * uu[i];
            if (END_ONLY) sumdt += x;
        }
        float gdl[4][4], gdu[4][4];  // [row rr][i]: step rr + 4i
        rows_all_gather(dl, gdl);
        rows_all_gather(du, gdu);
        const float bk[4] = {B4.x, B4.y, B4.z, B4.w};
        const float ck[4] = {C4.x, C4.y, C4.z, C4.w};
        // main: 16 steps, 4 states; P index j = i + 4*rr holds step rr + 4*i
        float P[16];
        StepLoop<4>::run([&](auto gc) {  // groups of 4 steps: 16 decays issued ahead
            constexpr int g = decltype(gc)::value;
            float ab[4][4];
#pragma unroll
            for (int e = 0; e < 4; ++e)
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const int s = 4 * g + e;
                    ab[e][k] = fast_exp2(gdl[s & 3][s >> 2] * A2[k]);
                }
            StepLoop<4>::run([&](auto ec) {
                constexpr int s = 4 * g + decltype(ec)::value;
                const float dus = gdu[s & 3][s >> 2];
                float acc = 0.0f;
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    h[k] = fmaf(ab[s - 4 * g][k], h[k], dpp<kDppBcast<s>>(bk[k]) * dus);
                    if constexpr (!END_ONLY) acc = fmac_bcast<s>(acc, ck[k], h[k]);
                }
                P[(s >> 2) + 4 * (s & 3)] = acc;  // j = i + 4*rr for s = rr + 4*i
            });
        });
        if constexpr (!END_ONLY) {
            float Y[4];
            rows_reduce_scatter(P, Y);  // Y[i]: step r + 4i
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int s = r + 4 * i;
                float y = fmaf(Dd, uu[i], Y[i]);
                if (HAS_Z) y *= silu(zz[i]);
                s_out[buf][s][cb] = y;
            }
        }
    };

    // pipeline: iteration k stages chunk k+1's inputs, stores chunk k-1's outputs, computes
    // chunk k; one barrier per chunk.
#pragma unroll
    for (int k = 0; k < PF; ++k) fetch(k, tbeg + (int64_t)k * TCH);
    stage_in(0, 0);
    float4 B4 = rb[0], C4 = rc[0];
    fetch(0, tbeg + (int64_t)PF * TCH);
    lds_barrier();
    for (int64_t tb0 = tbeg; tb0 < tend; tb0 += PF * TCH) {
        StepLoop<PF>::run([&](auto kc) __attribute__((always_inline)) {
            constexpr int k = decltype(kc)::value;
            constexpr int kn = (k + 1) % PF;
            constexpr int buf = k & 1;  // PF is even
            const int64_t t0 = tb0 + k * TCH;
            if (t0 >= tend) return;  // uniform
            stage_in(kn, buf ^ 1);
            if (t0 > tbeg) store_out(t0 - TCH, END_ONLY ? 0 : buf ^ 1);
            const float4 Bn = rb[kn], Cn = rc[kn];
            fetch(kn, t0 + TCH + (int64_t)PF * TCH);
            compute(t0, buf, B4, C4);
            B4 = Bn;
            C4 = Cn;
            lds_barrier();
        });
    }
    if constexpr (!END_ONLY) {
        const int64_t nch = (tend - tbeg + TCH - 1) / TCH;
        store_out(tbeg + (nch - 1) * TCH, (int)((nch - 1) & 1));
        if (last_state && dvalid && seg == sg.nseg - 1) {
#pragma unroll
            for (int k = 0; k < 4; ++k) last_state[(b * Dm + d) * NS + 4 * r + k] = h[k];
        }
    } else {
        // segment end state (from zero) and total dt; rows hold different steps of a channel
        float t1 = sumdt, t2 = sumdt;
        swap16(t1, t2);
        float sa = t1 + t2;  // rows {0,1} pair and {2,3} pair
        float t3 = sa, t4 = sa;
        swap32(t3, t4);
        sumdt = t3 + t4;
        if (dvalid) {
            float* he = sg.seg_hend + (int64_t)seg * Bt * Dm * NS;
            float* de = sg.seg_decay + (int64_t)seg * Bt * Dm * NS;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                he[(b * Dm + d) * NS + 4 * r + k] = h[k];
                de[(b * Dm + d) * NS + 4 * r + k] = fast_exp2(A2[k] * sumdt);
            }
        }
    }
}

// Leaner wave-complete kernel with every wave on its own. Same decomposition as
// scan_wave_kernel, fewer VALU instructions per state update (which is what bounds it):
//   * addresses are 32-bit offsets from per-row base pointers, advanced by a constant per chunk
//     and clamped with one min;
//   * steps past the segment end are guarded only in a segment's last chunk;
//   * dt and dt*u reach the other rows through LDS (each lane writes its 4 steps as one float4,
//     reads its channel's 16 as four) instead of register swaps;
//   * the readout's first term is a DPP multiply, so no accumulator is zeroed;
//   * each wave stages its own 16 channels x 16 steps tiles (one float4 per lane per operand,
//     64-byte row pieces) in its own LDS region, so the waves of a block never wait for each
//     other (LDS operations of one wave execute in order, so program order alone orders each
//     wave's staging writes and reads).
// WPB waves per block (64 * WPB threads). Requires L * Dm < 2^31 (32-bit offsets within a
// batch row).
// DTPK > 0 (bf16 storage): the block's dt_proj fused in, rank = 32 DTPK. delta is not read; each
// chunk's dt tile [16 steps x 16 channels] = dt_lo [16 x rank] . w_dt[16 channels x rank]^T is
// formed on the matrix core (DTPK v_mfma_f32_16x16x32_bf16, fp32 sums), rounded to bf16 as the
// unfused path stores dt, and staged in the delta slot, so the rest of the kernel is unchanged.
// Lane (r, c) holds w_dt's row for channel c and dt_lo's row for step c of the chunk (8 K values
// per 16-lane group), and receives dt of steps 4r..4r+3 of channel c. The rank is a template
// argument so that every load is unconditional (the wait counts stay exact).
template <typename T, int PF, bool HAS_Z, bool SOFTPLUS, bool END_ONLY, int WPB, int DTPK = 0>
__global__ __launch_bounds__(64 * WPB) void scan_wave3_kernel(
    int64_t L, int64_t Dm, int ntiles, int64_t Bt,
    const T* __restrict__ u, const T* __restrict__ delta, const float* __restrict__ A,
    const T* __restrict__ Bm, const T* __restrict__ Cm, const float* __restrict__ Dv,
    const T* __restrict__ z, const float* __restrict__ dt_bias, T* __restrict__ out,
    const float* __restrict__ init_state, float* __restrict__ last_state, WaveSeg sg) {
    constexpr int NS = 16, TCH = 16;
    constexpr int GS = 20;  // gather row stride (floats): 16 values + pad
    constexpr bool USE_Z = HAS_Z && !END_ONLY;
    __shared__ __attribute__((aligned(16))) float s_in[WPB][2][3][TCH][16];  // [w][buf][u|dt|z][step][ch]
    __shared__ __attribute__((aligned(16))) float s_out[WPB][END_ONLY ? 1 : 2][TCH][16];
    __shared__ __attribute__((aligned(16))) float s_g[WPB][2][16][GS];  // [w][dt|dt*u][ch][4i + r]

    const int nblk = gridDim.x;
    int id = blockIdx.x;
    if ((nblk & 7) == 0) id = (id & 7) * (nblk >> 3) + (id >> 3);  // XCD-aware order
    const int tile = id % ntiles;
    const int64_t b = (id / ntiles) % Bt;
    const int seg = (int)(id / ntiles / Bt);
    const int64_t tbeg = (int64_t)seg * sg.seg_len;
    const int64_t tend = tbeg + sg.seg_len < L ? tbeg + sg.seg_len : L;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int w = tid >> 6;
    const int r = lane >> 4;
    const int c = lane & 15;
    const int64_t c0 = ((int64_t)tile * WPB + w) * 16;  // this wave's 16 channels
    const int cb = c;
    const int64_t d = c0 + cb;
    const bool dvalid = d < Dm;
    const int64_t dc = dvalid ? d : Dm - 1;
    const int mrow = lane >> 2, mcl = (lane & 3) * 4;  // staging: step row, 4 channels
    const int64_t mch = c0 + mcl;
    const bool mvalid = mch < Dm;

    // per-row bases; 32-bit offsets inside the row
    const T* ub = u + b * L * Dm;
    const T* db = delta + b * L * Dm;
    const T* zb = USE_Z ? z + b * L * Dm : nullptr;
    T* ob = END_ONLY ? nullptr : out + b * L * Dm;
    const T* Bb = Bm + b * L * NS;
    const T* Cb = Cm + b * L * NS;
    const uint32_t D32 = (uint32_t)Dm;
    const uint32_t mcol = (uint32_t)(mvalid ? mch : 0);
    const uint32_t x_last = (uint32_t)(tend - 1) * D32 + mcol;          // clamp of tile offsets
    const uint32_t bc_last = (uint32_t)(tend - 1) * NS + 4 * r;         // clamp of B/C offsets
    const uint32_t x_first = (uint32_t)(tbeg + mrow) * D32 + mcol;      // first chunk's offsets
    const uint32_t bc_first = (uint32_t)(tbeg + c) * NS + 4 * r;
    // next fetch: forwards from the segment's first chunk, or (END_ONLY) backwards from its last
    uint32_t x_next = (uint32_t)((END_ONLY ? tend - TCH : tbeg) + mrow) * D32 + mcol;
    uint32_t bc_next = (uint32_t)((END_ONLY ? tend - TCH : tbeg) + c) * NS + 4 * r;
    const uint32_t x_step = TCH * D32, bc_step = TCH * NS;

    float A2[4], h[4];
    const float* h0 = END_ONLY ? nullptr
                    : (sg.nseg > 1 ? sg.seg_init + (int64_t)seg * Bt * Dm * NS : init_state);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        A2[k] = A[dc * NS + 4 * r + k] * kLog2e;
        h[k] = h0 ? h0[(b * Dm + dc) * NS + 4 * r + k] : 0.0f;
    }
    const float Dd = Dv ? Dv[dc] : 0.0f;
    const float bias = dt_bias ? dt_bias[dc] : 0.0f;
    // END_ONLY: decay from the segment's end back to the step reached, per state, and the sum of
    // dt over those steps (the decay is exp(A * S))
    float Q[4] = {1.0f, 1.0f, 1.0f, 1.0f};
    float S = 0.0f;

    // fused dt projection: w_dt fragments of this lane's channel, and dt_lo row offsets (32-bit
    // inside the batch row) that advance with the chunks like the tile offsets
    constexpr bool DTP = DTPK > 0;
    constexpr int NKB = DTP ? DTPK : 1;
    static_assert(!(DTP && END_ONLY), "the fused dt projection has no end-state pass");
    typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
    typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4_t;
    bf16x8_t wdtf[NKB];
    bf16x8_t rdl[PF][NKB];
    const uint16_t* dlb = nullptr;
    uint32_t dl_next = 0, dl_first = 0, dl_last = 0, dl_step = 0;
    if constexpr (DTP) {
        const uint32_t R = 32 * DTPK;
        const int kq = 8 * (lane >> 4);
        const uint16_t* wr = sg.wdt + dc * R + kq;
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb) wdtf[kb] = *reinterpret_cast<const bf16x8_t*>(wr + 32 * kb);
        dlb = sg.dtlo + b * L * R;
        dl_first = (uint32_t)(tbeg + c) * R + kq;
        dl_last = (uint32_t)(tend - 1) * R + kq;
        dl_next = (uint32_t)((END_ONLY ? tend - TCH : tbeg) + c) * R + kq;
        dl_step = TCH * R;
    }

    float4 ru[PF], rd[PF], rz[PF], rb[PF], rc[PF];
    auto fetch = [&](int k) __attribute__((always_inline)) {
        const uint32_t xo = x_next < x_last ? x_next : x_last;
        ru[k] = Vec4<T>::load(ub + xo);
        if constexpr (DTP) {
            const uint32_t o = dl_next < dl_last ? dl_next : dl_last;
#pragma unroll
            for (int kb = 0; kb < NKB; ++kb) rdl[k][kb] = *reinterpret_cast<const bf16x8_t*>(dlb + o + 32 * kb);
        } else {
            rd[k] = Vec4<T>::load(db + xo);
        }
        rz[k] = USE_Z ? Vec4<T>::load(zb + xo) : make_float4(0, 0, 0, 0);
        const uint32_t bo = bc_next < bc_last ? bc_next : bc_last;
        rb[k] = Vec4<T>::load(Bb + bo);
        rc[k] = END_ONLY ? make_float4(0, 0, 0, 0) : Vec4<T>::load(Cb + bo);
        if constexpr (END_ONLY) {  // backwards; past the segment's start the first chunk repeats
            x_next = x_next >= x_first + x_step ? x_next - x_step : x_first;
            bc_next = bc_next >= bc_first + bc_step ? bc_next - bc_step : bc_first;
            if constexpr (DTP) dl_next = dl_next >= dl_first + dl_step ? dl_next - dl_step : dl_first;
        } else {
            x_next += x_step;
            bc_next += bc_step;
            if constexpr (DTP) dl_next += dl_step;
        }
    };
    // DTP: the dt tile of the chunk in slot k on the matrix core (lane (r, c) gets steps 4r..4r+3
    // of channel c), and its staging, rounded to bf16, in the delta slot of LDS buffer buf
    auto dt_tile = [&](int k) __attribute__((always_inline)) {
        f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
        if constexpr (DTP) {
#pragma unroll
            for (int kb = 0; kb < NKB; ++kb) acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(rdl[k][kb], wdtf[kb], acc, 0, 0, 0);
        }
        return acc;
    };
    auto stage_dt = [&](const f32x4_t& acc, int buf) __attribute__((always_inline)) {
        // round to bf16 (pack_bf16x2: round to nearest even) and widen back
#pragma unroll
        for (int j = 0; j < 4; j += 2) {
            const uint32_t pk = pack_bf16x2(acc[j], acc[j + 1]);
            s_in[w][buf][1][4 * r + j][c] = __uint_as_float(pk << 16);
            s_in[w][buf][1][4 * r + j + 1][c] = __uint_as_float(pk & 0xffff0000u);
        }
    };
    auto stage_in = [&](int k, int buf) __attribute__((always_inline)) {
        *reinterpret_cast<float4*>(&s_in[w][buf][0][mrow][mcl]) = ru[k];
        if constexpr (!DTP) *reinterpret_cast<float4*>(&s_in[w][buf][1][mrow][mcl]) = rd[k];
        if (USE_Z) *reinterpret_cast<float4*>(&s_in[w][buf][2][mrow][mcl]) = rz[k];
    };
    auto store_out = [&](int64_t t0, int buf) __attribute__((always_inline)) {
        if constexpr (!END_ONLY) {
            const int64_t t = t0 + mrow;
            if (mvalid && t < tend)
                Vec4<T>::store(ob + ((uint32_t)t * D32 + mcol),
                               *reinterpret_cast<const float4*>(&s_out[w][buf][mrow][mcl]));
        }
    };

    // math for one chunk: inputs from s_in[buf], outputs into s_out[buf]; FULL = all 16 steps
    // inside the segment
    auto compute = [&](int64_t t0, int buf, const float4& B4, const float4& C4, auto full_c)
        __attribute__((always_inline)) {
        constexpr bool FULL = decltype(full_c)::value;
        const int nvalid = FULL ? TCH : (int)(tend - t0);
        float uu[4], zz[4], dl[4], du[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int s = r + 4 * i;
            uu[i] = s_in[w][buf][0][s][cb];
            float x = s_in[w][buf][1][s][cb] + bias;
            zz[i] = USE_Z ? s_in[w][buf][2][s][cb] : 0.0f;
            if (SOFTPLUS) x = softplus(x);
            if (!FULL) x = s < nvalid ? x : 0.0f;  // steps past the end leave the state unchanged
            dl[i] = x;
            du[i] = x * uu[i];
        }
        // row all-gather through LDS: lane (r, c) holds steps r + 4i, stored step-major
        // (s_g[.][cb][s], s = 4i + r) so the float4 at [4g] is exactly the steps of group g and
        // each group's read can be in flight while the previous group computes
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            s_g[w][0][cb][4 * i + r] = dl[i];
            s_g[w][1][cb][4 * i + r] = du[i];
        }
        __builtin_amdgcn_wave_barrier();
        float gdl[4][4], gdu[4][4];  // [row rr][i]: step rr + 4i
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float4 a = *reinterpret_cast<const float4*>(&s_g[w][0][cb][4 * i]);
            const float4 q = *reinterpret_cast<const float4*>(&s_g[w][1][cb][4 * i]);
            gdl[0][i] = a.x; gdl[1][i] = a.y; gdl[2][i] = a.z; gdl[3][i] = a.w;
            gdu[0][i] = q.x; gdu[1][i] = q.y; gdu[2][i] = q.z; gdu[3][i] = q.w;
        }
        const float bk[4] = {B4.x, B4.y, B4.z, B4.w};
        const float ck[4] = {C4.x, C4.y, C4.z, C4.w};
        float P[16];
        if constexpr (END_ONLY) {
            // steps 15..0: h += exp(A * S) * B*dt*u, then S += dt; h is the end state from a zero
            // state at the step reached, S the sum of dt from there to the end. The decay to the
            // end is formed from S (one exponential per state-step) rather than as a running
            // product of the per-step decays (an exponential and a multiply).
            StepLoop<16>::run([&](auto ec) {
                constexpr int s = 15 - decltype(ec)::value;
                const float dus = gdu[s & 3][s >> 2];
#pragma unroll
                for (int k = 0; k < 4; ++k)
                    h[k] = fmaf(fast_exp2(A2[k] * S), dpp<kDppBcast<s>>(bk[k]) * dus, h[k]);
                S += gdl[s & 3][s >> 2];
            });
#pragma unroll
            for (int k = 0; k < 4; ++k) Q[k] = fast_exp2(A2[k] * S);
        } else {
        StepLoop<4>::run([&](auto gc) {
            constexpr int g = decltype(gc)::value;
            float ab[4][4];
#pragma unroll
            for (int e = 0; e < 4; ++e)
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const int s = 4 * g + e;
                    ab[e][k] = fast_exp2(gdl[s & 3][s >> 2] * A2[k]);
                }
            StepLoop<4>::run([&](auto ec) {
                constexpr int s = 4 * g + decltype(ec)::value;
                const float dus = gdu[s & 3][s >> 2];
#pragma unroll
                for (int k = 0; k < 4; ++k) h[k] = fmaf(ab[s - 4 * g][k], h[k], dpp<kDppBcast<s>>(bk[k]) * dus);
                if constexpr (!END_ONLY) {
                    float acc = dpp<kDppBcast<s>>(ck[0]) * h[0];
                    acc = fmac_bcast<s>(acc, ck[1], h[1]);
                    acc = fmac_bcast<s>(acc, ck[2], h[2]);
                    acc = fmac_bcast<s>(acc, ck[3], h[3]);
                    P[(s >> 2) + 4 * (s & 3)] = acc;  // j = i + 4*rr for s = rr + 4*i
                }
            });
        });
        }
        if constexpr (!END_ONLY) {
            float Y[4];
            rows_reduce_scatter(P, Y);  // Y[i]: step r + 4i
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int s = r + 4 * i;
                float y = fmaf(Dd, uu[i], Y[i]);
                if (HAS_Z) y *= silu(zz[i]);
                s_out[w][buf][s][cb] = y;
            }
        }
    };

#pragma unroll
    for (int k = 0; k < PF; ++k) fetch(k);
    stage_in(0, 0);
    if constexpr (DTP) stage_dt(dt_tile(0), 0);
    float4 B4 = rb[0], C4 = rc[0];
    fetch(0);
    // END_ONLY: the segment's chunks from the last back to the first (all whole: segment lengths
    // are multiples of 16 and the last, possibly partial, segment has no end-state pass). It
    // stops after the first chunk at which every state of the wave's channels has decayed below
    // 2^-32 (kDecayDrop) on its way to the segment's end: what is left out is that decay times
    // the state at that step (and times the entry state, whose decay over the whole segment is
    // smaller still), 2^-32 of values the recurrence holds to 2^-24 (a NaN or growing decay never
    // stops it). The segment then publishes a decay of 0, so its entry state is not carried.
    bool dropped = false;
    if constexpr (END_ONLY) {
        bool stop = false;  // uniform
        for (int64_t q0 = 0; !stop; q0 += PF) {
            StepLoop<PF>::run([&](auto kc) __attribute__((always_inline)) {
                constexpr int k = decltype(kc)::value;
                constexpr int kn = (k + 1) % PF;
                constexpr int buf = k & 1;  // PF is even
                if (stop) return;
                const int64_t t0 = tend - (q0 + k + 1) * TCH;
                if (t0 < tbeg) {
                    stop = true;
                    return;
                }
                stage_in(kn, buf ^ 1);
                const float4 Bn = rb[kn];
                fetch(kn);
                compute(t0, buf, B4, C4, std::true_type{});
                B4 = Bn;
                __builtin_amdgcn_wave_barrier();
                const float qm = fmaxf(fmaxf(Q[0], Q[1]), fmaxf(Q[2], Q[3]));
                if (__ballot(dvalid && !(qm < kDecayDrop)) == 0) {
                    stop = true;
                    dropped = t0 > tbeg;
                }
            });
        }
    }
    for (int64_t tb0 = tbeg; !END_ONLY && tb0 < tend; tb0 += PF * TCH) {
        StepLoop<PF>::run([&](auto kc) __attribute__((always_inline)) {
            constexpr int k = decltype(kc)::value;
            constexpr int kn = (k + 1) % PF;
            constexpr int buf = k & 1;  // PF is even
            const int64_t t0 = tb0 + k * TCH;
            if (t0 >= tend) return;  // uniform
            // DTP: the next chunk's dt tile starts on the matrix core here and is staged after
            // this chunk's math, which hides its latency (its slot is refetched just below)
            [[maybe_unused]] const f32x4_t dnext = dt_tile(kn);
            stage_in(kn, buf ^ 1);
            if (t0 > tbeg) store_out(t0 - TCH, END_ONLY ? 0 : buf ^ 1);
            const float4 Bn = rb[kn], Cn = rc[kn];
            fetch(kn);
            if (t0 + TCH <= tend)
                compute(t0, buf, B4, C4, std::true_type{});
            else
                compute(t0, buf, B4, C4, std::false_type{});
            if constexpr (DTP) stage_dt(dnext, buf ^ 1);
            B4 = Bn;
            C4 = Cn;
            __builtin_amdgcn_wave_barrier();
        });
    }
    if constexpr (!END_ONLY) {
        const int64_t nch = (tend - tbeg + TCH - 1) / TCH;
        store_out(tbeg + (nch - 1) * TCH, (int)((nch - 1) & 1));
        if (last_state && dvalid && seg == sg.nseg - 1) {
#pragma unroll
            for (int k = 0; k < 4; ++k) last_state[(b * Dm + d) * NS + 4 * r + k] = h[k];
        }
    } else {
        if (dvalid) {
            float* he = sg.seg_hend + (int64_t)seg * Bt * Dm * NS;
            float* de = sg.seg_decay + (int64_t)seg * Bt * Dm * NS;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                he[(b * Dm + d) * NS + 4 * r + k] = h[k];
                de[(b * Dm + d) * NS + 4 * r + k] = dropped ? 0.0f : Q[k];
            }
        }
    }
}


// Entry state of every segment: h_in[0] = init (or 0); h_in[k] = decay[k-1] * h_in[k-1] +
// hend[k-1], per (b, d, n). Writes seg_init[k] for k = 0..nseg-1 (reads hend/decay of the first
// nseg-1 segments only).
__global__ __launch_bounds__(256) void scan_seg_carry_kernel(
    int64_t Bt, int64_t Dm, int nseg, const float* __restrict__ init_state,
    const float* __restrict__ hend, const float* __restrict__ decay, float* __restrict__ seg_init) {
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t per = Bt * Dm * 16;
    if (gid >= per) return;
    float hc = init_state ? init_state[gid] : 0.0f;
    seg_init[gid] = hc;
    for (int k = 0; k + 1 < nseg; ++k) {  // the last segment's end state is not produced
        hc = fmaf(decay[(int64_t)k * per + gid], hc, hend[(int64_t)k * per + gid]);
        seg_init[(int64_t)(k + 1) * per + gid] = hc;
    }
}

// global_load_lds of VB bytes per lane: lane i's VB bytes at g land at l + i * VB. Non-temporal
// (each element is read once; config 2 bf16 152.9 -> 151.6 us).
template <int VB> __device__ inline void load_lds(const void* g, void* l);
template <> __device__ inline void load_lds<16>(const void* g, void* l) {
    __builtin_amdgcn_global_load_lds((gvoid_t*)g, (lvoid_t*)l, 16, 0, 2);
}
template <> __device__ inline void load_lds<4>(const void* g, void* l) {
    __builtin_amdgcn_global_load_lds((gvoid_t*)g, (lvoid_t*)l, 4, 0, 2);
}

// LDS reads written as inline asm that complete inside the statement (s_waitcnt lgkmcnt(0)).
// The element wave of scan_ws_kernel reads LDS while its global_load_lds loads are still in
// flight; for compiler-visible LDS reads the compiler inserts a wait for all of those loads
// (vmcnt(0)), which would drain the load ring every chunk. These reads are ordered by the
// wave's own explicit vmcnt waits instead. Addresses are LDS byte offsets.
typedef float hx_f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t hx_u32x2 __attribute__((ext_vector_type(2)));
__device__ inline uint32_t lds_off(const void* p) { return (uint32_t)(uintptr_t)p; }
__device__ inline float4 to_f4(hx_f32x4 v) { return make_float4(v[0], v[1], v[2], v[3]); }
__device__ inline float4 bf16x4_to_f4(hx_u32x2 v) {
    return make_float4(__uint_as_float(v[0] << 16), __uint_as_float(v[0] & 0xffff0000u),
                       __uint_as_float(v[1] << 16), __uint_as_float(v[1] & 0xffff0000u));
}
// r[j][o] = 4 storage elements at a[j] + o * OPB, o < NOP (2 or 3), j < 3; fp32 (16-byte reads)
// or bf16 (8-byte reads) storage
template <typename T, int NOP, int OPB> struct RingRead;
template <int OPB> struct RingRead<float, 3, OPB> {
    __device__ static inline void run(const uint32_t (&a)[3], float4 (&r)[3][3]) {
        hx_f32x4 v[3][3];
        asm volatile(
            "ds_read_b128 %0, %9\n\tds_read_b128 %1, %9 offset:%12\n\tds_read_b128 %2, %9 offset:%13\n\t"
            "ds_read_b128 %3, %10\n\tds_read_b128 %4, %10 offset:%12\n\tds_read_b128 %5, %10 offset:%13\n\t"
            "ds_read_b128 %6, %11\n\tds_read_b128 %7, %11 offset:%12\n\tds_read_b128 %8, %11 offset:%13\n\t"
            "s_waitcnt lgkmcnt(0)"
            : "=&v"(v[0][0]), "=&v"(v[0][1]), "=&v"(v[0][2]), "=&v"(v[1][0]), "=&v"(v[1][1]), "=&v"(v[1][2]),
              "=&v"(v[2][0]), "=&v"(v[2][1]), "=&v"(v[2][2])
            : "v"(a[0]), "v"(a[1]), "v"(a[2]), "n"(OPB), "n"(2 * OPB)
            : "memory");
#pragma unroll
        for (int j = 0; j < 3; ++j)
#pragma unroll
            for (int o = 0; o < 3; ++o) r[j][o] = to_f4(v[j][o]);
    }
};
template <int OPB> struct RingRead<float, 2, OPB> {
    __device__ static inline void run(const uint32_t (&a)[3], float4 (&r)[3][3]) {
        hx_f32x4 v[3][2];
        asm volatile(
            "ds_read_b128 %0, %6\n\tds_read_b128 %1, %6 offset:%9\n\t"
            "ds_read_b128 %2, %7\n\tds_read_b128 %3, %7 offset:%9\n\t"
            "ds_read_b128 %4, %8\n\tds_read_b128 %5, %8 offset:%9\n\t"
            "s_waitcnt lgkmcnt(0)"
            : "=&v"(v[0][0]), "=&v"(v[0][1]), "=&v"(v[1][0]), "=&v"(v[1][1]), "=&v"(v[2][0]), "=&v"(v[2][1])
            : "v"(a[0]), "v"(a[1]), "v"(a[2]), "n"(OPB)
            : "memory");
#pragma unroll
        for (int j = 0; j < 3; ++j)
#pragma unroll
            for (int o = 0; o < 2; ++o) r[j][o] = to_f4(v[j][o]);
    }
};
template <int OPB> struct RingRead<uint16_t, 3, OPB> {
    __device__ static inline void run(const uint32_t (&a)[3], float4 (&r)[3][3]) {
        hx_u32x2 v[3][3];
        asm volatile(
            "ds_read_b64 %0, %9\n\tds_read_b64 %1, %9 offset:%12\n\tds_read_b64 %2, %9 offset:%13\n\t"
            "ds_read_b64 %3, %10\n\tds_read_b64 %4, %10 offset:%12\n\tds_read_b64 %5, %10 offset:%13\n\t"
            "ds_read_b64 %6, %11\n\tds_read_b64 %7, %11 offset:%12\n\tds_read_b64 %8, %11 offset:%13\n\t"
            "s_waitcnt lgkmcnt(0)"
            : "=&v"(v[0][0]), "=&v"(v[0][1]), "=&v"(v[0][2]), "=&v"(v[1][0]), "=&v"(v[1][1]), "=&v"(v[1][2]),
              "=&v"(v[2][0]), "=&v"(v[2][1]), "=&v"(v[2][2])
            : "v"(a[0]), "v"(a[1]), "v"(a[2]), "n"(OPB), "n"(2 * OPB)
            : "memory");
#pragma unroll
        for (int j = 0; j < 3; ++j)
#pragma unroll
            for (int o = 0; o < 3; ++o) r[j][o] = bf16x4_to_f4(v[j][o]);
    }
};
template <int OPB> struct RingRead<uint16_t, 2, OPB> {
    __device__ static inline void run(const uint32_t (&a)[3], float4 (&r)[3][3]) {
        hx_u32x2 v[3][2];
        asm volatile(
            "ds_read_b64 %0, %6\n\tds_read_b64 %1, %6 offset:%9\n\t"
            "ds_read_b64 %2, %7\n\tds_read_b64 %3, %7 offset:%9\n\t"
            "ds_read_b64 %4, %8\n\tds_read_b64 %5, %8 offset:%9\n\t"
            "s_waitcnt lgkmcnt(0)"
            : "=&v"(v[0][0]), "=&v"(v[0][1]), "=&v"(v[1][0]), "=&v"(v[1][1]), "=&v"(v[2][0]), "=&v"(v[2][1])
            : "v"(a[0]), "v"(a[1]), "v"(a[2]), "n"(OPB)
            : "memory");
#pragma unroll
        for (int j = 0; j < 3; ++j)
#pragma unroll
            for (int o = 0; o < 2; ++o) r[j][o] = bf16x4_to_f4(v[j][o]);
    }
};

// r[m][o] = the fp32 words at a + o * OPB + 64 m and 768 bytes further (one channel at two steps
// 4 rows of 48 channels apart), o < NOP (2 or 3), m < 3: ds_read2_b32 with dword offsets 16m and
// 16m + 192.
template <int NOP, int OPB> struct RingRead2 {
    __device__ static inline void run(uint32_t a, float2 (&r)[3][3]) {
        const uint32_t a1 = a + OPB, a2 = a + 2 * OPB;
        hx_u32x2 v[3][3];
        if constexpr (NOP == 3) {
            asm volatile(
                "ds_read2_b32 %0, %9 offset1:192\n\tds_read2_b32 %1, %10 offset1:192\n\tds_read2_b32 %2, %11 offset1:192\n\t"
                "ds_read2_b32 %3, %9 offset0:16 offset1:208\n\tds_read2_b32 %4, %10 offset0:16 offset1:208\n\t"
                "ds_read2_b32 %5, %11 offset0:16 offset1:208\n\t"
                "ds_read2_b32 %6, %9 offset0:32 offset1:224\n\tds_read2_b32 %7, %10 offset0:32 offset1:224\n\t"
                "ds_read2_b32 %8, %11 offset0:32 offset1:224\n\t"
                "s_waitcnt lgkmcnt(0)"
                : "=&v"(v[0][0]), "=&v"(v[0][1]), "=&v"(v[0][2]), "=&v"(v[1][0]), "=&v"(v[1][1]), "=&v"(v[1][2]),
                  "=&v"(v[2][0]), "=&v"(v[2][1]), "=&v"(v[2][2])
                : "v"(a), "v"(a1), "v"(a2)
                : "memory");
        } else {
            (void)a2;
            asm volatile(
                "ds_read2_b32 %0, %6 offset1:192\n\tds_read2_b32 %1, %7 offset1:192\n\t"
                "ds_read2_b32 %2, %6 offset0:16 offset1:208\n\tds_read2_b32 %3, %7 offset0:16 offset1:208\n\t"
                "ds_read2_b32 %4, %6 offset0:32 offset1:224\n\tds_read2_b32 %5, %7 offset0:32 offset1:224\n\t"
                "s_waitcnt lgkmcnt(0)"
                : "=&v"(v[0][0]), "=&v"(v[0][1]), "=&v"(v[1][0]), "=&v"(v[1][1]), "=&v"(v[2][0]), "=&v"(v[2][1])
                : "v"(a), "v"(a1)
                : "memory");
        }
#pragma unroll
        for (int m = 0; m < 3; ++m)
#pragma unroll
            for (int o = 0; o < NOP; ++o) r[m][o] = make_float2(__uint_as_float(v[m][o][0]), __uint_as_float(v[m][o][1]));
    }
};

// bf16 ring of scan_ws2_kernel: r[m][o] = the bf16 channel `odd` of the dword at
// a + o * OPB + 32 m and of the dword 384 bytes further (one channel pair at two steps 4 rows of
// 48 bf16 channels apart), widened to fp32; ds_read2_b32 with dword offsets 8m and 8m + 96.
template <int NOP, int OPB> struct RingRead2Bf16 {
    __device__ static inline void run(uint32_t a, int odd, float2 (&r)[3][3]) {
        const uint32_t a1 = a + OPB, a2 = a + 2 * OPB;
        hx_u32x2 v[3][3];
        if constexpr (NOP == 3) {
            asm volatile(
                "ds_read2_b32 %0, %9 offset1:96\n\tds_read2_b32 %1, %10 offset1:96\n\tds_read2_b32 %2, %11 offset1:96\n\t"
                "ds_read2_b32 %3, %9 offset0:8 offset1:104\n\tds_read2_b32 %4, %10 offset0:8 offset1:104\n\t"
                "ds_read2_b32 %5, %11 offset0:8 offset1:104\n\t"
                "ds_read2_b32 %6, %9 offset0:16 offset1:112\n\tds_read2_b32 %7, %10 offset0:16 offset1:112\n\t"
                "ds_read2_b32 %8, %11 offset0:16 offset1:112\n\t"
                "s_waitcnt lgkmcnt(0)"
                : "=&v"(v[0][0]), "=&v"(v[0][1]), "=&v"(v[0][2]), "=&v"(v[1][0]), "=&v"(v[1][1]), "=&v"(v[1][2]),
                  "=&v"(v[2][0]), "=&v"(v[2][1]), "=&v"(v[2][2])
                : "v"(a), "v"(a1), "v"(a2)
                : "memory");
        } else {
            (void)a2;
            asm volatile(
                "ds_read2_b32 %0, %6 offset1:96\n\tds_read2_b32 %1, %7 offset1:96\n\t"
                "ds_read2_b32 %2, %6 offset0:8 offset1:104\n\tds_read2_b32 %3, %7 offset0:8 offset1:104\n\t"
                "ds_read2_b32 %4, %6 offset0:16 offset1:112\n\tds_read2_b32 %5, %7 offset0:16 offset1:112\n\t"
                "s_waitcnt lgkmcnt(0)"
                : "=&v"(v[0][0]), "=&v"(v[0][1]), "=&v"(v[1][0]), "=&v"(v[1][1]), "=&v"(v[2][0]), "=&v"(v[2][1])
                : "v"(a), "v"(a1)
                : "memory");
        }
#pragma unroll
        for (int m = 0; m < 3; ++m)
#pragma unroll
            for (int o = 0; o < NOP; ++o) {
                const uint32_t x = v[m][o][0], y = v[m][o][1];
                r[m][o] = make_float2(__uint_as_float(odd ? (x & 0xffff0000u) : (x << 16)),
                                      __uint_as_float(odd ? (y & 0xffff0000u) : (y << 16)));
            }
    }
};

// Output-stage reads of scan_ws2_kernel's element waves, as inline asm (see RingRead): for
// m < 3, y0/y1[m] = the float2 at ay + 1024 m (+ 3072 for the upper half's partials), uu[m] =
// the float2 at ax + 1280 m (u), gz[m] the same OPS bytes further (SiLU(z)) when HZ.
template <bool HZ, int OPS> struct HandoverRead {
    __device__ static inline void run(uint32_t ay, uint32_t ax, float2 (&y0)[3], float2 (&y1)[3],
                                      float2 (&uu)[3], float2 (&gz)[3]) {
        hx_u32x2 a[3], bq[3], u[3], zz[3];
        if constexpr (HZ) {
            asm volatile(
                "ds_read_b64 %0, %12\n\tds_read_b64 %1, %12 offset:1024\n\tds_read_b64 %2, %12 offset:2048\n\t"
                "ds_read_b64 %3, %12 offset:3072\n\tds_read_b64 %4, %12 offset:4096\n\tds_read_b64 %5, %12 offset:5120\n\t"
                "ds_read_b64 %6, %13\n\tds_read_b64 %7, %13 offset:1280\n\tds_read_b64 %8, %13 offset:2560\n\t"
                "ds_read_b64 %9, %13 offset:%14\n\tds_read_b64 %10, %13 offset:%15\n\tds_read_b64 %11, %13 offset:%16\n\t"
                "s_waitcnt lgkmcnt(0)"
                : "=&v"(a[0]), "=&v"(a[1]), "=&v"(a[2]), "=&v"(bq[0]), "=&v"(bq[1]), "=&v"(bq[2]),
                  "=&v"(u[0]), "=&v"(u[1]), "=&v"(u[2]), "=&v"(zz[0]), "=&v"(zz[1]), "=&v"(zz[2])
                : "v"(ay), "v"(ax), "n"(OPS), "n"(OPS + 1280), "n"(OPS + 2560)
                : "memory");
        } else {
            asm volatile(
                "ds_read_b64 %0, %9\n\tds_read_b64 %1, %9 offset:1024\n\tds_read_b64 %2, %9 offset:2048\n\t"
                "ds_read_b64 %3, %9 offset:3072\n\tds_read_b64 %4, %9 offset:4096\n\tds_read_b64 %5, %9 offset:5120\n\t"
                "ds_read_b64 %6, %10\n\tds_read_b64 %7, %10 offset:1280\n\tds_read_b64 %8, %10 offset:2560\n\t"
                "s_waitcnt lgkmcnt(0)"
                : "=&v"(a[0]), "=&v"(a[1]), "=&v"(a[2]), "=&v"(bq[0]), "=&v"(bq[1]), "=&v"(bq[2]),
                  "=&v"(u[0]), "=&v"(u[1]), "=&v"(u[2])
                : "v"(ay), "v"(ax)
                : "memory");
        }
#pragma unroll
        for (int m = 0; m < 3; ++m) {
            y0[m] = make_float2(__uint_as_float(a[m][0]), __uint_as_float(a[m][1]));
            y1[m] = make_float2(__uint_as_float(bq[m][0]), __uint_as_float(bq[m][1]));
            uu[m] = make_float2(__uint_as_float(u[m][0]), __uint_as_float(u[m][1]));
            gz[m] = HZ ? make_float2(__uint_as_float(zz[m][0]), __uint_as_float(zz[m][1])) : make_float2(1.0f, 1.0f);
        }
    }
};

// One element stored through a raw buffer resource: offsets at or past the resource's size are
// dropped by the hardware, so a store needs no branch (and the compiler's wait counts stay exact).
// Cache policy of the split-state kernel's input loads and of the warp-specialised kernels'
// output stores: non-temporal (each element is read or written once; config 2 132.0 -> 130.3
// us). The wave kernel keeps the default: streaming its loads and stores measured config 4
// 0.70 -> 0.80 ms (the end-state pass's reads are read again by the full pass) and config 3
// slower.
constexpr int kStream = 2;
__device__ inline void buf_store(float v, __amdgpu_buffer_rsrc_t rs, uint32_t off, float*) {
    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), rs, off, 0, kStream);
}
__device__ inline void buf_store(float v, __amdgpu_buffer_rsrc_t rs, uint32_t off, uint16_t*) {
    __builtin_amdgcn_raw_buffer_store_b16(Storage<uint16_t>::round(v), rs, off, 0, kStream);
}
constexpr int kBufRsrcWord3 = 0x00020000;  // gfx9 raw buffer: 32-bit data format, no swizzle

// ----------------------------------------------------------------------------- warp-specialised
// A block of 4 waves owns 48 channels of one batch row, and its waves have different jobs:
//   * waves 0..2 ("state waves") each own 16 of the channels x all 16 states in the layout of
//     scan_wave3_kernel (lane (r, c): channel c, states 4r..4r+3; B/C of step t0+j in lane j of
//     row r, reaching the multiplies by DPP row_newbcast). Per state update they issue one
//     v_exp, dt*A, B*(dt*u), the FMA and the DPP readout FMA; per chunk they reduce-scatter the
//     per-row readouts across rows (lane (r, c) ends with steps r + 4i of channel c), add D*u,
//     apply the gate and store, in scan_wave3_kernel's operation order (the two kernels give
//     bit-identical results);
//   * wave 3 (the "element wave") does the rest of the per-(t, channel) work for the 48
//     channels: u/delta/z move from HBM straight into an NR-deep LDS ring (gfx950
//     global_load_lds: 64 lanes x VB bytes into one contiguous piece of LDS per instruction,
//     so a chunk lands as [operand][step][48 channels] rows) under the wave's own vmcnt waits;
//     from there it computes softplus(delta + bias), dt*u and SiLU(z).
// The roles hand over through LDS with one barrier per 16-step chunk and a 3-deep buffer: in
// phase p the state waves scan chunk p (dt, dt*u read during phase p-1; u, SiLU(z) from
// buffer p%3) and read chunk p+1's dt and dt*u, while the element wave prepares chunk p+2 into
// buffer (p+2)%3. Steps past the end get dt = 0 and dt*u = 0, which leave the state unchanged,
// and their stores fall outside the buffer resource. The dynamic LDS request keeps one block per
// CU, so every SIMD runs one wave. Requires Dm % 4 == 0, 16-byte rows,
// (L + 16) * Dm * es < 2^32 (byte offsets of a batch row, padded steps included, in 32 bits).
template <typename T, int NR, bool HAS_Z, bool SOFTPLUS>
__global__ __launch_bounds__(256) void scan_ws_kernel(
    int64_t L, int64_t Dm, int ngrp,
    const T* __restrict__ u, const T* __restrict__ delta, const float* __restrict__ A,
    const T* __restrict__ Bm, const T* __restrict__ Cm, const float* __restrict__ Dv,
    const T* __restrict__ z, const float* __restrict__ dt_bias, T* __restrict__ out,
    const float* __restrict__ init_state, float* __restrict__ last_state) {
    constexpr int NS = 16, TCH = 16, GCH = 48, DS = 20;
    // Hand-over buffers [buf][dt | dt*u | u | SiLU(z)][ch][.], rows padded to 20 words:
    // dt and dt*u by step (a state lane reads its channel's 16 steps as 4 float4s); u and
    // SiLU(z) with step r + 4i at index 4r + i (the order in which the state waves' lanes hold
    // the steps after the reduce-scatter: one float4 per lane)
    __shared__ __attribute__((aligned(16))) float s_x[3][4][GCH][DS];

    const int nblk = gridDim.x;
    int id = blockIdx.x;
    if ((nblk & 7) == 0) id = (id & 7) * (nblk >> 3) + (id >> 3);  // XCD-aware order
    const int grp = id % ngrp;
    const int64_t b = id / ngrp;
    const int64_t cblk = (int64_t)grp * GCH;
    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nch = (int)((L + TCH - 1) / TCH);
    const uint32_t D32 = (uint32_t)Dm;

    if (w < 3) {
        // ------------------------------------------------------------ state wave
        const int r = lane >> 4, c = lane & 15;
        const int lch = 16 * w + c;  // channel within the block
        const int64_t d = cblk + lch;
        const bool dvalid = d < Dm;
        const int64_t dc = dvalid ? d : Dm - 1;
        float A2[4], h[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            A2[k] = A[dc * NS + 4 * r + k] * kLog2e;
            h[k] = init_state ? init_state[(b * Dm + dc) * NS + 4 * r + k] : 0.0f;
        }
        const float Dd = Dv ? Dv[dc] : 0.0f;
        const T* Bb = Bm + b * L * NS;
        const T* Cb = Cm + b * L * NS;
        const uint32_t bc_last = (uint32_t)(L - 1) * NS + 4 * r;
        uint32_t bc_next = (uint32_t)c * NS + 4 * r;
        float4 rb[2], rc[2];
        auto fetch = [&](int k) __attribute__((always_inline)) {
            const uint32_t bo = bc_next < bc_last ? bc_next : bc_last;
            rb[k] = Vec4<T>::load(Bb + bo);
            rc[k] = Vec4<T>::load(Cb + bo);
            bc_next += TCH * NS;
        };
        const uint32_t nrec = (uint32_t)(L * Dm * (int64_t)sizeof(T));
        const uint32_t row_bytes = D32 * (uint32_t)sizeof(T);
        // byte offset of (step r, this channel); invalid channels start past the end
        const uint32_t lane_off = dvalid ? ((uint32_t)r * D32 + (uint32_t)d) * (uint32_t)sizeof(T) : nrec;
        const __amdgpu_buffer_rsrc_t ors =
            __builtin_amdgcn_make_buffer_rsrc(out + b * L * Dm, (short)0, (int)nrec, kBufRsrcWord3);
        float dl[2][16], du[2][16];
        auto read_dt = [&](auto kc, int b3) __attribute__((always_inline)) {
            constexpr int k = decltype(kc)::value;
            const float* p0 = &s_x[b3][0][lch][0];
            const float* p1 = &s_x[b3][1][lch][0];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float4 a = *reinterpret_cast<const float4*>(p0 + 4 * i);
                const float4 q = *reinterpret_cast<const float4*>(p1 + 4 * i);
                dl[k][4 * i] = a.x; dl[k][4 * i + 1] = a.y; dl[k][4 * i + 2] = a.z; dl[k][4 * i + 3] = a.w;
                du[k][4 * i] = q.x; du[k][4 * i + 1] = q.y; du[k][4 * i + 2] = q.z; du[k][4 * i + 3] = q.w;
            }
        };
        fetch(0);
        fetch(1);
        lds_barrier();  // chunks 0 and 1 prepared
        read_dt(std::integral_constant<int, 0>{}, 0);
        int b3 = 0;  // p % 3
        for (int p0 = 0; p0 < nch; p0 += 2) {
            StepLoop<2>::run([&](auto kc) __attribute__((always_inline)) {
                constexpr int k = decltype(kc)::value;  // = p & 1: dt register set and B/C slot
                const int p = p0 + k;
                if (p >= nch) return;  // uniform
                const int b3n = b3 == 2 ? 0 : b3 + 1;
                if (p + 1 < nch) read_dt(std::integral_constant<int, k ^ 1>{}, b3n);
                const float4 fu = *reinterpret_cast<const float4*>(&s_x[b3][2][lch][4 * r]);  // u
                const float4 fz = HAS_Z ? *reinterpret_cast<const float4*>(&s_x[b3][3][lch][4 * r])
                                        : make_float4(1.0f, 1.0f, 1.0f, 1.0f);
                const float fuv[4] = {fu.x, fu.y, fu.z, fu.w};
                const float fzv[4] = {fz.x, fz.y, fz.z, fz.w};
                const float bk[4] = {rb[k].x, rb[k].y, rb[k].z, rb[k].w};
                const float ck[4] = {rc[k].x, rc[k].y, rc[k].z, rc[k].w};
                float P[16];
                StepLoop<4>::run([&](auto gc) __attribute__((always_inline)) {
                    constexpr int g = decltype(gc)::value;
                    float ab[4][4];
#pragma unroll
                    for (int e = 0; e < 4; ++e)
#pragma unroll
                        for (int kk = 0; kk < 4; ++kk) ab[e][kk] = fast_exp2(dl[k][4 * g + e] * A2[kk]);
                    StepLoop<4>::run([&](auto ec) __attribute__((always_inline)) {
                        constexpr int e = decltype(ec)::value;
                        constexpr int s = 4 * g + e;
#pragma unroll
                        for (int kk = 0; kk < 4; ++kk)
                            h[kk] = fmaf(ab[e][kk], h[kk], dpp<kDppBcast<s>>(bk[kk]) * du[k][s]);
                        float acc = dpp<kDppBcast<s>>(ck[0]) * h[0];
                        acc = fmac_bcast<s>(acc, ck[1], h[1]);
                        acc = fmac_bcast<s>(acc, ck[2], h[2]);
                        acc = fmac_bcast<s>(acc, ck[3], h[3]);
                        P[(s >> 2) + 4 * (s & 3)] = acc;  // j = i + 4*rr for s = rr + 4*i
                    });
                });
                fetch(k);  // chunk p + 2, into the slot this chunk's B/C came from
                float Y[4];
                rows_reduce_scatter(P, Y);  // Y[i]: step r + 4i
                // step r + 4i of this chunk sits at lane_off + (16p + 4i) * row bytes; steps past
                // the end land at or past nrec and are dropped. Lanes of channels past Dm stay at
                // nrec: adding the chunk term could wrap their 32-bit offset back below nrec.
                const uint32_t chunk_off =
                    dvalid ? lane_off + (uint32_t)p * (uint32_t)TCH * row_bytes : nrec;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    float y = fmaf(Dd, fuv[i], Y[i]);  // as scan_wave3_kernel: identical results
                    if (HAS_Z) y *= fzv[i];
                    buf_store(y, ors, chunk_off + 4 * i * row_bytes, (T*)nullptr);
                }
                b3 = b3n;
                lds_barrier();
            });
        }
        if (last_state && dvalid) {
#pragma unroll
            for (int k = 0; k < 4; ++k) last_state[(b * Dm + d) * NS + 4 * r + k] = h[k];
        }
    } else {
        // ------------------------------------------------------------ element wave
        constexpr int ES = (int)sizeof(T);
        constexpr int VB = ES == 4 ? 16 : 4;           // bytes per lane per load
        constexpr int ROWB = GCH * ES;                 // one step of 48 channels
        constexpr int OPB = TCH * ROWB;                // one operand of one chunk
        constexpr int NI = OPB / (64 * VB);            // loads per operand per chunk
        constexpr int LPR = ROWB / VB;                 // lanes per step row
        constexpr int NOP = HAS_Z ? 3 : 2;
        constexpr int LPC = NOP * NI;                  // loads per chunk
        constexpr int STB = NOP * OPB;                 // LDS bytes per ring stage
        constexpr int WAITN = (NR - 1) * LPC;
        static_assert(OPB % (64 * VB) == 0 && WAITN <= 63, "load split / vmcnt range");
        extern __shared__ __attribute__((aligned(16))) char s_ring[];  // [NR][operand][step][ch]

        // this lane's source offsets (elements within a batch row, chunk 0) per load instruction
        uint32_t srow[NI], scol[NI];
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const int q = 64 * i + lane;
            srow[i] = (uint32_t)(q / LPR);
            const int64_t ch = cblk + (q % LPR) * (VB / ES);
            scol[i] = (uint32_t)(ch < Dm ? ch : 0);  // a lane's channels are all valid or all not
        }
        const T* ub = u + b * L * Dm;
        const T* db = delta + b * L * Dm;
        const T* zb = HAS_Z ? z + b * L * Dm : nullptr;
        const uint32_t t_last = (uint32_t)(L - 1);
        auto issue = [&](int stage, int q) __attribute__((always_inline)) {
            char* dst = s_ring + stage * STB;
#pragma unroll
            for (int i = 0; i < NI; ++i) {
                uint32_t t = (uint32_t)q * TCH + srow[i];
                t = t < t_last ? t : t_last;  // rows past the end: loaded, never used
                const uint32_t off = t * D32 + scol[i];
                load_lds<VB>(ub + off, dst + i * 64 * VB);
                load_lds<VB>(db + off, dst + OPB + i * 64 * VB);
                if (HAS_Z) load_lds<VB>(zb + off, dst + 2 * OPB + i * 64 * VB);
            }
        };

        // element group j (0..2) of a chunk: step sj[j], channels cj[j] .. cj[j]+3 of the block
        int sj[3], cj[3];
        float bias_r[3][4];
#pragma unroll
        for (int j = 0; j < 3; ++j) {
            const int q = 64 * j + lane;
            sj[j] = q / 12;
            cj[j] = (q % 12) * 4;
            const int64_t ch = cblk + cj[j];
            const bool cv = ch < Dm;  // Dm % 4 == 0: a group is all valid or all invalid
#pragma unroll
            for (int e = 0; e < 4; ++e) bias_r[j][e] = (dt_bias && cv) ? dt_bias[ch + e] : 0.0f;
        }
        // chunk q, from ring stage `stage`, into buffer b3
        auto prepare = [&](int stage, int b3, int q) __attribute__((always_inline)) {
            const char* src = s_ring + stage * STB;
            uint32_t ra[3];
#pragma unroll
            for (int j = 0; j < 3; ++j) ra[j] = lds_off(src + sj[j] * ROWB + cj[j] * ES);
            float4 raw[3][3];  // [j][u | delta | z]
            RingRead<T, NOP, OPB>::run(ra, raw);
#pragma unroll
            for (int j = 0; j < 3; ++j) {
                const bool tv = (int64_t)q * TCH + sj[j] < L;
                const int sp = (sj[j] & 3) * 4 + (sj[j] >> 2);  // step r + 4i at 4r + i
                float x[4], xu[4], uv[4], fz[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    float v = f4get(raw[j][1], e) + bias_r[j][e];
                    if (SOFTPLUS) v = softplus(v);
                    v = tv ? v : 0.0f;
                    const float uu = f4get(raw[j][0], e);
                    x[e] = v;
                    xu[e] = v * uu;
                    uv[e] = uu;
                    fz[e] = HAS_Z ? silu(f4get(raw[j][NOP - 1], e)) : 1.0f;
                }
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    s_x[b3][0][cj[j] + e][sj[j]] = x[e];
                    s_x[b3][1][cj[j] + e][sj[j]] = xu[e];
                    s_x[b3][2][cj[j] + e][sp] = uv[e];
                    if (HAS_Z) s_x[b3][3][cj[j] + e][sp] = fz[e];
                }
            }
        };
        auto wait_loads = [&]() __attribute__((always_inline)) {
            asm volatile("s_waitcnt vmcnt(%0)" ::"n"(WAITN) : "memory");
        };
        auto barrier = [&]() __attribute__((always_inline)) {
            asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        };
        // ring stage of chunk q is q % NR; every chunk index issues exactly LPC loads (clamped
        // rows past the end), so the wait count is the same before every prepare
#pragma unroll
        for (int k = 0; k < NR; ++k) issue(k, k);
        int stage = 0;  // q % NR of the next chunk to prepare
        int b3 = 0;     // q % 3 of the next chunk to prepare
        int q = 0;      // next chunk to prepare
        auto step = [&]() __attribute__((always_inline)) {
            wait_loads();
            prepare(stage, b3, q);
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // stage read before it is refilled
            issue(stage, q + NR);
            stage = stage + 1 == NR ? 0 : stage + 1;
            b3 = b3 == 2 ? 0 : b3 + 1;
            ++q;
        };
        step();               // chunk 0
        if (nch > 1) step();  // chunk 1
        barrier();
        for (int p = 0; p < nch; ++p) {
            if (p + 2 < nch) step();  // chunk p + 2
            barrier();
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // no load still writing LDS at exit
    }
}

// ----------------------------------------------------------------------------- split-state form
// Warp-specialised scan with every SIMD running two waves, so one wave's waits (hand-over
// barrier, B/C loads, LDS reads, dependent issue) overlap the other's issue. A block of 8 waves
// owns 48 channels of one batch row (fp32 or bf16 storage; the arithmetic is fp32):
//   * waves 0..2 and 4..6 are state waves: wave w < 3 holds states 0..7 of channel group w,
//     wave w > 3 states 8..15 of group w - 4 (lane (r, c): channel c, states 8h + 2r, 8h + 2r + 1;
//     B/C of step t0 + j in lane j of row r). Each reduce-scatters its 8 states' readouts
//     across rows and publishes the per-step partial sums of its half in LDS (s_y);
//   * waves 3 and 7 are element waves, each owning half of every chunk's steps for all 48
//     channels: they prepare softplus(delta + bias), dt*u, u and SiLU(z) two chunks ahead of the
//     scan, and one phase after a chunk is scanned (after the chunk barrier) they finish it: the
//     two halves' partial sums, D*u, the gate and the stores.
// Waves of a block are placed on SIMDs round-robin, so waves w and w + 4 share a SIMD: SIMDs
// 0..2 each run a lower and an upper state wave, SIMD 3 the two element waves. The hand-over
// buffers hold each channel's 16 steps in the order 4 (s % 4) + s / 4 for all four operands.
// The readout is summed as (states 0..7) + (states 8..15), so results match scan_ws_kernel to
// rounding, not bit for bit. Requires Dm % 4 == 0 (Dm % 8 == 0 for bf16 storage), 16-byte rows,
// (L + 48) * Dm * es < 2^32.
template <typename T> struct Pair;
template <> struct Pair<float> {
    __device__ static inline float2 load(const float* p) { return *reinterpret_cast<const float2*>(p); }
};
template <> struct Pair<uint16_t> {
    __device__ static inline float2 load(const uint16_t* p) {
        const uint32_t r = *reinterpret_cast<const uint32_t*>(p);
        return make_float2(__uint_as_float(r << 16), __uint_as_float(r & 0xffff0000u));
    }
};

template <typename T, int NR, bool HAS_Z, bool SOFTPLUS>
__global__ __launch_bounds__(512) void scan_ws2_kernel(
    int64_t L, int64_t Dm, int ngrp,
    const T* __restrict__ u, const T* __restrict__ delta, const float* __restrict__ A,
    const T* __restrict__ Bm, const T* __restrict__ Cm, const float* __restrict__ Dv,
    const T* __restrict__ z, const float* __restrict__ dt_bias, T* __restrict__ out,
    const float* __restrict__ init_state, float* __restrict__ last_state) {
    constexpr int NS = 16, TCH = 16, GCH = 48, DS = 20;
    constexpr int NOP = HAS_Z ? 3 : 2;
    constexpr int ES = (int)sizeof(T);
    constexpr int NLD = ES / 2;               // 64-lane x 16-byte loads per operand of a half chunk
    constexpr int OPB = NLD * 1024;           // ring slot of one operand of a half chunk (8 steps x
                                              // 48 channels = 1536 or 768 bytes, padded to whole loads)
    constexpr int STB = NOP * OPB;            // one ring stage
    constexpr int RING = 2 * NR * STB;        // both element waves' rings
    // All LDS is the dynamic allocation, rings first: the LDS base of a load to LDS is a 16-bit
    // byte address, so the rings must lie below 64 KiB. Then the hand-over buffers
    // s_x[buf][dt | dt*u | u | SiLU(z)][ch][20] and the lower halves' readouts s_y[2][group][lane].
    extern __shared__ __attribute__((aligned(16))) char s_dyn[];
    static_assert(RING <= 65536 - 1024, "rings below 64 KiB");
    auto& s_x = *reinterpret_cast<float(*)[3][4][GCH][DS]>(s_dyn + RING);
    auto& s_y = *reinterpret_cast<float4(*)[2][2][3][64]>(s_dyn + RING + sizeof(float) * 3 * 4 * GCH * DS);

    const int nblk = gridDim.x;
    int id = blockIdx.x;
    if ((nblk & 7) == 0) id = (id & 7) * (nblk >> 3) + (id >> 3);  // XCD-aware order
    const int grp = id % ngrp;
    const int64_t b = id / ngrp;
    const int64_t cblk = (int64_t)grp * GCH;
    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nch = (int)((L + TCH - 1) / TCH);

    auto state_wave = [&](auto hc) __attribute__((always_inline)) {
        constexpr int HH = decltype(hc)::value;  // 0: states 0..7, 1: states 8..15
        const int g = HH ? w - 4 : w;
        const int r = lane >> 4, c = lane & 15;
        const int lch = 16 * g + c;
        const int st0 = 8 * HH + 2 * r;
        const int64_t d = cblk + lch;
        const bool dvalid = d < Dm;
        const int64_t dc = dvalid ? d : Dm - 1;
        float A2[2], h[2];
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            A2[k] = A[dc * NS + st0 + k] * kLog2e;
            h[k] = init_state ? init_state[(b * Dm + dc) * NS + st0 + k] : 0.0f;
        }
        const T* Bb = Bm + b * L * NS;
        const T* Cb = Cm + b * L * NS;
        const uint32_t bc_last = (uint32_t)(L - 1) * NS + st0;
        uint32_t bc_next = (uint32_t)c * NS + st0;
        float2 rb[2], rc[2];
        auto fetch = [&](int k) __attribute__((always_inline)) {
            const uint32_t bo = bc_next < bc_last ? bc_next : bc_last;
            rb[k] = Pair<T>::load(Bb + bo);
            rc[k] = Pair<T>::load(Cb + bo);
            bc_next += TCH * NS;
        };
        float dl[2][16], du[2][16];
        auto read_dt = [&](auto kc, int b3) __attribute__((always_inline)) {
            constexpr int k = decltype(kc)::value;
            const float* p0 = &s_x[b3][0][lch][0];
            const float* p1 = &s_x[b3][1][lch][0];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float4 a = *reinterpret_cast<const float4*>(p0 + 4 * i);
                const float4 q = *reinterpret_cast<const float4*>(p1 + 4 * i);
                // index 4i + j of a channel row holds step 4j + i
                dl[k][i] = a.x; dl[k][4 + i] = a.y; dl[k][8 + i] = a.z; dl[k][12 + i] = a.w;
                du[k][i] = q.x; du[k][4 + i] = q.y; du[k][8 + i] = q.z; du[k][12 + i] = q.w;
            }
        };
        fetch(0);
        fetch(1);
        lds_barrier();  // chunks 0 and 1 prepared
        read_dt(std::integral_constant<int, 0>{}, 0);
        int b3 = 0;  // p % 3
        for (int p0 = 0; p0 < nch; p0 += 2) {
            StepLoop<2>::run([&](auto kc) __attribute__((always_inline)) {
                constexpr int k = decltype(kc)::value;  // = p & 1: dt register set and B/C slot
                const int p = p0 + k;
                if (p >= nch) return;  // uniform
                const int b3n = b3 == 2 ? 0 : b3 + 1;
                if (p + 1 < nch) read_dt(std::integral_constant<int, k ^ 1>{}, b3n);
                const float bk[2] = {rb[k].x, rb[k].y};
                const float ck[2] = {rc[k].x, rc[k].y};
                float P[16];
                StepLoop<4>::run([&](auto gc) __attribute__((always_inline)) {
                    constexpr int g4 = decltype(gc)::value;
                    float ab[4][2];
#pragma unroll
                    for (int e = 0; e < 4; ++e)
#pragma unroll
                        for (int kk = 0; kk < 2; ++kk) ab[e][kk] = fast_exp2(dl[k][4 * g4 + e] * A2[kk]);
                    StepLoop<4>::run([&](auto ec) __attribute__((always_inline)) {
                        constexpr int e = decltype(ec)::value;
                        constexpr int s = 4 * g4 + e;
#pragma unroll
                        for (int kk = 0; kk < 2; ++kk)
                            h[kk] = fmaf(ab[e][kk], h[kk], dpp<kDppBcast<s>>(bk[kk]) * du[k][s]);
                        float acc = dpp<kDppBcast<s>>(ck[0]) * h[0];
                        acc = fmac_bcast<s>(acc, ck[1], h[1]);
                        P[(s >> 2) + 4 * (s & 3)] = acc;  // j = i + 4*rr for s = rr + 4*i
                    });
                });
                fetch(k);  // chunk p + 2, into the slot this chunk's B/C came from
                float Y[4];
                rows_reduce_scatter(P, Y);  // Y[i]: step r + 4i, this half's 8 states
                s_y[p & 1][HH][g][lane] = make_float4(Y[0], Y[1], Y[2], Y[3]);  // the element waves finish it
                b3 = b3n;
                lds_barrier();
            });
        }
        if (last_state && dvalid) {
#pragma unroll
            for (int k = 0; k < 2; ++k) last_state[(b * Dm + d) * NS + st0 + k] = h[k];
        }
    };

    if (w == 3 || w == 7) {
        // ------------------------------------------------------------ element waves
        // wave 3 prepares steps 0..7 of every chunk, wave 7 steps 8..15, for all 48 channels.
        // Each streams its 8 steps of u/delta/z straight into its own NR-deep LDS ring with
        // buffer loads to LDS (2 x 64 lanes x 16 bytes per operand, the last 512 bytes padding;
        // reads past the end of the batch row return zeros). Every chunk issues the same LPC
        // full-wave loads, with no branch the compiler could split, so the explicit vmcnt waits
        // count exactly. Lane (c, s2) then handles channels c, c + 16, c + 32 at
        // steps s2 and s2 + 4 of the wave's half: ring reads and hand-over writes of a wave
        // instruction touch distinct banks.
        const int e = w >> 2;
        constexpr int ROWB = GCH * ES;     // one step of 48 channels
        constexpr int LPR = ROWB / 16;     // load lanes per step row
        constexpr int EPP = 16 / ES;       // channels per 16-byte piece
        constexpr int LPC = NOP * NLD;     // loads per chunk
        constexpr int WAITN = (NR - 1) * LPC;
        static_assert(WAITN <= 63, "vmcnt range");
        char* ring = s_dyn + e * NR * STB;  // [NR][op][8 steps][48 ch]
        const uint32_t nrec = (uint32_t)(L * Dm * ES);
        const __amdgpu_buffer_rsrc_t rs_u =
            __builtin_amdgcn_make_buffer_rsrc((void*)(u + b * L * Dm), (short)0, (int)nrec, kBufRsrcWord3);
        const __amdgpu_buffer_rsrc_t rs_d =
            __builtin_amdgcn_make_buffer_rsrc((void*)(delta + b * L * Dm), (short)0, (int)nrec, kBufRsrcWord3);
        const __amdgpu_buffer_rsrc_t rs_z = __builtin_amdgcn_make_buffer_rsrc(
            (void*)(HAS_Z ? z + b * L * Dm : u + b * L * Dm), (short)0, (int)nrec, kBufRsrcWord3);
        // load instruction i, lane q: bytes 1024 i + 16 q of the half chunk = step 8e + (64 i + q) / LPR,
        // channels EPP ((64 i + q) % LPR) ..; pieces of channels past Dm read channel 0 (never
        // used); lanes past the 8 rows fill the slot's padding with chunk data that is never read
        uint32_t loff[2];  // NLD <= 2 used (a bound that depends on T, captured by the lambdas
                           // below, makes the host pass drop the kernels' launch stubs)
#pragma unroll
        for (int i = 0; i < NLD; ++i) {
            const int q = 64 * i + lane;
            const int64_t ch = cblk + (q % LPR) * EPP;
            loff[i] = q < 8 * LPR ? (uint32_t)(((8 * e + q / LPR) * Dm + (ch < Dm ? ch : 0)) * ES) : 0u;
        }
        const uint32_t chunk_bytes = (uint32_t)(TCH * Dm * ES);
        auto issue = [&](int stage, int qc) __attribute__((always_inline)) {
            char* dst = ring + stage * STB;
            const uint32_t cb = (uint32_t)qc * chunk_bytes;
#pragma unroll
            for (int i = 0; i < NLD; ++i) {
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rs_u, (lvoid_t*)(dst + 1024 * i), 16, loff[i] + cb, 0, 0, kStream);
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rs_d, (lvoid_t*)(dst + OPB + 1024 * i), 16, loff[i] + cb, 0, 0, kStream);
                if (HAS_Z)
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs_z, (lvoid_t*)(dst + 2 * OPB + 1024 * i), 16, loff[i] + cb, 0, 0, kStream);
            }
        };
        const int c = lane & 15, s2 = lane >> 4;
        float bias_r[3];
#pragma unroll
        for (int m = 0; m < 3; ++m) {
            const int64_t ch = cblk + c + 16 * m;
            bias_r[m] = (dt_bias && ch < Dm) ? dt_bias[ch] : 0.0f;
        }
        // chunk qc from ring stage `stage` into hand-over buffer b3: steps 8e + s2 + 4i (i < 2)
        // go to index 4 s2 + 2e + i of each channel row (the state waves' step order)
        auto prepare = [&](int stage, int b3, int qc) __attribute__((always_inline)) {
            float2 raw[3][3];  // [m][u | delta | z], .x step s2, .y step s2 + 4
            if constexpr (ES == 4) {
                RingRead2<NOP, OPB>::run(lds_off(ring + stage * STB + s2 * ROWB + c * 4), raw);
            } else {
                // the dword holding channels c & ~1 and c | 1; this lane's half by c's parity
                RingRead2Bf16<NOP, OPB>::run(lds_off(ring + stage * STB + s2 * ROWB + (c >> 1) * 4), c & 1, raw);
            }
#pragma unroll
            for (int m = 0; m < 3; ++m) {
                const int ch = c + 16 * m;
                float x[2], xu[2], uv[2], fz[2];
#pragma unroll
                for (int i = 0; i < 2; ++i) {
                    const bool tv = (int64_t)qc * TCH + 8 * e + s2 + 4 * i < L;
                    const float uu = i ? raw[m][0].y : raw[m][0].x;
                    float v = (i ? raw[m][1].y : raw[m][1].x) + bias_r[m];
                    if (SOFTPLUS) v = softplus(v);
                    v = tv ? v : 0.0f;
                    x[i] = v;
                    xu[i] = v * uu;
                    uv[i] = uu;
                    fz[i] = HAS_Z ? silu(i ? raw[m][NOP - 1].y : raw[m][NOP - 1].x) : 1.0f;
                }
                // inline-asm stores: for compiler-visible LDS stores the compiler would first wait
                // for every buffer load still writing the ring (vmcnt(0)); the barrier that ends
                // the phase waits for these stores (lgkmcnt(0))
                const uint32_t ha = lds_off(&s_x[b3][0][ch][4 * s2 + 2 * e]);
                const hx_u32x2 vx = {__float_as_uint(x[0]), __float_as_uint(x[1])};
                const hx_u32x2 vxu = {__float_as_uint(xu[0]), __float_as_uint(xu[1])};
                const hx_u32x2 vu = {__float_as_uint(uv[0]), __float_as_uint(uv[1])};
                const hx_u32x2 vz = {__float_as_uint(fz[0]), __float_as_uint(fz[1])};
                constexpr int OPS = GCH * DS * 4;  // bytes between the hand-over operands
                asm volatile("ds_write_b64 %0, %1\n\tds_write_b64 %0, %2 offset:%5\n\tds_write_b64 %0, %3 offset:%6"
                             :: "v"(ha), "v"(vx), "v"(vxu), "v"(vu), "v"(vz), "n"(OPS), "n"(2 * OPS) : "memory");
                if (HAS_Z) asm volatile("ds_write_b64 %0, %1 offset:%2" :: "v"(ha), "v"(vz), "n"(3 * OPS) : "memory");
            }
        };
        // outputs of chunk pc (its readouts published in phase pc, read in phase pc + 1): lane
        // (c, s2) sums both halves' partials for channels c + 16m at steps 8e + s2 + 4i, adds D*u,
        // applies the gate and stores; steps past the end fall at or past nrec (dropped), lanes of
        // channels past Dm stay at nrec
        float Dd[3];
        uint32_t obase[3];
#pragma unroll
        for (int m = 0; m < 3; ++m) {
            const int64_t ch = cblk + c + 16 * m;
            Dd[m] = (Dv && ch < Dm) ? Dv[ch] : 0.0f;
            obase[m] = ch < Dm ? (uint32_t)(((8 * e + s2) * Dm + ch) * ES) : nrec;
        }
        const __amdgpu_buffer_rsrc_t ors =
            __builtin_amdgcn_make_buffer_rsrc((void*)(out + b * L * Dm), (short)0, (int)nrec, kBufRsrcWord3);
        const uint32_t row4 = (uint32_t)(4 * Dm * ES);  // 4 steps
        auto finish = [&](int pc) __attribute__((always_inline)) {
            const uint32_t ay = lds_off(&s_y[pc & 1][0][0][s2 * 16 + c]) + 8 * e;
            const uint32_t ax = lds_off(&s_x[pc % 3][2][c][4 * s2 + 2 * e]);
            float2 y0[3], y1[3], uu[3], gz[3];
            HandoverRead<HAS_Z, GCH * DS * 4>::run(ay, ax, y0, y1, uu, gz);
#pragma unroll
            for (int m = 0; m < 3; ++m) {
                const uint32_t o = obase[m] < nrec ? obase[m] + (uint32_t)pc * chunk_bytes : nrec;
#pragma unroll
                for (int i = 0; i < 2; ++i) {
                    float y = fmaf(Dd[m], i ? uu[m].y : uu[m].x, (i ? y0[m].y : y0[m].x) + (i ? y1[m].y : y1[m].x));
                    if (HAS_Z) y *= i ? gz[m].y : gz[m].x;
                    buf_store(y, ors, o + (uint32_t)i * row4, (T*)nullptr);
                }
            }
        };

        auto barrier = [&]() __attribute__((always_inline)) {
            asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        };
        // ring stage of chunk q is q % NR; every chunk index issues exactly LPC loads and every
        // finish exactly 6 stores (stores count in vmcnt too). The wait before preparing chunk q
        // lets through what was issued after chunk q's loads: NR - 1 chunks of loads, plus, from
        // phase NR on, NR finishes' stores; before that, fewer stores were issued and the
        // smaller count only waits longer. The ring reads complete inside prepare, so the stage
        // is refilled right after it.
        constexpr int WAITS = WAITN + NR * 6;
        static_assert(WAITS <= 63, "vmcnt range");
#pragma unroll
        for (int k = 0; k < NR; ++k) issue(k, k);
        int stage = 0, b3 = 0, q = 0;
        auto step = [&](auto wc) __attribute__((always_inline)) {
            asm volatile("s_waitcnt vmcnt(%0)" ::"n"(decltype(wc)::value) : "memory");
            prepare(stage, b3, q);
            issue(stage, q + NR);
            stage = stage + 1 == NR ? 0 : stage + 1;
            b3 = b3 == 2 ? 0 : b3 + 1;
            ++q;
        };
        step(std::integral_constant<int, WAITN>{});                // chunk 0
        if (nch > 1) step(std::integral_constant<int, WAITN>{});  // chunk 1
        barrier();
        for (int p = 0; p < nch; ++p) {
            if (p > 0) finish(p - 1);  // before chunk p + 2 overwrites that chunk's u and SiLU(z)
            if (p + 2 < nch) {         // chunk p + 2
                if (p >= NR) step(std::integral_constant<int, WAITS>{});
                else step(std::integral_constant<int, WAITN>{});
            }
            barrier();
        }
        if (nch > 0) finish(nch - 1);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // no load still writing LDS at exit
    } else if (w < 3) {
        state_wave(std::integral_constant<int, 0>{});
    } else {
        state_wave(std::integral_constant<int, 1>{});
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

// dstate == 16 with 16-byte aligned state/A/B/C rows: the same arithmetic as state_update_kernel
// with the per-thread state, A, B and C rows moved as 16-byte vectors (4 float4 each; B and C as
// 16-byte groups of their storage type), cutting ~70 load/store instructions per thread to ~16.
template <typename T>
__global__ __launch_bounds__(128) void state_update16_kernel(
    int64_t Bt, int64_t Dm, int softplus_on, float* __restrict__ state,
    const T* __restrict__ u, const T* __restrict__ delta, const float* __restrict__ A,
    const T* __restrict__ Bm, const T* __restrict__ Cm, const float* __restrict__ Dv,
    const T* __restrict__ z, const float* __restrict__ dt_bias, T* __restrict__ out) {
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= Bt * Dm) return;
    const int64_t b = gid / Dm, d = gid - b * Dm;
    const float uv = ld(u + gid);
    float dl = ld(delta + gid) + (dt_bias ? dt_bias[d] : 0.0f);
    if (softplus_on) dl = softplus(dl);
    const float du = dl * uv;
    float h[16], a[16], bb[16], cc[16];
    float4* hs = reinterpret_cast<float4*>(state + gid * 16);
    const float4* as = reinterpret_cast<const float4*>(A + d * 16);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const float4 hv = hs[q], av = as[q];
        h[4 * q] = hv.x; h[4 * q + 1] = hv.y; h[4 * q + 2] = hv.z; h[4 * q + 3] = hv.w;
        a[4 * q] = av.x; a[4 * q + 1] = av.y; a[4 * q + 2] = av.z; a[4 * q + 3] = av.w;
        const float4 bv = Vec4<T>::load(Bm + b * 16 + 4 * q), cv = Vec4<T>::load(Cm + b * 16 + 4 * q);
        bb[4 * q] = bv.x; bb[4 * q + 1] = bv.y; bb[4 * q + 2] = bv.z; bb[4 * q + 3] = bv.w;
        cc[4 * q] = cv.x; cc[4 * q + 1] = cv.y; cc[4 * q + 2] = cv.z; cc[4 * q + 3] = cv.w;
    }
    float y = 0.0f;
#pragma unroll
    for (int n = 0; n < 16; ++n) {
        const float ab = fast_exp2(dl * (a[n] * kLog2e));
        h[n] = fmaf(ab, h[n], du * bb[n]);
        y = fmaf(cc[n], h[n], y);
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) hs[q] = make_float4(h[4 * q], h[4 * q + 1], h[4 * q + 2], h[4 * q + 3]);
    if (Dv) y = fmaf(Dv[d], uv, y);
    if (z) y *= silu(ld(z + gid));
    Storage<T>::store(out + gid, y);
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
    void* ws = nullptr;      // caller workspace for the segmented long-sequence path (nullable:
    size_t ws_bytes = 0;     // without one the sequence is never segmented)
};

// Time segments of the wave path: only when the (batch, 64-channel tile) pairs alone cannot fill
// the GPU (about 512 blocks, segments of at least 1024 steps), or as forced by
// hx_set_scan_segments; 16-step aligned. Returns the count and sets *seg_len.
int64_t scan_segments(const ScanArgs& a, int64_t* seg_len_out) {
    const int64_t pairs = ((a.Dm + 63) / 64) * a.Bt;
    int64_t nseg = 1;
    if (g_scan_segments > 0) {
        nseg = g_scan_segments;
    } else if (pairs < 256 && a.L >= 4096) {
        const int64_t want = (512 + pairs - 1) / pairs;
        const int64_t cap = a.L / 1024;
        nseg = want < cap ? want : cap;
        if (nseg < 1) nseg = 1;
    }
    int64_t seg_len = (a.L + nseg - 1) / nseg;
    seg_len = (seg_len + 15) / 16 * 16;
    *seg_len_out = seg_len;
    return (a.L + seg_len - 1) / seg_len;
}
// Scratch of a segmented scan: end states, entry states and decays, each [nseg][B][D][16].
size_t scan_seg_bytes(int64_t Bt, int64_t Dm, int64_t nseg) {
    if (nseg <= 1) return 0;
    const size_t per = (size_t)Bt * Dm * 16;
    return (size_t)nseg * 3 * per * sizeof(float);
}

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

// VER: 1 scan_wave_kernel (64-bit row offsets), 3 scan_wave3_kernel with 4 waves per block
template <typename T, int PF, bool HAS_Z, bool SP, bool END_ONLY, int VER>
int launch_wave_one(const ScanArgs& a, const WaveSeg& sg) {
    constexpr int WPB = 4;
    const int64_t ntiles = (a.Dm + 16 * WPB - 1) / (16 * WPB);
    // the end-state pass skips the last segment: nothing consumes its end state
    const int64_t nseg_run = END_ONLY ? sg.nseg - 1 : sg.nseg;
    HX_REQUIRE(ntiles * a.Bt * nseg_run <= 0x7fffffff, HX_ERR_UNSUPPORTED,
               "selective scan: %lld blocks exceed the grid", (long long)(ntiles * a.Bt * nseg_run));
    dim3 grid((unsigned)(ntiles * a.Bt * nseg_run));
    if constexpr (VER >= 3)
        hipLaunchKernelGGL((scan_wave3_kernel<T, PF, HAS_Z, SP, END_ONLY, WPB>), grid, dim3(64 * WPB), 0,
                           a.stream, a.L, a.Dm, (int)ntiles, a.Bt, (const T*)a.u, (const T*)a.delta, a.A,
                           (const T*)a.B, (const T*)a.C, a.D, (const T*)a.z, a.dt_bias, (T*)a.out,
                           a.init_state, a.last_state, sg);
    else
        hipLaunchKernelGGL((scan_wave_kernel<T, PF, HAS_Z, SP, END_ONLY>), grid, dim3(256), 0,
                           a.stream, a.L, a.Dm, (int)ntiles, a.Bt, (const T*)a.u, (const T*)a.delta, a.A,
                           (const T*)a.B, (const T*)a.C, a.D, (const T*)a.z, a.dt_bias, (T*)a.out,
                           a.init_state, a.last_state, sg);
    HX_LAUNCH_CHECK();
    return HX_OK;
}

template <typename T, int PF, bool HAS_Z, bool SP, int VER>
int launch_wave(const ScanArgs& a) {
    int64_t seg_len = a.L;
    const int64_t nseg = a.ws ? scan_segments(a, &seg_len) : 1;
    if (nseg <= 1) return launch_wave_one<T, PF, HAS_Z, SP, false, VER>(a, WaveSeg{a.L, 1, nullptr, nullptr, nullptr});
    const size_t need = scan_seg_bytes(a.Bt, a.Dm, nseg);
    HX_REQUIRE(a.ws_bytes >= need && aligned(a.ws, 16), HX_ERR_INVALID_INPUT,
               "selective scan: workspace of %zu bytes (16-byte aligned) needed, %zu given "
               "(hx_selective_scan_workspace_size)", need, a.ws_bytes);
    const size_t per = (size_t)a.Bt * a.Dm * 16;
    float* hend = (float*)a.ws;
    float* seg_init = hend + (size_t)nseg * per;
    float* decay = seg_init + (size_t)nseg * per;
    int rc = launch_wave_one<T, PF, false, SP, true, VER>(a, WaveSeg{seg_len, (int)nseg, nullptr, hend, decay});
    if (rc != HX_OK) return rc;
    hipLaunchKernelGGL(scan_seg_carry_kernel, dim3((unsigned)((per + 255) / 256)), dim3(256), 0,
                       a.stream, a.Bt, a.Dm, (int)nseg, a.init_state, hend, decay, seg_init);
    HX_LAUNCH_CHECK();
    return launch_wave_one<T, PF, HAS_Z, SP, false, VER>(a, WaveSeg{seg_len, (int)nseg, seg_init, nullptr, nullptr});
}

template <typename T, int PF, int VER = 1>
int dispatch_wave(const ScanArgs& a) {
    const bool hz = a.z != nullptr;
    if (hz && a.softplus) return launch_wave<T, PF, true, true, VER>(a);
    if (hz) return launch_wave<T, PF, true, false, VER>(a);
    if (a.softplus) return launch_wave<T, PF, false, true, VER>(a);
    return launch_wave<T, PF, false, false, VER>(a);
}

// Dynamic LDS of the warp-specialised kernel: its NR-stage ring of u/delta/z chunks, rounded
// up so that with the static LDS (s_x) the block holds more than half a CU's 160 KB and no CU
// runs two of its blocks: one wave per SIMD, the element wave on a SIMD of its own. Granted per
// kernel and device through hipFuncSetAttribute (cached).
constexpr size_t kWsStaticLds = 3 * 4 * 48 * 20 * 4;
// scan_ws2_kernel: 2 element waves x NR stages x operands x 2048-byte slots, then the
// hand-over buffers and the readout buffers; at least 84 KB so that one block runs per CU
size_t ws2_dyn_lds(int NR, bool has_z, size_t es) {
    const size_t need = (size_t)2 * NR * (has_z ? 3 : 2) * (es == 4 ? 2048 : 1024) + kWsStaticLds + 2 * 2 * 3 * 64 * 16;
    return need > 84 * 1024 ? need : 84 * 1024;
}
// scan_ws_kernel: its ring starts right after the static hand-over buffers and, like every LDS
// target of a load to LDS, must end below 64 KiB (46080 + 2 x 3 x 3072 = 64512 at fp32)
size_t ws_dyn_lds(int NR, bool has_z, size_t es, size_t stat) {
    const size_t ring = (size_t)NR * (has_z ? 3 : 2) * 16 * 48 * es;
    const size_t need = 84 * 1024 - stat;
    return ring > need ? ring : need;
}
bool ws_lds_ok(const void* fn, size_t bytes, size_t stat) { return grant_dynamic_lds(fn, bytes, stat); }

template <typename T, int NR, bool HAS_Z, bool SP, bool SPLIT>
int launch_ws(const ScanArgs& a) {
    const int64_t ngrp = (a.Dm + 47) / 48;
    HX_REQUIRE(ngrp * a.Bt <= 0x7fffffff, HX_ERR_UNSUPPORTED,
               "selective scan: %lld blocks exceed the grid", (long long)(ngrp * a.Bt));
    const void* fn = SPLIT ? (const void*)scan_ws2_kernel<T, NR, HAS_Z, SP>
                           : (const void*)scan_ws_kernel<T, NR, HAS_Z, SP>;
    // the split kernel keeps all its LDS in the dynamic allocation (rings, hand-over, readouts)
    const size_t stat = SPLIT ? 0 : kWsStaticLds;
    const size_t dyn = SPLIT ? ws2_dyn_lds(NR, HAS_Z, sizeof(T)) : ws_dyn_lds(NR, HAS_Z, sizeof(T), stat);
    HX_REQUIRE(ws_lds_ok(fn, dyn, stat), HX_ERR_UNSUPPORTED,
               "selective scan: the device does not grant %zu bytes of LDS per block", dyn + stat);
    if constexpr (SPLIT)
        hipLaunchKernelGGL((scan_ws2_kernel<T, NR, HAS_Z, SP>), dim3((unsigned)(ngrp * a.Bt)), dim3(512),
                           dyn, a.stream, a.L, a.Dm, (int)ngrp, (const T*)a.u, (const T*)a.delta, a.A,
                           (const T*)a.B, (const T*)a.C, a.D, (const T*)a.z, a.dt_bias, (T*)a.out,
                           a.init_state, a.last_state);
    else
        hipLaunchKernelGGL((scan_ws_kernel<T, NR, HAS_Z, SP>), dim3((unsigned)(ngrp * a.Bt)), dim3(256),
                           dyn, a.stream, a.L, a.Dm, (int)ngrp, (const T*)a.u, (const T*)a.delta, a.A,
                           (const T*)a.B, (const T*)a.C, a.D, (const T*)a.z, a.dt_bias, (T*)a.out,
                           a.init_state, a.last_state);
    HX_LAUNCH_CHECK();
    return HX_OK;
}

template <typename T, int NR, bool SPLIT = false>
int dispatch_ws(const ScanArgs& a) {
    const bool hz = a.z != nullptr;
    if (hz && a.softplus) return launch_ws<T, NR, true, true, SPLIT>(a);
    if (hz) return launch_ws<T, NR, true, false, SPLIT>(a);
    if (a.softplus) return launch_ws<T, NR, false, true, SPLIT>(a);
    return launch_ws<T, NR, false, false, SPLIT>(a);
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


// Whether the automatic choice takes the warp-specialised kernel over scan_wave3_kernel. Both
// are bound by the state waves' issue rate. wave3 runs one wave per SIMD per 16 channels; the
// warp-specialised kernel one block per CU per 48 channels (3 state waves plus the element
// wave), and its state waves are the faster of the two (measured on MI355X at config 2: 0.89 of
// wave3's time per round) because the element wave takes the per-element work off them. A round
// is one wave per SIMD (wave3) or one block per CU (warp-specialised); a partial round costs a
// full one. The long-sequence shapes that wave3 cuts into time segments stay with wave3.
bool ws_preferred(const ScanArgs& a, size_t es) {
    if ((a.L + 16) * a.Dm * (int64_t)es >= (1LL << 32) || g_scan_segments > 0) return false;
    const int64_t pairs = a.Bt * ((a.Dm + 63) / 64);
    if (pairs < 256 && a.L >= 4096) return false;  // wave3 segments these
    const int64_t cus = device_cus();
    const int64_t ws_rounds = (a.Bt * ((a.Dm + 47) / 48) + cus - 1) / cus;
    const int64_t w3_rounds = (a.Bt * ((a.Dm + 15) / 16) + 4 * cus - 1) / (4 * cus);
    return (double)ws_rounds * 0.89 < (double)w3_rounds;
}

// Whether scan_ws2_kernel takes these sizes: byte offsets of a batch row with the ring's lead in
// 32 bits, and for bf16 whole 8-channel pieces per row (no 16-byte load straddles the row's end).
template <typename T>
bool ws2_ok(const ScanArgs& a) {
    return (a.L + 48) * a.Dm * (int64_t)sizeof(T) < (1LL << 32) && (sizeof(T) == 4 || a.Dm % 8 == 0);
}

// Kernel variant of the calling thread: 0 = auto, -1 = generic, 8 = the fast kernel, 40 =
// scan_wave_kernel, 42 = scan_wave3_kernel, 44 = the warp-specialised kernel, 46 = its
// split-state form (where ws2_ok holds; otherwise the fast kernel) (set by
// hx_set_scan_variant; a measurement knob, per thread so concurrent callers do not see each
// other's setting).
thread_local int g_scan_variant = 0;

template <typename T>
int run_scan(const ScanArgs& a) {
    const size_t es = sizeof(T);
    const bool fast_ok = a.N == 16 && aligned(a.B, 16 * es) && aligned(a.C, 16 * es);
    const int v = g_scan_variant;
    if (!fast_ok || v < 0) return dispatch_generic<T>(a);
    const bool tile_ok = a.Dm % 4 == 0 && aligned(a.u, 16) && aligned(a.delta, 16) &&
                         aligned(a.out, 16) && (!a.z || aligned(a.z, 16)) &&
                         (!a.D || aligned(a.D, 16)) && (!a.dt_bias || aligned(a.dt_bias, 16)) &&
                         a.Bt * ((a.Dm + 63) / 64) <= 0x7fffffff;
    if (v == 0) {  // auto: the wave-complete kernels where their float4 access is legal
        if (tile_ok) {
            if (ws_preferred(a, sizeof(T))) {
                // fp32: the split-state form (two waves per SIMD; config 2 132.5 vs 145.4 us).
                // bf16 keeps the 4-wave form, which measured faster there (154.9 vs 162.1 us).
                if constexpr (std::is_same<T, float>::value)
                    if (ws2_ok<T>(a)) return dispatch_ws<T, 3, true>(a);
                return dispatch_ws<T, 2>(a);
            }
            return a.L * a.Dm < (1LL << 31) ? dispatch_wave<T, 2, 3>(a) : dispatch_wave<T, 2>(a);
        }
        return dispatch_fast<T, 8, 16>(a);
    }
    switch (v) {
        case 40: if (tile_ok) return dispatch_wave<T, 2>(a); break;
        case 42: if (tile_ok && a.L * a.Dm < (1LL << 31)) return dispatch_wave<T, 2, 3>(a); break;
        case 44:
            if (tile_ok && (a.L + 16) * a.Dm * (int64_t)sizeof(T) < (1LL << 32)) return dispatch_ws<T, 2>(a);
            break;
        case 46:
            if (tile_ok && ws2_ok<T>(a)) return dispatch_ws<T, 3, true>(a);
            break;
        default: break;
    }
    return dispatch_fast<T, 8, 16>(a);
}

// Workspace bytes the dispatch of run_scan would use for these sizes (pointers assumed aligned;
// a path that needs none leaves a given workspace unused).
size_t scan_workspace_bytes(const ScanArgs& a, size_t es) {
    const int v = g_scan_variant;
    if (a.N != 16 || a.Dm % 4 != 0 || a.L <= 0 || a.Bt <= 0 || a.Dm <= 0) return 0;
    if (v != 0 && v != 40 && v != 42) return 0;  // generic, fast and warp-specialised: none
    if (v == 0 && ws_preferred(a, es)) return 0;
    int64_t seg_len = 0;
    return scan_seg_bytes(a.Bt, a.Dm, scan_segments(a, &seg_len));
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

namespace hx {
namespace {
int scan_entry(int64_t batch, int64_t seqlen, int64_t dim, int64_t dstate, int dtype,
               int delta_softplus, const void* u, const void* delta, const float* A, const void* B,
               const void* C, const float* D, const void* z, const float* dt_bias, void* out,
               const float* init_state, float* last_state, void* workspace, size_t workspace_bytes,
               void* stream) {
    if (int rc = check_common(batch, seqlen, dim, dstate, dtype)) return rc;
    if (batch == 0 || dim == 0) return HX_OK;
    HX_REQUIRE(A != nullptr, HX_ERR_INVALID_INPUT, "selective scan: A is NULL");
    if (seqlen == 0) {
        // Zero-length sequence: no output rows; the final state is the initial state.
        if (last_state) {
            const size_t bytes = (size_t)batch * dim * dstate * sizeof(float);
            if (init_state)
                HX_HIP_CHECK(hipMemcpyAsync(last_state, init_state, bytes, hipMemcpyDeviceToDevice,
                                            as_stream(stream)));
            else  // a fill kernel, not a memset (this call may be captured into a graph)
                return hx_fill_f32((int64_t)(bytes / sizeof(float)), 0.0f, last_state, stream);
        }
        return HX_OK;
    }
    HX_REQUIRE(u && delta && B && C && out, HX_ERR_INVALID_INPUT,
               "selective scan: u, delta, B, C and out must be non-NULL");
    ScanArgs a{batch, seqlen, dim, dstate, delta_softplus != 0, u, delta, A, B, C, D, z, dt_bias,
               out, init_state, last_state, as_stream(stream), workspace, workspace_bytes};
    return dtype == HX_F32 ? run_scan<float>(a) : run_scan<uint16_t>(a);
}
}  // namespace
}  // namespace hx

namespace hx {
bool scan_variant_is_auto() { return g_scan_variant == 0; }

bool scan_dtproj_ok(int64_t batch, int64_t seqlen, int64_t dim, int64_t rank) {
    return rank >= 32 && rank <= 128 && rank % 32 == 0 && dim % 4 == 0 && seqlen * dim < (1LL << 31) &&
           batch >= 1 && batch <= 65535 && batch * ((dim + 63) / 64) <= 0x7fffffff;
}

int scan_fwd_dtproj(int64_t batch, int64_t seqlen, int64_t dim, const uint16_t* u, const uint16_t* dtlo,
                    int64_t rank, const uint16_t* w_dt, const float* A, const uint16_t* B,
                    const uint16_t* C, const float* D, const uint16_t* z, const float* dt_bias,
                    uint16_t* out, float* last_state, hipStream_t stream) {
    HX_REQUIRE(scan_dtproj_ok(batch, seqlen, dim, rank), HX_ERR_UNSUPPORTED,
               "selective scan with dt_proj: sizes outside the fused path (batch %lld, seqlen %lld, "
               "dim %lld, dt_rank %lld)", (long long)batch, (long long)seqlen, (long long)dim, (long long)rank);
    if (seqlen == 0)  // no steps (the empty operands may be NULL): the final state is the zero initial state
        return last_state ? hx_fill_f32(batch * dim * 16, 0.0f, last_state, stream) : (int)HX_OK;
    HX_REQUIRE(u && dtlo && w_dt && A && B && C && z && out, HX_ERR_INVALID_INPUT,
               "selective scan with dt_proj: a required pointer is NULL");
    HX_REQUIRE(aligned(u, 16) && aligned(z, 16) && aligned(out, 16) && aligned(dtlo, 16) && aligned(w_dt, 16) &&
                   aligned(B, 32) && aligned(C, 32) && (!D || aligned(D, 16)) && (!dt_bias || aligned(dt_bias, 16)),
               HX_ERR_UNSUPPORTED, "selective scan with dt_proj: operands not 16-byte aligned");
    constexpr int WPB = 4;
    const int64_t ntiles = (dim + 16 * WPB - 1) / (16 * WPB);
    WaveSeg sg{seqlen, 1, nullptr, nullptr, nullptr};
    sg.dtlo = dtlo;
    sg.wdt = w_dt;
    sg.rank = (int)rank;
    auto go = [&](auto kern) {
        hipLaunchKernelGGL(kern, dim3((unsigned)(ntiles * batch)), dim3(64 * WPB), 0, stream, seqlen, dim,
                           (int)ntiles, batch, u, (const uint16_t*)nullptr, A, B, C, D, z, dt_bias, out,
                           (const float*)nullptr, last_state, sg);
        HX_LAUNCH_CHECK();
        return (int)HX_OK;
    };
    switch (rank / 32) {
        case 1: return go(scan_wave3_kernel<uint16_t, 2, true, true, false, WPB, 1>);
        case 2: return go(scan_wave3_kernel<uint16_t, 2, true, true, false, WPB, 2>);
        case 3: return go(scan_wave3_kernel<uint16_t, 2, true, true, false, WPB, 3>);
        default: return go(scan_wave3_kernel<uint16_t, 2, true, true, false, WPB, 4>);
    }
}
}  // namespace hx

extern "C" int hx_selective_scan_dtproj_fwd(int64_t batch, int64_t seqlen, int64_t dim, int64_t dt_rank,
                                            const void* u, const void* dt_lo, const void* w_dt,
                                            const float* A, const void* B, const void* C, const float* D,
                                            const void* z, const float* dt_bias, void* out,
                                            float* last_state, void* stream) {
    using namespace hx;
    HX_REQUIRE(batch >= 0 && seqlen >= 0 && dim >= 0 && dt_rank >= 0, HX_ERR_INVALID_DIMENSION,
               "selective scan with dt_proj: negative size");
    if (batch == 0 || dim == 0) return HX_OK;
    return scan_fwd_dtproj(batch, seqlen, dim, (const uint16_t*)u, (const uint16_t*)dt_lo, dt_rank,
                           (const uint16_t*)w_dt, A, (const uint16_t*)B, (const uint16_t*)C, D,
                           (const uint16_t*)z, dt_bias, (uint16_t*)out, last_state, as_stream(stream));
}

extern "C" int hx_selective_scan_fwd(int64_t batch, int64_t seqlen, int64_t dim, int64_t dstate,
                                     int dtype, int delta_softplus, const void* u,
                                     const void* delta, const float* A, const void* B,
                                     const void* C, const float* D, const void* z,
                                     const float* dt_bias, void* out, const float* init_state,
                                     float* last_state, void* stream) {
    return hx::scan_entry(batch, seqlen, dim, dstate, dtype, delta_softplus, u, delta, A, B, C, D,
                          z, dt_bias, out, init_state, last_state, nullptr, 0, stream);
}

extern "C" size_t hx_selective_scan_workspace_size(int64_t batch, int64_t seqlen, int64_t dim,
                                                   int64_t dstate, int dtype) {
    if (dtype != HX_F32 && dtype != HX_BF16) return 0;
    hx::ScanArgs a{batch, seqlen, dim, dstate, 1, nullptr, nullptr, nullptr, nullptr, nullptr,
                   nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr};
    return hx::scan_workspace_bytes(a, dtype == HX_F32 ? 4 : 2);
}

extern "C" int hx_selective_scan_fwd_ws(int64_t batch, int64_t seqlen, int64_t dim, int64_t dstate,
                                        int dtype, int delta_softplus, const void* u,
                                        const void* delta, const float* A, const void* B,
                                        const void* C, const float* D, const void* z,
                                        const float* dt_bias, void* out, const float* init_state,
                                        float* last_state, void* workspace, size_t workspace_bytes,
                                        void* stream) {
    HX_REQUIRE(workspace != nullptr || workspace_bytes == 0, HX_ERR_INVALID_INPUT,
               "selective scan: NULL workspace with %zu bytes", workspace_bytes);
    return hx::scan_entry(batch, seqlen, dim, dstate, dtype, delta_softplus, u, delta, A, B, C, D,
                          z, dt_bias, out, init_state, last_state,
                          workspace_bytes ? workspace : nullptr, workspace_bytes, stream);
}

// ------------------------------------------------------------------ no-allocation entry point
// Scratch of hx_selective_scan_fwd_noalloc: the segmented long-sequence path's end states, entry
// states and segment decays (the same layout a caller workspace holds for
// hx_selective_scan_fwd_ws). One copy per device, resident until the process ends. Nothing in it
// has to start at zero: the end-state pass writes every end state and decay the carry kernel
// reads, and the carry kernel writes every entry state the output pass reads.
constexpr size_t kScanScratchBytes = (size_t)8 << 20;
static __device__ __align__(256) unsigned char scratch[kScanScratchBytes];

namespace hx {
namespace {
std::mutex g_scratch_mu;
void* g_scratch_dev[64] = {};  // device address of `scratch`, per device
}  // namespace

// Looks up the current device's address of `scratch` once per device (hipGetSymbolAddress with
// that device current). Host code passes this address, never the array's name, to kernels.
int scan_scratch_setup(void** out) {
    int dev = 0;
    HX_HIP_CHECK(hipGetDevice(&dev));
    HX_REQUIRE(dev >= 0 && dev < 64, HX_ERR_UNSUPPORTED, "scan scratch: device %d >= 64", dev);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_dev[dev] == nullptr) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        HX_REQUIRE(e == hipSuccess && p != nullptr, HX_ERR_BACKEND,
                   "scan scratch: hipGetSymbolAddress failed on device %d: %s", dev,
                   hipGetErrorString(e));
        g_scratch_dev[dev] = p;
    }
    if (out) *out = g_scratch_dev[dev];
    return HX_OK;
}
}  // namespace hx

extern "C" int hx_selective_scan_fwd_noalloc(int64_t batch, int64_t seqlen, int64_t dim,
                                             int64_t dstate, int dtype, int delta_softplus,
                                             const void* u, const void* delta, const float* A,
                                             const void* B, const void* C, const float* D,
                                             const void* z, const float* dt_bias, void* out,
                                             const float* init_state, float* last_state,
                                             void* stream) {
    if (int rc = hx::check_common(batch, seqlen, dim, dstate, dtype)) return rc;
    const size_t need = hx_selective_scan_workspace_size(batch, seqlen, dim, dstate, dtype);
    HX_REQUIRE(need <= kScanScratchBytes, HX_ERR_UNSUPPORTED,
               "selective scan (no-alloc): %zu bytes of scratch needed, the device scratch holds "
               "%zu (use hx_selective_scan_fwd_ws with a caller workspace)",
               need, kScanScratchBytes);
    void* ws = nullptr;
    if (need > 0)
        if (int rc = hx::scan_scratch_setup(&ws)) return rc;
    return hx::scan_entry(batch, seqlen, dim, dstate, dtype, delta_softplus, u, delta, A, B, C, D,
                          z, dt_bias, out, init_state, last_state, ws,
                          need > 0 ? kScanScratchBytes : 0, stream);
}

extern "C" int hx_set_scan_variant(int variant) {
    HX_REQUIRE(variant == 0 || variant == -1 || variant == 8 || variant == 40 || variant == 42 ||
                   variant == 44 || variant == 46,
               HX_ERR_INVALID_INPUT, "hx_set_scan_variant: %d is not one of 0, -1, 8, 40, 42, 44, 46",
               variant);
    hx::g_scan_variant = variant;
    return HX_OK;
}

extern "C" int hx_set_scan_segments(int nseg) {
    HX_REQUIRE(nseg >= 0 && nseg <= 4096, HX_ERR_INVALID_INPUT,
               "hx_set_scan_segments: %d outside 0..4096", nseg);
    hx::g_scan_segments = nseg;
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
    const size_t bc_align = dtype == HX_F32 ? 16 : 8;  // one 4-element group of B / C
    if (dstate == 16 && hx::aligned(state, 16) && hx::aligned(A, 16) && hx::aligned(B, bc_align) &&
        hx::aligned(C, bc_align)) {
        if (dtype == HX_F32)
            hipLaunchKernelGGL(hx::state_update16_kernel<float>, grid, dim3(128), 0, s, batch, dim,
                               delta_softplus, state, (const float*)u, (const float*)delta, A,
                               (const float*)B, (const float*)C, D, (const float*)z, dt_bias,
                               (float*)out);
        else
            hipLaunchKernelGGL(hx::state_update16_kernel<uint16_t>, grid, dim3(128), 0, s, batch, dim,
                               delta_softplus, state, (const uint16_t*)u, (const uint16_t*)delta, A,
                               (const uint16_t*)B, (const uint16_t*)C, D, (const uint16_t*)z, dt_bias,
                               (uint16_t*)out);
        HX_LAUNCH_CHECK();
        return HX_OK;
    }
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

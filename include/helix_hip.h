/*
 * helix_hip.h — C ABI of libhelix_hip.so, the MI355X (gfx950) backend for HelixML's
 * state-space-model forward path.
 *
 * This is the drop-in boundary a Rust `crates/backend-hip` binds with an `extern "C"` block.
 * Every entry point takes plain pointers, sizes and
 * enums: no HIP, torch or C++ types cross it. Inputs and outputs are allocated by the caller
 * (hx_malloc, or any HIP allocation on the same device). No compute entry point allocates:
 * scratch memory is a caller-owned workspace whose size the matching *_workspace_size function
 * returns (the block and layer forwards, the long-sequence scan, the S4 paths).
 * A `stream` argument is a hipStream_t passed as void*
 * (NULL = the legacy default stream). All compute entry points are stream-ordered and
 * asynchronous; they validate shapes on the host before any launch and return a status code.
 * No C++ exception or panic crosses this boundary.
 *
 * Layout conventions (row-major, contiguous, the reference's [tokens, channels] order,
 * crates/nn/src/lib.rs:121-123 and :889):
 *   u, delta, z, out : [batch, seqlen, dim]      (channels contiguous)
 *   B, C (selective) : [batch, seqlen, dstate]
 *   A                : [dim, dstate]  fp32
 *   D, dt_bias       : [dim]          fp32
 *   state            : [batch, dim, dstate] fp32
 */
#ifndef HELIX_HIP_H
#define HELIX_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes. One per tensor_core::TensorError variant
 * (reference crates/tensor-core/src/error.rs:7-37), so the Rust side maps them 1:1. */
typedef enum {
    HX_OK = 0,
    HX_ERR_SHAPE_MISMATCH = 1,     /* TensorError::ShapeMismatch      (error.rs:9)  */
    HX_ERR_INVALID_DIMENSION = 2,  /* TensorError::InvalidDimension   (error.rs:12) */
    HX_ERR_DEVICE_MISMATCH = 3,    /* TensorError::DeviceMismatch     (error.rs:15) */
    HX_ERR_DTYPE_MISMATCH = 4,     /* TensorError::DTypeMismatch      (error.rs:18) */
    HX_ERR_UNSUPPORTED = 5,        /* TensorError::UnsupportedOperation (error.rs:21) */
    HX_ERR_ALLOCATION = 6,         /* TensorError::AllocationFailed   (error.rs:24) */
    HX_ERR_BACKEND = 7,            /* TensorError::BackendError       (error.rs:27) */
    HX_ERR_SERIALIZATION = 8,      /* TensorError::SerializationError (error.rs:30) */
    HX_ERR_INVALID_INPUT = 9,      /* TensorError::InvalidInput       (error.rs:36) */
    HX_ERR_INVALID_CHECKPOINT = 10 /* TensorError::InvalidCheckpoint  (error.rs:33) */
} hx_status;

/* Storage dtypes. Arithmetic and recurrent state are always fp32.
 * (tensor_core::DType has no BF16, crates/tensor-core/src/dtype.rs:8-37; HX_BF16 is the
 * storage format the north-star config 3 asks for.) */
typedef enum { HX_F32 = 0, HX_BF16 = 1 } hx_dtype;

/* ------------------------------------------------------------------ runtime */
/* Library version, (major << 16) | (minor << 8) | patch. */
int hx_version(void);
/* Selects and initialises `device`. Replaces nothing in the reference (its Device enum has no
 * ROCm variant, tensor-core/src/device.rs:8-25); the Rust side calls it from HipTensor's ctor. */
int hx_init(int device);
/* Device allocation / free / copies; back HipTensor storage (the reference's
 * Tensor::to_device, tensor-core/src/tensor.rs:54, and CpuTensor's owned ndarray). */
int hx_malloc(void** ptr, size_t bytes);
int hx_free(void* ptr);
int hx_memcpy_h2d(void* dst, const void* src, size_t bytes);
int hx_memcpy_d2h(void* dst, const void* src, size_t bytes);
int hx_memcpy_d2d(void* dst, const void* src, size_t bytes, void* stream);
/* Waits for all work on the device. */
int hx_sync(void);
/* Compute units and global memory bytes of `device` (for hal::ComputeBackend::compute_units and
 * capabilities, hal/src/backend.rs:31-35). */
int hx_device_info(int device, int* compute_units, size_t* memory_bytes);
/* Fraction of time `device` was busy over the driver's last sampling window (amdgpu's
 * gpu_busy_percent in sysfs, 0..1), for hal::ComputeBackend::utilization (hal/src/backend.rs:
 * 65-66). HX_ERR_UNSUPPORTED where the driver does not expose it. */
int hx_device_utilization(int device, double* busy_fraction);
/* Text of the last error raised on the calling thread ("" if none). Becomes the message of
 * TensorError::BackendError / the variant matching the status. */
const char* hx_last_error(void);

/* ------------------------------------------------------------------ fused selective scan */
/* Fused Mamba selective-scan forward, one pass over HBM.
 * Replaces the composite the reference spells as nn::ssm::MambaBlock::selective_ssm
 * (crates/nn/src/ssm.rs:474-483, which delegates to S4Block::forward_ssm, ssm.rs:138-186) with
 * the selective semantics the reference's own discretisation implies (Abar = exp(dt*A),
 * ssm.rs:108-116; Bbar = dt*B, ssm.rs:127-130) and SiLU gating (backend-cpu/src/lib.rs:1158-1162):
 *   dt    = softplus(delta + dt_bias)        (softplus only if delta_softplus != 0)
 *   h[n]  = exp(dt*A[d,n]) * h[n] + dt*u*B[b,t,n]
 *   y     = sum_n C[b,t,n]*h[n] + D[d]*u
 *   out   = y * silu(z)                       (if z != NULL)
 * dtype selects the storage type of u, delta, z, B, C and out; A, D, dt_bias, state are fp32.
 * init_state (nullable) seeds h; last_state (nullable) receives h after the last step.
 * Uses no scratch memory: a sequence is never cut into time segments here (see _ws below). */
int hx_selective_scan_fwd(int64_t batch, int64_t seqlen, int64_t dim, int64_t dstate,
                          int dtype, int delta_softplus,
                          const void* u, const void* delta, const float* A,
                          const void* B, const void* C, const float* D,
                          const void* z, const float* dt_bias,
                          void* out, const float* init_state, float* last_state,
                          void* stream);

/* hx_selective_scan_fwd with a caller workspace for the long-sequence path: when the
 * (batch, channel) tiles alone cannot fill the GPU (few channels, long seqlen), the sequence is
 * cut into time segments whose end states (from a zero state) are accumulated backwards from
 * each segment's end until every state's decay to the end is below 2^-48, their entry states
 * chained by a carry kernel, then rescanned with outputs (results agree with the unsegmented
 * scan to fp32 rounding). workspace: device memory of at least hx_selective_scan_workspace_size(...) bytes,
 * 16-byte aligned (0 bytes: no segments); it holds no state between calls. Same reference
 * counterpart as hx_selective_scan_fwd (the per-step loop of ssm.rs:166-182). */
size_t hx_selective_scan_workspace_size(int64_t batch, int64_t seqlen, int64_t dim,
                                        int64_t dstate, int dtype);
int hx_selective_scan_fwd_ws(int64_t batch, int64_t seqlen, int64_t dim, int64_t dstate,
                             int dtype, int delta_softplus,
                             const void* u, const void* delta, const float* A,
                             const void* B, const void* C, const float* D,
                             const void* z, const float* dt_bias,
                             void* out, const float* init_state, float* last_state,
                             void* workspace, size_t workspace_bytes, void* stream);

/* hx_selective_scan_fwd_ws without the workspace argument, for callers that cannot allocate
 * (code under HIP graph capture, serving loops, harnesses that forbid hipMalloc): the segmented
 * long-sequence path uses an 8 MiB device-resident scratch array of the library instead (one per
 * device, held until the process ends; hx_init or the first call on a device resolves its
 * address). Calls nothing that allocates. Shapes whose segmented path needs more than 8 MiB
 * (hx_selective_scan_workspace_size > 8 MiB, e.g. with hx_set_scan_segments forcing thousands of
 * segments) are rejected with HX_ERR_UNSUPPORTED. Every call on a device shares that scratch:
 * calls that overlap on one device (concurrent streams or threads) race; stream-ordered calls on
 * one stream do not. No counterpart in the reference (which has no device path): it exists for
 * callers that cannot allocate. Results are identical to hx_selective_scan_fwd_ws's. */
int hx_selective_scan_fwd_noalloc(int64_t batch, int64_t seqlen, int64_t dim, int64_t dstate,
                                  int dtype, int delta_softplus,
                                  const void* u, const void* delta, const float* A,
                                  const void* B, const void* C, const float* D,
                                  const void* z, const float* dt_bias,
                                  void* out, const float* init_state, float* last_state,
                                  void* stream);

/* Single-step recurrent decode (state update only), for token-by-token generation:
 * the same arithmetic as one time step of hx_selective_scan_fwd with seqlen 1, updating
 * `state` [batch, dim, dstate] in place. u, delta, z, out: [batch, dim]; B, C: [batch, dstate].
 * No reference counterpart beyond the per-step body of ssm.rs:166-182. */
int hx_selective_state_update(int64_t batch, int64_t dim, int64_t dstate,
                              int dtype, int delta_softplus,
                              float* state, const void* u, const void* delta, const float* A,
                              const void* B, const void* C, const float* D,
                              const void* z, const float* dt_bias, void* out,
                              void* stream);

/* ------------------------------------------------------------------ S4 recurrences */
/* nn::ssm::S4Block::discretize(dt)'s real decay (crates/nn/src/ssm.rs:113-120) on HOST arrays:
 * a[n] = expf(a_real[n]*dt) * cosf(a_imag[n]*dt), each product rounded to f32 first, with the
 * libm the reference's f32::exp / f32::cos call, so the result is the reference's bit for bit.
 * The caller uploads `a` (dstate floats) for hx_s4_ref_fwd / hx_s4_ref_fwd_parallel: the
 * discretisation needs no device round trip per forward. dstate <= 64. */
int hx_s4_discretize(int64_t dstate, float dt, const float* a_real, const float* a_imag, float* a);

/* Reference-faithful nn::ssm::S4Block::forward_ssm (crates/nn/src/ssm.rs:138-186) given the
 * discretised decay a (device, [dstate], from hx_s4_discretize) and Bd = dt*B (ssm.rs:127-130),
 * one state h[dstate] SHARED by all channels:
 *   h = a (.) h + Bd . x[:, t];   y[t][m] = (C . h)[m] + D[m] * x[m][t]
 * x: [d_model, seqlen] row-major (column t is u_t, ssm.rs:168-169).
 * y: memory [seqlen, d_model] (CpuTensor::stack(..., 1) of per-step vectors writes rows in time
 *    order, backend-cpu/src/lib.rs:277-296; the shape field it reports is [d_model, seqlen]).
 * gate (nullable) [d_model]: y[t][m] *= gate[m] — fuses nn::ssm::MambaBlock's gating
 *    (ssm.rs:460-461, broadcast_to repeat-rows, backend-cpu/src/lib.rs:1388-1404).
 * B: [dstate, d_model], C: [d_model, dstate], D: [d_model]. dstate <= 64.
 * workspace: at least hx_s4_ref_workspace_size(...) bytes of device memory, 256-byte aligned.
 * Asynchronous on `stream` (no host round trip). */
size_t hx_s4_ref_workspace_size(int64_t d_model, int64_t dstate, int64_t seqlen);
int hx_s4_ref_fwd(int64_t d_model, int64_t dstate, int64_t seqlen, float dt,
                  const float* x, const float* a, const float* B, const float* C, const float* D,
                  const float* gate, float* y, void* workspace, size_t workspace_bytes,
                  void* stream);

/* Time-parallel variant of hx_s4_ref_fwd for long sequences (same arguments and layouts,
 * dstate <= 16): the 16 state recurrences are solved in 256-step chunks with a carry chain (the
 * chunk decay a^256 formed from the same rounded a) and products may contract to FMA, so results
 * agree with reference mode to rounding (within 1e-4) instead of bit for bit. workspace: at
 * least hx_s4_ref_parallel_workspace_size(...) bytes, 256-byte aligned. Replaces the per-step
 * loop of S4Block::forward_ssm (crates/nn/src/ssm.rs:166-182) for L in the tens of thousands. */
size_t hx_s4_ref_parallel_workspace_size(int64_t d_model, int64_t dstate, int64_t seqlen);
int hx_s4_ref_fwd_parallel(int64_t d_model, int64_t dstate, int64_t seqlen, float dt,
                           const float* x, const float* a, const float* B, const float* C,
                           const float* D, const float* gate, float* y, void* workspace,
                           size_t workspace_bytes, void* stream);

/* S4D diagonal complex recurrence (per-channel state, S4D discretisation with the same
 * ZOH-on-A / Euler-on-B choice as ssm.rs:108-130), the complex form of what
 * S4Block::discretize computes and then drops (A_d_imag, ssm.rs:121-125):
 *   Abar[d,n] = exp(dt[d]*(a_re[d,n] + i*a_im[d,n])), Bbar = dt[d]*B[d,n] (complex)
 *   h[d,n] = Abar*h + Bbar*x[b,t,d];  y[b,t,d] = 2*Re(sum_n C[d,n]*h[d,n]) + D[d]*x[b,t,d]
 * x, y: [batch, seqlen, dim] fp32. a_re, a_im, B_re, B_im, C_re, C_im: [dim, dstate]; dt, D: [dim].
 * workspace: at least hx_s4d_workspace_size(...) bytes (segment states of the long-sequence
 * path; 0 when the sequence is not segmented), 16-byte aligned. */
size_t hx_s4d_workspace_size(int64_t batch, int64_t seqlen, int64_t dim, int64_t dstate);
int hx_s4d_complex_fwd(int64_t batch, int64_t seqlen, int64_t dim, int64_t dstate,
                       const float* x, const float* dt,
                       const float* a_re, const float* a_im,
                       const float* B_re, const float* B_im,
                       const float* C_re, const float* C_im,
                       const float* D, float* y, void* workspace, size_t workspace_bytes,
                       void* stream);

/* ------------------------------------------------------------------ dense */
/* nn::Linear::forward (crates/nn/src/lib.rs:120-134): Y[r][o] = sum_k X[r][k]*W[o][k] + bias[o],
 * W in the reference's [out_features, in_features] layout; bias nullable.
 * act: 0 = none, 1 = SiLU fused on the output (nn::MambaBlock::forward_mamba's
 * Linear -> silu, lib.rs:894-900). fp32 storage and accumulate. */
int hx_linear_f32(int64_t rows, int64_t in_features, int64_t out_features,
                  const float* X, const float* W, const float* bias, int act,
                  float* Y, void* stream);

/* bf16 matrix-core GEMM for the Mamba block's projections: Y = X . W^T (+ bias)(, SiLU), the
 * nn::Linear layout (crates/nn/src/lib.rs:120-134, weight [out, in]). X [M, K] (row stride ldx),
 * W [N, K] (row stride ldw), bf16 (16-byte aligned rows take the fast 16-byte-load path, any
 * other stride an element-load path); fp32 accumulate; out_dtype HX_F32 or
 * HX_BF16. Columns [0, split1) go to Y0 (row stride ld0), [split1, split2) to Y1, [split2, N) to
 * Y2 (split1 = split2 = N for a single output). act: bit 0 applies SiLU, bit 1 accumulates
 * (Y = Y + result, after the SiLU if both are set): the residual add of a pre-norm layer. */
int hx_gemm_bf16(int64_t M, int64_t N, int64_t K, const void* X, int64_t ldx,
                 const void* W, int64_t ldw, const float* bias, int act, int out_dtype,
                 void* Y0, int64_t ld0, int64_t split1, void* Y1, int64_t ld1,
                 int64_t split2, void* Y2, int64_t ld2, void* stream);
/* hx_gemm_bf16 with K split into `splits` (1..16) slices of whole 64-wide K tiles, for products
 * with a narrow N and a long K that leave the GPU mostly idle (the block's x_proj: N 160, K 4096):
 * each slice's fp32 partial goes to `workspace` (at least splits * M * N * 4 bytes, 16-byte
 * aligned, caller-owned), then one pass sums the partials in slice order and applies the same
 * epilogue and outputs as hx_gemm_bf16. Requires K % (64 * splits) == 0 and 16-byte aligned rows
 * (HX_ERR_UNSUPPORTED otherwise). Same Linear layout (crates/nn/src/lib.rs:120-134); the summation
 * order differs from hx_gemm_bf16's only in where the slices' fp32 sums are added. */
int hx_gemm_bf16_splitk(int64_t M, int64_t N, int64_t K, const void* X, int64_t ldx,
                        const void* W, int64_t ldw, const float* bias, int act, int out_dtype,
                        void* Y0, int64_t ld0, int64_t split1, void* Y1, int64_t ld1,
                        int64_t split2, void* Y2, int64_t ld2, int splits, void* workspace,
                        size_t workspace_bytes, void* stream);

/* Causal depthwise conv1d over time + bias + SiLU (the Mamba block's conv, kernel `width` <= 4):
 * y[b,t,d] = silu(bias[d] + sum_j weight[d,j] * x[b, t-width+1+j, d]) with zero padding.
 * x: [batch, seqlen, dim] with row stride ldx (so it can be the x half of in_proj's output);
 * y contiguous; dtype HX_F32 or HX_BF16 storage; weight [dim, width], bias [dim] fp32. */
int hx_conv1d_silu(int64_t batch, int64_t seqlen, int64_t dim, int64_t width, int dtype,
                   const void* x, int64_t ldx, const float* weight, const float* bias, void* y,
                   void* stream);

/* The Mamba block's dt projection and selective scan in one launch (the steps
 * dt = dt_lo . w_dt^T; y = selective_scan(u, dt, ...) of hx_mamba_block_fwd below): bf16 storage,
 * dstate 16, softplus(dt + dt_bias), SiLU(z) gate, zero initial state. Each 16-step chunk's
 * [16 steps x 16 channels] dt tile is formed on the matrix core from dt_lo [batch, seqlen, dt_rank]
 * and w_dt [dim, dt_rank] (bf16, 16-byte aligned rows), rounded to bf16 as a stored dt would be,
 * so no dt tensor is written or read. The other operands as hx_selective_scan_fwd's with
 * dtype HX_BF16 (z required). dt_rank 32, 64, 96 or 128, seqlen * dim < 2^31, dim % 4 == 0;
 * HX_ERR_UNSUPPORTED otherwise. No counterpart in the reference (its block never projects dt);
 * a fusion of two of the block's steps. */
int hx_selective_scan_dtproj_fwd(int64_t batch, int64_t seqlen, int64_t dim, int64_t dt_rank,
                                 const void* u, const void* dt_lo, const void* w_dt, const float* A,
                                 const void* B, const void* C, const float* D, const void* z,
                                 const float* dt_bias, void* out, float* last_state, void* stream);

/* Full Mamba block forward, bf16 storage / fp32 arithmetic:
 *   x|z = x . w_in^T; xc = SiLU(conv1d(x)); dt_lo|B|C = xc . w_x^T; dt = dt_lo . w_dt^T;
 *   y = selective_scan(xc, dt, A, B, C, D, z, dt_bias, softplus); out = y . w_out^T.
 * The block the reference's exported MambaBlock allocates parameters for
 * (crates/nn/src/lib.rs:846-885) but whose forward is only Linear -> SiLU -> Linear (lib.rs:888-906).
 * x, out [batch, seqlen, d_model] bf16; w_in [2*d_inner, d_model], w_x [dt_rank + 2*dstate,
 * d_inner], w_dt [d_inner, dt_rank], w_out [d_model, d_inner] bf16; conv_w [d_inner, d_conv],
 * conv_b, dt_bias, D [d_inner], A [d_inner, dstate] fp32. dstate 16, d_inner % 4 == 0, d_conv
 * 1..4. workspace: device memory of at least
 * hx_mamba_block_workspace_size(...) bytes, owned by the caller. */
size_t hx_mamba_block_workspace_size(int64_t batch, int64_t seqlen, int64_t d_inner,
                                     int64_t dt_rank, int64_t dstate);
int hx_mamba_block_fwd(int64_t batch, int64_t seqlen, int64_t d_model, int64_t d_inner,
                       int64_t dstate, int64_t dt_rank, int64_t d_conv,
                       const void* x, const void* w_in, const float* conv_w, const float* conv_b,
                       const void* w_x, const void* w_dt, const float* dt_bias, const float* A,
                       const float* D, const void* w_out, void* out, void* workspace,
                       size_t workspace_bytes, void* stream);

/* ---- byte-level SSM LM: 12 x (RMSNorm + Mamba) with embedding and head ---- */

/* Token embedding gather: out[t][:] = table[tokens[t]][:]; tokens outside [0, vocab) give a zero
 * row. table [vocab, dim] fp32, out [n_tokens, dim] fp32. (The reference has no Embedding layer;
 * its byte LM feeds random inputs, examples/ssm_byte_lm/src/main.rs:121-129.) */
int hx_embedding_fwd(int64_t n_tokens, int64_t vocab, int64_t dim, const int32_t* tokens,
                     const float* table, float* out, void* stream);

/* nn::RMSNorm::forward (crates/nn/src/lib.rs:258-285) over rows of x [rows, dim] fp32:
 * y = x / sqrt(mean(x^2) + eps) * weight, y fp32 or bf16 (out_dtype). The reference draws the
 * epsilon per row from U[eps, eps + 1e-8) (lib.rs:262); this uses eps itself. */
int hx_rmsnorm_fwd(int64_t rows, int64_t dim, const float* x, const float* weight, float eps,
                   int out_dtype, void* y, void* stream);

/* One recurrent step of the causal conv: y[b][d] = silu(bias[d] + sum_{j<w-1} weight[d][j] *
 * state[b][j][d] + weight[d][w-1] * x[b][d]), then state shifts in x. state [batch][w-1][dim]
 * fp32 (in/out); x rows of stride ldx; y [batch][dim]; dtype of x and y HX_F32 / HX_BF16. */
int hx_conv1d_step(int64_t batch, int64_t dim, int64_t width, int dtype, const void* x,
                   int64_t ldx, const float* weight, const float* bias, float* state, void* y,
                   void* stream);

/* One pre-norm LM layer over a prefill: resid [batch, seqlen, d_model] fp32 (in/out) +=
 * MambaBlock(RMSNorm(resid)), with the block of hx_mamba_block_fwd. Optional outputs for the
 * decode hand-off: ssm_state [batch, d_inner, dstate] (the scan's state after the last step) and
 * conv_state [batch, d_conv-1, d_inner] (the last d_conv-1 conv inputs). workspace: at least
 * hx_mamba_layer_workspace_size(batch, seqlen, ...) bytes of device memory. */
size_t hx_mamba_layer_workspace_size(int64_t batch, int64_t seqlen, int64_t d_model,
                                     int64_t d_inner, int64_t dt_rank, int64_t dstate);
int hx_mamba_layer_fwd(int64_t batch, int64_t seqlen, int64_t d_model, int64_t d_inner,
                       int64_t dstate, int64_t dt_rank, int64_t d_conv, float* resid,
                       const float* norm_w, float eps, const void* w_in, const float* conv_w,
                       const float* conv_b, const void* w_x, const void* w_dt,
                       const float* dt_bias, const float* A, const float* D, const void* w_out,
                       float* ssm_state, float* conv_state, void* workspace,
                       size_t workspace_bytes, void* stream);

/* One recurrent decode step of the same layer for one token per sequence: resid [batch,
 * d_model] fp32 (in/out); ssm_state and conv_state (layouts as above) are read and advanced.
 * workspace: hx_mamba_layer_workspace_size(batch, 1, ...) bytes. */
int hx_mamba_layer_decode(int64_t batch, int64_t d_model, int64_t d_inner, int64_t dstate,
                          int64_t dt_rank, int64_t d_conv, float* resid, const float* norm_w,
                          float eps, const void* w_in, const float* conv_w, const float* conv_b,
                          const void* w_x, const void* w_dt, const float* dt_bias,
                          const float* A, const float* D, const void* w_out, float* ssm_state,
                          float* conv_state, void* workspace, size_t workspace_bytes,
                          void* stream);

/* CpuTensor::matmul 2-D x 2-D (crates/backend-cpu/src/lib.rs:644-678): Y = A[M,K] . B[K,N]. */
int hx_matmul_f32(int64_t M, int64_t K, int64_t N, const float* A, const float* B, float* Y,
                  void* stream);

/* ------------------------------------------------------------------ tensor primitives */
/* The CpuTensor operations a HipTensor needs to implement the reference's traits on the device
 * (crates/tensor-core/src/tensor.rs:7-209), fp32, row-major. Shape checks and the reference's
 * error variants are the caller's (the HipTensor layer): only element counts cross here. */

/* Equal-shape elementwise y = a op b over n elements: CpuTensor::add/sub/mul/div
 * (crates/backend-cpu/src/lib.rs:570-632). One IEEE operation per element (bit-exact). */
typedef enum { HX_ADD = 0, HX_SUB = 1, HX_MUL = 2, HX_DIV = 3 } hx_binary_op;
int hx_binary_f32(int op, int64_t n, const float* a, const float* b, float* y, void* stream);

/* Elementwise y = f(x[, scalar]) over n elements (crates/backend-cpu/src/lib.rs):
 * HX_EXP exp (777-784), HX_COS cos (803-809), HX_SIN sin (795-801), HX_SQRT sqrt (768-775,
 * correctly rounded), HX_SILU x / (1 + exp(-x)) (1154-1170), HX_NEG -x (895-902), HX_MUL_SCALAR
 * x * scalar (925-932), HX_ADD_SCALAR x + scalar (916-922), HX_ABS |x| (822-828), HX_LOG ln x
 * (786-793), HX_SIGMOID 1 / (1 + exp(-x)) (1172-1178). exp/cos/sin/log use the device math
 * library where the reference calls host libm (results within a few ulp). */
typedef enum {
    HX_EXP = 0, HX_COS = 1, HX_SIN = 2, HX_SQRT = 3, HX_SILU = 4, HX_NEG = 5, HX_MUL_SCALAR = 6,
    HX_ADD_SCALAR = 7, HX_ABS = 8, HX_LOG = 9, HX_SIGMOID = 10
} hx_unary_op;
int hx_unary_f32(int op, int64_t n, const float* x, float scalar, float* y, void* stream);

/* Mean over the middle axis of x viewed as [outer, len, inner]: y[o][i] = sum_l x[o][l][i] / len
 * (TensorReduce::mean of one axis, crates/backend-cpu/src/lib.rs:995-1010, i.e. ndarray 0.15's
 * mean_axis = sum_axis / len), bit-exact with ndarray's summation order: lane_fold = 1 (the
 * reduced axis is the array's last, minimum-stride axis; requires inner == 1) sums each lane with
 * eight partial sums over elements k mod 8 combined as ((p0+p4) + (p1+p5) + (p2+p6) + (p3+p7)) and
 * then the len mod 8 trailing elements; lane_fold = 0 adds the len sub-views in axis order.
 * len == 0 is rejected (the reference unwraps ndarray's None there). */
int hx_mean_axis_f32(int64_t outer, int64_t len, int64_t inner, int lane_fold, const float* x,
                     float* y, void* stream);

/* Exact strided copy of a logical block of `shape` (ndim <= HX_MAX_DIMS, strides in elements,
 * a source stride may be 0): dst[sum_j c_j*dst_strides[j]] = src[sum_j c_j*src_strides[j]]. The
 * HipTensor layer expresses reshape/contiguous (94-113), transpose (115-137), slice (139-183),
 * cat (185-252), stack (254-335, 390-467) and broadcast_to (1352-1518, 511-560) with it. */
#define HX_MAX_DIMS 8
int hx_copy_strided_f32(int ndim, const int64_t* shape, const float* src,
                        const int64_t* src_strides, float* dst, const int64_t* dst_strides,
                        void* stream);

/* y[0..n) = value: Tensor zeros / ones / from_scalar (crates/backend-cpu/src/lib.rs:1273-1301,
 * 904-914). */
int hx_fill_f32(int64_t n, float value, float* y, void* stream);
/* n x n identity: TensorRandom::eye (crates/backend-cpu/src/lib.rs:1303-1316). */
int hx_eye_f32(int64_t n, float* y, void* stream);

/* ------------------------------------------------------------------ tuning */
/* Selects the selective-scan kernel variant for later calls on the calling thread: 0 = auto
 * (default), -1 = the generic one-thread-per-channel kernel (any dstate <= 64, no alignment
 * needs), 8 = the fast kernel (8 waves split the states of 64 channels), 40 = the wave-complete
 * kernel (a wave owns 16 channels x 16 states; 64-bit row offsets), 42 = its leaner form with
 * per-wave staging, 44 = the warp-specialised kernel (3 state waves + 1 element wave per CU, 48
 * channels per block), 46 = its split-state form (6 state waves holding half of each channel's
 * states + 2 element waves; bf16 storage needs dim % 8 == 0; the automatic choice for fp32
 * wherever 44 would be, while bf16 keeps 44).
 * A forced variant also makes the Mamba block and layer forwards run their dt projection and
 * scan as two steps (with the forced scan kernel) instead of hx_selective_scan_dtproj_fwd.
 * A measurement knob with no reference counterpart; results agree within fp32 rounding for
 * every variant. */
int hx_set_scan_variant(int variant);
/* Selects the bf16 GEMM kernel for later calls on the calling thread: 0 auto, 1 128x128 tiles,
 * 3 small-M 32x32 / 32x64 tiles with K split over 4 waves (K % 8 == 0),
 * 4 direct-to-LDS 256x128 tiles (K % 64 == 0), 5 direct-to-LDS 256x256 tiles with 64-wide K tiles
 * (K % 64 == 0), 6 the same with 32-wide K tiles in a 4-stage ring (K % 32 == 0), 7 the narrow
 * kernel: 64-row tiles holding every column (N <= 256, K % 64 == 0), 8 the persistent form of 5
 * (one block per CU walks its tiles, the K-tile ring runs on across them; same bits as 5; the
 * automatic choice where K <= 1024 and there are at least two tiles per CU). A shape a forced kernel cannot take goes to the 128x128 kernel (the
 * small-M one for small shapes). A measurement knob. */
int hx_set_gemm_kernel(int k);
/* S4D knobs for later calls on the calling thread: path 0 auto (wave path for dstate 16), 1 the
 * per-channel thread path; time segments 0 auto, n forced. */
int hx_set_s4d_path(int path);
int hx_set_s4d_segments(int nseg);
/* Number of time segments the long-sequence path splits a scan into, for later calls on the
 * calling thread (0 = automatic: only when the (batch, 64-channel) tiles cannot fill the GPU and
 * seqlen >= 4096). Segments are scanned in parallel from a zero state, their entry states chained
 * by a carry kernel, then rescanned with outputs. A measurement knob; results agree within fp32
 * rounding for every setting. */
int hx_set_scan_segments(int nseg);

#ifdef __cplusplus
}
#endif
#endif /* HELIX_HIP_H */

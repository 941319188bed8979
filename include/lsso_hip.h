/*
 * lsso_hip.h -- C ABI of the MI355X (gfx950) native LSSO mixer library.
 *
 * The library implements the DYNAMIC + Rank-Rotary LSSO mixer and its two
 * biased projections as hand-written CDNA4 kernels.  Every entry point takes
 * plain device pointers, sizes and a hipStream_t; the library never allocates
 * device memory.  Callers size the scratch buffers with the *_workspace_bytes
 * queries and own every allocation; the one exception,
 * lsso_hip_mixer_forward_static, uses a device array that is part of the
 * library's code object instead.  All launches are asynchronous and
 * stream-ordered; no entry point synchronizes the host.
 *
 * Return values: 0 on success, a negative LSSO_HIP_E* code on failure.  The
 * message of the most recent failure on the calling thread is available from
 * lsso_hip_last_error().
 *
 * Each declaration cites the reference interface it replaces.  Reference
 * paths are relative to the Yang916-yy/LSSO source tree.
 */
#ifndef LSSO_HIP_H_
#define LSSO_HIP_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LSSO_HIP_CONTRACT_VERSION 1

/* Error codes. */
#define LSSO_HIP_OK 0
#define LSSO_HIP_EINVAL (-1)      /* invalid shape, pointer or size */
#define LSSO_HIP_EUNSUPPORTED (-2) /* valid input outside the native contract */
#define LSSO_HIP_ERUNTIME (-3)    /* a HIP runtime call or launch failed */

/* Element types accepted by the projection entry point. */
#define LSSO_HIP_F16 1
#define LSSO_HIP_BF16 2

/* Position metadata layouts for the mixer (reference csrc/ball/common.cuh:245-257). */
#define LSSO_HIP_POSITIONS_DEFAULT 0 /* p_t = t - (N - 1) / 2, computed on device */
#define LSSO_HIP_POSITIONS_SHARED 1  /* centered float32 [N]                      */
#define LSSO_HIP_POSITIONS_BATCHED 2 /* centered float32 [B, N]                   */

/* Geometry of one mixer call.  `projected` is [batch, length, heads*rank +
 * heads*head_dim] bfloat16, the output is [batch, length, heads*head_dim]
 * bfloat16 (reference csrc/ball/common.cuh:60-67, FastPathShape). */
typedef struct lsso_hip_mixer_shape {
    int64_t batch;
    int64_t length;
    int64_t heads;
    int64_t rank;
    int64_t head_dim;
} lsso_hip_mixer_shape;

/* Native contract version of this library.
 * Replaces: torch.ops.lsso_equilibrium.contract_version
 * (csrc/ball/binding.cpp:72-74, lsso/ball/cuda.py:28-54). */
int lsso_hip_contract_version(void);

/* Offload target the library was compiled for ("gfx950").
 * Replaces: the per-SM artifact name check (lsso/ball/cuda.py:200-208). */
const char* lsso_hip_target(void);

/* Message of the most recent failure on the calling thread ("" if none).
 * Replaces: TORCH_CHECK messages (csrc/ball/common.cuh:194-269). */
const char* lsso_hip_last_error(void);

/* Validate a mixer geometry on the host without touching the GPU.
 * Replaces: validate_fast_inputs shape checks (csrc/ball/common.cuh:194-269). */
int lsso_hip_mixer_validate(const lsso_hip_mixer_shape* shape, int positions_mode);

/* Device scratch bytes needed by lsso_hip_mixer_forward for this geometry.
 * Replaces: the at::empty workspace allocations of launch_generic_forward
 * (csrc/ball/forward.cu:1227-1449). */
int lsso_hip_mixer_workspace_bytes(const lsso_hip_mixer_shape* shape,
                                   int positions_mode, size_t* bytes);

/* Number of float32 values in the per-call training tape (0 if the caller
 * passes tape == NULL).  The tape holds only compact per-(sample, head)
 * state, no token-sized frame: per system (b, h), in order, L, Theta,
 * (I + K)^-1 and L^-1 (r x r each, row-major), then Z and U (r x d each).
 * Replaces: training_tape_layout (csrc/ball/common.cuh:84-108). */
int lsso_hip_mixer_tape_floats(const lsso_hip_mixer_shape* shape, size_t* floats);

/* Complete DYNAMIC + Rank-Rotary mixer forward:
 *   mixed = eta C + P [2 (I + K)^-1 Z - (1 + eta) Z],  Z = P^T C,
 * evaluated through P = A L^-T with L L^T = A^T A + I.
 * inverse_frequency: optional host array of rank/2 float32 rotary
 * frequencies (NULL: computed as 10000^(-j/(rank/2)) in float32).
 * valid_counts: optional device float32 [batch] (>= 1) when a mask is used;
 * masked rows of `projected` must be zero.  tape: optional device buffer of
 * lsso_hip_mixer_tape_floats() floats that receives the compact state.
 * Replaces: torch.ops.lsso_equilibrium.forward_inference / forward_train
 * (csrc/ball/binding.cpp:84-90, csrc/ball/forward.cu:1505-1556,
 *  lsso/ball/cuda.py:283-323). */
int lsso_hip_mixer_forward(const lsso_hip_mixer_shape* shape,
                           const void* projected,
                           const float* core_base_raw,
                           const float* core_drive_weight,
                           const float* eta_raw,
                           const float* inverse_frequency,
                           const float* centered_positions,
                           int positions_mode,
                           const float* valid_counts,
                           void* output,
                           float* tape,
                           void* workspace,
                           size_t workspace_bytes,
                           void* stream);

/* Size of the device array that lsso_hip_mixer_forward_static uses as its
 * workspace (64 MiB; each GPU the library runs on holds one). */
#define LSSO_HIP_STATIC_SCRATCH_BYTES ((size_t)64 << 20)

/* lsso_hip_mixer_forward without a caller workspace, and without any device
 * allocation: the workspace is a device array of the library's own, of
 * LSSO_HIP_STATIC_SCRATCH_BYTES per GPU, held from the library's first use on
 * a GPU until the process ends.  Geometries whose
 * lsso_hip_mixer_workspace_bytes() exceeds that size are rejected with
 * LSSO_HIP_EUNSUPPORTED (B = 64, N = 4096, H = 8, r = 32, d = 32 needs about
 * 21 MB).  All calls on one GPU share its array: calls in flight at the same
 * time on one GPU (on different streams) race, calls ordered on one stream do
 * not.  Arguments and results are those of lsso_hip_mixer_forward.  The
 * stream must belong to the current device (LSSO_HIP_EINVAL otherwise).  The
 * first call on a device looks the array's address up (hipGetSymbolAddress);
 * make that call outside stream capture, after which calls can be captured
 * into a HIP graph and replayed (the kernels write every scratch byte they
 * read, so no memset is recorded).
 * No counterpart in the reference: this entry point is for callers that cannot
 * allocate device memory (code under HIP graph capture, serving loops,
 * harnesses that forbid hipMalloc). */
int lsso_hip_mixer_forward_static(const lsso_hip_mixer_shape* shape,
                                  const void* projected,
                                  const float* core_base_raw,
                                  const float* core_drive_weight,
                                  const float* eta_raw,
                                  const float* inverse_frequency,
                                  const float* centered_positions,
                                  int positions_mode,
                                  const float* valid_counts,
                                  void* output,
                                  float* tape,
                                  void* stream);

/* Device scratch bytes needed by lsso_hip_mixer_backward.
 * Replaces: the at::empty allocations of backward_cuda
 * (csrc/ball/backward.cu:1386-1400). */
int lsso_hip_mixer_backward_workspace_bytes(const lsso_hip_mixer_shape* shape,
                                            int positions_mode, size_t* bytes);

/* First-order backward of lsso_hip_mixer_forward, given the tape that a call
 * with a tape pointer recorded.  grad_output: bfloat16 [batch, length,
 * heads*head_dim] (masked rows zero); outputs grad_projected bfloat16 like
 * projected, and float32 grad_base [H, r, r], grad_drive [H, d, r] and
 * grad_eta [H] (sums over the batch in a fixed order: deterministic).
 * Any head_dim (heads wider than 64 take the compact VJP in 32-column
 * panels).  Positions, counts and inverse_frequency as in the forward.
 * Replaces: torch.ops.lsso_equilibrium.backward (csrc/ball/binding.cpp:92-95,
 * csrc/ball/backward.cu:1386-1667, lsso/ball/cuda.py:256-280). */
int lsso_hip_mixer_backward(const lsso_hip_mixer_shape* shape,
                            const void* grad_output,
                            const void* projected,
                            const float* core_base_raw,
                            const float* core_drive_weight,
                            const float* eta_raw,
                            const float* inverse_frequency,
                            const float* centered_positions,
                            int positions_mode,
                            const float* valid_counts,
                            const float* tape,
                            void* grad_projected,
                            float* grad_base,
                            float* grad_drive,
                            float* grad_eta,
                            void* workspace,
                            size_t workspace_bytes,
                            void* stream);

/* lsso_hip_mixer_backward, and, when grad_projected_column_sums (float32
 * [H*(rank+head_dim)]) is not NULL, the FP32 sums over all rows of each
 * column of grad_projected: the bias gradient of the input projection
 * (grad_output.sum(dim=rows, dtype=float32) in _TensorCoreLinear.backward).
 * The sums are taken from the token map's output tiles, so grad_projected is
 * not read again; they are added in a fixed order.  Same workspace as
 * lsso_hip_mixer_backward.
 * Replaces: torch.ops.lsso_equilibrium.backward followed by the input
 * projection's bias reduction (csrc/ball/backward.cu:1386-1667;
 * lsso/ball/reference.py:236-245). */
int lsso_hip_mixer_backward_ex(const lsso_hip_mixer_shape* shape,
                               const void* grad_output,
                               const void* projected,
                               const float* core_base_raw,
                               const float* core_drive_weight,
                               const float* eta_raw,
                               const float* inverse_frequency,
                               const float* centered_positions,
                               int positions_mode,
                               const float* valid_counts,
                               const float* tape,
                               void* grad_projected,
                               float* grad_base,
                               float* grad_drive,
                               float* grad_eta,
                               float* grad_projected_column_sums,
                               void* workspace,
                               size_t workspace_bytes,
                               void* stream);

/* 1 if lsso_hip_mixer_forward_projected handles this shape, 0 if not (use
 * lsso_hip_mixer_forward followed by lsso_hip_linear), or a negative code for
 * an invalid shape.  The fused path covers heads <= 8, head_dim a multiple of
 * 16 up to 64, heads*head_dim <= 256 and heads*(rank+head_dim) <= 640.
 * Replaces: the choice between the native mixer and its output projection
 * in LSSO._forward_cuda (lsso/ball/model.py:389-405). */
int lsso_hip_mixer_projected_supported(const lsso_hip_mixer_shape* shape);

/* Mixer forward fused with the biased output projection (inference):
 *   y = cast(bf16(mixed) bf16(out_weight)^T + out_bias),  row_mask rows -> 0,
 * with mixed as in lsso_hip_mixer_forward, computed per token tile in LDS and
 * never written to memory.  The result is bitwise that of
 * lsso_hip_mixer_forward followed by lsso_hip_linear(mixed, out_weight,
 * out_bias, row_mask).  out_weight: float32 [H*d, H*d]; out_bias: float32
 * [H*d] or NULL; row_mask: uint8 [batch*length] or NULL; y: [batch, length,
 * H*d] of y_dtype (LSSO_HIP_F16 or LSSO_HIP_BF16), 16-byte aligned.  The
 * workspace is that of lsso_hip_mixer_forward.
 * Replaces: fast_mix followed by tensor_core_linear in LSSO._forward_cuda
 * (lsso/ball/model.py:389-405; lsso/ball/cuda.py:283-323,
 *  lsso/ball/reference.py:347-408). */
int lsso_hip_mixer_forward_projected(const lsso_hip_mixer_shape* shape,
                                     const void* projected,
                                     const float* core_base_raw,
                                     const float* core_drive_weight,
                                     const float* eta_raw,
                                     const float* inverse_frequency,
                                     const float* centered_positions,
                                     int positions_mode,
                                     const float* valid_counts,
                                     const float* out_weight,
                                     const float* out_bias,
                                     const uint8_t* row_mask,
                                     void* y,
                                     int y_dtype,
                                     void* workspace,
                                     size_t workspace_bytes,
                                     void* stream);

/* 1 if lsso_hip_layer_forward handles this shape, 0 if not (use
 * lsso_hip_linear and lsso_hip_mixer_forward), or a negative code for an
 * invalid shape.  The fused layer covers head_dim a multiple of 16 up to 64
 * and a model width H*head_dim up to 384.
 * Replaces: the choice of the native path in LSSO._forward_cuda
 * (lsso/ball/model.py:270-405). */
int lsso_hip_layer_supported(const lsso_hip_mixer_shape* shape);

/* Device scratch bytes needed by lsso_hip_layer_forward (the mixer workspace
 * plus the packed projection, and the mixed block when the output projection
 * cannot be fused). */
int lsso_hip_layer_workspace_bytes(const lsso_hip_mixer_shape* shape, int positions_mode,
                                   size_t* bytes);

/* The whole LSSO layer forward (inference), x [batch, length, H*d] -> y:
 *   packed = bf16(x in_weight^T + in_bias)   (row_mask rows -> 0)
 *   mixed  = the mixer of lsso_hip_mixer_forward on packed
 *   y      = cast(bf16(mixed) out_weight^T + out_bias)  (row_mask rows -> 0)
 * The input projection runs fused with the mixer's token reductions (one pass
 * over x per head group) at rank <= 32, and as its own kernel before the
 * reductions from rank 48 on, where that is faster; the output projection
 * runs fused with the apply when
 * lsso_hip_mixer_projected_supported() allows, so packed is read back once
 * and mixed never reaches HBM.  The result is bitwise that of lsso_hip_linear,
 * lsso_hip_mixer_forward and lsso_hip_linear in sequence.  in_weight: float32
 * [H*(rank+d), H*d]; in_bias: float32 [H*(rank+d)] or NULL; out_weight:
 * float32 [H*d, H*d]; out_bias: float32 [H*d] or NULL; row_mask: uint8
 * [batch*length] or NULL; x and y 16-byte aligned, of dtypes x_dtype and
 * y_dtype (LSSO_HIP_F16 or LSSO_HIP_BF16).  Positions, counts and
 * inverse_frequency as in lsso_hip_mixer_forward.
 * Replaces: tensor_core_linear -> fast_mix -> tensor_core_linear in
 * LSSO._forward_cuda (lsso/ball/model.py:270-405; lsso/ball/reference.py:347-408,
 * lsso/ball/cuda.py:283-323). */
int lsso_hip_layer_forward(const lsso_hip_mixer_shape* shape,
                           const void* x,
                           int x_dtype,
                           const float* in_weight,
                           const float* in_bias,
                           const uint8_t* row_mask,
                           const float* core_base_raw,
                           const float* core_drive_weight,
                           const float* eta_raw,
                           const float* inverse_frequency,
                           const float* centered_positions,
                           int positions_mode,
                           const float* valid_counts,
                           const float* out_weight,
                           const float* out_bias,
                           void* y,
                           int y_dtype,
                           void* workspace,
                           size_t workspace_bytes,
                           void* stream);

/* lsso_hip_layer_forward with timing marks for profiling callers: events
 * points to 8 hipEvent_t handles created with timing enabled (entries may be
 * NULL); events[2k] takes the begin of the first kernel and events[2k+1] the
 * end of the last kernel of stage k: 0 the phase table, 1 the fused input
 * projection + reductions, 2 the compact solve, 3 the apply + output
 * projection.  The kernel dispatches record them (hipExtLaunchKernel), so the
 * timing adds no queue packet between the kernels.  Results are those of
 * lsso_hip_layer_forward.
 * Replaces: the CUDA events around the timed region of the reference's
 * benchmark (benchmarks/benchmark_ball.py:189-206), moved inside the call so
 * that each stage is timed on its own. */
int lsso_hip_layer_forward_timed(const lsso_hip_mixer_shape* shape,
                                 const void* x,
                                 int x_dtype,
                                 const float* in_weight,
                                 const float* in_bias,
                                 const uint8_t* row_mask,
                                 const float* core_base_raw,
                                 const float* core_drive_weight,
                                 const float* eta_raw,
                                 const float* inverse_frequency,
                                 const float* centered_positions,
                                 int positions_mode,
                                 const float* valid_counts,
                                 const float* out_weight,
                                 const float* out_bias,
                                 void* y,
                                 int y_dtype,
                                 void* workspace,
                                 size_t workspace_bytes,
                                 void* stream,
                                 void* const* events);

/* Training forward of the input projection and the mixer, one call:
 *   packed = lsso_hip_linear(x, in_weight, in_bias, row_mask) (BF16),
 *   mixed  = lsso_hip_mixer_forward(packed, ..., tape),
 * with the projection fused with the token reductions at rank <= 32 (so x is
 * read once and packed is written once, then read once more by the apply)
 * and run as its own kernel from rank 48 on, where that is faster.  Both outputs
 * and the tape are bitwise those of the two calls; packed and the tape are
 * what lsso_hip_mixer_backward and the projection's backward need.  Shapes as
 * lsso_hip_layer_supported (ask it first); x: [batch, length, H*head_dim] of
 * x_dtype, 16-byte aligned; packed: BF16 [batch, length, H*(rank+head_dim)],
 * 16-byte aligned; mixed: BF16 [batch, length, H*head_dim]; tape: NULL or
 * lsso_hip_mixer_tape_floats() floats.  The workspace is that of
 * lsso_hip_mixer_forward.
 * Replaces: tensor_core_linear followed by fast_mix under autograd in
 * LSSO._forward_cuda (lsso/ball/model.py:270-405; lsso/ball/cuda.py:220-255). */
int lsso_hip_project_mix_forward(const lsso_hip_mixer_shape* shape,
                                 const void* x,
                                 int x_dtype,
                                 const float* in_weight,
                                 const float* in_bias,
                                 const uint8_t* row_mask,
                                 const float* core_base_raw,
                                 const float* core_drive_weight,
                                 const float* eta_raw,
                                 const float* inverse_frequency,
                                 const float* centered_positions,
                                 int positions_mode,
                                 const float* valid_counts,
                                 void* packed,
                                 void* mixed,
                                 float* tape,
                                 void* workspace,
                                 size_t workspace_bytes,
                                 void* stream);

/* Training forward of the whole layer, one call: lsso_hip_project_mix_forward
 * (packed, mixed and the tape for the backward) followed by the output
 * projection y = lsso_hip_linear(mixed, out_weight, out_bias, row_mask,
 * y_dtype).  Inside the fused readout's envelope
 * (lsso_hip_mixer_projected_supported, packed rows up to 640 columns) the
 * apply and the output projection run as one kernel that also stores mixed,
 * so mixed is written once and not read back; outside it, as two kernels.
 * All four outputs are bitwise those of the separate calls.  Workspace:
 * lsso_hip_mixer_workspace_bytes.
 * Replaces: the module's training forward, K1 + forward_train + K5
 * (lsso/ball/model.py:270-405 with csrc/ball/binding.cpp:80-95). */
int lsso_hip_layer_forward_train(const lsso_hip_mixer_shape* shape,
                                 const void* x,
                                 int x_dtype,
                                 const float* in_weight,
                                 const float* in_bias,
                                 const uint8_t* row_mask,
                                 const float* core_base_raw,
                                 const float* core_drive_weight,
                                 const float* eta_raw,
                                 const float* inverse_frequency,
                                 const float* centered_positions,
                                 int positions_mode,
                                 const float* valid_counts,
                                 const float* out_weight,
                                 const float* out_bias,
                                 void* packed,
                                 void* mixed,
                                 float* tape,
                                 void* y,
                                 int y_dtype,
                                 void* workspace,
                                 size_t workspace_bytes,
                                 void* stream);

/* Device scratch bytes needed by lsso_hip_linear. */
int lsso_hip_linear_workspace_bytes(int64_t rows, int64_t in_features,
                                    int64_t out_features, size_t* bytes);

/* Biased projection y = cast(bf16(x) bf16(W)^T + b): BF16 multiplicands,
 * FP32 accumulation, FP32 bias added before one final FP16/BF16 store.
 * x: [rows, in_features] with row stride x_row_stride elements (unit column
 * stride), dtype x_dtype.  weight: float32 [out_features, in_features]
 * contiguous.  bias: float32 [out_features] or NULL.  row_mask: optional
 * device uint8 [rows]; rows whose byte is 0 are written as zeros whatever
 * their x holds, NaN included (the masked-token contract of the reference's native forward,
 * lsso/ball/model.py:371-383, 402-404).  y: contiguous [rows, out_features]
 * of dtype y_dtype.
 * Replaces: tensor_core_linear / _biased_gemm (lsso/ball/reference.py:20-75,
 * 78-97, 347-408). */
int lsso_hip_linear(const void* x, int x_dtype, int64_t rows,
                    int64_t in_features, int64_t x_row_stride,
                    const float* weight, const float* bias,
                    const uint8_t* row_mask, int64_t out_features,
                    void* y, int y_dtype,
                    void* workspace, size_t workspace_bytes, void* stream);

/* Device scratch bytes needed by lsso_hip_linear_grad_columns. */
int lsso_hip_linear_grad_columns_workspace_bytes(int64_t rows, int64_t cols, size_t* bytes);

/* Upstream-gradient pass of the biased projection's backward, one read of g:
 * g: [rows, cols] of g_dtype (LSSO_HIP_F16 or LSSO_HIP_BF16) with row stride
 * g_row_stride elements (unit column stride); row_mask: optional device uint8
 * [rows], rows whose byte is 0 count as zero.  When g_bf16 is not NULL it
 * receives g rounded to BF16 (round to nearest even), contiguous [rows, cols],
 * excluded rows zero: the BF16 operand of the weight-gradient GEMM.  When
 * column_sums is not NULL it receives the FP32 sum of each column over the
 * kept rows (the bias gradient), added in a fixed order.  Either output may be
 * NULL; with both NULL the call does nothing.
 * Replaces: grad_output.to(torch.bfloat16) and grad_output.sum(dim=rows,
 * dtype=torch.float32) in _TensorCoreLinear.backward
 * (lsso/ball/reference.py:205-247). */
int lsso_hip_linear_grad_columns(const void* g, int g_dtype, int64_t rows, int64_t cols,
                                 int64_t g_row_stride, const uint8_t* row_mask,
                                 void* g_bf16, float* column_sums,
                                 void* workspace, size_t workspace_bytes, void* stream);

/* Device scratch bytes needed by lsso_hip_linear_weight_grad. */
int lsso_hip_linear_weight_grad_workspace_bytes(int64_t rows, int64_t in_features,
                                                int64_t out_features, size_t* bytes);

/* Weight and bias gradients of the biased projection, one pass over g and x:
 *   grad_weight[n][k] = sum over rows m of bf16(g[m][n]) bf16(x[m][k])  (FP32)
 *   grad_bias[n]      = sum over rows m of g[m][n]                       (FP32)
 * g: [rows, out_features] of g_dtype with row stride g_row_stride; x: [rows,
 * in_features] of x_dtype with row stride x_row_stride (LSSO_HIP_F16 or
 * LSSO_HIP_BF16, unit column strides).  row_mask: optional device uint8
 * [rows]; rows whose byte is 0 count as zero whatever g and x hold.
 * grad_weight: float32 [out_features, in_features] (written, not
 * accumulated); grad_bias: float32 [out_features] or NULL.  FP32
 * accumulation over row splits whose partials are added in a fixed order:
 * deterministic.
 * Replaces: grad_weight = bf16(grad)^T bf16(x) and grad_bias = grad.sum(rows)
 * in _TensorCoreLinear.backward (lsso/ball/reference.py:205-247). */
int lsso_hip_linear_weight_grad(const void* g, int g_dtype, int64_t g_row_stride,
                                const void* x, int x_dtype, int64_t x_row_stride,
                                int64_t rows, int64_t in_features, int64_t out_features,
                                const uint8_t* row_mask, float* grad_weight, float* grad_bias,
                                void* workspace, size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* LSSO_HIP_H_ */

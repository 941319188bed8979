// Kernel argument blocks and launchers shared between the kernel translation
// units and the C ABI.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <cstdint>

namespace lsso_hip {

// Events recorded by kernel dispatches themselves (hipExtLaunchKernel):
// `start` with the begin of the next dispatch, `stop` with the end of every
// dispatch, so that after a group of launches it holds the last one's end.
// Set per stage by the timed entry point around its own launches and cleared
// before it returns; unset, dispatches are plain launches.  Unlike
// hipEventRecord, this adds no queue packet between the kernels.
struct DispatchEvents {
    hipEvent_t start = nullptr;
    hipEvent_t stop = nullptr;
};
DispatchEvents& dispatch_events();   // this thread's

template <typename... KArgs, typename... Args>
inline void dispatch(void (*kernel)(KArgs...), dim3 grid, dim3 block, hipStream_t stream, Args... args) {
    DispatchEvents& events = dispatch_events();
    if (events.start == nullptr && events.stop == nullptr) {
        hipLaunchKernelGGL(kernel, grid, block, 0, stream, args...);
        return;
    }
    hipExtLaunchKernelGGL(kernel, grid, block, 0, stream, events.start, events.stop, 0, args...);
    events.start = nullptr;
}

constexpr int kMaxPairs = 32;

struct PhaseArgs {
    const float* positions;  // centered positions or nullptr (default grid)
    uint32_t* phases;        // packed FP16 (cos, sin), [count]
    int64_t count;           // (batches) * length * pairs
    int64_t length;
    int pairs;
    float inverse_frequency[kMaxPairs];
};

struct ReduceArgs {
    const uint16_t* projected;  // BF16 [B, N, width] (relation columns)
    const uint16_t* content;    // BF16 rows whose head-h columns are contracted with A
    int64_t content_stride;     // elements between consecutive tokens of `content`
    int gram;                   // also accumulate G = A^T A
    const uint32_t* phases;
    float* partials;            // [B, H, chunks, partial_stride]
    int64_t batch;
    int64_t length;
    int64_t heads;
    int64_t head_dim;
    int64_t width;              // heads * rank + heads * head_dim
    int64_t phase_batch_stride; // 0 (shared) or length * pairs
    int64_t chunks;
    int64_t chunk_tokens;       // multiple of 32
    int64_t column_groups;
    int64_t partial_stride;     // rank * rank + rank * head_dim
    int64_t total_waves;
    int64_t group_heads;        // staged form: heads per workgroup (0: one wave per work item)
};

struct SolveArgs {
    const float* partials;
    int64_t chunks;
    int64_t partial_stride;
    int64_t batch;
    int64_t length;
    int64_t heads;
    int64_t head_dim;
    const float* base;          // [H, R, R]
    const float* drive;         // [H, d, R]
    const float* eta_raw;       // [H]
    const float* valid_counts;  // [B] or nullptr
    float* zbuf;                // [B*H, R, d]
    uint16_t* mop;              // apply operand records
    float* tape;                // optional
    int64_t tape_stride;
};

struct ApplyArgs {
    const uint16_t* projected;
    const uint32_t* phases;
    const uint16_t* mop;
    const float* eta_raw;
    uint16_t* output;           // BF16 [B, N, H*d]
    int64_t batch;
    int64_t length;
    int64_t heads;
    int64_t head_dim;
    int64_t width;
    int64_t out_width;
    int64_t phase_batch_stride;
    int64_t chunks;
    int64_t chunk_tokens;       // multiple of 16
    int64_t feature_blocks;     // ceil(head_dim / 16)
    int64_t block_groups;       // ceil(feature_blocks / NFBW)
    int64_t total_waves;
    int64_t group_heads;        // staged form: heads per workgroup (0: one wave per work item)
    int64_t ranges;             // staged form: token ranges per sample
    int64_t range_tokens;       // staged form: tokens per range (a multiple of 16)
};

// Apply fused with the output projection: y = cast(bf16(mixed) bf16(W_o)^T
// + b_o) with mixed = eta C + rot(R) M' computed per 64-token tile in LDS.
struct MixProjectArgs {
    const uint16_t* projected;  // BF16 [B, N, width]
    const uint32_t* phases;
    const uint16_t* mop;        // apply operand records
    const float* eta_raw;       // [H]
    const float* weight;        // FP32 [D, D] (D = H * head_dim)
    const float* bias;          // FP32 [D] or nullptr
    const uint8_t* row_mask;    // [B * N] or nullptr
    void* y;                    // FP16/BF16 [B, N, D]
    uint16_t* mixed;            // BF16 [B, N, D] (the apply output, kept for training) or nullptr
    int64_t batch;
    int64_t length;
    int64_t heads;
    int64_t head_dim;
    int64_t width;
    int64_t out_features;       // D
    int64_t feature_blocks;     // head_dim / 16
    int64_t phase_batch_stride;
    int64_t ranges;             // token ranges per sample (one workgroup each)
    int64_t range_tokens;       // multiple of the 64-token tile
};

// Backward of the mixer (one compact system per workgroup).
struct BwdSolveArgs {
    const float* partials;      // S-part holds A^T dY per chunk
    int64_t chunks;
    int64_t partial_stride;
    const float* tape;          // [L | Theta | (I+K)^-1 | L^-1 | Z | U] per system
    int64_t tape_stride;
    const float* drive;         // [H, d, R]
    const float* eta_raw;       // [H]
    const float* valid_counts;  // [B] or nullptr
    int64_t batch;
    int64_t length;
    int64_t heads;
    int64_t head_dim;
    uint16_t* records;          // token-map operand records per system
    int64_t record_stride;      // in bf16
    int64_t off_m, off_e, off_g, off_f;
    int feature_k32;
    float* dtheta_part;         // [B*H, R, R]
    float* ddrive_part;         // [B*H, d, R]
    float* deta_part;           // [B*H]
};

struct BwdApplyArgs {
    const uint16_t* projected;  // BF16 [B, N, width]
    const uint16_t* grad_output;// BF16 [B, N, H*d]
    int64_t grad_stride;        // H*d
    const uint32_t* phases;
    int64_t phase_batch_stride;
    const uint16_t* records;
    int64_t record_stride;
    int64_t off_m, off_e, off_g, off_f;
    const float* eta_raw;
    uint16_t* grad_projected;   // BF16 [B, N, width]
    float* dot_part;            // [B*H, chunks]: <dY, C> per chunk
    float* column_part;         // [B*chunks, width]: column sums of grad_projected, or nullptr
    int64_t batch;
    int64_t length;
    int64_t heads;
    int64_t head_dim;
    int64_t width;
    int64_t chunks;
    int64_t chunk_tokens;       // multiple of 16
    int64_t total_waves;
};

struct ParamReduceArgs {
    const float* dtheta_part;
    const float* ddrive_part;
    const float* deta_part;
    const float* dot_part;
    const float* eta_raw;
    float* grad_base;           // [H, R, R]
    float* grad_drive;          // [H, d, R]
    float* grad_eta;            // [H]
    int64_t batch;
    int64_t heads;
    int64_t rank;
    int64_t head_dim;
    int64_t chunks;
};

struct LinearArgs {
    const void* x;
    int64_t rows;
    int64_t in_features;
    int64_t x_stride;
    const float* weight;        // FP32 [out, in]
    const float* bias;          // FP32 [out] or nullptr
    const uint8_t* row_mask;    // [rows] or nullptr; 0 rows are zeroed
    int64_t out_features;
    void* y;
    int64_t tiles;              // ceil(rows / tile_rows)
    int64_t column_groups;
    int x_vector;               // 16-byte x loads are legal
    int w_vector;               // 16-byte W loads are legal (K % 4 == 0, W 16-byte aligned)
    int y_vector;               // 16-byte y stores are legal
};

// Upstream-gradient pass of the projection's backward: BF16 copy and FP32
// column sums of g [rows, cols] in one read.
struct GradColumnsArgs {
    const void* g;              // FP16/BF16 [rows, cols], row stride g_stride
    int64_t rows;
    int64_t cols;
    int64_t g_stride;
    const uint8_t* row_mask;    // [rows] or nullptr; 0 rows count as zero
    uint16_t* g_bf16;           // BF16 [rows, cols] contiguous, or nullptr
    float* partials;            // [splits, cols] column sums per split, or nullptr
    int64_t rows_per_split;
    int chunks_per_slab;        // 8-column chunks per workgroup: divides 256
};

// Input projection fused with the L-reductions (one pass over x per head
// group): packed = bf16(x W^T + b) per 64-token tile in LDS, contracted into
// the G / S partials of each head of the group and optionally written out.
struct ProjectReduceArgs {
    const void* x;              // FP16/BF16 [B, N, D], rows contiguous
    const float* weight;        // FP32 [width, D]
    const float* bias;          // FP32 [width] or nullptr
    const uint8_t* row_mask;    // [B * N] or nullptr; 0 rows project to zero
    const uint32_t* phases;
    int64_t phase_batch_stride;
    uint16_t* packed;           // BF16 [B, N, width] or nullptr
    float* partials;            // [B, H, chunks, partial_stride]
    int64_t batch;
    int64_t length;
    int64_t heads;
    int64_t head_dim;
    int64_t in_features;        // D
    int64_t width;              // H * (rank + head_dim)
    int64_t chunks;
    int64_t chunk_tokens;       // multiple of the 64-token tile
    int64_t partial_stride;
    int64_t group_heads;        // heads per head group
    int64_t head_groups;
};

// Weight and bias gradient of the biased projection: FP32 partials per row
// split of sum_m bf16(g[m][n]) bf16(x[m][k]) and of sum_m g[m][n].
struct WeightGradArgs {
    const void* g;              // FP16/BF16 [rows, out_features], row stride g_stride
    int64_t g_stride;
    const void* x;              // FP16/BF16 [rows, in_features], row stride x_stride
    int64_t x_stride;
    const uint8_t* row_mask;    // [rows] or nullptr; 0 rows count as zero
    int64_t rows;
    int64_t out_features;
    int64_t in_features;
    float* partials;            // [splits, out_features, in_features]
    float* bias_partials;       // [splits, out_features] or nullptr
    int64_t rows_per_split;     // multiple of 32
    int64_t splits;
    int64_t tiles_n;
    int64_t tiles_k;
    int vec;                    // 16-byte loads of g and x are legal
};

hipError_t launch_phase(const PhaseArgs& a, hipStream_t stream);
hipError_t launch_reduce(int rank, const ReduceArgs& a, int cpw, bool vec, hipStream_t stream);
// Heads per workgroup of the staged reduce for this geometry, or 0 where it
// does not apply (the one-wave-per-item reduce_kernel runs instead).
int64_t reduce_staged_group_heads(int64_t rank, int64_t heads, int64_t head_dim, int64_t column_groups,
                                  int64_t content_stride, bool vec);
hipError_t launch_solve(int rank, const SolveArgs& a, int64_t systems, hipStream_t stream);
hipError_t launch_apply(int rank, const ApplyArgs& a, int nfbw, bool vec, hipStream_t stream);
// Heads per workgroup of the staged apply for this geometry, or 0 where it
// does not apply.
int64_t apply_staged_group_heads(int64_t rank, int64_t heads, int64_t head_dim, int nfbw, bool vec);

// Projection launcher; k_steps = ceil(in_features / 16) rounded to a
// compiled tier.  Returns hipErrorInvalidValue for an unsupported tier.
// Shapes the fused apply + output projection handles: heads <= 8, head_dim a
// multiple of 16 up to 64, D = heads * head_dim <= 256, width <= 640.
bool mix_project_supported(int64_t rank, int64_t heads, int64_t head_dim, int64_t width);
int mix_project_tile_rows();
hipError_t launch_mix_project(int rank, const MixProjectArgs& a, int y_dtype, hipStream_t stream);

bool backward_supported(int64_t rank, int64_t head_dim);
// Record offsets (bf16 elements) of the token-map operands of one system;
// returns the per-system record size.
int64_t bwd_record_layout(int64_t rank, int64_t head_dim, int64_t* off_m, int64_t* off_e,
                          int64_t* off_g, int64_t* off_f, int* feature_k32);
hipError_t launch_bwd_solve(int rank, const BwdSolveArgs& a, int64_t systems, hipStream_t stream);
hipError_t launch_bwd_apply(int rank, const BwdApplyArgs& a, bool dk32, bool vec, hipStream_t stream);
// True when launch_bwd_apply runs the resident token map, which also writes
// column_part when it is set.
bool bwd_apply_resident(int rank, int64_t head_dim, bool vec);
hipError_t launch_column_sum(const float* partials, int64_t splits, int64_t cols, float* out,
                             hipStream_t stream);
// Two column sums over the same number of splits in one launch (partials2
// may be null when cols2 is 0).
hipError_t launch_column_sums(const float* partials, int64_t cols, float* out, const float* partials2,
                              int64_t cols2, float* out2, int64_t splits, hipStream_t stream);
hipError_t launch_param_reduce(const ParamReduceArgs& a, hipStream_t stream);

hipError_t launch_linear(const LinearArgs& a, int k_steps, int x_dtype, int y_dtype,
                         int grid_groups, hipStream_t stream);
// Heads per group of the fused projection + reduce for this geometry, or 0
// when the shape is outside the fused envelope.
int project_reduce_group_heads(int64_t rank, int64_t heads, int64_t head_dim,
                               int64_t in_features);
int project_reduce_tile_rows();
hipError_t launch_project_reduce(int rank, const ProjectReduceArgs& a, int x_dtype, int grid,
                                 hipStream_t stream);
hipError_t launch_grad_columns(const GradColumnsArgs& a, int g_dtype, bool vec, int64_t splits,
                               int64_t slabs, float* column_sums, hipStream_t stream);
void plan_weight_grad(int64_t rows, int64_t in_features, int64_t out_features, int64_t* splits,
                      int64_t* rows_per_split);
int weight_grad_tile();
hipError_t launch_weight_grad(const WeightGradArgs& a, int g_dtype, int x_dtype, hipStream_t stream);
int linear_tile_rows(int k_steps);
int linear_columns_per_group(int k_steps);
int linear_k_tier(int64_t in_features);

}  // namespace lsso_hip

// C ABI of the gfx950 LSSO library: host-side validation, workspace
// planning and stream-ordered launches.  Nothing here allocates device
// memory or synchronizes the host.

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstdlib>
#include <mutex>
#include <string>

#include "lsso_hip.h"
#include "lsso_internal.h"

namespace lsso_hip {

DispatchEvents& dispatch_events() {
    thread_local DispatchEvents events;
    return events;
}

}  // namespace lsso_hip

namespace {

thread_local std::string g_last_error;

int fail(int code, const std::string& message) {
    g_last_error = message;
    return code;
}

int hip_failure(hipError_t error, const char* where) {
    return fail(LSSO_HIP_ERUNTIME,
                std::string(where) + " failed: " + hipGetErrorString(error));
}

int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }
size_t align_up(size_t value) { return (value + 255) & ~static_cast<size_t>(255); }

// Token chunk of the L-reductions.  It depends on nothing but itself, so a
// sequence is cut into the same chunks (and its G / S partials are summed in
// the same order) whatever the batch holds: a sample's outputs and input
// gradients are bitwise the same alone or in any batch.  The reference gets
// the same property from its fixed 32-token tile partials
// (csrc/ball/forward.cu:510-628).  512 tokens keeps the partial traffic small
// (2 partial sets per 1,024 tokens) while B = 64 sequences of 1,024 tokens
// still give 128 chunks, about one per compute unit and head group.
constexpr int64_t kReduceChunkTokens = 512;
constexpr int64_t kApplyTargetWaves = 4096;
constexpr int64_t kApplyStagedTargetGroups = 512;   // workgroups of the staged apply

// From 4,096 tokens on, chunks of 1,024 tokens halve the partials the
// reductions write and the solve reads (8.4 MB each at C3) and still leave
// four chunks per sequence (measured: the C3 call 0.251 against 0.256 ms, C4
// 485.7 against 490.2 us).  Shorter sequences keep 512-token chunks: at 2,048
// tokens, two chunks per sequence leave the standalone reduce too few waves
// (the C5 step 1,166 against 1,139 us).  The choice depends on the sequence
// length only, never on the batch.
int64_t reduce_chunk_tokens(int64_t length) {
    return length >= 4096 ? 2 * kReduceChunkTokens : kReduceChunkTokens;
}

struct MixerPlan {
    int64_t batch, length, heads, rank, head_dim;
    int64_t width, out_width, pairs, phase_batches;
    int cpw;
    int64_t column_groups, reduce_chunks, reduce_chunk_tokens;
    int nfbw;
    int64_t feature_blocks, block_groups, apply_chunks, apply_chunk_tokens;
    int64_t partial_stride, tape_stride;
    size_t off_phases, off_partials, off_zbuf, off_mop, total;
};

void plan_chunks(int64_t length, int64_t waves_per_chunk, int64_t target_waves,
                 int64_t granularity, int64_t* chunks, int64_t* chunk_tokens) {
    const int64_t max_chunks = ceil_div(length, granularity);
    int64_t wanted = ceil_div(target_waves, waves_per_chunk);
    if (wanted < 1) wanted = 1;
    if (wanted > max_chunks) wanted = max_chunks;
    const int64_t tokens = ceil_div(ceil_div(length, wanted), granularity) * granularity;
    *chunk_tokens = tokens;
    *chunks = ceil_div(length, tokens);
}

int make_plan(const lsso_hip_mixer_shape* shape, int positions_mode, MixerPlan* p) {
    if (shape == nullptr) {
        return fail(LSSO_HIP_EINVAL, "shape must not be NULL");
    }
    p->batch = shape->batch;
    p->length = shape->length;
    p->heads = shape->heads;
    p->rank = shape->rank;
    p->head_dim = shape->head_dim;
    if (p->batch <= 0 || p->length <= 0 || p->heads <= 0) {
        return fail(LSSO_HIP_EINVAL, "B, N, and H must be positive");
    }
    if (p->rank != 16 && p->rank != 32 && p->rank != 48 && p->rank != 64) {
        return fail(LSSO_HIP_EUNSUPPORTED,
                    "the HIP fast path supports rank in {16, 32, 48, 64}, got " +
                        std::to_string(p->rank));
    }
    if (p->head_dim <= 0) {
        return fail(LSSO_HIP_EINVAL,
                    "projected width must exceed H*R for a nonempty content channel");
    }
    if (positions_mode != LSSO_HIP_POSITIONS_DEFAULT &&
        positions_mode != LSSO_HIP_POSITIONS_SHARED &&
        positions_mode != LSSO_HIP_POSITIONS_BATCHED) {
        return fail(LSSO_HIP_EINVAL, "positions_mode must be 0 (default), 1 ([N]) or 2 ([B, N])");
    }
    p->width = p->heads * (p->rank + p->head_dim);
    p->out_width = p->heads * p->head_dim;
    p->pairs = p->rank / 2;
    p->phase_batches = positions_mode == LSSO_HIP_POSITIONS_BATCHED ? p->batch : 1;
    // The phase kernel indexes (position, 4 pairs) pieces with 32-bit integers.
    if (p->phase_batches * p->length > (int64_t{1} << 31) / p->pairs * 4) {
        return fail(LSSO_HIP_EUNSUPPORTED, "the phase table (B*N*rank/2 entries with per-sample "
                                           "positions, else N*rank/2) must stay below 2^33 entries");
    }

    // Two 32-feature column groups per reduction wave where the registers
    // allow two waves per SIMD (rank <= 32); from rank 48 on the two-group
    // form runs one wave per SIMD, and one group per wave is faster.
    p->cpw = p->head_dim > 32 && p->rank <= 32 ? 2 : 1;
    p->column_groups = ceil_div(p->head_dim, 32 * p->cpw);
    // Chunks are whole 64-token tiles, so the fused projection + reduce and
    // the standalone reduce share one chunking (and their partials agree).
    static_assert(kReduceChunkTokens % 64 == 0, "reduce chunks are whole projection tiles");
    p->reduce_chunk_tokens = reduce_chunk_tokens(p->length);
    p->reduce_chunks = ceil_div(p->length, p->reduce_chunk_tokens);
    if (lsso_hip::project_reduce_tile_rows() != 64) {
        return fail(LSSO_HIP_ERUNTIME, "internal: the projection tile is not 64 rows");
    }

    p->feature_blocks = ceil_div(p->head_dim, 16);
    p->nfbw = p->feature_blocks >= 4 ? 4 : (p->feature_blocks == 3 ? 4 : static_cast<int>(p->feature_blocks));
    p->block_groups = ceil_div(p->feature_blocks, p->nfbw);
    plan_chunks(p->length, p->batch * p->heads * p->block_groups, kApplyTargetWaves, 16,
                &p->apply_chunks, &p->apply_chunk_tokens);

    p->partial_stride = p->rank * p->rank + p->rank * p->head_dim;
    p->tape_stride = 4 * p->rank * p->rank + 2 * p->rank * p->head_dim;

    const int64_t systems = p->batch * p->heads;
    size_t offset = 0;
    p->off_phases = offset;
    offset = align_up(offset + sizeof(uint32_t) * p->phase_batches * p->length * p->pairs);
    p->off_partials = offset;
    offset = align_up(offset + sizeof(float) * systems * p->reduce_chunks * p->partial_stride);
    p->off_zbuf = offset;
    offset = align_up(offset + sizeof(float) * systems * p->rank * p->head_dim);
    p->off_mop = offset;
    offset = align_up(offset + sizeof(uint16_t) * systems * p->feature_blocks * 64 * (p->rank / 2));
    p->total = offset;
    return LSSO_HIP_OK;
}

bool aligned(const void* pointer, uintptr_t bytes) {
    return (reinterpret_cast<uintptr_t>(pointer) % bytes) == 0;
}

}  // namespace

extern "C" {

int lsso_hip_contract_version(void) { return LSSO_HIP_CONTRACT_VERSION; }

const char* lsso_hip_target(void) { return "gfx950"; }

const char* lsso_hip_last_error(void) { return g_last_error.c_str(); }

int lsso_hip_mixer_validate(const lsso_hip_mixer_shape* shape, int positions_mode) {
    MixerPlan plan;
    return make_plan(shape, positions_mode, &plan);
}

int lsso_hip_mixer_workspace_bytes(const lsso_hip_mixer_shape* shape, int positions_mode,
                                   size_t* bytes) {
    if (bytes == nullptr) {
        return fail(LSSO_HIP_EINVAL, "bytes must not be NULL");
    }
    MixerPlan plan;
    const int status = make_plan(shape, positions_mode, &plan);
    if (status != LSSO_HIP_OK) {
        return status;
    }
    *bytes = plan.total;
    return LSSO_HIP_OK;
}

int lsso_hip_mixer_tape_floats(const lsso_hip_mixer_shape* shape, size_t* floats) {
    if (floats == nullptr) {
        return fail(LSSO_HIP_EINVAL, "floats must not be NULL");
    }
    MixerPlan plan;
    const int status = make_plan(shape, LSSO_HIP_POSITIONS_DEFAULT, &plan);
    if (status != LSSO_HIP_OK) {
        return status;
    }
    *floats = static_cast<size_t>(plan.batch * plan.heads * plan.tape_stride);
    return LSSO_HIP_OK;
}

}  // extern "C"

namespace {

// Device pointers of the mixer workspace.
struct MixerBuffers {
    uint32_t* phases;
    float* partials;
    float* zbuf;
    uint16_t* mop;
};

int check_mixer_call(const MixerPlan& plan, const void* projected, const float* core_base_raw,
                     const float* core_drive_weight, const float* eta_raw, const void* output,
                     const float* centered_positions, int positions_mode, void* workspace,
                     size_t workspace_bytes, MixerBuffers* buffers) {
    if (projected == nullptr || core_base_raw == nullptr || core_drive_weight == nullptr ||
        eta_raw == nullptr || output == nullptr) {
        return fail(LSSO_HIP_EINVAL, "projected, parameters and output must not be NULL");
    }
    if (positions_mode != LSSO_HIP_POSITIONS_DEFAULT && centered_positions == nullptr) {
        return fail(LSSO_HIP_EINVAL, "centered_positions must not be NULL for this positions_mode");
    }
    if (workspace == nullptr || workspace_bytes < plan.total) {
        return fail(LSSO_HIP_EINVAL, "workspace is smaller than lsso_hip_mixer_workspace_bytes()");
    }
    if (!aligned(workspace, 256)) {
        return fail(LSSO_HIP_EINVAL, "workspace must be 256-byte aligned");
    }
    if (!aligned(projected, 2) || !aligned(output, 2)) {
        return fail(LSSO_HIP_EINVAL, "projected and output must be 2-byte aligned 16-bit buffers");
    }
    char* ws = static_cast<char*>(workspace);
    buffers->phases = reinterpret_cast<uint32_t*>(ws + plan.off_phases);
    buffers->partials = reinterpret_cast<float*>(ws + plan.off_partials);
    buffers->zbuf = reinterpret_cast<float*>(ws + plan.off_zbuf);
    buffers->mop = reinterpret_cast<uint16_t*>(ws + plan.off_mop);
    return LSSO_HIP_OK;
}

int64_t phase_batch_stride(const MixerPlan& plan, int positions_mode) {
    return positions_mode == LSSO_HIP_POSITIONS_BATCHED ? plan.length * plan.pairs : 0;
}

bool vector_rows(const MixerPlan& plan, const void* projected, const void* output) {
    return plan.width % 8 == 0 && plan.head_dim % 4 == 0 && aligned(projected, 16) &&
           aligned(output, 16);
}

int run_phase(const MixerPlan& plan, const MixerBuffers& buf, const float* inverse_frequency,
              const float* centered_positions, int positions_mode, hipStream_t stream) {
    lsso_hip::PhaseArgs phase{};
    phase.positions = positions_mode == LSSO_HIP_POSITIONS_DEFAULT ? nullptr : centered_positions;
    phase.phases = buf.phases;
    phase.count = plan.phase_batches * plan.length * plan.pairs;
    phase.length = plan.length;
    phase.pairs = static_cast<int>(plan.pairs);
    for (int j = 0; j < plan.pairs; ++j) {
        phase.inverse_frequency[j] = inverse_frequency != nullptr
            ? inverse_frequency[j]
            : std::pow(10000.0f, -static_cast<float>(j) / static_cast<float>(plan.pairs));
    }
    const hipError_t error = lsso_hip::launch_phase(phase, stream);
    return error == hipSuccess ? LSSO_HIP_OK : hip_failure(error, "phase_kernel launch");
}

int run_solve(const MixerPlan& plan, const MixerBuffers& buf, const float* core_base_raw,
              const float* core_drive_weight, const float* eta_raw, const float* valid_counts,
              float* tape, hipStream_t stream) {
    lsso_hip::SolveArgs solve{};
    solve.partials = buf.partials;
    solve.chunks = plan.reduce_chunks;
    solve.partial_stride = plan.partial_stride;
    solve.batch = plan.batch;
    solve.length = plan.length;
    solve.heads = plan.heads;
    solve.head_dim = plan.head_dim;
    solve.base = core_base_raw;
    solve.drive = core_drive_weight;
    solve.eta_raw = eta_raw;
    solve.valid_counts = valid_counts;
    solve.zbuf = buf.zbuf;
    solve.mop = buf.mop;
    solve.tape = tape;
    solve.tape_stride = plan.tape_stride;
    const hipError_t error = lsso_hip::launch_solve(static_cast<int>(plan.rank), solve,
                                                    plan.batch * plan.heads, stream);
    return error == hipSuccess ? LSSO_HIP_OK : hip_failure(error, "solve_kernel launch");
}

// Phase table, L-reductions and the compact solve: everything up to the
// apply operand records.
int run_reduce(const MixerPlan& plan, const MixerBuffers& buf, const void* projected,
               int positions_mode, bool vec, hipStream_t stream);

int run_compact(const MixerPlan& plan, const MixerBuffers& buf, const void* projected,
                const float* core_base_raw, const float* core_drive_weight, const float* eta_raw,
                const float* inverse_frequency, const float* centered_positions,
                int positions_mode, const float* valid_counts, float* tape, bool vec,
                hipStream_t stream) {
    int status = run_phase(plan, buf, inverse_frequency, centered_positions, positions_mode, stream);
    if (status != LSSO_HIP_OK) {
        return status;
    }
    status = run_reduce(plan, buf, projected, positions_mode, vec, stream);
    if (status != LSSO_HIP_OK) {
        return status;
    }
    return run_solve(plan, buf, core_base_raw, core_drive_weight, eta_raw, valid_counts, tape,
                     stream);
}

// The token reductions of packed (G and S partials per chunk).
int run_reduce(const MixerPlan& plan, const MixerBuffers& buf, const void* projected,
               int positions_mode, bool vec, hipStream_t stream) {
    lsso_hip::ReduceArgs reduce{};
    reduce.projected = static_cast<const uint16_t*>(projected);
    reduce.content = static_cast<const uint16_t*>(projected) + plan.heads * plan.rank;
    reduce.content_stride = plan.width;
    reduce.gram = 1;
    reduce.phases = buf.phases;
    reduce.partials = buf.partials;
    reduce.batch = plan.batch;
    reduce.length = plan.length;
    reduce.heads = plan.heads;
    reduce.head_dim = plan.head_dim;
    reduce.width = plan.width;
    reduce.phase_batch_stride = phase_batch_stride(plan, positions_mode);
    reduce.chunks = plan.reduce_chunks;
    reduce.chunk_tokens = plan.reduce_chunk_tokens;
    reduce.column_groups = plan.column_groups;
    reduce.partial_stride = plan.partial_stride;
    reduce.total_waves = plan.batch * plan.heads * plan.reduce_chunks * plan.column_groups;
    reduce.group_heads = plan.cpw == 1 ? lsso_hip::reduce_staged_group_heads(plan.rank, plan.heads, plan.head_dim,
                                                                              plan.column_groups, reduce.content_stride,
                                                                              vec && plan.head_dim % 8 == 0)
                                       : 0;
    const hipError_t error =
        lsso_hip::launch_reduce(static_cast<int>(plan.rank), reduce, plan.cpw, vec, stream);
    return error == hipSuccess ? LSSO_HIP_OK : hip_failure(error, "reduce_kernel launch");
}

int run_apply(const MixerPlan& plan, const MixerBuffers& buf, const void* projected,
              const float* eta_raw, int positions_mode, void* output, bool vec,
              hipStream_t stream) {
    lsso_hip::ApplyArgs apply{};
    apply.projected = static_cast<const uint16_t*>(projected);
    apply.phases = buf.phases;
    apply.mop = buf.mop;
    apply.eta_raw = eta_raw;
    apply.output = static_cast<uint16_t*>(output);
    apply.batch = plan.batch;
    apply.length = plan.length;
    apply.heads = plan.heads;
    apply.head_dim = plan.head_dim;
    apply.width = plan.width;
    apply.out_width = plan.out_width;
    apply.phase_batch_stride = phase_batch_stride(plan, positions_mode);
    apply.chunks = plan.apply_chunks;
    apply.chunk_tokens = plan.apply_chunk_tokens;
    apply.feature_blocks = plan.feature_blocks;
    apply.block_groups = plan.block_groups;
    apply.total_waves = plan.batch * plan.heads * plan.apply_chunks * plan.block_groups;
    // From rank 48 on the apply stages whole row runs per group of heads:
    // about two workgroups per CU, whole 32-token pairs of steps per range.
    apply.group_heads = lsso_hip::apply_staged_group_heads(plan.rank, plan.heads, plan.head_dim, plan.nfbw,
                                                           vec && plan.head_dim % 8 == 0);
    if (apply.group_heads > 0) {
        const int64_t groups = ceil_div(plan.heads, apply.group_heads);
        apply.ranges = std::max<int64_t>(1, ceil_div(kApplyStagedTargetGroups, plan.batch * groups));
        apply.range_tokens = ceil_div(ceil_div(plan.length, apply.ranges), 32) * 32;
        apply.ranges = ceil_div(plan.length, apply.range_tokens);
    }
    const hipError_t error =
        lsso_hip::launch_apply(static_cast<int>(plan.rank), apply, plan.nfbw, vec, stream);
    return error == hipSuccess ? LSSO_HIP_OK : hip_failure(error, "apply_kernel launch");
}

int compute_units(int* units) {
    int device = 0;
    hipError_t error = hipGetDevice(&device);
    if (error != hipSuccess) {
        return hip_failure(error, "hipGetDevice");
    }
    error = hipDeviceGetAttribute(units, hipDeviceAttributeMultiprocessorCount, device);
    if (error != hipSuccess) {
        return hip_failure(error, "hipDeviceGetAttribute");
    }
    return LSSO_HIP_OK;
}

// Fused apply + output projection into y (shape inside mix_project_supported).
int run_mix_project(const MixerPlan& plan, const MixerBuffers& buf, const void* projected,
                    const float* eta_raw, int positions_mode, const float* out_weight,
                    const float* out_bias, const uint8_t* row_mask, void* y, int y_dtype,
                    hipStream_t stream, void* mixed = nullptr) {
    int units = 0;
    const int status = compute_units(&units);
    if (status != LSSO_HIP_OK) {
        return status;
    }
    // One persistent workgroup per compute unit, each on a contiguous token
    // range of one sample (ranges are whole tiles).
    const int64_t tile = lsso_hip::mix_project_tile_rows();
    int64_t ranges = ceil_div(units, plan.batch);
    const int64_t max_ranges = ceil_div(plan.length, tile);
    if (ranges > max_ranges) ranges = max_ranges;
    const int64_t range_tokens = ceil_div(ceil_div(plan.length, ranges), tile) * tile;
    ranges = ceil_div(plan.length, range_tokens);

    lsso_hip::MixProjectArgs mix{};
    mix.projected = static_cast<const uint16_t*>(projected);
    mix.phases = buf.phases;
    mix.mop = buf.mop;
    mix.eta_raw = eta_raw;
    mix.weight = out_weight;
    mix.bias = out_bias;
    mix.row_mask = row_mask;
    mix.y = y;
    mix.mixed = static_cast<uint16_t*>(mixed);
    mix.batch = plan.batch;
    mix.length = plan.length;
    mix.heads = plan.heads;
    mix.head_dim = plan.head_dim;
    mix.width = plan.width;
    mix.out_features = plan.out_width;
    mix.feature_blocks = plan.feature_blocks;
    mix.phase_batch_stride = phase_batch_stride(plan, positions_mode);
    mix.ranges = ranges;
    mix.range_tokens = range_tokens;
    const hipError_t error =
        lsso_hip::launch_mix_project(static_cast<int>(plan.rank), mix, y_dtype, stream);
    return error == hipSuccess ? LSSO_HIP_OK : hip_failure(error, "mix_project_kernel launch");
}

// Biased projection launch (arguments already validated).
int run_linear(const void* x, int x_dtype, int64_t rows, int64_t in_features,
               int64_t x_row_stride, const float* weight, const float* bias,
               const uint8_t* row_mask, int64_t out_features, void* y, int y_dtype,
               hipStream_t stream) {
    const int tier = lsso_hip::linear_k_tier(in_features);
    int units = 0;
    const int status = compute_units(&units);
    if (status != LSSO_HIP_OK) {
        return status;
    }
    lsso_hip::LinearArgs args{};
    args.x = x;
    args.rows = rows;
    args.in_features = in_features;
    args.x_stride = x_row_stride;
    args.weight = weight;
    args.bias = bias;
    args.row_mask = row_mask;
    args.out_features = out_features;
    args.y = y;
    args.tiles = ceil_div(rows, lsso_hip::linear_tile_rows(tier));
    args.column_groups = ceil_div(out_features, lsso_hip::linear_columns_per_group(tier));
    args.x_vector = (in_features % 8 == 0 && x_row_stride % 8 == 0 && aligned(x, 16)) ? 1 : 0;
    args.w_vector = (in_features % 4 == 0 && aligned(weight, 16)) ? 1 : 0;
    args.y_vector = (out_features % 8 == 0 && aligned(y, 16)) ? 1 : 0;
    int64_t groups = units / args.column_groups;
    // With several column groups, a whole number of XCD rounds lets the
    // kernel deal the column groups of one row tile to one XCD, so x is
    // re-read from that XCD's L2: at 3 groups (640 or 768 outputs) 80 groups
    // on 240 CUs beat 85 on 255 (C5 step 1.127 against 1.131 ms, C4 forward
    // 0.466 against 0.472 ms).
    if (args.column_groups > 1 && groups >= 8) groups -= groups % 8;
    if (groups < 1) groups = 1;
    if (groups > args.tiles) groups = args.tiles;
    const hipError_t error =
        lsso_hip::launch_linear(args, tier, x_dtype, y_dtype, static_cast<int>(groups), stream);
    return error == hipSuccess ? LSSO_HIP_OK : hip_failure(error, "linear_kernel launch");
}

bool projected_shape_supported(const MixerPlan& plan) {
    return lsso_hip::mix_project_supported(plan.rank, plan.heads, plan.head_dim, plan.width);
}

}  // namespace

extern "C" {

int lsso_hip_mixer_forward(const lsso_hip_mixer_shape* shape, const void* projected,
                           const float* core_base_raw, const float* core_drive_weight,
                           const float* eta_raw, const float* inverse_frequency,
                           const float* centered_positions, int positions_mode,
                           const float* valid_counts, void* output, float* tape,
                           void* workspace, size_t workspace_bytes, void* stream_handle) {
    MixerPlan plan;
    int status = make_plan(shape, positions_mode, &plan);
    if (status != LSSO_HIP_OK) {
        return status;
    }
    MixerBuffers buf{};
    status = check_mixer_call(plan, projected, core_base_raw, core_drive_weight, eta_raw, output,
                              centered_positions, positions_mode, workspace, workspace_bytes, &buf);
    if (status != LSSO_HIP_OK) {
        return status;
    }
    hipStream_t stream = static_cast<hipStream_t>(stream_handle);
    const bool vec = vector_rows(plan, projected, output);
    status = run_compact(plan, buf, projected, core_base_raw, core_drive_weight, eta_raw,
                         inverse_frequency, centered_positions, positions_mode, valid_counts, tape,
                         vec, stream);
    if (status != LSSO_HIP_OK) {
        return status;
    }

    return run_apply(plan, buf, projected, eta_raw, positions_mode, output, vec, stream);
}

}  // extern "C"

// ---------------------------------------------------------------------------
// Allocation-free mixer forward.
//
// lsso_hip_mixer_forward_static runs lsso_hip_mixer_forward with the
// workspace in `scratch`, a device array of the library's own, so that a
// caller that cannot allocate device memory (code under HIP graph capture, a
// serving loop, a harness that forbids hipMalloc) passes only its inputs and
// outputs.  Each GPU holds its own copy of the array from the library's
// first use on it until the process ends.  In host code the name `scratch`
// is a host-side stand-in, not a device address: the array's address on a
// device comes from hipGetSymbolAddress, looked up once per device with that
// device current and kept in g_static_scratch, and only that address is
// handed to kernels.
//
// Every call on one GPU uses that GPU's single array, so two calls in flight
// at the same time on one GPU (on different streams) race; calls ordered on
// one stream do not.  Nothing in the array has to start at zero: every byte
// a call reads (phase table, G / S partials, Z, apply records) was written
// earlier in the same call.
namespace {

constexpr size_t kStaticScratchBytes = LSSO_HIP_STATIC_SCRATCH_BYTES;
constexpr int kStaticScratchDevices = 64;

}  // namespace

static __device__ __align__(256) unsigned char scratch[kStaticScratchBytes];

namespace {

std::mutex g_static_scratch_lock;
void* g_static_scratch[kStaticScratchDevices];

// Device address of `scratch` on the current device, which must be the
// stream's device: hipGetSymbolAddress answers for the current device only.
int static_scratch(hipStream_t stream, void** address) {
    int device = 0;
    hipError_t error = hipGetDevice(&device);
    if (error != hipSuccess) {
        return hip_failure(error, "hipGetDevice");
    }
    int stream_device = device;
    error = hipStreamGetDevice(stream, &stream_device);
    if (error != hipSuccess) {
        return hip_failure(error, "hipStreamGetDevice");
    }
    if (stream_device != device) {
        return fail(LSSO_HIP_EINVAL,
                    "the stream belongs to device " + std::to_string(stream_device) + " but device " +
                        std::to_string(device) +
                        " is current; make the stream's device current before calling "
                        "lsso_hip_mixer_forward_static");
    }
    if (device < 0 || device >= kStaticScratchDevices) {
        return fail(LSSO_HIP_EUNSUPPORTED,
                    "the static scratch serves devices 0.." +
                        std::to_string(kStaticScratchDevices - 1) + ", got device " +
                        std::to_string(device));
    }
    std::lock_guard<std::mutex> lock(g_static_scratch_lock);
    if (g_static_scratch[device] == nullptr) {
        void* pointer = nullptr;
        error = hipGetSymbolAddress(&pointer, HIP_SYMBOL(scratch));
        if (error != hipSuccess) {
            return hip_failure(error, "hipGetSymbolAddress(scratch)");
        }
        if (pointer == nullptr || !aligned(pointer, 256)) {
            return fail(LSSO_HIP_ERUNTIME, "the static scratch has no 256-byte aligned device address");
        }
        g_static_scratch[device] = pointer;
    }
    *address = g_static_scratch[device];
    return LSSO_HIP_OK;
}

}  // namespace

extern "C" {

int lsso_hip_mixer_forward_static(const lsso_hip_mixer_shape* shape, const void* projected,
                                  const float* core_base_raw, const float* core_drive_weight,
                                  const float* eta_raw, const float* inverse_frequency,
                                  const float* centered_positions, int positions_mode,
                                  const float* valid_counts, void* output, float* tape,
                                  void* stream_handle) {
    MixerPlan plan;
    int status = make_plan(shape, positions_mode, &plan);
    if (status != LSSO_HIP_OK) {
        return status;
    }
    if (plan.total > kStaticScratchBytes) {
        return fail(LSSO_HIP_EUNSUPPORTED,
                    "this geometry needs " + std::to_string(plan.total) +
                        " workspace bytes, more than the static scratch's " +
                        std::to_string(kStaticScratchBytes) +
                        "; use lsso_hip_mixer_forward with a caller workspace");
    }
    void* workspace = nullptr;
    status = static_scratch(static_cast<hipStream_t>(stream_handle), &workspace);
    if (status != LSSO_HIP_OK) {
        return status;
    }
    return lsso_hip_mixer_forward(shape, projected, core_base_raw, core_drive_weight, eta_raw,
                                  inverse_frequency, centered_positions, positions_mode,
                                  valid_counts, output, tape, workspace, kStaticScratchBytes,
                                  stream_handle);
}

int lsso_hip_mixer_projected_supported(const lsso_hip_mixer_shape* shape) {
    MixerPlan plan;
    const int status = make_plan(shape, LSSO_HIP_POSITIONS_DEFAULT, &plan);
    if (status != LSSO_HIP_OK) {
        return status;
    }
    return projected_shape_supported(plan) ? 1 : 0;
}

int lsso_hip_mixer_forward_projected(const lsso_hip_mixer_shape* shape, const void* projected,
                                     const float* core_base_raw, const float* core_drive_weight,
                                     const float* eta_raw, const float* inverse_frequency,
                                     const float* centered_positions, int positions_mode,
                                     const float* valid_counts, const float* out_weight,
                                     const float* out_bias, const uint8_t* row_mask, void* y,
                                     int y_dtype, void* workspace, size_t workspace_bytes,
                                     void* stream_handle) {
    MixerPlan plan;
    int status = make_plan(shape, positions_mode, &plan);
    if (status != LSSO_HIP_OK) {
        return status;
    }
    if (!projected_shape_supported(plan)) {
        return fail(LSSO_HIP_EUNSUPPORTED,
                    "the fused mixer + output projection supports heads <= 8, head_dim a multiple "
                    "of 16 up to 64, H*head_dim <= 256 and H*(rank+head_dim) <= 640; use "
                    "lsso_hip_mixer_forward followed by lsso_hip_linear");
    }
    if (y_dtype != LSSO_HIP_F16 && y_dtype != LSSO_HIP_BF16) {
        return fail(LSSO_HIP_EINVAL, "y_dtype must be LSSO_HIP_F16 or LSSO_HIP_BF16");
    }
    if (out_weight == nullptr) {
        return fail(LSSO_HIP_EINVAL, "out_weight must not be NULL");
    }
    MixerBuffers buf{};
    status = check_mixer_call(plan, projected, core_base_raw, core_drive_weight, eta_raw, y,
                              centered_positions, positions_mode, workspace, workspace_bytes, &buf);
    if (status != LSSO_HIP_OK) {
        return status;
    }
    if (!aligned(projected, 16) || !aligned(y, 16)) {
        return fail(LSSO_HIP_EINVAL, "the fused path needs 16-byte aligned projected and y buffers");
    }
    hipStream_t stream = static_cast<hipStream_t>(stream_handle);
    status = run_compact(plan, buf, projected, core_base_raw, core_drive_weight, eta_raw,
                         inverse_frequency, centered_positions, positions_mode, valid_counts,
                         nullptr, true, stream);
    if (status != LSSO_HIP_OK) {
        return status;
    }

    return run_mix_project(plan, buf, projected, eta_raw, positions_mode, out_weight, out_bias,
                           row_mask, y, y_dtype, stream);
}

}  // extern "C"

namespace {

constexpr int64_t kGradTargetGroups = 512;

struct GradColumnsPlan {
    int chunks_per_slab;
    int64_t slabs, splits, rows_per_split;
};

// Chunks of 8 columns are dealt to slabs of a power-of-two width (the largest
// that divides the chunk count, up to 64; else the smallest covering it), and
// rows to about 512 / slabs splits of at least eight passes each.
void plan_grad_columns(int64_t rows, int64_t cols, GradColumnsPlan* p) {
    const int64_t chunks = ceil_div(cols, 8);
    int cw = 1;
    while (cw < 64 && chunks % (2 * cw) == 0) {
        cw *= 2;
    }
    if (cw < 8) {
        cw = 1;
        while (cw < 64 && cw < chunks) {
            cw *= 2;
        }
    }
    p->chunks_per_slab = cw;
    p->slabs = ceil_div(chunks, cw);
    const int64_t row_lanes = 256 / cw;
    int64_t splits = ceil_div(kGradTargetGroups, p->slabs);
    const int64_t most = std::max<int64_t>(1, ceil_div(rows, row_lanes * 8));
    splits = std::min(splits, most);
    p->rows_per_split = std::max<int64_t>(1, ceil_div(rows, splits));
    p->splits = rows == 0 ? 0 : ceil_div(rows, p->rows_per_split);
}

struct BackwardPlan {
    int64_t record_stride, off_m, off_e, off_g, off_f;
    int feature_k32;
    size_t off_phases, off_partials, off_records, off_dtheta, off_ddrive, off_deta, off_dot;
    size_t off_columns, total;
};

int make_backward_plan(const MixerPlan& plan, BackwardPlan* bp) {
    if (!lsso_hip::backward_supported(plan.rank, plan.head_dim)) {
        return fail(LSSO_HIP_EUNSUPPORTED,
                    "the HIP mixer backward supports rank in {16, 32, 48, 64}, got " +
                        std::to_string(plan.rank));
    }
    bp->record_stride = lsso_hip::bwd_record_layout(plan.rank, plan.head_dim, &bp->off_m, &bp->off_e,
                                                    &bp->off_g, &bp->off_f, &bp->feature_k32);
    const int64_t systems = plan.batch * plan.heads;
    size_t offset = 0;
    bp->off_phases = offset;
    offset = align_up(offset + sizeof(uint32_t) * plan.phase_batches * plan.length * plan.pairs);
    bp->off_partials = offset;
    offset = align_up(offset + sizeof(float) * systems * plan.reduce_chunks * plan.partial_stride);
    bp->off_records = offset;
    offset = align_up(offset + sizeof(uint16_t) * systems * bp->record_stride);
    bp->off_dtheta = offset;
    offset = align_up(offset + sizeof(float) * systems * plan.rank * plan.rank);
    bp->off_ddrive = offset;
    offset = align_up(offset + sizeof(float) * systems * plan.head_dim * plan.rank);
    bp->off_deta = offset;
    offset = align_up(offset + sizeof(float) * systems);
    bp->off_dot = offset;
    offset = align_up(offset + sizeof(float) * systems * plan.apply_chunks);
    // Column-sum partials of grad_projected: one row per (sample, chunk) from
    // the token map, or one per split of the one-pass gradient kernel.
    bp->off_columns = offset;
    const int64_t column_rows = std::max<int64_t>(plan.batch * plan.apply_chunks, kGradTargetGroups);
    offset = align_up(offset + sizeof(float) * column_rows * plan.width);
    bp->total = offset;
    return LSSO_HIP_OK;
}

}  // namespace

extern "C" {

int lsso_hip_mixer_backward_workspace_bytes(const lsso_hip_mixer_shape* shape, int positions_mode,
                                            size_t* bytes) {
    if (bytes == nullptr) {
        return fail(LSSO_HIP_EINVAL, "bytes must not be NULL");
    }
    MixerPlan plan;
    int status = make_plan(shape, positions_mode, &plan);
    if (status != LSSO_HIP_OK) {
        return status;
    }
    BackwardPlan bp;
    status = make_backward_plan(plan, &bp);
    if (status != LSSO_HIP_OK) {
        return status;
    }
    *bytes = bp.total;
    return LSSO_HIP_OK;
}

int lsso_hip_mixer_backward(const lsso_hip_mixer_shape* shape, const void* grad_output,
                            const void* projected, const float* core_base_raw,
                            const float* core_drive_weight, const float* eta_raw,
                            const float* inverse_frequency, const float* centered_positions,
                            int positions_mode, const float* valid_counts, const float* tape,
                            void* grad_projected, float* grad_base, float* grad_drive,
                            float* grad_eta, void* workspace, size_t workspace_bytes,
                            void* stream_handle) {
    return lsso_hip_mixer_backward_ex(shape, grad_output, projected, core_base_raw,
                                      core_drive_weight, eta_raw, inverse_frequency,
                                      centered_positions, positions_mode, valid_counts, tape,
                                      grad_projected, grad_base, grad_drive, grad_eta, nullptr,
                                      workspace, workspace_bytes, stream_handle);
}

int lsso_hip_mixer_backward_ex(const lsso_hip_mixer_shape* shape, const void* grad_output,
                               const void* projected, const float* core_base_raw,
                               const float* core_drive_weight, const float* eta_raw,
                               const float* inverse_frequency, const float* centered_positions,
                               int positions_mode, const float* valid_counts, const float* tape,
                               void* grad_projected, float* grad_base, float* grad_drive,
                               float* grad_eta, float* grad_projected_column_sums,
                               void* workspace, size_t workspace_bytes, void* stream_handle) {
    (void)core_base_raw;  // Theta is read from the tape
    MixerPlan plan;
    int status = make_plan(shape, positions_mode, &plan);
    if (status != LSSO_HIP_OK) {
        return status;
    }
    BackwardPlan bp;
    status = make_backward_plan(plan, &bp);
    if (status != LSSO_HIP_OK) {
        return status;
    }
    if (grad_output == nullptr || projected == nullptr || core_drive_weight == nullptr ||
        eta_raw == nullptr || tape == nullptr || grad_projected == nullptr || grad_base == nullptr ||
        grad_drive == nullptr || grad_eta == nullptr) {
        return fail(LSSO_HIP_EINVAL, "backward tensors must not be NULL");
    }
    if (positions_mode != LSSO_HIP_POSITIONS_DEFAULT && centered_positions == nullptr) {
        return fail(LSSO_HIP_EINVAL, "centered_positions must not be NULL for this positions_mode");
    }
    if (workspace == nullptr || workspace_bytes < bp.total || !aligned(workspace, 256)) {
        return fail(LSSO_HIP_EINVAL,
                    "workspace must be 256-byte aligned and hold lsso_hip_mixer_backward_workspace_bytes()");
    }
    if (!aligned(grad_output, 4) || !aligned(projected, 4) || !aligned(grad_projected, 8)) {
        return fail(LSSO_HIP_EINVAL, "grad_output, projected and grad_projected must be aligned bfloat16 buffers");
    }
    hipStream_t stream = static_cast<hipStream_t>(stream_handle);
    char* ws = static_cast<char*>(workspace);
    uint32_t* phases = reinterpret_cast<uint32_t*>(ws + bp.off_phases);
    float* partials = reinterpret_cast<float*>(ws + bp.off_partials);
    uint16_t* records = reinterpret_cast<uint16_t*>(ws + bp.off_records);
    float* dtheta = reinterpret_cast<float*>(ws + bp.off_dtheta);
    float* ddrive = reinterpret_cast<float*>(ws + bp.off_ddrive);
    float* deta = reinterpret_cast<float*>(ws + bp.off_deta);
    float* dot = reinterpret_cast<float*>(ws + bp.off_dot);

    lsso_hip::PhaseArgs phase{};
    phase.positions = positions_mode == LSSO_HIP_POSITIONS_DEFAULT ? nullptr : centered_positions;
    phase.phases = phases;
    phase.count = plan.phase_batches * plan.length * plan.pairs;
    phase.length = plan.length;
    phase.pairs = static_cast<int>(plan.pairs);
    for (int j = 0; j < plan.pairs; ++j) {
        phase.inverse_frequency[j] = inverse_frequency != nullptr
            ? inverse_frequency[j]
            : std::pow(10000.0f, -static_cast<float>(j) / static_cast<float>(plan.pairs));
    }
    hipError_t error = lsso_hip::launch_phase(phase, stream);
    if (error != hipSuccess) {
        return hip_failure(error, "phase_kernel launch");
    }

    // dm partials: A^T dY per chunk through the forward's reduction.
    const bool vec = plan.width % 8 == 0 && plan.head_dim % 4 == 0 && aligned(projected, 16) &&
                     aligned(grad_output, 16);
    lsso_hip::ReduceArgs reduce{};
    reduce.projected = static_cast<const uint16_t*>(projected);
    reduce.content = static_cast<const uint16_t*>(grad_output);
    reduce.content_stride = plan.out_width;
    reduce.gram = 0;
    reduce.phases = phases;
    reduce.partials = partials;
    reduce.batch = plan.batch;
    reduce.length = plan.length;
    reduce.heads = plan.heads;
    reduce.head_dim = plan.head_dim;
    reduce.width = plan.width;
    reduce.phase_batch_stride = phase_batch_stride(plan, positions_mode);
    reduce.chunks = plan.reduce_chunks;
    reduce.chunk_tokens = plan.reduce_chunk_tokens;
    reduce.column_groups = plan.column_groups;
    reduce.partial_stride = plan.partial_stride;
    reduce.total_waves = plan.batch * plan.heads * plan.reduce_chunks * plan.column_groups;
    reduce.group_heads = plan.cpw == 1 ? lsso_hip::reduce_staged_group_heads(plan.rank, plan.heads, plan.head_dim,
                                                                              plan.column_groups, reduce.content_stride,
                                                                              vec && plan.head_dim % 8 == 0)
                                       : 0;
    error = lsso_hip::launch_reduce(static_cast<int>(plan.rank), reduce, plan.cpw, vec, stream);
    if (error != hipSuccess) {
        return hip_failure(error, "reduce_kernel launch (backward)");
    }

    lsso_hip::BwdSolveArgs solve{};
    solve.partials = partials;
    solve.chunks = plan.reduce_chunks;
    solve.partial_stride = plan.partial_stride;
    solve.tape = tape;
    solve.tape_stride = plan.tape_stride;
    solve.drive = core_drive_weight;
    solve.eta_raw = eta_raw;
    solve.valid_counts = valid_counts;
    solve.batch = plan.batch;
    solve.length = plan.length;
    solve.heads = plan.heads;
    solve.head_dim = plan.head_dim;
    solve.records = records;
    solve.record_stride = bp.record_stride;
    solve.off_m = bp.off_m;
    solve.off_e = bp.off_e;
    solve.off_g = bp.off_g;
    solve.off_f = bp.off_f;
    solve.feature_k32 = bp.feature_k32;
    solve.dtheta_part = dtheta;
    solve.ddrive_part = ddrive;
    solve.deta_part = deta;
    error = lsso_hip::launch_bwd_solve(static_cast<int>(plan.rank), solve, plan.batch * plan.heads,
                                       stream);
    if (error != hipSuccess) {
        return hip_failure(error, "bwd_solve_kernel launch");
    }

    lsso_hip::BwdApplyArgs apply{};
    apply.projected = static_cast<const uint16_t*>(projected);
    apply.grad_output = static_cast<const uint16_t*>(grad_output);
    apply.grad_stride = plan.out_width;
    apply.phases = phases;
    apply.phase_batch_stride = phase_batch_stride(plan, positions_mode);
    apply.records = records;
    apply.record_stride = bp.record_stride;
    apply.off_m = bp.off_m;
    apply.off_e = bp.off_e;
    apply.off_g = bp.off_g;
    apply.off_f = bp.off_f;
    apply.eta_raw = eta_raw;
    apply.grad_projected = static_cast<uint16_t*>(grad_projected);
    apply.dot_part = dot;
    float* column_part = reinterpret_cast<float*>(ws + bp.off_columns);
    apply.batch = plan.batch;
    apply.length = plan.length;
    apply.heads = plan.heads;
    apply.head_dim = plan.head_dim;
    apply.width = plan.width;
    apply.chunks = plan.apply_chunks;
    apply.chunk_tokens = plan.apply_chunk_tokens;
    apply.total_waves = plan.batch * plan.heads * plan.apply_chunks;
    // Whole 16-byte (K32) or 8-byte (K16) feature runs per lane.
    const bool bwd_vec = plan.head_dim % 8 == 0 && plan.width % 8 == 0 && aligned(projected, 16) &&
                         aligned(grad_output, 16) && aligned(grad_projected, 16);
    const bool fused_sums = grad_projected_column_sums != nullptr &&
                            lsso_hip::bwd_apply_resident(static_cast<int>(plan.rank), plan.head_dim, bwd_vec);
    apply.column_part = fused_sums ? column_part : nullptr;
    error = lsso_hip::launch_bwd_apply(static_cast<int>(plan.rank), apply, bp.feature_k32 != 0,
                                       bwd_vec, stream);
    if (error != hipSuccess) {
        return hip_failure(error, "bwd_apply_kernel launch");
    }
    if (fused_sums) {
        error = lsso_hip::launch_column_sum(column_part, plan.batch * plan.apply_chunks, plan.width,
                                            grad_projected_column_sums, stream);
        if (error != hipSuccess) {
            return hip_failure(error, "column_sum_kernel launch");
        }
    } else if (grad_projected_column_sums != nullptr) {
        // The general token map: one read of grad_projected for its sums.
        GradColumnsPlan gp;
        plan_grad_columns(plan.batch * plan.length, plan.width, &gp);
        lsso_hip::GradColumnsArgs ga{};
        ga.g = grad_projected;
        ga.rows = plan.batch * plan.length;
        ga.cols = plan.width;
        ga.g_stride = plan.width;
        ga.partials = column_part;
        ga.rows_per_split = gp.rows_per_split;
        ga.chunks_per_slab = gp.chunks_per_slab;
        const bool vec = plan.width % 8 == 0 && aligned(grad_projected, 16);
        error = lsso_hip::launch_grad_columns(ga, LSSO_HIP_BF16, vec, gp.splits, gp.slabs,
                                              grad_projected_column_sums, stream);
        if (error != hipSuccess) {
            return hip_failure(error, "grad_columns_kernel launch (backward)");
        }
    }

    lsso_hip::ParamReduceArgs params{};
    params.dtheta_part = dtheta;
    params.ddrive_part = ddrive;
    params.deta_part = deta;
    params.dot_part = dot;
    params.eta_raw = eta_raw;
    params.grad_base = grad_base;
    params.grad_drive = grad_drive;
    params.grad_eta = grad_eta;
    params.batch = plan.batch;
    params.heads = plan.heads;
    params.rank = plan.rank;
    params.head_dim = plan.head_dim;
    params.chunks = plan.apply_chunks;
    error = lsso_hip::launch_param_reduce(params, stream);
    if (error != hipSuccess) {
        return hip_failure(error, "param_reduce_kernel launch");
    }
    return LSSO_HIP_OK;
}

}  // extern "C"

namespace {

}  // namespace

extern "C" {

int lsso_hip_linear_grad_columns_workspace_bytes(int64_t rows, int64_t cols, size_t* bytes) {
    if (bytes == nullptr) {
        return fail(LSSO_HIP_EINVAL, "bytes must not be NULL");
    }
    if (rows < 0 || cols <= 0) {
        return fail(LSSO_HIP_EINVAL, "rows must be >= 0 and cols must be positive");
    }
    GradColumnsPlan plan;
    plan_grad_columns(rows, cols, &plan);
    *bytes = align_up(sizeof(float) * plan.splits * cols);
    return LSSO_HIP_OK;
}

int lsso_hip_linear_grad_columns(const void* g, int g_dtype, int64_t rows, int64_t cols,
                                 int64_t g_row_stride, const uint8_t* row_mask, void* g_bf16,
                                 float* column_sums, void* workspace, size_t workspace_bytes,
                                 void* stream_handle) {
    if (rows < 0 || cols <= 0) {
        return fail(LSSO_HIP_EINVAL, "rows must be >= 0 and cols must be positive");
    }
    if (g_dtype != LSSO_HIP_F16 && g_dtype != LSSO_HIP_BF16) {
        return fail(LSSO_HIP_EUNSUPPORTED, "the gradient dtype must be float16 or bfloat16");
    }
    if (g_row_stride < cols) {
        return fail(LSSO_HIP_EINVAL, "g_row_stride must be >= cols");
    }
    if (g_bf16 == nullptr && column_sums == nullptr) {
        return LSSO_HIP_OK;
    }
    if (rows > 0 && g == nullptr) {
        return fail(LSSO_HIP_EINVAL, "g must not be NULL");
    }
    if (!aligned(g, 2) || !aligned(g_bf16, 2) || !aligned(column_sums, 4)) {
        return fail(LSSO_HIP_EINVAL, "g, g_bf16 and column_sums must be aligned to their element size");
    }
    GradColumnsPlan plan;
    plan_grad_columns(rows, cols, &plan);
    const size_t needed = column_sums == nullptr ? 0 : align_up(sizeof(float) * plan.splits * cols);
    if (needed > 0 && (workspace == nullptr || workspace_bytes < needed || !aligned(workspace, 16))) {
        return fail(LSSO_HIP_EINVAL, "workspace must be 16-byte aligned and hold " +
                                         std::to_string(needed) + " bytes");
    }
    lsso_hip::GradColumnsArgs args{};
    args.g = g;
    args.rows = rows;
    args.cols = cols;
    args.g_stride = g_row_stride;
    args.row_mask = row_mask;
    args.g_bf16 = static_cast<uint16_t*>(g_bf16);
    args.partials = column_sums == nullptr ? nullptr : static_cast<float*>(workspace);
    args.rows_per_split = plan.rows_per_split;
    args.chunks_per_slab = plan.chunks_per_slab;
    const bool vec = cols % 8 == 0 && g_row_stride % 8 == 0 && aligned(g, 16) && aligned(g_bf16, 16);
    const hipError_t error = lsso_hip::launch_grad_columns(
        args, g_dtype, vec, plan.splits, plan.slabs, column_sums,
        static_cast<hipStream_t>(stream_handle));
    if (error != hipSuccess) {
        return hip_failure(error, "grad_columns_kernel launch");
    }
    return LSSO_HIP_OK;
}

int lsso_hip_linear_workspace_bytes(int64_t rows, int64_t in_features, int64_t out_features,
                                    size_t* bytes) {
    if (bytes == nullptr) {
        return fail(LSSO_HIP_EINVAL, "bytes must not be NULL");
    }
    if (rows < 0 || in_features <= 0 || out_features <= 0) {
        return fail(LSSO_HIP_EINVAL, "rows must be >= 0 and features must be positive");
    }
    *bytes = 0;
    return LSSO_HIP_OK;
}

int lsso_hip_linear(const void* x, int x_dtype, int64_t rows, int64_t in_features,
                    int64_t x_row_stride, const float* weight, const float* bias,
                    const uint8_t* row_mask, int64_t out_features, void* y, int y_dtype,
                    void* workspace, size_t workspace_bytes, void* stream_handle) {
    (void)workspace;
    (void)workspace_bytes;
    if (rows < 0 || in_features <= 0 || out_features <= 0) {
        return fail(LSSO_HIP_EINVAL, "rows must be >= 0 and features must be positive");
    }
    if ((x_dtype != LSSO_HIP_F16 && x_dtype != LSSO_HIP_BF16) ||
        (y_dtype != LSSO_HIP_F16 && y_dtype != LSSO_HIP_BF16)) {
        return fail(LSSO_HIP_EUNSUPPORTED, "projection dtypes must be float16 or bfloat16");
    }
    if (x_row_stride < in_features) {
        return fail(LSSO_HIP_EINVAL, "x_row_stride must be >= in_features");
    }
    if (rows == 0) {
        return LSSO_HIP_OK;
    }
    if (x == nullptr || weight == nullptr || y == nullptr) {
        return fail(LSSO_HIP_EINVAL, "x, weight and y must not be NULL");
    }
    return run_linear(x, x_dtype, rows, in_features, x_row_stride, weight, bias, row_mask,
                      out_features, y, y_dtype, static_cast<hipStream_t>(stream_handle));
}

}  // extern "C"

namespace {

struct WeightGradPlan {
    int64_t splits, rows_per_split;
    size_t off_bias, total;
};

void make_weight_grad_plan(int64_t rows, int64_t in_features, int64_t out_features,
                           WeightGradPlan* p) {
    lsso_hip::plan_weight_grad(rows, in_features, out_features, &p->splits, &p->rows_per_split);
    p->off_bias = align_up(sizeof(float) * p->splits * out_features * in_features);
    p->total = align_up(p->off_bias + sizeof(float) * p->splits * out_features);
}

}  // namespace

extern "C" {

int lsso_hip_linear_weight_grad_workspace_bytes(int64_t rows, int64_t in_features,
                                                int64_t out_features, size_t* bytes) {
    if (bytes == nullptr) {
        return fail(LSSO_HIP_EINVAL, "bytes must not be NULL");
    }
    if (rows < 0 || in_features <= 0 || out_features <= 0) {
        return fail(LSSO_HIP_EINVAL, "rows must be >= 0 and features must be positive");
    }
    WeightGradPlan plan;
    make_weight_grad_plan(rows, in_features, out_features, &plan);
    *bytes = plan.total;
    return LSSO_HIP_OK;
}

int lsso_hip_linear_weight_grad(const void* g, int g_dtype, int64_t g_row_stride, const void* x,
                                int x_dtype, int64_t x_row_stride, int64_t rows,
                                int64_t in_features, int64_t out_features,
                                const uint8_t* row_mask, float* grad_weight, float* grad_bias,
                                void* workspace, size_t workspace_bytes, void* stream_handle) {
    if (rows < 0 || in_features <= 0 || out_features <= 0) {
        return fail(LSSO_HIP_EINVAL, "rows must be >= 0 and features must be positive");
    }
    if ((g_dtype != LSSO_HIP_F16 && g_dtype != LSSO_HIP_BF16) ||
        (x_dtype != LSSO_HIP_F16 && x_dtype != LSSO_HIP_BF16)) {
        return fail(LSSO_HIP_EUNSUPPORTED, "the gradient and activation dtypes must be float16 or bfloat16");
    }
    if (g_row_stride < out_features || x_row_stride < in_features) {
        return fail(LSSO_HIP_EINVAL, "g_row_stride must be >= out_features and x_row_stride >= in_features");
    }
    if (grad_weight == nullptr) {
        return fail(LSSO_HIP_EINVAL, "grad_weight must not be NULL");
    }
    if (rows > 0 && (g == nullptr || x == nullptr)) {
        return fail(LSSO_HIP_EINVAL, "g and x must not be NULL");
    }
    if (!aligned(g, 2) || !aligned(x, 2) || !aligned(grad_weight, 4) || !aligned(grad_bias, 4)) {
        return fail(LSSO_HIP_EINVAL, "g, x, grad_weight and grad_bias must be aligned to their element size");
    }
    WeightGradPlan plan;
    make_weight_grad_plan(rows, in_features, out_features, &plan);
    if (workspace == nullptr || workspace_bytes < plan.total || !aligned(workspace, 256)) {
        return fail(LSSO_HIP_EINVAL, "workspace must be 256-byte aligned and hold " +
                                         std::to_string(plan.total) + " bytes");
    }
    hipStream_t stream = static_cast<hipStream_t>(stream_handle);
    float* partials = static_cast<float*>(workspace);
    float* bias_partials = reinterpret_cast<float*>(static_cast<char*>(workspace) + plan.off_bias);
    lsso_hip::WeightGradArgs args{};
    args.g = g;
    args.g_stride = g_row_stride;
    args.x = x;
    args.x_stride = x_row_stride;
    args.row_mask = row_mask;
    args.rows = rows;
    args.out_features = out_features;
    args.in_features = in_features;
    args.partials = partials;
    args.bias_partials = grad_bias != nullptr ? bias_partials : nullptr;
    args.rows_per_split = plan.rows_per_split;
    args.splits = plan.splits;
    args.tiles_n = ceil_div(out_features, lsso_hip::weight_grad_tile());
    args.tiles_k = ceil_div(in_features, lsso_hip::weight_grad_tile());
    args.vec = (out_features % 8 == 0 && in_features % 8 == 0 && g_row_stride % 8 == 0 &&
                x_row_stride % 8 == 0 && aligned(g, 16) && aligned(x, 16)) ? 1 : 0;
    hipError_t error = lsso_hip::launch_weight_grad(args, g_dtype, x_dtype, stream);
    if (error != hipSuccess) {
        return hip_failure(error, "weight_grad_kernel launch");
    }
    // The weight's and the bias's split partials are summed in one launch.
    error = lsso_hip::launch_column_sums(partials, out_features * in_features, grad_weight,
                                         grad_bias != nullptr ? bias_partials : nullptr,
                                         grad_bias != nullptr ? out_features : 0, grad_bias, plan.splits,
                                         stream);
    if (error != hipSuccess) {
        return hip_failure(error, "column_sum_kernel launch (weight and bias gradients)");
    }
    return LSSO_HIP_OK;
}

}  // extern "C"

namespace {

// The whole-layer forward: x -> (projection + reductions) -> solve ->
// (apply + output projection) -> y.  Returns the heads per projection group,
// or 0 when the geometry is outside the fused projection + reduce envelope.
int layer_group_heads(const MixerPlan& plan) {
    return lsso_hip::project_reduce_group_heads(plan.rank, plan.heads, plan.head_dim,
                                                plan.out_width);
}

struct LayerPlan {
    size_t off_packed, off_mixed, total;
    bool fused_out;
};

void make_layer_plan(const MixerPlan& plan, LayerPlan* lp) {
    size_t offset = plan.total;
    lp->off_packed = offset;
    offset = align_up(offset + sizeof(uint16_t) * plan.batch * plan.length * plan.width);
    lp->fused_out = projected_shape_supported(plan);
    lp->off_mixed = offset;
    if (!lp->fused_out) {
        offset = align_up(offset + sizeof(uint16_t) * plan.batch * plan.length * plan.out_width);
    }
    lp->total = offset;
}

int layer_forward_impl(const lsso_hip_mixer_shape* shape, const void* x, int x_dtype,
                       const float* in_weight, const float* in_bias, const uint8_t* row_mask,
                       const float* core_base_raw, const float* core_drive_weight,
                       const float* eta_raw, const float* inverse_frequency,
                       const float* centered_positions, int positions_mode,
                       const float* valid_counts, const float* out_weight, const float* out_bias,
                       void* y, int y_dtype, void* workspace, size_t workspace_bytes,
                       void* stream_handle, void* const* events);
int run_project_reduce(const MixerPlan& plan, const MixerBuffers& buf, const void* x, int x_dtype,
                       const float* in_weight, const float* in_bias, const uint8_t* row_mask,
                       void* packed, int positions_mode, int group_heads, hipStream_t stream);

}  // namespace

namespace {

// Input projection + mixer with the tape (lsso_hip_project_mix_forward) and,
// when out_weight is set, the output projection into y: fused with the apply
// (which then also stores mixed) inside the fused readout's envelope, else
// lsso_hip_linear over mixed.
int project_mix_impl(const lsso_hip_mixer_shape* shape, const void* x, int x_dtype,
                     const float* in_weight, const float* in_bias, const uint8_t* row_mask,
                     const float* core_base_raw, const float* core_drive_weight,
                     const float* eta_raw, const float* inverse_frequency,
                     const float* centered_positions, int positions_mode,
                     const float* valid_counts, const float* out_weight, const float* out_bias,
                     void* packed, void* mixed, float* tape, void* y, int y_dtype, void* workspace,
                     size_t workspace_bytes, void* stream_handle) {
    MixerPlan plan;
    int status = make_plan(shape, positions_mode, &plan);
    if (status != LSSO_HIP_OK) {
        return status;
    }
    const int group_heads = layer_group_heads(plan);
    if (group_heads == 0) {
        return fail(LSSO_HIP_EUNSUPPORTED,
                    "the fused projection + mixer supports head_dim a multiple of 16 up to 64 and "
                    "H*head_dim <= 384; use lsso_hip_linear and lsso_hip_mixer_forward");
    }
    if (x_dtype != LSSO_HIP_F16 && x_dtype != LSSO_HIP_BF16) {
        return fail(LSSO_HIP_EINVAL, "x_dtype must be LSSO_HIP_F16 or LSSO_HIP_BF16");
    }
    if (x == nullptr || in_weight == nullptr) {
        return fail(LSSO_HIP_EINVAL, "x and in_weight must not be NULL");
    }
    if (!aligned(x, 16) || !aligned(packed, 16)) {
        return fail(LSSO_HIP_EINVAL, "x and packed must be 16-byte aligned");
    }
    MixerBuffers buf{};
    status = check_mixer_call(plan, packed, core_base_raw, core_drive_weight, eta_raw, mixed,
                              centered_positions, positions_mode, workspace, workspace_bytes, &buf);
    if (status != LSSO_HIP_OK) {
        return status;
    }
    hipStream_t stream = static_cast<hipStream_t>(stream_handle);
    status = run_phase(plan, buf, inverse_frequency, centered_positions, positions_mode, stream);
    if (status != LSSO_HIP_OK) {
        return status;
    }
    status = run_project_reduce(plan, buf, x, x_dtype, in_weight, in_bias, row_mask, packed,
                                positions_mode, group_heads, stream);
    if (status != LSSO_HIP_OK) {
        return status;
    }
    status = run_solve(plan, buf, core_base_raw, core_drive_weight, eta_raw, valid_counts, tape,
                       stream);
    if (status != LSSO_HIP_OK) {
        return status;
    }
    if (out_weight == nullptr) {
        return run_apply(plan, buf, packed, eta_raw, positions_mode, mixed,
                         vector_rows(plan, packed, mixed), stream);
    }
    if (projected_shape_supported(plan)) {
        return run_mix_project(plan, buf, packed, eta_raw, positions_mode, out_weight, out_bias,
                               row_mask, y, y_dtype, stream, mixed);
    }
    status = run_apply(plan, buf, packed, eta_raw, positions_mode, mixed,
                       vector_rows(plan, packed, mixed), stream);
    if (status != LSSO_HIP_OK) {
        return status;
    }
    return run_linear(mixed, LSSO_HIP_BF16, plan.batch * plan.length, plan.out_width,
                      plan.out_width, out_weight, out_bias, row_mask, plan.out_width, y, y_dtype,
                      stream);
}


}  // namespace

extern "C" {

int lsso_hip_layer_supported(const lsso_hip_mixer_shape* shape) {
    MixerPlan plan;
    const int status = make_plan(shape, LSSO_HIP_POSITIONS_DEFAULT, &plan);
    if (status != LSSO_HIP_OK) {
        return status;
    }
    return layer_group_heads(plan) > 0 ? 1 : 0;
}

int lsso_hip_layer_workspace_bytes(const lsso_hip_mixer_shape* shape, int positions_mode,
                                   size_t* bytes) {
    if (bytes == nullptr) {
        return fail(LSSO_HIP_EINVAL, "bytes must not be NULL");
    }
    MixerPlan plan;
    const int status = make_plan(shape, positions_mode, &plan);
    if (status != LSSO_HIP_OK) {
        return status;
    }
    LayerPlan lp;
    make_layer_plan(plan, &lp);
    *bytes = lp.total;
    return LSSO_HIP_OK;
}

int lsso_hip_layer_forward(const lsso_hip_mixer_shape* shape, const void* x, int x_dtype,
                           const float* in_weight, const float* in_bias, const uint8_t* row_mask,
                           const float* core_base_raw, const float* core_drive_weight,
                           const float* eta_raw, const float* inverse_frequency,
                           const float* centered_positions, int positions_mode,
                           const float* valid_counts, const float* out_weight,
                           const float* out_bias, void* y, int y_dtype, void* workspace,
                           size_t workspace_bytes, void* stream_handle) {
    return layer_forward_impl(shape, x, x_dtype, in_weight, in_bias, row_mask, core_base_raw,
                              core_drive_weight, eta_raw, inverse_frequency, centered_positions,
                              positions_mode, valid_counts, out_weight, out_bias, y, y_dtype,
                              workspace, workspace_bytes, stream_handle, nullptr);
}

int lsso_hip_layer_forward_timed(const lsso_hip_mixer_shape* shape, const void* x, int x_dtype,
                                 const float* in_weight, const float* in_bias,
                                 const uint8_t* row_mask, const float* core_base_raw,
                                 const float* core_drive_weight, const float* eta_raw,
                                 const float* inverse_frequency, const float* centered_positions,
                                 int positions_mode, const float* valid_counts,
                                 const float* out_weight, const float* out_bias, void* y,
                                 int y_dtype, void* workspace, size_t workspace_bytes,
                                 void* stream_handle, void* const* events) {
    if (events == nullptr) {
        return fail(LSSO_HIP_EINVAL, "events must not be NULL");
    }
    return layer_forward_impl(shape, x, x_dtype, in_weight, in_bias, row_mask, core_base_raw,
                              core_drive_weight, eta_raw, inverse_frequency, centered_positions,
                              positions_mode, valid_counts, out_weight, out_bias, y, y_dtype,
                              workspace, workspace_bytes, stream_handle, events);
}

int lsso_hip_project_mix_forward(const lsso_hip_mixer_shape* shape, const void* x, int x_dtype,
                                 const float* in_weight, const float* in_bias,
                                 const uint8_t* row_mask, const float* core_base_raw,
                                 const float* core_drive_weight, const float* eta_raw,
                                 const float* inverse_frequency, const float* centered_positions,
                                 int positions_mode, const float* valid_counts, void* packed,
                                 void* mixed, float* tape, void* workspace, size_t workspace_bytes,
                                 void* stream_handle) {
    return project_mix_impl(shape, x, x_dtype, in_weight, in_bias, row_mask, core_base_raw,
                            core_drive_weight, eta_raw, inverse_frequency, centered_positions,
                            positions_mode, valid_counts, nullptr, nullptr, packed, mixed, tape,
                            nullptr, 0, workspace, workspace_bytes, stream_handle);
}

int lsso_hip_layer_forward_train(const lsso_hip_mixer_shape* shape, const void* x, int x_dtype,
                                 const float* in_weight, const float* in_bias,
                                 const uint8_t* row_mask, const float* core_base_raw,
                                 const float* core_drive_weight, const float* eta_raw,
                                 const float* inverse_frequency, const float* centered_positions,
                                 int positions_mode, const float* valid_counts,
                                 const float* out_weight, const float* out_bias, void* packed,
                                 void* mixed, float* tape, void* y, int y_dtype, void* workspace,
                                 size_t workspace_bytes, void* stream_handle) {
    if (out_weight == nullptr || y == nullptr || mixed == nullptr) {
        return fail(LSSO_HIP_EINVAL, "out_weight, mixed and y must not be NULL");
    }
    if (y_dtype != LSSO_HIP_F16 && y_dtype != LSSO_HIP_BF16) {
        return fail(LSSO_HIP_EINVAL, "y_dtype must be LSSO_HIP_F16 or LSSO_HIP_BF16");
    }
    if (!aligned(y, 16) || !aligned(mixed, 16)) {
        return fail(LSSO_HIP_EINVAL, "y and mixed must be 16-byte aligned");
    }
    return project_mix_impl(shape, x, x_dtype, in_weight, in_bias, row_mask, core_base_raw,
                            core_drive_weight, eta_raw, inverse_frequency, centered_positions,
                            positions_mode, valid_counts, out_weight, out_bias, packed, mixed, tape,
                            y, y_dtype, workspace, workspace_bytes, stream_handle);
}

}  // extern "C"

namespace {

// The fused projection + reduce reads x once per head group and runs one
// head's reductions per wave beside the projection.  From rank 48 on the
// separate projection and staged reduce are faster: a group holds three heads
// (one reduction wave idle) and each head's reduction, with two pair slots per
// lane, sets the tile's pace.  Measured on one MI355X with the spill-free
// rank-48/64 kernels: at B = 64, N = 2048, H = 8, r = 48, d = 32 (the
// training forward) 146.5 us fused against 75.3 + 53.5 us for the projection
// and the staged reduce; at B = 32, N = 4096, H = 6, r = 64, D = 384 the stage
// took 284.7 us fused against 169.6 us.
//
// LSSO_HIP_FUSED_PROJECTION overrides the rule for A/B measurements and
// tests: "1" fuses at every rank the fused kernel supports, "0" never fuses.
// Either way the results are the same bits.
bool fused_projection_pays(const MixerPlan& plan) {
    const char* mode = std::getenv("LSSO_HIP_FUSED_PROJECTION");
    if (mode != nullptr && mode[0] == '1' && mode[1] == '\0') {
        return true;
    }
    if (mode != nullptr && mode[0] == '0' && mode[1] == '\0') {
        return false;
    }
    return plan.rank <= 32;
}

// The input projection and the token reductions: writes `packed` (bitwise
// lsso_hip_linear's output) and the reduce partials of buf (bitwise
// reduce_kernel's), fused in one kernel where that pays.
int run_project_reduce(const MixerPlan& plan, const MixerBuffers& buf, const void* x, int x_dtype,
                       const float* in_weight, const float* in_bias, const uint8_t* row_mask,
                       void* packed, int positions_mode, int group_heads, hipStream_t stream) {
    if (!fused_projection_pays(plan)) {
        const int status = run_linear(x, x_dtype, plan.batch * plan.length, plan.out_width,
                                      plan.out_width, in_weight, in_bias, row_mask, plan.width,
                                      packed, LSSO_HIP_BF16, stream);
        if (status != LSSO_HIP_OK) {
            return status;
        }
        return run_reduce(plan, buf, packed, positions_mode, vector_rows(plan, packed, packed),
                          stream);
    }
    int units = 0;
    const int status = compute_units(&units);
    if (status != LSSO_HIP_OK) {
        return status;
    }
    lsso_hip::ProjectReduceArgs pr{};
    pr.x = x;
    pr.weight = in_weight;
    pr.bias = in_bias;
    pr.row_mask = row_mask;
    pr.phases = buf.phases;
    pr.phase_batch_stride = phase_batch_stride(plan, positions_mode);
    pr.packed = static_cast<uint16_t*>(packed);
    pr.partials = buf.partials;
    pr.batch = plan.batch;
    pr.length = plan.length;
    pr.heads = plan.heads;
    pr.head_dim = plan.head_dim;
    pr.in_features = plan.out_width;
    pr.width = plan.width;
    pr.chunks = plan.reduce_chunks;
    pr.chunk_tokens = plan.reduce_chunk_tokens;
    pr.partial_stride = plan.partial_stride;
    pr.group_heads = group_heads;
    pr.head_groups = ceil_div(plan.heads, group_heads);
    // One persistent workgroup per compute unit; the blocks of the head
    // groups of one item are dealt to the same XCD when the count allows.
    const int64_t items = plan.batch * plan.reduce_chunks;
    int64_t per_group = units / pr.head_groups;
    if (per_group < 1) per_group = 1;
    if (per_group > items) per_group = items;
    if (per_group >= 8) per_group -= per_group % 8;
    const hipError_t error = lsso_hip::launch_project_reduce(
        static_cast<int>(plan.rank), pr, x_dtype, static_cast<int>(per_group * pr.head_groups),
        stream);
    return error == hipSuccess ? LSSO_HIP_OK : hip_failure(error, "project_reduce_kernel launch");
}

int layer_forward_impl(const lsso_hip_mixer_shape* shape, const void* x, int x_dtype,
                       const float* in_weight, const float* in_bias, const uint8_t* row_mask,
                       const float* core_base_raw, const float* core_drive_weight,
                       const float* eta_raw, const float* inverse_frequency,
                       const float* centered_positions, int positions_mode,
                       const float* valid_counts, const float* out_weight, const float* out_bias,
                       void* y, int y_dtype, void* workspace, size_t workspace_bytes,
                       void* stream_handle, void* const* events) {
    MixerPlan plan;
    int status = make_plan(shape, positions_mode, &plan);
    if (status != LSSO_HIP_OK) {
        return status;
    }
    const int group_heads = layer_group_heads(plan);
    if (group_heads == 0) {
        return fail(LSSO_HIP_EUNSUPPORTED,
                    "the fused layer forward supports head_dim a multiple of 16 up to 64 and "
                    "H*head_dim <= 384; use lsso_hip_linear and lsso_hip_mixer_forward");
    }
    if ((x_dtype != LSSO_HIP_F16 && x_dtype != LSSO_HIP_BF16) ||
        (y_dtype != LSSO_HIP_F16 && y_dtype != LSSO_HIP_BF16)) {
        return fail(LSSO_HIP_EINVAL, "x_dtype and y_dtype must be LSSO_HIP_F16 or LSSO_HIP_BF16");
    }
    if (x == nullptr || in_weight == nullptr || out_weight == nullptr) {
        return fail(LSSO_HIP_EINVAL, "x, in_weight and out_weight must not be NULL");
    }
    if (!aligned(x, 16)) {
        return fail(LSSO_HIP_EINVAL, "x must be 16-byte aligned");
    }
    LayerPlan lp;
    make_layer_plan(plan, &lp);
    if (workspace == nullptr || workspace_bytes < lp.total) {
        return fail(LSSO_HIP_EINVAL, "workspace is smaller than lsso_hip_layer_workspace_bytes()");
    }
    MixerBuffers buf{};
    void* packed = static_cast<char*>(workspace) + lp.off_packed;
    status = check_mixer_call(plan, packed, core_base_raw, core_drive_weight, eta_raw, y,
                              centered_positions, positions_mode, workspace, plan.total, &buf);
    if (status != LSSO_HIP_OK) {
        return status;
    }
    if (!aligned(y, 16)) {
        return fail(LSSO_HIP_EINVAL, "y must be 16-byte aligned");
    }
    hipStream_t stream = static_cast<hipStream_t>(stream_handle);
    // Optional timing: events[2 k] and events[2 k + 1] take the begin of the
    // first and the end of the last kernel of stage k (0 phase table,
    // 1 projection + reductions, 2 compact solve, 3 apply + output
    // projection), recorded by the dispatches themselves; NULL entries are
    // skipped.  The guard clears them on every return.
    struct StageEvents {
        void* const* events;
        void set(int stage) const {
            lsso_hip::DispatchEvents& d = lsso_hip::dispatch_events();
            d.start = events != nullptr ? static_cast<hipEvent_t>(events[2 * stage]) : nullptr;
            d.stop = events != nullptr ? static_cast<hipEvent_t>(events[2 * stage + 1]) : nullptr;
        }
        ~StageEvents() { lsso_hip::dispatch_events() = lsso_hip::DispatchEvents{}; }
    } stage{events};
    stage.set(0);
    status = run_phase(plan, buf, inverse_frequency, centered_positions, positions_mode, stream);
    if (status != LSSO_HIP_OK) {
        return status;
    }
    stage.set(1);
    status = run_project_reduce(plan, buf, x, x_dtype, in_weight, in_bias, row_mask, packed,
                                positions_mode, group_heads, stream);
    if (status != LSSO_HIP_OK) {
        return status;
    }
    stage.set(2);
    status = run_solve(plan, buf, core_base_raw, core_drive_weight, eta_raw, valid_counts, nullptr,
                       stream);
    if (status != LSSO_HIP_OK) {
        return status;
    }
    stage.set(3);
    if (lp.fused_out) {
        status = run_mix_project(plan, buf, packed, eta_raw, positions_mode, out_weight, out_bias,
                                 row_mask, y, y_dtype, stream);
    } else {
        void* mixed = static_cast<char*>(workspace) + lp.off_mixed;
        status = run_apply(plan, buf, packed, eta_raw, positions_mode, mixed, true, stream);
        if (status == LSSO_HIP_OK) {
            status = run_linear(mixed, LSSO_HIP_BF16, plan.batch * plan.length, plan.out_width,
                                plan.out_width, out_weight, out_bias, row_mask, plan.out_width, y,
                                y_dtype, stream);
        }
    }
    return status;
}

}  // namespace

// gfx950 kernels of the DYNAMIC + Rank-Rotary LSSO mixer.
//
// Algebra (per sample b, head h; reference lsso/ball/reference.py:411-572,
// lsso/ball/model.py:245-268, 407-496): with A = rot(R) / sqrt(n) and C the
// content,  P = qr_soft_frame(A) = A L^-T where L L^T = A^T A + I (the QR of
// [A/s; I/s] has R_qr = L^T / s, so the detached scale s cancels).  Hence
//   Z = P^T C = L^-1 S,            S = A^T C,  G = A^T A
//   Theta = Theta0 + Z W_drive / sqrt(n),  K = F F^T + Omega
//   U = (I + K)^-1 Z,  X = 2U - (1 + eta) Z
//   Y = eta C + P X = eta C + rot(R) M',  M' = L^-T X / sqrt(n).
// The token-sized frame P is never formed.  The mixer is two streaming passes
// over `projected` (reduce: G and S; apply: Y) around one compact solve per
// (b, h).
//
// Kernels:
//   phase_kernel   FP16 (cos, sin) table, FP32 angle = p * inv_freq
//                  (reference.py:704-715)
//   reduce_kernel  G = sum rot(R)^T rot(R), S = sum rot(R)^T C over a token
//                  chunk; BF16 hi/lo split operands on 16x16x32 MFMA
//   solve_kernel   Cholesky, triangular solves, Theta/F/K assembly, partial
//                  pivot LU of I + K, M' in the apply operand layout
//   apply_kernel   Y^T = M'^T rot(R)^T + eta C^T on MFMA, BF16 store

#include "lsso_device.h"
#include "lsso_internal.h"
#include "lsso_reduce.h"

namespace lsso_hip {

// ---------------------------------------------------------------------------
// Phase table: one thread per (position, 4 consecutive pairs), 32-bit
// indices and a compile-time pair count, so the index split is a multiply
// (a 64-bit division per entry cost more than the sines) and each thread
// writes one 16-byte piece.
template <int PAIRS>
__global__ __launch_bounds__(256) void phase_kernel(PhaseArgs a) {
    constexpr uint32_t kQuads = PAIRS / 4;
    const uint32_t index = blockIdx.x * 256u + threadIdx.x;
    if (index >= static_cast<uint32_t>(a.count / 4)) {
        return;
    }
    const uint32_t position_index = index / kQuads;
    const int quad = static_cast<int>(index - position_index * kQuads);
    const float position = a.positions != nullptr
        ? a.positions[position_index]
        : static_cast<float>(position_index) - 0.5f * static_cast<float>(a.length - 1);
    u32x4 out;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const float angle = position * a.inverse_frequency[4 * quad + e];
        float sine;
        float cosine;
        sincosf(angle, &sine, &cosine);
        out[e] = pack_f16(cosine, sine);
    }
    *reinterpret_cast<u32x4*>(a.phases + 4 * static_cast<uint64_t>(index)) = out;
}

// ---------------------------------------------------------------------------
// Reduce.
template <int R, int CPW, bool VEC>
__global__ __launch_bounds__(256, 2) void reduce_kernel(ReduceArgs a) {
    using L = ReduceLayout<R>;
    constexpr int NRB = L::kRowBlocks;
    constexpr int NGB = L::kGramBlocks;
    const int lane = threadIdx.x & 63;
    // Wave-uniform, so the work item and the buffer bases below are scalar.
    // (Renumbering the workgroups of one (sample, chunk) onto one XCD, as
    // the apply does, measured slower here: 97.7 against 91.3 us at rank 64.)
    const int64_t wave = static_cast<int64_t>(blockIdx.x) * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if (wave >= a.total_waves) {
        return;
    }
    int64_t rest = wave;
    const int cg = static_cast<int>(rest % a.column_groups);
    rest /= a.column_groups;
    const int64_t h = rest % a.heads;
    rest /= a.heads;
    const int64_t chunk = rest % a.chunks;
    const int64_t b = rest / a.chunks;
    const int q = lane & 15;
    const int g = lane >> 4;
    const bool do_gram = a.gram != 0 && cg == 0;

    // One accumulator per block, 32-token steps in token order: the fused
    // projection + reduce kernel accumulates in the same order, so both
    // produce the same partials bit for bit.
    f32x4 acc_g[NGB];
    f32x4 acc_s[NRB][2 * CPW];
#pragma unroll
    for (int i = 0; i < NGB; ++i) {
        acc_g[i] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
    }
#pragma unroll
    for (int x = 0; x < NRB; ++x) {
#pragma unroll
        for (int c = 0; c < 2 * CPW; ++c) {
            acc_s[x][c] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
        }
    }

    const int64_t begin = chunk * a.chunk_tokens;
    const int64_t end = begin + a.chunk_tokens < a.length ? begin + a.chunk_tokens : a.length;
    ReduceTile<R, CPW> tile_a;
    ReduceTile<R, CPW> tile_b;
    if constexpr (VEC) {
        // Raw-buffer loads: steps past the chunk read zeros without an access,
        // so every load issues unconditionally, two steps ahead.
        const ReduceLanes<R, CPW> lanes = reduce_lanes<R, CPW>(a, h, cg, q, g);
        // The first two steps' loads go out in the loop's order (a, then b),
        // so that the wait at the top of the loop counts only step a's.
        reduce_load_buffer<R, CPW>(tile_a, a, lanes, b, begin, end);
        __builtin_amdgcn_sched_barrier(0);
        reduce_load_buffer<R, CPW>(tile_b, a, lanes, b, begin + 32, end);
        __builtin_amdgcn_sched_barrier(0);
        // A step past the chunk's end holds zeros, and adding their zero
        // products leaves the accumulators' bits unchanged, so both steps
        // are reduced without a branch (a branch in the loop made the
        // compiler wait for every load in flight at the top of the loop).
        // Each step's operands are rotated and split first; the loads two
        // steps ahead then go out into the freed tile registers, before the
        // step's MFMAs, so their latency runs under those MFMAs and the next
        // step.
        auto step = [&](ReduceTile<R, CPW>& tile, int64_t ahead) {
            u32x4 a_hi[NRB];
            u32x4 a_lo[NRB];
            u32x4 b_c[2 * CPW];
            reduce_relation_operands<R, CPW>(tile, a_hi, a_lo);
            reduce_content_operands<R, CPW>(tile, b_c);
            // Pin the operands here: left alone, the compiler sinks their
            // arithmetic to the MFMAs, past the loads below, so that the old
            // and the new tile are live at once and the loop carries copies
            // that wait for every load in flight.
#pragma unroll
            for (int x = 0; x < NRB; ++x) {
                asm volatile("" : "+v"(a_hi[x]), "+v"(a_lo[x]));
            }
#pragma unroll
            for (int c = 0; c < 2 * CPW; ++c) {
                asm volatile("" : "+v"(b_c[c]));
            }
            __builtin_amdgcn_sched_barrier(0);
            reduce_load_buffer<R, CPW>(tile, a, lanes, b, ahead, end);
            __builtin_amdgcn_sched_barrier(0);
            if (do_gram) {
                reduce_gram_mfma<R>(a_hi, a_lo, acc_g);
            }
            reduce_cross_mfma<R, CPW>(a_hi, a_lo, b_c, acc_s);
        };
        for (int64_t t0 = begin; t0 < end; t0 += 64) {
            step(tile_a, t0 + 64);
            step(tile_b, t0 + 96);
        }
    } else {
        reduce_load<R, CPW, VEC>(tile_a, a, b, h, cg, q, g, begin, end);
        if (begin + 32 < end) {
            reduce_load<R, CPW, VEC>(tile_b, a, b, h, cg, q, g, begin + 32, end);
        }
        for (int64_t t0 = begin; t0 < end; t0 += 64) {
            reduce_compute<R, CPW>(tile_a, do_gram, acc_g, acc_s);
            if (t0 + 64 < end) {
                reduce_load<R, CPW, VEC>(tile_a, a, b, h, cg, q, g, t0 + 64, end);
            }
            if (t0 + 32 < end) {
                reduce_compute<R, CPW>(tile_b, do_gram, acc_g, acc_s);
                if (t0 + 96 < end) {
                    reduce_load<R, CPW, VEC>(tile_b, a, b, h, cg, q, g, t0 + 96, end);
                }
            }
        }
    }

    float* part = a.partials + ((b * a.heads + h) * a.chunks + chunk) * a.partial_stride;
    if (do_gram) {
        store_gram_partial<R>(part, acc_g, q, g);
    }
    store_cross_partial<R, CPW>(part + R * R, acc_s, q, g, cg, a.head_dim);
}

// ---------------------------------------------------------------------------
// Reduce from staged row runs.  One workgroup per (sample, chunk, group of
// heads), one wave per (head of the group, column group).  Each 32-token step
// loads, with every thread of the workgroup, the group's relation columns and
// content columns of the step's rows (one contiguous run of each row per
// stream) and the step's phase rows as 16-byte pieces into LDS, so that HBM
// serves whole runs instead of each wave's 64- and 128-byte pieces of every
// row; each wave then reads its head's operands from LDS in the reduce_load
// layout and runs the reduce_kernel MFMA chains in the same token order, so
// the partials are those of reduce_kernel bit for bit.  The loads of step
// k + 1 are in flight during step k's reductions.
constexpr int kStagedWaves = 8;              // at most, per workgroup
constexpr int kStagedCols = 512;             // group columns (relation + content) per row, at most
constexpr int kStagedRelPieces = 3;          // 16-byte pieces per thread and step, at most
constexpr int kStagedConPieces = 2;
constexpr int kStagedPhasePieces = 1;

template <int R, int CPW>
__global__ __launch_bounds__(kStagedWaves * 64) void reduce_staged_kernel(ReduceArgs a) {
    using L = ReduceLayout<R>;
    constexpr int PS = L::kPairSlots;
    constexpr int PAIRS = R / 2;
    constexpr int NRB = L::kRowBlocks;
    constexpr int NGB = L::kGramBlocks;
    constexpr int PHP = PAIRS + 2;               // phase row pitch (u32)
    __shared__ __attribute__((aligned(16))) uint16_t s_rows[2][32 * (kStagedCols + 4)];
    __shared__ __attribute__((aligned(16))) uint32_t s_ph[2][32 * PHP];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int threads = blockDim.x;
    const int64_t groups = (a.heads + a.group_heads - 1) / a.group_heads;
    int64_t rest = blockIdx.x;
    const int64_t group = rest % groups;
    rest /= groups;
    const int64_t chunk = rest % a.chunks;
    const int64_t b = rest / a.chunks;
    const int64_t h0 = group * a.group_heads;
    const int hg = static_cast<int>(a.group_heads < a.heads - h0 ? a.group_heads : a.heads - h0);
    const int d = static_cast<int>(a.head_dim);
    const int cgs = static_cast<int>(a.column_groups);
    const int unit = wave / cgs;                 // head of the group
    const int cg = wave - unit * cgs;
    const bool active = unit < hg;
    const int64_t begin = chunk * a.chunk_tokens;
    const int64_t end = begin + a.chunk_tokens < a.length ? begin + a.chunk_tokens : a.length;

    // Row runs: relation columns h0 R .. (h0 + hg) R of `projected`, content
    // columns h0 d .. (h0 + hg) d of `content`; in LDS a row holds the
    // relation run then the content run.  The pitch keeps rows 8 apart in
    // different banks (2 mod 8 dwords).
    const int rel_pieces = hg * R / 8;
    const int con_pieces = hg * d / 8;
    const int cols = 8 * (rel_pieces + con_pieces);
    const int pitch = ((cols + 15) / 16) * 16 + 4;
    uint32_t rel_off[kStagedRelPieces];
    uint32_t con_off[kStagedConPieces];
    uint32_t ph_off[kStagedPhasePieces];
    int rel_lds[kStagedRelPieces];
    int con_lds[kStagedConPieces];
    int ph_lds[kStagedPhasePieces];
#pragma unroll
    for (int i = 0; i < kStagedRelPieces; ++i) {
        const int piece = tid + i * threads;
        const int row = piece / (rel_pieces > 0 ? rel_pieces : 1);
        const int c = piece - row * rel_pieces;
        const bool live = piece < 32 * rel_pieces;
        rel_off[i] = live ? 2u * static_cast<uint32_t>(row * a.width + 8 * c) : kOutOfRange;
        rel_lds[i] = live ? row * pitch + 8 * c : -1;
    }
#pragma unroll
    for (int i = 0; i < kStagedConPieces; ++i) {
        const int piece = tid + i * threads;
        const int row = piece / (con_pieces > 0 ? con_pieces : 1);
        const int c = piece - row * con_pieces;
        const bool live = piece < 32 * con_pieces;
        con_off[i] = live ? 2u * static_cast<uint32_t>(row * a.content_stride + 8 * c) : kOutOfRange;
        con_lds[i] = live ? row * pitch + 8 * (rel_pieces + c) : -1;
    }
#pragma unroll
    for (int i = 0; i < kStagedPhasePieces; ++i) {
        const int piece = tid + i * threads;
        const int row = piece / (PAIRS / 4);
        const int c = piece - row * (PAIRS / 4);
        const bool live = piece < 32 * (PAIRS / 4);
        ph_off[i] = live ? 16u * static_cast<uint32_t>(piece) : kOutOfRange;
        ph_lds[i] = live ? row * PHP + 4 * c : -1;
    }
    struct Stage {
        u32x4 rel[kStagedRelPieces];
        u32x4 con[kStagedConPieces];
        u32x4 ph[kStagedPhasePieces];
    };
    auto load = [&](Stage& st, int64_t t0) {
        const int64_t rows = end - t0;
        const BufferRsrc rel = make_buffer(a.projected + (b * a.length + t0) * a.width + h0 * R, 2 * rows * a.width);
        const BufferRsrc con = make_buffer(a.content + (b * a.length + t0) * a.content_stride + h0 * d,
                                           2 * rows * a.content_stride);
        const BufferRsrc ph = make_buffer(a.phases + b * a.phase_batch_stride + t0 * PAIRS, 4 * rows * PAIRS);
#pragma unroll
        for (int i = 0; i < kStagedRelPieces; ++i) {
            st.rel[i] = buffer_load16_stream(rel, rel_off[i]);
        }
#pragma unroll
        for (int i = 0; i < kStagedConPieces; ++i) {
            st.con[i] = buffer_load16_stream(con, con_off[i]);
        }
#pragma unroll
        for (int i = 0; i < kStagedPhasePieces; ++i) {
            st.ph[i] = buffer_load16(ph, ph_off[i]);
        }
    };
    auto commit = [&](const Stage& st, int buf) {
#pragma unroll
        for (int i = 0; i < kStagedRelPieces; ++i) {
            if (rel_lds[i] >= 0) {
                *reinterpret_cast<u32x4*>(&s_rows[buf][rel_lds[i]]) = st.rel[i];
            }
        }
#pragma unroll
        for (int i = 0; i < kStagedConPieces; ++i) {
            if (con_lds[i] >= 0) {
                *reinterpret_cast<u32x4*>(&s_rows[buf][con_lds[i]]) = st.con[i];
            }
        }
#pragma unroll
        for (int i = 0; i < kStagedPhasePieces; ++i) {
            if (ph_lds[i] >= 0) {
                uint32_t* dst = &s_ph[buf][ph_lds[i]];
                *reinterpret_cast<u32x2*>(dst) = (u32x2){st.ph[i][0], st.ph[i][1]};
                *reinterpret_cast<u32x2*>(dst + 2) = (u32x2){st.ph[i][2], st.ph[i][3]};
            }
        }
    };

    f32x4 acc_g[NGB];
    f32x4 acc_s[NRB][2 * CPW];
#pragma unroll
    for (int i = 0; i < NGB; ++i) {
        acc_g[i] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
    }
#pragma unroll
    for (int x = 0; x < NRB; ++x) {
#pragma unroll
        for (int c = 0; c < 2 * CPW; ++c) {
            acc_s[x][c] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
        }
    }
    const int q = lane & 15;
    const int g = lane >> 4;
    const bool do_gram = a.gram != 0 && cg == 0;
    // This lane's operands in a staged step (the reduce_load layout: tokens
    // 8 g .. 8 g + 7, pair slots PS q .., feature pairs of column group cg).
    const bool pv = PS * q < PAIRS;
    const int rel_col = unit * R + 2 * PS * q;
    const int con_col = 8 * rel_pieces + unit * d + 2 * (cg * 16 * CPW + q);
    auto read_tile = [&](ReduceTile<R, CPW>& t, int buf) {
        const uint16_t* rows = &s_rows[buf][(8 * g) * pitch];
        const uint32_t* phs = &s_ph[buf][(8 * g) * PHP + PS * q];
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) {
            if constexpr (PS == 2) {
                u32x2 r = {0u, 0u};
                u32x2 p = {0u, 0u};
                if (pv) {
                    r = *reinterpret_cast<const u32x2*>(rows + jj * pitch + rel_col);
                    p = *reinterpret_cast<const u32x2*>(phs + jj * PHP);
                }
                t.rel[jj][0] = r.x;
                t.rel[jj][1] = r.y;
                t.ph[jj][0] = p.x;
                t.ph[jj][1] = p.y;
            } else {
                t.rel[jj][0] = pv ? *reinterpret_cast<const uint32_t*>(rows + jj * pitch + rel_col) : 0u;
                t.ph[jj][0] = pv ? phs[jj * PHP] : 0u;
            }
#pragma unroll
            for (int c = 0; c < CPW; ++c) {
                t.con[jj][c] = 2 * (cg * 16 * CPW + 16 * c + q) < d
                    ? *reinterpret_cast<const uint32_t*>(rows + jj * pitch + con_col + 32 * c)
                    : 0u;
            }
        }
    };

    // Two register stages: the loads of step k + 2 go out at the start of
    // step k, so each has two steps of reductions to arrive before its
    // commit at the end of step k + 1.  Steps past the chunk load zeros
    // without an access and reduce to an unchanged accumulator, so the loop
    // runs whole pairs of steps.
    auto reduce_step = [&](int buf) {
        if (active) {
            ReduceTile<R, CPW> t;
            read_tile(t, buf);
            reduce_compute<R, CPW>(t, do_gram, acc_g, acc_s);
        }
    };
    Stage stage_a;
    Stage stage_b;
    load(stage_a, begin);
    __builtin_amdgcn_sched_barrier(0);
    load(stage_b, begin + 32);
    __builtin_amdgcn_sched_barrier(0);
    commit(stage_a, 0);
    __syncthreads();
    for (int64_t t0 = begin; t0 < end; t0 += 64) {
        load(stage_a, t0 + 64);
        reduce_step(0);
        commit(stage_b, 1);
        __syncthreads();
        load(stage_b, t0 + 96);
        reduce_step(1);
        commit(stage_a, 0);
        __syncthreads();
    }
    if (active) {
        float* part = a.partials + ((b * a.heads + h0 + unit) * a.chunks + chunk) * a.partial_stride;
        if (do_gram) {
            store_gram_partial<R>(part, acc_g, q, g);
        }
        store_cross_partial<R, CPW>(part + R * R, acc_s, q, g, cg, a.head_dim);
    }
}

int64_t reduce_staged_group_heads(int64_t rank, int64_t heads, int64_t head_dim, int64_t column_groups,
                                  int64_t content_stride, bool vec) {
    // Rows read as 16-byte pieces: relation and content runs whole pieces.
    if (!vec || rank < 48 || head_dim % 8 != 0 || column_groups < 1 || column_groups > kStagedWaves) {
        return 0;
    }
    // Up to 8 waves and kStagedCols columns per workgroup, and at most two
    // workgroups' worth of heads (so the grid keeps at least two workgroups
    // per sample and chunk).
    int64_t group = kStagedWaves / column_groups;
    while (group > 1 && group * (rank + head_dim) > kStagedCols) --group;
    if (group * 2 > heads && heads > 1) group = (heads + 1) / 2;
    if (group < 1) return 0;
    // Pieces per thread within the staging registers.
    const int64_t threads = 64 * group * column_groups;
    if (32 * group * rank / 8 > kStagedRelPieces * threads || 32 * group * head_dim / 8 > kStagedConPieces * threads ||
        32 * (rank / 2) / 4 > kStagedPhasePieces * threads) {
        return 0;
    }
    (void)content_stride;
    return group;
}

// ---------------------------------------------------------------------------
// Solve: one 256-thread workgroup per (b, h) system.
//
//   A = G / n + I = L L^T            blocked Cholesky
//   L^-1                             forward substitution, one column per lane
//   Z = L^-1 S / sqrt(n)             product
//   Theta = Theta0 + Z W / sqrt(n)   product
//   I + K = I + F F^T + Omega        product
//   (I + K)^-1                       Gauss-Jordan on the diagonal pivots
//   U = (I + K)^-1 Z, X = 2U - (1 + eta) Z, M' = L^-T X / sqrt(n)   products
//
// The Cholesky factor is blocked in 8-column panels in wave 0 (the diagonal
// block and the panel pass through LDS, one row per lane).  The substitution
// for L^-1 reads each row of L^T as one batch ahead of its FMAs.  I + K has a
// positive definite symmetric part, so Gauss-Jordan needs no row exchanges:
// at rank 32 it runs in wave 0 with each row split over the two wave halves,
// from rank 48 on (and at rank 16) over all four waves with a quarter of
// every row per lane and one barrier per step.  The products use all four
// waves on FP32 MFMA tiles.
constexpr int kSolveThreads = 256;
constexpr int kSolvePanel = 64;

template <int R>
struct SolveLayout {
    static constexpr int kLD = R + 4;              // R x R matrices (16-byte rows)
    static constexpr int kPLD = kSolvePanel + 4;   // R x panel matrices
    static constexpr int kChunks = R / 16;         // 16-float register chunks per row
    static constexpr int kTiles = (R / 16) * (R / 16);     // 16 x 16 tiles of an R x R matrix
    static constexpr int kTilesPerWave = (kTiles + 3) / 4;
    static constexpr int kChunkBatch = R <= 32 ? 8 : 4;    // chunk loads in flight per element
    static constexpr int kLinv = 0;                       // L^-1 rows
    static constexpr int kLinvT = kLinv + R * kLD;        // L^-1 transposed
    static constexpr int kTheta = kLinvT + R * kLD;       // Theta
    static constexpr int kWork = kTheta + R * kLD;        // A; F; the rank-32 pivot-row buffer
    static constexpr int kSys = kWork + R * kLD;          // I + K, then (I + K)^-1
    static constexpr int kPanelA = kSys + R * kLD;        // S^T panel; W^T panel; X^T panel
    static constexpr int kPanelASize = R * kPLD > kSolvePanel * kLD ? R * kPLD : kSolvePanel * kLD;
    static constexpr int kPanelB = kPanelA + kPanelASize; // Z panel; M' panel
    static constexpr int kTotal = kPanelB + R * kPLD;
};

// f(std::integral_constant<int, i>) for i = I .. N - 1, unrolled at compile
// time.
template <int N, int I = 0, typename F>
__device__ __forceinline__ void unroll_to(F&& f) {
    if constexpr (I < N) {
        f(std::integral_constant<int, I>{});
        unroll_to<N, I + 1>(f);
    }
}

// LDS ordering between lanes of one wave: its LDS instructions execute in
// issue order, so only the compiler must be kept from reordering.
__device__ __forceinline__ void wave_lds_order() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Cholesky factor of an R-column block of an SPD matrix whose rows are held
// one per lane in l (the block's R diagonal rows in lanes 0 .. R - 1, rows
// below the block in the lanes after them, zero rows past the matrix), by
// 8-column panels.  Per panel:
//   1. rows c0..c0+7 of the diagonal block go through LDS to every lane, and
//      every lane factors the 8 x 8 block itself (right-looking, in registers);
//   2. each lane solves its own panel entries against that factor,
//      L_i,m = (a_im - sum_{m'<m} L_i,m' L_m,m') / L_mm, in ascending m' (the
//      order of the block factorization, so the block's own lanes reproduce
//      it bit for bit; L_mm = p * rsq(p) in both);
//   3. the panel goes through LDS and each lane applies the rank-8 update
//      a_ij -= sum_m L_im L_jm to its columns right of the panel.
// Two LDS round trips per panel instead of one per column.  s_diag holds 64
// floats, s_panel 8 R, s_inv_diag R (16-byte aligned).  Panels recurse at
// compile time so every register index is static.  On return l is the lane's
// row of L's block column (zero above the diagonal) and s_inv_diag[m] =
// 1 / L_mm.
template <int R, int LD, int C0>
__device__ __forceinline__ void cholesky_panel(float* s_diag, float* s_panel, float* s_inv_diag, int lane,
                                               float (&l)[R]) {
    if constexpr (C0 < R) {
        constexpr int B = 8;
        wave_lds_order();
        if (lane >= C0 && lane < C0 + B) {
            *reinterpret_cast<f32x4*>(s_diag + (lane - C0) * B) = (f32x4){l[C0], l[C0 + 1], l[C0 + 2], l[C0 + 3]};
            *reinterpret_cast<f32x4*>(s_diag + (lane - C0) * B + 4) =
                (f32x4){l[C0 + 4], l[C0 + 5], l[C0 + 6], l[C0 + 7]};
        }
        wave_lds_order();
        float d[B][B];
#pragma unroll
        for (int r = 0; r < B; ++r) {
#pragma unroll
            for (int c = 0; c < B; c += 4) {
                const f32x4 v = *reinterpret_cast<const f32x4*>(s_diag + r * B + c);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    d[r][c + e] = v[e];
                }
            }
        }
        // Pivots of A = G/n + I stay >= 1, so rsq needs no range handling.
        float rs[B];
#pragma unroll
        for (int m = 0; m < B; ++m) {
            const float pivot = d[m][m];
            rs[m] = __builtin_amdgcn_rsqf(pivot);
            d[m][m] = pivot * rs[m];
#pragma unroll
            for (int r = m + 1; r < B; ++r) {
                d[r][m] *= rs[m];
            }
#pragma unroll
            for (int r = m + 1; r < B; ++r) {
#pragma unroll
                for (int c = m + 1; c <= r; ++c) {
                    d[r][c] = fmaf(-d[r][m], d[c][m], d[r][c]);
                }
            }
        }
        float x[B];
#pragma unroll
        for (int m = 0; m < B; ++m) {
            float acc = l[C0 + m];
#pragma unroll
            for (int mp = 0; mp < m; ++mp) {
                acc = fmaf(-x[mp], d[m][mp], acc);
            }
            x[m] = acc * rs[m];
        }
#pragma unroll
        for (int m = 0; m < B; ++m) {
            x[m] = lane < C0 + m ? 0.0f : x[m];
            l[C0 + m] = x[m];
        }
        if (lane == 0) {
            *reinterpret_cast<f32x4*>(s_inv_diag + C0) = (f32x4){rs[0], rs[1], rs[2], rs[3]};
            *reinterpret_cast<f32x4*>(s_inv_diag + C0 + 4) = (f32x4){rs[4], rs[5], rs[6], rs[7]};
        }
        if constexpr (C0 + B < R) {
            wave_lds_order();
            if (lane < R) {
                *reinterpret_cast<f32x4*>(s_panel + lane * B) = (f32x4){x[0], x[1], x[2], x[3]};
                *reinterpret_cast<f32x4*>(s_panel + lane * B + 4) = (f32x4){x[4], x[5], x[6], x[7]};
            }
            wave_lds_order();
            // The panel rows are read in batches of 8, each batch's reads
            // issued before the previous batch's FMAs (scheduling barriers
            // keep the compiler from moving each read next to its use, which
            // would expose one LDS latency per row).
            constexpr int kBatch = 8;
            constexpr int kRows = R - C0 - B;
            constexpr int kBatches = (kRows + kBatch - 1) / kBatch;
            f32x4 cur[kBatch][2];
            f32x4 nxt[kBatch][2];
            auto read_batch = [&](f32x4 (&dst)[kBatch][2], int batch) {
#pragma unroll
                for (int t = 0; t < kBatch; ++t) {
                    const int j = C0 + B + batch * kBatch + t;
                    if (j < R) {
                        dst[t][0] = *reinterpret_cast<const f32x4*>(s_panel + j * B);
                        dst[t][1] = *reinterpret_cast<const f32x4*>(s_panel + j * B + 4);
                    }
                }
            };
            read_batch(cur, 0);
#pragma unroll
            for (int batch = 0; batch < kBatches; ++batch) {
                if (batch + 1 < kBatches) {
                    read_batch(nxt, batch + 1);
                }
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int t = 0; t < kBatch; ++t) {
                    const int j = C0 + B + batch * kBatch + t;
                    if (j < R) {
                        float acc = l[j];
#pragma unroll
                        for (int m = 0; m < 4; ++m) {
                            acc = fmaf(-x[m], cur[t][0][m], acc);
                        }
#pragma unroll
                        for (int m = 0; m < 4; ++m) {
                            acc = fmaf(-x[4 + m], cur[t][1][m], acc);
                        }
                        l[j] = acc;
                    }
                }
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int t = 0; t < kBatch; ++t) {
                    cur[t][0] = nxt[t][0];
                    cur[t][1] = nxt[t][1];
                }
            }
        }
        cholesky_panel<R, LD, C0 + B>(s_diag, s_panel, s_inv_diag, lane, l);
    }
}

// Column `lane` of L^-1 from L^T (row-major in LDS, row stride LD) whose
// diagonal holds 1 / L_ii, right-looking: x_i = x_i / L_ii, then
// x_i' -= L_i'i x_i for every i' > i, so each x_i' sums its terms in
// ascending i.  The reads of row I are issued as one batch as soon as step
// I - 1 has scaled x_{I-1} (an empty asm makes their address depend on it),
// so they are in flight during step I - 1's FMAs; left to itself the
// compiler either places each read next to its use (one LDS latency per
// quad) or hoists every row's reads to the start (and spills).
template <int R, int LD, int I>
__device__ __forceinline__ void lower_inverse_step(const float* lt, float (&x)[R]) {
    if constexpr (I < R) {
        constexpr int qd = I / 4;   // quad holding the diagonal
        int zero = 0;
        if constexpr (I > 0) {
            asm volatile("" : "+v"(zero) : "v"(x[I - 1]));
        }
        const float* row_ptr = lt + I * LD + zero;
        f32x4 row[R / 4];
#pragma unroll
        for (int q = qd; q < R / 4; ++q) {
            row[q] = *reinterpret_cast<const f32x4*>(row_ptr + 4 * q);
        }
        x[I] *= row[qd][I % 4];
#pragma unroll
        for (int q = qd; q < R / 4; ++q) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                if (4 * q + e > I) {
                    x[4 * q + e] = fmaf(-row[q][e], x[I], x[4 * q + e]);
                }
            }
        }
        lower_inverse_step<R, LD, I + 1>(lt, x);
    }
}

template <int R, int LD>
__device__ __forceinline__ void lower_inverse_column(const float* lt, int lane, float (&x)[R]) {
#pragma unroll
    for (int i = 0; i < R; ++i) {
        x[i] = lane == i ? 1.0f : 0.0f;
    }
    lower_inverse_step<R, LD, 0>(lt, x);
}

// Rows first, first + step, ... (< R) of columns c0 .. c0 + width of
// S / sqrt(n), S = the cross-moment partials summed over chunks in ascending
// order, into an LDS panel holding S^T (row c at c * pitch), one column per
// lane; columns past the width store zero.  ROWS >= the rows per caller wave.
template <int R, int ROWS, int BATCH>
__device__ __forceinline__ void load_cross_panel(const float* part, int64_t stride, int chunks, int d, int c0,
                                                 int width, float root, float* panel, int pitch, int lane,
                                                 int first, int step) {
    const int c = lane < width ? lane : width - 1;
    float acc[ROWS];
#pragma unroll
    for (int t = 0; t < ROWS; ++t) {
        acc[t] = 0.0f;
    }
    const float* src = part + R * R + c0 + c;
    for (int ch0 = 0; ch0 < chunks; ch0 += BATCH) {
        float v[ROWS][BATCH];
#pragma unroll
        for (int t = 0; t < ROWS; ++t) {
            const int i = first + step * t;
            const int row = i < R ? i : first;
#pragma unroll
            for (int u = 0; u < BATCH; ++u) {
                const int ch = ch0 + u < chunks ? ch0 + u : chunks - 1;
                v[t][u] = src[ch * stride + row * d];
            }
        }
#pragma unroll
        for (int t = 0; t < ROWS; ++t) {
#pragma unroll
            for (int u = 0; u < BATCH; ++u) {
                if (ch0 + u < chunks) {
                    acc[t] += v[t][u];
                }
            }
        }
    }
#pragma unroll
    for (int t = 0; t < ROWS; ++t) {
        const int i = first + step * t;
        if (i < R) {
            panel[lane * pitch + i] = lane < width ? acc[t] / root : 0.0f;
        }
    }
}

// Tiles first, first + STEP, ... (< TILES, NT tiles per block row) of a
// product on v_mfma_f32_16x16x4_f32 with K terms (a multiple of 16), in
// blocks of 16 terms: lane (r, q) = (lane % 16, lane / 16) reads
// A(i0 + r, k .. k + 3) through a4(i, k) and B(k .. k + 3, j0 + r) through
// b4(j, k), k = 16 blk + 4 q, and the block's four MFMAs take element s of
// both, so step s sums terms 16 blk + s + {0, 4, 8, 12}.  Every call sums a
// tile's terms in this same order.  One 16-byte read per operand and block
// (from a row-major A and a B stored transposed; a B that is only stored
// row-major is read as four words from rows 4 apart, which fall in different
// LDS banks): reading a word per MFMA from rows 1 apart left a 64 x 64 x 64
// product at more than twice its MFMA time, bound by LDS bank conflicts.
// Each block's operands are read one block (four MFMAs) before use, across
// tile boundaries; two tiles' accumulators alternate when the wave has an
// even number of tiles.  init(t) is the starting accumulator of the wave's
// t-th tile and store(t, i, j, acc) takes the lane's part of its result,
// rows i .. i + 3 of column j; the stores run after the wave's last MFMA
// (an epilogue between tiles leaves the matrix pipe idle while it waits on
// its own LDS reads).  A tile index past TILES computes on tile 0's operands
// and is not stored.  Operands must not overlap the results of the same
// call.
template <int TILES, int NT, int K, int STEP, typename LoadA, typename LoadB, typename Init, typename Store>
__device__ __forceinline__ void tile_products(int first, int lane, LoadA a4, LoadB b4, Init init, Store store) {
    static_assert(K % 16 == 0 && K > 0, "K in blocks of 16");
    constexpr int TPW = (TILES + STEP - 1) / STEP;
    constexpr int KB = K / 16;
    constexpr int G = TPW % 2 == 0 ? 2 : 1;
    constexpr int NU = TPW * KB;   // units of one tile and one block
    // The lane index is made opaque so that the operand addresses are formed
    // here and not hoisted out of enclosing loops, where they would stay live.
    const int lane_o = opaque_int(lane);
    const int r16 = lane_o & 15;
    const int q4 = lane_o >> 4;
    // Unit n: tile t = G (n / (G KB)) + n % G of the wave, block (n / G) % KB.
    f32x4 ra[2];
    f32x4 rb[2];
    auto issue = [&](auto nc) {
        constexpr int n = decltype(nc)::value;
        constexpr int t = G * (n / (G * KB)) + n % G;
        constexpr int k = 16 * ((n / G) % KB);
        const int tile = first + STEP * t < TILES ? first + STEP * t : 0;
        ra[n % 2] = a4(16 * (tile / NT) + r16, k + 4 * q4);
        rb[n % 2] = b4(16 * (tile % NT) + r16, k + 4 * q4);
    };
    f32x4 acc[TPW];
#pragma unroll
    for (int t = 0; t < TPW; ++t) {
        acc[t] = init(t);
    }
    issue(std::integral_constant<int, 0>{});
    unroll_to<NU>([&](auto nc) {
        constexpr int n = decltype(nc)::value;
        constexpr int t = G * (n / (G * KB)) + n % G;
        if constexpr (n + 1 < NU) {
            issue(std::integral_constant<int, n + 1>{});
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(ra[n % 2][s], rb[n % 2][s], acc[t], 0, 0, 0);
        }
    });
#pragma unroll
    for (int t = 0; t < TPW; ++t) {
        const int tile = first + STEP * t;
        if (tile < TILES) {
            store(t, 16 * (tile / NT) + 4 * q4, 16 * (tile % NT) + r16, acc[t]);
        }
    }
}

// Four consecutive floats of an LDS row (16-byte aligned).
__device__ __forceinline__ f32x4 lds_quad(const float* p) {
    return *reinterpret_cast<const f32x4*>(p);
}

// Rows k .. k + 3 of column j of a row-major LDS matrix (row stride ld).
__device__ __forceinline__ f32x4 lds_column_quad(const float* base, int ld, int k, int j) {
    return (f32x4){base[k * ld + j], base[(k + 1) * ld + j], base[(k + 2) * ld + j], base[(k + 3) * ld + j]};
}

// One M x N block product (M, N multiples of 16, K of 16), tiles first,
// first + STEP, ... of the result for this wave: store(i, j, sum_k A(i, k)
// B(k, j)) in the order of tile_products, with a4 and b4 as there.  Operands
// and results must not overlap.
template <int M, int N, int K, int STEP, typename LoadA, typename LoadB, typename Store>
__device__ __forceinline__ void block_product(int first, int lane, LoadA a4, LoadB b4, Store store) {
    tile_products<(M / 16) * (N / 16), N / 16, K, STEP>(
        first, lane, a4, b4, [](int) { return (f32x4){0.0f, 0.0f, 0.0f, 0.0f}; },
        [&](int, int i, int j, const f32x4& acc) {
#pragma unroll
            for (int mm = 0; mm < 4; ++mm) {
                store(i + mm, j, acc[mm]);
            }
        });
}

// f(std::integral_constant<int, n>) for the column tiles n = 1 .. 4 of a
// 64-column panel.
template <typename F>
__device__ __forceinline__ void with_column_tiles(int ncols, F&& f) {
    switch (ncols) {
        case 1: f(std::integral_constant<int, 1>{}); break;
        case 2: f(std::integral_constant<int, 2>{}); break;
        case 3: f(std::integral_constant<int, 3>{}); break;
        default: f(std::integral_constant<int, 4>{}); break;
    }
}

// Gauss-Jordan of a rank-16 system on one wave (the in-place form, pivots on
// the diagonal: I + K has a positive definite symmetric part, so every
// leading minor is nonzero and no row exchanges are needed), each row split
// over the wave's four quarters: lane l holds columns 4 (l / 16) .. + 3 of row
// l % 16.  Step k: the rows' column-k value comes from the quarter holding it
// by ds_bpermute, the pivot by v_readlane, and each quarter reads its part of
// pivot row k from lane k of the quarter by ds_swizzle (inside each 32-lane
// group, keeping the quarter bit), so no step makes an LDS memory round
// trip; each step eliminates column k from every other row with the
// unscaled pivot row and keeps column k as column k of the growing inverse.
// Row k ends, scaled by 1 / pivot_k, at row k of s_out.
template <int LD>
__device__ __forceinline__ void gauss_jordan_quarters(const float* s_sys, float* s_out, int lane) {
    const int quarter = lane >> 4;
    const int row = lane & 15;
    f32x4 t = *reinterpret_cast<const f32x4*>(s_sys + row * LD + 4 * quarter);
    float own_pivot = 1.0f;
    unroll_to<16>([&](auto kc) {
        constexpr int k = decltype(kc)::value;
        const bool owner = quarter == (k >> 2);
        const float own = t[k & 3];
        const float x = __shfl(own, row + 16 * (k >> 2));
        const float pivot = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(own), 16 * (k >> 2) + k));
        const float inv_pivot = __builtin_amdgcn_rcpf(pivot);
        const float f = row == k ? 0.0f : x * inv_pivot;
        // Bit mode: source lane ((i & 16) | k) of each 32-lane group.
        f32x4 pivot_row;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            pivot_row[e] = __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(t[e]), 16 | (k << 5)));
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            t[e] = fmaf(-f, pivot_row[e], t[e]);
        }
        if (owner) {
            t[k & 3] = row == k ? 1.0f : -f;
        }
        if (row == k) {
            own_pivot = pivot;
        }
    });
    t = t * __builtin_amdgcn_rcpf(own_pivot);
    wave_lds_order();
    *reinterpret_cast<f32x4*>(s_out + row * LD + 4 * quarter) = t;
}

// (I + K)^-1 of a 32 x 32 block in place (row stride LD) by 2 x 2 blocks of
// 16: with the block [[P, Q], [M21, T]], P^-1 and S^-1 = (T - M21 W1)^-1 by
// the rank-16 elimination and the four corners from W1 = P^-1 Q and
// W2 = M21 P^-1, as in the rank-48 and rank-64 solve.  Wave 0 runs the
// chain (P^-1; W1; S; S^-1; then the bottom-left and top-left corners) while
// wave 1 forms W2 and then the top-right corner, with two barriers in all;
// W1 and W2 go to rows 0-15 and 16-31 of scratch.  Every wave of the
// workgroup calls it.
template <int LD>
__device__ __forceinline__ void invert32_by_blocks(float* m, float* scratch, int wave, int lane) {
    float* p = m;
    float* q = m + 16;
    float* m21 = m + 16 * LD;
    float* t = m + 16 * LD + 16;
    float* w1 = scratch;
    float* w2 = scratch + 16 * LD;
    if (wave == 0) {
        gauss_jordan_quarters<LD>(p, p, lane);
    }
    __syncthreads();
    if (wave == 0) {
        block_product<16, 16, 16, 1>(0, lane, [&](int i, int k) { return lds_quad(p + i * LD + k); },
                                     [&](int j, int k) { return lds_column_quad(q, LD, k, j); },
                                     [&](int i, int j, float v) { w1[i * LD + j] = v; });
        wave_lds_order();
        block_product<16, 16, 16, 1>(0, lane, [&](int i, int k) { return lds_quad(m21 + i * LD + k); },
                                     [&](int j, int k) { return lds_column_quad(w1, LD, k, j); },
                                     [&](int i, int j, float v) { t[i * LD + j] -= v; });
        wave_lds_order();
        gauss_jordan_quarters<LD>(t, t, lane);
    } else if (wave == 1) {
        block_product<16, 16, 16, 1>(0, lane, [&](int i, int k) { return lds_quad(m21 + i * LD + k); },
                                     [&](int j, int k) { return lds_column_quad(p, LD, k, j); },
                                     [&](int i, int j, float v) { w2[i * LD + j] = v; });
    }
    __syncthreads();
    if (wave == 0) {
        // Bottom-left -S^-1 W2 over M21, then top-left P^-1 - W1 (bottom-left).
        block_product<16, 16, 16, 1>(0, lane, [&](int i, int k) { return lds_quad(t + i * LD + k); },
                                     [&](int j, int k) { return lds_column_quad(w2, LD, k, j); },
                                     [&](int i, int j, float v) { m21[i * LD + j] = -v; });
        wave_lds_order();
        block_product<16, 16, 16, 1>(0, lane, [&](int i, int k) { return lds_quad(w1 + i * LD + k); },
                                     [&](int j, int k) { return lds_column_quad(m21, LD, k, j); },
                                     [&](int i, int j, float v) { p[i * LD + j] -= v; });
    } else if (wave == 1) {
        // Top-right -W1 S^-1 over Q.
        block_product<16, 16, 16, 1>(0, lane, [&](int i, int k) { return lds_quad(w1 + i * LD + k); },
                                     [&](int j, int k) { return lds_column_quad(t, LD, k, j); },
                                     [&](int i, int j, float v) { q[i * LD + j] = -v; });
    }
}

template <int R>
// Two workgroups per CU (512 systems on 256 CUs in one round): the register
// budget is held to 256 per lane, which costs rank 48 a few spills.
__global__ __launch_bounds__(kSolveThreads, 2) void solve_kernel(SolveArgs a) {
    using SL = SolveLayout<R>;
    using AL = ApplyLayout<R>;
    constexpr int Q = SL::kChunks;
    constexpr int LD = SL::kLD;
    constexpr int PLD = SL::kPLD;
    __shared__ __attribute__((aligned(16))) float smem[SL::kTotal];
    float* s_linv = smem + SL::kLinv;
    float* s_linvt = smem + SL::kLinvT;
    float* s_theta = smem + SL::kTheta;
    float* s_work = smem + SL::kWork;
    float* s_sys = smem + SL::kSys;
    float* s_pa = smem + SL::kPanelA;
    float* s_pb = smem + SL::kPanelB;

    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int64_t system = blockIdx.x;
    const int64_t b = system / a.heads;
    const int64_t h = system - b * a.heads;
    const int d = static_cast<int>(a.head_dim);
    const int chunks = static_cast<int>(a.chunks);
    const int64_t stride = a.partial_stride;
    const float count = a.valid_counts != nullptr ? a.valid_counts[b] : static_cast<float>(a.length);
    const float root = sqrtf(count);
    const float eta = bounded_complement(a.eta_raw[h]);
    const float* part = a.partials + system * chunks * stride;
    float* tape = a.tape != nullptr ? a.tape + system * a.tape_stride : nullptr;
    const int r16 = lane & 15;
    const int q4 = lane >> 4;
    const int first_width = d < kSolvePanel ? d : kSolvePanel;
    const float* drive = a.drive + h * d * R;

    // Theta0 entries of this wave's Theta tiles and the first drive panel
    // (rows 0 .. 63 of W, zero past d).  Up to rank 32 they are loaded now,
    // so that their latency overlaps the factorization; at larger ranks the
    // registers they would hold through it cost occupancy, and they are
    // loaded where they are used.
    constexpr bool kPrefetch = true;
    auto base_tile = [&](int t) {
        const int tile = wave + 4 * t < SL::kTiles ? wave + 4 * t : 0;
        const int i0 = 16 * (tile / (R / 16)) + 4 * q4;
        const int j = 16 * (tile % (R / 16)) + r16;
        f32x4 v;
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            v[m] = a.base[(h * R + i0 + m) * R + j];
        }
        return v;
    };
    f32x4 base_pre[SL::kTilesPerWave];
    if constexpr (kPrefetch) {
#pragma unroll
        for (int t = 0; t < SL::kTilesPerWave; ++t) {
            base_pre[t] = base_tile(t);
        }
    }
    // Quad e of W^T's panel at drive row c0: W[c0 + 4 (e % 16) + u][e / 16]
    // for u = 0 .. 3, zero past the width.
    auto drive_quad = [&](int c0, int width, int e) {
        const int j = e >> 4;
        const int c = 4 * (e & 15);
        f32x4 w;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            w[u] = c + u < width ? drive[(c0 + c + u) * R + j] : 0.0f;
        }
        return w;
    };
    constexpr int kDriveQuads = kSolvePanel * R / 4 / kSolveThreads;
    f32x4 drive_pre[kDriveQuads];
    if constexpr (kPrefetch) {
#pragma unroll
        for (int u = 0; u < kDriveQuads; ++u) {
            drive_pre[u] = drive_quad(0, first_width, tid + u * kSolveThreads);
        }
    }

    // ---- A = G / n + I; chunk partials summed in ascending order, each
    // thread keeping kChunkBatch chunks of loads in flight --------------------
    {
        constexpr int kQuads = (R * R / 4 + kSolveThreads - 1) / kSolveThreads;
        f32x4 acc[kQuads];
        const float* src[kQuads];
#pragma unroll
        for (int t = 0; t < kQuads; ++t) {
            const int q = tid + t * kSolveThreads;
            acc[t] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
            src[t] = part + 4 * (q < R * R / 4 ? q : 0);
        }
        for (int ch0 = 0; ch0 < chunks; ch0 += SL::kChunkBatch) {
            f32x4 v[kQuads][SL::kChunkBatch];
#pragma unroll
            for (int t = 0; t < kQuads; ++t) {
#pragma unroll
                for (int u = 0; u < SL::kChunkBatch; ++u) {
                    const int ch = ch0 + u < chunks ? ch0 + u : chunks - 1;
                    v[t][u] = *reinterpret_cast<const f32x4*>(src[t] + ch * stride);
                }
            }
#pragma unroll
            for (int t = 0; t < kQuads; ++t) {
#pragma unroll
                for (int u = 0; u < SL::kChunkBatch; ++u) {
                    if (ch0 + u < chunks) {
                        acc[t] += v[t][u];
                    }
                }
            }
        }
#pragma unroll
        for (int t = 0; t < kQuads; ++t) {
            const int q = tid + t * kSolveThreads;
            if (q < R * R / 4) {
                const int i = (4 * q) / R;
                const int j = 4 * q - i * R;
                f32x4 value;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    value[e] = acc[t][e] / count + (j + e == i ? 1.0f : 0.0f);
                }
                *reinterpret_cast<f32x4*>(s_work + i * LD + j) = value;
            }
        }
        // L^-1 and L^-T start at zero: only their lower (upper) blocks are
        // written.
        for (int q = tid; q < R * LD / 4; q += kSolveThreads) {
            *reinterpret_cast<f32x4*>(s_linv + 4 * q) = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
            *reinterpret_cast<f32x4*>(s_linvt + 4 * q) = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
        }
    }
    __syncthreads();

    // ---- Cholesky of A and L^-1 by 16-column blocks, then L^-1's blocks
    // below the diagonal.  Column block j (j0 = 16 j): lane l of wave 0 holds
    // row j0 + l of the block's 16 columns of A, reduced by the earlier
    // blocks; the 8-column panel factorization makes it row j0 + l of L's
    // block column (rows past R hold zeros); L goes to L's space (s_sys, free
    // until I + K is assembled) and L_jj^T, with 1 / L_ii on its diagonal,
    // over A_jj (spent).  Steps of one barrier each, with a lookahead of one
    // block: in step j wave 0 applies block j - 1 to column block j (the
    // rank-16 update A_Ij -= L_I,j-1 L_j,j-1^T on MFMA tiles) and factors
    // column block j, while wave 1 forms L_j-1,j-1^-1 one column per lane and
    // waves 2-3 apply block j - 1 to the columns past j.  Only the panel
    // factorizations and one block-column update per step are on the chain;
    // in steps 0 and 1 the other waves also sum the first S panel.
    // The diagonal blocks' inverses then join by doubling: for neighbouring
    // groups a (top) and b of h rows, L^-1_ba = -L^-1_bb (L_ba L^-1_aa).
    {
        constexpr int B = R / 16;
        unroll_to<B + 1>([&](auto jc) {
            constexpr int j = decltype(jc)::value;
            constexpr int j0 = 16 * j;
            // The first S panel is summed beside the first two steps: rows
            // 0 .. 3 kRows0 - 1 by waves 1-3 in step 0, the rest by waves 2-3
            // in step 1 (beside wave 1's first inverse).
            constexpr int kRows0 = (R / 2 + 2) / 3;
            if constexpr (j == 0) {
                if (wave != 0) {
                    load_cross_panel<R, kRows0, SL::kChunkBatch>(part, stride, chunks, d, 0, first_width, root, s_pa,
                                                                 LD, lane, wave - 1, 3);
                }
            }
            if constexpr (j == 1) {
                if (wave >= 2) {
                    load_cross_panel<R, (R - 3 * kRows0 + 1) / 2, SL::kChunkBatch>(
                        part, stride, chunks, d, 0, first_width, root, s_pa, LD, lane, 3 * kRows0 + wave - 2, 2);
                }
            }
            if constexpr (j < B) {
                if (wave == 0) {
                    if constexpr (j >= 1) {
                        block_product<R - j0, 16, 16, 1>(
                            0, lane, [&](int i, int k) { return lds_quad(s_sys + (j0 + i) * LD + j0 - 16 + k); },
                            [&](int c, int k) { return lds_quad(s_sys + (j0 + c) * LD + j0 - 16 + k); },
                            [&](int i, int c, float value) { s_work[(j0 + i) * LD + j0 + c] -= value; });
                        wave_lds_order();
                    }
                    constexpr int kRows = R - j0;
                    const bool live = lane < kRows;
                    float v[16];
                    {
                        const float* own = s_work + (live ? j0 + lane : j0) * LD + j0;
#pragma unroll
                        for (int c = 0; c < 16; c += 4) {
                            const f32x4 q = *reinterpret_cast<const f32x4*>(own + c);
#pragma unroll
                            for (int e = 0; e < 4; ++e) {
                                v[c + e] = live ? q[e] : 0.0f;
                            }
                        }
                    }
                    float* s_inv_diag = s_theta + 64 + 8 * 16;
                    cholesky_panel<16, LD, 0>(s_theta, s_theta + 64, s_inv_diag, lane, v);
                    wave_lds_order();
                    if (live) {
#pragma unroll
                        for (int c = 0; c < 16; c += 4) {
                            *reinterpret_cast<f32x4*>(s_sys + (j0 + lane) * LD + j0 + c) =
                                (f32x4){v[c], v[c + 1], v[c + 2], v[c + 3]};
                        }
                    }
                    if (lane < 16) {
                        const float own_inv = s_inv_diag[lane];
#pragma unroll
                        for (int m = 0; m < 16; ++m) {
                            s_work[(j0 + m) * LD + j0 + lane] = m == lane ? own_inv : v[m];
                        }
                    }
                }
            }
            if constexpr (j >= 1) {
                constexpr int p0 = j0 - 16;   // the previous block
                if (wave == 1) {
                    float x[16];
                    lower_inverse_column<16, LD>(s_work + p0 * LD + p0, lane, x);
                    if (lane < 16) {
#pragma unroll
                        for (int i = 0; i < 16; i += 4) {
                            *reinterpret_cast<f32x4*>(s_linvt + (p0 + lane) * LD + p0 + i) =
                                (f32x4){x[i], x[i + 1], x[i + 2], x[i + 3]};
                        }
#pragma unroll
                        for (int i = 0; i < 16; ++i) {
                            s_linv[(p0 + i) * LD + p0 + lane] = x[i];
                        }
                    }
                }
                if constexpr (j + 1 < B) {
                    constexpr int n0 = j0 + 16;   // columns past block j
                    if (wave >= 2) {
                        block_product<R - n0, R - n0, 16, 2>(
                            wave - 2, lane, [&](int i, int k) { return lds_quad(s_sys + (n0 + i) * LD + p0 + k); },
                            [&](int c, int k) { return lds_quad(s_sys + (n0 + c) * LD + p0 + k); },
                            [&](int i, int c, float value) { s_work[(n0 + i) * LD + n0 + c] -= value; });
                    }
                }
            }
            __syncthreads();
        });
        // Doubling: groups of h rows, h = 16, 32, ...; every pair of groups
        // (a0, b0 = a0 + h, hb = min(h, R - b0) rows) in two products,
        // T = L_ba L^-1_aa (its transpose into the Z panel, free until the Z
        // products) and L^-1_ba = -L^-1_bb T.  Pairs of one level run on
        // different waves.
        unroll_to<4>([&](auto lc) {
            constexpr int h = 16 << decltype(lc)::value;
            if constexpr (h < R) {
                constexpr int kPairs = (R + 2 * h - 1) / (2 * h);
                unroll_to<kPairs>([&](auto pc) {
                    constexpr int a0 = 2 * h * decltype(pc)::value;
                    constexpr int b0 = a0 + h;
                    if constexpr (b0 < R) {
                        constexpr int hb = R - b0 < h ? R - b0 : h;
                        constexpr int kWaves = 4 / kPairs;
                        constexpr int w0 = decltype(pc)::value * kWaves;
                        if (wave >= w0 && wave < w0 + kWaves) {
                            block_product<hb, h, h, kWaves>(
                                wave - w0, lane, [&](int i, int k) { return lds_quad(s_sys + (b0 + i) * LD + a0 + k); },
                                [&](int c, int k) { return lds_quad(s_linvt + (a0 + c) * LD + a0 + k); },
                                [&](int i, int c, float value) { s_pb[(a0 + c) * PLD + i] = value; });
                        }
                    }
                });
                __syncthreads();
                unroll_to<kPairs>([&](auto pc) {
                    constexpr int a0 = 2 * h * decltype(pc)::value;
                    constexpr int b0 = a0 + h;
                    if constexpr (b0 < R) {
                        constexpr int hb = R - b0 < h ? R - b0 : h;
                        constexpr int kWaves = 4 / kPairs;
                        constexpr int w0 = decltype(pc)::value * kWaves;
                        if (wave >= w0 && wave < w0 + kWaves) {
                            block_product<hb, h, hb, kWaves>(
                                wave - w0, lane, [&](int i, int k) { return lds_quad(s_linv + (b0 + i) * LD + b0 + k); },
                                [&](int c, int k) { return lds_quad(s_pb + (a0 + c) * PLD + k); },
                                [&](int i, int c, float value) {
                                    s_linv[(b0 + i) * LD + a0 + c] = -value;
                                    s_linvt[(a0 + c) * LD + b0 + i] = -value;
                                });
                        }
                    }
                });
                __syncthreads();
            }
        });
    }
    if (tape != nullptr) {
        for (int q = tid; q < R * R / 4; q += kSolveThreads) {
            const int i = (4 * q) / R;
            const int j = 4 * q - i * R;
            const f32x4 l = *reinterpret_cast<const f32x4*>(s_sys + i * LD + j);
            f32x4 lower;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                lower[e] = j + e <= i ? l[e] : 0.0f;
            }
            *reinterpret_cast<f32x4*>(tape + 4 * q) = lower;
            *reinterpret_cast<f32x4*>(tape + 3 * R * R + 4 * q) = *reinterpret_cast<const f32x4*>(s_linv + i * LD + j);
        }
    }

    // ---- Z panels (Z = L^-1 S / sqrt(n)) and Theta = Z W accumulation, on
    // FP32 MFMA 16 x 16 tiles; wave w takes tiles w, w + 4, ... --------------
    float* zbuf = a.zbuf + system * R * d;
    // The product epilogues write Z and U to global memory through raw
    // buffers (empty when not wanted): a plain store beside the epilogues'
    // LDS stores was merged with them into generic (flat) stores, whose
    // counter makes every later LDS wait a full drain.
    const BufferRsrc zbuf_out = make_buffer(zbuf, d > kSolvePanel ? int64_t{4} * R * d : 0);
    const BufferRsrc tape_out = make_buffer(tape, tape != nullptr ? int64_t{4} * a.tape_stride : 0);
    f32x4 theta_acc[SL::kTilesPerWave];
#pragma unroll
    for (int t = 0; t < SL::kTilesPerWave; ++t) {
        theta_acc[t] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
    }
    for (int c0 = 0; c0 < d; c0 += kSolvePanel) {
        const int width = d - c0 < kSolvePanel ? d - c0 : kSolvePanel;
        const int ncols = (width + 15) / 16;   // column tiles; S is zero past the width
        if (c0 > 0) {
            load_cross_panel<R, R / 4, SL::kChunkBatch>(part, stride, chunks, d, c0, width, root, s_pa, LD, lane,
                                                        wave, 4);
            __syncthreads();
        }
        with_column_tiles(ncols, [&](auto nc) {
            constexpr int NC = decltype(nc)::value;
            tile_products<(R / 16) * NC, NC, R, 4>(
                wave, lane, [&](int i, int k) { return lds_quad(s_linv + i * LD + k); },
                [&](int j, int k) { return lds_quad(s_pa + j * LD + k); },
                [](int) { return (f32x4){0.0f, 0.0f, 0.0f, 0.0f}; },
                [&](int, int i4, int c, const f32x4& z) {
#pragma unroll
                    for (int m = 0; m < 4; ++m) {
                        const int i = i4 + m;
                        s_pb[i * PLD + c] = z[m];
                        const uint32_t at = c < width ? 4u * static_cast<uint32_t>(i * d + c0 + c) : kOutOfRange;
                        buffer_store_f32(z[m], zbuf_out, at);
                        buffer_store_f32(z[m], tape_out, at + (c < width ? 16u * R * R : 0u));
                    }
                });
        });
        __syncthreads();
        // W^T of drive rows c0 .. c0 + 63 (zero past the width), row stride PLD.
#pragma unroll
        for (int u = 0; u < kDriveQuads; ++u) {
            const int e = tid + u * kSolveThreads;
            *reinterpret_cast<f32x4*>(s_pa + (e >> 4) * PLD + 4 * (e & 15)) =
                kPrefetch && c0 == 0 ? drive_pre[u] : drive_quad(c0, width, e);
        }
        __syncthreads();
        with_column_tiles(ncols, [&](auto nc) {
            constexpr int NC = decltype(nc)::value;
            tile_products<SL::kTiles, R / 16, 16 * NC, 4>(
                wave, lane, [&](int i, int k) { return lds_quad(s_pb + i * PLD + k); },
                [&](int j, int k) { return lds_quad(s_pa + j * PLD + k); }, [&](int t) { return theta_acc[t]; },
                [&](int t, int, int, const f32x4& v) { theta_acc[t] = v; });
        });
        __syncthreads();
    }

    // ---- Theta = Theta0 + acc / sqrt(n); F = tril(Theta, -1) + diag(softplus)
#pragma unroll
    for (int t = 0; t < SL::kTilesPerWave; ++t) {
        const int tile = wave + 4 * t;
        if (tile < SL::kTiles) {
            const int i0 = 16 * (tile / (R / 16));
            const int j = 16 * (tile % (R / 16)) + r16;
            if constexpr (!kPrefetch) {
                base_pre[t] = base_tile(t);
            }
            float diagonal = 0.0f;
            float theta[4];
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                const int i = i0 + 4 * q4 + m;
                theta[m] = base_pre[t][m] + theta_acc[t][m] / root;
                s_theta[i * LD + j] = theta[m];
                if (tape != nullptr) {
                    tape[R * R + i * R + j] = theta[m];
                }
                diagonal = j == i ? theta[m] : diagonal;
            }
            // At most one of a lane's four elements is on the diagonal: one
            // softplus per lane, and none in off-diagonal tiles.
            if (i0 == 16 * (tile % (R / 16))) {
                diagonal = softplus_one(diagonal);
            }
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                const int i = i0 + 4 * q4 + m;
                s_work[i * LD + j] = j < i ? theta[m] : (j == i ? diagonal : 0.0f);
            }
        }
    }
    __syncthreads();

    // ---- I + K = I + F F^T + Omega in FP32 (reference.py:491-497); all R
    // products summed (F is lower triangular, the rest add exact zeros).
    tile_products<SL::kTiles, R / 16, R, 4>(
        wave, lane, [&](int i, int k) { return lds_quad(s_work + i * LD + k); },
        [&](int j, int k) { return lds_quad(s_work + j * LD + k); },
        [](int) { return (f32x4){0.0f, 0.0f, 0.0f, 0.0f}; },
        [&](int, int i4, int c, const f32x4& sum) {
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                const int i = i4 + m;
                // Both entries are read (in bounds) and one is selected, so
                // the epilogue has no branches around its reads.
                const float upper = s_theta[i * LD + c];
                const float lower = s_theta[c * LD + i];
                const float skew = c > i ? upper : (c < i ? -lower : 0.0f);
                s_sys[i * LD + c] = sum[m] + skew + (c == i ? 1.0f : 0.0f);
            }
        });
    __syncthreads();

    // ---- (I + K)^-1 by Gauss-Jordan on all four waves, in place, on the diagonal
    // pivots: I + K = I + F F^T + Omega has the symmetric part I + F F^T >= I,
    // so every leading principal minor is positive and elimination without
    // row exchanges exists (its growth is bounded by the skew part relative to
    // the symmetric part: Golub and Van Loan, "Unsymmetric positive definite
    // linear systems", Linear Algebra Appl. 28, 1979).  Step k eliminates
    // column k from every other row with the unscaled pivot row and keeps
    // column k as column k of the growing inverse; row k ends as pivot_k
    // times row k of the inverse.
    // The eliminations are 16 x 16, on one wave with each row split over the
    // wave's quarters and no barrier per step; 32 x 32 blocks go by 2 x 2
    // blocks of 16 (invert32_by_blocks: 6.7k cycles against 10.4k for a
    // one-wave rank-32 elimination with rows split over the wave's halves),
    // and ranks past 32 by 2 x 2 blocks of those.
    if constexpr (R == 32) {
        invert32_by_blocks<LD>(s_sys, s_work, wave, lane);
    } else if constexpr (R >= 48) {
        // From rank 48 on, by blocks: with I + K = [[P, Q], [M21, T]] and P
        // 32 x 32, P^-1 (rank-32 elimination, wave 0), W1 = P^-1 Q and
        // W2 = M21 P^-1, the Schur complement S = T - M21 W1 and S^-1, then
        // (I + K)^-1 = [[P^-1 + W1 S^-1 W2, -W1 S^-1], [-S^-1 W2, S^-1]].
        // P and S inherit the positive definite symmetric part, so neither
        // elimination needs row exchanges.  Two chains of at most 32 steps
        // instead of one of R steps.
        constexpr int H1 = 32;
        constexpr int H2 = R - H1;
        // Theta's space is free once I + K is assembled.
        invert32_by_blocks<LD>(s_sys, s_theta, wave, lane);
        __syncthreads();
        block_product<H1, H2, H1, 4>(wave, lane,
                      [&](int i, int k) { return lds_quad(s_sys + i * LD + k); },
                      [&](int j, int k) { return lds_column_quad(s_sys + H1, LD, k, j); },
                      [&](int i, int j, float v) { s_work[i * LD + j] = v; });
        block_product<H2, H1, H1, 4>(wave, lane,
                      [&](int i, int k) { return lds_quad(s_sys + (H1 + i) * LD + k); },
                      [&](int j, int k) { return lds_column_quad(s_sys, LD, k, j); },
                      [&](int i, int j, float v) { s_work[(H1 + i) * LD + j] = v; });
        __syncthreads();
        block_product<H2, H2, H1, 4>(wave, lane,
                      [&](int i, int k) { return lds_quad(s_sys + (H1 + i) * LD + k); },
                      [&](int j, int k) { return lds_column_quad(s_work, LD, k, j); },
                      [&](int i, int j, float v) { s_sys[(H1 + i) * LD + H1 + j] -= v; });
        __syncthreads();
        if constexpr (H2 == 32) {
            invert32_by_blocks<LD>(s_sys + H1 * LD + H1, s_theta, wave, lane);
        } else {
            if (wave == 0) {
                gauss_jordan_quarters<LD>(s_sys + H1 * LD + H1, s_sys + H1 * LD + H1, lane);
            }
        }
        __syncthreads();
        block_product<H2, H1, H2, 4>(wave, lane,
                      [&](int i, int k) { return lds_quad(s_sys + (H1 + i) * LD + H1 + k); },
                      [&](int j, int k) { return lds_column_quad(s_work + H1 * LD, LD, k, j); },
                      [&](int i, int j, float v) { s_sys[(H1 + i) * LD + j] = -v; });
        block_product<H1, H2, H2, 4>(wave, lane,
                      [&](int i, int k) { return lds_quad(s_work + i * LD + k); },
                      [&](int j, int k) { return lds_column_quad(s_sys + H1 * LD + H1, LD, k, j); },
                      [&](int i, int j, float v) { s_sys[i * LD + H1 + j] = -v; });
        __syncthreads();
        block_product<H1, H1, H2, 4>(wave, lane,
                      [&](int i, int k) { return lds_quad(s_work + i * LD + k); },
                      [&](int j, int k) { return lds_column_quad(s_sys + H1 * LD, LD, k, j); },
                      [&](int i, int j, float v) { s_sys[i * LD + j] -= v; });
    } else {
        if (wave == 0) {
            gauss_jordan_quarters<LD>(s_sys, s_sys, lane);
        }
    }
    __syncthreads();
    if (tape != nullptr) {
        for (int q = tid; q < R * R / 4; q += kSolveThreads) {
            const int i = (4 * q) / R;
            const int j = 4 * q - i * R;
            *reinterpret_cast<f32x4*>(tape + 2 * R * R + 4 * q) = *reinterpret_cast<const f32x4*>(s_sys + i * LD + j);
        }
    }

    // ---- U, X, M' panels, written as apply operand records -----------------
    const int blocks = (d + 15) / 16;
    for (int c0 = 0; c0 < blocks * 16; c0 += kSolvePanel) {
        const int width = d - c0 < kSolvePanel ? d - c0 : kSolvePanel;
        if (d > kSolvePanel) {
            for (int e = tid; e < R * kSolvePanel; e += kSolveThreads) {
                const int i = e / kSolvePanel;
                const int c = e - i * kSolvePanel;
                s_pb[i * PLD + c] = c < width ? zbuf[i * d + c0 + c] : 0.0f;
            }
            __syncthreads();
        }
        const int ncols = (width + 15) / 16;
        with_column_tiles(ncols, [&](auto nc) {
            constexpr int NC = decltype(nc)::value;
            tile_products<(R / 16) * NC, NC, R, 4>(
                wave, lane, [&](int i, int k) { return lds_quad(s_sys + i * LD + k); },
                [&](int j, int k) { return lds_column_quad(s_pb, PLD, k, j); },
                [](int) { return (f32x4){0.0f, 0.0f, 0.0f, 0.0f}; },
                [&](int, int i4, int c, const f32x4& u) {
#pragma unroll
                    for (int m = 0; m < 4; ++m) {
                        const int i = i4 + m;
                        buffer_store_f32(u[m], tape_out,
                                         c < width ? 4u * static_cast<uint32_t>(4 * R * R + R * d + i * d + c0 + c)
                                                   : kOutOfRange);
                        s_pa[c * LD + i] = 2.0f * u[m] - (1.0f + eta) * s_pb[i * PLD + c];
                    }
                });
        });
        __syncthreads();
        with_column_tiles(ncols, [&](auto nc) {
            constexpr int NC = decltype(nc)::value;
            tile_products<(R / 16) * NC, NC, R, 4>(
                wave, lane, [&](int i, int k) { return lds_quad(s_linvt + i * LD + k); },
                [&](int j, int k) { return lds_quad(s_pa + j * LD + k); },
                [](int) { return (f32x4){0.0f, 0.0f, 0.0f, 0.0f}; },
                [&](int, int i4, int c, const f32x4& m_acc) {
#pragma unroll
                    for (int m = 0; m < 4; ++m) {
                        s_pb[(i4 + m) * PLD + c] = c < width ? m_acc[m] / root : 0.0f;
                    }
                });
        });
        __syncthreads();
        {
            // Record of feature block fb, lane g4 * 16 + column % 16.
            const int fb_local = tid >> 6;
            const int fb = c0 / 16 + fb_local;
            if (fb < blocks) {
                const int g4 = lane >> 4;
                const int column = fb_local * 16 + (lane & 15);
                uint16_t* record = a.mop + ((system * blocks + fb) * 64 + lane) * AL::kLaneHalfs;
#pragma unroll
                for (int st = 0; st < AL::kSteps32; ++st) {
#pragma unroll
                    for (int i = 0; i < 8; i += 2) {
                        uint32_t hi, lo;
                        split_bf16(s_pb[AL::rank32(st, g4, i) * PLD + column],
                                   s_pb[AL::rank32(st, g4, i + 1) * PLD + column], hi, lo);
                        *reinterpret_cast<uint32_t*>(record + AL::offset32(st) + i) = hi;
                        *reinterpret_cast<uint32_t*>(record + AL::offset32(st) + 8 + i) = lo;
                    }
                }
#pragma unroll
                for (int st = 0; st < AL::kSteps16; ++st) {
#pragma unroll
                    for (int i = 0; i < 4; i += 2) {
                        uint32_t hi, lo;
                        split_bf16(s_pb[AL::rank16(st, g4, i) * PLD + column],
                                   s_pb[AL::rank16(st, g4, i + 1) * PLD + column], hi, lo);
                        *reinterpret_cast<uint32_t*>(record + AL::offset16(st) + i) = hi;
                        *reinterpret_cast<uint32_t*>(record + AL::offset16(st) + 4 + i) = lo;
                    }
                }
            }
        }
        __syncthreads();
    }
}

// ---------------------------------------------------------------------------
// Apply.
template <int R, int NFBW>
struct ApplyOperands {
    using AL = ApplyLayout<R>;
    u32x4 hi32[NFBW][AL::kSteps32 > 0 ? AL::kSteps32 : 1];
    u32x4 lo32[NFBW][AL::kSteps32 > 0 ? AL::kSteps32 : 1];
    u32x2 hi16[NFBW][AL::kSteps16 > 0 ? AL::kSteps16 : 1];
    u32x2 lo16[NFBW][AL::kSteps16 > 0 ? AL::kSteps16 : 1];
};

template <int R, int NFBW, bool VEC>
__global__ __launch_bounds__(256) void apply_kernel(ApplyArgs a) {
    using AL = ApplyLayout<R>;
    constexpr int PAIRS = R / 2;
    const int lane = threadIdx.x & 63;
    // Wave-uniform, so the work item and the buffer bases below are scalar.
    // The waves of one (sample, chunk) read the same rows and phases: their
    // workgroups are renumbered onto one XCD (shared L2).
    const int64_t wave = xcd_local_block(blockIdx.x, gridDim.x) * 4 +
                         __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if (wave >= a.total_waves) {
        return;
    }
    int64_t rest = wave;
    const int64_t fbg = rest % a.block_groups;
    rest /= a.block_groups;
    const int64_t h = rest % a.heads;
    rest /= a.heads;
    const int64_t chunk = rest % a.chunks;
    const int64_t b = rest / a.chunks;
    const int q = lane & 15;
    const int g = lane >> 4;
    const int64_t d = a.head_dim;
    const int64_t system = b * a.heads + h;
    const float eta = bounded_complement(a.eta_raw[h]);

    ApplyOperands<R, NFBW> op;
#pragma unroll
    for (int f = 0; f < NFBW; ++f) {
        const int64_t fb = fbg * NFBW + f;
        const bool live = fb < a.feature_blocks;
        const uint16_t* record =
            a.mop + ((system * a.feature_blocks + (live ? fb : 0)) * 64 + lane) * AL::kLaneHalfs;
#pragma unroll
        for (int s = 0; s < AL::kSteps32; ++s) {
            op.hi32[f][s] = live ? *reinterpret_cast<const u32x4*>(record + AL::offset32(s))
                                 : (u32x4){0u, 0u, 0u, 0u};
            op.lo32[f][s] = live ? *reinterpret_cast<const u32x4*>(record + AL::offset32(s) + 8)
                                 : (u32x4){0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int s = 0; s < AL::kSteps16; ++s) {
            op.hi16[f][s] = live ? *reinterpret_cast<const u32x2*>(record + AL::offset16(s))
                                 : (u32x2){0u, 0u};
            op.lo16[f][s] = live ? *reinterpret_cast<const u32x2*>(record + AL::offset16(s) + 4)
                                 : (u32x2){0u, 0u};
        }
    }

    const int64_t begin = chunk * a.chunk_tokens;
    const int64_t end = begin + a.chunk_tokens < a.length ? begin + a.chunk_tokens : a.length;
    const int64_t content_offset = a.heads * R + h * d;

    // The raw operands of one 16-token step (relation pairs, phases and, at
    // rank 64, the content of this wave's feature blocks).  At rank 64 the
    // loop issues the next step's loads before it rotates and multiplies the
    // current step, so their latency runs under this step's MFMAs (125.7 ->
    // 100.6 us at B32 N4096 H6 d64).  At lower ranks the registers this takes
    // would cost waves per SIMD (7 -> 5 at rank 32, 109 -> 118 us), so each
    // step loads its own operands and reads the content just before its store.
    constexpr bool kPipelined = R == 64;
    // Relation pairs and phases of ranks 32 s + 8 g .. + 7 (the 32-rank
    // steps) or 16 s + 4 g .. + 3 (the 16-rank step) of one token.
    auto load32 = [&](const uint16_t* row, const uint32_t* phase_row, int s, u32x4& rel, u32x4& ph) {
        const int first_rank = 32 * s + 8 * g;
        if constexpr (VEC) {
            rel = *reinterpret_cast<const u32x4*>(row + h * R + first_rank);
            ph = *reinterpret_cast<const u32x4*>(phase_row + first_rank / 2);
        } else {
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                rel[p] = load_pair<false>(row + h * R + first_rank + 2 * p, true);
                ph[p] = phase_row[first_rank / 2 + p];
            }
        }
    };
    auto load16 = [&](const uint16_t* row, const uint32_t* phase_row, int s, u32x2& rel, u32x2& ph) {
        const int first_rank = 16 * s + 4 * g;
        if constexpr (VEC) {
            rel = *reinterpret_cast<const u32x2*>(row + h * R + first_rank);
            ph = *reinterpret_cast<const u32x2*>(phase_row + first_rank / 2);
        } else {
#pragma unroll
            for (int p = 0; p < 2; ++p) {
                rel[p] = load_pair<false>(row + h * R + first_rank + 2 * p, true);
                ph[p] = phase_row[first_rank / 2 + p];
            }
        }
    };
    struct StepLoads {
        u32x4 rel32[AL::kSteps32 > 0 ? AL::kSteps32 : 1];
        u32x4 ph32[AL::kSteps32 > 0 ? AL::kSteps32 : 1];
        u32x2 rel16[AL::kSteps16 > 0 ? AL::kSteps16 : 1];
        u32x2 ph16[AL::kSteps16 > 0 ? AL::kSteps16 : 1];
        u32x2 con[NFBW];
    };
    // All operands of the 16-token step at t0 (the pipelined form).
    auto load_step = [&](int64_t t0, StepLoads& l) {
        const int64_t token = t0 + q;
        const int64_t safe_token = token < end ? token : begin;
        const uint16_t* row = a.projected + (b * a.length + safe_token) * a.width;
        const uint32_t* phase_row = a.phases + b * a.phase_batch_stride + safe_token * PAIRS;
#pragma unroll
        for (int s = 0; s < AL::kSteps32; ++s) {
            load32(row, phase_row, s, l.rel32[s], l.ph32[s]);
        }
#pragma unroll
        for (int s = 0; s < AL::kSteps16; ++s) {
            load16(row, phase_row, s, l.rel16[s], l.ph16[s]);
        }
        if constexpr (VEC) {
#pragma unroll
            for (int f = 0; f < NFBW; ++f) {
                const int64_t feature = (fbg * NFBW + f) * 16 + 4 * g;
                l.con[f] = feature + 3 < d
                               ? *reinterpret_cast<const u32x2*>(row + content_offset + feature)
                               : (u32x2){0u, 0u};
            }
        }
    };

    if constexpr (VEC) {
        // Raw-buffer form: a step's buffers start at its first token and end
        // at the chunk's end, so the loads of tokens past the chunk return
        // zeros and their stores are dropped, with no branch, and the per-lane
        // byte offsets are the same for every step (only the scalar bases
        // move).  Loads, products and stores are those of the pointer form
        // below.
        const uint32_t row_bytes = 2u * static_cast<uint32_t>(a.width);
        const uint32_t rel_lane = static_cast<uint32_t>(q) * row_bytes + 2u * static_cast<uint32_t>(h * R);
        const uint32_t ph_lane = 4u * static_cast<uint32_t>(q * PAIRS);
        uint32_t con_lane[NFBW];
        uint32_t out_lane[NFBW];
#pragma unroll
        for (int f = 0; f < NFBW; ++f) {
            const int64_t feature = (fbg * NFBW + f) * 16 + 4 * g;
            const bool fv = feature < d;
            con_lane[f] = fv ? static_cast<uint32_t>(q) * row_bytes + 2u * static_cast<uint32_t>(content_offset + feature)
                             : kOutOfRange;
            out_lane[f] = fv ? 2u * static_cast<uint32_t>(q * a.out_width + h * d + feature) : kOutOfRange;
        }
        auto rel_buffer = [&](int64_t t0) {
            return make_buffer(a.projected + (b * a.length + t0) * a.width, 2 * (end - t0) * a.width);
        };
        auto load_rotation = [&](int64_t t0, StepLoads& l) {
            const BufferRsrc rel = rel_buffer(t0);
            const BufferRsrc ph = make_buffer(a.phases + b * a.phase_batch_stride + t0 * PAIRS, 4 * (end - t0) * PAIRS);
#pragma unroll
            for (int s = 0; s < AL::kSteps32; ++s) {
                const uint32_t first_rank = 32 * s + 8 * g;
                l.rel32[s] = buffer_load16(rel, rel_lane + 2u * first_rank);
                l.ph32[s] = buffer_load16(ph, ph_lane + 2u * first_rank);
            }
#pragma unroll
            for (int s = 0; s < AL::kSteps16; ++s) {
                const uint32_t first_rank = 16 * s + 4 * g;
                l.rel16[s] = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(rel, rel_lane + 2u * first_rank, 0, 0));
                l.ph16[s] = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(ph, ph_lane + 2u * first_rank, 0, 0));
            }
        };
        auto load_content = [&](int64_t t0, StepLoads& l) {
            const BufferRsrc rel = rel_buffer(t0);
#pragma unroll
            for (int f = 0; f < NFBW; ++f) {
                l.con[f] = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(rel, con_lane[f], 0, 0));
            }
        };
        // Steps alternate between two register stages.  A step rotates and
        // splits its relation pairs, then (their registers free) issues the
        // loads of the stage's next step two steps ahead, then multiplies and
        // stores, and then issues that step's content loads: every load has a
        // whole step of work behind it before its first use.
        auto step = [&](StepLoads& l, int64_t t0) {
            u32x4 b_hi32[AL::kSteps32 > 0 ? AL::kSteps32 : 1];
            u32x4 b_lo32[AL::kSteps32 > 0 ? AL::kSteps32 : 1];
#pragma unroll
            for (int s = 0; s < AL::kSteps32; ++s) {
                float v[8];
#pragma unroll
                for (int p = 0; p < 4; ++p) {
                    rotate_pair(l.rel32[s][p], l.ph32[s][p], v[2 * p], v[2 * p + 1]);
                }
#pragma unroll
                for (int p = 0; p < 4; ++p) {
                    uint32_t hi, lo;
                    split_bf16(v[2 * p], v[2 * p + 1], hi, lo);
                    b_hi32[s][p] = hi;
                    b_lo32[s][p] = lo;
                }
                // Keep the compiler from sinking this arithmetic past the
                // loads below (the old and new stage would then be live at
                // once and the loop would carry copies that wait for them).
                asm volatile("" : "+v"(b_hi32[s]), "+v"(b_lo32[s]));
            }
            u32x2 b_hi16[AL::kSteps16 > 0 ? AL::kSteps16 : 1];
            u32x2 b_lo16[AL::kSteps16 > 0 ? AL::kSteps16 : 1];
#pragma unroll
            for (int s = 0; s < AL::kSteps16; ++s) {
                float v[4];
#pragma unroll
                for (int p = 0; p < 2; ++p) {
                    rotate_pair(l.rel16[s][p], l.ph16[s][p], v[2 * p], v[2 * p + 1]);
                }
#pragma unroll
                for (int p = 0; p < 2; ++p) {
                    uint32_t hi, lo;
                    split_bf16(v[2 * p], v[2 * p + 1], hi, lo);
                    b_hi16[s][p] = hi;
                    b_lo16[s][p] = lo;
                }
                asm volatile("" : "+v"(b_hi16[s]), "+v"(b_lo16[s]));
            }
            __builtin_amdgcn_sched_barrier(0);
            load_rotation(t0 + 32, l);
            __builtin_amdgcn_sched_barrier(0);
            const BufferRsrc out = make_buffer(a.output + (b * a.length + t0) * a.out_width,
                                               2 * (end - t0) * a.out_width);
            // The feature blocks' chains interleave (each keeps its own MFMA
            // order).  A block past the head's features has zero records and
            // an out-of-range store, so it needs no branch.
            f32x4 acc[NFBW];
#pragma unroll
            for (int f = 0; f < NFBW; ++f) {
                acc[f] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
            }
#pragma unroll
            for (int s = 0; s < AL::kSteps32; ++s) {
#pragma unroll
                for (int f = 0; f < NFBW; ++f) {
                    acc[f] = mfma16x16x32(op.hi32[f][s], b_hi32[s], acc[f]);
                }
#pragma unroll
                for (int f = 0; f < NFBW; ++f) {
                    acc[f] = mfma16x16x32(op.hi32[f][s], b_lo32[s], acc[f]);
                }
#pragma unroll
                for (int f = 0; f < NFBW; ++f) {
                    acc[f] = mfma16x16x32(op.lo32[f][s], b_hi32[s], acc[f]);
                }
            }
#pragma unroll
            for (int s = 0; s < AL::kSteps16; ++s) {
#pragma unroll
                for (int f = 0; f < NFBW; ++f) {
                    acc[f] = mfma16x16x16(op.hi16[f][s], b_hi16[s], acc[f]);
                }
#pragma unroll
                for (int f = 0; f < NFBW; ++f) {
                    acc[f] = mfma16x16x16(op.hi16[f][s], b_lo16[s], acc[f]);
                }
#pragma unroll
                for (int f = 0; f < NFBW; ++f) {
                    acc[f] = mfma16x16x16(op.lo16[f][s], b_hi16[s], acc[f]);
                }
            }
#pragma unroll
            for (int f = 0; f < NFBW; ++f) {
                const u32x2 c = l.con[f];
                u32x2 y;
                y.x = pack_bf16(fmaf(eta, bf16_lo(c.x), acc[f][0]), fmaf(eta, bf16_hi(c.x), acc[f][1]));
                y.y = pack_bf16(fmaf(eta, bf16_lo(c.y), acc[f][2]), fmaf(eta, bf16_hi(c.y), acc[f][3]));
                __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(__attribute__((ext_vector_type(2))) unsigned int, y),
                                                      out, out_lane[f], 0, 0);
            }
            __builtin_amdgcn_sched_barrier(0);
            load_content(t0 + 32, l);
            __builtin_amdgcn_sched_barrier(0);
        };
        StepLoads stage_a;
        StepLoads stage_b;
        load_rotation(begin, stage_a);
        load_content(begin, stage_a);
        __builtin_amdgcn_sched_barrier(0);
        load_rotation(begin + 16, stage_b);
        load_content(begin + 16, stage_b);
        __builtin_amdgcn_sched_barrier(0);
        // A step past the chunk loads zeros and its stores are dropped, so
        // the loop runs whole pairs of steps without a branch.
        for (int64_t t0 = begin; t0 < end; t0 += 32) {
            step(stage_a, t0);
            step(stage_b, t0 + 16);
        }
        return;
    }

    StepLoads next;
    if constexpr (kPipelined) {
        if (begin < end) {
            load_step(begin, next);
        }
    }
    for (int64_t t0 = begin; t0 < end; t0 += 16) {
        StepLoads cur;
        if constexpr (kPipelined) {
            cur = next;
            if (t0 + 16 < end) {
                load_step(t0 + 16, next);
            }
        }
        const int64_t token = t0 + q;
        const bool live = token < end;
        const int64_t safe_token = live ? token : begin;
        const uint16_t* row = a.projected + (b * a.length + safe_token) * a.width;
        const uint32_t* phase_row = a.phases + b * a.phase_batch_stride + safe_token * PAIRS;

        u32x4 b_hi32[AL::kSteps32 > 0 ? AL::kSteps32 : 1];
        u32x4 b_lo32[AL::kSteps32 > 0 ? AL::kSteps32 : 1];
#pragma unroll
        for (int s = 0; s < AL::kSteps32; ++s) {
            u32x4 rel;
            u32x4 ph;
            if constexpr (kPipelined) {
                rel = cur.rel32[s];
                ph = cur.ph32[s];
            } else {
                load32(row, phase_row, s, rel, ph);
            }
            float v[8];
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                rotate_pair(rel[p], ph[p], v[2 * p], v[2 * p + 1]);
            }
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                uint32_t hi, lo;
                split_bf16(v[2 * p], v[2 * p + 1], hi, lo);
                b_hi32[s][p] = hi;
                b_lo32[s][p] = lo;
            }
        }
        u32x2 b_hi16[AL::kSteps16 > 0 ? AL::kSteps16 : 1];
        u32x2 b_lo16[AL::kSteps16 > 0 ? AL::kSteps16 : 1];
#pragma unroll
        for (int s = 0; s < AL::kSteps16; ++s) {
            u32x2 rel;
            u32x2 ph;
            if constexpr (kPipelined) {
                rel = cur.rel16[s];
                ph = cur.ph16[s];
            } else {
                load16(row, phase_row, s, rel, ph);
            }
            float v[4];
#pragma unroll
            for (int p = 0; p < 2; ++p) {
                rotate_pair(rel[p], ph[p], v[2 * p], v[2 * p + 1]);
            }
#pragma unroll
            for (int p = 0; p < 2; ++p) {
                uint32_t hi, lo;
                split_bf16(v[2 * p], v[2 * p + 1], hi, lo);
                b_hi16[s][p] = hi;
                b_lo16[s][p] = lo;
            }
        }

#pragma unroll
        for (int f = 0; f < NFBW; ++f) {
            const int64_t fb = fbg * NFBW + f;
            if (fb >= a.feature_blocks) {
                continue;
            }
            f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int s = 0; s < AL::kSteps32; ++s) {
                acc = mfma16x16x32(op.hi32[f][s], b_hi32[s], acc);
                acc = mfma16x16x32(op.hi32[f][s], b_lo32[s], acc);
                acc = mfma16x16x32(op.lo32[f][s], b_hi32[s], acc);
            }
#pragma unroll
            for (int s = 0; s < AL::kSteps16; ++s) {
                acc = mfma16x16x16(op.hi16[f][s], b_hi16[s], acc);
                acc = mfma16x16x16(op.hi16[f][s], b_lo16[s], acc);
                acc = mfma16x16x16(op.lo16[f][s], b_hi16[s], acc);
            }
            if (!live) {
                continue;
            }
            const int64_t feature = fb * 16 + 4 * g;
            uint16_t* out = a.output + (b * a.length + token) * a.out_width + h * d + feature;
            if (VEC && feature + 3 < d) {
                const u32x2 c = kPipelined ? cur.con[f]
                                           : *reinterpret_cast<const u32x2*>(row + content_offset + feature);
                u32x2 y;
                y.x = pack_bf16(fmaf(eta, bf16_lo(c.x), acc[0]), fmaf(eta, bf16_hi(c.x), acc[1]));
                y.y = pack_bf16(fmaf(eta, bf16_lo(c.y), acc[2]), fmaf(eta, bf16_hi(c.y), acc[3]));
                *reinterpret_cast<u32x2*>(out) = y;
            } else {
                const uint16_t* content = row + content_offset + feature;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    if (feature + i < d) {
                        out[i] = to_bf16_bits(fmaf(eta, bf16_bits_to_float(content[i]), acc[i]));
                    }
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Apply from staged row runs (the reduce's staging, for the readout).  One
// workgroup per (sample, token range, group of heads), one wave per head of
// the group covering its NFB feature blocks.  Each 16-token step's relation
// and content runs and phase rows are loaded by every thread of the
// workgroup as 16-byte pieces two steps ahead and committed to LDS; each wave
// reads its head's operands from LDS in the apply layout and runs the
// apply_kernel products (same records, MFMA order and rounding, so the same
// bits); the mixed rows of the group go out through an LDS tile as 16-byte
// pieces of one contiguous run per row.
constexpr int kApplyStagedWaves = 4;
constexpr int kApplyStagedCols = 512;        // group relation + content columns, at most
constexpr int kApplyStagedOut = 256;         // group output columns, at most
constexpr int kApplyStagedRel = 2;           // 16-byte pieces per thread and step, at most:
constexpr int kApplyStagedCon = 2;           //   relation, content and phase pieces,
constexpr int kApplyStagedPh = 2;
constexpr int kApplyStagedOutPieces = 2;     //   and stored mixed pieces

template <int R, int NFB>
__global__ __launch_bounds__(kApplyStagedWaves * 64) void apply_staged_kernel(ApplyArgs a) {
    using AL = ApplyLayout<R>;
    constexpr int PAIRS = R / 2;
    constexpr int PHP = PAIRS + 4;               // phase row pitch (u32)
    constexpr int S32 = AL::kSteps32 > 0 ? AL::kSteps32 : 1;
    constexpr int S16 = AL::kSteps16 > 0 ? AL::kSteps16 : 1;
    __shared__ __attribute__((aligned(16))) uint16_t s_rows[2][16 * (kApplyStagedCols + 8)];
    __shared__ __attribute__((aligned(16))) uint32_t s_ph[2][16 * PHP];
    __shared__ __attribute__((aligned(16))) uint16_t s_out[2][16 * (kApplyStagedOut + 8)];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int threads = blockDim.x;
    const int64_t groups = (a.heads + a.group_heads - 1) / a.group_heads;
    int64_t rest = blockIdx.x;
    const int64_t group = rest % groups;
    rest /= groups;
    const int64_t range = rest % a.ranges;
    const int64_t b = rest / a.ranges;
    const int64_t h0 = group * a.group_heads;
    const int hg = static_cast<int>(a.group_heads < a.heads - h0 ? a.group_heads : a.heads - h0);
    const int d = static_cast<int>(a.head_dim);
    const int unit = wave;
    const bool active = unit < hg;
    const int64_t h = h0 + (active ? unit : 0);
    const int64_t begin = range * a.range_tokens;
    const int64_t end = begin + a.range_tokens < a.length ? begin + a.range_tokens : a.length;
    if (begin >= end) {
        return;   // uniform over the workgroup
    }
    const int q = lane & 15;
    const int g = lane >> 4;
    const float eta = bounded_complement(a.eta_raw[h]);

    // This head's operand records (as apply_kernel; blocks past the head's
    // features read zeros).
    u32x4 op_hi32[NFB][S32];
    u32x4 op_lo32[NFB][S32];
    u32x2 op_hi16[NFB][S16];
    u32x2 op_lo16[NFB][S16];
    {
        const int64_t system = b * a.heads + h;
#pragma unroll
        for (int f = 0; f < NFB; ++f) {
            const bool live = f < a.feature_blocks;
            const uint16_t* record =
                a.mop + ((system * a.feature_blocks + (live ? f : 0)) * 64 + lane) * AL::kLaneHalfs;
#pragma unroll
            for (int s = 0; s < AL::kSteps32; ++s) {
                op_hi32[f][s] = live ? *reinterpret_cast<const u32x4*>(record + AL::offset32(s)) : (u32x4){0u, 0u, 0u, 0u};
                op_lo32[f][s] = live ? *reinterpret_cast<const u32x4*>(record + AL::offset32(s) + 8) : (u32x4){0u, 0u, 0u, 0u};
            }
#pragma unroll
            for (int s = 0; s < AL::kSteps16; ++s) {
                op_hi16[f][s] = live ? *reinterpret_cast<const u32x2*>(record + AL::offset16(s)) : (u32x2){0u, 0u};
                op_lo16[f][s] = live ? *reinterpret_cast<const u32x2*>(record + AL::offset16(s) + 4) : (u32x2){0u, 0u};
            }
        }
    }

    // Staged pieces of a step: the relation run and the content run of
    // each of its 16 rows, and its phase rows (16-byte pieces, at most
    // kApplyStagedRel / Con / Ph per thread).
    const int rel_pieces = hg * R / 8;
    const int con_pieces = hg * d / 8;
    const int pitch = ((8 * (rel_pieces + con_pieces) + 15) / 16) * 16 + 8;
    const int out_pieces = hg * d / 8;
    const int out_pitch = ((8 * out_pieces + 15) / 16) * 16 + 8;
    uint32_t rel_off[kApplyStagedRel];
    uint32_t con_off[kApplyStagedCon];
    uint32_t ph_off[kApplyStagedPh];
    int rel_lds[kApplyStagedRel];
    int con_lds[kApplyStagedCon];
    int ph_lds[kApplyStagedPh];
#pragma unroll
    for (int i = 0; i < kApplyStagedRel; ++i) {
        const int piece = tid + i * threads;
        const int row = piece / rel_pieces;
        const int c = piece - row * rel_pieces;
        const bool live = piece < 16 * rel_pieces;
        rel_off[i] = live ? 2u * static_cast<uint32_t>(row * a.width + 8 * c) : kOutOfRange;
        rel_lds[i] = live ? row * pitch + 8 * c : -1;
    }
#pragma unroll
    for (int i = 0; i < kApplyStagedCon; ++i) {
        const int piece = tid + i * threads;
        const int row = piece / con_pieces;
        const int c = piece - row * con_pieces;
        const bool live = piece < 16 * con_pieces;
        con_off[i] = live ? 2u * static_cast<uint32_t>(row * a.width + 8 * c) : kOutOfRange;
        con_lds[i] = live ? row * pitch + 8 * (rel_pieces + c) : -1;
    }
#pragma unroll
    for (int i = 0; i < kApplyStagedPh; ++i) {
        const int piece = tid + i * threads;
        const int row = piece / (PAIRS / 4);
        const int c = piece - row * (PAIRS / 4);
        const bool live = piece < 16 * (PAIRS / 4);
        ph_off[i] = live ? 16u * static_cast<uint32_t>(piece) : kOutOfRange;
        ph_lds[i] = live ? row * PHP + 4 * c : -1;
    }
    struct Stage {
        u32x4 rel[kApplyStagedRel];
        u32x4 con[kApplyStagedCon];
        u32x4 ph[kApplyStagedPh];
    };
    auto load = [&](Stage& st, int64_t t0) {
        const int64_t rows = end - t0;
        const uint16_t* row0 = a.projected + (b * a.length + t0) * a.width;
        const BufferRsrc rel = make_buffer(row0 + h0 * R, 2 * rows * a.width);
        const BufferRsrc con = make_buffer(row0 + a.heads * R + h0 * d, 2 * rows * a.width);
        const BufferRsrc ph = make_buffer(a.phases + b * a.phase_batch_stride + t0 * PAIRS, 4 * rows * PAIRS);
#pragma unroll
        for (int i = 0; i < kApplyStagedRel; ++i) {
            st.rel[i] = buffer_load16_stream(rel, rel_off[i]);
        }
#pragma unroll
        for (int i = 0; i < kApplyStagedCon; ++i) {
            st.con[i] = buffer_load16_stream(con, con_off[i]);
        }
#pragma unroll
        for (int i = 0; i < kApplyStagedPh; ++i) {
            st.ph[i] = buffer_load16(ph, ph_off[i]);
        }
    };
    auto commit = [&](const Stage& st, int buf) {
#pragma unroll
        for (int i = 0; i < kApplyStagedRel; ++i) {
            if (rel_lds[i] >= 0) {
                *reinterpret_cast<u32x4*>(&s_rows[buf][rel_lds[i]]) = st.rel[i];
            }
        }
#pragma unroll
        for (int i = 0; i < kApplyStagedCon; ++i) {
            if (con_lds[i] >= 0) {
                *reinterpret_cast<u32x4*>(&s_rows[buf][con_lds[i]]) = st.con[i];
            }
        }
#pragma unroll
        for (int i = 0; i < kApplyStagedPh; ++i) {
            if (ph_lds[i] >= 0) {
                *reinterpret_cast<u32x4*>(&s_ph[buf][ph_lds[i]]) = st.ph[i];
            }
        }
    };
    // Output pieces of this thread: row, run column.
    uint32_t out_off[kApplyStagedOutPieces];
    int out_lds[kApplyStagedOutPieces];
#pragma unroll
    for (int i = 0; i < kApplyStagedOutPieces; ++i) {
        const int piece = tid + i * threads;
        const bool live = piece < 16 * out_pieces;
        const int row = piece / (out_pieces > 0 ? out_pieces : 1);
        const int c = piece - row * out_pieces;
        out_off[i] = live ? 2u * static_cast<uint32_t>(row * a.out_width + 8 * c) : kOutOfRange;
        out_lds[i] = live ? row * out_pitch + 8 * c : 0;
    }

    const int rel_col = unit * R;
    const int con_col = 8 * rel_pieces + unit * d;
    auto compute = [&](int buf, int obuf) {
        if (!active) {
            return;
        }
        const uint16_t* prow = &s_rows[buf][q * pitch];
        const uint32_t* phrow = &s_ph[buf][q * PHP];
        u32x4 b_hi32[S32];
        u32x4 b_lo32[S32];
#pragma unroll
        for (int s = 0; s < AL::kSteps32; ++s) {
            const int first_rank = 32 * s + 8 * g;
            const u32x4 rel = *reinterpret_cast<const u32x4*>(prow + rel_col + first_rank);
            const u32x4 ph = *reinterpret_cast<const u32x4*>(phrow + first_rank / 2);
            float v[8];
#pragma unroll
            for (int pp = 0; pp < 4; ++pp) {
                rotate_pair(rel[pp], ph[pp], v[2 * pp], v[2 * pp + 1]);
            }
#pragma unroll
            for (int pp = 0; pp < 4; ++pp) {
                uint32_t hi, lo;
                split_bf16(v[2 * pp], v[2 * pp + 1], hi, lo);
                b_hi32[s][pp] = hi;
                b_lo32[s][pp] = lo;
            }
        }
        u32x2 b_hi16[S16];
        u32x2 b_lo16[S16];
#pragma unroll
        for (int s = 0; s < AL::kSteps16; ++s) {
            const int first_rank = 16 * s + 4 * g;
            const u32x2 rel = *reinterpret_cast<const u32x2*>(prow + rel_col + first_rank);
            const u32x2 ph = *reinterpret_cast<const u32x2*>(phrow + first_rank / 2);
            float v[4];
#pragma unroll
            for (int pp = 0; pp < 2; ++pp) {
                rotate_pair(rel[pp], ph[pp], v[2 * pp], v[2 * pp + 1]);
            }
#pragma unroll
            for (int pp = 0; pp < 2; ++pp) {
                uint32_t hi, lo;
                split_bf16(v[2 * pp], v[2 * pp + 1], hi, lo);
                b_hi16[s][pp] = hi;
                b_lo16[s][pp] = lo;
            }
        }
        f32x4 acc[NFB];
#pragma unroll
        for (int f = 0; f < NFB; ++f) {
            acc[f] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
        }
#pragma unroll
        for (int s = 0; s < AL::kSteps32; ++s) {
#pragma unroll
            for (int f = 0; f < NFB; ++f) {
                acc[f] = mfma16x16x32(op_hi32[f][s], b_hi32[s], acc[f]);
            }
#pragma unroll
            for (int f = 0; f < NFB; ++f) {
                acc[f] = mfma16x16x32(op_hi32[f][s], b_lo32[s], acc[f]);
            }
#pragma unroll
            for (int f = 0; f < NFB; ++f) {
                acc[f] = mfma16x16x32(op_lo32[f][s], b_hi32[s], acc[f]);
            }
        }
#pragma unroll
        for (int s = 0; s < AL::kSteps16; ++s) {
#pragma unroll
            for (int f = 0; f < NFB; ++f) {
                acc[f] = mfma16x16x16(op_hi16[f][s], b_hi16[s], acc[f]);
            }
#pragma unroll
            for (int f = 0; f < NFB; ++f) {
                acc[f] = mfma16x16x16(op_hi16[f][s], b_lo16[s], acc[f]);
            }
#pragma unroll
            for (int f = 0; f < NFB; ++f) {
                acc[f] = mfma16x16x16(op_lo16[f][s], b_hi16[s], acc[f]);
            }
        }
        uint16_t* orow = &s_out[obuf][q * out_pitch + unit * d];
#pragma unroll
        for (int f = 0; f < NFB; ++f) {
            const int feature = 16 * f + 4 * g;
            if (feature < d) {
                const u32x2 c = *reinterpret_cast<const u32x2*>(prow + con_col + feature);
                u32x2 y;
                y.x = pack_bf16(fmaf(eta, bf16_lo(c.x), acc[f][0]), fmaf(eta, bf16_hi(c.x), acc[f][1]));
                y.y = pack_bf16(fmaf(eta, bf16_lo(c.y), acc[f][2]), fmaf(eta, bf16_hi(c.y), acc[f][3]));
                *reinterpret_cast<u32x2*>(orow + feature) = y;
            }
        }
    };
    auto store = [&](int obuf, int64_t t0) {
        const BufferRsrc out = make_buffer(a.output + (b * a.length + t0) * a.out_width + h0 * d,
                                           2 * (end - t0) * a.out_width);
#pragma unroll
        for (int i = 0; i < kApplyStagedOutPieces; ++i) {
            buffer_store16(*reinterpret_cast<const u32x4*>(&s_out[obuf][out_lds[i]]), out, out_off[i]);
        }
    };

    // Two register stages (loads two steps ahead), two row buffers and two
    // output tiles: one barrier per step.  Steps past the range load zeros
    // and store nothing.
    Stage stage_a;
    Stage stage_b;
    load(stage_a, begin);
    __builtin_amdgcn_sched_barrier(0);
    load(stage_b, begin + 16);
    __builtin_amdgcn_sched_barrier(0);
    commit(stage_a, 0);
    __syncthreads();
    for (int64_t t0 = begin; t0 < end; t0 += 32) {
        load(stage_a, t0 + 32);
        compute(0, 0);
        commit(stage_b, 1);
        __syncthreads();
        store(0, t0);
        load(stage_b, t0 + 48);
        compute(1, 1);
        commit(stage_a, 0);
        __syncthreads();
        store(1, t0 + 16);
    }
}

int64_t apply_staged_group_heads(int64_t rank, int64_t heads, int64_t head_dim, int nfbw, bool vec) {
    if (!vec || rank < 48 || head_dim % 8 != 0 || (head_dim + 15) / 16 > nfbw) {
        return 0;
    }
    int64_t group = kApplyStagedWaves;
    while (group > 1 && (group * (rank + head_dim) > kApplyStagedCols || group * head_dim > kApplyStagedOut)) {
        --group;
    }
    if (group * 2 > heads && heads > 1) group = (heads + 1) / 2;
    const int64_t threads = 64 * group;
    if (16 * group * rank / 8 > kApplyStagedRel * threads || 16 * group * head_dim / 8 > kApplyStagedCon * threads ||
        16 * (rank / 2) / 4 > kApplyStagedPh * threads || 16 * group * head_dim / 8 > kApplyStagedOutPieces * threads) {
        return 0;
    }
    return group;
}

// ---------------------------------------------------------------------------
// Launchers.
template <int R>
static hipError_t launch_reduce(const ReduceArgs& a, int cpw, bool vec, hipStream_t stream) {
    if (a.group_heads > 0) {
        const int64_t groups = (a.heads + a.group_heads - 1) / a.group_heads;
        const dim3 staged_grid(static_cast<unsigned>(a.batch * a.chunks * groups));
        const dim3 block(static_cast<unsigned>(64 * a.group_heads * a.column_groups));
        // The staged form runs from rank 48 on, where one column group of
        // 32 features per wave is the plan.
        if constexpr (R >= 48) {
            if (cpw == 1) {
                dispatch(reduce_staged_kernel<R, 1>, staged_grid, block, stream, a);
                return hipGetLastError();
            }
        }
        return hipErrorInvalidValue;
    }
    const dim3 grid(static_cast<unsigned>((a.total_waves + 3) / 4));
    if (cpw == 1) {
        if (vec) {
            dispatch(reduce_kernel<R, 1, true>, grid, 256, stream, a);
        } else {
            dispatch(reduce_kernel<R, 1, false>, grid, 256, stream, a);
        }
    } else {
        if (vec) {
            dispatch(reduce_kernel<R, 2, true>, grid, 256, stream, a);
        } else {
            dispatch(reduce_kernel<R, 2, false>, grid, 256, stream, a);
        }
    }
    return hipGetLastError();
}

template <int R>
static hipError_t launch_apply(const ApplyArgs& a, int nfbw, bool vec, hipStream_t stream) {
    if (a.group_heads > 0) {
        const int64_t groups = (a.heads + a.group_heads - 1) / a.group_heads;
        const dim3 staged_grid(static_cast<unsigned>(a.batch * a.ranges * groups));
        const dim3 block(static_cast<unsigned>(64 * a.group_heads));
        if constexpr (R >= 48) {
            switch (nfbw) {
                case 1: dispatch(apply_staged_kernel<R, 1>, staged_grid, block, stream, a); break;
                case 2: dispatch(apply_staged_kernel<R, 2>, staged_grid, block, stream, a); break;
                default: dispatch(apply_staged_kernel<R, 4>, staged_grid, block, stream, a); break;
            }
            return hipGetLastError();
        }
        return hipErrorInvalidValue;
    }
    const dim3 grid(static_cast<unsigned>((a.total_waves + 3) / 4));
    switch (nfbw) {
        case 1:
            if (vec) dispatch(apply_kernel<R, 1, true>, grid, 256, stream, a);
            else dispatch(apply_kernel<R, 1, false>, grid, 256, stream, a);
            break;
        case 2:
            if (vec) dispatch(apply_kernel<R, 2, true>, grid, 256, stream, a);
            else dispatch(apply_kernel<R, 2, false>, grid, 256, stream, a);
            break;
        default:
            if (vec) dispatch(apply_kernel<R, 4, true>, grid, 256, stream, a);
            else dispatch(apply_kernel<R, 4, false>, grid, 256, stream, a);
            break;
    }
    return hipGetLastError();
}

hipError_t launch_phase(const PhaseArgs& a, hipStream_t stream) {
    // The table has pairs = rank / 2 in {8, 16, 24, 32} entries per position
    // and fewer than 2^32 entries (the plan bounds B * N * pairs).
    const dim3 grid(static_cast<unsigned>((a.count / 4 + 255) / 256));
    switch (a.pairs) {
        case 8: dispatch(phase_kernel<8>, grid, 256, stream, a); break;
        case 16: dispatch(phase_kernel<16>, grid, 256, stream, a); break;
        case 24: dispatch(phase_kernel<24>, grid, 256, stream, a); break;
        default: dispatch(phase_kernel<32>, grid, 256, stream, a); break;
    }
    return hipGetLastError();
}

hipError_t launch_reduce(int rank, const ReduceArgs& a, int cpw, bool vec, hipStream_t stream) {
    switch (rank) {
        case 16: return launch_reduce<16>(a, cpw, vec, stream);
        case 32: return launch_reduce<32>(a, cpw, vec, stream);
        case 48: return launch_reduce<48>(a, cpw, vec, stream);
        default: return launch_reduce<64>(a, cpw, vec, stream);
    }
}

hipError_t launch_solve(int rank, const SolveArgs& a, int64_t systems, hipStream_t stream) {
    const dim3 grid(static_cast<unsigned>(systems));
    switch (rank) {
        case 16: dispatch(solve_kernel<16>, grid, kSolveThreads, stream, a); break;
        case 32: dispatch(solve_kernel<32>, grid, kSolveThreads, stream, a); break;
        case 48: dispatch(solve_kernel<48>, grid, kSolveThreads, stream, a); break;
        default: dispatch(solve_kernel<64>, grid, kSolveThreads, stream, a); break;
    }
    return hipGetLastError();
}

hipError_t launch_apply(int rank, const ApplyArgs& a, int nfbw, bool vec, hipStream_t stream) {
    switch (rank) {
        case 16: return launch_apply<16>(a, nfbw, vec, stream);
        case 32: return launch_apply<32>(a, nfbw, vec, stream);
        case 48: return launch_apply<48>(a, nfbw, vec, stream);
        default: return launch_apply<64>(a, nfbw, vec, stream);
    }
}

}  // namespace lsso_hip

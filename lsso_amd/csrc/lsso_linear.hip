// gfx950 biased projection y = cast(bf16(x) bf16(W)^T + b).
//
// Contract (reference lsso/ball/reference.py:20-75, 170-203, 347-408): BF16
// multiplicands (x rounded to BF16 with round-to-nearest-even, W likewise),
// FP32 accumulation, FP32 bias added to the accumulator, one final FP16 or
// BF16 store; FP16 output never rounds through BF16.
//
// Schedule: persistent workgroups of 8 waves.  Each wave keeps a 32-column
// slice of W (BF16, K padded to 16) in registers for the whole launch, so the
// weights are read once per workgroup; past K = 384 two waves share a slice,
// one per half of K.  64-row x tiles (32-row once
// K > 384, so that two of them and the split's partials fit LDS) are staged
// through a double-buffered LDS tile (converted to BF16 once) and shared by
// the workgroup's waves.
// The MFMA computes y^T = W x^T on v_mfma_f32_32x32x16_bf16; in that form a
// lane's accumulators are 4 runs of 4 consecutive output features of one
// row.  The rounded tile is staged in LDS and written back in 16-byte pieces
// of whole row segments (scattered 8-byte writes cost half the store rate).

#include "lsso_device.h"
#include "lsso_internal.h"
#include "lsso_hip.h"

namespace lsso_hip {

constexpr int kXcds = 8;   // accelerator complex dies of an MI355X
constexpr int kStreamRowsHost = 128;   // tile of the K-streaming tier
constexpr int kStreamColsHost = 128;

// Rows per x tile: 64, or 32 once K exceeds 384.
template <int KSTEPS>
constexpr int linear_tile_rows_k() { return KSTEPS <= 24 ? 64 : 32; }

// Waves per workgroup: eight, two per SIMD at up to 256 registers each.  Up
// to K = 384 each wave holds its whole 32-column slice (96 VGPRs at K = 384;
// with four waves, one per SIMD, the K = 384 tier took 175 us instead of
// 131 us for 32 x 4096 rows of 384 -> 768) and the K order is a single
// chain, the one the fused projection kernels reproduce bit for bit.  Past
// K = 384 two waves share each 32-column slice, one per half of K, and add
// their accumulators through LDS.
template <int KSTEPS>
constexpr int linear_waves() { return 8; }
template <int KSTEPS>
constexpr int linear_ksplit() { return KSTEPS >= 32 ? 2 : 1; }

// Tier 0 is the K-streaming kernel (any in_features above 640).
int linear_tile_rows(int k_steps) { return k_steps == 0 ? kStreamRowsHost : (k_steps <= 24 ? 64 : 32); }
int linear_columns_per_group(int k_steps) {
    return k_steps == 0 ? kStreamColsHost : (k_steps <= 24 ? 8 : 4) * 32;
}

int linear_k_tier(int64_t in_features) {
    if (in_features <= 64) return 4;
    if (in_features <= 128) return 8;
    if (in_features <= 192) return 12;
    if (in_features <= 256) return 16;
    if (in_features <= 384) return 24;
    if (in_features <= 512) return 32;
    if (in_features <= 640) return 40;
    return 0;   // K-streaming tier
}

// Load 8 consecutive x elements as BF16 one element at a time (rows whose
// length or stride rules out 16-byte loads).  Out-of-range rows and columns
// read a clamped in-bounds address and are zeroed by select.  Masked rows are
// loaded like any other: the output rows they feed are zeroed in the epilogue.
template <int XT>
__device__ __forceinline__ u32x4 load_x_chunk_scalar(const LinearArgs& a, int64_t row, int64_t k0) {
    const int64_t safe_row = row < a.rows ? row : a.rows - 1;
    const uint16_t* x = static_cast<const uint16_t*>(a.x) + safe_row * a.x_stride;
    float v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const bool live = row < a.rows && k0 + i < a.in_features;
        const uint16_t bits = x[live ? k0 + i : 0];
        float value;
        if constexpr (XT == LSSO_HIP_BF16) {
            value = bf16_bits_to_float(bits);
        } else {
            value = f16_bits_to_float(bits);
        }
        v[i] = live ? value : 0.0f;
    }
    u32x4 out;
#pragma unroll
    for (int p = 0; p < 4; ++p) {
        out[p] = pack_bf16(v[2 * p], v[2 * p + 1]);
    }
    return out;
}

// A staged x chunk: raw bits as loaded plus their liveness, so that the
// loads of the next tile stay in flight while the current tile is multiplied
// and only their conversion waits for them.
struct XChunk {
    u32x4 raw;
    int live;
};

template <int XT, bool XVEC>
__device__ __forceinline__ XChunk fetch_x_chunk(const LinearArgs& a, int64_t row, int64_t k0) {
    XChunk c;
    if constexpr (XVEC) {
        const bool in_range = row < a.rows && k0 < a.in_features;
        const int64_t safe_row = row < a.rows ? row : a.rows - 1;
        const uint16_t* x = static_cast<const uint16_t*>(a.x) + safe_row * a.x_stride;
        c.raw = *reinterpret_cast<const u32x4*>(x + (in_range ? k0 : 0));
        c.live = in_range;
    } else {
        c.raw = load_x_chunk_scalar<XT>(a, row, k0);
        c.live = 1;
    }
    return c;
}

// BF16 bits of a staged chunk (zero outside the matrix).
template <int XT, bool XVEC>
__device__ __forceinline__ u32x4 finish_x_chunk(const XChunk& c) {
    u32x4 out;
#pragma unroll
    for (int p = 0; p < 4; ++p) {
        uint32_t value = c.raw[p];
        if constexpr (XVEC && XT == LSSO_HIP_F16) {
            value = pack_bf16(f16_lo(value), f16_hi(value));
        }
        out[p] = c.live ? value : 0u;
    }
    return out;
}

template <int YT>
__device__ __forceinline__ uint16_t to_output_bits(float value) {
    if constexpr (YT == LSSO_HIP_BF16) {
        return to_bf16_bits(value);
    } else {
        return to_f16_bits(value);
    }
}

template <int KSTEPS, int XT, int YT, bool XVEC>
__global__ __launch_bounds__(linear_waves<KSTEPS>() * 64) void linear_kernel(LinearArgs a) {
    constexpr int kWaves = linear_waves<KSTEPS>();
    constexpr int KSPLIT = linear_ksplit<KSTEPS>();
    constexpr int KW = KSTEPS / KSPLIT;                 // K steps per wave
    constexpr int kSlices = kWaves / KSPLIT;            // 32-column slices per group
    constexpr int kTileRows = linear_tile_rows_k<KSTEPS>();
    constexpr int MB = kTileRows / 32;                  // 32-row MFMA blocks per tile
    constexpr int kGroupColumns = kSlices * 32;
    constexpr int KP = 16 * KSTEPS + 8;                  // LDS row pitch (bf16)
    constexpr int kChunksPerRow = 2 * KSTEPS;           // 8-element chunks
    constexpr int kThreads = kWaves * 64;
    constexpr int kChunksPerThread = kTileRows * kChunksPerRow / kThreads;
    static_assert(kTileRows * kChunksPerRow % kThreads == 0, "tile split");
    __shared__ __attribute__((aligned(16))) uint16_t s_x[2][kTileRows * KP];
    __shared__ __attribute__((aligned(16))) float s_bias[kGroupColumns];
    constexpr int YP = kGroupColumns + 8;                 // staged output row pitch
    constexpr int kStoreChunks = kTileRows * kGroupColumns / 8 / kThreads;
    static_assert(kTileRows * kGroupColumns / 8 % kThreads == 0, "store split");
    __shared__ __attribute__((aligned(16))) uint16_t s_y[kTileRows * YP];
    // Upper-K partial accumulators of a split tile, per slice, block, element and lane.
    __shared__ float s_part[KSPLIT == 2 ? kSlices * MB * 16 * 64 : 1];
    // Row flags of the tile being multiplied and of the next one.
    __shared__ int s_keep[2][kTileRows];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int half = lane >> 5;
    // Workgroups are dealt to the eight XCDs round-robin by block index.  When
    // the grid allows, the column groups of one row tile are given to blocks
    // of the same XCD, so the second read of each x tile hits that XCD's L2.
    int64_t cg, group_index;
    if (gridDim.x % (kXcds * a.column_groups) == 0) {
        const int64_t xcd = blockIdx.x % kXcds;
        const int64_t slot = blockIdx.x / kXcds;
        cg = slot % a.column_groups;
        group_index = (slot / a.column_groups) * kXcds + xcd;
    } else {
        cg = blockIdx.x % a.column_groups;
        group_index = blockIdx.x / a.column_groups;
    }
    const int64_t group_count = gridDim.x / a.column_groups;
    const int slice = wave % kSlices;
    const int khalf = wave / kSlices;
    const int kofs = KW * khalf;                        // first K step of this wave
    const int64_t n0 = cg * kGroupColumns + slice * 32;
    const bool slice_live = __builtin_amdgcn_readfirstlane(n0 < a.out_features ? 1 : 0) != 0;
    const int64_t K = a.in_features;
    const int64_t N = a.out_features;

    u32x4 wreg[KW];
    load_weight_slice<KW>(wreg, a.weight, N, K, n0, lane, int64_t{16} * kofs);
    for (int c = tid; c < kGroupColumns; c += kThreads) {
        const int64_t n = cg * kGroupColumns + c;
        s_bias[c] = (a.bias != nullptr && n < N) ? a.bias[n] : 0.0f;
    }

    // A tile's row flags are staged with its x: thread r < kTileRows reads
    // the mask byte of row r through a raw buffer over the tile's valid rows
    // (rows past the matrix, and every row when there is no mask, read as
    // zero without an access), so no load waits inside the tile loop.
    XChunk stage[kChunksPerThread];
    uint32_t stage_mask = 0;
    int64_t stage_rows = 0;
    auto load_stage = [&](int64_t tile) {
#pragma unroll
        for (int c = 0; c < kChunksPerThread; ++c) {
            const int chunk = tid + c * kThreads;
            const int rr = chunk / kChunksPerRow;
            const int cc = chunk - rr * kChunksPerRow;
            stage[c] = fetch_x_chunk<XT, XVEC>(a, tile * kTileRows + rr, 8 * cc);
        }
        stage_rows = a.rows - tile * kTileRows;
        const BufferRsrc mask = make_buffer(a.row_mask != nullptr ? a.row_mask + tile * kTileRows : nullptr,
                                            a.row_mask != nullptr ? stage_rows : 0);
        stage_mask = buffer_load_byte(mask, static_cast<uint32_t>(tid));
    };
    auto write_stage = [&](int buf) {
#pragma unroll
        for (int c = 0; c < kChunksPerThread; ++c) {
            const int chunk = tid + c * kThreads;
            const int rr = chunk / kChunksPerRow;
            const int cc = chunk - rr * kChunksPerRow;
            *reinterpret_cast<u32x4*>(&s_x[buf][rr * KP + 8 * cc]) = finish_x_chunk<XT, XVEC>(stage[c]);
        }
        if (tid < kTileRows) {
            s_keep[buf][tid] = tid < stage_rows && (a.row_mask == nullptr || stage_mask != 0);
        }
    };

    int64_t tile = group_index;
    if (tile < a.tiles) {
        load_stage(tile);
        write_stage(0);
    }
    __syncthreads();
    int buf = 0;
    for (; tile < a.tiles; tile += group_count) {
        const int64_t next = tile + group_count;
        // Memory operations complete in issue order as far as the wait
        // counter is concerned, so the order below matters: the row mask
        // bytes (needed first) are requested before the next tile's x, and the
        // next tile's x is consumed before this tile's y stores are issued.
        bool keep[MB];
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
            keep[mb] = s_keep[buf][mb * 32 + (lane & 31)] != 0;
        }
        if (next < a.tiles) {
            load_stage(next);
        }
        // The FP32 bias is the accumulators' starting value (in the lower-K
        // wave of a split slice): element 4 qd + e is feature
        // slice * 32 + 8 qd + 4 half + e of the group.
        f32x16 acc[MB];
#pragma unroll
        for (int qd = 0; qd < 4; ++qd) {
            const f32x4 bias = khalf == 0 ? *reinterpret_cast<const f32x4*>(&s_bias[slice * 32 + 8 * qd + 4 * half])
                                          : (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    acc[mb][4 * qd + e] = bias[e];
                }
            }
        }
        // Operand reads run one group of two K steps ahead of the MFMAs, so
        // at most eight x fragments are live next to the resident W slice.
        constexpr int kGroup = 2;
        u32x4 xb[2][kGroup][MB];
        auto read_group = [&](int slot, int k_base) {
#pragma unroll
            for (int ks = 0; ks < kGroup; ++ks) {
#pragma unroll
                for (int mb = 0; mb < MB; ++mb) {
                    xb[slot][ks][mb] = *reinterpret_cast<const u32x4*>(
                        &s_x[buf][(mb * 32 + (lane & 31)) * KP + 16 * (kofs + k_base + ks) + 8 * half]);
                }
            }
        };
        // A slice wholly past the output width (the last column group of an
        // output that is not a whole number of groups: 384 or 640 columns)
        // skips its products, which would only multiply zero weights, and
        // leaves its SIMD to the other wave; it still stages, stores and
        // meets every barrier.
        if (slice_live) {
            read_group(0, 0);
#pragma unroll
            for (int k2 = 0; k2 < KW; k2 += kGroup) {
                const int slot = (k2 / kGroup) & 1;
                if (k2 + kGroup < KW) {
                    read_group(slot ^ 1, k2 + kGroup);
                }
#pragma unroll
                for (int ks = 0; ks < kGroup; ++ks) {
#pragma unroll
                    for (int mb = 0; mb < MB; ++mb) {
                        acc[mb] = mfma32x32x16(wreg[k2 + ks], xb[slot][ks][mb], acc[mb]);
                    }
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        if constexpr (KSPLIT == 2) {
            // The upper-K waves hand their accumulators to the lower-K waves
            // of the same slice, which add them (lower + upper) and finish.
            if (khalf == 1) {
#pragma unroll
                for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
                    for (int i = 0; i < 16; ++i) {
                        s_part[((slice * MB + mb) * 16 + i) * 64 + lane] = acc[mb][i];
                    }
                }
            }
            __syncthreads();
            if (khalf == 0) {
#pragma unroll
                for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
                    for (int i = 0; i < 16; ++i) {
                        acc[mb][i] += s_part[((slice * MB + mb) * 16 + i) * 64 + lane];
                    }
                }
            }
        }
        // y^T block: lane holds row m = lane%32 of the 32-row block and
        // features n0 + 8 q + 4 half + r for q, r in 0..3.  The tile is
        // rounded and staged in LDS, then written back row by row so that
        // each store instruction covers whole contiguous row segments.
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
            if (khalf != 0) {
                break;   // wave-uniform: the upper-K waves have handed over
            }
            const int mr = mb * 32 + (lane & 31);
            if (__ballot(keep[mb]) != ~0ull) {
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    acc[mb][i] = keep[mb] ? acc[mb][i] : 0.0f;
                }
            }
#pragma unroll
            for (int qd = 0; qd < 4; ++qd) {
                const int c = slice * 32 + 8 * qd + 4 * half;
                const float v0 = acc[mb][4 * qd + 0];
                const float v1 = acc[mb][4 * qd + 1];
                const float v2 = acc[mb][4 * qd + 2];
                const float v3 = acc[mb][4 * qd + 3];
                u32x2 packed;
                if constexpr (YT == LSSO_HIP_BF16) {
                    packed.x = pack_bf16(v0, v1);
                    packed.y = pack_bf16(v2, v3);
                } else {
                    packed.x = pack_f16(v0, v1);
                    packed.y = pack_f16(v2, v3);
                }
                *reinterpret_cast<u32x2*>(&s_y[mr * YP + c]) = packed;
            }
        }
        __syncthreads();
        if (next < a.tiles) {
            write_stage(buf ^ 1);
        }
        if (a.y_vector) {
            // 16-byte pieces through a raw buffer over the tile's valid rows:
            // pieces past the matrix are dropped without a branch.
            const int64_t col0 = cg * kGroupColumns;
            const int64_t tile_rows = a.rows - tile * kTileRows < kTileRows ? a.rows - tile * kTileRows : kTileRows;
            const BufferRsrc ybuf = make_buffer(static_cast<uint16_t*>(a.y) + tile * kTileRows * N, 2 * tile_rows * N);
#pragma unroll
            for (int i = 0; i < kStoreChunks; ++i) {
                const int chunk = tid + i * kThreads;
                const int mr = chunk / (kGroupColumns / 8);
                const int c8 = 8 * (chunk - mr * (kGroupColumns / 8));
                const int64_t n = col0 + c8;
                buffer_store16(*reinterpret_cast<const u32x4*>(&s_y[mr * YP + c8]), ybuf,
                               n < N ? 2u * static_cast<uint32_t>(mr * N + n) : kOutOfRange);
            }
        } else {
            const int64_t col0 = cg * kGroupColumns;
#pragma unroll
            for (int i = 0; i < kStoreChunks; ++i) {
                const int chunk = tid + i * kThreads;
                const int mr = chunk / (kGroupColumns / 8);
                const int c8 = 8 * (chunk - mr * (kGroupColumns / 8));
                const int64_t m = tile * kTileRows + mr;
                const int64_t n = col0 + c8;
                if (m < a.rows && n < N) {
                    const u32x4 v = *reinterpret_cast<const u32x4*>(&s_y[mr * YP + c8]);
                    uint16_t* dst = static_cast<uint16_t*>(a.y) + m * N + n;
                    if (a.y_vector) {
                        *reinterpret_cast<u32x4*>(dst) = v;
                    } else {
#pragma unroll
                        for (int r = 0; r < 8; ++r) {
                            if (n + r < N) {
                                dst[r] = static_cast<uint16_t>(v[r >> 1] >> (16 * (r & 1)));
                            }
                        }
                    }
                }
            }
        }
        __syncthreads();
        buf ^= 1;
    }
}

// ---------------------------------------------------------------------------
// K-streaming tier (in_features > 640): the W rows no longer fit the waves'
// registers, so both operands stream through LDS.  A workgroup of four waves
// computes a 128-row x 128-column output tile; each wave a 64 x 64 quarter
// (2 x 2 blocks of v_mfma_f32_32x32x16_bf16 on y^T = W x^T).  K is taken in
// stages of 64: the x and W stages of k-tile t + 1 are loaded into registers
// (W converted from FP32 to BF16, x from FP16 to BF16, round to nearest even)
// while k-tile t is multiplied from the other LDS buffer.  The K order is one
// FP32 chain per output, ascending.  Row tiles sharing x are dealt to one XCD.
constexpr int kStreamRows = 128;
constexpr int kStreamCols = 128;
constexpr int kStreamK = 64;
constexpr int kStreamThreads = 256;

template <int XT, int YT>
__global__ __launch_bounds__(kStreamThreads) void linear_stream_kernel(LinearArgs a) {
    constexpr int KP = kStreamK + 8;                 // LDS row pitch (bf16)
    constexpr int kChunks = kStreamRows * (kStreamK / 8) / kStreamThreads;   // 16-byte pieces per thread
    constexpr int YP = kStreamCols + 8;
    __shared__ __attribute__((aligned(16))) uint16_t s_x[2][kStreamRows * KP];
    __shared__ __attribute__((aligned(16))) uint16_t s_w[2][kStreamCols * KP];
    __shared__ __attribute__((aligned(16))) uint16_t s_y[kStreamRows * YP];
    __shared__ __attribute__((aligned(16))) float s_bias[kStreamCols];
    __shared__ int s_keep[kStreamRows];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int half = lane >> 5;
    const int64_t M = a.rows;
    const int64_t N = a.out_features;
    const int64_t K = a.in_features;
    const int64_t tiles_n = a.column_groups;
    // Block b runs on XCD b % 8; the column tiles of one row tile share it.
    const int64_t xcd = blockIdx.x % kXcds;
    const int64_t slot = blockIdx.x / kXcds;
    const int64_t mt = (slot / tiles_n) * kXcds + xcd;
    const int64_t nt = slot % tiles_n;
    if (mt >= a.tiles) {
        return;
    }
    const int64_t m0 = mt * kStreamRows;
    const int64_t n0 = nt * kStreamCols;
    for (int c = tid; c < kStreamCols; c += kStreamThreads) {
        const int64_t n = n0 + c;
        s_bias[c] = (a.bias != nullptr && n < N) ? a.bias[n] : 0.0f;
    }
    for (int r = tid; r < kStreamRows; r += kStreamThreads) {
        const int64_t m = m0 + r;
        s_keep[r] = m < M && (a.row_mask == nullptr || a.row_mask[m] != 0);
    }

    const uint16_t* x = static_cast<const uint16_t*>(a.x);
    u32x4 xs[kChunks];
    f32x4 ws[kChunks][2];
    // Piece i of this thread: row (tid + 256 i) / 8, columns 8 ((tid + 256 i) % 8) .. + 7.
    auto load = [&](int64_t k0) {
#pragma unroll
        for (int i = 0; i < kChunks; ++i) {
            const int piece = tid + i * kStreamThreads;
            const int r = piece >> 3;
            const int64_t k = k0 + 8 * (piece & 7);
            const int64_t m = m0 + r;
            const int64_t n = n0 + r;
            if (a.x_vector) {
                const bool live = m < M && k < K;
                xs[i] = live ? *reinterpret_cast<const u32x4*>(x + m * a.x_stride + k) : u32x4{};
            } else {
                uint32_t v[4];
#pragma unroll
                for (int p = 0; p < 4; ++p) {
                    const uint32_t lo = (m < M && k + 2 * p < K) ? x[m * a.x_stride + k + 2 * p] : 0u;
                    const uint32_t hi = (m < M && k + 2 * p + 1 < K) ? x[m * a.x_stride + k + 2 * p + 1] : 0u;
                    v[p] = lo | (hi << 16);
                }
                xs[i] = (u32x4){v[0], v[1], v[2], v[3]};
            }
            if (a.w_vector) {
                const bool live0 = n < N && k < K;
                const bool live1 = n < N && k + 4 < K;
                ws[i][0] = live0 ? *reinterpret_cast<const f32x4*>(a.weight + n * K + k) : f32x4{};
                ws[i][1] = live1 ? *reinterpret_cast<const f32x4*>(a.weight + n * K + k + 4) : f32x4{};
            } else {
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const bool live = n < N && k + e < K;
                    ws[i][e / 4][e % 4] = live ? a.weight[n * K + k + e] : 0.0f;
                }
            }
        }
    };
    auto store = [&](int buf) {
#pragma unroll
        for (int i = 0; i < kChunks; ++i) {
            const int piece = tid + i * kStreamThreads;
            const int r = piece >> 3;
            const int c = 8 * (piece & 7);
            u32x4 xv = xs[i];
            if constexpr (XT == LSSO_HIP_F16) {
#pragma unroll
                for (int p = 0; p < 4; ++p) {
                    xv[p] = pack_bf16(f16_lo(xv[p]), f16_hi(xv[p]));
                }
            }
            *reinterpret_cast<u32x4*>(&s_x[buf][r * KP + c]) = xv;
            const u32x4 wv = {pack_bf16(ws[i][0][0], ws[i][0][1]), pack_bf16(ws[i][0][2], ws[i][0][3]),
                              pack_bf16(ws[i][1][0], ws[i][1][1]), pack_bf16(ws[i][1][2], ws[i][1][3])};
            *reinterpret_cast<u32x4*>(&s_w[buf][r * KP + c]) = wv;
        }
    };

    const int wn = wave & 1;    // 64-column half of the tile
    const int wm = wave >> 1;   // 64-row half of the tile
    f32x16 acc[2][2];
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
#pragma unroll
        for (int mb = 0; mb < 2; ++mb) {
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                acc[nb][mb][e] = 0.0f;
            }
        }
    }
    const int64_t k_tiles = (K + kStreamK - 1) / kStreamK;
    load(0);
    store(0);
    __syncthreads();
    for (int64_t kt = 0; kt < k_tiles; ++kt) {
        const int buf = static_cast<int>(kt & 1);
        if (kt + 1 < k_tiles) {
            load((kt + 1) * kStreamK);
        }
        const uint16_t* wt = s_w[buf];
        const uint16_t* xt = s_x[buf];
#pragma unroll
        for (int kk = 0; kk < kStreamK / 16; ++kk) {
            u32x4 wf[2];
            u32x4 xf[2];
#pragma unroll
            for (int b = 0; b < 2; ++b) {
                wf[b] = *reinterpret_cast<const u32x4*>(&wt[(wn * 64 + b * 32 + (lane & 31)) * KP + 16 * kk + 8 * half]);
                xf[b] = *reinterpret_cast<const u32x4*>(&xt[(wm * 64 + b * 32 + (lane & 31)) * KP + 16 * kk + 8 * half]);
            }
#pragma unroll
            for (int nb = 0; nb < 2; ++nb) {
#pragma unroll
                for (int mb = 0; mb < 2; ++mb) {
                    acc[nb][mb] = mfma32x32x16(wf[nb], xf[mb], acc[nb][mb]);
                }
            }
        }
        if (kt + 1 < k_tiles) {
            store(buf ^ 1);
        }
        __syncthreads();
    }

    // Epilogue: bias, row mask, one rounding; the tile goes out through LDS
    // as 16-byte pieces of whole row segments.  Lane (half, m) of block
    // (nb, mb) holds row m of the 32-row block and features 8 q + 4 half + r.
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
#pragma unroll
        for (int mb = 0; mb < 2; ++mb) {
            const int mr = wm * 64 + mb * 32 + (lane & 31);
            const bool keep = s_keep[mr] != 0;
#pragma unroll
            for (int qd = 0; qd < 4; ++qd) {
                const int c = wn * 64 + nb * 32 + 8 * qd + 4 * half;
                const f32x4 bias = *reinterpret_cast<const f32x4*>(&s_bias[c]);
                const float v0 = keep ? acc[nb][mb][4 * qd + 0] + bias[0] : 0.0f;
                const float v1 = keep ? acc[nb][mb][4 * qd + 1] + bias[1] : 0.0f;
                const float v2 = keep ? acc[nb][mb][4 * qd + 2] + bias[2] : 0.0f;
                const float v3 = keep ? acc[nb][mb][4 * qd + 3] + bias[3] : 0.0f;
                u32x2 packed;
                if constexpr (YT == LSSO_HIP_BF16) {
                    packed.x = pack_bf16(v0, v1);
                    packed.y = pack_bf16(v2, v3);
                } else {
                    packed.x = pack_f16(v0, v1);
                    packed.y = pack_f16(v2, v3);
                }
                *reinterpret_cast<u32x2*>(&s_y[mr * YP + c]) = packed;
            }
        }
    }
    __syncthreads();
    constexpr int kStorePieces = kStreamRows * kStreamCols / 8 / kStreamThreads;
#pragma unroll
    for (int i = 0; i < kStorePieces; ++i) {
        const int piece = tid + i * kStreamThreads;
        const int mr = piece / (kStreamCols / 8);
        const int c8 = 8 * (piece - mr * (kStreamCols / 8));
        const int64_t m = m0 + mr;
        const int64_t n = n0 + c8;
        if (m < M && n < N) {
            const u32x4 v = *reinterpret_cast<const u32x4*>(&s_y[mr * YP + c8]);
            uint16_t* dst = static_cast<uint16_t*>(a.y) + m * N + n;
            if (a.y_vector) {
                *reinterpret_cast<u32x4*>(dst) = v;
            } else {
#pragma unroll
                for (int r = 0; r < 8; ++r) {
                    if (n + r < N) {
                        dst[r] = static_cast<uint16_t>(v[r >> 1] >> (16 * (r & 1)));
                    }
                }
            }
        }
    }
}

template <int KSTEPS, bool XVEC>
static hipError_t launch_linear_kv(const LinearArgs& a, int x_dtype, int y_dtype, dim3 grid,
                                   hipStream_t stream) {
    const dim3 block(linear_waves<KSTEPS>() * 64);
    if (x_dtype == LSSO_HIP_F16) {
        if (y_dtype == LSSO_HIP_F16) {
            dispatch(linear_kernel<KSTEPS, LSSO_HIP_F16, LSSO_HIP_F16, XVEC>, grid, block, stream, a);
        } else {
            dispatch(linear_kernel<KSTEPS, LSSO_HIP_F16, LSSO_HIP_BF16, XVEC>, grid, block, stream, a);
        }
    } else {
        if (y_dtype == LSSO_HIP_F16) {
            dispatch(linear_kernel<KSTEPS, LSSO_HIP_BF16, LSSO_HIP_F16, XVEC>, grid, block, stream, a);
        } else {
            dispatch(linear_kernel<KSTEPS, LSSO_HIP_BF16, LSSO_HIP_BF16, XVEC>, grid, block, stream, a);
        }
    }
    return hipGetLastError();
}

template <int KSTEPS>
static hipError_t launch_linear_k(const LinearArgs& a, int x_dtype, int y_dtype, dim3 grid,
                                  hipStream_t stream) {
    return a.x_vector ? launch_linear_kv<KSTEPS, true>(a, x_dtype, y_dtype, grid, stream)
                      : launch_linear_kv<KSTEPS, false>(a, x_dtype, y_dtype, grid, stream);
}

hipError_t launch_linear(const LinearArgs& a, int k_steps, int x_dtype, int y_dtype,
                         int grid_groups, hipStream_t stream) {
    if (k_steps == 0) {
        // One block per output tile; row tiles rounded up to whole XCD rounds.
        static_assert(kStreamRows == kStreamRowsHost && kStreamCols == kStreamColsHost, "tile");
        const int64_t rounds = (a.tiles + kXcds - 1) / kXcds;
        const dim3 grid(static_cast<unsigned>(rounds * kXcds * a.column_groups));
        const dim3 block(kStreamThreads);
        if (x_dtype == LSSO_HIP_F16) {
            if (y_dtype == LSSO_HIP_F16) {
                dispatch(linear_stream_kernel<LSSO_HIP_F16, LSSO_HIP_F16>, grid, block, stream, a);
            } else {
                dispatch(linear_stream_kernel<LSSO_HIP_F16, LSSO_HIP_BF16>, grid, block, stream, a);
            }
        } else {
            if (y_dtype == LSSO_HIP_F16) {
                dispatch(linear_stream_kernel<LSSO_HIP_BF16, LSSO_HIP_F16>, grid, block, stream, a);
            } else {
                dispatch(linear_stream_kernel<LSSO_HIP_BF16, LSSO_HIP_BF16>, grid, block, stream, a);
            }
        }
        return hipGetLastError();
    }
    const dim3 grid(static_cast<unsigned>(grid_groups * a.column_groups));
    switch (k_steps) {
        case 4: return launch_linear_k<4>(a, x_dtype, y_dtype, grid, stream);
        case 8: return launch_linear_k<8>(a, x_dtype, y_dtype, grid, stream);
        case 12: return launch_linear_k<12>(a, x_dtype, y_dtype, grid, stream);
        case 16: return launch_linear_k<16>(a, x_dtype, y_dtype, grid, stream);
        case 24: return launch_linear_k<24>(a, x_dtype, y_dtype, grid, stream);
        case 32: return launch_linear_k<32>(a, x_dtype, y_dtype, grid, stream);
        case 40: return launch_linear_k<40>(a, x_dtype, y_dtype, grid, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace lsso_hip

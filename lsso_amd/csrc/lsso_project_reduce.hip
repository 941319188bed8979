// gfx950 input projection fused with the L-reductions.
//
// The reference runs the biased input projection (reference.py:347-408) and
// then the mixer's token reductions over its output (model.py:389-398,
// reference.py:411-447).  Here one pass over x does both per 64-token tile:
//   1. packed = bf16(x W^T + b) for the columns of a group of heads, computed
//      in LDS with exactly the linear_kernel arithmetic (BF16 operands on
//      v_mfma_f32_32x32x16_bf16, FP32 bias, RNE rounding, masked rows zero);
//   2. G += rot(R)^T rot(R) and S += rot(R)^T C for each head of the group,
//      with exactly the reduce_kernel MFMA chains in the same token order;
//   3. optionally, the packed tile is written out (the apply pass reads it).
// The packed tensor is therefore never read back from HBM for the reduction,
// and the partials equal those of linear_kernel followed by reduce_kernel bit
// for bit.
//
// A head group's columns are laid out in LDS as [R of its heads | C of its
// heads] ("virtual" columns); wave w keeps the BF16 W rows of virtual columns
// 32 w .. 32 w + 31 in registers for the whole launch.  After the projection
// each wave owns one reduction unit: unit 2 j accumulates head j's G, unit
// 2 j + 1 its S.  Workgroups are persistent over (sample, token chunk) items
// of one head group; the groups of one item sit on the same XCD so that the
// second read of an x tile hits that XCD's L2.

#include "lsso_device.h"
#include "lsso_internal.h"
#include "lsso_reduce.h"
#include "lsso_hip.h"

namespace lsso_hip {

namespace {

constexpr int kPrTile = 64;
constexpr int kPrXcds = 8;

template <int KSTEPS>
constexpr int pr_waves() { return KSTEPS <= 16 ? 8 : 4; }

int pr_k_tier(int64_t in_features) {
    if (in_features <= 128) return 8;
    if (in_features <= 192) return 12;
    if (in_features <= 256) return 16;
    if (in_features <= 384) return 24;
    return 0;
}

}  // namespace

int project_reduce_tile_rows() { return kPrTile; }

int project_reduce_group_heads(int64_t rank, int64_t heads, int64_t head_dim,
                               int64_t in_features) {
    const int tier = pr_k_tier(in_features);
    const bool rank_ok = rank == 16 || rank == 32 || rank == 48 || rank == 64;
    if (tier == 0 || !rank_ok || heads < 1 || head_dim < 16 || head_dim > 64 ||
        head_dim % 16 != 0 || in_features % 8 != 0) {
        return 0;
    }
    const int64_t waves = tier <= 16 ? 8 : 4;
    int64_t group = (waves * 32) / (rank + head_dim);
    if (group > waves / 2) group = waves / 2;
    if (group > heads) group = heads;
    // The chunk-end exchange of the odd halves' accumulators (one 16-byte
    // f32x4 per lane and MFMA block, per head) must fit the packed tile
    // buffer of 64 x (waves * 32 + 4) bf16.
    const int64_t row_blocks = 2 * ((rank / 2 + 15) / 16);
    const int64_t gram_blocks = row_blocks * (row_blocks + 1) / 2;
    const int64_t cross_blocks = row_blocks * 2 * (head_dim > 32 ? 2 : 1);
    const int64_t blocks = gram_blocks > cross_blocks ? gram_blocks : cross_blocks;
    const int64_t buffer_bytes = int64_t{kPrTile} * (waves * 32 + 4) * 2;
    while (group > 0 && group * blocks * 64 * 16 > buffer_bytes) --group;
    return static_cast<int>(group);
}

template <int KSTEPS, int R, int CPW, int XT>
__global__ __launch_bounds__(pr_waves<KSTEPS>() * 64) void project_reduce_kernel(ProjectReduceArgs a) {
    using L = ReduceLayout<R>;
    constexpr int PS = L::kPairSlots;
    constexpr int NRB = L::kRowBlocks;
    constexpr int NGB = L::kGramBlocks;
    constexpr int PAIRS = R / 2;
    constexpr int kWaves = pr_waves<KSTEPS>();
    constexpr int kThreads = kWaves * 64;
    constexpr int VW = kWaves * 32;                 // virtual columns of a group
    constexpr int KP = 16 * KSTEPS + 8;             // x tile pitch (bf16)
    // Pitches of 2 (mod 8) dwords put the rows 8 apart that one reduction
    // read touches in different LDS banks.
    constexpr int YP = VW + 4;                      // packed tile pitch (bf16)
    constexpr int PHP = PAIRS + 2;                  // phase tile pitch (u32)
    constexpr int kChunksPerRow = 2 * KSTEPS;       // 8-element x pieces
    constexpr int kXChunks = kPrTile * kChunksPerRow / kThreads;
    static_assert(kPrTile * kChunksPerRow % kThreads == 0, "x tile split");
    constexpr int kPhasePieces = kPrTile * PAIRS / 4;  // 16-byte phase pieces
    constexpr int kPhaseChunks = (kPhasePieces + kThreads - 1) / kThreads;
    constexpr int kStoreChunks = kPrTile * VW / 8 / kThreads;
    static_assert(kPrTile * VW / 8 % kThreads == 0, "store split");

    // x tiles: the tile being projected and the next one (double buffer);
    // phases: the tile being reduced, the tile being projected and the next
    // one (triple buffer); keep flags: projected and next tile.
    __shared__ __attribute__((aligned(16))) uint16_t s_x[2][kPrTile * KP];
    __shared__ __attribute__((aligned(16))) uint16_t s_y[kPrTile * YP];
    __shared__ __attribute__((aligned(16))) uint32_t s_ph[3][kPrTile * PHP];
    __shared__ __attribute__((aligned(16))) float s_bias[VW];
    __shared__ int s_col[VW];
    __shared__ int s_keep[2][kPrTile];  // the tile's rows that project (1) or are zeroed (0)

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;

    const int64_t groups = a.head_groups;
    int64_t group, slot;
    if (gridDim.x % (kPrXcds * groups) == 0) {
        const int64_t xcd = blockIdx.x % kPrXcds;
        const int64_t s = blockIdx.x / kPrXcds;
        group = s % groups;
        slot = (s / groups) * kPrXcds + xcd;
    } else {
        group = blockIdx.x % groups;
        slot = blockIdx.x / groups;
    }
    const int64_t slots = gridDim.x / groups;
    const int64_t items = a.batch * a.chunks;
    const int64_t h0 = group * a.group_heads;
    const int64_t hg = a.group_heads < a.heads - h0 ? a.group_heads : a.heads - h0;
    const int64_t D = a.in_features;
    const int64_t d = a.head_dim;

    // Packed column of a virtual column, or -1 past the group's columns.
    auto packed_column = [&](int64_t c) -> int64_t {
        if (c < hg * R) return h0 * R + c;
        if (c < hg * (R + d)) return a.heads * R + h0 * d + (c - hg * R);
        return -1;
    };
    for (int c = tid; c < VW; c += kThreads) {
        const int64_t n = packed_column(c);
        s_col[c] = static_cast<int>(n);
        s_bias[c] = (a.bias != nullptr && n >= 0) ? a.bias[n] : 0.0f;
    }
    u32x4 wreg[KSTEPS];
    load_weight_row<KSTEPS>(wreg, a.weight, packed_column(wave * 32 + (lane & 31)), D, lane);

    // This wave's reduction unit: head j = wave / 2 of the group, over the
    // even (wave even) or odd 32-token half of every tile; the halves are
    // added when the chunk ends (even + odd, as reduce_kernel does).
    const int unit_head = wave >> 1;
    const int unit_half = wave & 1;
    const bool unit_active = unit_head < hg;

    f32x4 acc_g[NGB];
    f32x4 acc_s[NRB][2 * CPW];
    auto clear_units = [&]() {
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
    };
    clear_units();

    // A tile of the workgroup's sequence: tokens [t0, t0 + 64) of item
    // (sample b, chunk); tiles past `end` of the chunk are not part of it.
    struct Cursor {
        int64_t item, b, chunk, end, t0;
    };
    auto open_item = [&](int64_t item) {
        Cursor c;
        c.item = item;
        c.b = item / a.chunks;
        c.chunk = item - c.b * a.chunks;
        c.t0 = c.chunk * a.chunk_tokens;
        c.end = c.t0 + a.chunk_tokens < a.length ? c.t0 + a.chunk_tokens : a.length;
        return c;
    };
    // The next tile: the next one of this chunk, else the first of the next
    // item of this workgroup (item >= items marks the end).
    auto advance = [&](const Cursor& c) {
        if (c.t0 + kPrTile < c.end) {
            Cursor n = c;
            n.t0 += kPrTile;
            return n;
        }
        const int64_t next_item = c.item + slots;
        if (next_item < items) {
            return open_item(next_item);
        }
        Cursor n = c;
        n.item = items;
        return n;
    };

    // Register stage of one tile: x pieces (raw bits + liveness) and phases.
    // Two stages alternate, so the loads of two tiles are in flight while a
    // third is computed.
    struct Stage {
        u32x4 x[kXChunks];
        u32x4 ph[kPhaseChunks];
        uint32_t mask;   // row mask byte of row tid (tid < 64)
        int rows;        // valid rows of the tile
    };
    // Loads of a tile through raw buffers sized to its valid rows: rows past
    // the chunk (and an exhausted cursor, rows = 0) read as zeros without a
    // memory access, and no load is conditional.
    auto load_stage = [&](Stage& st, const Cursor& c) {
        const int tid_o = opaque_int(tid);
        const int rows = c.item < items ? static_cast<int>(c.end - c.t0 < kPrTile ? c.end - c.t0 : kPrTile) : 0;
        st.rows = rows;
        const BufferRsrc mbuf = make_buffer(
            a.row_mask + (a.row_mask != nullptr ? c.b * a.length + c.t0 : 0),
            a.row_mask != nullptr ? rows : 0);
        st.mask = buffer_load_byte(mbuf, static_cast<uint32_t>(tid_o));
        const BufferRsrc xbuf = make_buffer(
            static_cast<const uint16_t*>(a.x) + (c.b * a.length + c.t0) * D, int64_t{2} * rows * D);
#pragma unroll
        for (int i = 0; i < kXChunks; ++i) {
            const int chunk = tid_o + i * kThreads;
            const int rr = chunk / kChunksPerRow;
            const int cc = chunk - rr * kChunksPerRow;
            const uint32_t offset = 8 * cc < D ? 2u * static_cast<uint32_t>(rr * static_cast<int>(D) + 8 * cc)
                                               : kOutOfRange;
            st.x[i] = buffer_load16(xbuf, offset);
        }
        const BufferRsrc pbuf = make_buffer(a.phases + c.b * a.phase_batch_stride + c.t0 * PAIRS,
                                            int64_t{4} * rows * PAIRS);
#pragma unroll
        for (int p = 0; p < kPhaseChunks; ++p) {
            const int piece = tid_o + p * kThreads;
            const uint32_t offset = (kPhasePieces % kThreads == 0 || piece < kPhasePieces)
                                        ? 16u * static_cast<uint32_t>(piece) : kOutOfRange;
            st.ph[p] = buffer_load16(pbuf, offset);
        }
    };
    // Tile of a stage into LDS: x as BF16 (inside the overlapped block, no
    // branches), then the keep flags and phases (outside it).
    auto write_stage_x = [&](const Stage& st, int x_buf) {
        const int tid_o = opaque_int(tid);
#pragma unroll
        for (int i = 0; i < kXChunks; ++i) {
            const int chunk = tid_o + i * kThreads;
            const int rr = chunk / kChunksPerRow;
            const int cc = chunk - rr * kChunksPerRow;
            u32x4 v;
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                uint32_t value = st.x[i][p];
                if constexpr (XT == LSSO_HIP_F16) {
                    value = pack_bf16(f16_lo(value), f16_hi(value));
                }
                v[p] = value;
            }
            *reinterpret_cast<u32x4*>(&s_x[x_buf][rr * KP + 8 * cc]) = v;
        }
    };
    auto write_stage_meta = [&](const Stage& st, int x_buf, int phase_buf) {
        const int tid_o = opaque_int(tid);
        if (tid_o < kPrTile) {
            s_keep[x_buf][tid_o] = tid_o < st.rows && (a.row_mask == nullptr || st.mask != 0);
        }
#pragma unroll
        for (int p = 0; p < kPhaseChunks; ++p) {
            const int piece = tid_o + p * kThreads;
            if (kPhasePieces % kThreads == 0 || piece < kPhasePieces) {
                const int rr = piece / (PAIRS / 4);
                const int pc = piece - rr * (PAIRS / 4);
                uint32_t* dst = &s_ph[phase_buf][rr * PHP + 4 * pc];
                *reinterpret_cast<u32x2*>(dst) = (u32x2){st.ph[p][0], st.ph[p][1]};
                *reinterpret_cast<u32x2*>(dst + 2) = (u32x2){st.ph[p][2], st.ph[p][3]};
            }
        }
    };
    auto write_stage = [&](const Stage& st, int x_buf, int phase_buf) {
        write_stage_x(st, x_buf);
        write_stage_meta(st, x_buf, phase_buf);
    };

    // Reduction operands of head j for the 32 tokens of half st of the tile
    // in s_y (the reduce_load layout: lane (q, g) holds tokens 8 g .. 8 g + 7).
    auto lds_tile = [&](ReduceTile<R, CPW>& t, int phase_buf, int st) {
        const int lane_o = opaque_int(lane);
        const int q = lane_o & 15;
        const int g = lane_o >> 4;
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) {
            const int row = 32 * st + 8 * g + jj;
            const uint16_t* yrow = s_y + row * YP;
            const uint32_t* prow = s_ph[phase_buf] + row * PHP;
            if constexpr (PS == 2) {
                const bool pv = PS * q < PAIRS;
                u32x2 r = {0u, 0u};
                u32x2 p = {0u, 0u};
                if (pv) {
                    r = *reinterpret_cast<const u32x2*>(yrow + unit_head * R + 2 * PS * q);
                    p = *reinterpret_cast<const u32x2*>(prow + PS * q);
                }
                t.rel[jj][0] = r.x;
                t.rel[jj][1] = r.y;
                t.ph[jj][0] = p.x;
                t.ph[jj][1] = p.y;
            } else {
                const bool pv = q < PAIRS;
                t.rel[jj][0] = pv ? *reinterpret_cast<const uint32_t*>(yrow + unit_head * R + 2 * q) : 0u;
                t.ph[jj][0] = pv ? prow[q] : 0u;
            }
#pragma unroll
            for (int c = 0; c < CPW; ++c) {
                const int feature = 2 * (16 * c + q);
                t.con[jj][c] = feature < d
                    ? *reinterpret_cast<const uint32_t*>(yrow + hg * R + unit_head * d + feature)
                    : 0u;
            }
        }
    };

    // Rows of a cursor's tile inside its chunk (0 for an exhausted cursor).
    auto tile_rows = [&](const Cursor& c) -> int {
        return c.item < items ? static_cast<int>(c.end - c.t0 < kPrTile ? c.end - c.t0 : kPrTile) : 0;
    };

    // One step of the software pipeline, for tile k = `cur`:
    //   - issue the loads of tile k + 2 (`ahead`) into `load`;
    //   - one barrier-free block: the projection MFMAs of tile k (s_x[k & 1]),
    //     the reductions and packed store of tile k - 1 (`prev`, in s_y), and
    //     the move of tile k + 1 from `next` into s_x[(k + 1) & 1], so that
    //     MFMA, VALU and memory work of three tiles overlap;
    //   - the chunk end of tile k - 1 if it closes its chunk;
    //   - the epilogue of tile k into s_y.
    // Every access of the block is in bounds whether or not its tile exists
    // (an absent tile reads zeros and stores nothing), so the block has no
    // branches; LDS starts zeroed, so reducing an absent tile adds zeros.
    auto step = [&](const Cursor& prev, const Cursor& cur, const Cursor& nx1, const Cursor& ahead,
                    Stage& load, const Stage& next, int k3, int k2) {
        load_stage(load, ahead);

        // Projection of tile k for this wave's 32 virtual columns, in slices
        // of two K steps; each slice also carries a share of the other work
        // of the block (the reductions and packed store of tile k - 1, the
        // x of tile k + 1), in a fixed order that scheduling fences keep, so
        // that the VALU, LDS and memory work runs under the MFMAs.
        f32x16 acc[2];
#pragma unroll
        for (int mb = 0; mb < 2; ++mb) {
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                acc[mb][i] = 0.0f;
            }
        }
        const int lane_k = opaque_int(lane);
        const int row_k = lane_k & 31;
        const int half_k = lane_k >> 5;
        const uint16_t* xt = s_x[k2];
        auto read_x = [&](u32x4 (&xf)[2][2], int slice) {
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
                for (int mb = 0; mb < 2; ++mb) {
                    xf[ks][mb] = *reinterpret_cast<const u32x4*>(
                        &xt[(mb * 32 + row_k) * KP + 16 * (2 * slice + ks) + 8 * half_k]);
                }
            }
        };

        ReduceTile<R, CPW> t;
        u32x4 a_hi[NRB];
        u32x4 a_lo[NRB];
        u32x4 b_c[2 * CPW];
        const int rows_prev = tile_rows(prev);
        // The other work, as items 0 .. kItems - 1.
        constexpr int kItems = 11;
        auto other = [&](int item) {
            if (item == 0) {
                lds_tile(t, k3 == 0 ? 2 : k3 - 1, unit_half);
            } else if (item >= 1 && item <= 4) {
                reduce_relation_operands_pair<R, CPW>(t, item - 1, a_hi, a_lo);
            } else if (item == 5) {
                reduce_content_operands<R, CPW>(t, b_c);
            } else if (item == 6) {
                reduce_gram_mfma<R>(a_hi, a_lo, acc_g);
            } else if (item == 7) {
                reduce_cross_mfma<R, CPW>(a_hi, a_lo, b_c, acc_s);
            } else if (item == 8 || item == 9) {
                // Packed tile k - 1 out, as 16-byte pieces of the group's two
                // column runs; rows past its chunk (or an absent tile) fall
                // outside the buffer and are dropped.
                const BufferRsrc obuf = make_buffer(
                    a.packed + (a.packed != nullptr ? (prev.b * a.length + prev.t0) * a.width : 0),
                    a.packed != nullptr ? int64_t{2} * rows_prev * a.width : 0);
                const int tid_o = opaque_int(tid);
                constexpr int kHalf = (kStoreChunks + 1) / 2;
#pragma unroll
                for (int i = 0; i < kStoreChunks; ++i) {
                    if ((item == 8) == (i < kHalf)) {
                        const int piece = tid_o + i * kThreads;
                        const int mr = piece / (VW / 8);
                        const int c8 = 8 * (piece - mr * (VW / 8));
                        const int n = s_col[c8];
                        const u32x2 lo = *reinterpret_cast<const u32x2*>(&s_y[mr * YP + c8]);
                        const u32x2 hi = *reinterpret_cast<const u32x2*>(&s_y[mr * YP + c8 + 4]);
                        const u32x4 v = {lo.x, lo.y, hi.x, hi.y};
                        const uint32_t offset =
                            n >= 0 ? 2u * static_cast<uint32_t>(mr * static_cast<int>(a.width) + n)
                                   : kOutOfRange;
                        buffer_store16(v, obuf, offset);
                    }
                }
            } else if (item == 10) {
                // Tile k + 1's x into LDS (its loads were issued one step ago).
                write_stage_x(next, k2 ^ 1);
            }
        };

        constexpr int kSlices = KSTEPS / 2;
        static_assert(KSTEPS % 2 == 0, "slices of two K steps");
        u32x4 xf[2][2][2];
        read_x(xf[0], 0);
#pragma unroll
        for (int slice = 0; slice < kSlices; ++slice) {
            if (slice + 1 < kSlices) {
                read_x(xf[(slice + 1) & 1], slice + 1);
            }
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
                for (int mb = 0; mb < 2; ++mb) {
                    acc[mb] = mfma32x32x16(wreg[2 * slice + ks], xf[slice & 1][ks][mb], acc[mb]);
                }
            }
#pragma unroll
            for (int item = slice * kItems / kSlices; item < (slice + 1) * kItems / kSlices; ++item) {
                other(item);
            }
            __builtin_amdgcn_sched_barrier(0);
        }

        // Chunk end of tile k - 1: the odd halves are added to the even ones
        // through s_y (free once every wave is past the block above), G
        // first, then S; the even waves store the partials.
        if (prev.item < items && cur.item != prev.item) {
            const int lane_o = opaque_int(lane);
            f32x4* xchg = reinterpret_cast<f32x4*>(s_y);
            __syncthreads();
            if (unit_active && unit_half == 1) {
#pragma unroll
                for (int i = 0; i < NGB; ++i) {
                    xchg[(unit_head * NGB + i) * 64 + lane_o] = acc_g[i];
                }
            }
            __syncthreads();
            if (unit_active && unit_half == 0) {
#pragma unroll
                for (int i = 0; i < NGB; ++i) {
                    acc_g[i] += xchg[(unit_head * NGB + i) * 64 + lane_o];
                }
            }
            __syncthreads();
            if (unit_active && unit_half == 1) {
#pragma unroll
                for (int x = 0; x < NRB; ++x) {
#pragma unroll
                    for (int c = 0; c < 2 * CPW; ++c) {
                        xchg[((unit_head * NRB + x) * 2 * CPW + c) * 64 + lane_o] = acc_s[x][c];
                    }
                }
            }
            __syncthreads();
            if (unit_active && unit_half == 0) {
#pragma unroll
                for (int x = 0; x < NRB; ++x) {
#pragma unroll
                    for (int c = 0; c < 2 * CPW; ++c) {
                        acc_s[x][c] += xchg[((unit_head * NRB + x) * 2 * CPW + c) * 64 + lane_o];
                    }
                }
                const int q = lane_o & 15;
                const int g = lane_o >> 4;
                float* part = a.partials +
                              ((prev.b * a.heads + h0 + unit_head) * a.chunks + prev.chunk) * a.partial_stride;
                store_gram_partial<R>(part, acc_g, q, g);
                store_cross_partial<R, CPW>(part + R * R, acc_s, q, g, 0, d);
            }
            clear_units();
        }
        __syncthreads();

        // Tile k + 1's keep flags and phases; they go to buffers that nothing
        // reads in this step.
        write_stage_meta(next, k2 ^ 1, k3 == 2 ? 0 : k3 + 1);

        // Epilogue of tile k: bias, row mask and BF16 rounding into s_y.
        if (cur.item < items) {
#pragma unroll
            for (int mb = 0; mb < 2; ++mb) {
                const int mr = mb * 32 + row_k;
                const bool keep = s_keep[k2][mr] != 0;
#pragma unroll
                for (int qd = 0; qd < 4; ++qd) {
                    const int c = wave * 32 + 8 * qd + 4 * half_k;
                    const f32x4 bias = *reinterpret_cast<const f32x4*>(&s_bias[c]);
                    const float v0 = keep ? acc[mb][4 * qd + 0] + bias[0] : 0.0f;
                    const float v1 = keep ? acc[mb][4 * qd + 1] + bias[1] : 0.0f;
                    const float v2 = keep ? acc[mb][4 * qd + 2] + bias[2] : 0.0f;
                    const float v3 = keep ? acc[mb][4 * qd + 3] + bias[3] : 0.0f;
                    u32x2 packed;
                    packed.x = pack_bf16(v0, v1);
                    packed.y = pack_bf16(v2, v3);
                    *reinterpret_cast<u32x2*>(&s_y[mr * YP + c]) = packed;
                }
            }
        }
        __syncthreads();
    };

    if (slot >= items) {
        return;
    }
    // LDS that an absent previous tile is reduced from starts at zero.
    for (int i = tid; i < kPrTile * YP / 2; i += kThreads) {
        reinterpret_cast<uint32_t*>(s_y)[i] = 0u;
    }
    for (int i = tid; i < 3 * kPrTile * PHP; i += kThreads) {
        (&s_ph[0][0])[i] = 0u;
    }
    Stage stage_a;
    Stage stage_b;
    Cursor cur = open_item(slot);
    Cursor nx1 = advance(cur);
    load_stage(stage_a, cur);
    load_stage(stage_b, nx1);
    __syncthreads();
    write_stage(stage_a, 0, 0);
    __syncthreads();
    Cursor prev = cur;
    prev.item = items;
    // Tile k's loads go to stage k % 2, its x to s_x[k % 2] and its phases to
    // s_ph[k % 3]; the loop body is unrolled twice so that the stages keep
    // fixed registers.  One extra step after the last tile drains it.
    int k3 = 0;
    while (true) {
        Cursor nx2 = nx1.item < items ? advance(nx1) : nx1;
        step(prev, cur, nx1, nx2, stage_a, stage_b, k3, 0);
        if (cur.item >= items) {
            break;
        }
        prev = cur;
        cur = nx1;
        nx1 = nx2;
        k3 = k3 == 2 ? 0 : k3 + 1;
        nx2 = nx1.item < items ? advance(nx1) : nx1;
        step(prev, cur, nx1, nx2, stage_b, stage_a, k3, 1);
        if (cur.item >= items) {
            break;
        }
        prev = cur;
        cur = nx1;
        nx1 = nx2;
        k3 = k3 == 2 ? 0 : k3 + 1;
    }
}

namespace {

template <int KSTEPS, int R, int CPW>
hipError_t launch_pr_x(const ProjectReduceArgs& a, int x_dtype, int grid, hipStream_t stream) {
    const dim3 block(pr_waves<KSTEPS>() * 64);
    if (x_dtype == LSSO_HIP_F16) {
        project_reduce_kernel<KSTEPS, R, CPW, LSSO_HIP_F16><<<grid, block, 0, stream>>>(a);
    } else {
        project_reduce_kernel<KSTEPS, R, CPW, LSSO_HIP_BF16><<<grid, block, 0, stream>>>(a);
    }
    return hipGetLastError();
}

template <int KSTEPS, int R>
hipError_t launch_pr_c(const ProjectReduceArgs& a, int x_dtype, int grid, hipStream_t stream) {
    return a.head_dim > 32 ? launch_pr_x<KSTEPS, R, 2>(a, x_dtype, grid, stream)
                           : launch_pr_x<KSTEPS, R, 1>(a, x_dtype, grid, stream);
}

template <int KSTEPS>
hipError_t launch_pr_r(int rank, const ProjectReduceArgs& a, int x_dtype, int grid,
                       hipStream_t stream) {
    switch (rank) {
        case 16: return launch_pr_c<KSTEPS, 16>(a, x_dtype, grid, stream);
        case 32: return launch_pr_c<KSTEPS, 32>(a, x_dtype, grid, stream);
        case 48: return launch_pr_c<KSTEPS, 48>(a, x_dtype, grid, stream);
        default: return launch_pr_c<KSTEPS, 64>(a, x_dtype, grid, stream);
    }
}

}  // namespace

hipError_t launch_project_reduce(int rank, const ProjectReduceArgs& a, int x_dtype, int grid,
                                 hipStream_t stream) {
    switch (pr_k_tier(a.in_features)) {
        case 8: return launch_pr_r<8>(rank, a, x_dtype, grid, stream);
        case 12: return launch_pr_r<12>(rank, a, x_dtype, grid, stream);
        case 16: return launch_pr_r<16>(rank, a, x_dtype, grid, stream);
        case 24: return launch_pr_r<24>(rank, a, x_dtype, grid, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace lsso_hip

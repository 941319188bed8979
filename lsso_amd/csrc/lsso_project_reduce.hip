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
// heads] ("virtual" columns).  The waves are specialized, so that each SIMD
// runs one MFMA-bound and one VALU-bound wave side by side:
//   - projection waves (the first half) keep the BF16 W rows of 64 virtual
//     columns each in registers for the whole launch, project tile k and
//     write its BF16 packed tile into LDS;
//   - reduction waves (the second half), one per head of the group, reduce
//     tile k - 1 from LDS in token order, store it to HBM, and stage the x,
//     phases and row mask of the following tiles (raw buffer loads two tiles
//     ahead, so that memory latency stays hidden).
// One barrier per tile separates the steps.  Workgroups are persistent over
// (sample, token chunk) items of one head group; the groups of one item sit
// on the same XCD so that the second read of an x tile hits that XCD's L2.

#include "lsso_device.h"
#include "lsso_internal.h"
#include "lsso_reduce.h"
#include "lsso_hip.h"

namespace lsso_hip {

namespace {

constexpr int kPrTile = 64;
constexpr int kPrXcds = 8;

// Waves per workgroup: 4 projection + 4 reduction waves (two per SIMD)
// while the projection waves' W (64 columns x K) fits; 2 + 2 (one per SIMD,
// with the accumulation registers) for K = 384.
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
    // One reduction wave per head; the group's columns fit the projection
    // waves' 64 columns each.
    int64_t group = (waves / 2 * 64) / (rank + head_dim);
    if (group > waves / 2) group = waves / 2;
    if (group > heads) group = heads;
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
    constexpr int kProj = kWaves / 2;               // projection waves
    constexpr int kIo = kWaves / 2 * 64;            // threads of the reduction waves
    constexpr int VW = kProj * 64;                  // virtual columns of a group
    constexpr int KP = 16 * KSTEPS + 8;             // x tile pitch (bf16)
    // Pitches of 2 (mod 8) dwords put the rows 8 apart that one reduction
    // read touches in different LDS banks.
    constexpr int YP = VW + 4;                      // packed tile pitch (bf16)
    constexpr int PHP = PAIRS + 2;                  // phase tile pitch (u32)
    constexpr int kChunksPerRow = 2 * KSTEPS;       // 8-element x pieces
    constexpr int kXChunks = kPrTile * kChunksPerRow / kIo;
    static_assert(kPrTile * kChunksPerRow % kIo == 0, "x tile split");
    constexpr int kPhasePieces = kPrTile * PAIRS / 4;  // 16-byte phase pieces
    constexpr int kPhaseChunks = (kPhasePieces + kIo - 1) / kIo;

    // x tiles: projected and next (double buffer); packed tiles: being
    // written and being reduced (double buffer); phases: being reduced,
    // projected and next (triple buffer); keep flags: projected and next.
    __shared__ __attribute__((aligned(16))) uint16_t s_x[2][kPrTile * KP];
    __shared__ __attribute__((aligned(16))) uint16_t s_y[2][kPrTile * YP];
    __shared__ __attribute__((aligned(16))) uint32_t s_ph[3][kPrTile * PHP];
    __shared__ int s_keep[2][kPrTile];
    __shared__ int s_keep_all[2];
    __shared__ __attribute__((aligned(16))) float s_bias[VW];
    __shared__ int s_col[VW];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

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
    if (slot >= items) {
        return;
    }

    // Packed column of a virtual column, or -1 past the group's columns.
    auto packed_column = [&](int64_t c) -> int64_t {
        if (c < hg * R) return h0 * R + c;
        if (c < hg * (R + d)) return a.heads * R + h0 * d + (c - hg * R);
        return -1;
    };
    for (int c = tid; c < VW; c += kWaves * 64) {
        const int64_t n = packed_column(c);
        s_col[c] = static_cast<int>(n);
        s_bias[c] = (a.bias != nullptr && n >= 0) ? a.bias[n] : 0.0f;
    }

    // A tile of the workgroup's sequence: tokens [t0, t0 + 64) of item
    // (sample b, chunk); item >= items marks the end of the sequence.  The
    // bookkeeping is 32-bit (the host keeps B * N below 2^31).
    const int n_items = static_cast<int>(items);
    const int n_slots = static_cast<int>(slots);
    const int n_chunks = static_cast<int>(a.chunks);
    const int chunk_tokens = static_cast<int>(a.chunk_tokens);
    const int length = static_cast<int>(a.length);
    struct Cursor {
        int item, b, chunk, end, t0;
    };
    auto open_item = [&](int item) {
        Cursor c;
        c.item = item;
        c.b = item / n_chunks;
        c.chunk = item - c.b * n_chunks;
        c.t0 = c.chunk * chunk_tokens;
        c.end = c.t0 + chunk_tokens < length ? c.t0 + chunk_tokens : length;
        return c;
    };
    auto advance = [&](const Cursor& c) {
        if (c.item >= n_items || c.t0 + kPrTile < c.end) {
            Cursor n = c;
            n.t0 += kPrTile;
            return n;
        }
        const int next_item = c.item + n_slots;
        if (next_item < n_items) {
            return open_item(next_item);
        }
        Cursor n = c;
        n.item = n_items;
        return n;
    };
    auto tile_rows = [&](const Cursor& c) -> int {
        return c.item < n_items ? (c.end - c.t0 < kPrTile ? c.end - c.t0 : kPrTile) : 0;
    };
    // First row of a cursor's tile in the [B * N] row space.
    auto tile_row0 = [&](const Cursor& c) -> int64_t {
        return static_cast<int64_t>(c.b) * length + c.t0;
    };

    if (wave < kProj) {
        // ----------------------------------------------------------------
        // Projection waves.
        const int lane_c = lane & 31;
        u32x4 wreg[2][KSTEPS];
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) {
            load_weight_row_k8<KSTEPS>(wreg[nb], a.weight, packed_column(wave * 64 + nb * 32 + lane_c), a.width, D, lane);
        }
        __syncthreads();   // s_bias, s_col and tile 0 are in LDS
        // The packed tile k - 1 (in s_y[(k - 1) & 1]) goes out during tile
        // k's MFMAs, as 16-byte pieces of the group's two column runs: this
        // wave's VMEM slots are idle while its MFMAs run.  Rows past the
        // chunk (or an absent tile) fall outside the buffer and are dropped.
        constexpr int kProjStores = kPrTile * VW / 8 / (kProj * 64);
        static_assert(kProjStores % 2 == 0 && KSTEPS % (kProjStores / 2) == 0, "store interleave");
        static_assert((kProj * 64) % (VW / 8) == 0, "store pieces keep their column");
        // Piece i of this thread: row tid / (VW / 8) + i * kPieceRows, the
        // same 8 virtual columns for every i, so one offset per thread serves
        // all pieces (plus a constant row stride).
        constexpr int kPieceRows = kProj * 64 / (VW / 8);
        const int store_row = tid / (VW / 8);
        const int store_c8 = 8 * (tid - store_row * (VW / 8));
        const int store_col = static_cast<int>(packed_column(store_c8));
        const uint32_t store_base = store_col >= 0
            ? 2u * static_cast<uint32_t>(store_row * static_cast<int>(a.width) + store_col) : kOutOfRange;
        const uint32_t store_step = 2u * static_cast<uint32_t>(kPieceRows * a.width);
        const int store_lds = store_row * YP + store_c8;
        auto read_piece = [&](const uint16_t* yprev, int i) {
            const u32x2 lo = *reinterpret_cast<const u32x2*>(&yprev[store_lds + i * kPieceRows * YP]);
            const u32x2 hi = *reinterpret_cast<const u32x2*>(&yprev[store_lds + i * kPieceRows * YP + 4]);
            return (u32x4){lo.x, lo.y, hi.x, hi.y};
        };
        auto write_piece = [&](const BufferRsrc& obuf, const u32x4& v, int i) {
            buffer_store16_stream(v, obuf, store_base + static_cast<uint32_t>(i) * store_step);
        };
        auto store_piece = [&](const BufferRsrc& obuf, const uint16_t* yprev, int i) {
            write_piece(obuf, read_piece(yprev, i), i);
        };
        auto store_buffer = [&](const Cursor& prev) {
            return make_buffer(a.packed + (a.packed != nullptr ? tile_row0(prev) * a.width : 0),
                               a.packed != nullptr ? int64_t{2} * tile_rows(prev) * a.width : 0);
        };
        Cursor cur = open_item(static_cast<int>(slot));
        Cursor prev = cur;
        prev.item = n_items;
        int k2 = 0;
        while (cur.item < n_items) {
            const uint16_t* xt = s_x[k2];
            uint16_t* yt = s_y[k2];
            const uint16_t* yprev = s_y[k2 ^ 1];
            const BufferRsrc obuf = store_buffer(prev);
            // Rows are all kept unless the tile is partial or masked.
            const bool all_keep = __builtin_amdgcn_readfirstlane(s_keep_all[k2]) != 0;
            // Two 32-row halves of the tile, each with both column blocks.
#pragma unroll 1
            for (int mb = 0; mb < 2; ++mb) {
                const int lane_o = opaque_int(lane);
                const int row_k = lane_o & 31;
                const int half_k = lane_o >> 5;
                const uint16_t* xrow = xt + (mb * 32 + row_k) * KP + 8 * half_k;
                // Everything this half reads from LDS besides the x fragments
                // is issued before its MFMAs, so no read waits inside the
                // loop: the epilogue's bias and row flag, and each packed
                // piece one store interval before its store.
                const int mr = mb * 32 + row_k;
                const bool keep = all_keep || s_keep[k2][mr] != 0;
                f32x4 bias[2][4];
#pragma unroll
                for (int nb = 0; nb < 2; ++nb) {
#pragma unroll
                    for (int qd = 0; qd < 4; ++qd) {
                        bias[nb][qd] = *reinterpret_cast<const f32x4*>(&s_bias[wave * 64 + nb * 32 + 8 * qd + 4 * half_k]);
                    }
                }
                constexpr int kHalfStores = kProjStores / 2;
                constexpr int kEvery = KSTEPS / kHalfStores;
                u32x4 piece = read_piece(yprev, mb * kHalfStores);
                // The FP32 bias is the accumulators' starting value (element
                // 4 qd + e of block nb is column 8 qd + 4 half + e of it).
                f32x16 acc[2];
#pragma unroll
                for (int nb = 0; nb < 2; ++nb) {
#pragma unroll
                    for (int qd = 0; qd < 4; ++qd) {
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            acc[nb][4 * qd + e] = bias[nb][qd][e];
                        }
                    }
                }
                // x fragments kXAhead K steps ahead of their MFMAs.
                constexpr int kXAhead = 3;
                u32x4 xf[kXAhead + 1];
#pragma unroll
                for (int ks = 0; ks < kXAhead; ++ks) {
                    xf[ks] = *reinterpret_cast<const u32x4*>(xrow + 16 * ks);
                }
#pragma unroll
                for (int ks = 0; ks < KSTEPS; ++ks) {
                    if (ks + kXAhead < KSTEPS) {
                        xf[(ks + kXAhead) % (kXAhead + 1)] =
                            *reinterpret_cast<const u32x4*>(xrow + 16 * (ks + kXAhead));
                    }
#pragma unroll
                    for (int nb = 0; nb < 2; ++nb) {
                        acc[nb] = mfma32x32x16(wreg[nb][ks], xf[ks % (kXAhead + 1)], acc[nb]);
                    }
                    if (ks % kEvery == kEvery - 1) {
                        const int i = mb * kHalfStores + ks / kEvery;
                        write_piece(obuf, piece, i);
                        if (ks / kEvery + 1 < kHalfStores) {
                            piece = read_piece(yprev, i + 1);
                        }
                    }
                    __builtin_amdgcn_sched_barrier(0);
                }
                // Row mask (only for a tile with dropped rows) and BF16
                // rounding into the packed tile.
                if (!all_keep) {
#pragma unroll
                    for (int nb = 0; nb < 2; ++nb) {
#pragma unroll
                        for (int i = 0; i < 16; ++i) {
                            acc[nb][i] = keep ? acc[nb][i] : 0.0f;
                        }
                    }
                }
#pragma unroll
                for (int nb = 0; nb < 2; ++nb) {
#pragma unroll
                    for (int qd = 0; qd < 4; ++qd) {
                        const int c = wave * 64 + nb * 32 + 8 * qd + 4 * half_k;
                        u32x2 packed;
                        packed.x = pack_bf16(acc[nb][4 * qd + 0], acc[nb][4 * qd + 1]);
                        packed.y = pack_bf16(acc[nb][4 * qd + 2], acc[nb][4 * qd + 3]);
                        *reinterpret_cast<u32x2*>(&yt[mr * YP + c]) = packed;
                    }
                }
            }
            __syncthreads();
            prev = cur;
            cur = advance(cur);
            k2 ^= 1;
        }
        // Drain: the last tile's packed store, beside the reduction waves'
        // last step.
        {
            const BufferRsrc obuf = store_buffer(prev);
#pragma unroll
            for (int i = 0; i < kProjStores; ++i) {
                store_piece(obuf, s_y[k2 ^ 1], i);
            }
        }
        __syncthreads();
        return;
    }

    // --------------------------------------------------------------------
    // Reduction waves: unit head = wave - kProj; the thread index io covers
    // the staging and store work.
    const int io = tid - kProj * 64;
    const int unit_head = wave - kProj;
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

    // Register stage of one tile: x pieces, phases, row mask byte, and the
    // tile's valid rows.  Loads go through raw buffers sized to the valid
    // rows: rows past the chunk (and an exhausted cursor) read as zeros
    // without a memory access.
    struct Stage {
        u32x4 x[kXChunks];
        u32x4 ph[kPhaseChunks];
        uint32_t mask;
        int rows;
    };
    // Per-thread addressing of the staging work: chunk i of thread io is x
    // piece io + i * kIo; when kIo is a multiple of the pieces per row, every
    // chunk of a thread sits in the same column at a fixed row stride, so a
    // single base plus constants addresses all of them.
    constexpr bool kRowStride = kIo % kChunksPerRow == 0;
    constexpr int kRowStep = kIo / kChunksPerRow;
    constexpr bool kPhaseStride = kIo % (PAIRS / 4) == 0;
    // A stage is loaded in two halves (`part` 0: row mask, phases and the
    // first half of the x pieces; 1: the rest), issued at the start and at
    // the end of a step: the wave's loads then wait less for the memory
    // pipeline behind the projection waves' packed stores (measured 0.8%
    // faster per call than issuing all of them at once, and slower again
    // with four parts).
    auto load_stage = [&](Stage& st, const Cursor& c, int part) {
        const int io_o = opaque_int(io);
        const int rows = tile_rows(c);
        st.rows = rows;
        if (part == 0) {
            const BufferRsrc mbuf = make_buffer(
                a.row_mask + (a.row_mask != nullptr ? tile_row0(c) : 0),
                a.row_mask != nullptr ? rows : 0);
            st.mask = buffer_load_byte(mbuf, static_cast<uint32_t>(io_o));
        }
        const BufferRsrc xbuf = make_buffer(
            static_cast<const uint16_t*>(a.x) + tile_row0(c) * D, int64_t{2} * rows * D);
        const int Di = static_cast<int>(D);
        if constexpr (kRowStride) {
            const int rr0 = io_o / kChunksPerRow;
            const int cc = io_o - rr0 * kChunksPerRow;
            const uint32_t base = 8 * cc < Di ? 2u * static_cast<uint32_t>(rr0 * Di + 8 * cc) : kOutOfRange;
#pragma unroll
            for (int i = 0; i < kXChunks; ++i) {
                if ((i < kXChunks / 2) == (part == 0)) {
                    st.x[i] = buffer_load16_stream(xbuf, base + 2u * static_cast<uint32_t>(i * kRowStep * Di));
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < kXChunks; ++i) {
                if ((i < kXChunks / 2) == (part == 0)) {
                    const int chunk = io_o + i * kIo;
                    const int rr = chunk / kChunksPerRow;
                    const int cc = chunk - rr * kChunksPerRow;
                    const uint32_t offset =
                        8 * cc < Di ? 2u * static_cast<uint32_t>(rr * Di + 8 * cc) : kOutOfRange;
                    st.x[i] = buffer_load16_stream(xbuf, offset);
                }
            }
        }
        if (part != 0) {
            return;
        }
        const BufferRsrc pbuf = make_buffer(a.phases + c.b * a.phase_batch_stride + int64_t{c.t0} * PAIRS,
                                            int64_t{4} * rows * PAIRS);
#pragma unroll
        for (int p = 0; p < kPhaseChunks; ++p) {
            const int piece = io_o + p * kIo;
            const uint32_t offset = (kPhasePieces % kIo == 0 || piece < kPhasePieces)
                                        ? 16u * static_cast<uint32_t>(piece) : kOutOfRange;
            st.ph[p] = buffer_load16(pbuf, offset);
        }
    };
    auto write_stage = [&](const Stage& st, int x_buf, int phase_buf) {
        const int io_o = opaque_int(io);
        if (io_o < kPrTile) {
            const bool keep = io_o < st.rows && (a.row_mask == nullptr || st.mask != 0);
            s_keep[x_buf][io_o] = keep;
            // The first reduction wave holds the tile's 64 rows.
            const bool all = __ballot(keep) == ~0ull;
            if (io_o == 0) {
                s_keep_all[x_buf] = all;
            }
        }
        auto convert = [&](const u32x4& raw) {
            u32x4 v;
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                uint32_t value = raw[p];
                if constexpr (XT == LSSO_HIP_F16) {
                    value = pack_bf16(f16_lo(value), f16_hi(value));
                }
                v[p] = value;
            }
            return v;
        };
        if constexpr (kRowStride) {
            const int rr0 = io_o / kChunksPerRow;
            const int cc = io_o - rr0 * kChunksPerRow;
            uint16_t* base = &s_x[x_buf][rr0 * KP + 8 * cc];
#pragma unroll
            for (int i = 0; i < kXChunks; ++i) {
                *reinterpret_cast<u32x4*>(base + i * kRowStep * KP) = convert(st.x[i]);
            }
        } else {
#pragma unroll
            for (int i = 0; i < kXChunks; ++i) {
                const int chunk = io_o + i * kIo;
                const int rr = chunk / kChunksPerRow;
                const int cc = chunk - rr * kChunksPerRow;
                *reinterpret_cast<u32x4*>(&s_x[x_buf][rr * KP + 8 * cc]) = convert(st.x[i]);
            }
        }
#pragma unroll
        for (int p = 0; p < kPhaseChunks; ++p) {
            const int piece = io_o + p * kIo;
            if (kPhasePieces % kIo == 0 || piece < kPhasePieces) {
                int rr, pc;
                if constexpr (kPhaseStride) {
                    const int rr0 = io_o / (PAIRS / 4);
                    pc = io_o - rr0 * (PAIRS / 4);
                    rr = rr0 + p * (kIo / (PAIRS / 4));
                } else {
                    rr = piece / (PAIRS / 4);
                    pc = piece - rr * (PAIRS / 4);
                }
                uint32_t* dst = &s_ph[phase_buf][rr * PHP + 4 * pc];
                *reinterpret_cast<u32x2*>(dst) = (u32x2){st.ph[p][0], st.ph[p][1]};
                *reinterpret_cast<u32x2*>(dst + 2) = (u32x2){st.ph[p][2], st.ph[p][3]};
            }
        }
    };

    // Reduction operands of this wave's head for the 32 tokens of half st
    // of a packed tile (the reduce_load layout: lane (q, g) holds tokens
    // 8 g .. 8 g + 7).  One base per operand; the rows are constant offsets.
    auto lds_tile = [&](ReduceTile<R, CPW>& t, const uint16_t* yt, const uint32_t* pt, int st) {
        const int lane_o = opaque_int(lane);
        const int q = lane_o & 15;
        const int g = lane_o >> 4;
        const uint16_t* rbase = yt + (32 * st + 8 * g) * YP + unit_head * R + 2 * PS * q;
        const uint32_t* pbase = pt + (32 * st + 8 * g) * PHP + PS * q;
        const uint16_t* cbase = yt + (32 * st + 8 * g) * YP + hg * R + unit_head * d + 2 * q;
        const bool pv = PS * q < PAIRS;
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) {
            if constexpr (PS == 2) {
                u32x2 r = {0u, 0u};
                u32x2 p = {0u, 0u};
                if (pv) {
                    r = *reinterpret_cast<const u32x2*>(rbase + jj * YP);
                    p = *reinterpret_cast<const u32x2*>(pbase + jj * PHP);
                }
                t.rel[jj][0] = r.x;
                t.rel[jj][1] = r.y;
                t.ph[jj][0] = p.x;
                t.ph[jj][1] = p.y;
            } else {
                t.rel[jj][0] = pv ? *reinterpret_cast<const uint32_t*>(rbase + jj * YP) : 0u;
                t.ph[jj][0] = pv ? pbase[jj * PHP] : 0u;
            }
#pragma unroll
            for (int c = 0; c < CPW; ++c) {
                t.con[jj][c] = 2 * (16 * c + q) < d
                    ? *reinterpret_cast<const uint32_t*>(cbase + jj * YP + 32 * c)
                    : 0u;
            }
        }
    };

    // One step for tile k (`cur`): loads of tile k + 2 (in two halves, around
    // the reductions), reductions and (if it closes its chunk) partials of
    // tile k - 1, tile k + 1 into LDS.
    auto step = [&](const Cursor& prev, const Cursor& cur, const Cursor& nx1, const Cursor& ahead,
                    Stage& load, const Stage& next, int k2, int k3) {
        load_stage(load, ahead, 0);
        if (prev.item < n_items) {
            const uint16_t* yt = s_y[k2 ^ 1];
            const uint32_t* pt = s_ph[k3 == 0 ? 2 : k3 - 1];
            if (unit_active) {
                if constexpr (R <= 32) {
                    // Both halves' operands are read before either is
                    // reduced, so the second half's LDS reads are in flight
                    // during the first half's math (rows past a partial tile
                    // read stale LDS and are not reduced).
                    ReduceTile<R, CPW> t0;
                    ReduceTile<R, CPW> t1;
                    lds_tile(t0, yt, pt, 0);
                    lds_tile(t1, yt, pt, 1);
                    reduce_compute<R, CPW>(t0, true, acc_g, acc_s);
                    if (prev.t0 + 32 < prev.end) {
                        reduce_compute<R, CPW>(t1, true, acc_g, acc_s);
                    }
                } else {
                    // One half at a time: the operands of one 32-token half
                    // are live at once.
#pragma unroll 1
                    for (int st = 0; st < 2; ++st) {
                        if (prev.t0 + 32 * st < prev.end) {
                            ReduceTile<R, CPW> t;
                            lds_tile(t, yt, pt, st);
                            reduce_compute<R, CPW>(t, true, acc_g, acc_s);
                        }
                    }
                }
            }
            if (cur.item != prev.item) {
                if (unit_active) {
                    const int q = lane & 15;
                    const int g = lane >> 4;
                    float* part = a.partials +
                                  ((prev.b * a.heads + h0 + unit_head) * a.chunks + prev.chunk) *
                                      a.partial_stride;
                    store_gram_partial<R>(part, acc_g, q, g);
                    store_cross_partial<R, CPW>(part + R * R, acc_s, q, g, 0, d);
                }
                clear_units();
            }
        }
        load_stage(load, ahead, 1);
        if (nx1.item < n_items) {
            write_stage(next, k2 ^ 1, k3 == 2 ? 0 : k3 + 1);
        }
        __syncthreads();
    };

    if constexpr (R > 32) {
        // From rank 48 on the reductions hold more registers than two
        // stages leave free, so one stage serves: a step first commits tile
        // k + 1 (loaded during the previous step) to LDS, then issues the
        // loads of tile k + 2 into the same registers, then reduces tile
        // k - 1.  The loads have one step to arrive.
        Stage st;
        Cursor cur = open_item(static_cast<int>(slot));
        Cursor nx1 = advance(cur);
        load_stage(st, cur, 0);
        load_stage(st, cur, 1);
        write_stage(st, 0, 0);
        load_stage(st, nx1, 0);
        load_stage(st, nx1, 1);
        __syncthreads();   // s_bias, s_col and tile 0 are in LDS
        Cursor prev = cur;
        prev.item = n_items;
        int k2 = 0;
        int k3 = 0;
        while (true) {
            const Cursor nx2 = advance(nx1);
            if (nx1.item < n_items) {
                write_stage(st, k2 ^ 1, k3 == 2 ? 0 : k3 + 1);
            }
            load_stage(st, nx2, 0);
            load_stage(st, nx2, 1);
            if (prev.item < n_items) {
                const uint16_t* yt = s_y[k2 ^ 1];
                const uint32_t* pt = s_ph[k3 == 0 ? 2 : k3 - 1];
                if (unit_active) {
#pragma unroll 1
                    for (int half = 0; half < 2; ++half) {
                        if (prev.t0 + 32 * half < prev.end) {
                            ReduceTile<R, CPW> t;
                            lds_tile(t, yt, pt, half);
                            reduce_compute<R, CPW>(t, true, acc_g, acc_s);
                        }
                    }
                }
                if (cur.item != prev.item) {
                    if (unit_active) {
                        // The store offsets are formed here, once per chunk,
                        // rather than kept in registers across the loop.
                        const int lane_o = opaque_int(lane);
                        const int q = lane_o & 15;
                        const int g = lane_o >> 4;
                        float* part = a.partials +
                                      ((prev.b * a.heads + h0 + unit_head) * a.chunks + prev.chunk) *
                                          a.partial_stride;
                        store_gram_partial<R>(part, acc_g, q, g);
                        store_cross_partial<R, CPW>(part + R * R, acc_s, q, g, 0, d);
                    }
                    clear_units();
                }
            }
            __syncthreads();
            if (cur.item >= n_items) {
                break;
            }
            prev = cur;
            cur = nx1;
            nx1 = nx2;
            k2 ^= 1;
            k3 = k3 == 2 ? 0 : k3 + 1;
        }
        return;
    }

    Stage stage_a;
    Stage stage_b;
    Cursor cur = open_item(static_cast<int>(slot));
    Cursor nx1 = advance(cur);
    load_stage(stage_a, cur, 0);
    load_stage(stage_a, cur, 1);
    load_stage(stage_b, nx1, 0);
    load_stage(stage_b, nx1, 1);
    write_stage(stage_a, 0, 0);
    __syncthreads();   // s_bias, s_col and tile 0 are in LDS
    Cursor prev = cur;
    prev.item = n_items;
    // Tile k is staged in registers stage k % 2, its x and packed tile in
    // buffers k % 2 and its phases in buffer k % 3; the loop body is
    // unrolled twice so that the stages keep fixed registers.  The step
    // after the last tile (cur exhausted) drains it.
    int k3 = 0;
    while (true) {
        Cursor nx2 = advance(nx1);
        step(prev, cur, nx1, nx2, stage_a, stage_b, 0, k3);
        if (cur.item >= n_items) {
            break;
        }
        prev = cur;
        cur = nx1;
        nx1 = nx2;
        k3 = k3 == 2 ? 0 : k3 + 1;
        nx2 = advance(nx1);
        step(prev, cur, nx1, nx2, stage_b, stage_a, 1, k3);
        if (cur.item >= n_items) {
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
        dispatch(project_reduce_kernel<KSTEPS, R, CPW, LSSO_HIP_F16>, grid, block, stream, a);
    } else {
        dispatch(project_reduce_kernel<KSTEPS, R, CPW, LSSO_HIP_BF16>, grid, block, stream, a);
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

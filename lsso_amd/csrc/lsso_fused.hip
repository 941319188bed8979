// gfx950 apply fused with the output projection.
//
//   mixed = bf16(eta C + rot(R) M')                 (apply, reference.py:500-572)
//   y     = cast(bf16(mixed) bf16(W_o)^T + b_o)     (output projection, reference.py:20-75)
//
// One persistent workgroup of 8 waves owns a contiguous token range of one
// sample and walks it in 32-token tiles, with the waves split by role (one
// of each per SIMD, so one wave's VALU work overlaps the other's MFMAs):
//   - 4 apply waves (two heads each for H > 4) turn tile k's packed rows
//     (BF16, R and C of every head, in LDS) into its mixed block with the
//     apply MFMAs (the same operand records, MFMA order and rounding as the
//     standalone apply), write it, BF16-rounded, into an LDS tile
//     [32 tokens, D], and stage the rows and phases of the next tiles;
//   - 4 projection waves multiply tile k - 1's mixed tile by their resident
//     BF16 W_o slice (64 output features each) on v_mfma_f32_32x32x16_bf16,
//     in the standalone projection's K order, add the FP32 bias, zero masked
//     rows and write the rounded output as 16-byte pieces of whole rows.
// One barrier per tile.  The mixed tensor therefore never reaches HBM, and
// the result is bitwise the same as apply followed by the projection.

#include "lsso_device.h"
#include "lsso_internal.h"
#include "lsso_hip.h"

namespace lsso_hip {

constexpr int kMixRows = 32;                       // tokens per tile
constexpr int kMixWaves = 8;
constexpr int kMixThreads = 64 * kMixWaves;
constexpr int kMixProjWaves = 4;                   // waves 0..3: output projection
constexpr int kMixApplyWaves = kMixWaves - kMixProjWaves;
constexpr int kMixIoThreads = 64 * kMixApplyWaves; // apply waves also stage the rows
// Packed rows (BF16) of up to 512 columns, or of up to 640 in a second tier
// (rank 48 at H = 8, d = 32: W = 640), whose larger packed tiles still fit
// LDS (about 144 KB) and whose staging takes 10 instead of 8 16-byte pieces
// per thread.
constexpr int kMixMaxWidth = 640;
template <int WMAX>
constexpr int mix_pitch() { return WMAX + 8; }      // LDS row pitch of the packed tile
constexpr int kMixKSteps = 16;                     // D <= 256
constexpr int kMixDPitch = 16 * kMixKSteps + 8;    // LDS row pitch of the mixed tile
constexpr int kMixStPitch = 64 + 8;                // LDS row pitch of a projection wave's output
template <int WMAX>
constexpr int mix_chunks() { return kMixRows * WMAX / 8 / kMixIoThreads; }

bool mix_project_supported(int64_t rank, int64_t heads, int64_t head_dim, int64_t width) {
    const bool rank_ok = rank == 16 || rank == 32 || rank == 48 || rank == 64;
    return rank_ok && heads >= 1 && heads <= 2 * kMixApplyWaves && head_dim >= 16 && head_dim % 16 == 0 &&
           head_dim <= 64 && heads * head_dim <= 16 * kMixKSteps && width <= kMixMaxWidth &&
           width % 8 == 0;
}

int mix_project_tile_rows() { return kMixRows; }

// HPW: heads per apply wave (1 for H <= 4, else 2); DEPTH: row tiles staged
// in registers ahead of the one being applied (1 or 2); WMAX: the packed row
// tier (512 or 640 columns); MIXED: also store the mixed tiles (a.mixed);
// MASKED: a row mask is given (a.row_mask).  Without one no mask byte is
// loaded: its load, carried from step to step, made the compiler wait at
// the end of every step for all the loads in flight.
template <int R, int NFB, int YT, int DEPTH, int HPW, int WMAX, bool MIXED, bool MASKED>
__global__ __launch_bounds__(kMixThreads) void mix_project_kernel(MixProjectArgs a) {
    using AL = ApplyLayout<R>;
    constexpr int kMixPitch = mix_pitch<WMAX>();
    constexpr int kMixChunks = mix_chunks<WMAX>();
    constexpr int PAIRS = R / 2;
    constexpr int PHP = PAIRS + 4;                 // LDS phase row pitch (u32)
    constexpr int S32 = AL::kSteps32 > 0 ? AL::kSteps32 : 1;
    constexpr int S16 = AL::kSteps16 > 0 ? AL::kSteps16 : 1;
    __shared__ __attribute__((aligned(16))) uint16_t s_pk[2][kMixRows * kMixPitch];
    __shared__ __attribute__((aligned(16))) uint32_t s_ph[2][kMixRows * PHP];
    __shared__ __attribute__((aligned(16))) uint16_t s_mx[2][kMixRows * kMixDPitch];
    __shared__ __attribute__((aligned(16))) uint16_t s_st[kMixProjWaves][kMixRows * kMixStPitch];
    __shared__ __attribute__((aligned(16))) float s_bias[16 * kMixKSteps];
    __shared__ uint8_t s_keep[3][kMixRows];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int64_t b = blockIdx.x / a.ranges;
    const int64_t range = blockIdx.x - b * a.ranges;
    const int64_t begin = range * a.range_tokens;
    const int64_t end = a.length < begin + a.range_tokens ? a.length : begin + a.range_tokens;
    if (begin >= end) {
        return;  // uniform over the workgroup
    }
    const int64_t H = a.heads;
    const int64_t d = a.head_dim;
    const int64_t D = a.out_features;
    const int64_t W = a.width;
    const int Di = static_cast<int>(D);
    const int begin_i = static_cast<int>(begin);
    const int end_i = static_cast<int>(end);
    const int n_tiles = (end_i - begin_i + kMixRows - 1) / kMixRows;
    auto tile_t0 = [&](int t) { return begin_i + t * kMixRows; };
    auto tile_rows = [&](int t) { return end_i - tile_t0(t) < kMixRows ? end_i - tile_t0(t) : kMixRows; };

    for (int c = tid; c < 16 * kMixKSteps; c += kMixThreads) {
        s_bias[c] = (a.bias != nullptr && c < D) ? a.bias[c] : 0.0f;
    }
    // The mixed tiles' columns past D are the zero K padding of the product.
    for (int i = tid; i < 2 * kMixRows * kMixDPitch / 8; i += kMixThreads) {
        reinterpret_cast<u32x4*>(&s_mx[0][0])[i] = (u32x4){0u, 0u, 0u, 0u};
    }

    // Step k (one barrier each, k = 0 .. n_tiles): the apply waves turn tile
    // k's rows into its mixed tile and move tile k + 1's rows into LDS; the
    // projection waves project tile k - 1's mixed tile and store its output.
    if (wave < kMixProjWaves) {
        // ----------------------------------------------------------------
        // Projection waves: output features n0 .. n0 + 63, resident BF16
        // W_o rows, the standalone projection's K order and rounding.
        const int n0 = 64 * wave;
        const int lane_c = lane & 31;
        const int half = lane >> 5;
        const int ksteps = (Di + 15) / 16;
        u32x4 wreg[2][kMixKSteps];
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) {
            const int n = n0 + 32 * nb + lane_c;
            load_weight_row_k8<kMixKSteps>(wreg[nb], a.weight, n < Di ? n : -1, D, D, lane);
        }
        // Output pieces of this lane: row p / 8, features n0 + 8 (p % 8) ..,
        // for p = lane + 64 i (16 bytes each).
        uint16_t* stage = s_st[wave];
        uint32_t piece_off[kMixRows * 8 / 64];
        int piece_lds[kMixRows * 8 / 64];
#pragma unroll
        for (int i = 0; i < kMixRows * 8 / 64; ++i) {
            const int p = lane + 64 * i;
            const int row = p >> 3;
            const int c8 = 8 * (p & 7);
            piece_lds[i] = row * kMixStPitch + c8;
            piece_off[i] = n0 + c8 < Di ? 2u * static_cast<uint32_t>(row * Di + n0 + c8) : kOutOfRange;
        }
        __syncthreads();   // bias, zero padding and tile 0's rows are in LDS
        const bool active = n0 < Di;
        for (int k = 0; k <= n_tiles; ++k) {
            if (k >= 1 && active) {
                const int t = k - 1;
                const uint16_t* xt = s_mx[t & 1];
                const bool keep = s_keep[t % 3][lane_c] != 0;
                f32x4 bias[2][4];
#pragma unroll
                for (int nb = 0; nb < 2; ++nb) {
#pragma unroll
                    for (int qd = 0; qd < 4; ++qd) {
                        bias[nb][qd] = *reinterpret_cast<const f32x4*>(&s_bias[n0 + 32 * nb + 8 * qd + 4 * half]);
                    }
                }
                // The FP32 bias is the accumulators' starting value (element
                // 4 qd + e of block nb is feature n0 + 32 nb + 8 qd + 4 half + e).
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
                const uint16_t* xrow = xt + lane_c * kMixDPitch + 8 * half;
                // Mixed fragments kXAhead K steps ahead of their MFMAs.
                constexpr int kXAhead = 3;
                u32x4 xf[kXAhead + 1];
#pragma unroll
                for (int ks = 0; ks < kXAhead; ++ks) {
                    xf[ks] = *reinterpret_cast<const u32x4*>(xrow + 16 * ks);
                }
#pragma unroll
                for (int ks = 0; ks < kMixKSteps; ++ks) {
                    if (ks + kXAhead < kMixKSteps) {
                        xf[(ks + kXAhead) % (kXAhead + 1)] =
                            *reinterpret_cast<const u32x4*>(xrow + 16 * (ks + kXAhead));
                    }
                    if (ks < ksteps) {
#pragma unroll
                        for (int nb = 0; nb < 2; ++nb) {
                            acc[nb] = mfma32x32x16(wreg[nb][ks], xf[ks % (kXAhead + 1)], acc[nb]);
                        }
                    }
                }
                // Row mask (only for a tile with dropped rows) and rounding
                // into this wave's output stage, then 16-byte pieces of whole
                // rows to HBM.
                if (__ballot(keep) != ~0ull) {
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
                        const int c = 32 * nb + 8 * qd + 4 * half;
                        const float v0 = acc[nb][4 * qd + 0];
                        const float v1 = acc[nb][4 * qd + 1];
                        const float v2 = acc[nb][4 * qd + 2];
                        const float v3 = acc[nb][4 * qd + 3];
                        u32x2 packed;
                        if constexpr (YT == LSSO_HIP_BF16) {
                            packed.x = pack_bf16(v0, v1);
                            packed.y = pack_bf16(v2, v3);
                        } else {
                            packed.x = pack_f16(v0, v1);
                            packed.y = pack_f16(v2, v3);
                        }
                        *reinterpret_cast<u32x2*>(stage + lane_c * kMixStPitch + c) = packed;
                    }
                }
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                const BufferRsrc ybuf = make_buffer(
                    static_cast<uint16_t*>(a.y) + (b * a.length + tile_t0(t)) * D, int64_t{2} * tile_rows(t) * Di);
#pragma unroll
                for (int i = 0; i < kMixRows * 8 / 64; ++i) {
                    buffer_store16(*reinterpret_cast<const u32x4*>(stage + piece_lds[i]), ybuf, piece_off[i]);
                }
            }
            if (MIXED && k >= 1) {
                // The training entry also keeps the mixed tile (the output
                // projection's backward needs it): 16-byte pieces of whole
                // rows, from the LDS tile the MFMAs above read.
                const int t = k - 1;
                const uint16_t* xt = s_mx[t & 1];
                const int row_pieces = Di / 8;
                const BufferRsrc mbuf = make_buffer(a.mixed + (b * a.length + tile_t0(t)) * D,
                                                    int64_t{2} * tile_rows(t) * Di);
                for (int p = wave * 64 + lane; p < kMixRows * row_pieces; p += 64 * kMixProjWaves) {
                    const int row = p / row_pieces;
                    const int c8 = 8 * (p - row * row_pieces);
                    buffer_store16(*reinterpret_cast<const u32x4*>(xt + row * kMixDPitch + c8), mbuf,
                                   2u * static_cast<uint32_t>(row * Di + c8));
                }
            }
            __syncthreads();
        }
        return;
    }

    // --------------------------------------------------------------------
    // Apply waves: heads j and j + 4 (j = wave - 4), the standalone apply's
    // operand records, MFMA order and rounding; thread io stages the rows.
    const int j = wave - kMixProjWaves;
    const int io = tid - 64 * kMixProjWaves;
    u32x4 op_hi32[HPW][NFB][S32];
    u32x4 op_lo32[HPW][NFB][S32];
    u32x2 op_hi16[HPW][NFB][S16];
    u32x2 op_lo16[HPW][NFB][S16];
    float eta[HPW];
#pragma unroll
    for (int u = 0; u < HPW; ++u) {
        const int64_t h = j + kMixApplyWaves * u < H ? j + kMixApplyWaves * u : 0;
        eta[u] = bounded_complement(a.eta_raw[h]);
        const int64_t system = b * H + h;
#pragma unroll
        for (int f = 0; f < NFB; ++f) {
            const bool live = f < a.feature_blocks;
            const uint16_t* record =
                a.mop + ((system * a.feature_blocks + (live ? f : 0)) * 64 + lane) * AL::kLaneHalfs;
#pragma unroll
            for (int s = 0; s < AL::kSteps32; ++s) {
                op_hi32[u][f][s] = *reinterpret_cast<const u32x4*>(record + AL::offset32(s));
                op_lo32[u][f][s] = *reinterpret_cast<const u32x4*>(record + AL::offset32(s) + 8);
            }
#pragma unroll
            for (int s = 0; s < AL::kSteps16; ++s) {
                op_hi16[u][f][s] = *reinterpret_cast<const u32x2*>(record + AL::offset16(s));
                op_lo16[u][f][s] = *reinterpret_cast<const u32x2*>(record + AL::offset16(s) + 4);
            }
        }
    }

    // Staging: a tile's packed rows are one contiguous block, so chunk c of
    // this thread is bytes 16 (io + c kMixIoThreads) of it; its LDS slot
    // (padded pitch) is fixed per thread.  Loads go through raw buffers sized
    // to the tile's valid rows, so rows past the range read as zeros.
    const int Wi = static_cast<int>(W);
    const int row_chunks = Wi / 8;
    const int tile_chunks = kMixRows * row_chunks;
    int lds_chunk[kMixChunks];
#pragma unroll
    for (int c = 0; c < kMixChunks; ++c) {
        const int idx = io + c * kMixIoThreads;
        const int row = idx / row_chunks;
        lds_chunk[c] = idx < tile_chunks ? row * kMixPitch + 8 * (idx - row * row_chunks) : -1;
    }
    const int phase_lds = io < kMixRows * (PAIRS / 4) ? (io / (PAIRS / 4)) * PHP + 4 * (io % (PAIRS / 4)) : -1;
    const uint16_t* sample_rows = a.projected + b * a.length * W;
    const uint32_t* sample_phases = a.phases + b * a.phase_batch_stride;
    struct Stage {
        u32x4 chunk[kMixChunks];
        u32x4 phase;
        uint32_t mask;
    };
    auto fetch = [&](Stage& st, int t) {
        const int rows = tile_rows(t);
        const int t0 = tile_t0(t);
        const BufferRsrc pk = make_buffer(sample_rows + static_cast<int64_t>(t0) * Wi, int64_t{2} * rows * Wi);
#pragma unroll
        for (int c = 0; c < kMixChunks; ++c) {
            st.chunk[c] = buffer_load16_stream(pk, 16u * static_cast<uint32_t>(io + c * kMixIoThreads));
        }
        const BufferRsrc ph = make_buffer(sample_phases + static_cast<int64_t>(t0) * PAIRS,
                                          int64_t{4} * rows * PAIRS);
        st.phase = buffer_load16(ph, phase_lds >= 0 ? 16u * static_cast<uint32_t>(io) : kOutOfRange);
        if constexpr (MASKED) {
            const BufferRsrc mbuf = make_buffer(a.row_mask + b * a.length + t0, rows);
            st.mask = buffer_load_byte(mbuf, static_cast<uint32_t>(io < kMixRows ? io : kMixRows));
        }
    };
    auto commit = [&](const Stage& st, int t) {
        uint16_t* pk = s_pk[t & 1];
#pragma unroll
        for (int c = 0; c < kMixChunks; ++c) {
            if (lds_chunk[c] >= 0) {
                *reinterpret_cast<u32x4*>(pk + lds_chunk[c]) = st.chunk[c];
            }
        }
        if (phase_lds >= 0) {
            *reinterpret_cast<u32x4*>(s_ph[t & 1] + phase_lds) = st.phase;
        }
        if (io < kMixRows) {
            s_keep[t % 3][io] = io < tile_rows(t) && (!MASKED || st.mask != 0);
        }
    };

    // Mixed tile t of this wave's heads into s_mx[t & 1], 16-token sub-tiles.
    // All LDS operands of the tile (every head slot and sub-tile) are read
    // first, so the reads of later sub-tiles are in flight during the math
    // of earlier ones.
    struct ApplyIn {
        u32x4 rel32[S32];
        u32x4 ph32[S32];
        u32x2 rel16[S16];
        u32x2 ph16[S16];
        u32x2 con[NFB];
    };
    auto apply_tile = [&](int t) {
        const uint16_t* pk = s_pk[t & 1];
        const uint32_t* phs = s_ph[t & 1];
        uint16_t* mx = s_mx[t & 1];
        const int q = lane & 15;
        const int g = lane >> 4;
        ApplyIn in[HPW][kMixRows / 16];
#pragma unroll
        for (int u = 0; u < HPW; ++u) {
            const int64_t h = j + kMixApplyWaves * u < H ? j + kMixApplyWaves * u : j;
#pragma unroll
            for (int sub = 0; sub < kMixRows / 16; ++sub) {
                const int r = sub * 16 + q;
                const uint16_t* prow = pk + r * kMixPitch;
                const uint32_t* phrow = phs + r * PHP;
#pragma unroll
                for (int s = 0; s < AL::kSteps32; ++s) {
                    const int first_rank = 32 * s + 8 * g;
                    in[u][sub].rel32[s] = *reinterpret_cast<const u32x4*>(prow + h * R + first_rank);
                    in[u][sub].ph32[s] = *reinterpret_cast<const u32x4*>(phrow + first_rank / 2);
                }
#pragma unroll
                for (int s = 0; s < AL::kSteps16; ++s) {
                    const int first_rank = 16 * s + 4 * g;
                    in[u][sub].rel16[s] = *reinterpret_cast<const u32x2*>(prow + h * R + first_rank);
                    in[u][sub].ph16[s] = *reinterpret_cast<const u32x2*>(phrow + first_rank / 2);
                }
#pragma unroll
                for (int f = 0; f < NFB; ++f) {
                    const int64_t feature = h * d + 16 * (f < a.feature_blocks ? f : 0) + 4 * g;
                    in[u][sub].con[f] = *reinterpret_cast<const u32x2*>(prow + H * R + feature);
                }
            }
        }
#pragma unroll
        for (int sub = 0; sub < kMixRows / 16; ++sub) {
#pragma unroll
            for (int u = 0; u < HPW; ++u) {
                const int64_t h = j + kMixApplyWaves * u;
                if (h >= H) {
                    continue;   // wave-uniform
                }
                const ApplyIn& op = in[u][sub];
                const int r = sub * 16 + q;
                u32x4 b_hi32[S32];
                u32x4 b_lo32[S32];
#pragma unroll
                for (int s = 0; s < AL::kSteps32; ++s) {
                    float v[8];
#pragma unroll
                    for (int p = 0; p < 4; ++p) {
                        rotate_pair(op.rel32[s][p], op.ph32[s][p], v[2 * p], v[2 * p + 1]);
                    }
#pragma unroll
                    for (int p = 0; p < 4; ++p) {
                        uint32_t hi, lo;
                        split_bf16(v[2 * p], v[2 * p + 1], hi, lo);
                        b_hi32[s][p] = hi;
                        b_lo32[s][p] = lo;
                    }
                }
                u32x2 b_hi16[S16];
                u32x2 b_lo16[S16];
#pragma unroll
                for (int s = 0; s < AL::kSteps16; ++s) {
                    float v[4];
#pragma unroll
                    for (int p = 0; p < 2; ++p) {
                        rotate_pair(op.rel16[s][p], op.ph16[s][p], v[2 * p], v[2 * p + 1]);
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
                for (int f = 0; f < NFB; ++f) {
                    if (f < a.feature_blocks) {
                        f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                        for (int s = 0; s < AL::kSteps32; ++s) {
                            acc = mfma16x16x32(op_hi32[u][f][s], b_hi32[s], acc);
                            acc = mfma16x16x32(op_hi32[u][f][s], b_lo32[s], acc);
                            acc = mfma16x16x32(op_lo32[u][f][s], b_hi32[s], acc);
                        }
#pragma unroll
                        for (int s = 0; s < AL::kSteps16; ++s) {
                            acc = mfma16x16x16(op_hi16[u][f][s], b_hi16[s], acc);
                            acc = mfma16x16x16(op_hi16[u][f][s], b_lo16[s], acc);
                            acc = mfma16x16x16(op_lo16[u][f][s], b_hi16[s], acc);
                        }
                        const int64_t feature = h * d + 16 * f + 4 * g;
                        const u32x2 c = op.con[f];
                        u32x2 y;
                        y.x = pack_bf16(fmaf(eta[u], bf16_lo(c.x), acc[0]), fmaf(eta[u], bf16_hi(c.x), acc[1]));
                        y.y = pack_bf16(fmaf(eta[u], bf16_lo(c.y), acc[2]), fmaf(eta[u], bf16_hi(c.y), acc[3]));
                        *reinterpret_cast<u32x2*>(mx + r * kMixDPitch + feature) = y;
                    }
                }
            }
        }
    };

    Stage stage_a;
    Stage stage_b;
    fetch(stage_a, 0);
    if constexpr (DEPTH == 2) {
        __builtin_amdgcn_sched_barrier(0);
        fetch(stage_b, 1);
    }
    commit(stage_a, 0);
    __syncthreads();   // bias, zero padding and tile 0's rows are in LDS
    if constexpr (DEPTH == 2) {
        // Tile t's rows are staged in stage_a (t even) or stage_b (t odd);
        // the loop body covers an even and an odd tile so that the stages
        // keep fixed registers.
        // The fetch two tiles ahead is issued even past the range (its
        // buffers are then empty: zeros, no access): a fetch under a branch
        // made the compiler wait at the next commit for every load in
        // flight, this step's fetch included, which undid the second stage.
        auto step = [&](int k, Stage& refill, const Stage& next) {
            if (k < n_tiles) {
                fetch(refill, k + 2);
                __builtin_amdgcn_sched_barrier(0);
                apply_tile(k);
                if (k + 1 < n_tiles) {
                    commit(next, k + 1);
                }
            }
            __syncthreads();
        };
        for (int k = 0; k <= n_tiles; k += 2) {
            step(k, stage_a, stage_b);
            if (k + 1 <= n_tiles) {
                step(k + 1, stage_b, stage_a);
            }
        }
    } else {
        for (int k = 0; k <= n_tiles; ++k) {
            if (k < n_tiles) {
                fetch(stage_a, k + 1);
                apply_tile(k);
                if (k + 1 < n_tiles) {
                    commit(stage_a, k + 1);
                }
            }
            __syncthreads();
        }
    }
}

// Two row tiles in flight where the register budget allows it (operand
// records of at most four 32-rank feature blocks per wave), one otherwise.
template <int R, int NFB, int HPW, int WMAX>
constexpr int mix_depth() { return HPW * NFB * ((R + 31) / 32) <= 4 && WMAX <= 512 ? 2 : 1; }

template <int R, int NFB, int HPW, int WMAX, bool MIXED, bool MASKED>
static void launch_mix_project_mm(const MixProjectArgs& a, int y_dtype, dim3 grid, hipStream_t stream) {
    constexpr int kDepth = mix_depth<R, NFB, HPW, WMAX>();
    if (y_dtype == LSSO_HIP_F16) {
        dispatch(mix_project_kernel<R, NFB, LSSO_HIP_F16, kDepth, HPW, WMAX, MIXED, MASKED>, grid, kMixThreads,
                 stream, a);
    } else {
        dispatch(mix_project_kernel<R, NFB, LSSO_HIP_BF16, kDepth, HPW, WMAX, MIXED, MASKED>, grid, kMixThreads,
                 stream, a);
    }
}

template <int R, int NFB, int HPW, int WMAX, bool MIXED>
static void launch_mix_project_m(const MixProjectArgs& a, int y_dtype, dim3 grid, hipStream_t stream) {
    if (a.row_mask != nullptr) {
        launch_mix_project_mm<R, NFB, HPW, WMAX, MIXED, true>(a, y_dtype, grid, stream);
    } else {
        launch_mix_project_mm<R, NFB, HPW, WMAX, MIXED, false>(a, y_dtype, grid, stream);
    }
}

template <int R, int NFB, int HPW, int WMAX>
static hipError_t launch_mix_project_w(const MixProjectArgs& a, int y_dtype, dim3 grid,
                                       hipStream_t stream) {
    if (a.mixed != nullptr) {
        launch_mix_project_m<R, NFB, HPW, WMAX, true>(a, y_dtype, grid, stream);
    } else {
        launch_mix_project_m<R, NFB, HPW, WMAX, false>(a, y_dtype, grid, stream);
    }
    return hipGetLastError();
}

// Packed rows wider than 512 occur only from rank 48 on (H * d <= 256).
template <int R, int NFB, int HPW>
static hipError_t launch_mix_project_hpw(const MixProjectArgs& a, int y_dtype, dim3 grid,
                                         hipStream_t stream) {
    if constexpr (R >= 48) {
        if (a.width > 512) {
            return launch_mix_project_w<R, NFB, HPW, 640>(a, y_dtype, grid, stream);
        }
    }
    return launch_mix_project_w<R, NFB, HPW, 512>(a, y_dtype, grid, stream);
}

template <int R, int NFB>
static hipError_t launch_mix_project_nfb(const MixProjectArgs& a, int y_dtype, dim3 grid,
                                         hipStream_t stream) {
    if (a.heads > kMixApplyWaves) {
        return launch_mix_project_hpw<R, NFB, 2>(a, y_dtype, grid, stream);
    }
    return launch_mix_project_hpw<R, NFB, 1>(a, y_dtype, grid, stream);
}

template <int R>
static hipError_t launch_mix_project_r(const MixProjectArgs& a, int y_dtype, dim3 grid,
                                       hipStream_t stream) {
    if (a.feature_blocks <= 1) {
        return launch_mix_project_nfb<R, 1>(a, y_dtype, grid, stream);
    }
    if (a.feature_blocks <= 2) {
        return launch_mix_project_nfb<R, 2>(a, y_dtype, grid, stream);
    }
    return launch_mix_project_nfb<R, 4>(a, y_dtype, grid, stream);
}

hipError_t launch_mix_project(int rank, const MixProjectArgs& a, int y_dtype, hipStream_t stream) {
    const dim3 grid(static_cast<unsigned>(a.batch * a.ranges));
    switch (rank) {
        case 16: return launch_mix_project_r<16>(a, y_dtype, grid, stream);
        case 32: return launch_mix_project_r<32>(a, y_dtype, grid, stream);
        case 48: return launch_mix_project_r<48>(a, y_dtype, grid, stream);
        default: return launch_mix_project_r<64>(a, y_dtype, grid, stream);
    }
}

}  // namespace lsso_hip

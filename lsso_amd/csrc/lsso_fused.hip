// gfx950 apply fused with the output projection.
//
//   mixed = bf16(eta C + rot(R) M')                 (apply, reference.py:500-572)
//   y     = cast(bf16(mixed) bf16(W_o)^T + b_o)     (output projection, reference.py:20-75)
//
// One persistent workgroup of 8 waves owns a contiguous token range of one
// sample and walks it in 32-token tiles.  Per tile:
//   1. the packed rows (BF16, R and C of every head) sit in LDS; the rows
//      and phases of the next one or two tiles are in flight into registers;
//   2. wave h computes head h's mixed block with the apply MFMAs (the same
//      operand records, MFMA order and rounding as the standalone apply) and
//      writes it, BF16-rounded, into an LDS tile [32 tokens, D];
//   3. wave w multiplies that tile by its resident BF16 W_o slice (32 output
//      features) on v_mfma_f32_32x32x16_bf16, in the standalone projection's
//      K order, adds the FP32 bias and zeroes masked rows;
//   4. the rounded output is staged in LDS and written as 16-byte pieces of
//      whole rows.
// Two barriers per tile: after the mixed block is complete, and after the
// output stage and the next tile's rows are in LDS.
// The mixed tensor therefore never reaches HBM, and the result is bitwise the
// same as apply followed by the projection.

#include "lsso_device.h"
#include "lsso_internal.h"
#include "lsso_hip.h"

namespace lsso_hip {

constexpr int kMixRows = 32;                       // tokens per tile
constexpr int kMixRowBlocks = kMixRows / 32;       // 32-row MFMA blocks per tile
constexpr int kMixWaves = 8;
constexpr int kMixThreads = 64 * kMixWaves;
constexpr int kMixMaxWidth = 512;                  // packed row, BF16
constexpr int kMixPitch = kMixMaxWidth + 8;        // LDS row pitch of the packed tile
constexpr int kMixKSteps = 16;                     // D <= 256
constexpr int kMixDPitch = 16 * kMixKSteps + 8;    // LDS row pitch of the mixed / output tile
constexpr int kMixChunks = kMixRows * kMixMaxWidth / 8 / kMixThreads;
constexpr int kMixStoreChunks = kMixRows * (16 * kMixKSteps / 8) / kMixThreads;

bool mix_project_supported(int64_t rank, int64_t heads, int64_t head_dim, int64_t width) {
    const bool rank_ok = rank == 16 || rank == 32 || rank == 48 || rank == 64;
    return rank_ok && heads >= 1 && heads <= kMixWaves && head_dim >= 16 && head_dim % 16 == 0 &&
           head_dim <= 64 && heads * head_dim <= 16 * kMixKSteps && width <= kMixMaxWidth &&
           width % 8 == 0;
}

int mix_project_tile_rows() { return kMixRows; }

template <int R, int NFB, int YT, int DEPTH>
__global__ __launch_bounds__(kMixThreads) void mix_project_kernel(MixProjectArgs a) {
    using AL = ApplyLayout<R>;
    constexpr int PAIRS = R / 2;
    constexpr int PHP = PAIRS + 4;                 // LDS phase row pitch (u32)
    constexpr int S32 = AL::kSteps32 > 0 ? AL::kSteps32 : 1;
    constexpr int S16 = AL::kSteps16 > 0 ? AL::kSteps16 : 1;
    __shared__ __attribute__((aligned(16))) uint16_t s_pk[kMixRows * kMixPitch];
    __shared__ __attribute__((aligned(16))) uint32_t s_ph[kMixRows * PHP];
    __shared__ __attribute__((aligned(16))) uint16_t s_mx[kMixRows * kMixDPitch];
    __shared__ __attribute__((aligned(16))) uint16_t s_st[kMixRows * kMixDPitch];
    __shared__ __attribute__((aligned(16))) float s_bias[16 * kMixKSteps];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int half = lane >> 5;
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
    const int ksteps = static_cast<int>((D + 15) / 16);

    // Head `wave`: apply operands for the whole range (one sample).
    const bool apply_wave = wave < H;
    const int64_t h = apply_wave ? wave : 0;
    const float eta = bounded_complement(a.eta_raw[h]);
    u32x4 op_hi32[NFB][S32];
    u32x4 op_lo32[NFB][S32];
    u32x2 op_hi16[NFB][S16];
    u32x2 op_lo16[NFB][S16];
    {
        const int64_t system = b * H + h;
#pragma unroll
        for (int f = 0; f < NFB; ++f) {
            const bool live = f < a.feature_blocks;
            const uint16_t* record =
                a.mop + ((system * a.feature_blocks + (live ? f : 0)) * 64 + lane) * AL::kLaneHalfs;
#pragma unroll
            for (int s = 0; s < AL::kSteps32; ++s) {
                op_hi32[f][s] = *reinterpret_cast<const u32x4*>(record + AL::offset32(s));
                op_lo32[f][s] = *reinterpret_cast<const u32x4*>(record + AL::offset32(s) + 8);
            }
#pragma unroll
            for (int s = 0; s < AL::kSteps16; ++s) {
                op_hi16[f][s] = *reinterpret_cast<const u32x2*>(record + AL::offset16(s));
                op_lo16[f][s] = *reinterpret_cast<const u32x2*>(record + AL::offset16(s) + 4);
            }
        }
    }
    // Output features 32 wave .. +31: resident W_o slice.
    const int64_t n0 = 32 * wave;
    u32x4 wreg[kMixKSteps];
    load_weight_slice<kMixKSteps>(wreg, a.weight, D, D, n0, lane);
    for (int c = tid; c < 16 * kMixKSteps; c += kMixThreads) {
        s_bias[c] = (a.bias != nullptr && c < D) ? a.bias[c] : 0.0f;
    }
    // The mixed tile's columns past D are the zero K padding of the product.
    for (int i = tid; i < kMixRows * kMixDPitch / 8; i += kMixThreads) {
        reinterpret_cast<u32x4*>(s_mx)[i] = (u32x4){0u, 0u, 0u, 0u};
    }

    // Staging of upcoming tiles: packed chunks and phases held in registers
    // (DEPTH tiles ahead) while the current tile is processed.  A tile's
    // packed rows are one contiguous block, so chunk c of this thread is
    // bytes 16 (tid + c kMixThreads) of it; the LDS slots (padded pitch) and
    // the store pieces are fixed per thread and computed once.  Loads and
    // stores go through raw buffers sized to the tile's valid rows, so rows
    // past the range read as zeros and are not stored, without branches.
    const int Wi = static_cast<int>(W);
    const int Di = static_cast<int>(D);
    const int row_chunks = Wi / 8;
    const int tile_chunks = kMixRows * row_chunks;
    int lds_chunk[kMixChunks];
#pragma unroll
    for (int c = 0; c < kMixChunks; ++c) {
        const int idx = tid + c * kMixThreads;
        const int row = idx / row_chunks;
        lds_chunk[c] = idx < tile_chunks ? row * kMixPitch + 8 * (idx - row * row_chunks) : -1;
    }
    const int phase_lds = tid < kMixRows * (PAIRS / 4)
        ? (tid / (PAIRS / 4)) * PHP + 4 * (tid % (PAIRS / 4)) : -1;
    const int row_pieces = Di / 8;
    int store_lds[kMixStoreChunks];
    uint32_t store_off[kMixStoreChunks];
#pragma unroll
    for (int i = 0; i < kMixStoreChunks; ++i) {
        const int idx = tid + i * kMixThreads;
        const int row = idx / row_pieces;
        const int c8 = 8 * (idx - row * row_pieces);
        store_lds[i] = row * kMixDPitch + c8;
        store_off[i] = row < kMixRows ? 2u * static_cast<uint32_t>(row * Di + c8) : kOutOfRange;
    }
    const int end_i = static_cast<int>(end);
    const uint16_t* sample_rows = a.projected + b * a.length * W;
    const uint32_t* sample_phases = a.phases + b * a.phase_batch_stride;
    auto tile_rows = [&](int t0) { return end_i - t0 < kMixRows ? end_i - t0 : kMixRows; };
    struct Stage {
        u32x4 chunk[kMixChunks];
        u32x4 phase;
    };
    auto fetch = [&](Stage& st, int t0) {
        const int rows = tile_rows(t0);
        const BufferRsrc pk = make_buffer(sample_rows + static_cast<int64_t>(t0) * Wi, int64_t{2} * rows * Wi);
#pragma unroll
        for (int c = 0; c < kMixChunks; ++c) {
            st.chunk[c] = buffer_load16(pk, 16u * static_cast<uint32_t>(tid + c * kMixThreads));
        }
        const BufferRsrc ph = make_buffer(sample_phases + static_cast<int64_t>(t0) * PAIRS,
                                          int64_t{4} * rows * PAIRS);
        st.phase = buffer_load16(ph, phase_lds >= 0 ? 16u * static_cast<uint32_t>(tid) : kOutOfRange);
    };
    auto commit = [&](const Stage& st) {
#pragma unroll
        for (int c = 0; c < kMixChunks; ++c) {
            if (lds_chunk[c] >= 0) {
                *reinterpret_cast<u32x4*>(s_pk + lds_chunk[c]) = st.chunk[c];
            }
        }
        if (phase_lds >= 0) {
            *reinterpret_cast<u32x4*>(s_ph + phase_lds) = st.phase;
        }
    };

    // One tile: the packed rows of tile t0 are in LDS; `issue` receives the
    // rows DEPTH tiles ahead and `consume` (the next tile's rows, issued
    // earlier) is moved to LDS once this tile's mixed block has been read.
    // The wait counter retires memory operations in issue order, so the
    // mask bytes are requested before the next rows and the rows consumed
    // before this tile's stores are issued.
    auto iteration = [&](int t0, Stage& issue, Stage& consume) {
        const int rows = tile_rows(t0);
        const BufferRsrc mbuf = make_buffer(
            a.row_mask + (a.row_mask != nullptr ? b * a.length + t0 : 0), a.row_mask != nullptr ? rows : 0);
        bool keep[kMixRowBlocks];
#pragma unroll
        for (int mb = 0; mb < kMixRowBlocks; ++mb) {
            const int m = mb * 32 + (lane & 31);
            const uint32_t byte = buffer_load_byte(mbuf, static_cast<uint32_t>(m));
            keep[mb] = m < rows && (a.row_mask == nullptr || byte != 0);
        }
        const int ahead = t0 + DEPTH * kMixRows;
        if (ahead < end_i) {
            fetch(issue, ahead);
        }

        // ---- apply: head `wave`, 16-token sub-tiles -----------------------
        if (apply_wave) {
            const int q = lane & 15;
            const int g = lane >> 4;
#pragma unroll 1
            for (int sub = 0; sub < kMixRows / 16; ++sub) {
                const int r = sub * 16 + q;
                const uint16_t* prow = s_pk + r * kMixPitch;
                const uint32_t* phrow = s_ph + r * PHP;
                u32x4 b_hi32[S32];
                u32x4 b_lo32[S32];
#pragma unroll
                for (int s = 0; s < AL::kSteps32; ++s) {
                    const int first_rank = 32 * s + 8 * g;
                    const u32x4 rel = *reinterpret_cast<const u32x4*>(prow + h * R + first_rank);
                    const u32x4 ph = *reinterpret_cast<const u32x4*>(phrow + first_rank / 2);
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
                u32x2 b_hi16[S16];
                u32x2 b_lo16[S16];
#pragma unroll
                for (int s = 0; s < AL::kSteps16; ++s) {
                    const int first_rank = 16 * s + 4 * g;
                    const u32x2 rel = *reinterpret_cast<const u32x2*>(prow + h * R + first_rank);
                    const u32x2 ph = *reinterpret_cast<const u32x2*>(phrow + first_rank / 2);
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
                for (int f = 0; f < NFB; ++f) {
                    if (f < a.feature_blocks) {
                        f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                        for (int s = 0; s < AL::kSteps32; ++s) {
                            acc = mfma16x16x32(op_hi32[f][s], b_hi32[s], acc);
                            acc = mfma16x16x32(op_hi32[f][s], b_lo32[s], acc);
                            acc = mfma16x16x32(op_lo32[f][s], b_hi32[s], acc);
                        }
#pragma unroll
                        for (int s = 0; s < AL::kSteps16; ++s) {
                            acc = mfma16x16x16(op_hi16[f][s], b_hi16[s], acc);
                            acc = mfma16x16x16(op_hi16[f][s], b_lo16[s], acc);
                            acc = mfma16x16x16(op_lo16[f][s], b_hi16[s], acc);
                        }
                        const int64_t feature = h * d + 16 * f + 4 * g;
                        const u32x2 c = *reinterpret_cast<const u32x2*>(prow + H * R + feature);
                        u32x2 y;
                        y.x = pack_bf16(fmaf(eta, bf16_lo(c.x), acc[0]), fmaf(eta, bf16_hi(c.x), acc[1]));
                        y.y = pack_bf16(fmaf(eta, bf16_lo(c.y), acc[2]), fmaf(eta, bf16_hi(c.y), acc[3]));
                        *reinterpret_cast<u32x2*>(s_mx + r * kMixDPitch + feature) = y;
                    }
                }
            }
        }
        __syncthreads();

        // ---- output projection: features n0 .. n0 + 31 -------------------
        // Operand reads run one pair of K steps ahead of the MFMAs.
        f32x16 acc[kMixRowBlocks];
#pragma unroll
        for (int mb = 0; mb < kMixRowBlocks; ++mb) {
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                acc[mb][i] = 0.0f;
            }
        }
        if (n0 < D) {
            u32x4 xb[2][2][kMixRowBlocks];
            auto read_pair = [&](int slot, int k0) {
#pragma unroll
                for (int u = 0; u < 2; ++u) {
#pragma unroll
                    for (int mb = 0; mb < kMixRowBlocks; ++mb) {
                        xb[slot][u][mb] = *reinterpret_cast<const u32x4*>(
                            s_mx + (mb * 32 + (lane & 31)) * kMixDPitch + 16 * (k0 + u) + 8 * half);
                    }
                }
            };
            read_pair(0, 0);
#pragma unroll
            for (int k2 = 0; k2 < kMixKSteps; k2 += 2) {
                const int slot = (k2 / 2) & 1;
                if (k2 + 2 < kMixKSteps && k2 + 2 < ksteps) {
                    read_pair(slot ^ 1, k2 + 2);
                }
#pragma unroll
                for (int u = 0; u < 2; ++u) {
                    if (k2 + u < ksteps) {
#pragma unroll
                        for (int mb = 0; mb < kMixRowBlocks; ++mb) {
                            acc[mb] = mfma32x32x16(wreg[k2 + u], xb[slot][u][mb], acc[mb]);
                        }
                    }
                }
            }
            // Rounded output tile into the store stage (its own buffer, so no
            // wave waits for the others to finish reading the mixed tile).
#pragma unroll
            for (int mb = 0; mb < kMixRowBlocks; ++mb) {
                const int mr = mb * 32 + (lane & 31);
#pragma unroll
                for (int qd = 0; qd < 4; ++qd) {
                    const int c = static_cast<int>(n0) + 8 * qd + 4 * half;
                    if (c < D) {
                        const f32x4 bias = *reinterpret_cast<const f32x4*>(&s_bias[c]);
                        const float v0 = keep[mb] ? acc[mb][4 * qd + 0] + bias[0] : 0.0f;
                        const float v1 = keep[mb] ? acc[mb][4 * qd + 1] + bias[1] : 0.0f;
                        const float v2 = keep[mb] ? acc[mb][4 * qd + 2] + bias[2] : 0.0f;
                        const float v3 = keep[mb] ? acc[mb][4 * qd + 3] + bias[3] : 0.0f;
                        u32x2 packed;
                        if constexpr (YT == LSSO_HIP_BF16) {
                            packed.x = pack_bf16(v0, v1);
                            packed.y = pack_bf16(v2, v3);
                        } else {
                            packed.x = pack_f16(v0, v1);
                            packed.y = pack_f16(v2, v3);
                        }
                        *reinterpret_cast<u32x2*>(s_st + mr * kMixDPitch + c) = packed;
                    }
                }
            }
        }
        // The next tile's rows replace this tile's (read before the barrier
        // above); the stage is complete after this barrier.
        if (t0 + kMixRows < end_i) {
            commit(consume);
        }
        __syncthreads();
        {
            const BufferRsrc ybuf = make_buffer(
                static_cast<uint16_t*>(a.y) + (b * a.length + t0) * D, int64_t{2} * rows * Di);
#pragma unroll
            for (int i = 0; i < kMixStoreChunks; ++i) {
                buffer_store16(*reinterpret_cast<const u32x4*>(s_st + store_lds[i]), ybuf, store_off[i]);
            }
        }
    };

    const int begin_i = static_cast<int>(begin);
    Stage stage_a;
    Stage stage_b;
    fetch(stage_a, begin_i);
    if constexpr (DEPTH == 2) {
        if (begin_i + kMixRows < end_i) {
            fetch(stage_b, begin_i + kMixRows);
        }
    }
    commit(stage_a);
    __syncthreads();
    if constexpr (DEPTH == 2) {
        // Tiles alternate between the two stage sets: tile t consumes the set
        // issued two tiles earlier and reissues it.
        for (int t0 = begin_i; t0 < end_i; t0 += 2 * kMixRows) {
            iteration(t0, stage_a, stage_b);
            if (t0 + kMixRows < end_i) {
                iteration(t0 + kMixRows, stage_b, stage_a);
            }
        }
    } else {
        for (int t0 = begin_i; t0 < end_i; t0 += kMixRows) {
            iteration(t0, stage_a, stage_a);
        }
    }
}

// Two tiles in flight where the register budget allows it (operand records
// of at most two 32-rank feature blocks), one otherwise.
template <int R, int NFB>
constexpr int mix_depth() { return NFB * ((R + 31) / 32) <= 4 ? 2 : 1; }

template <int R, int NFB>
static hipError_t launch_mix_project_nfb(const MixProjectArgs& a, int y_dtype, dim3 grid,
                                         hipStream_t stream) {
    constexpr int kDepth = mix_depth<R, NFB>();
    if (y_dtype == LSSO_HIP_F16) {
        mix_project_kernel<R, NFB, LSSO_HIP_F16, kDepth><<<grid, kMixThreads, 0, stream>>>(a);
    } else {
        mix_project_kernel<R, NFB, LSSO_HIP_BF16, kDepth><<<grid, kMixThreads, 0, stream>>>(a);
    }
    return hipGetLastError();
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

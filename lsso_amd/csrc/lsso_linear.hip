// gfx950 biased projection y = cast(bf16(x) bf16(W)^T + b).
//
// Contract (reference lsso/ball/reference.py:20-75, 170-203, 347-408): BF16
// multiplicands (x rounded to BF16 with round-to-nearest-even, W likewise),
// FP32 accumulation, FP32 bias added to the accumulator, one final FP16 or
// BF16 store; FP16 output never rounds through BF16.
//
// Schedule: persistent workgroups of 8 waves (4 when K > 256).  Each wave
// keeps a 32-column slice of W (BF16, K padded to 16) in registers for the
// whole launch, so the weights are read once per workgroup.  64-row x tiles
// are staged through a double-buffered LDS tile (converted to BF16 once) and
// shared by the workgroup's waves.
// The MFMA computes y^T = W x^T on v_mfma_f32_32x32x16_bf16; in that form a
// lane's accumulators are 4 runs of 4 consecutive output features of one
// row, stored as 8-byte writes.

#include "lsso_device.h"
#include "lsso_internal.h"
#include "lsso_hip.h"

namespace lsso_hip {

constexpr int kLinearTileRows = 64;

// Waves per workgroup: eight (two per SIMD, 256 registers each) while the
// resident W slice fits; four once K exceeds 256.
template <int KSTEPS>
constexpr int linear_waves() { return KSTEPS <= 16 ? 8 : 4; }

int linear_tile_rows() { return kLinearTileRows; }
int linear_columns_per_group(int k_steps) { return (k_steps <= 16 ? 8 : 4) * 32; }

int linear_k_tier(int64_t in_features) {
    if (in_features <= 64) return 4;
    if (in_features <= 128) return 8;
    if (in_features <= 192) return 12;
    if (in_features <= 256) return 16;
    if (in_features <= 384) return 24;
    if (in_features <= 512) return 32;
    return 0;
}

// Load 8 consecutive x elements as BF16.  Out-of-range rows and columns read
// a clamped in-bounds address and are zeroed by select, so the tile load has
// no divergent branches.
template <int XT>
__device__ __forceinline__ u32x4 load_x_chunk(const LinearArgs& a, int64_t row, int64_t k0) {
    const int64_t safe_row = row < a.rows ? row : a.rows - 1;
    const bool row_live = row < a.rows && (a.row_mask == nullptr || a.row_mask[safe_row] != 0);
    const uint16_t* x = static_cast<const uint16_t*>(a.x) + safe_row * a.x_stride;
    u32x4 out;
    if (a.x_vector) {
        const bool live = row_live && k0 < a.in_features;
        const u32x4 raw = *reinterpret_cast<const u32x4*>(x + (live ? k0 : 0));
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            uint32_t value = raw[p];
            if constexpr (XT == LSSO_HIP_F16) {
                value = pack_bf16(f16_lo(value), f16_hi(value));
            }
            out[p] = live ? value : 0u;
        }
        return out;
    }
    float v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const bool live = row_live && k0 + i < a.in_features;
        const uint16_t bits = x[live ? k0 + i : 0];
        float value;
        if constexpr (XT == LSSO_HIP_BF16) {
            value = bf16_bits_to_float(bits);
        } else {
            value = f16_bits_to_float(bits);
        }
        v[i] = live ? value : 0.0f;
    }
#pragma unroll
    for (int p = 0; p < 4; ++p) {
        out[p] = pack_bf16(v[2 * p], v[2 * p + 1]);
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

template <int KSTEPS, int XT, int YT>
__global__ __launch_bounds__(linear_waves<KSTEPS>() * 64) void linear_kernel(LinearArgs a) {
    constexpr int kWaves = linear_waves<KSTEPS>();
    constexpr int kGroupColumns = kWaves * 32;
    constexpr int KP = 16 * KSTEPS + 8;                  // LDS row pitch (bf16)
    constexpr int kChunksPerRow = 2 * KSTEPS;           // 8-element chunks
    constexpr int kThreads = kWaves * 64;
    constexpr int kChunksPerThread = kLinearTileRows * kChunksPerRow / kThreads;
    static_assert(kLinearTileRows * kChunksPerRow % kThreads == 0, "tile split");
    __shared__ __attribute__((aligned(16))) uint16_t s_x[2][kLinearTileRows * KP];
    __shared__ __attribute__((aligned(16))) float s_bias[kGroupColumns];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int half = lane >> 5;
    const int64_t cg = blockIdx.x % a.column_groups;
    const int64_t group_index = blockIdx.x / a.column_groups;
    const int64_t group_count = gridDim.x / a.column_groups;
    const int64_t n0 = cg * kGroupColumns + wave * 32;
    const int64_t K = a.in_features;
    const int64_t N = a.out_features;

    // W slice: lane holds row n0 + lane%32, k = 16 ks + 8 half + 0..7.  Rows
    // are read as float4 pairs when K is a multiple of 4 (16-byte rows).
    u32x4 wreg[KSTEPS];
    {
        const int64_t n = n0 + (lane & 31);
        const bool nv = n < N;
        const float* wrow = a.weight + (nv ? n : 0) * K;
        const bool vector_rows = (K % 4) == 0;
#pragma unroll
        for (int ks = 0; ks < KSTEPS; ++ks) {
            const int64_t k0 = 16 * ks + 8 * half;
            float v[8];
            if (vector_rows && nv && k0 + 8 <= K) {
                const f32x4 lo = *reinterpret_cast<const f32x4*>(wrow + k0);
                const f32x4 hi = *reinterpret_cast<const f32x4*>(wrow + k0 + 4);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    v[i] = lo[i];
                    v[4 + i] = hi[i];
                }
            } else {
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const bool live = nv && k0 + i < K;
                    const float value = wrow[live ? k0 + i : 0];
                    v[i] = live ? value : 0.0f;
                }
            }
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                wreg[ks][p] = pack_bf16(v[2 * p], v[2 * p + 1]);
            }
            // Convert one K step at a time: keeps the FP32 staging of W from
            // being hoisted next to the whole BF16 slice.
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    for (int c = tid; c < kGroupColumns; c += kThreads) {
        const int64_t n = cg * kGroupColumns + c;
        s_bias[c] = (a.bias != nullptr && n < N) ? a.bias[n] : 0.0f;
    }

    u32x4 stage[kChunksPerThread];
    auto load_stage = [&](int64_t tile) {
#pragma unroll
        for (int c = 0; c < kChunksPerThread; ++c) {
            const int chunk = tid + c * kThreads;
            const int rr = chunk / kChunksPerRow;
            const int cc = chunk - rr * kChunksPerRow;
            stage[c] = load_x_chunk<XT>(a, tile * kLinearTileRows + rr, 8 * cc);
        }
    };
    auto write_stage = [&](int buf) {
#pragma unroll
        for (int c = 0; c < kChunksPerThread; ++c) {
            const int chunk = tid + c * kThreads;
            const int rr = chunk / kChunksPerRow;
            const int cc = chunk - rr * kChunksPerRow;
            *reinterpret_cast<u32x4*>(&s_x[buf][rr * KP + 8 * cc]) = stage[c];
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
        if (next < a.tiles) {
            load_stage(next);
        }
        f32x16 acc[2];
#pragma unroll
        for (int mb = 0; mb < 2; ++mb) {
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                acc[mb][i] = 0.0f;
            }
        }
        // Operand reads run one group of two K steps ahead of the MFMAs, so
        // at most eight x fragments are live next to the resident W slice.
        constexpr int kGroup = 2;
        u32x4 xb[2][kGroup][2];
        auto read_group = [&](int slot, int k_base) {
#pragma unroll
            for (int ks = 0; ks < kGroup; ++ks) {
#pragma unroll
                for (int mb = 0; mb < 2; ++mb) {
                    xb[slot][ks][mb] = *reinterpret_cast<const u32x4*>(
                        &s_x[buf][(mb * 32 + (lane & 31)) * KP + 16 * (k_base + ks) + 8 * half]);
                }
            }
        };
        read_group(0, 0);
#pragma unroll
        for (int k2 = 0; k2 < KSTEPS; k2 += kGroup) {
            const int slot = (k2 / kGroup) & 1;
            if (k2 + kGroup < KSTEPS) {
                read_group(slot ^ 1, k2 + kGroup);
            }
#pragma unroll
            for (int ks = 0; ks < kGroup; ++ks) {
#pragma unroll
                for (int mb = 0; mb < 2; ++mb) {
                    acc[mb] = mfma32x32x16(wreg[k2 + ks], xb[slot][ks][mb], acc[mb]);
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        // y^T block: lane holds row m = lane%32 of the 32-row block and
        // features n0 + 8 q + 4 half + r for q, r in 0..3.
#pragma unroll
        for (int mb = 0; mb < 2; ++mb) {
            const int64_t m = tile * kLinearTileRows + mb * 32 + (lane & 31);
            if (m < a.rows) {
                const bool keep = a.row_mask == nullptr || a.row_mask[m] != 0;
                uint16_t* yrow = static_cast<uint16_t*>(a.y) + m * N;
#pragma unroll
                for (int qd = 0; qd < 4; ++qd) {
                    const int64_t n = n0 + 8 * qd + 4 * half;
                    const f32x4 bias = *reinterpret_cast<const f32x4*>(
                        &s_bias[wave * 32 + 8 * qd + 4 * half]);
                    const float v0 = keep ? acc[mb][4 * qd + 0] + bias[0] : 0.0f;
                    const float v1 = keep ? acc[mb][4 * qd + 1] + bias[1] : 0.0f;
                    const float v2 = keep ? acc[mb][4 * qd + 2] + bias[2] : 0.0f;
                    const float v3 = keep ? acc[mb][4 * qd + 3] + bias[3] : 0.0f;
                    if (a.y_vector && n + 3 < N) {
                        u32x2 packed;
                        if constexpr (YT == LSSO_HIP_BF16) {
                            packed.x = pack_bf16(v0, v1);
                            packed.y = pack_bf16(v2, v3);
                        } else {
                            packed.x = pack_f16(v0, v1);
                            packed.y = pack_f16(v2, v3);
                        }
                        *reinterpret_cast<u32x2*>(yrow + n) = packed;
                    } else {
                        const float v[4] = {v0, v1, v2, v3};
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            if (n + r < N) {
                                yrow[n + r] = to_output_bits<YT>(v[r]);
                            }
                        }
                    }
                }
            }
        }
        if (next < a.tiles) {
            write_stage(buf ^ 1);
        }
        __syncthreads();
        buf ^= 1;
    }
}

template <int KSTEPS>
static hipError_t launch_linear_k(const LinearArgs& a, int x_dtype, int y_dtype, dim3 grid,
                                  hipStream_t stream) {
    const dim3 block(linear_waves<KSTEPS>() * 64);
    if (x_dtype == LSSO_HIP_F16) {
        if (y_dtype == LSSO_HIP_F16) {
            linear_kernel<KSTEPS, LSSO_HIP_F16, LSSO_HIP_F16><<<grid, block, 0, stream>>>(a);
        } else {
            linear_kernel<KSTEPS, LSSO_HIP_F16, LSSO_HIP_BF16><<<grid, block, 0, stream>>>(a);
        }
    } else {
        if (y_dtype == LSSO_HIP_F16) {
            linear_kernel<KSTEPS, LSSO_HIP_BF16, LSSO_HIP_F16><<<grid, block, 0, stream>>>(a);
        } else {
            linear_kernel<KSTEPS, LSSO_HIP_BF16, LSSO_HIP_BF16><<<grid, block, 0, stream>>>(a);
        }
    }
    return hipGetLastError();
}

hipError_t launch_linear(const LinearArgs& a, int k_steps, int x_dtype, int y_dtype,
                         int grid_groups, hipStream_t stream) {
    const dim3 grid(static_cast<unsigned>(grid_groups * a.column_groups));
    switch (k_steps) {
        case 4: return launch_linear_k<4>(a, x_dtype, y_dtype, grid, stream);
        case 8: return launch_linear_k<8>(a, x_dtype, y_dtype, grid, stream);
        case 12: return launch_linear_k<12>(a, x_dtype, y_dtype, grid, stream);
        case 16: return launch_linear_k<16>(a, x_dtype, y_dtype, grid, stream);
        case 24: return launch_linear_k<24>(a, x_dtype, y_dtype, grid, stream);
        case 32: return launch_linear_k<32>(a, x_dtype, y_dtype, grid, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace lsso_hip

// gfx950 weight (and bias) gradient of the biased projection
// (reference lsso/ball/reference.py:205-247):
//   grad_weight[n][k] = sum over rows m of bf16(g[m][n]) * bf16(x[m][k])   (FP32)
//   grad_bias[n]      = sum over rows m of g[m][n]                          (FP32)
// with rows that the row mask excludes counting as zero.
//
// The contraction runs over rows, the strided dimension of both row-major
// operands, while an MFMA fragment needs 8 consecutive rows of one column.
// Each workgroup (four waves) owns a 128 (n) x 128 (k) output tile and a
// split of consecutive rows, taken in 64-row stages.  Per stage, each thread
// loads one 8-row x 8-column block of g (waves 0-1) or x (waves 2-3) as eight
// 16-byte row pieces, one stage ahead of its use; rounds it to BF16 (the
// reference's operands); transposes it in registers (byte permutes); and
// writes its 8 columns to LDS column-major, so that every MFMA fragment
// (v_mfma_f32_32x32x16_bf16, A = g^T, B = x, K = rows) is one 16-byte LDS
// read.  Each wave accumulates a 64 x 64 quarter of the tile.  A split writes
// FP32 partials [split][n][k]; column_sum_kernel adds the splits in order, so
// the result is deterministic.  The bias sums are taken from the g blocks (in
// g's own precision, as the reference sums g) by the k-tile-0 workgroups.
// The workgroups of one row split are dealt to one XCD, so that the re-reads
// of g and x by the neighbouring tiles hit that XCD's L2.

#include "lsso_device.h"
#include "lsso_internal.h"
#include "lsso_hip.h"

namespace lsso_hip {

namespace {

constexpr int kWgTile = 128;            // output tile edge (n and k)
constexpr int kWgRows = 64;             // rows per stage (four MFMA K steps)
constexpr int kWgThreads = 256;
constexpr int kWgPitch = kWgRows + 8;   // column-major LDS pitch (bf16)

// LDS offset (bf16) of rows 8 g .. 8 g + 7 of a stage column.  The 8-row
// group index is XOR-swizzled by bits 4-6 of the column, so that both the
// transposed block writes (16 lanes: 16 columns 8 apart, one row group) and
// the fragment reads (consecutive columns, one row group) spread over all
// LDS banks; with the plain layout, columns 8 apart land on two bank groups.
__device__ __forceinline__ int stage_offset(int column, int group) {
    return column * kWgPitch + 8 * (group ^ ((column >> 4) & 7));
}
constexpr int kWgXcds = 8;
// Resident workgroups per XCD on MI355X: 32 CUs x 2 (the two stage buffers
// take 76 KB of a CU's 160 KB of LDS).
constexpr int kWgSlotsPerXcd = 64;

template <int T>
__device__ __forceinline__ float bits_to_float(uint32_t bits) {
    if constexpr (T == LSSO_HIP_BF16) {
        return bf16_bits_to_float(static_cast<uint16_t>(bits));
    } else {
        return f16_bits_to_float(static_cast<uint16_t>(bits));
    }
}

// 8 elements of one row (columns c .. c + 7 of a [rows, cols] matrix), zero
// past the columns and for a dead row; VEC: one 16-byte load (cols and the
// row stride multiples of 8).
template <bool VEC>
__device__ __forceinline__ u32x4 load_piece(const uint16_t* base, int64_t row, int64_t stride,
                                            int64_t c, int64_t cols, bool live) {
    if constexpr (VEC) {
        return (live && c < cols) ? *reinterpret_cast<const u32x4*>(base + row * stride + c) : u32x4{};
    } else {
        u32x4 v;
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            const uint32_t lo = (live && c + 2 * p < cols) ? base[row * stride + c + 2 * p] : 0u;
            const uint32_t hi = (live && c + 2 * p + 1 < cols) ? base[row * stride + c + 2 * p + 1] : 0u;
            v[p] = lo | (hi << 16);
        }
        return v;
    }
}

template <int T>
__device__ __forceinline__ u32x4 to_bf16_piece(const u32x4& raw) {
    if constexpr (T == LSSO_HIP_BF16) {
        return raw;
    } else {
        u32x4 v;
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            v[p] = pack_bf16(f16_lo(raw[p]), f16_hi(raw[p]));
        }
        return v;
    }
}

// Column c of an 8 x 8 block of 16-bit values given as 8 rows of 8: the
// block's rows 2p and 2p + 1 of that column form dword p.
__device__ __forceinline__ u32x4 block_column(const u32x4 (&rows)[8], int c) {
    const int q = c >> 1;
    u32x4 out;
#pragma unroll
    for (int p = 0; p < 4; ++p) {
        const uint32_t a = rows[2 * p][q];
        const uint32_t b = rows[2 * p + 1][q];
        // Byte selectors of v_perm_b32 over {b : a}: low halves or high halves.
        out[p] = __builtin_amdgcn_perm(b, a, (c & 1) ? 0x07060302u : 0x05040100u);
    }
    return out;
}

}  // namespace

template <int GT, int XT, bool VEC>
__global__ __launch_bounds__(kWgThreads) void weight_grad_kernel(WeightGradArgs a) {
    // Column-major stage buffers: s_t[buf][operand][column * kWgPitch + row].
    __shared__ __attribute__((aligned(16))) uint16_t s_t[2][2][kWgTile * kWgPitch];
    __shared__ float s_sum[kWgRows / 8][kWgTile];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int half = lane >> 5;
    const int64_t tiles = a.tiles_n * a.tiles_k;
    int64_t tile = blockIdx.x;
    int64_t split = 0;
    if (a.splits > 1) {
        // Row splits dealt round-robin over the XCDs, each XCD walking all
        // output tiles of its splits.  With one split the grid holds one
        // workgroup per output tile.
        const int64_t xcd = blockIdx.x % kWgXcds;
        const int64_t slot = blockIdx.x / kWgXcds;
        tile = slot % tiles;
        split = (slot / tiles) * kWgXcds + xcd;
        if (split >= a.splits) {
            return;
        }
    }
    const int64_t nt = tile / a.tiles_k;
    const int64_t kt = tile - nt * a.tiles_k;
    const int64_t n0 = nt * kWgTile;
    const int64_t k0 = kt * kWgTile;
    const int64_t N = a.out_features;
    const int64_t K = a.in_features;
    const int64_t r0 = split * a.rows_per_split;
    const int64_t r1 = r0 + a.rows_per_split < a.rows ? r0 + a.rows_per_split : a.rows;

    // This thread's 8 x 8 block of each stage: operand (waves 0-1: g, 2-3: x),
    // rows 8 rb .. + 7 and columns 8 cb .. + 7 of the stage's 64 x 128 tile.
    const int operand = wave >> 1;                  // wave-uniform
    const int block = tid & 127;
    const int rb = block >> 4;
    const int cb = block & 15;
    const bool is_g = operand == 0;
    const uint16_t* src = static_cast<const uint16_t*>(is_g ? a.g : a.x);
    const int64_t stride = is_g ? a.g_stride : a.x_stride;
    const int64_t cols = is_g ? N : K;
    const int64_t c0 = (is_g ? n0 : k0) + 8 * cb;
    const bool sums = is_g && a.bias_partials != nullptr && kt == 0;

    u32x4 raw[8];
    float colsum[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        colsum[e] = 0.0f;
    }
    auto load = [&](int64_t base) {
#pragma unroll
        for (int r = 0; r < 8; ++r) {
            const int64_t m = base + 8 * rb + r;
            bool keep = m < r1;
            if (keep && a.row_mask != nullptr) {
                keep = a.row_mask[m] != 0;
            }
            raw[r] = load_piece<VEC>(src, keep ? m : r0, stride, c0, cols, keep);
        }
    };
    auto store = [&](int buf) {
        u32x4 rows[8];
        if (is_g) {
#pragma unroll
            for (int r = 0; r < 8; ++r) {
                rows[r] = to_bf16_piece<GT>(raw[r]);
                if (sums) {
                    // Excluded rows were loaded as zeros; the sums take g in its own precision.
#pragma unroll
                    for (int p = 0; p < 4; ++p) {
                        colsum[2 * p] += bits_to_float<GT>(raw[r][p] & 0xffffu);
                        colsum[2 * p + 1] += bits_to_float<GT>(raw[r][p] >> 16);
                    }
                }
            }
        } else {
#pragma unroll
            for (int r = 0; r < 8; ++r) {
                rows[r] = to_bf16_piece<XT>(raw[r]);
            }
        }
        uint16_t* dst = s_t[buf][operand];
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            *reinterpret_cast<u32x4*>(dst + stage_offset(8 * cb + c, rb)) = block_column(rows, c);
        }
    };

    const int wn = wave & 1;    // 64-row (n) half of the output tile
    const int wk = wave >> 1;   // 64-column (k) half of the output tile
    f32x16 acc[2][2];
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                acc[nb][kb][e] = 0.0f;
            }
        }
    }
    auto compute = [&](int buf) {
        const uint16_t* gt = s_t[buf][0];
        const uint16_t* xt = s_t[buf][1];
#pragma unroll
        for (int kk = 0; kk < kWgRows / 16; ++kk) {
            const int group = 2 * kk + half;
            u32x4 af[2];
            u32x4 bf[2];
#pragma unroll
            for (int b = 0; b < 2; ++b) {
                af[b] = *reinterpret_cast<const u32x4*>(gt + stage_offset(wn * 64 + b * 32 + (lane & 31), group));
                bf[b] = *reinterpret_cast<const u32x4*>(xt + stage_offset(wk * 64 + b * 32 + (lane & 31), group));
            }
#pragma unroll
            for (int nb = 0; nb < 2; ++nb) {
#pragma unroll
                for (int kb = 0; kb < 2; ++kb) {
                    acc[nb][kb] = mfma32x32x16(af[nb], bf[kb], acc[nb][kb]);
                }
            }
        }
    };
    // One stage ahead: the loads of stage s + 1 are issued before stage s is
    // multiplied, and written to the other LDS buffer after it.
    int buf = 0;
    if (r0 < r1) {
        load(r0);
        store(0);
    }
    __syncthreads();
    for (int64_t base = r0; base < r1; base += kWgRows) {
        const bool more = base + kWgRows < r1;
        if (more) {
            load(base + kWgRows);
        }
        compute(buf);
        if (more) {
            store(buf ^ 1);
        }
        __syncthreads();
        buf ^= 1;
    }

    // Partials: lane (half, j) of block (nb, kb) holds column k = j and rows
    // n = 8 q + 4 half + e of the block, for accumulator entry 4 q + e.
    float* out = a.partials + split * N * K;
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
            const int64_t k = k0 + wk * 64 + kb * 32 + (lane & 31);
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int64_t n = n0 + wn * 64 + nb * 32 + 8 * (e / 4) + 4 * half + (e % 4);
                if (n < N && k < K) {
                    out[n * K + k] = acc[nb][kb][e];
                }
            }
        }
    }
    if (a.bias_partials != nullptr && kt == 0) {
        if (sums) {
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                s_sum[rb][8 * cb + e] = colsum[e];
            }
        }
        __syncthreads();
        if (tid < kWgTile) {
            float total = 0.0f;
#pragma unroll
            for (int r = 0; r < kWgRows / 8; ++r) {
                total += s_sum[r][tid];
            }
            if (n0 + tid < N) {
                a.bias_partials[split * N + n0 + tid] = total;
            }
        }
    }
}

void plan_weight_grad(int64_t rows, int64_t in_features, int64_t out_features, int64_t* splits,
                      int64_t* rows_per_split) {
    const int64_t tiles = ((out_features + kWgTile - 1) / kWgTile) * ((in_features + kWgTile - 1) / kWgTile);
    const int64_t stages = (rows + kWgRows - 1) / kWgRows;
    // As many row splits per XCD as let all of that XCD's workgroups (its
    // splits x the output tiles) be resident at once: one more, nearly empty
    // round of workgroups would take as long as the first.  When the output
    // tiles alone fill every resident slot of the device, splitting the rows
    // gains no occupancy and only multiplies the FP32 partials (splits x N x
    // K floats, written and summed again), so the rows stay in one split.
    int64_t per_xcd = kWgSlotsPerXcd / tiles;
    if (per_xcd < 1) per_xcd = 1;
    int64_t want = tiles >= kWgXcds * kWgSlotsPerXcd ? 1 : kWgXcds * per_xcd;
    if (want > stages) want = stages;
    if (want < 1) want = 1;
    const int64_t per = (rows + want - 1) / want;
    *rows_per_split = ((per + kWgRows - 1) / kWgRows) * kWgRows;
    *splits = rows == 0 ? 0 : (rows + *rows_per_split - 1) / *rows_per_split;
}

template <int GT, int XT>
static void launch_wg(const WeightGradArgs& a, dim3 grid, hipStream_t stream) {
    if (a.vec) {
        weight_grad_kernel<GT, XT, true><<<grid, kWgThreads, 0, stream>>>(a);
    } else {
        weight_grad_kernel<GT, XT, false><<<grid, kWgThreads, 0, stream>>>(a);
    }
}

hipError_t launch_weight_grad(const WeightGradArgs& a, int g_dtype, int x_dtype, hipStream_t stream) {
    if (a.splits == 0) {
        return hipSuccess;
    }
    const int64_t tiles = a.tiles_n * a.tiles_k;
    const int64_t rounds = (a.splits + kWgXcds - 1) / kWgXcds;
    const dim3 grid(static_cast<unsigned>(a.splits == 1 ? tiles : rounds * kWgXcds * tiles));
    if (g_dtype == LSSO_HIP_F16) {
        if (x_dtype == LSSO_HIP_F16) {
            launch_wg<LSSO_HIP_F16, LSSO_HIP_F16>(a, grid, stream);
        } else {
            launch_wg<LSSO_HIP_F16, LSSO_HIP_BF16>(a, grid, stream);
        }
    } else {
        if (x_dtype == LSSO_HIP_F16) {
            launch_wg<LSSO_HIP_BF16, LSSO_HIP_F16>(a, grid, stream);
        } else {
            launch_wg<LSSO_HIP_BF16, LSSO_HIP_BF16>(a, grid, stream);
        }
    }
    return hipGetLastError();
}

int weight_grad_tile() { return kWgTile; }

}  // namespace lsso_hip

// gfx950 upstream-gradient pass of the biased projection's backward
// (reference lsso/ball/reference.py:205-247).
//
// The reference rounds the upstream gradient to BF16 for the weight-gradient
// GEMM and sums it in FP32 over all rows for the bias gradient.  One pass over
// g does both: every (row, 8-column chunk) is read once, rounded to BF16 and
// written (when a BF16 copy is asked for), and added to per-thread FP32
// column sums.  Rows excluded by the row mask count as zero.
//
// Schedule: blockIdx.y is a slab of `cw` 8-column chunks; blockIdx.x is a
// split of consecutive rows.  Thread t takes chunk t % cw and every
// (256 / cw)-th row of the split, eight rows' loads in flight.  The row lanes
// of a chunk are combined in LDS in lane order and the split writes one FP32
// partial per column; column_sum_kernel adds the splits in a fixed order, so
// the sums are deterministic.

#include "lsso_device.h"
#include "lsso_internal.h"
#include "lsso_hip.h"

namespace lsso_hip {

constexpr int kGradThreads = 256;
constexpr int kGradRowsInFlight = 8;

template <int GT>
__device__ __forceinline__ float grad_bits_to_float(uint16_t bits) {
    if constexpr (GT == LSSO_HIP_BF16) {
        return bf16_bits_to_float(bits);
    } else {
        return f16_bits_to_float(bits);
    }
}

template <int GT, bool VEC>
__global__ __launch_bounds__(kGradThreads) void grad_columns_kernel(GradColumnsArgs a) {
    const int t = threadIdx.x;
    const int cw = a.chunks_per_slab;
    const int row_lanes = kGradThreads / cw;
    const int row_lane = t / cw;
    const int64_t col0 = (static_cast<int64_t>(blockIdx.y) * cw + (t - row_lane * cw)) * 8;
    const bool col_live = col0 < a.cols;
    const int64_t r0 = static_cast<int64_t>(blockIdx.x) * a.rows_per_split;
    const int64_t r1 = r0 + a.rows_per_split < a.rows ? r0 + a.rows_per_split : a.rows;
    const uint16_t* g = static_cast<const uint16_t*>(a.g);

    float acc[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        acc[i] = 0.0f;
    }
    for (int64_t base = r0 + row_lane; base < r1; base += static_cast<int64_t>(row_lanes) * kGradRowsInFlight) {
        float v[kGradRowsInFlight][8];
        bool live[kGradRowsInFlight];
        bool keep[kGradRowsInFlight];
#pragma unroll
        for (int u = 0; u < kGradRowsInFlight; ++u) {
            const int64_t row = base + static_cast<int64_t>(u) * row_lanes;
            live[u] = row < r1 && col_live;
            const int64_t safe_row = live[u] ? row : r0;
            keep[u] = live[u] && (a.row_mask == nullptr || a.row_mask[safe_row] != 0);
            const uint16_t* src = g + safe_row * a.g_stride;
            if constexpr (VEC) {
                const u32x4 raw = *reinterpret_cast<const u32x4*>(src + (col_live ? col0 : 0));
#pragma unroll
                for (int p = 0; p < 4; ++p) {
                    if constexpr (GT == LSSO_HIP_BF16) {
                        v[u][2 * p] = bf16_lo(raw[p]);
                        v[u][2 * p + 1] = bf16_hi(raw[p]);
                    } else {
                        v[u][2 * p] = f16_lo(raw[p]);
                        v[u][2 * p + 1] = f16_hi(raw[p]);
                    }
                }
            } else {
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const bool in = col_live && col0 + i < a.cols;
                    v[u][i] = grad_bits_to_float<GT>(src[in ? col0 + i : 0]);
                }
            }
        }
#pragma unroll
        for (int u = 0; u < kGradRowsInFlight; ++u) {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                v[u][i] = keep[u] ? v[u][i] : 0.0f;
                acc[i] += v[u][i];
            }
            if (a.g_bf16 != nullptr && live[u]) {
                const int64_t row = base + static_cast<int64_t>(u) * row_lanes;
                uint16_t* dst = a.g_bf16 + row * a.cols + col0;
                if constexpr (VEC) {
                    u32x4 packed;
#pragma unroll
                    for (int p = 0; p < 4; ++p) {
                        packed[p] = pack_bf16(v[u][2 * p], v[u][2 * p + 1]);
                    }
                    *reinterpret_cast<u32x4*>(dst) = packed;
                } else {
#pragma unroll
                    for (int i = 0; i < 8; ++i) {
                        if (col0 + i < a.cols) {
                            dst[i] = to_bf16_bits(v[u][i]);
                        }
                    }
                }
            }
        }
    }
    if (a.partials == nullptr) {
        return;
    }
    // Row lanes of each column, combined in lane order.
    __shared__ float s_sum[kGradThreads * 8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        s_sum[t * 8 + i] = acc[i];
    }
    __syncthreads();
    for (int idx = t; idx < cw * 8; idx += kGradThreads) {
        const int64_t column = static_cast<int64_t>(blockIdx.y) * cw * 8 + idx;
        float total = 0.0f;
        for (int lane = 0; lane < row_lanes; ++lane) {
            total += s_sum[lane * cw * 8 + idx];
        }
        if (column < a.cols) {
            a.partials[static_cast<int64_t>(blockIdx.x) * a.cols + column] = total;
        }
    }
}

// out[c] = sum over splits s of partials[s][c]: 32 columns x 8 split lanes
// per workgroup; split lane l adds splits l, l + 8, ... in order (sixteen
// loads in flight), then the lanes are added in lane order.  One launch can
// serve two such sums over the same splits (a weight gradient and its bias):
// the first `blocks` workgroups take the first, the rest the second.
__global__ __launch_bounds__(kGradThreads) void column_sum_kernel(const float* partials, int64_t splits,
                                                                  int64_t cols, float* out,
                                                                  const float* partials2, int64_t cols2,
                                                                  float* out2, int64_t blocks) {
    constexpr int kLanes = kGradThreads / 32;
    constexpr int kLoads = 16;
    const int c = threadIdx.x & 31;
    const int lane = threadIdx.x >> 5;
    int64_t block = blockIdx.x;
    if (block >= blocks) {   // uniform over the workgroup
        block -= blocks;
        partials = partials2;
        cols = cols2;
        out = out2;
    }
    const int64_t column = block * 32 + c;
    const int64_t safe_column = column < cols ? column : 0;
    float acc = 0.0f;
    for (int64_t s0 = lane; s0 < splits; s0 += kLanes * kLoads) {
        float v[kLoads];
#pragma unroll
        for (int u = 0; u < kLoads; ++u) {
            const int64_t s = s0 + static_cast<int64_t>(u) * kLanes;
            v[u] = partials[(s < splits ? s : 0) * cols + safe_column];
        }
#pragma unroll
        for (int u = 0; u < kLoads; ++u) {
            if (s0 + static_cast<int64_t>(u) * kLanes < splits) {
                acc += v[u];
            }
        }
    }
    __shared__ float s_acc[kLanes][32];
    s_acc[lane][c] = acc;
    __syncthreads();
    if (lane == 0 && column < cols) {
        float total = 0.0f;
#pragma unroll
        for (int l = 0; l < kLanes; ++l) {
            total += s_acc[l][c];
        }
        out[column] = total;
    }
}

hipError_t launch_column_sum(const float* partials, int64_t splits, int64_t cols, float* out,
                             hipStream_t stream) {
    return launch_column_sums(partials, cols, out, nullptr, 0, nullptr, splits, stream);
}

hipError_t launch_column_sums(const float* partials, int64_t cols, float* out, const float* partials2,
                              int64_t cols2, float* out2, int64_t splits, hipStream_t stream) {
    const int64_t blocks = (cols + 31) / 32;
    const int64_t blocks2 = (cols2 + 31) / 32;
    const dim3 grid(static_cast<unsigned>(blocks + blocks2));
    column_sum_kernel<<<grid, kGradThreads, 0, stream>>>(partials, splits, cols, out, partials2, cols2, out2,
                                                         blocks);
    return hipGetLastError();
}

hipError_t launch_grad_columns(const GradColumnsArgs& a, int g_dtype, bool vec, int64_t splits,
                               int64_t slabs, float* column_sums, hipStream_t stream) {
    const dim3 grid(static_cast<unsigned>(splits), static_cast<unsigned>(slabs));
    if (splits == 0) {
        // No rows: the column sums are zero.
    } else if (g_dtype == LSSO_HIP_BF16) {
        if (vec) {
            grad_columns_kernel<LSSO_HIP_BF16, true><<<grid, kGradThreads, 0, stream>>>(a);
        } else {
            grad_columns_kernel<LSSO_HIP_BF16, false><<<grid, kGradThreads, 0, stream>>>(a);
        }
    } else {
        if (vec) {
            grad_columns_kernel<LSSO_HIP_F16, true><<<grid, kGradThreads, 0, stream>>>(a);
        } else {
            grad_columns_kernel<LSSO_HIP_F16, false><<<grid, kGradThreads, 0, stream>>>(a);
        }
    }
    hipError_t error = hipGetLastError();
    if (error != hipSuccess || column_sums == nullptr) {
        return error;
    }
    return launch_column_sum(a.partials, splits, a.cols, column_sums, stream);
}

}  // namespace lsso_hip

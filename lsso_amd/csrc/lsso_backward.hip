// gfx950 first-order backward of the LSSO mixer (reference: lsso/ball/cuda.py:256-280,
// csrc/ball/backward.cu:326-1667), restated for the Gram-Cholesky forward.
//
// Per system (b, h) with a = rot(R) / sqrt(n), P = a L^-T, L L^T = a^T a + I:
//   forward:  s = a^T C, z = L^-1 s, Theta = Theta0 + z W / sqrt(n),
//             u = (I + K)^-1 z, x = 2u - (1 + eta) z, m = L^-T x,
//             Y = eta C + a m.
//   backward (dY given):
//     dm = a^T dY                                     (token reduction)
//     dx = L^-1 dm,  v = (I + K)^-T (2 dx),  dK = -v u^T
//     dF = (dK + dK^T) F
//     dTheta = tril(dF, -1) + diag(dF_ii sigmoid(Theta_ii + log(e - 1)))
//              + triu(dK - dK^T, 1)
//     dz = -(1 + eta) dx + v + dTheta W^T / sqrt(n),   ds = L^-T dz
//     Lbar = tril(-m dx^T - ds z^T),  Mbar = L^-T Phi(L^T Lbar) L^-1
//            (Phi: lower triangle, halved diagonal),   Gamma = Mbar + Mbar^T
//     dW = z^T dTheta / sqrt(n),  deta = <dY, C> - <dx, z>
//   per token (token map):
//     dA = dY M'^T + C (ds / sqrt(n))^T + A Gamma / n      (A = rot(R), M' = m / sqrt(n))
//     dC = eta dY + A ds / sqrt(n),   dR = rot^T(dA).
// Kernels: the token reduction reuses reduce_kernel with dY as its content;
// bwd_solve_kernel runs the compact algebra of one system in LDS and writes
// the token-map operands as MFMA records; bwd_apply_kernel is the token map;
// param_reduce_kernel sums parameter gradients over the batch in fixed order.

#include <type_traits>

#include "lsso_device.h"
#include "lsso_internal.h"
#include "lsso_hip.h"

namespace lsso_hip {

constexpr int kBwdThreads = 256;
constexpr int kBwdMaxHeadDim = 64;

bool backward_supported(int64_t rank, int64_t head_dim) {
    return (rank == 16 || rank == 32 || rank == 48 || rank == 64) && head_dim >= 1;
}

// ---------------------------------------------------------------------------
// MFMA operand records of an M x K FP32 matrix split into BF16 hi + lo.
// K32 steps (16x16x32): lane (g, q) of row block rb and step s holds row
// 16 rb + q, columns 32 s + 8 g .. +7 (hi then lo, 16 bf16).  K16 steps
// (16x16x16): columns 16 s + 4 g .. +3 (8 bf16).  Rows and columns past the
// matrix are zero.
template <bool K32>
struct RecordShape {
    static constexpr int kWidth = K32 ? 32 : 16;     // K per step
    static constexpr int kPerLane = K32 ? 8 : 4;     // values per lane per part
    static constexpr int kLaneHalfs = 2 * kPerLane;  // hi + lo
};

template <bool K32>
__host__ __device__ constexpr int64_t record_halfs(int64_t rows, int64_t cols) {
    using RS = RecordShape<K32>;
    return ((rows + 15) / 16) * ((cols + RS::kWidth - 1) / RS::kWidth) * 64 * RS::kLaneHalfs;
}

// Writes the records of `value(i, k)` (i < rows, k < cols) with all threads
// of the workgroup.
template <bool K32, typename Value>
__device__ __forceinline__ void write_records(uint16_t* out, int rows, int cols, Value value) {
    using RS = RecordShape<K32>;
    const int row_blocks = (rows + 15) / 16;
    const int steps = (cols + RS::kWidth - 1) / RS::kWidth;
    const int lanes = row_blocks * steps * 64;
    for (int idx = threadIdx.x; idx < lanes; idx += blockDim.x) {
        const int lane = idx & 63;
        const int step = (idx >> 6) % steps;
        const int rb = (idx >> 6) / steps;
        const int row = 16 * rb + (lane & 15);
        const int k0 = RS::kWidth * step + RS::kPerLane * (lane >> 4);
        uint16_t* rec = out + static_cast<int64_t>(idx) * RS::kLaneHalfs;
#pragma unroll
        for (int i = 0; i < RS::kPerLane; i += 2) {
            const float v0 = (row < rows && k0 + i < cols) ? value(row, k0 + i) : 0.0f;
            const float v1 = (row < rows && k0 + i + 1 < cols) ? value(row, k0 + i + 1) : 0.0f;
            uint32_t hi, lo;
            split_bf16(v0, v1, hi, lo);
            *reinterpret_cast<uint32_t*>(rec + i) = hi;
            *reinterpret_cast<uint32_t*>(rec + RS::kPerLane + i) = lo;
        }
    }
}

// C[i][j] = sum_k A(i, k) B(k, j) over an M x N output on FP32 MFMA
// (v_mfma_f32_16x16x4_f32, 16 x 16 tiles, wave w of the workgroup takes
// tiles w, w + 4, ...): lane (r, q) = (lane % 16, lane / 16) supplies
// A(i0 + r, k + q) and B(k + q, j0 + r) per step of 4 and holds rows
// i0 + 4 q .. + 3 of column j0 + r of the tile.  Each operand element is
// read once per tile; a per-element dot product would read every A row and
// B column once per output and is bound by the LDS return path.  Elements
// past M, N or K read as zero.  K <= KMAX; the K loop is unrolled to KMAX
// so that a tile's operand reads are all issued before its MFMAs.
template <int KMAX, typename FA, typename FB, typename Store>
__device__ __forceinline__ void block_product(int M, int N, int K, FA a, FB b, Store store) {
    const int wave = threadIdx.x >> 6;
    const int waves = blockDim.x >> 6;
    const int lane = threadIdx.x & 63;
    const int r = lane & 15;
    const int q = lane >> 4;
    const int ncols = (N + 15) / 16;
    const int tiles = ((M + 15) / 16) * ncols;
    for (int tile = wave; tile < tiles; tile += waves) {
        const int i0 = 16 * (tile / ncols);
        const int j0 = 16 * (tile - (tile / ncols) * ncols);
        const int i = i0 + r;
        const int j = j0 + r;
        float av[KMAX / 4];
        float bv[KMAX / 4];
#pragma unroll
        for (int s = 0; s < KMAX / 4; ++s) {
            const int kk = 4 * s + q;
            av[s] = (i < M && kk < K) ? a(i, kk) : 0.0f;
            bv[s] = (j < N && kk < K) ? b(kk, j) : 0.0f;
        }
        f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int s = 0; s < KMAX / 4; ++s) {
            if (4 * s < K) {
                acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av[s], bv[s], acc, 0, 0, 0);
            }
        }
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            const int row = i0 + 4 * q + m;
            if (row < M && j < N) {
                store(row, j, acc[m]);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Compact backward of one system.  DMAX: the bound of head_dim (32 or 64)
// that sizes the d-length products.
template <int R, int DMAX>
__global__ __launch_bounds__(kBwdThreads) void bwd_solve_kernel(BwdSolveArgs a) {
    constexpr int PR = R + 1;                         // r x r pitch
    constexpr int PD = DMAX + 1;                      // r x d pitch (two workgroups per CU at d <= 32)
    __shared__ float s_linv[R * PR];
    __shared__ float s_k[R * PR];    // (I+K)^-1 -> dK -> L -> Mbar
    __shared__ float s_f[R * PR];    // Theta -> F -> Lbar -> P Linv
    __shared__ float s_d[R * PR];    // dF -> dTheta -> P
    __shared__ float s_z[R * PD];
    __shared__ float s_u[R * PD];    // u -> ds
    __shared__ float s_x[R * PD];    // x -> dx
    __shared__ float s_m[R * PD];
    __shared__ float s_v[R * PD];    // dm -> v -> dz
    __shared__ float s_diag[R];
    __shared__ float s_red[kBwdThreads / 64];

    const int tid = threadIdx.x;
    const int64_t system = blockIdx.x;
    const int64_t b = system / a.heads;
    const int64_t h = system - b * a.heads;
    const int d = static_cast<int>(a.head_dim);
    const float count = a.valid_counts != nullptr ? a.valid_counts[b] : static_cast<float>(a.length);
    const float root = sqrtf(count);
    const float eta = bounded_complement(a.eta_raw[h]);
    const float* tape = a.tape + system * a.tape_stride;
    const float* part = a.partials + system * a.chunks * a.partial_stride + R * R;
    const float* drive = a.drive + h * d * R;

    // ---- loads: every load of a thread is issued before its first LDS store
    // (the loads are latency-bound; a rolled loop would wait for each), as
    // 16-byte pieces of the tape's rows (and of the r x d rows and partials
    // when head_dim is a multiple of 4); L is held in registers until its
    // phase.
    constexpr int kSquare = (R * R / 4 + kBwdThreads - 1) / kBwdThreads;   // quads per thread
    f32x4 l_pre[kSquare];
    {
        f32x4 linv[kSquare];
        f32x4 inv[kSquare];
        f32x4 theta[kSquare];
#pragma unroll
        for (int t = 0; t < kSquare; ++t) {
            const int q = tid + t * kBwdThreads;
            const int idx = 4 * (q < R * R / 4 ? q : 0);
            linv[t] = *reinterpret_cast<const f32x4*>(tape + 3 * R * R + idx);
            inv[t] = *reinterpret_cast<const f32x4*>(tape + 2 * R * R + idx);
            theta[t] = *reinterpret_cast<const f32x4*>(tape + R * R + idx);
            l_pre[t] = *reinterpret_cast<const f32x4*>(tape + idx);
        }
        // z, u and the chunk sums of dm (r x d), W floats per item.
        auto rect = [&](auto vec_c) {
            constexpr int W = decltype(vec_c)::value ? 4 : 1;
            using T = typename std::conditional<W == 4, f32x4, float>::type;
            constexpr int kRect = (R * kBwdMaxHeadDim / W + kBwdThreads - 1) / kBwdThreads;
            const int items = R * d / W;
            auto at = [&](int t) {
                const int item = tid + t * kBwdThreads;
                return W * (item < items ? item : 0);
            };
            auto elem = [](const T& v, int e) {
                if constexpr (W == 4) {
                    return v[e];
                } else {
                    return v;
                }
            };
            T zv[kRect];
            T uv[kRect];
            T dmv[kRect];
#pragma unroll
            for (int t = 0; t < kRect; ++t) {
                zv[t] = *reinterpret_cast<const T*>(tape + 4 * R * R + at(t));
                uv[t] = *reinterpret_cast<const T*>(tape + 4 * R * R + R * d + at(t));
                dmv[t] = T{};
            }
            // Chunk partials in ascending order, four chunks' loads in flight
            // (one chunk at a time waited out each chunk's load latency).
            constexpr int kChunkBatch = 4;
            for (int ch0 = 0; ch0 < a.chunks; ch0 += kChunkBatch) {
                T pv[kChunkBatch][kRect];
#pragma unroll
                for (int u = 0; u < kChunkBatch; ++u) {
                    const int64_t ch = ch0 + u < a.chunks ? ch0 + u : a.chunks - 1;
#pragma unroll
                    for (int t = 0; t < kRect; ++t) {
                        pv[u][t] = *reinterpret_cast<const T*>(part + ch * a.partial_stride + at(t));
                    }
                }
#pragma unroll
                for (int u = 0; u < kChunkBatch; ++u) {
                    if (ch0 + u < a.chunks) {
#pragma unroll
                        for (int t = 0; t < kRect; ++t) {
                            dmv[t] += pv[u][t];
                        }
                    }
                }
            }
#pragma unroll
            for (int t = 0; t < kRect; ++t) {
                const int item = tid + t * kBwdThreads;
                if (item < items) {
#pragma unroll
                    for (int e = 0; e < W; ++e) {
                        const int idx = W * item + e;
                        const int i = idx / d;
                        const int f = idx - i * d;
                        const float z = elem(zv[t], e);
                        const float u = elem(uv[t], e);
                        s_z[i * PD + f] = z;
                        s_u[i * PD + f] = u;
                        s_x[i * PD + f] = 2.0f * u - (1.0f + eta) * z;
                        s_v[i * PD + f] = elem(dmv[t], e) / root;
                    }
                }
            }
        };
        if (d % 4 == 0) {
            rect(std::true_type{});
        } else {
            rect(std::false_type{});
        }
#pragma unroll
        for (int t = 0; t < kSquare; ++t) {
            const int q = tid + t * kBwdThreads;
            if (q < R * R / 4) {
                const int i = (4 * q) / R;
                const int j = 4 * q - i * R;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    s_linv[i * PR + j + e] = linv[t][e];
                    s_k[i * PR + j + e] = inv[t][e];
                    s_f[i * PR + j + e] = theta[t][e];
                }
            }
        }
    }
    __syncthreads();

    // ---- m = L^-T x;  dx = L^-1 dm ------------------------------------------
    block_product<R>(R, d, R, [&](int i, int k) { return s_linv[k * PR + i]; },
                  [&](int k, int j) { return s_x[k * PD + j]; },
                  [&](int i, int j, float v) { s_m[i * PD + j] = v; });
    __syncthreads();
    block_product<R>(R, d, R, [&](int i, int k) { return s_linv[i * PR + k]; },
                  [&](int k, int j) { return s_v[k * PD + j]; },
                  [&](int i, int j, float v) { s_x[i * PD + j] = v; });
    __syncthreads();
    // ---- v = (I + K)^-T (2 dx) ----------------------------------------------
    block_product<R>(R, d, R, [&](int i, int k) { return s_k[k * PR + i]; },
                  [&](int k, int j) { return 2.0f * s_x[k * PD + j]; },
                  [&](int i, int j, float v) { s_v[i * PD + j] = v; });
    __syncthreads();
    // ---- dK = -v u^T;  F and diag(Theta) -------------------------------------
    block_product<DMAX>(R, R, d, [&](int i, int k) { return s_v[i * PD + k]; },
                  [&](int k, int j) { return s_u[j * PD + k]; },
                  [&](int i, int j, float v) { s_k[i * PR + j] = -v; });
    for (int idx = tid; idx < R * R; idx += kBwdThreads) {
        const int i = idx / R;
        const int j = idx - i * R;
        const float theta = s_f[i * PR + j];
        float value = j < i ? theta : 0.0f;
        if (i == j) {
            s_diag[i] = theta;
            value = softplus_one(theta);
        }
        s_f[i * PR + j] = value;
    }
    __syncthreads();
    // ---- dF = (dK + dK^T) F;  dTheta -----------------------------------------
    block_product<R>(R, R, R, [&](int i, int k) { return s_k[i * PR + k] + s_k[k * PR + i]; },
                  [&](int k, int j) { return s_f[k * PR + j]; },
                  [&](int i, int j, float v) { s_d[i * PR + j] = v; });
    __syncthreads();
    for (int idx = tid; idx < R * R; idx += kBwdThreads) {
        const int i = idx / R;
        const int j = idx - i * R;
        float g;
        if (j < i) {
            g = s_d[i * PR + j];
        } else if (j == i) {
            const float shifted = s_diag[i] + kSoftplusOneOffset;
            g = s_d[i * PR + j] / (1.0f + expf(-shifted));
        } else {
            g = s_k[i * PR + j] - s_k[j * PR + i];
        }
        s_d[i * PR + j] = g;
    }
    __syncthreads();
    // ---- parameter partials: dTheta, z^T dTheta / sqrt(n) ------------------
    {
        float* dtheta = a.dtheta_part + system * R * R;
        for (int idx = tid; idx < R * R; idx += kBwdThreads) {
            const int i = idx / R;
            const int j = idx - i * R;
            dtheta[idx] = s_d[i * PR + j];
        }
        float* ddrive = a.ddrive_part + system * d * R;
        block_product<R>(d, R, R, [&](int f, int k) { return s_z[k * PD + f]; },
                      [&](int k, int j) { return s_d[k * PR + j]; },
                      [&](int f, int j, float v) { ddrive[f * R + j] = v / root; });
    }
    // ---- dz = -(1 + eta) dx + v + dTheta W^T / sqrt(n) (in place in s_v) ---
    block_product<R>(R, d, R, [&](int i, int k) { return s_d[i * PR + k]; },
                  [&](int k, int f) { return drive[f * R + k]; },
                  [&](int i, int f, float v) {
                      s_v[i * PD + f] = -(1.0f + eta) * s_x[i * PD + f] + s_v[i * PD + f] + v / root;
                  });
    __syncthreads();
    // ---- ds = L^-T dz -> s_u;  -<dx, z> --------------------------------------
    block_product<R>(R, d, R, [&](int i, int k) { return s_linv[k * PR + i]; },
                  [&](int k, int j) { return s_v[k * PD + j]; },
                  [&](int i, int j, float v) { s_u[i * PD + j] = v; });
    {
        float partial = 0.0f;
        for (int idx = tid; idx < R * d; idx += kBwdThreads) {
            const int i = idx / d;
            const int f = idx - i * d;
            partial = fmaf(s_x[i * PD + f], s_z[i * PD + f], partial);
        }
        for (int offset = 32; offset > 0; offset >>= 1) {
            partial += __shfl_xor(partial, offset);
        }
        if ((tid & 63) == 0) {
            s_red[tid >> 6] = partial;
        }
    }
    __syncthreads();
    if (tid == 0) {
        float total = 0.0f;
        for (int w = 0; w < kBwdThreads / 64; ++w) {
            total += s_red[w];
        }
        a.deta_part[system] = -total;
    }
    // ---- Lbar = tril(-m dx^T - ds z^T) -> s_f;  L -> s_k ---------------------
    // m dx^T, then + ds z^T, negated below the diagonal.
    block_product<DMAX>(R, R, d, [&](int i, int f) { return s_m[i * PD + f]; },
                        [&](int f, int j) { return s_x[j * PD + f]; },
                        [&](int i, int j, float v) { s_f[i * PR + j] = v; });
    // Each element is stored by the lane that stored it above (same tiles,
    // same lane mapping), so no barrier is needed between the two products.
    block_product<DMAX>(R, R, d, [&](int i, int f) { return s_u[i * PD + f]; },
                        [&](int f, int j) { return s_z[j * PD + f]; },
                        [&](int i, int j, float v) { s_f[i * PR + j] = j <= i ? -(s_f[i * PR + j] + v) : 0.0f; });
#pragma unroll
    for (int t = 0; t < kSquare; ++t) {
        const int q = tid + t * kBwdThreads;
        if (q < R * R / 4) {
            const int i = (4 * q) / R;
            const int j = 4 * q - i * R;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                s_k[i * PR + j + e] = l_pre[t][e];
            }
        }
    }
    __syncthreads();
    // ---- P = Phi(L^T Lbar) -> s_d --------------------------------------------
    block_product<R>(R, R, R, [&](int i, int k) { return s_k[k * PR + i]; },
                  [&](int k, int j) { return s_f[k * PR + j]; },
                  [&](int i, int j, float v) {
                      s_d[i * PR + j] = j < i ? v : (j == i ? 0.5f * v : 0.0f);
                  });
    __syncthreads();
    // ---- Mbar = L^-T P L^-1 --------------------------------------------------
    block_product<R>(R, R, R, [&](int i, int k) { return s_d[i * PR + k]; },
                  [&](int k, int j) { return s_linv[k * PR + j]; },
                  [&](int i, int j, float v) { s_f[i * PR + j] = v; });
    __syncthreads();
    block_product<R>(R, R, R, [&](int i, int k) { return s_linv[k * PR + i]; },
                  [&](int k, int j) { return s_f[k * PR + j]; },
                  [&](int i, int j, float v) { s_k[i * PR + j] = v; });
    __syncthreads();

    // ---- token-map operand records -------------------------------------------
    const float inv_root = 1.0f / root;
    const float inv_count = 1.0f / count;
    uint16_t* rec = a.records + system * a.record_stride;
    constexpr bool kRank32 = (R % 32) == 0;
    if (a.feature_k32) {
        write_records<true>(rec + a.off_m, R, d, [&](int i, int f) { return s_m[i * PD + f] * inv_root; });
        write_records<true>(rec + a.off_e, R, d, [&](int i, int f) { return s_u[i * PD + f] * inv_root; });
    } else {
        write_records<false>(rec + a.off_m, R, d, [&](int i, int f) { return s_m[i * PD + f] * inv_root; });
        write_records<false>(rec + a.off_e, R, d, [&](int i, int f) { return s_u[i * PD + f] * inv_root; });
    }
    write_records<kRank32>(rec + a.off_g, R, R, [&](int i, int k) {
        return (s_k[i * PR + k] + s_k[k * PR + i]) * inv_count;
    });
    write_records<kRank32>(rec + a.off_f, d, R, [&](int f, int k) { return s_u[k * PD + f] * inv_root; });
}

// Records of rows [rb0, rb1) x K steps [s0, s1) of an M x K matrix whose
// full record has `steps` K steps (the layout of write_records).
template <bool K32, typename Value>
__device__ __forceinline__ void write_record_block(uint16_t* out, int rows, int cols, int rb0, int rb1,
                                                   int s0, int s1, Value value) {
    using RS = RecordShape<K32>;
    const int steps = (cols + RS::kWidth - 1) / RS::kWidth;
    const int width = s1 - s0;
    const int lanes = (rb1 - rb0) * width * 64;
    for (int idx = threadIdx.x; idx < lanes; idx += blockDim.x) {
        const int lane = idx & 63;
        const int step = s0 + (idx >> 6) % width;
        const int rb = rb0 + (idx >> 6) / width;
        const int row = 16 * rb + (lane & 15);
        const int k0 = RS::kWidth * step + RS::kPerLane * (lane >> 4);
        uint16_t* rec = out + ((static_cast<int64_t>(rb) * steps + step) * 64 + lane) * RS::kLaneHalfs;
#pragma unroll
        for (int i = 0; i < RS::kPerLane; i += 2) {
            const float v0 = (row < rows && k0 + i < cols) ? value(row, k0 + i) : 0.0f;
            const float v1 = (row < rows && k0 + i + 1 < cols) ? value(row, k0 + i + 1) : 0.0f;
            uint32_t hi, lo;
            split_bf16(v0, v1, hi, lo);
            *reinterpret_cast<uint32_t*>(rec + i) = hi;
            *reinterpret_cast<uint32_t*>(rec + RS::kPerLane + i) = lo;
        }
    }
}

// ---------------------------------------------------------------------------
// Compact backward of one system for head_dim > 64: the algebra of
// bwd_solve_kernel with the r x d quantities taken in panels of kWidePanel
// columns, so that LDS holds only r x r matrices and one panel of each r x d
// one.  The columns of every r x d product are independent, except for the
// sums over d: dK = -v u^T (needed before dTheta, which every panel's dz
// needs) and Lbar = -(m dx^T + ds z^T).  Pass 1 accumulates dK over the
// panels; pass 2 recomputes each panel's m, dx and v from the tape and the dm
// partials, then forms dz, ds, the Lbar sum, the <dx, z> sum, the drive
// gradient rows and the panel's token-map records.
constexpr int kWidePanel = 32;

template <int R>
__global__ __launch_bounds__(kBwdThreads) void bwd_solve_wide_kernel(BwdSolveArgs a) {
    constexpr int PR = R + 1;
    constexpr int PP = kWidePanel + 1;
    __shared__ float s_linv[R * PR];
    __shared__ float s_kinv[R * PR];   // (I+K)^-1 -> L (after pass 2)
    __shared__ float s_f[R * PR];      // Theta -> F -> Lbar -> Mbar
    __shared__ float s_dk[R * PR];     // dK -> L^-T P -> Mbar sym
    __shared__ float s_d[R * PR];      // dF -> dTheta -> P
    __shared__ float s_z[R * PP];
    __shared__ float s_u[R * PP];      // u -> ds
    __shared__ float s_dx[R * PP];
    __shared__ float s_m[R * PP];
    __shared__ float s_v[R * PP];      // dm -> v -> dz
    __shared__ float s_diag[R];
    __shared__ float s_red[kBwdThreads / 64];

    const int tid = threadIdx.x;
    const int64_t system = blockIdx.x;
    const int64_t b = system / a.heads;
    const int64_t h = system - b * a.heads;
    const int d = static_cast<int>(a.head_dim);
    const float count = a.valid_counts != nullptr ? a.valid_counts[b] : static_cast<float>(a.length);
    const float root = sqrtf(count);
    const float inv_root = 1.0f / root;
    const float eta = bounded_complement(a.eta_raw[h]);
    const float* tape = a.tape + system * a.tape_stride;
    const float* tape_z = tape + 4 * R * R;
    const float* tape_u = tape_z + R * d;
    const float* part = a.partials + system * a.chunks * a.partial_stride + R * R;
    const float* drive = a.drive + h * d * R;
    const int chunks = static_cast<int>(a.chunks);
    const int stride = static_cast<int>(a.partial_stride);

    for (int idx = tid; idx < R * R; idx += kBwdThreads) {
        const int i = idx / R;
        const int j = idx - i * R;
        s_linv[i * PR + j] = tape[3 * R * R + idx];
        s_kinv[i * PR + j] = tape[2 * R * R + idx];
        s_f[i * PR + j] = tape[R * R + idx];
        s_dk[i * PR + j] = 0.0f;
    }

    // A panel's z, u and dm / sqrt(n) (chunk partials summed in order) into LDS.
    auto load_panel = [&](int c0, int w) {
        for (int idx = tid; idx < R * w; idx += kBwdThreads) {
            const int i = idx / w;
            const int f = c0 + (idx - i * w);
            float dm = 0.0f;
            for (int ch = 0; ch < chunks; ++ch) {
                dm += part[ch * stride + i * d + f];
            }
            s_z[i * PP + f - c0] = tape_z[i * d + f];
            s_u[i * PP + f - c0] = tape_u[i * d + f];
            s_v[i * PP + f - c0] = dm / root;
        }
    };
    // dx = L^-1 dm (s_v -> s_dx), then v = (I + K)^-T (2 dx) (-> s_v).
    auto panel_dx_v = [&](int w) {
        block_product<R>(R, w, R, [&](int i, int k) { return s_linv[i * PR + k]; },
                         [&](int k, int j) { return s_v[k * PP + j]; },
                         [&](int i, int j, float v) { s_dx[i * PP + j] = v; });
        __syncthreads();
        block_product<R>(R, w, R, [&](int i, int k) { return s_kinv[k * PR + i]; },
                         [&](int k, int j) { return 2.0f * s_dx[k * PP + j]; },
                         [&](int i, int j, float v) { s_v[i * PP + j] = v; });
        __syncthreads();
    };
    __syncthreads();

    // ---- pass 1: dK = -sum over panels of v u^T ------------------------------
    for (int c0 = 0; c0 < d; c0 += kWidePanel) {
        const int w = d - c0 < kWidePanel ? d - c0 : kWidePanel;
        load_panel(c0, w);
        __syncthreads();
        panel_dx_v(w);
        block_product<kWidePanel>(R, R, w, [&](int i, int k) { return s_v[i * PP + k]; },
                                  [&](int k, int j) { return s_u[j * PP + k]; },
                                  [&](int i, int j, float v) { s_dk[i * PR + j] -= v; });
        __syncthreads();
    }

    // ---- F, dF = (dK + dK^T) F, dTheta ---------------------------------------
    for (int idx = tid; idx < R * R; idx += kBwdThreads) {
        const int i = idx / R;
        const int j = idx - i * R;
        const float theta = s_f[i * PR + j];
        float value = j < i ? theta : 0.0f;
        if (i == j) {
            s_diag[i] = theta;
            value = softplus_one(theta);
        }
        s_f[i * PR + j] = value;
    }
    __syncthreads();
    block_product<R>(R, R, R, [&](int i, int k) { return s_dk[i * PR + k] + s_dk[k * PR + i]; },
                     [&](int k, int j) { return s_f[k * PR + j]; },
                     [&](int i, int j, float v) { s_d[i * PR + j] = v; });
    __syncthreads();
    float* dtheta = a.dtheta_part + system * R * R;
    for (int idx = tid; idx < R * R; idx += kBwdThreads) {
        const int i = idx / R;
        const int j = idx - i * R;
        float g;
        if (j < i) {
            g = s_d[i * PR + j];
        } else if (j == i) {
            const float shifted = s_diag[i] + kSoftplusOneOffset;
            g = s_d[i * PR + j] / (1.0f + expf(-shifted));
        } else {
            g = s_dk[i * PR + j] - s_dk[j * PR + i];
        }
        s_d[i * PR + j] = g;
        dtheta[idx] = g;
        s_f[i * PR + j] = 0.0f;   // Lbar accumulator
    }
    __syncthreads();

    // ---- pass 2 ---------------------------------------------------------------
    uint16_t* rec = a.records + system * a.record_stride;
    float* ddrive = a.ddrive_part + system * d * R;
    float dot = 0.0f;
    for (int c0 = 0; c0 < d; c0 += kWidePanel) {
        const int w = d - c0 < kWidePanel ? d - c0 : kWidePanel;
        load_panel(c0, w);
        __syncthreads();
        // m = L^-T x with x = 2 u - (1 + eta) z.
        block_product<R>(R, w, R, [&](int i, int k) { return s_linv[k * PR + i]; },
                         [&](int k, int j) { return 2.0f * s_u[k * PP + j] - (1.0f + eta) * s_z[k * PP + j]; },
                         [&](int i, int j, float v) { s_m[i * PP + j] = v; });
        panel_dx_v(w);
        // Drive gradient rows c0 .. c0 + w: z^T dTheta / sqrt(n).
        block_product<R>(w, R, R, [&](int f, int k) { return s_z[k * PP + f]; },
                         [&](int k, int j) { return s_d[k * PR + j]; },
                         [&](int f, int j, float v) { ddrive[(c0 + f) * R + j] = v / root; });
        // dz = -(1 + eta) dx + v + dTheta W^T / sqrt(n), in place in s_v.
        block_product<R>(R, w, R, [&](int i, int k) { return s_d[i * PR + k]; },
                         [&](int k, int f) { return drive[(c0 + f) * R + k]; },
                         [&](int i, int f, float v) {
                             s_v[i * PP + f] = -(1.0f + eta) * s_dx[i * PP + f] + s_v[i * PP + f] + v / root;
                         });
        for (int idx = tid; idx < R * w; idx += kBwdThreads) {
            const int i = idx / w;
            const int f = idx - i * w;
            dot = fmaf(s_dx[i * PP + f], s_z[i * PP + f], dot);
        }
        __syncthreads();
        // ds = L^-T dz -> s_u (u is spent: m holds what it fed).
        block_product<R>(R, w, R, [&](int i, int k) { return s_linv[k * PR + i]; },
                         [&](int k, int j) { return s_v[k * PP + j]; },
                         [&](int i, int j, float v) { s_u[i * PP + j] = v; });
        __syncthreads();
        // Lbar sum: + m dx^T + ds z^T (each element stays with one lane).
        block_product<kWidePanel>(R, R, w, [&](int i, int f) { return s_m[i * PP + f]; },
                                  [&](int f, int j) { return s_dx[j * PP + f]; },
                                  [&](int i, int j, float v) { s_f[i * PR + j] += v; });
        block_product<kWidePanel>(R, R, w, [&](int i, int f) { return s_u[i * PP + f]; },
                                  [&](int f, int j) { return s_z[j * PP + f]; },
                                  [&](int i, int j, float v) { s_f[i * PR + j] += v; });
        // Token-map records of this panel's columns (M' = m / sqrt(n) and
        // ds / sqrt(n)) and rows (ds^T / sqrt(n)).
        if (a.feature_k32) {
            write_record_block<true>(rec + a.off_m, R, d, 0, R / 16, c0 / 32, (c0 + w + 31) / 32,
                                     [&](int i, int f) { return s_m[i * PP + f - c0] * inv_root; });
            write_record_block<true>(rec + a.off_e, R, d, 0, R / 16, c0 / 32, (c0 + w + 31) / 32,
                                     [&](int i, int f) { return s_u[i * PP + f - c0] * inv_root; });
        } else {
            write_record_block<false>(rec + a.off_m, R, d, 0, R / 16, c0 / 16, (c0 + w + 15) / 16,
                                      [&](int i, int f) { return s_m[i * PP + f - c0] * inv_root; });
            write_record_block<false>(rec + a.off_e, R, d, 0, R / 16, c0 / 16, (c0 + w + 15) / 16,
                                      [&](int i, int f) { return s_u[i * PP + f - c0] * inv_root; });
        }
        constexpr bool kRank32 = (R % 32) == 0;
        write_record_block<kRank32>(rec + a.off_f, d, R, c0 / 16, (c0 + w + 15) / 16, 0,
                                    R / RecordShape<kRank32>::kWidth,
                                    [&](int f, int k) { return s_u[k * PP + f - c0] * inv_root; });
        __syncthreads();
    }

    // ---- -<dx, z> --------------------------------------------------------------
    for (int offset = 32; offset > 0; offset >>= 1) {
        dot += __shfl_xor(dot, offset);
    }
    if ((tid & 63) == 0) {
        s_red[tid >> 6] = dot;
    }
    // ---- Lbar = tril(-(m dx^T + ds z^T)); L -> s_kinv --------------------------
    for (int idx = tid; idx < R * R; idx += kBwdThreads) {
        const int i = idx / R;
        const int j = idx - i * R;
        s_f[i * PR + j] = j <= i ? -s_f[i * PR + j] : 0.0f;
        s_kinv[i * PR + j] = tape[idx];
    }
    __syncthreads();
    if (tid == 0) {
        float total = 0.0f;
        for (int w = 0; w < kBwdThreads / 64; ++w) {
            total += s_red[w];
        }
        a.deta_part[system] = -total;
    }
    // ---- P = Phi(L^T Lbar) -> s_d ---------------------------------------------
    block_product<R>(R, R, R, [&](int i, int k) { return s_kinv[k * PR + i]; },
                     [&](int k, int j) { return s_f[k * PR + j]; },
                     [&](int i, int j, float v) {
                         s_d[i * PR + j] = j < i ? v : (j == i ? 0.5f * v : 0.0f);
                     });
    __syncthreads();
    // ---- Mbar = L^-T P L^-1 ----------------------------------------------------
    block_product<R>(R, R, R, [&](int i, int k) { return s_d[i * PR + k]; },
                     [&](int k, int j) { return s_linv[k * PR + j]; },
                     [&](int i, int j, float v) { s_f[i * PR + j] = v; });
    __syncthreads();
    block_product<R>(R, R, R, [&](int i, int k) { return s_linv[k * PR + i]; },
                     [&](int k, int j) { return s_f[k * PR + j]; },
                     [&](int i, int j, float v) { s_dk[i * PR + j] = v; });
    __syncthreads();
    const float inv_count = 1.0f / count;
    constexpr bool kRank32 = (R % 32) == 0;
    write_records<kRank32>(rec + a.off_g, R, R, [&](int i, int k) {
        return (s_dk[i * PR + k] + s_dk[k * PR + i]) * inv_count;
    });
}

// ---------------------------------------------------------------------------
// Token map: one wave per (b, chunk, h), 16 tokens per step.
template <int R, bool DK32, bool VEC>
__global__ __launch_bounds__(256) void bwd_apply_kernel(BwdApplyArgs a) {
    constexpr bool RK32 = (R % 32) == 0;
    using RR = RecordShape<RK32>;
    using RD = RecordShape<DK32>;
    constexpr int RBLK = R / 16;                        // rank row blocks
    constexpr int RSTEPS = R / RR::kWidth;              // rank K steps
    constexpr int PAIRS = R / 2;
    const int lane = threadIdx.x & 63;
    const int64_t wave = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
    if (wave >= a.total_waves) {
        return;
    }
    int64_t rest = wave;
    const int64_t h = rest % a.heads;
    rest /= a.heads;
    const int64_t chunk = rest % a.chunks;
    const int64_t b = rest / a.chunks;
    const int q = lane & 15;
    const int g = lane >> 4;
    const int64_t d = a.head_dim;
    const int64_t system = b * a.heads + h;
    const int dsteps = static_cast<int>((d + RD::kWidth - 1) / RD::kWidth);
    const int fblocks = static_cast<int>((d + 15) / 16);
    const float eta = bounded_complement(a.eta_raw[h]);
    const uint16_t* rec = a.records + system * a.record_stride;
    const uint16_t* rec_m = rec + a.off_m;
    const uint16_t* rec_e = rec + a.off_e;
    const uint16_t* rec_g = rec + a.off_g;
    const uint16_t* rec_f = rec + a.off_f;

    const int64_t begin = chunk * a.chunk_tokens;
    const int64_t end = begin + a.chunk_tokens < a.length ? begin + a.chunk_tokens : a.length;
    float dot = 0.0f;
    for (int64_t t0 = begin; t0 < end; t0 += 16) {
        const int64_t token = t0 + q;
        const bool live = token < end;
        const int64_t safe = live ? token : begin;
        const uint16_t* prow = a.projected + (b * a.length + safe) * a.width;
        const uint16_t* grow = a.grad_output + (b * a.length + safe) * a.grad_stride + h * d;
        const uint16_t* crow = prow + a.heads * R + h * d;
        const uint32_t* phrow = a.phases + b * a.phase_batch_stride + safe * PAIRS;
        uint16_t* out_row = a.grad_projected + (b * a.length + safe) * a.width;

        // Rotated relation as the B operand (rank K), split hi/lo.
        typedef typename std::conditional<RK32, u32x4, u32x2>::type RankOp;
        RankOp a_hi[RSTEPS];
        RankOp a_lo[RSTEPS];
#pragma unroll
        for (int s = 0; s < RSTEPS; ++s) {
            const int first = RR::kWidth * s + RR::kPerLane * g;
#pragma unroll
            for (int p = 0; p < RR::kPerLane / 2; ++p) {
                const uint32_t rel = live ? *reinterpret_cast<const uint32_t*>(prow + h * R + first + 2 * p) : 0u;
                const uint32_t ph = live ? phrow[first / 2 + p] : 0u;
                float e, o;
                rotate_pair(rel, ph, e, o);
                uint32_t hi, lo;
                split_bf16(e, o, hi, lo);
                a_hi[s][p] = hi;
                a_lo[s][p] = lo;
            }
        }
        // Features are taken in panels of kBwdMaxHeadDim: dY and C of one
        // panel are the B operands of its feature-K steps (exact in BF16);
        // the dA^T accumulators of every rank block run across all panels,
        // and the panel's dC blocks are finished inside it.  With one panel
        // (head_dim <= 64) the MFMA chains and the <dY, C> order are those of
        // the resident token map.
        typedef typename std::conditional<DK32, u32x4, u32x2>::type FeatOp;
        constexpr int kPanelSteps = kBwdMaxHeadDim / RD::kWidth;
        constexpr int kPanelBlocks = kBwdMaxHeadDim / 16;
        f32x4 acc_d[RBLK];
#pragma unroll
        for (int rb = 0; rb < RBLK; ++rb) {
            acc_d[rb] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
        }
        for (int panel = 0; panel * kPanelSteps < dsteps; ++panel) {
            const int s0 = panel * kPanelSteps;
            FeatOp y_op[kPanelSteps];
            FeatOp c_op[kPanelSteps];
#pragma unroll
            for (int ps = 0; ps < kPanelSteps; ++ps) {
                const int s = s0 + ps;
                y_op[ps] = FeatOp{};
                c_op[ps] = FeatOp{};
                if (s < dsteps) {
                    const int first = RD::kWidth * s + RD::kPerLane * g;
                    if constexpr (VEC) {
                        // d is a multiple of the per-lane run: whole runs or none.
                        const bool run = live && first < d;
                        y_op[ps] = run ? *reinterpret_cast<const FeatOp*>(grow + (run ? first : 0))
                                       : FeatOp{};
                        c_op[ps] = run ? *reinterpret_cast<const FeatOp*>(crow + (run ? first : 0))
                                       : FeatOp{};
#pragma unroll
                        for (int p = 0; p < RD::kPerLane / 2; ++p) {
                            dot = fmaf(bf16_lo(y_op[ps][p]), bf16_lo(c_op[ps][p]), dot);
                            dot = fmaf(bf16_hi(y_op[ps][p]), bf16_hi(c_op[ps][p]), dot);
                        }
                    } else {
#pragma unroll
                        for (int p = 0; p < RD::kPerLane / 2; ++p) {
                            const int f = first + 2 * p;
                            uint32_t yv = 0u, cv = 0u;
                            if (live && f < d) {
                                const uint32_t y_lo = grow[f];
                                const uint32_t c_lo = crow[f];
                                const uint32_t y_hi = f + 1 < d ? grow[f + 1] : 0u;
                                const uint32_t c_hi = f + 1 < d ? crow[f + 1] : 0u;
                                yv = y_lo | (y_hi << 16);
                                cv = c_lo | (c_hi << 16);
                            }
                            y_op[ps][p] = yv;
                            c_op[ps][p] = cv;
                            dot = fmaf(bf16_lo(yv), bf16_lo(cv), dot);
                            dot = fmaf(bf16_hi(yv), bf16_hi(cv), dot);
                        }
                    }
                }
            }

            // dA^T blocks, feature-K chain (dY, C): this panel's steps.
#pragma unroll
            for (int rb = 0; rb < RBLK; ++rb) {
#pragma unroll
                for (int ps = 0; ps < kPanelSteps; ++ps) {
                    const int s = s0 + ps;
                    if (s < dsteps) {
                        const int64_t o = ((static_cast<int64_t>(rb) * dsteps + s) * 64 + lane) * RD::kLaneHalfs;
                        if constexpr (DK32) {
                            const u32x4 mh = *reinterpret_cast<const u32x4*>(rec_m + o);
                            const u32x4 ml = *reinterpret_cast<const u32x4*>(rec_m + o + 8);
                            const u32x4 eh = *reinterpret_cast<const u32x4*>(rec_e + o);
                            const u32x4 el = *reinterpret_cast<const u32x4*>(rec_e + o + 8);
                            acc_d[rb] = mfma16x16x32(mh, y_op[ps], acc_d[rb]);
                            acc_d[rb] = mfma16x16x32(ml, y_op[ps], acc_d[rb]);
                            acc_d[rb] = mfma16x16x32(eh, c_op[ps], acc_d[rb]);
                            acc_d[rb] = mfma16x16x32(el, c_op[ps], acc_d[rb]);
                        } else {
                            const u32x2 mh = *reinterpret_cast<const u32x2*>(rec_m + o);
                            const u32x2 ml = *reinterpret_cast<const u32x2*>(rec_m + o + 4);
                            const u32x2 eh = *reinterpret_cast<const u32x2*>(rec_e + o);
                            const u32x2 el = *reinterpret_cast<const u32x2*>(rec_e + o + 4);
                            acc_d[rb] = mfma16x16x16(mh, y_op[ps], acc_d[rb]);
                            acc_d[rb] = mfma16x16x16(ml, y_op[ps], acc_d[rb]);
                            acc_d[rb] = mfma16x16x16(eh, c_op[ps], acc_d[rb]);
                            acc_d[rb] = mfma16x16x16(el, c_op[ps], acc_d[rb]);
                        }
                    }
                }
            }

            // dC^T blocks of this panel: eta dY + (ds / sqrt(n))^T A^T.
#pragma unroll
            for (int pb = 0; pb < kPanelBlocks; ++pb) {
                const int fb = panel * kPanelBlocks + pb;
                if (fb < fblocks) {
                    f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                    for (int s = 0; s < RSTEPS; ++s) {
                        const int64_t o = ((static_cast<int64_t>(fb) * RSTEPS + s) * 64 + lane) * RR::kLaneHalfs;
                        if constexpr (RK32) {
                            const u32x4 fh = *reinterpret_cast<const u32x4*>(rec_f + o);
                            const u32x4 fl = *reinterpret_cast<const u32x4*>(rec_f + o + 8);
                            acc = mfma16x16x32(fh, a_hi[s], acc);
                            acc = mfma16x16x32(fh, a_lo[s], acc);
                            acc = mfma16x16x32(fl, a_hi[s], acc);
                        } else {
                            const u32x2 fh = *reinterpret_cast<const u32x2*>(rec_f + o);
                            const u32x2 fl = *reinterpret_cast<const u32x2*>(rec_f + o + 4);
                            acc = mfma16x16x16(fh, a_hi[s], acc);
                            acc = mfma16x16x16(fh, a_lo[s], acc);
                            acc = mfma16x16x16(fl, a_hi[s], acc);
                        }
                    }
                    if (live) {
                        const int f0 = 16 * fb + 4 * g;
                        if (VEC && f0 + 4 <= d) {
                            const u32x2 dy = *reinterpret_cast<const u32x2*>(grow + f0);
                            u32x2 packed;
                            packed.x = pack_bf16(fmaf(eta, bf16_lo(dy.x), acc[0]), fmaf(eta, bf16_hi(dy.x), acc[1]));
                            packed.y = pack_bf16(fmaf(eta, bf16_lo(dy.y), acc[2]), fmaf(eta, bf16_hi(dy.y), acc[3]));
                            *reinterpret_cast<u32x2*>(out_row + a.heads * R + h * d + f0) = packed;
                        } else {
#pragma unroll
                            for (int i = 0; i < 4; ++i) {
                                if (f0 + i < d) {
                                    const float dy = bf16_bits_to_float(grow[f0 + i]);
                                    out_row[a.heads * R + h * d + f0 + i] = to_bf16_bits(fmaf(eta, dy, acc[i]));
                                }
                            }
                        }
                    }
                }
            }
        }

        // dA^T blocks, rank-K chain (A, kept apart from the feature chain),
        // then the rotation back to dR.
#pragma unroll
        for (int rb = 0; rb < RBLK; ++rb) {
            f32x4 acc_r = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int s = 0; s < RSTEPS; ++s) {
                const int64_t o = ((static_cast<int64_t>(rb) * RSTEPS + s) * 64 + lane) * RR::kLaneHalfs;
                if constexpr (RK32) {
                    const u32x4 gh = *reinterpret_cast<const u32x4*>(rec_g + o);
                    const u32x4 gl = *reinterpret_cast<const u32x4*>(rec_g + o + 8);
                    acc_r = mfma16x16x32(gh, a_hi[s], acc_r);
                    acc_r = mfma16x16x32(gh, a_lo[s], acc_r);
                    acc_r = mfma16x16x32(gl, a_hi[s], acc_r);
                } else {
                    const u32x2 gh = *reinterpret_cast<const u32x2*>(rec_g + o);
                    const u32x2 gl = *reinterpret_cast<const u32x2*>(rec_g + o + 4);
                    acc_r = mfma16x16x16(gh, a_hi[s], acc_r);
                    acc_r = mfma16x16x16(gh, a_lo[s], acc_r);
                    acc_r = mfma16x16x16(gl, a_hi[s], acc_r);
                }
            }
            // Lane holds dA[token q][ranks 16 rb + 4 g .. +3]: rotate back.
            if (live) {
                const int rank0 = 16 * rb + 4 * g;
                const u32x2 ph = *reinterpret_cast<const u32x2*>(phrow + rank0 / 2);
                float grad[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    grad[i] = acc_d[rb][i] + acc_r[i];
                }
                u32x2 packed;
#pragma unroll
                for (int p = 0; p < 2; ++p) {
                    const float cosine = f16_lo(ph[p]);
                    const float sine = f16_hi(ph[p]);
                    const float even = grad[2 * p] * cosine + grad[2 * p + 1] * sine;
                    const float odd = grad[2 * p + 1] * cosine - grad[2 * p] * sine;
                    packed[p] = pack_bf16(even, odd);
                }
                *reinterpret_cast<u32x2*>(out_row + h * R + rank0) = packed;
            }
        }
    }
    // <dY, C> of this wave's tokens.
    for (int offset = 32; offset > 0; offset >>= 1) {
        dot += __shfl_xor(dot, offset);
    }
    if (lane == 0) {
        a.dot_part[system * a.chunks + chunk] = dot;
    }
}

// Token map with the system's records held in registers for the whole chunk
// (head_dim = 16 D16 and records of at most 112 VGPRs, (3 R d + R^2) / 64):
// the loop streams only token rows, with each 16-token step's inputs read
// one step before it computes.  A step's output is staged in the wave's LDS
// tile and written as 16-byte pieces of each token's dR and dC runs.  The MFMA chains and the <dY, C> order are those
// of bwd_apply_kernel, so the two kernels agree bitwise.
template <int R, int D16>
struct BwdTokenInputs {
    static constexpr bool kRK32 = (R % 32) == 0;
    static constexpr bool kDK32 = (D16 % 2) == 0;
    using RR = RecordShape<kRK32>;
    using RD = RecordShape<kDK32>;
    static constexpr int kRankSteps = R / RR::kWidth;
    static constexpr int kFeatSteps = kDK32 ? D16 / 2 : D16;
    using RankOp = typename std::conditional<kRK32, u32x4, u32x2>::type;
    using FeatOp = typename std::conditional<kDK32, u32x4, u32x2>::type;
    RankOp rel[kRankSteps];
    RankOp ph[kRankSteps];
    FeatOp y[kFeatSteps];
    FeatOp c[kFeatSteps];

    // Lane (g, q) reads the runs of its token that the MFMA B operand takes;
    // a token past the chunk reads a valid row and keeps zeros.
    __device__ __forceinline__ void load(const uint16_t* rel_row, const uint16_t* content_row,
                                         const uint16_t* grad_row, const uint32_t* phase_row,
                                         int g, bool live) {
#pragma unroll
        for (int s = 0; s < kRankSteps; ++s) {
            const int first = RR::kWidth * s + RR::kPerLane * g;
            const RankOp r = *reinterpret_cast<const RankOp*>(rel_row + first);
            ph[s] = *reinterpret_cast<const RankOp*>(phase_row + first / 2);
            rel[s] = live ? r : RankOp{};
        }
#pragma unroll
        for (int s = 0; s < kFeatSteps; ++s) {
            const int first = RD::kWidth * s + RD::kPerLane * g;
            const FeatOp yv = *reinterpret_cast<const FeatOp*>(grad_row + first);
            const FeatOp cv = *reinterpret_cast<const FeatOp*>(content_row + first);
            y[s] = live ? yv : FeatOp{};
            c[s] = live ? cv : FeatOp{};
        }
    }
};

template <int R, int D16>
__global__ __launch_bounds__(256) void bwd_apply_resident_kernel(BwdApplyArgs a) {
    using In = BwdTokenInputs<R, D16>;
    using RR = typename In::RR;
    using RD = typename In::RD;
    using RankOp = typename In::RankOp;
    using FeatOp = typename In::FeatOp;
    constexpr int RBLK = R / 16;
    constexpr int RSTEPS = In::kRankSteps;
    constexpr int DSTEPS = In::kFeatSteps;
    constexpr int D = 16 * D16;
    constexpr int PAIRS = R / 2;
    // Output tile of a step, per wave: 16 tokens x [dR (R) | dC (D)] in BF16.
    constexpr int OP = R + D + 8;                     // row pitch (bf16)
    constexpr int kRowChunks = (R + D) / 8;           // 16-byte pieces per token
    constexpr int kStorePasses = (16 * kRowChunks + 63) / 64;
    __shared__ __attribute__((aligned(16))) uint16_t s_out[4][16 * OP];
    const int lane = threadIdx.x & 63;
    uint16_t* out_tile = s_out[threadIdx.x >> 6];
    const int64_t wave = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
    if (wave >= a.total_waves) {
        return;
    }
    int64_t rest = wave;
    const int64_t h = rest % a.heads;
    rest /= a.heads;
    const int64_t chunk = rest % a.chunks;
    const int64_t b = rest / a.chunks;
    const int q = lane & 15;
    const int g = lane >> 4;
    const int64_t system = b * a.heads + h;
    const float eta = bounded_complement(a.eta_raw[h]);
    const uint16_t* rec = a.records + system * a.record_stride;

    // Records: dA^T = M dY + E C + G A (rank row blocks), dC^T = F A.
    FeatOp m_hi[RBLK][DSTEPS], m_lo[RBLK][DSTEPS], e_hi[RBLK][DSTEPS], e_lo[RBLK][DSTEPS];
    RankOp g_hi[RBLK][RSTEPS], g_lo[RBLK][RSTEPS], f_hi[D16][RSTEPS], f_lo[D16][RSTEPS];
#pragma unroll
    for (int rb = 0; rb < RBLK; ++rb) {
#pragma unroll
        for (int s = 0; s < DSTEPS; ++s) {
            const int64_t o = ((rb * DSTEPS + s) * 64 + lane) * RD::kLaneHalfs;
            m_hi[rb][s] = *reinterpret_cast<const FeatOp*>(rec + a.off_m + o);
            m_lo[rb][s] = *reinterpret_cast<const FeatOp*>(rec + a.off_m + o + RD::kPerLane);
            e_hi[rb][s] = *reinterpret_cast<const FeatOp*>(rec + a.off_e + o);
            e_lo[rb][s] = *reinterpret_cast<const FeatOp*>(rec + a.off_e + o + RD::kPerLane);
        }
#pragma unroll
        for (int s = 0; s < RSTEPS; ++s) {
            const int64_t o = ((rb * RSTEPS + s) * 64 + lane) * RR::kLaneHalfs;
            g_hi[rb][s] = *reinterpret_cast<const RankOp*>(rec + a.off_g + o);
            g_lo[rb][s] = *reinterpret_cast<const RankOp*>(rec + a.off_g + o + RR::kPerLane);
        }
    }
#pragma unroll
    for (int fb = 0; fb < D16; ++fb) {
#pragma unroll
        for (int s = 0; s < RSTEPS; ++s) {
            const int64_t o = ((fb * RSTEPS + s) * 64 + lane) * RR::kLaneHalfs;
            f_hi[fb][s] = *reinterpret_cast<const RankOp*>(rec + a.off_f + o);
            f_lo[fb][s] = *reinterpret_cast<const RankOp*>(rec + a.off_f + o + RR::kPerLane);
        }
    }

    const int64_t begin = chunk * a.chunk_tokens;
    const int64_t end = begin + a.chunk_tokens < a.length ? begin + a.chunk_tokens : a.length;
    const uint16_t* proj = a.projected + b * a.length * a.width;
    const uint16_t* grad = a.grad_output + b * a.length * a.grad_stride + h * D;
    const uint32_t* phase = a.phases + b * a.phase_batch_stride;
    uint16_t* gout = a.grad_projected + b * a.length * a.width;
    const int64_t rel_off = h * R;
    const int64_t content_off = a.heads * R + h * D;
    auto fetch = [&](In& in, int64_t t0) {
        const int64_t token = t0 + q;
        const bool live = token < end;
        const int64_t safe = live ? token : begin;
        const uint16_t* prow = proj + safe * a.width;
        in.load(prow + rel_off, prow + content_off, grad + safe * a.grad_stride, phase + safe * PAIRS,
                g, live);
    };

    float dot = 0.0f;
    // Column sums of grad_projected over this wave's tokens, from the staged
    // output tiles: lane j holds columns 2 j, 2 j + 1 of [dR | dC].
    constexpr int kPairColumns = (R + D) / 2;
    static_assert(kPairColumns <= 64, "one column pair per lane");
    float col_even = 0.0f;
    float col_odd = 0.0f;
    // One 16-token step from its staged inputs.
    auto compute = [&](const In& cur, int64_t t0) {
        const int64_t token = t0 + q;
        const bool live = token < end;
        const int64_t safe = live ? token : begin;

        RankOp a_hi[RSTEPS];
        RankOp a_lo[RSTEPS];
#pragma unroll
        for (int s = 0; s < RSTEPS; ++s) {
#pragma unroll
            for (int p = 0; p < RR::kPerLane / 2; ++p) {
                float e, o;
                rotate_pair(cur.rel[s][p], cur.ph[s][p], e, o);
                uint32_t hi, lo;
                split_bf16(e, o, hi, lo);
                a_hi[s][p] = hi;
                a_lo[s][p] = lo;
            }
        }
#pragma unroll
        for (int s = 0; s < DSTEPS; ++s) {
#pragma unroll
            for (int p = 0; p < RD::kPerLane / 2; ++p) {
                dot = fmaf(bf16_lo(cur.y[s][p]), bf16_lo(cur.c[s][p]), dot);
                dot = fmaf(bf16_hi(cur.y[s][p]), bf16_hi(cur.c[s][p]), dot);
            }
        }

        // dA^T blocks: feature-K chain (dY, C) and rank-K chain (A) kept apart.
#pragma unroll
        for (int rb = 0; rb < RBLK; ++rb) {
            f32x4 acc_d = {0.0f, 0.0f, 0.0f, 0.0f};
            f32x4 acc_r = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int s = 0; s < DSTEPS; ++s) {
                if constexpr (In::kDK32) {
                    acc_d = mfma16x16x32(m_hi[rb][s], cur.y[s], acc_d);
                    acc_d = mfma16x16x32(m_lo[rb][s], cur.y[s], acc_d);
                    acc_d = mfma16x16x32(e_hi[rb][s], cur.c[s], acc_d);
                    acc_d = mfma16x16x32(e_lo[rb][s], cur.c[s], acc_d);
                } else {
                    acc_d = mfma16x16x16(m_hi[rb][s], cur.y[s], acc_d);
                    acc_d = mfma16x16x16(m_lo[rb][s], cur.y[s], acc_d);
                    acc_d = mfma16x16x16(e_hi[rb][s], cur.c[s], acc_d);
                    acc_d = mfma16x16x16(e_lo[rb][s], cur.c[s], acc_d);
                }
            }
#pragma unroll
            for (int s = 0; s < RSTEPS; ++s) {
                if constexpr (In::kRK32) {
                    acc_r = mfma16x16x32(g_hi[rb][s], a_hi[s], acc_r);
                    acc_r = mfma16x16x32(g_hi[rb][s], a_lo[s], acc_r);
                    acc_r = mfma16x16x32(g_lo[rb][s], a_hi[s], acc_r);
                } else {
                    acc_r = mfma16x16x16(g_hi[rb][s], a_hi[s], acc_r);
                    acc_r = mfma16x16x16(g_hi[rb][s], a_lo[s], acc_r);
                    acc_r = mfma16x16x16(g_lo[rb][s], a_hi[s], acc_r);
                }
            }
            // Lane holds dA[token q][ranks 16 rb + 4 g .. +3]: rotate back
            // into the output tile.
            {
                const int rank0 = 16 * rb + 4 * g;
                u32x2 ph;
                if constexpr (In::kRK32) {
                    ph = *reinterpret_cast<const u32x2*>(phase + safe * PAIRS + rank0 / 2);
                } else {
                    ph = cur.ph[rb];  // the K16 run of step rb is ranks 16 rb + 4 g .. +3
                }
                float gradv[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    gradv[i] = acc_d[i] + acc_r[i];
                }
                u32x2 packed;
#pragma unroll
                for (int p = 0; p < 2; ++p) {
                    const float cosine = f16_lo(ph[p]);
                    const float sine = f16_hi(ph[p]);
                    const float even = gradv[2 * p] * cosine + gradv[2 * p + 1] * sine;
                    const float odd = gradv[2 * p + 1] * cosine - gradv[2 * p] * sine;
                    packed[p] = pack_bf16(even, odd);
                }
                *reinterpret_cast<u32x2*>(&out_tile[q * OP + rank0]) = packed;
            }
        }
        // dC^T blocks: eta dY + (ds / sqrt(n))^T A^T.
#pragma unroll
        for (int fb = 0; fb < D16; ++fb) {
            f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int s = 0; s < RSTEPS; ++s) {
                if constexpr (In::kRK32) {
                    acc = mfma16x16x32(f_hi[fb][s], a_hi[s], acc);
                    acc = mfma16x16x32(f_hi[fb][s], a_lo[s], acc);
                    acc = mfma16x16x32(f_lo[fb][s], a_hi[s], acc);
                } else {
                    acc = mfma16x16x16(f_hi[fb][s], a_hi[s], acc);
                    acc = mfma16x16x16(f_hi[fb][s], a_lo[s], acc);
                    acc = mfma16x16x16(f_lo[fb][s], a_hi[s], acc);
                }
            }
            {
                const int f0 = 16 * fb + 4 * g;
                u32x2 dy;
                if constexpr (In::kDK32) {
                    dy = *reinterpret_cast<const u32x2*>(grad + safe * a.grad_stride + f0);
                } else {
                    dy = cur.y[fb];  // the K16 run of step fb is features 16 fb + 4 g .. +3
                }
                u32x2 packed;
                packed.x = pack_bf16(fmaf(eta, bf16_lo(dy.x), acc[0]), fmaf(eta, bf16_hi(dy.x), acc[1]));
                packed.y = pack_bf16(fmaf(eta, bf16_lo(dy.y), acc[2]), fmaf(eta, bf16_hi(dy.y), acc[3]));
                *reinterpret_cast<u32x2*>(&out_tile[q * OP + R + f0]) = packed;
            }
        }
        // The tile goes out as 16-byte pieces of each token's dR and dC runs
        // (the wave's own LDS region: its reads follow its writes in order).
#pragma unroll
        for (int pass = 0; pass < kStorePasses; ++pass) {
            const int idx = lane + 64 * pass;
            const int row = idx / kRowChunks;
            const int piece = idx - row * kRowChunks;
            if (idx < 16 * kRowChunks && t0 + row < end) {
                const u32x4 v = *reinterpret_cast<const u32x4*>(&out_tile[row * OP + 8 * piece]);
                const int64_t column = 8 * piece < R ? rel_off + 8 * piece : content_off + 8 * piece - R;
                *reinterpret_cast<u32x4*>(gout + (t0 + row) * a.width + column) = v;
            }
        }
        if (a.column_part != nullptr && lane < kPairColumns) {
            float even = 0.0f;
            float odd = 0.0f;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                if (t0 + r < end) {
                    const uint32_t v = *reinterpret_cast<const uint32_t*>(&out_tile[r * OP + 2 * lane]);
                    even += bf16_lo(v);
                    odd += bf16_hi(v);
                }
            }
            col_even += even;
            col_odd += odd;
        }
    };
    // Inputs are read one step ahead, alternating between two stages.
    In s0;
    In s1;
    fetch(s0, begin);
    for (int64_t t0 = begin; t0 < end; t0 += 32) {
        fetch(s1, t0 + 16);
        compute(s0, t0);
        if (t0 + 16 >= end) {
            break;
        }
        fetch(s0, t0 + 32);
        compute(s1, t0 + 16);
    }
    if (a.column_part != nullptr && lane < kPairColumns) {
        const int c = 2 * lane;
        const int64_t column = c < R ? rel_off + c : content_off + c - R;
        float* row = a.column_part + (b * a.chunks + chunk) * a.width + column;
        row[0] = col_even;
        row[1] = col_odd;
    }
    // <dY, C> of this wave's tokens.
    for (int offset = 32; offset > 0; offset >>= 1) {
        dot += __shfl_xor(dot, offset);
    }
    if (lane == 0) {
        a.dot_part[system * a.chunks + chunk] = dot;
    }
}

// Token map from staged row runs (the forward apply's staging): one
// workgroup per (sample, chunk, group of heads), one wave per head with that
// head's records in registers, as in the resident map.  Each 16-token step's
// relation, content and dY runs of the group and its phase rows are loaded
// by every thread as 16-byte pieces two steps ahead and committed to LDS;
// each wave reads its head's operands from LDS in the resident map's layout
// and runs its products (same records, MFMA order, rounding and <dY, C>
// order, so the same bits), and the group's dR and dC rows go out through an
// LDS tile as 16-byte pieces of their two contiguous runs per token.  The
// resident map reads each head's 16-token runs with per-wave loads of 8 to
// 16 bytes per row.
constexpr int kBwdStagedWaves = 4;
constexpr int kBwdStagedCols = 448;     // group relation + content + dY columns, at most
constexpr int kBwdStagedOut = 320;      // group dR + dC columns, at most
constexpr int kBwdStagedRel = 2;        // 16-byte pieces per thread and step, at most:
constexpr int kBwdStagedCon = 1;        //   relation, content, dY and phase pieces,
constexpr int kBwdStagedDy = 1;
constexpr int kBwdStagedPh = 1;
constexpr int kBwdStagedOutPieces = 3;  //   and stored dR / dC pieces

template <int R, int D16>
__global__ __launch_bounds__(kBwdStagedWaves * 64) void bwd_apply_staged_kernel(BwdApplyArgs a, int group_heads) {
    using In = BwdTokenInputs<R, D16>;
    using RR = typename In::RR;
    using RD = typename In::RD;
    using RankOp = typename In::RankOp;
    using FeatOp = typename In::FeatOp;
    constexpr int RBLK = R / 16;
    constexpr int RSTEPS = In::kRankSteps;
    constexpr int DSTEPS = In::kFeatSteps;
    constexpr int D = 16 * D16;
    constexpr int PAIRS = R / 2;
    constexpr int PHP = PAIRS + 4;                       // phase row pitch (u32)
    __shared__ __attribute__((aligned(16))) uint16_t s_rows[2][16 * (kBwdStagedCols + 8)];
    __shared__ __attribute__((aligned(16))) uint32_t s_ph[2][16 * PHP];
    __shared__ __attribute__((aligned(16))) uint16_t s_out[2][16 * (kBwdStagedOut + 8)];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int threads = blockDim.x;
    const int64_t groups = (a.heads + group_heads - 1) / group_heads;
    int64_t rest = blockIdx.x;
    const int64_t group = rest % groups;
    rest /= groups;
    const int64_t chunk = rest % a.chunks;
    const int64_t b = rest / a.chunks;
    const int64_t h0 = group * group_heads;
    const int hg = static_cast<int>(group_heads < a.heads - h0 ? group_heads : a.heads - h0);
    const int unit = wave;
    const bool active = unit < hg;
    const int64_t h = h0 + (active ? unit : 0);
    const int64_t begin = chunk * a.chunk_tokens;
    const int64_t end = begin + a.chunk_tokens < a.length ? begin + a.chunk_tokens : a.length;
    if (begin >= end) {
        return;   // uniform over the workgroup
    }
    const int q = lane & 15;
    const int g = lane >> 4;
    const int64_t system = b * a.heads + h;
    const float eta = bounded_complement(a.eta_raw[h]);
    const uint16_t* rec = a.records + system * a.record_stride;

    // Records: dA^T = M dY + E C + G A (rank row blocks), dC^T = F A.
    FeatOp m_hi[RBLK][DSTEPS], m_lo[RBLK][DSTEPS], e_hi[RBLK][DSTEPS], e_lo[RBLK][DSTEPS];
    RankOp g_hi[RBLK][RSTEPS], g_lo[RBLK][RSTEPS], f_hi[D16][RSTEPS], f_lo[D16][RSTEPS];
#pragma unroll
    for (int rb = 0; rb < RBLK; ++rb) {
#pragma unroll
        for (int s = 0; s < DSTEPS; ++s) {
            const int64_t o = ((rb * DSTEPS + s) * 64 + lane) * RD::kLaneHalfs;
            m_hi[rb][s] = *reinterpret_cast<const FeatOp*>(rec + a.off_m + o);
            m_lo[rb][s] = *reinterpret_cast<const FeatOp*>(rec + a.off_m + o + RD::kPerLane);
            e_hi[rb][s] = *reinterpret_cast<const FeatOp*>(rec + a.off_e + o);
            e_lo[rb][s] = *reinterpret_cast<const FeatOp*>(rec + a.off_e + o + RD::kPerLane);
        }
#pragma unroll
        for (int s = 0; s < RSTEPS; ++s) {
            const int64_t o = ((rb * RSTEPS + s) * 64 + lane) * RR::kLaneHalfs;
            g_hi[rb][s] = *reinterpret_cast<const RankOp*>(rec + a.off_g + o);
            g_lo[rb][s] = *reinterpret_cast<const RankOp*>(rec + a.off_g + o + RR::kPerLane);
        }
    }
#pragma unroll
    for (int fb = 0; fb < D16; ++fb) {
#pragma unroll
        for (int s = 0; s < RSTEPS; ++s) {
            const int64_t o = ((fb * RSTEPS + s) * 64 + lane) * RR::kLaneHalfs;
            f_hi[fb][s] = *reinterpret_cast<const RankOp*>(rec + a.off_f + o);
            f_lo[fb][s] = *reinterpret_cast<const RankOp*>(rec + a.off_f + o + RR::kPerLane);
        }
    }

    // Row layout of a staged step: [relation runs | content runs | dY runs]
    // of the group's heads, and the output tile's rows [dR runs | dC runs].
    const int rel_pieces = hg * R / 8;
    const int con_pieces = hg * D / 8;
    const int pitch = 8 * (rel_pieces + 2 * con_pieces) + 8;
    const int out_pieces = rel_pieces + con_pieces;
    const int out_pitch = 8 * out_pieces + 8;
    const int con_col = 8 * rel_pieces;
    const int dy_col = con_col + 8 * con_pieces;
    uint32_t rel_off[kBwdStagedRel], con_off[kBwdStagedCon], dy_off[kBwdStagedDy], ph_off[kBwdStagedPh];
    int rel_lds[kBwdStagedRel], con_lds[kBwdStagedCon], dy_lds[kBwdStagedDy], ph_lds[kBwdStagedPh];
#pragma unroll
    for (int i = 0; i < kBwdStagedRel; ++i) {
        const int piece = tid + i * threads;
        const int row = piece / rel_pieces;
        const int c = piece - row * rel_pieces;
        const bool live = piece < 16 * rel_pieces;
        rel_off[i] = live ? 2u * static_cast<uint32_t>(row * a.width + 8 * c) : kOutOfRange;
        rel_lds[i] = live ? row * pitch + 8 * c : -1;
    }
#pragma unroll
    for (int i = 0; i < kBwdStagedCon; ++i) {
        const int piece = tid + i * threads;
        const int row = piece / con_pieces;
        const int c = piece - row * con_pieces;
        const bool live = piece < 16 * con_pieces;
        con_off[i] = live ? 2u * static_cast<uint32_t>(row * a.width + 8 * c) : kOutOfRange;
        con_lds[i] = live ? row * pitch + con_col + 8 * c : -1;
    }
#pragma unroll
    for (int i = 0; i < kBwdStagedDy; ++i) {
        const int piece = tid + i * threads;
        const int row = piece / con_pieces;
        const int c = piece - row * con_pieces;
        const bool live = piece < 16 * con_pieces;
        dy_off[i] = live ? 2u * static_cast<uint32_t>(row * a.grad_stride + 8 * c) : kOutOfRange;
        dy_lds[i] = live ? row * pitch + dy_col + 8 * c : -1;
    }
#pragma unroll
    for (int i = 0; i < kBwdStagedPh; ++i) {
        const int piece = tid + i * threads;
        const int row = piece / (PAIRS / 4);
        const int c = piece - row * (PAIRS / 4);
        const bool live = piece < 16 * (PAIRS / 4);
        ph_off[i] = live ? 16u * static_cast<uint32_t>(piece) : kOutOfRange;
        ph_lds[i] = live ? row * PHP + 4 * c : -1;
    }
    struct Stage {
        u32x4 rel[kBwdStagedRel];
        u32x4 con[kBwdStagedCon];
        u32x4 dy[kBwdStagedDy];
        u32x4 ph[kBwdStagedPh];
    };
    auto load = [&](Stage& st, int64_t t0) {
        const int64_t rows = end - t0;
        const uint16_t* row0 = a.projected + (b * a.length + t0) * a.width;
        const BufferRsrc rel = make_buffer(row0 + h0 * R, 2 * rows * a.width);
        const BufferRsrc con = make_buffer(row0 + a.heads * R + h0 * D, 2 * rows * a.width);
        const BufferRsrc dy = make_buffer(a.grad_output + (b * a.length + t0) * a.grad_stride + h0 * D,
                                          2 * rows * a.grad_stride);
        const BufferRsrc ph = make_buffer(a.phases + b * a.phase_batch_stride + t0 * PAIRS, 4 * rows * PAIRS);
#pragma unroll
        for (int i = 0; i < kBwdStagedRel; ++i) {
            st.rel[i] = buffer_load16_stream(rel, rel_off[i]);
        }
#pragma unroll
        for (int i = 0; i < kBwdStagedCon; ++i) {
            st.con[i] = buffer_load16_stream(con, con_off[i]);
        }
#pragma unroll
        for (int i = 0; i < kBwdStagedDy; ++i) {
            st.dy[i] = buffer_load16_stream(dy, dy_off[i]);
        }
#pragma unroll
        for (int i = 0; i < kBwdStagedPh; ++i) {
            st.ph[i] = buffer_load16(ph, ph_off[i]);
        }
    };
    auto commit = [&](const Stage& st, int buf) {
#pragma unroll
        for (int i = 0; i < kBwdStagedRel; ++i) {
            if (rel_lds[i] >= 0) {
                *reinterpret_cast<u32x4*>(&s_rows[buf][rel_lds[i]]) = st.rel[i];
            }
        }
#pragma unroll
        for (int i = 0; i < kBwdStagedCon; ++i) {
            if (con_lds[i] >= 0) {
                *reinterpret_cast<u32x4*>(&s_rows[buf][con_lds[i]]) = st.con[i];
            }
        }
#pragma unroll
        for (int i = 0; i < kBwdStagedDy; ++i) {
            if (dy_lds[i] >= 0) {
                *reinterpret_cast<u32x4*>(&s_rows[buf][dy_lds[i]]) = st.dy[i];
            }
        }
#pragma unroll
        for (int i = 0; i < kBwdStagedPh; ++i) {
            if (ph_lds[i] >= 0) {
                *reinterpret_cast<u32x4*>(&s_ph[buf][ph_lds[i]]) = st.ph[i];
            }
        }
    };
    // Output pieces of this thread: row and column of the group's runs.
    uint32_t out_off[kBwdStagedOutPieces];
    int out_lds[kBwdStagedOutPieces];
#pragma unroll
    for (int i = 0; i < kBwdStagedOutPieces; ++i) {
        const int piece = tid + i * threads;
        const bool live = piece < 16 * out_pieces;
        const int row = piece / out_pieces;
        const int c = piece - row * out_pieces;
        const int64_t column = c < rel_pieces ? h0 * R + 8 * c : a.heads * R + h0 * D + 8 * (c - rel_pieces);
        out_off[i] = live ? 2u * static_cast<uint32_t>(row * a.width + column) : kOutOfRange;
        out_lds[i] = live ? row * out_pitch + 8 * c : 0;
    }

    float dot = 0.0f;
    // Column sums of this head's [dR | dC] columns over the chunk, from the
    // output tiles: lane j holds columns 2 j, 2 j + 1.
    constexpr int kPairColumns = (R + D) / 2;
    static_assert(kPairColumns <= 64, "one column pair per lane");
    float col_even = 0.0f;
    float col_odd = 0.0f;
    const int rel_col = unit * R;
    const int my_con = con_col + unit * D;
    const int my_dy = dy_col + unit * D;
    auto compute = [&](int buf, int obuf, int64_t t0) {
        if (!active) {
            return;
        }
        const uint16_t* prow = &s_rows[buf][q * pitch];
        const uint32_t* phrow = &s_ph[buf][q * PHP];
        uint16_t* orow = &s_out[obuf][q * out_pitch];
        In cur;
#pragma unroll
        for (int s = 0; s < RSTEPS; ++s) {
            const int first = RR::kWidth * s + RR::kPerLane * g;
            cur.rel[s] = *reinterpret_cast<const RankOp*>(prow + rel_col + first);
            cur.ph[s] = *reinterpret_cast<const RankOp*>(phrow + first / 2);
        }
#pragma unroll
        for (int s = 0; s < DSTEPS; ++s) {
            const int first = RD::kWidth * s + RD::kPerLane * g;
            cur.y[s] = *reinterpret_cast<const FeatOp*>(prow + my_dy + first);
            cur.c[s] = *reinterpret_cast<const FeatOp*>(prow + my_con + first);
        }
        RankOp a_hi[RSTEPS];
        RankOp a_lo[RSTEPS];
#pragma unroll
        for (int s = 0; s < RSTEPS; ++s) {
#pragma unroll
            for (int pp = 0; pp < RR::kPerLane / 2; ++pp) {
                float e, o;
                rotate_pair(cur.rel[s][pp], cur.ph[s][pp], e, o);
                uint32_t hi, lo;
                split_bf16(e, o, hi, lo);
                a_hi[s][pp] = hi;
                a_lo[s][pp] = lo;
            }
        }
#pragma unroll
        for (int s = 0; s < DSTEPS; ++s) {
#pragma unroll
            for (int pp = 0; pp < RD::kPerLane / 2; ++pp) {
                dot = fmaf(bf16_lo(cur.y[s][pp]), bf16_lo(cur.c[s][pp]), dot);
                dot = fmaf(bf16_hi(cur.y[s][pp]), bf16_hi(cur.c[s][pp]), dot);
            }
        }
#pragma unroll
        for (int rb = 0; rb < RBLK; ++rb) {
            f32x4 acc_d = {0.0f, 0.0f, 0.0f, 0.0f};
            f32x4 acc_r = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int s = 0; s < DSTEPS; ++s) {
                if constexpr (In::kDK32) {
                    acc_d = mfma16x16x32(m_hi[rb][s], cur.y[s], acc_d);
                    acc_d = mfma16x16x32(m_lo[rb][s], cur.y[s], acc_d);
                    acc_d = mfma16x16x32(e_hi[rb][s], cur.c[s], acc_d);
                    acc_d = mfma16x16x32(e_lo[rb][s], cur.c[s], acc_d);
                } else {
                    acc_d = mfma16x16x16(m_hi[rb][s], cur.y[s], acc_d);
                    acc_d = mfma16x16x16(m_lo[rb][s], cur.y[s], acc_d);
                    acc_d = mfma16x16x16(e_hi[rb][s], cur.c[s], acc_d);
                    acc_d = mfma16x16x16(e_lo[rb][s], cur.c[s], acc_d);
                }
            }
#pragma unroll
            for (int s = 0; s < RSTEPS; ++s) {
                if constexpr (In::kRK32) {
                    acc_r = mfma16x16x32(g_hi[rb][s], a_hi[s], acc_r);
                    acc_r = mfma16x16x32(g_hi[rb][s], a_lo[s], acc_r);
                    acc_r = mfma16x16x32(g_lo[rb][s], a_hi[s], acc_r);
                } else {
                    acc_r = mfma16x16x16(g_hi[rb][s], a_hi[s], acc_r);
                    acc_r = mfma16x16x16(g_hi[rb][s], a_lo[s], acc_r);
                    acc_r = mfma16x16x16(g_lo[rb][s], a_hi[s], acc_r);
                }
            }
            // Lane holds dA[token q][ranks 16 rb + 4 g .. +3]: rotate back.
            const int rank0 = 16 * rb + 4 * g;
            const u32x2 ph = *reinterpret_cast<const u32x2*>(phrow + rank0 / 2);
            float gradv[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                gradv[i] = acc_d[i] + acc_r[i];
            }
            u32x2 packed;
#pragma unroll
            for (int pp = 0; pp < 2; ++pp) {
                const float cosine = f16_lo(ph[pp]);
                const float sine = f16_hi(ph[pp]);
                const float even = gradv[2 * pp] * cosine + gradv[2 * pp + 1] * sine;
                const float odd = gradv[2 * pp + 1] * cosine - gradv[2 * pp] * sine;
                packed[pp] = pack_bf16(even, odd);
            }
            *reinterpret_cast<u32x2*>(orow + rel_col + rank0) = packed;
        }
        // dC^T blocks: eta dY + (ds / sqrt(n))^T A^T.
#pragma unroll
        for (int fb = 0; fb < D16; ++fb) {
            f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int s = 0; s < RSTEPS; ++s) {
                if constexpr (In::kRK32) {
                    acc = mfma16x16x32(f_hi[fb][s], a_hi[s], acc);
                    acc = mfma16x16x32(f_hi[fb][s], a_lo[s], acc);
                    acc = mfma16x16x32(f_lo[fb][s], a_hi[s], acc);
                } else {
                    acc = mfma16x16x16(f_hi[fb][s], a_hi[s], acc);
                    acc = mfma16x16x16(f_hi[fb][s], a_lo[s], acc);
                    acc = mfma16x16x16(f_lo[fb][s], a_hi[s], acc);
                }
            }
            const int f0 = 16 * fb + 4 * g;
            const u32x2 dyv = *reinterpret_cast<const u32x2*>(prow + my_dy + f0);
            u32x2 packed;
            packed.x = pack_bf16(fmaf(eta, bf16_lo(dyv.x), acc[0]), fmaf(eta, bf16_hi(dyv.x), acc[1]));
            packed.y = pack_bf16(fmaf(eta, bf16_lo(dyv.y), acc[2]), fmaf(eta, bf16_hi(dyv.y), acc[3]));
            *reinterpret_cast<u32x2*>(orow + con_col + unit * D + f0) = packed;
        }
        if (a.column_part != nullptr && lane < kPairColumns) {
            // The wave's own tile rows: its reads follow its writes in order.
            const int c = 2 * lane;
            const int col = c < R ? rel_col + c : con_col + unit * D + (c - R);
            float even = 0.0f;
            float odd = 0.0f;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                if (t0 + r < end) {
                    const uint32_t v = *reinterpret_cast<const uint32_t*>(&s_out[obuf][r * out_pitch + col]);
                    even += bf16_lo(v);
                    odd += bf16_hi(v);
                }
            }
            col_even += even;
            col_odd += odd;
        }
    };
    auto store = [&](int obuf, int64_t t0) {
        const BufferRsrc out = make_buffer(a.grad_projected + (b * a.length + t0) * a.width,
                                           2 * (end - t0) * a.width);
#pragma unroll
        for (int i = 0; i < kBwdStagedOutPieces; ++i) {
            buffer_store16(*reinterpret_cast<const u32x4*>(&s_out[obuf][out_lds[i]]), out, out_off[i]);
        }
    };

    // Two register stages (loads two steps ahead), two row buffers and two
    // output tiles: one barrier per step.  Steps past the chunk load zeros
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
        compute(0, 0, t0);
        commit(stage_b, 1);
        __syncthreads();
        store(0, t0);
        load(stage_b, t0 + 48);
        compute(1, 1, t0 + 16);
        commit(stage_a, 0);
        __syncthreads();
        store(1, t0 + 16);
    }
    if (active) {
        if (a.column_part != nullptr && lane < kPairColumns) {
            const int c = 2 * lane;
            const int64_t column = c < R ? h * R + c : a.heads * R + h * D + c - R;
            float* row = a.column_part + (b * a.chunks + chunk) * a.width + column;
            row[0] = col_even;
            row[1] = col_odd;
        }
        for (int offset = 32; offset > 0; offset >>= 1) {
            dot += __shfl_xor(dot, offset);
        }
        if (lane == 0) {
            a.dot_part[system * a.chunks + chunk] = dot;
        }
    }
}

// ---------------------------------------------------------------------------
// Parameter gradients.  One thread per element of dTheta0 and dW sums the
// batch in ascending order (sixteen samples' loads issued together); one wave
// per head sums deta and <dY, C> over every (sample, chunk), lane-strided and
// then by a fixed butterfly.
__global__ __launch_bounds__(256) void param_reduce_kernel(ParamReduceArgs a) {
    const int64_t rr = a.rank * a.rank;
    const int64_t dr = a.head_dim * a.rank;
    const int64_t elements = a.heads * (rr + dr);
    const int64_t element_blocks = (elements + 255) / 256;
    if (blockIdx.x >= element_blocks) {
        const int64_t h = blockIdx.x - element_blocks;
        const int lane = threadIdx.x;
        if (lane >= 64) {
            return;
        }
        float acc = 0.0f;
        for (int64_t b = lane; b < a.batch; b += 64) {
            acc += a.deta_part[b * a.heads + h];
        }
        const int64_t dots = a.batch * a.chunks;
        for (int64_t i = lane; i < dots; i += 64) {
            const int64_t b = i / a.chunks;
            acc += a.dot_part[(b * a.heads + h) * a.chunks + (i - b * a.chunks)];
        }
        for (int offset = 32; offset > 0; offset >>= 1) {
            acc += __shfl_xor(acc, offset);
        }
        if (lane == 0) {
            a.grad_eta[h] = acc * bounded_complement_derivative(a.eta_raw[h]);
        }
        return;
    }
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (idx >= elements) {
        return;
    }
    const int64_t h = idx / (rr + dr);
    const int64_t e = idx - h * (rr + dr);
    const float* source;
    int64_t stride;
    if (e < rr) {
        source = a.dtheta_part + h * rr + e;
        stride = a.heads * rr;
    } else {
        source = a.ddrive_part + h * dr + (e - rr);
        stride = a.heads * dr;
    }
    constexpr int kBatchLoads = 16;
    float acc = 0.0f;
    for (int64_t b0 = 0; b0 < a.batch; b0 += kBatchLoads) {
        float v[kBatchLoads];
#pragma unroll
        for (int u = 0; u < kBatchLoads; ++u) {
            const int64_t b = b0 + u < a.batch ? b0 + u : a.batch - 1;
            v[u] = source[b * stride];
        }
#pragma unroll
        for (int u = 0; u < kBatchLoads; ++u) {
            if (b0 + u < a.batch) {
                acc += v[u];
            }
        }
    }
    if (e < rr) {
        a.grad_base[h * rr + e] = acc;
    } else {
        a.grad_drive[h * dr + (e - rr)] = acc;
    }
}

// ---------------------------------------------------------------------------
// Launchers.
int64_t bwd_record_layout(int64_t rank, int64_t head_dim, int64_t* off_m, int64_t* off_e,
                          int64_t* off_g, int64_t* off_f, int* feature_k32) {
    const bool dk32 = head_dim % 32 == 0;
    const bool rk32 = rank % 32 == 0;
    const int64_t feature = dk32 ? record_halfs<true>(rank, head_dim) : record_halfs<false>(rank, head_dim);
    const int64_t gram = rk32 ? record_halfs<true>(rank, rank) : record_halfs<false>(rank, rank);
    const int64_t content = rk32 ? record_halfs<true>(head_dim, rank) : record_halfs<false>(head_dim, rank);
    *off_m = 0;
    *off_e = feature;
    *off_g = 2 * feature;
    *off_f = 2 * feature + gram;
    *feature_k32 = dk32 ? 1 : 0;
    return 2 * feature + gram + content;
}

hipError_t launch_bwd_solve(int rank, const BwdSolveArgs& a, int64_t systems, hipStream_t stream) {
    const dim3 grid(static_cast<unsigned>(systems));
    if (a.head_dim > kBwdMaxHeadDim) {
        switch (rank) {
            case 16: bwd_solve_wide_kernel<16><<<grid, kBwdThreads, 0, stream>>>(a); break;
            case 32: bwd_solve_wide_kernel<32><<<grid, kBwdThreads, 0, stream>>>(a); break;
            case 48: bwd_solve_wide_kernel<48><<<grid, kBwdThreads, 0, stream>>>(a); break;
            default: bwd_solve_wide_kernel<64><<<grid, kBwdThreads, 0, stream>>>(a); break;
        }
        return hipGetLastError();
    }
    const bool small = a.head_dim <= 32;
    switch (rank) {
        case 16: small ? bwd_solve_kernel<16, 32><<<grid, kBwdThreads, 0, stream>>>(a)
                       : bwd_solve_kernel<16, kBwdMaxHeadDim><<<grid, kBwdThreads, 0, stream>>>(a); break;
        case 32: small ? bwd_solve_kernel<32, 32><<<grid, kBwdThreads, 0, stream>>>(a)
                       : bwd_solve_kernel<32, kBwdMaxHeadDim><<<grid, kBwdThreads, 0, stream>>>(a); break;
        case 48: small ? bwd_solve_kernel<48, 32><<<grid, kBwdThreads, 0, stream>>>(a)
                       : bwd_solve_kernel<48, kBwdMaxHeadDim><<<grid, kBwdThreads, 0, stream>>>(a); break;
        default: small ? bwd_solve_kernel<64, 32><<<grid, kBwdThreads, 0, stream>>>(a)
                       : bwd_solve_kernel<64, kBwdMaxHeadDim><<<grid, kBwdThreads, 0, stream>>>(a); break;
    }
    return hipGetLastError();
}

template <int R>
static hipError_t launch_bwd_apply_r(const BwdApplyArgs& a, bool dk32, bool vec, hipStream_t stream) {
    const dim3 grid(static_cast<unsigned>((a.total_waves + 3) / 4));
    if (dk32) {
        if (vec) {
            bwd_apply_kernel<R, true, true><<<grid, 256, 0, stream>>>(a);
        } else {
            bwd_apply_kernel<R, true, false><<<grid, 256, 0, stream>>>(a);
        }
    } else {
        if (vec) {
            bwd_apply_kernel<R, false, true><<<grid, 256, 0, stream>>>(a);
        } else {
            bwd_apply_kernel<R, false, false><<<grid, 256, 0, stream>>>(a);
        }
    }
    return hipGetLastError();
}

template <int R, int D16>
static hipError_t launch_bwd_apply_resident(const BwdApplyArgs& a, hipStream_t stream) {
    const dim3 grid(static_cast<unsigned>((a.total_waves + 3) / 4));
    bwd_apply_resident_kernel<R, D16><<<grid, 256, 0, stream>>>(a);
    return hipGetLastError();
}

// Largest head_dim / 16 whose records stay resident ((3 R d + R^2) / 64 <= 112 VGPRs).
static int resident_max_d16(int rank) {
    return rank <= 32 ? 4 : (rank == 48 ? 2 : 1);
}

bool bwd_apply_resident(int rank, int64_t head_dim, bool vec) {
    const int64_t d16 = head_dim / 16;
    return vec && head_dim % 16 == 0 && d16 >= 1 && d16 <= resident_max_d16(rank);
}

// Heads per workgroup of the staged token map (0 when it does not apply):
// up to four, so that a step's runs and output tile fit the staging limits,
// and at most half the heads, so that a sample has at least two groups.
static int bwd_staged_group_heads(int rank, const BwdApplyArgs& a) {
    const int64_t d = a.head_dim;
    int64_t group = kBwdStagedWaves < a.heads ? kBwdStagedWaves : a.heads;
    while (group > 1 && (group * (rank + 2 * d) > kBwdStagedCols || group * (rank + d) > kBwdStagedOut)) {
        --group;
    }
    if (group * 2 > a.heads && a.heads > 1) group = (a.heads + 1) / 2;
    const int64_t threads = 64 * kBwdStagedWaves;
    if (group * (rank + 2 * d) > kBwdStagedCols || group * (rank + d) > kBwdStagedOut ||
        16 * group * rank / 8 > kBwdStagedRel * threads || 16 * group * d / 8 > kBwdStagedCon * threads ||
        16 * (rank / 2) / 4 > kBwdStagedPh * threads ||
        16 * group * (rank + d) / 8 > kBwdStagedOutPieces * threads || a.chunk_tokens % 16 != 0) {
        return 0;
    }
    return static_cast<int>(group);
}

template <int R, int D16>
static hipError_t launch_bwd_apply_token_map(const BwdApplyArgs& a, hipStream_t stream) {
    const int group = bwd_staged_group_heads(R, a);
    if (group > 0) {
        const int64_t groups = (a.heads + group - 1) / group;
        const dim3 grid(static_cast<unsigned>(a.batch * a.chunks * groups));
        bwd_apply_staged_kernel<R, D16><<<grid, kBwdStagedWaves * 64, 0, stream>>>(a, group);
        return hipGetLastError();
    }
    return launch_bwd_apply_resident<R, D16>(a, stream);
}

hipError_t launch_bwd_apply(int rank, const BwdApplyArgs& a, bool dk32, bool vec, hipStream_t stream) {
    const int d16 = static_cast<int>(a.head_dim / 16);
    if (bwd_apply_resident(rank, a.head_dim, vec)) {
        switch (rank * 8 + d16) {
            case 16 * 8 + 1: return launch_bwd_apply_token_map<16, 1>(a, stream);
            case 16 * 8 + 2: return launch_bwd_apply_token_map<16, 2>(a, stream);
            case 16 * 8 + 3: return launch_bwd_apply_token_map<16, 3>(a, stream);
            case 16 * 8 + 4: return launch_bwd_apply_token_map<16, 4>(a, stream);
            case 32 * 8 + 1: return launch_bwd_apply_token_map<32, 1>(a, stream);
            case 32 * 8 + 2: return launch_bwd_apply_token_map<32, 2>(a, stream);
            case 32 * 8 + 3: return launch_bwd_apply_token_map<32, 3>(a, stream);
            case 32 * 8 + 4: return launch_bwd_apply_token_map<32, 4>(a, stream);
            case 48 * 8 + 1: return launch_bwd_apply_token_map<48, 1>(a, stream);
            case 48 * 8 + 2: return launch_bwd_apply_token_map<48, 2>(a, stream);
            default: return launch_bwd_apply_token_map<64, 1>(a, stream);
        }
    }
    switch (rank) {
        case 16: return launch_bwd_apply_r<16>(a, dk32, vec, stream);
        case 32: return launch_bwd_apply_r<32>(a, dk32, vec, stream);
        case 48: return launch_bwd_apply_r<48>(a, dk32, vec, stream);
        default: return launch_bwd_apply_r<64>(a, dk32, vec, stream);
    }
}

hipError_t launch_param_reduce(const ParamReduceArgs& a, hipStream_t stream) {
    const int64_t elements = a.heads * (a.rank * a.rank + a.head_dim * a.rank);
    const dim3 grid(static_cast<unsigned>((elements + 255) / 256 + a.heads));
    param_reduce_kernel<<<grid, 256, 0, stream>>>(a);
    return hipGetLastError();
}

}  // namespace lsso_hip

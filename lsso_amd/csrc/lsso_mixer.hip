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

namespace lsso_hip {

// ---------------------------------------------------------------------------
// Rank layouts.
//
// Reduce: lane q = lane % 16 owns relation pairs [kPairSlots*q, +kPairSlots).
// The MFMA row block `blk` = 2*slot + parity holds rank 2*(kPairSlots*m +
// slot) + parity in row m.  Tokens are the K index of the MFMA, so the rank
// permutation is free; it lets every lane feed the MFMA straight from its
// own contiguous loads.
template <int R>
struct ReduceLayout {
    static constexpr int kPairs = R / 2;
    static constexpr int kPairSlots = (kPairs + 15) / 16;
    static constexpr int kRowBlocks = 2 * kPairSlots;
    static constexpr int kGramBlocks = kRowBlocks * (kRowBlocks + 1) / 2;
    __device__ static constexpr int rank(int blk, int m) {
        return 2 * (kPairSlots * m + blk / 2) + (blk & 1);
    }
    __device__ static constexpr bool valid(int blk, int m) {
        return kPairSlots * m + blk / 2 < kPairs;
    }
};

// Apply: the rank dimension is the MFMA K index.  Ranks that are multiples
// of 32 use K32 steps (16x16x32; lane group g holds ranks base + 8g .. +7),
// the others K16 steps (16x16x16; ranks base + 4g .. +3).  One accumulation
// chain never mixes the two MFMA shapes: a 16x16x32 result consumed as SrcC
// of a 16x16x16 produced wrong accumulators on gfx950 with this toolchain.
// Per lane the M' operand holds, per step, the hi values followed by the lo
// values.
template <int R>
struct ApplyLayout {
    static constexpr bool kWide = (R % 32) == 0;
    static constexpr int kSteps32 = kWide ? R / 32 : 0;
    static constexpr int kSteps16 = kWide ? 0 : R / 16;
    static constexpr int kLaneValues = R / 4;          // per hi or lo part
    static constexpr int kLaneHalfs = 2 * kLaneValues;  // bf16 per lane per block
    __device__ static constexpr int rank32(int s, int g, int i) { return 32 * s + 8 * g + i; }
    __device__ static constexpr int rank16(int s, int g, int i) { return 16 * s + 4 * g + i; }
    // offsets (in bf16) of the hi part of a step inside a lane record
    __device__ static constexpr int offset32(int s) { return 16 * s; }
    __device__ static constexpr int offset16(int s) { return 8 * s; }
};

// ---------------------------------------------------------------------------
// Phase table.
__global__ __launch_bounds__(256) void phase_kernel(PhaseArgs a) {
    const int64_t index = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (index >= a.count) {
        return;
    }
    const int pair = static_cast<int>(index % a.pairs);
    const int64_t position_index = index / a.pairs;
    const float position = a.positions != nullptr
        ? a.positions[position_index]
        : static_cast<float>(position_index) - 0.5f * static_cast<float>(a.length - 1);
    const float angle = position * a.inverse_frequency[pair];
    float sine;
    float cosine;
    sincosf(angle, &sine, &cosine);
    a.phases[index] = pack_f16(cosine, sine);
}

// ---------------------------------------------------------------------------
// Reduce.
template <bool VEC>
__device__ __forceinline__ uint32_t load_pair(const uint16_t* p, bool second_valid) {
    if constexpr (VEC) {
        return *reinterpret_cast<const uint32_t*>(p);
    } else {
        const uint32_t low = p[0];
        const uint32_t high = second_valid ? static_cast<uint32_t>(p[1]) : 0u;
        return low | (high << 16);
    }
}

template <int R, int CPW>
struct ReduceTile {
    static constexpr int PS = ReduceLayout<R>::kPairSlots;
    uint32_t rel[8][PS];
    uint32_t ph[8][PS];
    uint32_t con[8][CPW];
};

template <int R, int CPW, bool VEC>
__device__ __forceinline__ void reduce_load(ReduceTile<R, CPW>& t, const ReduceArgs& a,
                                            int64_t b, int64_t h, int cg, int q, int g,
                                            int64_t t0, int64_t end) {
    using L = ReduceLayout<R>;
    constexpr int PS = L::kPairSlots;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int64_t token = t0 + 8 * g + j;
        const bool live = token < end;
        const uint16_t* row = a.projected + (b * a.length + (live ? token : 0)) * a.width;
        const uint32_t* phase_row = a.phases + b * a.phase_batch_stride +
                                    (live ? token : 0) * L::kPairs;
        if constexpr (VEC && PS == 2) {
            const bool pv = live && (PS * q < L::kPairs);
            u32x2 r = {0u, 0u};
            u32x2 p = {0u, 0u};
            if (pv) {
                r = *reinterpret_cast<const u32x2*>(row + h * R + 2 * PS * q);
                p = *reinterpret_cast<const u32x2*>(phase_row + PS * q);
            }
            t.rel[j][0] = r.x;
            t.rel[j][1] = r.y;
            t.ph[j][0] = p.x;
            t.ph[j][1] = p.y;
        } else {
#pragma unroll
            for (int s = 0; s < PS; ++s) {
                const int pair = PS * q + s;
                const bool pv = live && pair < L::kPairs;
                t.rel[j][s] = pv ? load_pair<VEC>(row + h * R + 2 * pair, true) : 0u;
                t.ph[j][s] = pv ? phase_row[pair] : 0u;
            }
        }
#pragma unroll
        for (int c = 0; c < CPW; ++c) {
            const int64_t feature = 2 * (static_cast<int64_t>(cg) * 16 * CPW + 16 * c + q);
            const bool fv = live && feature < a.head_dim;
            t.con[j][c] = fv ? load_pair<VEC>(row + a.heads * R + h * a.head_dim + feature,
                                              feature + 1 < a.head_dim)
                             : 0u;
        }
    }
}

template <int R, int CPW>
__device__ __forceinline__ void reduce_compute(const ReduceTile<R, CPW>& t, bool do_gram,
                                               f32x4 (&acc_g)[ReduceLayout<R>::kGramBlocks],
                                               f32x4 (&acc_s)[ReduceLayout<R>::kRowBlocks][2 * CPW]) {
    using L = ReduceLayout<R>;
    constexpr int PS = L::kPairSlots;
    constexpr int NRB = L::kRowBlocks;
    u32x4 a_hi[NRB];
    u32x4 a_lo[NRB];
#pragma unroll
    for (int s = 0; s < PS; ++s) {
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
            float x0, y0, x1, y1;
            rotate_pair(t.rel[2 * jj][s], t.ph[2 * jj][s], x0, y0);
            rotate_pair(t.rel[2 * jj + 1][s], t.ph[2 * jj + 1][s], x1, y1);
            uint32_t hi, lo;
            split_bf16(x0, x1, hi, lo);
            a_hi[2 * s][jj] = hi;
            a_lo[2 * s][jj] = lo;
            split_bf16(y0, y1, hi, lo);
            a_hi[2 * s + 1][jj] = hi;
            a_lo[2 * s + 1][jj] = lo;
        }
    }
    u32x4 b_c[2 * CPW];
#pragma unroll
    for (int c = 0; c < CPW; ++c) {
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
            const uint32_t first = t.con[2 * jj][c];
            const uint32_t second = t.con[2 * jj + 1][c];
            b_c[2 * c][jj] = (first & 0xffffu) | (second << 16);
            b_c[2 * c + 1][jj] = (first >> 16) | (second & 0xffff0000u);
        }
    }
    if (do_gram) {
        int ab = 0;
#pragma unroll
        for (int x = 0; x < NRB; ++x) {
#pragma unroll
            for (int y = 0; y <= x; ++y) {
                acc_g[ab] = mfma16x16x32(a_hi[x], a_hi[y], acc_g[ab]);
                acc_g[ab] = mfma16x16x32(a_hi[x], a_lo[y], acc_g[ab]);
                acc_g[ab] = mfma16x16x32(a_lo[x], a_hi[y], acc_g[ab]);
                ++ab;
            }
        }
    }
#pragma unroll
    for (int x = 0; x < NRB; ++x) {
#pragma unroll
        for (int cb = 0; cb < 2 * CPW; ++cb) {
            acc_s[x][cb] = mfma16x16x32(a_hi[x], b_c[cb], acc_s[x][cb]);
            acc_s[x][cb] = mfma16x16x32(a_lo[x], b_c[cb], acc_s[x][cb]);
        }
    }
}

template <int R, int CPW, bool VEC>
__global__ __launch_bounds__(256) void reduce_kernel(ReduceArgs a) {
    using L = ReduceLayout<R>;
    constexpr int NRB = L::kRowBlocks;
    constexpr int NGB = L::kGramBlocks;
    const int lane = threadIdx.x & 63;
    const int64_t wave = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
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
    const bool do_gram = cg == 0;

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

    // D layout of a 16x16 MFMA block: lane holds rows 4g..4g+3 of column q.
    float* part = a.partials + ((b * a.heads + h) * a.chunks + chunk) * a.partial_stride;
    float* part_g = part;
    float* part_s = part + R * R;
    if (do_gram) {
        int ab = 0;
#pragma unroll
        for (int x = 0; x < NRB; ++x) {
#pragma unroll
            for (int y = 0; y <= x; ++y) {
                const bool cv = L::valid(y, q);
                const int col = L::rank(y, q);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int m = 4 * g + i;
                    if (cv && L::valid(x, m)) {
                        const int row = L::rank(x, m);
                        part_g[row * R + col] = acc_g[ab][i];
                        if (x != y) {
                            part_g[col * R + row] = acc_g[ab][i];
                        }
                    }
                }
                ++ab;
            }
        }
    }
#pragma unroll
    for (int x = 0; x < NRB; ++x) {
#pragma unroll
        for (int cb = 0; cb < 2 * CPW; ++cb) {
            const int64_t feature =
                2 * (static_cast<int64_t>(cg) * 16 * CPW + 16 * (cb / 2) + q) + (cb & 1);
            if (feature < a.head_dim) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int m = 4 * g + i;
                    if (L::valid(x, m)) {
                        part_s[L::rank(x, m) * a.head_dim + feature] = acc_s[x][cb][i];
                    }
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Solve: one 64-lane workgroup per (b, h) system.
constexpr int kSolvePanel = 64;

__device__ __forceinline__ void wave_argmax(float& value, int& index) {
#pragma unroll
    for (int offset = 32; offset > 0; offset >>= 1) {
        const float other_value = __shfl_xor(value, offset, 64);
        const int other_index = __shfl_xor(index, offset, 64);
        if (other_value > value || (other_value == value && other_index < index)) {
            value = other_value;
            index = other_index;
        }
    }
}

template <int R>
__global__ __launch_bounds__(64) void solve_kernel(SolveArgs a) {
    using AL = ApplyLayout<R>;
    constexpr int LD = R + 1;
    constexpr int PLD = kSolvePanel + 1;
    constexpr int kBlock = R / 8;  // Theta tile per lane: kBlock x kBlock
    __shared__ float s_chol[R * LD];
    __shared__ float s_lu[R * LD];
    __shared__ float s_theta[R * LD];
    __shared__ float s_panel[R * PLD];
    __shared__ float s_drive[kSolvePanel * LD];
    __shared__ float s_diag[R];
    __shared__ int s_perm[R];

    const int tid = threadIdx.x;
    const int64_t system = blockIdx.x;
    const int64_t b = system / a.heads;
    const int64_t h = system - b * a.heads;
    const int64_t d = a.head_dim;
    const float count = a.valid_counts != nullptr ? a.valid_counts[b] : static_cast<float>(a.length);
    const float root = sqrtf(count);
    const float eta = bounded_complement(a.eta_raw[h]);
    const float* part = a.partials + system * a.chunks * a.partial_stride;

    // G / n + I, summed over token chunks in ascending order.  partial_stride
    // is a multiple of 4 (R is a multiple of 16), so the G block is read as
    // float4 with every chunk's loads of a group in flight together.
    {
        constexpr int kG4 = R * R / 4;
        constexpr int kPer = (kG4 + 63) / 64;
        f32x4 acc[kPer];
#pragma unroll
        for (int p = 0; p < kPer; ++p) {
            acc[p] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
        }
        int64_t ch = 0;
        for (; ch + 4 <= a.chunks; ch += 4) {
            f32x4 v[4][kPer];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
#pragma unroll
                for (int p = 0; p < kPer; ++p) {
                    const int vec = tid + 64 * p;
                    v[u][p] = vec < kG4 ? *reinterpret_cast<const f32x4*>(part + (ch + u) * a.partial_stride + 4 * vec)
                                        : (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
                }
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
#pragma unroll
                for (int p = 0; p < kPer; ++p) {
                    acc[p] += v[u][p];
                }
            }
        }
        for (; ch < a.chunks; ++ch) {
#pragma unroll
            for (int p = 0; p < kPer; ++p) {
                const int vec = tid + 64 * p;
                if (vec < kG4) {
                    acc[p] += *reinterpret_cast<const f32x4*>(part + ch * a.partial_stride + 4 * vec);
                }
            }
        }
#pragma unroll
        for (int p = 0; p < kPer; ++p) {
            const int vec = tid + 64 * p;
            if (vec < kG4) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int idx = 4 * vec + e;
                    const int r = idx / R;
                    const int c = idx - r * R;
                    s_chol[r * LD + c] = acc[p][e] / count + (r == c ? 1.0f : 0.0f);
                }
            }
        }
        for (int idx = tid; idx < R * LD; idx += 64) {
            s_theta[idx] = 0.0f;
        }
    }
    __syncthreads();

    // Cholesky in LDL^T-update form: step k subtracts a_ik a_jk / a_kk from
    // the trailing lower triangle; lane i owns row i, so no step races.
    for (int k = 0; k < R - 1; ++k) {
        const int i = tid;
        if (i > k && i < R) {
            const float f = s_chol[i * LD + k] / s_chol[k * LD + k];
            for (int j = k + 1; j <= i; ++j) {
                s_chol[i * LD + j] -= f * s_chol[j * LD + k];
            }
        }
        __syncthreads();
    }
    if (tid < R) {
        s_diag[tid] = sqrtf(s_chol[tid * LD + tid]);
    }
    __syncthreads();
    for (int idx = tid; idx < R * R; idx += 64) {
        const int r = idx / R;
        const int c = idx - r * R;
        float value = 0.0f;
        if (c < r) {
            value = s_chol[r * LD + c] / s_diag[c];
        } else if (c == r) {
            value = s_diag[r];
        }
        s_chol[r * LD + c] = value;
    }
    __syncthreads();

    // Z = L^-1 S panel by panel (lane = column: S summed over chunks straight
    // into registers, then forward substitution); Theta accumulates Z W_drive
    // from LDS copies of the panel and of W_drive's rows.
    float* zbuf = a.zbuf + system * R * d;
    const float* drive = a.drive + h * d * R;
    const float* part_s = part + R * R;
    for (int64_t c0 = 0; c0 < d; c0 += kSolvePanel) {
        const int64_t width = d - c0 < kSolvePanel ? d - c0 : kSolvePanel;
        if (tid < width) {
            float z[R];
#pragma unroll
            for (int i = 0; i < R; ++i) {
                z[i] = 0.0f;
            }
            for (int64_t ch = 0; ch < a.chunks; ++ch) {
                const float* column = part_s + ch * a.partial_stride + c0 + tid;
#pragma unroll
                for (int i = 0; i < R; ++i) {
                    z[i] += column[i * d];
                }
            }
#pragma unroll
            for (int i = 0; i < R; ++i) {
                float value = z[i] / root;
#pragma unroll
                for (int k = 0; k < i; ++k) {
                    value -= s_chol[i * LD + k] * z[k];
                }
                z[i] = value / s_chol[i * LD + i];
            }
#pragma unroll
            for (int i = 0; i < R; ++i) {
                s_panel[i * PLD + tid] = z[i];
                zbuf[i * d + c0 + tid] = z[i];
            }
        }
        for (int idx = tid; idx < width * R; idx += 64) {
            const int f = idx / R;
            const int c = idx - f * R;
            s_drive[f * LD + c] = drive[(c0 + f) * R + c];
        }
        __syncthreads();
        {
            const int bi = tid / 8;
            const int bj = tid - 8 * bi;
            float acc[kBlock][kBlock];
#pragma unroll
            for (int x = 0; x < kBlock; ++x) {
#pragma unroll
                for (int y = 0; y < kBlock; ++y) {
                    acc[x][y] = s_theta[(kBlock * bi + x) * LD + kBlock * bj + y];
                }
            }
            for (int f = 0; f < width; ++f) {
                float zc[kBlock];
                float wr[kBlock];
#pragma unroll
                for (int x = 0; x < kBlock; ++x) {
                    zc[x] = s_panel[(kBlock * bi + x) * PLD + f];
                    wr[x] = s_drive[f * LD + kBlock * bj + x];
                }
#pragma unroll
                for (int x = 0; x < kBlock; ++x) {
#pragma unroll
                    for (int y = 0; y < kBlock; ++y) {
                        acc[x][y] = fmaf(zc[x], wr[y], acc[x][y]);
                    }
                }
            }
#pragma unroll
            for (int x = 0; x < kBlock; ++x) {
#pragma unroll
                for (int y = 0; y < kBlock; ++y) {
                    s_theta[(kBlock * bi + x) * LD + kBlock * bj + y] = acc[x][y];
                }
            }
        }
        __syncthreads();
    }

    // Theta = Theta0 + Z W_drive / sqrt(n); F holds the lower factor.
    const float* base = a.base + h * R * R;
    for (int idx = tid; idx < R * R; idx += 64) {
        const int r = idx / R;
        const int c = idx - r * R;
        const float theta = base[idx] + s_theta[r * LD + c] / root;
        s_theta[r * LD + c] = theta;
        float factor = 0.0f;
        if (c < r) {
            factor = theta;
        } else if (c == r) {
            factor = softplus_one(theta);
        }
        s_lu[r * LD + c] = factor;
    }
    __syncthreads();
    // I + K = I + F F^T + Omega with IEEE FP32 products (reference.py:491-497).
    {
        float row_values[R];
        const bool owner = tid < R;
        if (owner) {
#pragma unroll
            for (int c = 0; c < R; ++c) {
                const int limit = c < tid ? c : tid;
                float sum = 0.0f;
                for (int k = 0; k <= limit; ++k) {
                    sum = fmaf(s_lu[tid * LD + k], s_lu[c * LD + k], sum);
                }
                float skew = 0.0f;
                if (c > tid) {
                    skew = s_theta[tid * LD + c];
                } else if (c < tid) {
                    skew = -s_theta[c * LD + tid];
                }
                row_values[c] = sum + skew + (c == tid ? 1.0f : 0.0f);
            }
        }
        __syncthreads();
        if (owner) {
            for (int c = 0; c < R; ++c) {
                s_lu[tid * LD + c] = row_values[c];
            }
        }
        __syncthreads();
    }

    // LU with partial pivoting (first maximal |a_ik| wins, as LAPACK getrf).
    for (int k = 0; k < R; ++k) {
        float value = (tid >= k && tid < R) ? fabsf(s_lu[tid * LD + k]) : -1.0f;
        int index = tid;
        wave_argmax(value, index);
        const int pivot = __shfl(index, 0, 64);
        if (pivot != k && tid < R) {
            const float upper = s_lu[k * LD + tid];
            s_lu[k * LD + tid] = s_lu[pivot * LD + tid];
            s_lu[pivot * LD + tid] = upper;
        }
        if (tid == 0) {
            s_perm[k] = pivot;
        }
        __syncthreads();
        if (tid > k && tid < R) {
            const float f = s_lu[tid * LD + k] / s_lu[k * LD + k];
            s_lu[tid * LD + k] = f;
            for (int j = k + 1; j < R; ++j) {
                s_lu[tid * LD + j] -= f * s_lu[k * LD + j];
            }
        }
        __syncthreads();
    }

    if (a.tape != nullptr) {
        float* tape = a.tape + system * a.tape_stride;
        for (int idx = tid; idx < R * R; idx += 64) {
            const int r = idx / R;
            const int c = idx - r * R;
            tape[idx] = s_chol[r * LD + c];
            tape[R * R + idx] = s_theta[r * LD + c];
            tape[2 * R * R + idx] = s_lu[r * LD + c];
        }
        if (tid < R) {
            tape[3 * R * R + tid] = static_cast<float>(s_perm[tid]);
        }
    }

    // U = (I + K)^-1 Z, X = 2U - (1 + eta) Z, M' = L^-T X / sqrt(n); one
    // lane per column, written straight into the apply operand layout.
    const int64_t blocks = (d + 15) / 16;
    for (int64_t c0 = 0; c0 < blocks * 16; c0 += kSolvePanel) {
        const int64_t column = c0 + tid;
        if (column >= blocks * 16) {
            continue;
        }
        // u holds U, then X = 2U - (1 + eta) Z, then M' in place.
        float u[R];
        if (column < d) {
            float z[R];
#pragma unroll
            for (int i = 0; i < R; ++i) {
                z[i] = zbuf[i * d + column];
                s_panel[i * (kSolvePanel + 1) + tid] = z[i];
            }
            for (int k = 0; k < R; ++k) {
                const int p = s_perm[k];
                if (p != k) {
                    const float swap = s_panel[k * (kSolvePanel + 1) + tid];
                    s_panel[k * (kSolvePanel + 1) + tid] = s_panel[p * (kSolvePanel + 1) + tid];
                    s_panel[p * (kSolvePanel + 1) + tid] = swap;
                }
            }
#pragma unroll
            for (int i = 0; i < R; ++i) {
                float value = s_panel[i * (kSolvePanel + 1) + tid];
#pragma unroll
                for (int k = 0; k < i; ++k) {
                    value -= s_lu[i * LD + k] * u[k];
                }
                u[i] = value;
            }
#pragma unroll
            for (int i = R - 1; i >= 0; --i) {
                float value = u[i];
#pragma unroll
                for (int k = i + 1; k < R; ++k) {
                    value -= s_lu[i * LD + k] * u[k];
                }
                u[i] = value / s_lu[i * LD + i];
            }
            if (a.tape != nullptr) {
                float* tape = a.tape + system * a.tape_stride + 3 * R * R + R;
#pragma unroll
                for (int i = 0; i < R; ++i) {
                    tape[i * d + column] = z[i];
                    tape[R * d + i * d + column] = u[i];
                }
            }
#pragma unroll
            for (int i = 0; i < R; ++i) {
                u[i] = 2.0f * u[i] - (1.0f + eta) * z[i];
            }
#pragma unroll
            for (int i = R - 1; i >= 0; --i) {
                float value = u[i];
#pragma unroll
                for (int k = i + 1; k < R; ++k) {
                    value -= s_chol[k * LD + i] * u[k];
                }
                u[i] = value / s_chol[i * LD + i];
            }
#pragma unroll
            for (int i = 0; i < R; ++i) {
                u[i] = u[i] / root;
            }
        } else {
#pragma unroll
            for (int i = 0; i < R; ++i) {
                u[i] = 0.0f;
            }
        }
        // Operand record of (feature block fb, lane g*16 + column%16).
        const int64_t fb = column / 16;
        const int lane_low = static_cast<int>(column & 15);
        uint16_t* record_base = a.mop + ((system * blocks + fb) * 64) * AL::kLaneHalfs;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            uint16_t* record = record_base + (g * 16 + lane_low) * AL::kLaneHalfs;
#pragma unroll
            for (int s = 0; s < AL::kSteps32; ++s) {
#pragma unroll
                for (int i = 0; i < 8; i += 2) {
                    uint32_t hi, lo;
                    split_bf16(u[AL::rank32(s, g, i)], u[AL::rank32(s, g, i + 1)], hi, lo);
                    *reinterpret_cast<uint32_t*>(record + AL::offset32(s) + i) = hi;
                    *reinterpret_cast<uint32_t*>(record + AL::offset32(s) + 8 + i) = lo;
                }
            }
#pragma unroll
            for (int s = 0; s < AL::kSteps16; ++s) {
#pragma unroll
                for (int i = 0; i < 4; i += 2) {
                    uint32_t hi, lo;
                    split_bf16(u[AL::rank16(s, g, i)], u[AL::rank16(s, g, i + 1)], hi, lo);
                    *reinterpret_cast<uint32_t*>(record + AL::offset16(s) + i) = hi;
                    *reinterpret_cast<uint32_t*>(record + AL::offset16(s) + 4 + i) = lo;
                }
            }
        }
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
    const int64_t wave = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
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
    for (int64_t t0 = begin; t0 < end; t0 += 16) {
        const int64_t token = t0 + q;
        const bool live = token < end;
        const int64_t safe_token = live ? token : begin;
        const uint16_t* row = a.projected + (b * a.length + safe_token) * a.width;
        const uint32_t* phase_row = a.phases + b * a.phase_batch_stride + safe_token * PAIRS;

        u32x4 b_hi32[AL::kSteps32 > 0 ? AL::kSteps32 : 1];
        u32x4 b_lo32[AL::kSteps32 > 0 ? AL::kSteps32 : 1];
#pragma unroll
        for (int s = 0; s < AL::kSteps32; ++s) {
            const int first_rank = 32 * s + 8 * g;
            u32x4 rel;
            u32x4 ph;
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
            const int first_rank = 16 * s + 4 * g;
            u32x2 rel;
            u32x2 ph;
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
            const uint16_t* content = row + content_offset + feature;
            if (VEC && feature + 3 < d) {
                const u32x2 c = *reinterpret_cast<const u32x2*>(content);
                u32x2 y;
                y.x = pack_bf16(fmaf(eta, bf16_lo(c.x), acc[0]), fmaf(eta, bf16_hi(c.x), acc[1]));
                y.y = pack_bf16(fmaf(eta, bf16_lo(c.y), acc[2]), fmaf(eta, bf16_hi(c.y), acc[3]));
                *reinterpret_cast<u32x2*>(out) = y;
            } else {
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
// Launchers.
template <int R>
static hipError_t launch_reduce(const ReduceArgs& a, int cpw, bool vec, hipStream_t stream) {
    const dim3 grid(static_cast<unsigned>((a.total_waves + 3) / 4));
    if (cpw == 1) {
        if (vec) {
            reduce_kernel<R, 1, true><<<grid, 256, 0, stream>>>(a);
        } else {
            reduce_kernel<R, 1, false><<<grid, 256, 0, stream>>>(a);
        }
    } else {
        if (vec) {
            reduce_kernel<R, 2, true><<<grid, 256, 0, stream>>>(a);
        } else {
            reduce_kernel<R, 2, false><<<grid, 256, 0, stream>>>(a);
        }
    }
    return hipGetLastError();
}

template <int R>
static hipError_t launch_apply(const ApplyArgs& a, int nfbw, bool vec, hipStream_t stream) {
    const dim3 grid(static_cast<unsigned>((a.total_waves + 3) / 4));
    switch (nfbw) {
        case 1:
            if (vec) apply_kernel<R, 1, true><<<grid, 256, 0, stream>>>(a);
            else apply_kernel<R, 1, false><<<grid, 256, 0, stream>>>(a);
            break;
        case 2:
            if (vec) apply_kernel<R, 2, true><<<grid, 256, 0, stream>>>(a);
            else apply_kernel<R, 2, false><<<grid, 256, 0, stream>>>(a);
            break;
        default:
            if (vec) apply_kernel<R, 4, true><<<grid, 256, 0, stream>>>(a);
            else apply_kernel<R, 4, false><<<grid, 256, 0, stream>>>(a);
            break;
    }
    return hipGetLastError();
}

hipError_t launch_phase(const PhaseArgs& a, hipStream_t stream) {
    const dim3 grid(static_cast<unsigned>((a.count + 255) / 256));
    phase_kernel<<<grid, 256, 0, stream>>>(a);
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
        case 16: solve_kernel<16><<<grid, 64, 0, stream>>>(a); break;
        case 32: solve_kernel<32><<<grid, 64, 0, stream>>>(a); break;
        case 48: solve_kernel<48><<<grid, 64, 0, stream>>>(a); break;
        default: solve_kernel<64><<<grid, 64, 0, stream>>>(a); break;
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

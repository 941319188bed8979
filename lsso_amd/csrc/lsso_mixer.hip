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
#include "lsso_reduce.h"

namespace lsso_hip {

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
    const bool do_gram = a.gram != 0 && cg == 0;

    // One accumulator per block, 32-token steps in token order: the fused
    // projection + reduce kernel accumulates in the same order, so both
    // produce the same partials bit for bit.
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

    float* part = a.partials + ((b * a.heads + h) * a.chunks + chunk) * a.partial_stride;
    if (do_gram) {
        store_gram_partial<R>(part, acc_g, q, g);
    }
    store_cross_partial<R, CPW>(part + R * R, acc_s, q, g, cg, a.head_dim);
}

// ---------------------------------------------------------------------------
// Solve: one 256-thread workgroup per (b, h) system.
//
//   A = G / n + I = L L^T            Cholesky
//   L^-1                             forward substitution, one column per lane
//   Z = L^-1 S / sqrt(n)             product
//   Theta = Theta0 + Z W / sqrt(n)   product
//   I + K = I + F F^T + Omega        product
//   (I + K)^-1                       Gauss-Jordan with partial (row) pivoting
//   U = (I + K)^-1 Z, X = 2U - (1 + eta) Z, M' = L^-T X / sqrt(n)   products
//
// The two factorizations are sequential (one step per rank) and run in wave 0
// with one matrix row per lane held in registers.  A step's pivot row reaches
// the other lanes by v_readlane into scalar registers, one element per
// column, so a step is one chain of VALU instructions with no LDS round trip.
// Step loops stay rolled (the pivot lane and column are wave-uniform
// registers); the substitution for L^-1 has no cross-lane traffic and is
// unrolled.  The products use all four waves.
extern "C" __device__ unsigned int __ockl_wfred_max_u32(unsigned int);

constexpr int kSolveThreads = 256;
constexpr int kSolvePanel = 64;

template <int R>
struct SolveLayout {
    static constexpr int kLD = R + 4;              // R x R matrices (16-byte rows)
    static constexpr int kPLD = kSolvePanel + 4;   // R x panel matrices
    static constexpr int kChunks = R / 16;         // 16-float register chunks per row
    static constexpr int kThetaQuads = (R * R / 4 + kSolveThreads - 1) / kSolveThreads;
    static constexpr int kChunkBatch = R <= 32 ? 8 : 4;    // chunk loads in flight per element
    static constexpr int kLinv = 0;                       // L^-1 rows
    static constexpr int kLinvT = kLinv + R * kLD;        // L^-1 transposed
    static constexpr int kTheta = kLinvT + R * kLD;       // Theta
    static constexpr int kWork = kTheta + R * kLD;        // A; F; Gauss-Jordan rows in step order
    static constexpr int kSys = kWork + R * kLD;          // I + K, then (I + K)^-1
    static constexpr int kPanelA = kSys + R * kLD;        // S panel; drive panel; X panel
    static constexpr int kPanelB = kPanelA + R * kPLD;    // Z panel; M' panel
    static constexpr int kColumn = kPanelB + R * kPLD;    // 1 / L_ii
    static constexpr int kPivot = kColumn + 64;           // pivot row of each step
    static constexpr int kTotal = kPivot + R;
};

// A matrix row in registers: up to four 16-float vectors that are separate
// local values of the kernel, bound here by reference.  Kept apart (not an
// aggregate) so that a wave-uniform element index compiles to a relative
// register move rather than a private-memory array.
template <int Q>
struct RegRow {
    f32x16 &c0, &c1, &c2, &c3;
    template <int q>
    __device__ __forceinline__ f32x16& at() const {
        if constexpr (q == 0) {
            return c0;
        } else if constexpr (q == 1) {
            return c1;
        } else if constexpr (q == 2) {
            return c2;
        } else {
            return c3;
        }
    }
};

template <int Q, int q = 0>
__device__ __forceinline__ void row_zero(const RegRow<Q>& r) {
    if constexpr (q < Q) {
        r.template at<q>() = 0.0f;
        row_zero<Q, q + 1>(r);
    }
}

// Element k of a register row for a wave-uniform k.
template <int Q, int q = 0>
__device__ __forceinline__ float row_get(const RegRow<Q>& r, int k, float found = 0.0f) {
    if constexpr (q < Q) {
        const float c = r.template at<q>()[k & 15];
        return row_get<Q, q + 1>(r, k, (k >> 4) == q ? c : found);
    } else {
        return found;
    }
}

template <int Q, int q = 0>
__device__ __forceinline__ void row_set(const RegRow<Q>& r, int k, float value) {
    if constexpr (q < Q) {
        f32x16 t = r.template at<q>();
        const float old = t[k & 15];
        t[k & 15] = (k >> 4) == q ? value : old;
        r.template at<q>() = t;
        row_set<Q, q + 1>(r, k, value);
    }
}

template <int Q, int q = 0>
__device__ __forceinline__ void row_load(const RegRow<Q>& r, const float* p) {
    if constexpr (q < Q) {
        f32x16 t;
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            const f32x4 v = *reinterpret_cast<const f32x4*>(p + 16 * q + 4 * m);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                t[4 * m + e] = v[e];
            }
        }
        r.template at<q>() = t;
        row_load<Q, q + 1>(r, p);
    }
}

template <int Q, int q = 0>
__device__ __forceinline__ void row_store(float* p, const RegRow<Q>& r) {
    if constexpr (q < Q) {
        const f32x16 t = r.template at<q>();
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            *reinterpret_cast<f32x4*>(p + 16 * q + 4 * m) =
                (f32x4){t[4 * m], t[4 * m + 1], t[4 * m + 2], t[4 * m + 3]};
        }
        row_store<Q, q + 1>(p, r);
    }
}

// r -= f * x
template <int Q, int q = 0>
__device__ __forceinline__ void row_axpy(const RegRow<Q>& r, float f, const RegRow<Q>& x) {
    if constexpr (q < Q) {
        f32x16 t = r.template at<q>();
        const f32x16 xt = x.template at<q>();
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            t[e] = fmaf(-f, xt[e], t[e]);
        }
        r.template at<q>() = t;
        row_axpy<Q, q + 1>(r, f, x);
    }
}

template <int Q, int q = 0>
__device__ __forceinline__ void row_scale(const RegRow<Q>& r, float factor) {
    if constexpr (q < Q) {
        r.template at<q>() = r.template at<q>() * factor;
        row_scale<Q, q + 1>(r, factor);
    }
}

// Row `row` of the identity (row may differ between lanes).
template <int Q, int q = 0>
__device__ __forceinline__ void row_identity(const RegRow<Q>& r, int row) {
    if constexpr (q < Q) {
        f32x16 t;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            t[e] = 16 * q + e == row ? 1.0f : 0.0f;
        }
        r.template at<q>() = t;
        row_identity<Q, q + 1>(r, row);
    }
}

// Column `column` of an LDS matrix with row stride ld receives the row.
template <int Q, int q = 0>
__device__ __forceinline__ void row_store_column(float* p, int ld, int column, const RegRow<Q>& r) {
    if constexpr (q < Q) {
        const f32x16 t = r.template at<q>();
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            p[(16 * q + e) * ld + column] = t[e];
        }
        row_store_column<Q, q + 1>(p, ld, column, r);
    }
}

#define LSSO_REG_ROW(name)                                              \
    f32x16 name##_0 = 0.0f, name##_1 = 0.0f, name##_2 = 0.0f, name##_3 = 0.0f; \
    const RegRow<Q> name{name##_0, name##_1, name##_2, name##_3}

// LDS ordering between lanes of one wave: its LDS instructions execute in
// issue order, so only the compiler must be kept from reordering.
__device__ __forceinline__ void wave_lds_order() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// r -= f * (row of lane `source` of r), the source row read by v_readlane
// element by element.  The source lane must pass f = 0, so its row is the
// same before and after each element's update.
template <int Q, int q = 0>
__device__ __forceinline__ void row_axpy_lane(const RegRow<Q>& r, float f, int source) {
    if constexpr (q < Q) {
        f32x16 t = r.template at<q>();
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const float pivot_row = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(t[e]), source));
            t[e] = fmaf(-f, pivot_row, t[e]);
        }
        r.template at<q>() = t;
        row_axpy_lane<Q, q + 1>(r, f, source);
    }
}

// Column `lane` of L^-1 for lower-triangular L (row-major in LDS, row stride
// LD) and the reciprocal diagonal: x_i = (delta_i,lane - sum_{m<i} L_im x_m)
// / L_ii, summed in ascending m.  Rows of L are wave-uniform LDS reads.
template <int R, int LD>
__device__ __forceinline__ void lower_inverse_column(const float* l, const float* inv_diag, int lane,
                                                     float (&x)[R]) {
#pragma unroll
    for (int i = 0; i < R; ++i) {
        float acc = lane == i ? 1.0f : 0.0f;
#pragma unroll
        for (int m = 0; m < i; m += 4) {
            const f32x4 l4 = *reinterpret_cast<const f32x4*>(l + i * LD + m);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                if (m + e < i) {
                    acc = fmaf(-l4[e], x[m + e], acc);
                }
            }
        }
        x[i] = acc * inv_diag[i];
    }
}

template <int R>
__global__ __launch_bounds__(kSolveThreads) void solve_kernel(SolveArgs a) {
    using SL = SolveLayout<R>;
    using AL = ApplyLayout<R>;
    constexpr int Q = SL::kChunks;
    constexpr int LD = SL::kLD;
    constexpr int PLD = SL::kPLD;
    __shared__ __attribute__((aligned(16))) float smem[SL::kTotal];
    float* s_linv = smem + SL::kLinv;
    float* s_linvt = smem + SL::kLinvT;
    float* s_theta = smem + SL::kTheta;
    float* s_work = smem + SL::kWork;
    float* s_sys = smem + SL::kSys;
    float* s_pa = smem + SL::kPanelA;
    float* s_pb = smem + SL::kPanelB;
    int* s_pivot = reinterpret_cast<int*>(smem + SL::kPivot);

    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int64_t system = blockIdx.x;
    const int64_t b = system / a.heads;
    const int64_t h = system - b * a.heads;
    const int d = static_cast<int>(a.head_dim);
    const int chunks = static_cast<int>(a.chunks);
    const int64_t stride = a.partial_stride;
    const float count = a.valid_counts != nullptr ? a.valid_counts[b] : static_cast<float>(a.length);
    const float root = sqrtf(count);
    const float eta = bounded_complement(a.eta_raw[h]);
    const float* part = a.partials + system * chunks * stride;
    float* tape = a.tape != nullptr ? a.tape + system * a.tape_stride : nullptr;

    // ---- A = G / n + I; chunk partials summed in ascending order, each
    // thread keeping kChunkBatch chunks of loads in flight --------------------
    {
        constexpr int kQuads = (R * R / 4 + kSolveThreads - 1) / kSolveThreads;
        f32x4 acc[kQuads];
        const float* src[kQuads];
#pragma unroll
        for (int t = 0; t < kQuads; ++t) {
            const int q = tid + t * kSolveThreads;
            acc[t] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
            src[t] = part + 4 * (q < R * R / 4 ? q : 0);
        }
        for (int ch0 = 0; ch0 < chunks; ch0 += SL::kChunkBatch) {
            f32x4 v[kQuads][SL::kChunkBatch];
#pragma unroll
            for (int t = 0; t < kQuads; ++t) {
#pragma unroll
                for (int u = 0; u < SL::kChunkBatch; ++u) {
                    const int ch = ch0 + u < chunks ? ch0 + u : chunks - 1;
                    v[t][u] = *reinterpret_cast<const f32x4*>(src[t] + ch * stride);
                }
            }
#pragma unroll
            for (int t = 0; t < kQuads; ++t) {
#pragma unroll
                for (int u = 0; u < SL::kChunkBatch; ++u) {
                    if (ch0 + u < chunks) {
                        acc[t] += v[t][u];
                    }
                }
            }
        }
#pragma unroll
        for (int t = 0; t < kQuads; ++t) {
            const int q = tid + t * kSolveThreads;
            if (q < R * R / 4) {
                const int i = (4 * q) / R;
                const int j = 4 * q - i * R;
                f32x4 value;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    value[e] = acc[t][e] / count + (j + e == i ? 1.0f : 0.0f);
                }
                *reinterpret_cast<f32x4*>(s_work + i * LD + j) = value;
            }
        }
    }
    __syncthreads();

    // ---- Cholesky in wave 0, right-looking: step k takes f_i = a_ik / a_kk
    // and subtracts f_i times row k from every row i > k of the trailing
    // matrix; column k of L is a_ik / sqrt(a_kk).  Row k comes from lane k by
    // v_readlane.  Columns left of k in `work` are no longer read (L is built
    // in `lrow`).
    if (wave == 0) {
        const bool live = lane < R;
        LSSO_REG_ROW(work);
        LSSO_REG_ROW(lrow);
        if (live) {
            row_load(work, s_work + lane * LD);
        }
        float own_inv_root = 1.0f;
#pragma unroll 1
        for (int k = 0; k < R; ++k) {
            const float x = row_get(work, k);
            const float pivot = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), k));
            // Pivots of A = G/n + I are >= 1, so the hardware reciprocal,
            // square root and reciprocal square root (1 ulp) need no range
            // handling.
            const float inv_pivot = __builtin_amdgcn_rcpf(pivot);
            const float inv_root = __builtin_amdgcn_rsqf(pivot);
            const float root_pivot = __builtin_amdgcn_sqrtf(pivot);
            const float f = lane > k ? x * inv_pivot : 0.0f;
            row_axpy_lane(work, f, k);
            row_set(lrow, k, lane > k ? x * inv_root : (lane == k ? root_pivot : 0.0f));
            own_inv_root = lane == k ? inv_root : own_inv_root;
        }
        // L and 1 / L_ii to LDS for the substitution (A in s_work is spent).
        if (live) {
            row_store(s_work + lane * LD, lrow);
            smem[SL::kColumn + lane] = own_inv_root;
            if (tape != nullptr) {
                row_store(tape + lane * R, lrow);
            }
        }
        wave_lds_order();
        if (live) {
            float x[R];
            lower_inverse_column<R, LD>(s_work, smem + SL::kColumn, lane, x);
            // Lane c holds column c of L^-1: row c of L^-T and column c of L^-1.
#pragma unroll
            for (int i = 0; i < R; i += 4) {
                *reinterpret_cast<f32x4*>(s_linvt + lane * LD + i) = (f32x4){x[i], x[i + 1], x[i + 2], x[i + 3]};
            }
#pragma unroll
            for (int i = 0; i < R; ++i) {
                s_linv[i * LD + lane] = x[i];
            }
        }
    }
    __syncthreads();
    if (tape != nullptr) {
        for (int q = tid; q < R * R / 4; q += kSolveThreads) {
            const int i = (4 * q) / R;
            const int j = 4 * q - i * R;
            *reinterpret_cast<f32x4*>(tape + 3 * R * R + 4 * q) = *reinterpret_cast<const f32x4*>(s_linv + i * LD + j);
        }
    }

    // ---- Z panels (Z = L^-1 S / sqrt(n)) and Theta = Z W accumulation ------
    float* zbuf = a.zbuf + system * R * d;
    const float* drive = a.drive + h * d * R;
    f32x4 theta_acc[SL::kThetaQuads];
#pragma unroll
    for (int t = 0; t < SL::kThetaQuads; ++t) {
        theta_acc[t] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
    }
    for (int c0 = 0; c0 < d; c0 += kSolvePanel) {
        const int width = d - c0 < kSolvePanel ? d - c0 : kSolvePanel;
        {
            // S panel: thread (row wave + 4 t, column lane); columns past the
            // panel width load a clamped column and store zero.
            constexpr int kRows = R / 4;
            const int c = lane < width ? lane : width - 1;
            float acc[kRows];
#pragma unroll
            for (int t = 0; t < kRows; ++t) {
                acc[t] = 0.0f;
            }
            const float* src = part + R * R + wave * d + c0 + c;
            for (int ch0 = 0; ch0 < chunks; ch0 += SL::kChunkBatch) {
                float v[kRows][SL::kChunkBatch];
#pragma unroll
                for (int t = 0; t < kRows; ++t) {
#pragma unroll
                    for (int u = 0; u < SL::kChunkBatch; ++u) {
                        const int ch = ch0 + u < chunks ? ch0 + u : chunks - 1;
                        v[t][u] = src[ch * stride + 4 * t * d];
                    }
                }
#pragma unroll
                for (int t = 0; t < kRows; ++t) {
#pragma unroll
                    for (int u = 0; u < SL::kChunkBatch; ++u) {
                        if (ch0 + u < chunks) {
                            acc[t] += v[t][u];
                        }
                    }
                }
            }
#pragma unroll
            for (int t = 0; t < kRows; ++t) {
                s_pa[(wave + 4 * t) * PLD + lane] = lane < width ? acc[t] / root : 0.0f;
            }
        }
        __syncthreads();
        {
            float scol[R];
#pragma unroll
            for (int k = 0; k < R; ++k) {
                scol[k] = s_pa[k * PLD + lane];
            }
#pragma unroll 1
            for (int i = wave; i < R; i += 4) {
                const float* lrow = s_linv + i * LD;
                float acc = 0.0f;
#pragma unroll
                for (int k = 0; k < R; k += 4) {
                    const f32x4 l4 = *reinterpret_cast<const f32x4*>(lrow + k);
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        acc = fmaf(l4[e], scol[k + e], acc);
                    }
                }
                s_pb[i * PLD + lane] = acc;
                if (lane < width) {
                    zbuf[i * d + c0 + lane] = acc;
                    if (tape != nullptr) {
                        tape[4 * R * R + i * d + c0 + lane] = acc;
                    }
                }
            }
        }
        __syncthreads();
        for (int e = tid; e < kSolvePanel * R / 4; e += kSolveThreads) {
            const int c = (4 * e) / R;
            f32x4 w = {0.0f, 0.0f, 0.0f, 0.0f};
            if (c < width) {
                w = *reinterpret_cast<const f32x4*>(drive + (c0 + c) * R + (4 * e - c * R));
            }
            *reinterpret_cast<f32x4*>(s_pa + 4 * e) = w;
        }
        __syncthreads();
#pragma unroll
        for (int t = 0; t < SL::kThetaQuads; ++t) {
            const int q = tid + t * kSolveThreads;
            if (q < R * R / 4) {
                const int i = q / (R / 4);
                const int j = 4 * (q - i * (R / 4));
#pragma unroll 8
                for (int c = 0; c < width; ++c) {
                    const float z = s_pb[i * PLD + c];
                    const f32x4 w = *reinterpret_cast<const f32x4*>(s_pa + c * R + j);
                    theta_acc[t] = z * w + theta_acc[t];
                }
            }
        }
        __syncthreads();
    }

    // ---- Theta = Theta0 + acc / sqrt(n); F = tril(Theta, -1) + diag(softplus)
#pragma unroll
    for (int t = 0; t < SL::kThetaQuads; ++t) {
        const int q = tid + t * kSolveThreads;
        if (q < R * R / 4) {
            const int i = q / (R / 4);
            const int j = 4 * (q - i * (R / 4));
            const f32x4 base = *reinterpret_cast<const f32x4*>(a.base + (h * R + i) * R + j);
            const f32x4 theta = base + theta_acc[t] / root;
            *reinterpret_cast<f32x4*>(s_theta + i * LD + j) = theta;
            if (tape != nullptr) {
                *reinterpret_cast<f32x4*>(tape + R * R + i * R + j) = theta;
            }
            f32x4 factor;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                factor[e] = j + e < i ? theta[e] : 0.0f;
            }
            if (j <= i && i < j + 4) {
                factor[i - j] = softplus_one(theta[i - j]);
            }
            *reinterpret_cast<f32x4*>(s_work + i * LD + j) = factor;
        }
    }
    __syncthreads();

    // ---- I + K = I + F F^T + Omega, IEEE FP32 products (reference.py:491-497);
    // all R products summed (F is lower triangular, the rest add exact zeros).
#pragma unroll
    for (int t = 0; t < SL::kThetaQuads; ++t) {
        const int q = tid + t * kSolveThreads;
        if (q < R * R / 4) {
            const int i = q / (R / 4);
            const int j = 4 * (q - i * (R / 4));
            f32x4 sum = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll 2
            for (int k = 0; k < R; k += 4) {
                const f32x4 fi = *reinterpret_cast<const f32x4*>(s_work + i * LD + k);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const f32x4 fj = *reinterpret_cast<const f32x4*>(s_work + (j + e) * LD + k);
#pragma unroll
                    for (int m = 0; m < 4; ++m) {
                        sum[e] = fmaf(fi[m], fj[m], sum[e]);
                    }
                }
            }
            f32x4 value;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int c = j + e;
                float skew = 0.0f;
                if (c > i) {
                    skew = s_theta[i * LD + c];
                } else if (c < i) {
                    skew = -s_theta[c * LD + i];
                }
                value[e] = sum[e] + skew + (c == i ? 1.0f : 0.0f);
            }
            *reinterpret_cast<f32x4*>(s_sys + i * LD + j) = value;
        }
    }
    __syncthreads();

    // ---- (I + K)^-1 by Gauss-Jordan in wave 0, in place, with implicit row
    // pivoting: step k picks the largest |a_ik| over rows not yet used (first
    // row on ties, as the LU partial pivoting it replaces), eliminates column
    // k from every other row with the unscaled pivot row, and keeps column k
    // as column p_k of the growing inverse.  Row p_k ends as pi_k times row k
    // of the inverse with its columns in step order.
    if (wave == 0) {
        const bool live = lane < R;
        LSSO_REG_ROW(rowv);
        if (live) {
            row_load(rowv, s_sys + lane * LD);
        }
        bool open = live;
        int own_step = 0;
        float own_pivot = 1.0f;
#pragma unroll 1
        for (int k = 0; k < R; ++k) {
            const float x = row_get(rowv, k);
            const unsigned magnitude = __float_as_uint(fabsf(x));
            const unsigned best = __builtin_amdgcn_readfirstlane(__ockl_wfred_max_u32(open ? magnitude : 0u));
            const unsigned long long ties = __ballot(open && magnitude == best);
            const int p = __builtin_amdgcn_readfirstlane(static_cast<int>(__builtin_ctzll(ties)));
            const float pivot = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), p));
            const float inv_pivot = __builtin_amdgcn_rcpf(pivot);
            const float f = lane == p ? 0.0f : x * inv_pivot;
            row_axpy_lane(rowv, f, p);
            row_set(rowv, k, lane == p ? 1.0f : -f);
            if (lane == p) {
                open = false;
                own_step = k;
                own_pivot = pivot;
            }
            if (lane == 0) {
                s_pivot[k] = p;
            }
        }
        if (live) {
            row_scale(rowv, __builtin_amdgcn_rcpf(own_pivot));
            row_store(s_work + own_step * LD, rowv);
        }
    }
    __syncthreads();
    // Column order back to row numbers: inverse[k][p_m] = work[k][m].
    for (int e = tid; e < R * R; e += kSolveThreads) {
        const int k = e / R;
        const int m = e - k * R;
        s_sys[k * LD + s_pivot[m]] = s_work[k * LD + m];
    }
    __syncthreads();
    if (tape != nullptr) {
        for (int q = tid; q < R * R / 4; q += kSolveThreads) {
            const int i = (4 * q) / R;
            const int j = 4 * q - i * R;
            *reinterpret_cast<f32x4*>(tape + 2 * R * R + 4 * q) = *reinterpret_cast<const f32x4*>(s_sys + i * LD + j);
        }
    }

    // ---- U, X, M' panels, written as apply operand records -----------------
    const int blocks = (d + 15) / 16;
    for (int c0 = 0; c0 < blocks * 16; c0 += kSolvePanel) {
        const int width = d - c0 < kSolvePanel ? d - c0 : kSolvePanel;
        if (d > kSolvePanel) {
            for (int e = tid; e < R * kSolvePanel; e += kSolveThreads) {
                const int i = e / kSolvePanel;
                const int c = e - i * kSolvePanel;
                s_pb[i * PLD + c] = c < width ? zbuf[i * d + c0 + c] : 0.0f;
            }
            __syncthreads();
        }
        {
            float zcol[R];
#pragma unroll
            for (int k = 0; k < R; ++k) {
                zcol[k] = s_pb[k * PLD + lane];
            }
#pragma unroll 1
            for (int i = wave; i < R; i += 4) {
                const float* irow = s_sys + i * LD;
                float acc = 0.0f;
#pragma unroll
                for (int k = 0; k < R; k += 4) {
                    const f32x4 v4 = *reinterpret_cast<const f32x4*>(irow + k);
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        acc = fmaf(v4[e], zcol[k + e], acc);
                    }
                }
                if (tape != nullptr && lane < width) {
                    tape[4 * R * R + R * d + i * d + c0 + lane] = acc;
                }
                s_pa[i * PLD + lane] = 2.0f * acc - (1.0f + eta) * s_pb[i * PLD + lane];
            }
        }
        __syncthreads();
        {
            float xcol[R];
#pragma unroll
            for (int k = 0; k < R; ++k) {
                xcol[k] = s_pa[k * PLD + lane];
            }
#pragma unroll 1
            for (int i = wave; i < R; i += 4) {
                const float* trow = s_linvt + i * LD;
                float acc = 0.0f;
#pragma unroll
                for (int k = 0; k < R; k += 4) {
                    const f32x4 v4 = *reinterpret_cast<const f32x4*>(trow + k);
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        acc = fmaf(v4[e], xcol[k + e], acc);
                    }
                }
                s_pb[i * PLD + lane] = lane < width ? acc / root : 0.0f;
            }
        }
        __syncthreads();
        {
            // Record of feature block fb, lane g4 * 16 + column % 16.
            const int fb_local = tid >> 6;
            const int fb = c0 / 16 + fb_local;
            if (fb < blocks) {
                const int g4 = lane >> 4;
                const int column = fb_local * 16 + (lane & 15);
                uint16_t* record = a.mop + ((system * blocks + fb) * 64 + lane) * AL::kLaneHalfs;
#pragma unroll
                for (int st = 0; st < AL::kSteps32; ++st) {
#pragma unroll
                    for (int i = 0; i < 8; i += 2) {
                        uint32_t hi, lo;
                        split_bf16(s_pb[AL::rank32(st, g4, i) * PLD + column],
                                   s_pb[AL::rank32(st, g4, i + 1) * PLD + column], hi, lo);
                        *reinterpret_cast<uint32_t*>(record + AL::offset32(st) + i) = hi;
                        *reinterpret_cast<uint32_t*>(record + AL::offset32(st) + 8 + i) = lo;
                    }
                }
#pragma unroll
                for (int st = 0; st < AL::kSteps16; ++st) {
#pragma unroll
                    for (int i = 0; i < 4; i += 2) {
                        uint32_t hi, lo;
                        split_bf16(s_pb[AL::rank16(st, g4, i) * PLD + column],
                                   s_pb[AL::rank16(st, g4, i + 1) * PLD + column], hi, lo);
                        *reinterpret_cast<uint32_t*>(record + AL::offset16(st) + i) = hi;
                        *reinterpret_cast<uint32_t*>(record + AL::offset16(st) + 4 + i) = lo;
                    }
                }
            }
        }
        __syncthreads();
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
        case 16: solve_kernel<16><<<grid, kSolveThreads, 0, stream>>>(a); break;
        case 32: solve_kernel<32><<<grid, kSolveThreads, 0, stream>>>(a); break;
        case 48: solve_kernel<48><<<grid, kSolveThreads, 0, stream>>>(a); break;
        default: solve_kernel<64><<<grid, kSolveThreads, 0, stream>>>(a); break;
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

// Building blocks of the L-reductions G = sum rot(R)^T rot(R) and
// S = sum rot(R)^T C over a token chunk, shared by the standalone reduce
// kernel (operands from HBM) and the projection + reduce kernel (operands
// from the packed tile in LDS).  Both run the same MFMA chains in the same
// token order, so their partials agree bit for bit.
#pragma once

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

// ---------------------------------------------------------------------------
// Token-chunk reduction of one head: operands, MFMA chains and partial stores.
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
            const uint16_t* content_row = a.content + (b * a.length + (live ? token : 0)) * a.content_stride;
            t.con[j][c] = fv ? load_pair<VEC>(content_row + h * a.head_dim + feature,
                                              feature + 1 < a.head_dim)
                             : 0u;
        }
    }
}

// Raw-buffer form of reduce_load (rows whose relation pairs and content
// feature pairs are whole aligned dwords).  The three token streams of a
// step get raw buffers that start at the step's first token and end at the
// chunk's end, so tokens past the chunk read as zeros with no access and no
// branch, and the per-lane byte offsets (token 8 g of the step, plus a
// constant per token j) are the same for every step: only the scalar buffer
// bases move.  An absent pair slot or feature pair gets an offset past every
// buffer.  Loads and zeros are those of reduce_load<R, CPW, true>.
template <int R, int CPW>
struct ReduceLanes {
    uint32_t rel;
    uint32_t ph;
    uint32_t con[CPW];
};

template <int R, int CPW>
__device__ __forceinline__ ReduceLanes<R, CPW> reduce_lanes(const ReduceArgs& a, int64_t h, int cg, int q,
                                                           int g) {
    using L = ReduceLayout<R>;
    constexpr int PS = L::kPairSlots;
    ReduceLanes<R, CPW> o;
    const bool pv = PS * q < L::kPairs;
    const uint32_t row0 = 8u * static_cast<uint32_t>(g);
    o.rel = pv ? 2u * (row0 * static_cast<uint32_t>(a.width) + static_cast<uint32_t>(h * R) +
                       static_cast<uint32_t>(2 * PS * q))
               : kOutOfRange;
    o.ph = pv ? 4u * (row0 * L::kPairs + static_cast<uint32_t>(PS * q)) : kOutOfRange;
#pragma unroll
    for (int c = 0; c < CPW; ++c) {
        const int64_t feature = 2 * (static_cast<int64_t>(cg) * 16 * CPW + 16 * c + q);
        o.con[c] = feature < a.head_dim
            ? 2u * (row0 * static_cast<uint32_t>(a.content_stride) +
                    static_cast<uint32_t>(h * a.head_dim + feature))
            : kOutOfRange;
    }
    return o;
}

template <int R, int CPW>
__device__ __forceinline__ void reduce_load_buffer(ReduceTile<R, CPW>& t, const ReduceArgs& a,
                                                   const ReduceLanes<R, CPW>& o, int64_t b, int64_t t0,
                                                   int64_t end) {
    using L = ReduceLayout<R>;
    constexpr int PS = L::kPairSlots;
    const int64_t rows = end - t0;
    const BufferRsrc rel = make_buffer(a.projected + (b * a.length + t0) * a.width, 2 * rows * a.width);
    const BufferRsrc ph = make_buffer(a.phases + b * a.phase_batch_stride + t0 * L::kPairs,
                                      4 * rows * L::kPairs);
    const BufferRsrc con = make_buffer(a.content + (b * a.length + t0) * a.content_stride,
                                       2 * rows * a.content_stride);
    const uint32_t rel_step = 2u * static_cast<uint32_t>(a.width);
    const uint32_t con_step = 2u * static_cast<uint32_t>(a.content_stride);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        if constexpr (PS == 2) {
            const u32x2 r = __builtin_bit_cast(
                u32x2, __builtin_amdgcn_raw_buffer_load_b64(rel, o.rel + j * rel_step, 0, 0));
            const u32x2 p = __builtin_bit_cast(
                u32x2, __builtin_amdgcn_raw_buffer_load_b64(ph, o.ph + 4u * j * L::kPairs, 0, 0));
            t.rel[j][0] = r.x;
            t.rel[j][1] = r.y;
            t.ph[j][0] = p.x;
            t.ph[j][1] = p.y;
        } else {
            t.rel[j][0] = __builtin_amdgcn_raw_buffer_load_b32(rel, o.rel + j * rel_step, 0, 0);
            t.ph[j][0] = __builtin_amdgcn_raw_buffer_load_b32(ph, o.ph + 4u * j * L::kPairs, 0, 0);
        }
#pragma unroll
        for (int c = 0; c < CPW; ++c) {
            t.con[j][c] = __builtin_amdgcn_raw_buffer_load_b32(con, o.con[c] + j * con_step, 0, 0);
        }
    }
}

// Rotated relation operands of a 32-token step, split into BF16 hi + lo;
// the _pair form does token pair jj (tokens 2 jj and 2 jj + 1 of the lane).
template <int R, int CPW>
__device__ __forceinline__ void reduce_relation_operands_pair(
    const ReduceTile<R, CPW>& t, int jj, u32x4 (&a_hi)[ReduceLayout<R>::kRowBlocks],
    u32x4 (&a_lo)[ReduceLayout<R>::kRowBlocks]) {
    constexpr int PS = ReduceLayout<R>::kPairSlots;
#pragma unroll
    for (int s = 0; s < PS; ++s) {
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

template <int R, int CPW>
__device__ __forceinline__ void reduce_relation_operands(const ReduceTile<R, CPW>& t,
                                                         u32x4 (&a_hi)[ReduceLayout<R>::kRowBlocks],
                                                         u32x4 (&a_lo)[ReduceLayout<R>::kRowBlocks]) {
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
        reduce_relation_operands_pair<R, CPW>(t, jj, a_hi, a_lo);
    }
}

// Content operands of a 32-token step: feature pairs de-interleaved into the
// even- and odd-feature column blocks.
template <int R, int CPW>
__device__ __forceinline__ void reduce_content_operands(const ReduceTile<R, CPW>& t,
                                                        u32x4 (&b_c)[2 * CPW]) {
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
}

// G += A^T A over the step (hi*hi + hi*lo + lo*hi, lower block triangle).
template <int R>
__device__ __forceinline__ void reduce_gram_mfma(const u32x4 (&a_hi)[ReduceLayout<R>::kRowBlocks],
                                                 const u32x4 (&a_lo)[ReduceLayout<R>::kRowBlocks],
                                                 f32x4 (&acc_g)[ReduceLayout<R>::kGramBlocks]) {
    constexpr int NRB = ReduceLayout<R>::kRowBlocks;
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

// S += A^T C over the step (C is BF16, so hi*c + lo*c is exact to FP32).
template <int R, int CPW>
__device__ __forceinline__ void reduce_cross_mfma(const u32x4 (&a_hi)[ReduceLayout<R>::kRowBlocks],
                                                  const u32x4 (&a_lo)[ReduceLayout<R>::kRowBlocks],
                                                  const u32x4 (&b_c)[2 * CPW],
                                                  f32x4 (&acc_s)[ReduceLayout<R>::kRowBlocks][2 * CPW]) {
    constexpr int NRB = ReduceLayout<R>::kRowBlocks;
#pragma unroll
    for (int x = 0; x < NRB; ++x) {
#pragma unroll
        for (int cb = 0; cb < 2 * CPW; ++cb) {
            acc_s[x][cb] = mfma16x16x32(a_hi[x], b_c[cb], acc_s[x][cb]);
            acc_s[x][cb] = mfma16x16x32(a_lo[x], b_c[cb], acc_s[x][cb]);
        }
    }
}

template <int R, int CPW>
__device__ __forceinline__ void reduce_compute(const ReduceTile<R, CPW>& t, bool do_gram,
                                               f32x4 (&acc_g)[ReduceLayout<R>::kGramBlocks],
                                               f32x4 (&acc_s)[ReduceLayout<R>::kRowBlocks][2 * CPW]) {
    constexpr int NRB = ReduceLayout<R>::kRowBlocks;
    u32x4 a_hi[NRB];
    u32x4 a_lo[NRB];
    reduce_relation_operands<R, CPW>(t, a_hi, a_lo);
    u32x4 b_c[2 * CPW];
    reduce_content_operands<R, CPW>(t, b_c);
    if (do_gram) {
        reduce_gram_mfma<R>(a_hi, a_lo, acc_g);
    }
    reduce_cross_mfma<R, CPW>(a_hi, a_lo, b_c, acc_s);
}

// Partial stores.  D layout of a 16x16 MFMA block: lane (q, g) holds rows
// 4g..4g+3 of column q.  G is written in full (both triangles).
template <int R>
__device__ __forceinline__ void store_gram_partial(float* part_g,
                                                   const f32x4 (&acc_g)[ReduceLayout<R>::kGramBlocks],
                                                   int q, int g) {
    using L = ReduceLayout<R>;
    constexpr int NRB = L::kRowBlocks;
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

template <int R, int CPW>
__device__ __forceinline__ void store_cross_partial(
    float* part_s, const f32x4 (&acc_s)[ReduceLayout<R>::kRowBlocks][2 * CPW], int q, int g,
    int64_t column_group, int64_t head_dim) {
    using L = ReduceLayout<R>;
    constexpr int NRB = L::kRowBlocks;
    // 32-bit offsets: an R x head_dim block is small, and 64-bit products
    // would be hoisted as register pairs by callers that loop.
    const int d = static_cast<int>(head_dim);
    const int feature0 = 2 * (static_cast<int>(column_group) * 16 * CPW + q);
#pragma unroll
    for (int x = 0; x < NRB; ++x) {
#pragma unroll
        for (int cb = 0; cb < 2 * CPW; ++cb) {
            const int feature = feature0 + 32 * (cb / 2) + (cb & 1);
            if (feature < d) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int m = 4 * g + i;
                    if (L::valid(x, m)) {
                        part_s[L::rank(x, m) * d + feature] = acc_s[x][cb][i];
                    }
                }
            }
        }
    }
}
}  // namespace lsso_hip

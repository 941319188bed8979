// Device-side helpers shared by the gfx950 LSSO kernels: bit-exact BF16/FP16
// conversions, MFMA operand types and the bounded complement.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace lsso_hip {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// 1 - 2^-23: the one-ULP interior scale of the complement
// (reference lsso/ball/reference.py:464, csrc/ball/common.cuh:23).
constexpr float kInteriorScale = 1.0f - 0x1.0p-23f;
// log(e - 1), rounded to float32 as torch adds the Python double to a
// float32 tensor (reference lsso/ball/reference.py:13, 493).
constexpr float kSoftplusOneOffset = 0.541324854612918f;

__device__ __forceinline__ float bf16_lo(uint32_t packed) {
    return __uint_as_float(packed << 16);
}
__device__ __forceinline__ float bf16_hi(uint32_t packed) {
    return __uint_as_float(packed & 0xffff0000u);
}
__device__ __forceinline__ float bf16_bits_to_float(uint16_t bits) {
    return __uint_as_float(static_cast<uint32_t>(bits) << 16);
}
__device__ __forceinline__ float f16_lo(uint32_t packed) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(packed & 0xffffu)));
}
__device__ __forceinline__ float f16_hi(uint32_t packed) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(packed >> 16)));
}
__device__ __forceinline__ float f16_bits_to_float(uint16_t bits) {
    return static_cast<float>(__builtin_bit_cast(_Float16, bits));
}

// The value unchanged, but opaque to the optimizer: lane-dependent offsets
// computed from it stay next to their use inside a loop instead of being
// hoisted out of it and held in registers across the whole loop.
__device__ __forceinline__ int opaque_int(int value) {
    asm volatile("" : "+v"(value));
    return value;
}

// Workgroups are dealt to the eight XCDs of an MI355X round robin (workgroup
// i runs on XCD i % 8, each XCD with its own L2).  A kernel whose
// neighbouring work items read the same rows calls this to renumber its
// workgroups so that consecutive logical blocks run on one XCD, one after
// the other: logical block xcd * (n / 8) + k is physical block 8 k + xcd.
// Blocks past the last whole round of eight keep their index.
__device__ __forceinline__ int64_t xcd_local_block(int64_t physical, int64_t blocks) {
    const int64_t per_xcd = blocks / 8;
    if (physical >= per_xcd * 8) {
        return physical;
    }
    return (physical % 8) * per_xcd + physical / 8;
}

// Raw buffer access.  An access past a buffer's num_records bytes does not
// touch memory: loads return zero and stores are dropped.  Tile loops use
// this instead of branches around their edge accesses, so every memory
// instruction issues unconditionally and the compiler's wait counts stay
// exact (a conditional access makes the waits before later uses
// conservative, which serializes a software pipeline).
typedef __amdgpu_buffer_rsrc_t BufferRsrc;
constexpr int kBufferConfig = 0x00020000;         // gfx9 raw buffer, 32-bit data format
constexpr uint32_t kOutOfRange = 0x80000000u;     // an offset past every buffer here

__device__ __forceinline__ BufferRsrc make_buffer(const void* base, int64_t bytes) {
    const int records = bytes < 0 ? 0 : (bytes > 0x7fffffff ? 0x7fffffff : static_cast<int>(bytes));
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, records, kBufferConfig);
}
__device__ __forceinline__ u32x4 buffer_load16(BufferRsrc buffer, uint32_t offset) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(buffer, offset, 0, 0));
}
__device__ __forceinline__ uint32_t buffer_load_byte(BufferRsrc buffer, uint32_t offset) {
    return __builtin_amdgcn_raw_buffer_load_b8(buffer, offset, 0, 0);
}
__device__ __forceinline__ void buffer_store16(u32x4 value, BufferRsrc buffer, uint32_t offset) {
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(__attribute__((ext_vector_type(4))) unsigned int, value),
                                           buffer, offset, 0, 0);
}
__device__ __forceinline__ void buffer_store_f32(float value, BufferRsrc buffer, uint32_t offset) {
    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(value), buffer, offset, 0, 0);
}
// Streaming forms: the cache-policy operand 2 sets the instruction's `nt`
// bit, so the lines are kept in the caches as streaming (first to be
// evicted).  Used for the bulk token tensors a kernel touches once, so
// that they do not push out what is reused (weights, phase tables,
// partials, records, and the second head group's read of an x tile).  The
// store adds `sc1` (operand 16): a streaming write of 1 GiB with `nt` alone
// runs about 5% slower than a plain one, with `nt` and `sc1` as fast.
__device__ __forceinline__ u32x4 buffer_load16_stream(BufferRsrc buffer, uint32_t offset) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(buffer, offset, 0, 2));
}
__device__ __forceinline__ void buffer_store16_stream(u32x4 value, BufferRsrc buffer, uint32_t offset) {
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(__attribute__((ext_vector_type(4))) unsigned int, value),
                                           buffer, offset, 0, 2 | 16);
}

// Round two floats to BF16 (round to nearest even, v_cvt_pk_bf16_f32) and
// pack them, first value in the low half.
__device__ __forceinline__ uint32_t pack_bf16(float low, float high) {
    const bf16x2 value = __builtin_convertvector((f32x2){low, high}, bf16x2);
    return __builtin_bit_cast(uint32_t, value);
}
__device__ __forceinline__ uint16_t to_bf16_bits(float value) {
    return static_cast<uint16_t>(pack_bf16(value, 0.0f) & 0xffffu);
}
__device__ __forceinline__ uint16_t to_f16_bits(float value) {
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(value));
}
__device__ __forceinline__ uint32_t pack_f16(float low, float high) {
    return static_cast<uint32_t>(to_f16_bits(low)) |
           (static_cast<uint32_t>(to_f16_bits(high)) << 16);
}

// Split two floats into BF16 high parts and BF16 residuals so that
// hi + lo carries ~16 mantissa bits; products of split operands accumulated
// as hi*hi + hi*lo + lo*hi reproduce FP32 products to ~2^-17 relative.
__device__ __forceinline__ void split_bf16(float a, float b, uint32_t& hi, uint32_t& lo) {
    hi = pack_bf16(a, b);
    lo = pack_bf16(a - bf16_lo(hi), b - bf16_hi(hi));
}

__device__ __forceinline__ f32x4 mfma16x16x32(const u32x4& a, const u32x4& b, const f32x4& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(
        __builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma16x16x16(const u32x2& a, const u32x2& b, const f32x4& c) {
    typedef short s16x4 __attribute__((ext_vector_type(4)));
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(
        __builtin_bit_cast(s16x4, a), __builtin_bit_cast(s16x4, b), c, 0, 0, 0);
}
__device__ __forceinline__ f32x16 mfma32x32x16(const u32x4& a, const u32x4& b, const f32x16& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(
        __builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

// eta = (1 - 2^-23) tanh(raw) through the sign-split logistic identity
// (reference lsso/ball/reference.py:450-471).
__device__ __forceinline__ float bounded_complement(float raw) {
    const bool positive = raw >= 0.0f;
    const float exponent = positive ? expf(-2.0f * raw) : expf(2.0f * raw);
    const float numerator = positive ? 1.0f - exponent : exponent - 1.0f;
    return kInteriorScale * (numerator / (1.0f + exponent));
}

// d eta / d raw of bounded_complement (reference csrc/ball/common.cuh:30-34).
__device__ __forceinline__ float bounded_complement_derivative(float raw) {
    const float exponent = raw >= 0.0f ? expf(-2.0f * raw) : expf(2.0f * raw);
    const float denominator = 1.0f + exponent;
    return kInteriorScale * 4.0f * exponent / (denominator * denominator);
}

// torch.nn.functional.softplus with beta=1, threshold=20.
__device__ __forceinline__ float softplus_one(float raw) {
    const float shifted = raw + kSoftplusOneOffset;
    return shifted > 20.0f ? shifted : log1pf(expf(shifted));
}

// Rotate one (even, odd) relation pair by an FP16 (cos, sin) phase.  The
// BF16 x FP16 products are exact in FP32, so the one rounding of each sum
// matches the reference's FP32 rotation (reference.py:719-723).
__device__ __forceinline__ void rotate_pair(uint32_t relation_pair, uint32_t phase,
                                            float& even_out, float& odd_out) {
    const float even = bf16_lo(relation_pair);
    const float odd = bf16_hi(relation_pair);
    const float cosine = f16_lo(phase);
    const float sine = f16_hi(phase);
    even_out = even * cosine - odd * sine;
    odd_out = even * sine + odd * cosine;
}

// Apply operand layout: the rank dimension is the MFMA K index.  Ranks that
// are multiples of 32 use K32 steps (16x16x32; lane group g holds ranks
// base + 8g .. +7), the others K16 steps (16x16x16; ranks base + 4g .. +3).
// One accumulation chain never mixes the two MFMA shapes: a 16x16x32 result
// consumed as SrcC of a 16x16x16 produced wrong accumulators on gfx950 with
// this toolchain.  Per lane the M' operand holds, per step, the hi values
// followed by the lo values.
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

// Resident BF16 row of an FP32 weight [N, K] for y^T = W x^T on
// v_mfma_f32_32x32x16_bf16: the lane holds row n (zeros when n < 0) at
// columns 16 ks + 8 (lane / 32) + 0..7, RNE-rounded, zero past K.  Rows are
// read as float4 pairs when K is a multiple of 4.
template <int KSTEPS>
__device__ __forceinline__ void load_weight_row(u32x4 (&wreg)[KSTEPS], const float* weight,
                                                int64_t n, int64_t K, int lane, int64_t k_base = 0) {
    const int half = lane >> 5;
    const bool nv = n >= 0;
    const float* wrow = weight + (nv ? n : 0) * K;
    const bool vector_rows = (K % 4) == 0;
#pragma unroll
    for (int ks = 0; ks < KSTEPS; ++ks) {
        const int64_t k0 = k_base + 16 * ks + 8 * half;
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

// load_weight_row for K a multiple of 8, through one raw buffer over the
// whole [N, K] weight (wave-uniform descriptor, per-lane offsets; a row
// n < 0 and columns past K read as zeros): no per-element fallback, so
// loading several rows keeps no address registers alive.
template <int KSTEPS>
__device__ __forceinline__ void load_weight_row_k8(u32x4 (&wreg)[KSTEPS], const float* weight,
                                                   int64_t n, int64_t N, int64_t K, int lane) {
    const int half = lane >> 5;
    const BufferRsrc buffer = make_buffer(weight, 4 * N * K);
    const uint32_t row = n >= 0 ? static_cast<uint32_t>(4 * n * K) : kOutOfRange;
#pragma unroll
    for (int ks = 0; ks < KSTEPS; ++ks) {
        const uint32_t k0 = 16 * ks + 8 * half;
        const bool live = n >= 0 && k0 < K;
        const f32x4 lo = __builtin_bit_cast(f32x4, buffer_load16(buffer, live ? row + 4 * k0 : kOutOfRange));
        const f32x4 hi = __builtin_bit_cast(f32x4, buffer_load16(buffer, live ? row + 4 * k0 + 16 : kOutOfRange));
        wreg[ks][0] = pack_bf16(lo[0], lo[1]);
        wreg[ks][1] = pack_bf16(lo[2], lo[3]);
        wreg[ks][2] = pack_bf16(hi[0], hi[1]);
        wreg[ks][3] = pack_bf16(hi[2], hi[3]);
        // One K step at a time, so the FP32 staging of the whole row is never
        // live at once.
        __builtin_amdgcn_sched_barrier(0);
    }
}

// Resident slice of rows n0 .. n0 + 31 (one row per lane % 32), columns
// k_base .. k_base + 16 KSTEPS.
template <int KSTEPS>
__device__ __forceinline__ void load_weight_slice(u32x4 (&wreg)[KSTEPS], const float* weight,
                                                  int64_t N, int64_t K, int64_t n0, int lane,
                                                  int64_t k_base = 0) {
    const int64_t n = n0 + (lane & 31);
    load_weight_row<KSTEPS>(wreg, weight, n < N ? n : -1, K, lane, k_base);
}

}  // namespace lsso_hip

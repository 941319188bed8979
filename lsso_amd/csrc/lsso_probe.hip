// gfx950 HBM probes for the benchmark: the rate a plain streaming kernel
// reaches on this device, which is the practical ceiling the library's
// streaming kernels are compared with.  Not part of the mixer's C ABI
// (include/lsso_hip.h); built as its own library, liblsso_probe_gfx950.so.
//
// Each thread moves one 16-byte vector, 256 threads per workgroup: the
// launch holds as many independent loads in flight as the device can
// schedule, which measured faster than persistent or unrolled copies.

#include <hip/hip_runtime.h>

#include <cstdint>

namespace {

typedef uint32_t probe_u32x4 __attribute__((ext_vector_type(4)));

constexpr int kProbeThreads = 256;

template <bool STREAMING>
__global__ __launch_bounds__(kProbeThreads) void probe_copy_kernel(const probe_u32x4* __restrict__ src,
                                                                    probe_u32x4* __restrict__ dst) {
    const size_t i = static_cast<size_t>(blockIdx.x) * kProbeThreads + threadIdx.x;
    if constexpr (STREAMING) {
        __builtin_nontemporal_store(__builtin_nontemporal_load(&src[i]), &dst[i]);
    } else {
        dst[i] = src[i];
    }
}

__global__ __launch_bounds__(kProbeThreads) void probe_read_kernel(const probe_u32x4* __restrict__ src,
                                                                   uint32_t* __restrict__ sink) {
    const size_t i = static_cast<size_t>(blockIdx.x) * kProbeThreads + threadIdx.x;
    const probe_u32x4 v = src[i];
    const uint32_t folded = v.x ^ v.y ^ v.z ^ v.w;
    // A store that never happens for the filled test data (all bytes equal,
    // so the fold is zero) keeps the load live without write traffic.
    if (folded == 0x9e3779b9u) {
        sink[0] = folded;
    }
}

__global__ __launch_bounds__(kProbeThreads) void probe_write_kernel(probe_u32x4* __restrict__ dst) {
    const size_t i = static_cast<size_t>(blockIdx.x) * kProbeThreads + threadIdx.x;
    dst[i] = (probe_u32x4){static_cast<uint32_t>(i), 0u, 0u, 0u};
}

// The same write through a raw buffer store whose cache-policy operand is
// POLICY (2 = nt, 16 = sc1), one 4 KiB buffer per workgroup.
template <int POLICY>
__global__ __launch_bounds__(kProbeThreads) void probe_write_policy_kernel(probe_u32x4* __restrict__ dst) {
    const __amdgpu_buffer_rsrc_t buffer = __builtin_amdgcn_make_buffer_rsrc(
        dst + static_cast<size_t>(blockIdx.x) * kProbeThreads, 0, 16 * kProbeThreads, 0x00020000);
    const probe_u32x4 value = {blockIdx.x * kProbeThreads + threadIdx.x, 0u, 0u, 0u};
    __builtin_amdgcn_raw_buffer_store_b128(value, buffer, 16u * threadIdx.x, 0, POLICY);
}

// Shader clock of the moment: one lane runs `spins` dependent FMAs between
// two reads of the shader-clock counter (s_memtime) and of the constant-rate
// counter (s_memrealtime, hipDeviceAttributeWallClockRate), and stores both
// differences in record[0] and record[1] (record[2] keeps the chain's value
// live).  The ratio times the constant rate is the clock the probe ran at.
__global__ __launch_bounds__(64) void probe_clock_kernel(uint64_t* __restrict__ record, int spins) {
    if (threadIdx.x != 0) {
        return;
    }
    const uint64_t clock0 = clock64();
    const uint64_t wall0 = wall_clock64();
    float chain = 1.0f;
    for (int i = 0; i < spins; ++i) {
        chain = __builtin_fmaf(chain, 1.0000001f, 1.0e-7f);
    }
    const uint64_t clock1 = clock64();
    const uint64_t wall1 = wall_clock64();
    record[0] = clock1 - clock0;
    record[1] = wall1 - wall0;
    record[2] = static_cast<uint64_t>(chain > 2.0f);
}

constexpr uint64_t kProbeGranule = 16u * kProbeThreads;

bool probe_size_ok(uint64_t bytes) {
    return bytes > 0 && bytes % kProbeGranule == 0 && bytes / kProbeGranule <= 0x7fffffffu;
}

}  // namespace

extern "C" {

// Copies `bytes` (a multiple of 4,096, both buffers 16-byte aligned) from
// src to dst on `stream`.  streaming != 0 sets the nontemporal hint on the
// loads and stores.  Returns 0 or a hipError_t code; 22 (EINVAL) for a size
// or alignment it does not take.
int lsso_probe_copy(const void* src, void* dst, uint64_t bytes, int streaming, hipStream_t stream) {
    if (!probe_size_ok(bytes) || src == nullptr || dst == nullptr ||
        reinterpret_cast<uintptr_t>(src) % 16 != 0 || reinterpret_cast<uintptr_t>(dst) % 16 != 0) {
        return 22;
    }
    const dim3 grid(static_cast<unsigned>(bytes / kProbeGranule));
    const auto* s = static_cast<const probe_u32x4*>(src);
    auto* d = static_cast<probe_u32x4*>(dst);
    if (streaming != 0) {
        hipLaunchKernelGGL(probe_copy_kernel<true>, grid, dim3(kProbeThreads), 0, stream, s, d);
    } else {
        hipLaunchKernelGGL(probe_copy_kernel<false>, grid, dim3(kProbeThreads), 0, stream, s, d);
    }
    return static_cast<int>(hipGetLastError());
}

// Reads `bytes` of src; `sink` (4 bytes) is written only if the data folds
// to a fixed odd value, which a buffer filled with one byte value never does.
int lsso_probe_read(const void* src, void* sink, uint64_t bytes, hipStream_t stream) {
    if (!probe_size_ok(bytes) || src == nullptr || sink == nullptr ||
        reinterpret_cast<uintptr_t>(src) % 16 != 0) {
        return 22;
    }
    hipLaunchKernelGGL(probe_read_kernel, dim3(static_cast<unsigned>(bytes / kProbeGranule)),
                       dim3(kProbeThreads), 0, stream, static_cast<const probe_u32x4*>(src),
                       static_cast<uint32_t*>(sink));
    return static_cast<int>(hipGetLastError());
}

// Writes `bytes` of dst with the buffer-store cache-policy operand `policy`
// (0, 2 = nt, 16 = sc1 or 18 = both); 22 (EINVAL) for another value.
int lsso_probe_write_policy(void* dst, uint64_t bytes, int policy, hipStream_t stream) {
    if (!probe_size_ok(bytes) || dst == nullptr || reinterpret_cast<uintptr_t>(dst) % 16 != 0) {
        return 22;
    }
    const dim3 grid(static_cast<unsigned>(bytes / kProbeGranule));
    auto* d = static_cast<probe_u32x4*>(dst);
    switch (policy) {
        case 0: hipLaunchKernelGGL(probe_write_policy_kernel<0>, grid, dim3(kProbeThreads), 0, stream, d); break;
        case 2: hipLaunchKernelGGL(probe_write_policy_kernel<2>, grid, dim3(kProbeThreads), 0, stream, d); break;
        case 16: hipLaunchKernelGGL(probe_write_policy_kernel<16>, grid, dim3(kProbeThreads), 0, stream, d); break;
        case 18: hipLaunchKernelGGL(probe_write_policy_kernel<18>, grid, dim3(kProbeThreads), 0, stream, d); break;
        default: return 22;
    }
    return static_cast<int>(hipGetLastError());
}

// One probe_clock_kernel launch writing three uint64 values at record
// (8-byte aligned); `spins` in [1, 1 << 20].  Returns 0, 22 (EINVAL) for an
// argument it does not take, or a hipError_t code.
int lsso_probe_clock(void* record, int spins, hipStream_t stream) {
    if (record == nullptr || reinterpret_cast<uintptr_t>(record) % 8 != 0 || spins < 1 || spins > (1 << 20)) {
        return 22;
    }
    hipLaunchKernelGGL(probe_clock_kernel, dim3(1), dim3(64), 0, stream, static_cast<uint64_t*>(record), spins);
    return static_cast<int>(hipGetLastError());
}

// The constant counter's rate in kHz (hipDeviceAttributeWallClockRate of
// the current device), or a negative hipError_t code.
int lsso_probe_wall_clock_khz(void) {
    int device = 0;
    int rate = 0;
    hipError_t status = hipGetDevice(&device);
    if (status == hipSuccess) {
        status = hipDeviceGetAttribute(&rate, hipDeviceAttributeWallClockRate, device);
    }
    return status == hipSuccess ? rate : -static_cast<int>(status);
}

// Writes `bytes` of dst.
int lsso_probe_write(void* dst, uint64_t bytes, hipStream_t stream) {
    if (!probe_size_ok(bytes) || dst == nullptr || reinterpret_cast<uintptr_t>(dst) % 16 != 0) {
        return 22;
    }
    hipLaunchKernelGGL(probe_write_kernel, dim3(static_cast<unsigned>(bytes / kProbeGranule)),
                       dim3(kProbeThreads), 0, stream, static_cast<probe_u32x4*>(dst));
    return static_cast<int>(hipGetLastError());
}

}  // extern "C"

/*
 * k_synth.hip — device fills for the deterministic synthetic inputs of
 * include/apus_synth.h (integer-only, so the bytes equal the host
 * generator's), plus a small u32 fill used instead of memsets in
 * stream-ordered paths.
 */
#include "ghip_device.h"
#include "ghip_internal.h"

__device__ __forceinline__ uint64_t sy_mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

__device__ __forceinline__ uint64_t sy_u64(uint64_t key, uint64_t i) {
    return sy_mix64(key + (i + 1) * 0x9E3779B97F4A7C15ull);
}

/* 16 codes per thread: code = r < 127 ? r : r + 1, r = u64 % 254. */
__global__ __launch_bounds__(256) void k_synth_codes(uint8_t *out, size_t n,
                                                     uint64_t key, uint64_t offset) {
    const size_t nv = (n + 15) >> 4;
    for (size_t v = (size_t)blockIdx.x * 256 + threadIdx.x; v < nv;
         v += (size_t)gridDim.x * 256) {
        size_t i0 = v << 4;
        if (i0 + 16 <= n && ((uintptr_t)(out + i0) & 15) == 0) {
            ghip_u32x4 w = {0u, 0u, 0u, 0u};
#pragma unroll
            for (int j = 0; j < 16; j++) {
                uint32_t r = (uint32_t)(sy_u64(key, offset + i0 + j) % 254ull);
                uint32_t c = r < 127u ? r : r + 1u;
                w[j >> 2] |= c << (8 * (j & 3));
            }
            *(ghip_u32x4 *)(out + i0) = w;
        } else {
            for (size_t i = i0; i < n && i < i0 + 16; i++) {
                uint32_t r = (uint32_t)(sy_u64(key, offset + i) % 254ull);
                out[i] = (uint8_t)(r < 127u ? r : r + 1u);
            }
        }
    }
}

__global__ __launch_bounds__(256) void k_synth_bf16(uint16_t *out, size_t n,
                                                    uint64_t key, uint64_t offset,
                                                    const uint16_t *table) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n;
         i += (size_t)gridDim.x * 256)
        out[i] = table[sy_u64(key, offset + i) >> 48];
}

__global__ __launch_bounds__(256) void k_fill_u32(uint32_t *p, size_t n,
                                                  uint32_t value) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n;
         i += (size_t)gridDim.x * 256)
        p[i] = value;
}

static uint32_t sy_grid(size_t items) {
    size_t g = (items + 255) / 256;
    if (g < 1) g = 1;
    if (g > 65536) g = 65536;
    return (uint32_t)g;
}

extern "C" hipError_t ghip_launch_synth_codes(uint8_t *out, size_t n,
                                              uint64_t key, uint64_t offset,
                                              hipStream_t st) {
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(k_synth_codes, dim3(sy_grid((n + 15) / 16)), dim3(256), 0,
                       st, out, n, key, offset);
    return hipGetLastError();
}

extern "C" hipError_t ghip_launch_synth_bf16(uint16_t *out, size_t n,
                                             uint64_t key, uint64_t offset,
                                             const uint16_t *table,
                                             hipStream_t st) {
    if (n == 0) return hipSuccess;
    if (!table) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_synth_bf16, dim3(sy_grid(n)), dim3(256), 0, st, out, n,
                       key, offset, table);
    return hipGetLastError();
}

extern "C" hipError_t ghip_launch_fill_u32(uint32_t *p, size_t n, uint32_t value,
                                           hipStream_t st) {
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(k_fill_u32, dim3(sy_grid(n)), dim3(256), 0, st, p, n, value);
    return hipGetLastError();
}

/* One wave that waits `ticks` of the constant-rate wall clock and exits:
 * holds a stream for a fixed time with no memory traffic (a bounded wait:
 * every launch ends). */
__global__ __launch_bounds__(64) void k_hold(unsigned long long ticks) {
    const unsigned long long t0 = (unsigned long long)wall_clock64();
    while ((unsigned long long)wall_clock64() - t0 < ticks) __builtin_amdgcn_s_sleep(64);
}

extern "C" hipError_t ghip_launch_hold(uint64_t ticks, hipStream_t st) {
    hipLaunchKernelGGL(k_hold, dim3(1), dim3(64), 0, st, (unsigned long long)ticks);
    return hipGetLastError();
}

// convert_probe.hip - test-side probe of the handoff kernels' binary32 <-> binary16 conversions and arithmetic
// shortcuts.
//
// Runs sc_convert.hpp's f16_bits_rne over any range of binary32 bit patterns and f32_of_f16 over all 2^16 binary16
// patterns, on the device, so the test suite can compare every result with the CPU oracle; runs sc_arith.hpp's
// recip_rn and div127 over any range of inputs, both as values (for the CPU) and as a device-side count of the
// inputs where they differ from the IEEE division (this probe is built with correctly rounded f32 division).  Not
// part of the library.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "sc_arith.hpp"
#include "sc_convert.hpp"

namespace {

__global__ void f16_of_f32_kernel(uint32_t lo, uint64_t n, uint16_t* out) {
    for (uint64_t i = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += uint64_t(gridDim.x) * blockDim.x)
        out[i] = uint16_t(sc::f16_bits_rne(uint32_t(lo + i)));
}

// mode 0: recip_normal(d) vs 1.0f / d where recip_normal_ok(d); mode 1: div127(|a|) vs |a| / 127.0f (NaN inputs
// skipped; -0 counted as +0).
// Mismatches are counted in count[0]; the first few inputs that differ land in first[0..7] (slot by atomic index).
__global__ void arith_check_kernel(uint32_t lo, uint64_t n, int mode, unsigned long long* count, uint32_t* first) {
    for (uint64_t i = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += uint64_t(gridDim.x) * blockDim.x) {
        const uint32_t u = uint32_t(lo + i);
        const float x = __uint_as_float(u);
        if (x != x) continue;
        float got, want;
        if (mode == 0) {
            if (!sc::recip_normal_ok(x)) continue;
            got = sc::recip_normal(x);
            want = 1.0f / x;
        } else {
            const float a = __builtin_fabsf(x);
            got = sc::div127(a);
            want = a / 127.0f;
        }
        if (__float_as_uint(got) != __float_as_uint(want)) {
            const unsigned long long k = atomicAdd(count, 1ull);
            if (k < 8) first[k] = u;
        }
    }
}

__global__ void recip_kernel(uint32_t lo, uint64_t n, uint32_t* out) {
    for (uint64_t i = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += uint64_t(gridDim.x) * blockDim.x)
        out[i] = __float_as_uint(sc::recip_normal(__uint_as_float(uint32_t(lo + i))));
}

__global__ void f32_of_f16_kernel(uint32_t* out) {
    const uint32_t h = blockIdx.x * blockDim.x + threadIdx.x;
    if (h < 65536u) out[h] = __float_as_uint(sc::f32_of_f16(h));
}

}  // namespace

// Converts the n binary32 patterns lo, lo + 1, ... (lo + n <= 2^32) into host_out[n]; 0 on success.
extern "C" int probe_f16_of_f32(uint32_t lo, uint64_t n, uint16_t* host_out) {
    if (n == 0) return 0;
    if (!host_out || uint64_t(lo) + n > (uint64_t(1) << 32)) return -1;
    uint16_t* dev = nullptr;
    if (hipMalloc(&dev, n * sizeof(uint16_t)) != hipSuccess) return -2;
    hipLaunchKernelGGL(f16_of_f32_kernel, dim3(8192), dim3(256), 0, 0, lo, n, dev);
    hipError_t e = hipGetLastError();
    if (e == hipSuccess) e = hipMemcpy(host_out, dev, n * sizeof(uint16_t), hipMemcpyDeviceToHost);
    (void) hipFree(dev);
    return e == hipSuccess ? 0 : -3;
}

// Converts all 2^16 binary16 patterns into host_out[65536] (binary32 bits); 0 on success.
extern "C" int probe_f32_of_f16(uint32_t* host_out) {
    if (!host_out) return -1;
    uint32_t* dev = nullptr;
    if (hipMalloc(&dev, 65536 * sizeof(uint32_t)) != hipSuccess) return -2;
    hipLaunchKernelGGL(f32_of_f16_kernel, dim3(256), dim3(256), 0, 0, dev);
    hipError_t e = hipGetLastError();
    if (e == hipSuccess) e = hipMemcpy(host_out, dev, 65536 * sizeof(uint32_t), hipMemcpyDeviceToHost);
    (void) hipFree(dev);
    return e == hipSuccess ? 0 : -3;
}

// Counts the inputs lo .. lo + n - 1 where the shortcut (mode 0 recip_normal, mode 1 div127) differs from the IEEE
// division on the device; *count and first[8] on the host.  0 on success.
extern "C" int probe_arith_mismatches(uint32_t lo, uint64_t n, int mode, unsigned long long* count, uint32_t* first) {
    if (!count || !first || uint64_t(lo) + n > (uint64_t(1) << 32) || (mode != 0 && mode != 1)) return -1;
    void* dev = nullptr;
    if (hipMalloc(&dev, 64) != hipSuccess) return -2;
    hipError_t e = hipMemset(dev, 0, 64);
    auto* c = static_cast<unsigned long long*>(dev);
    auto* f = reinterpret_cast<uint32_t*>(static_cast<uint8_t*>(dev) + 16);
    if (e == hipSuccess && n) {
        hipLaunchKernelGGL(arith_check_kernel, dim3(16384), dim3(256), 0, 0, lo, n, mode, c, f);
        e = hipGetLastError();
    }
    if (e == hipSuccess) e = hipMemcpy(count, c, 8, hipMemcpyDeviceToHost);
    if (e == hipSuccess) e = hipMemcpy(first, f, 32, hipMemcpyDeviceToHost);
    (void) hipFree(dev);
    return e == hipSuccess ? 0 : -3;
}

// recip_normal of the n binary32 patterns lo, lo + 1, ... into host_out[n] (bits); 0 on success.
extern "C" int probe_recip(uint32_t lo, uint64_t n, uint32_t* host_out) {
    if (n == 0) return 0;
    if (!host_out || uint64_t(lo) + n > (uint64_t(1) << 32)) return -1;
    uint32_t* dev = nullptr;
    if (hipMalloc(&dev, n * sizeof(uint32_t)) != hipSuccess) return -2;
    hipLaunchKernelGGL(recip_kernel, dim3(8192), dim3(256), 0, 0, lo, n, dev);
    hipError_t e = hipGetLastError();
    if (e == hipSuccess) e = hipMemcpy(host_out, dev, n * sizeof(uint32_t), hipMemcpyDeviceToHost);
    (void) hipFree(dev);
    return e == hipSuccess ? 0 : -3;
}

// convert_probe.hip - test-side probe of the handoff kernels' binary32 <-> binary16 conversions.
//
// Runs sc_convert.hpp's f16_bits_rne over any range of binary32 bit patterns and f32_of_f16 over all 2^16 binary16
// patterns, on the device, so the test suite can compare every result with the CPU oracle.  Not part of the library.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "sc_convert.hpp"

namespace {

__global__ void f16_of_f32_kernel(uint32_t lo, uint64_t n, uint16_t* out) {
    for (uint64_t i = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += uint64_t(gridDim.x) * blockDim.x)
        out[i] = uint16_t(sc::f16_bits_rne(uint32_t(lo + i)));
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

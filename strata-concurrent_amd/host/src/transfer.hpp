// transfer.hpp - how the host layer moves bytes: every copy of one public call is enqueued on this thread's
// transfer stream (a non-blocking HIP stream owned by libsc_handoff.so) and the call waits once at its end.
#pragma once

#include <cstddef>
#include <string>

namespace strata::core::detail {

/// Enqueues a copy of n bytes (any direction: device, pinned or pageable host).  False + error on failure.
bool enqueue_copy(void* dst, const void* src, size_t n, std::string& error, const char* what);
/// Waits for this thread's transfer stream.
bool finish_transfers(std::string& error, const char* what);
/// Waits for the whole device (the reference's sync before save and after restore).
bool device_synchronize(std::string& error, const char* what);
/// The transfer stream (a hipStream_t), created on first use; null when it cannot be created.
void* transfer_stream();
/// The last C-ABI error message.
std::string abi_error();

/// Makes `device` current for a scope (-1 or the current device: nothing), restoring the caller's after it.
struct OnDevice {
    int previous = -1;
    explicit OnDevice(int device);
    ~OnDevice();
    OnDevice(const OnDevice&) = delete;
    OnDevice& operator=(const OnDevice&) = delete;
};

}  // namespace strata::core::detail

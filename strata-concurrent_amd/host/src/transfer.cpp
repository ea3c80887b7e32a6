// transfer.cpp - the host layer's copies and synchronization, all through libsc_handoff.so's C-ABI.
#include "transfer.hpp"

#include "sc_handoff.h"

namespace strata::core::detail {

namespace {
// One transfer stream per thread: the engine thread and a handoff thread (the reference runs a cross-process
// copy-out on its own thread) never serialize on each other's copies.
struct ThreadStream {
    void* stream = nullptr;
    bool tried = false;
    ~ThreadStream() {
        if (stream) sc_stream_destroy(stream);
    }
};
thread_local ThreadStream t_stream;
}  // namespace

std::string abi_error() { return sc_last_error(); }

void* transfer_stream() {
    if (!t_stream.tried) {
        t_stream.tried = true;
        if (sc_stream_create(&t_stream.stream) != SC_OK) t_stream.stream = nullptr;
    }
    return t_stream.stream;
}

bool enqueue_copy(void* dst, const void* src, size_t n, std::string& error, const char* what) {
    if (!n) return true;
    void* s = transfer_stream();
    if (!s) {
        error = std::string(what) + ": " + abi_error();
        return false;
    }
    if (sc_copy_async(dst, src, n, s) == SC_OK) return true;
    error = std::string(what) + ": " + abi_error();
    return false;
}

bool finish_transfers(std::string& error, const char* what) {
    void* s = t_stream.stream;
    if (!s || sc_stream_sync(s) == SC_OK) return true;
    error = std::string(what) + ": " + abi_error();
    return false;
}

bool device_synchronize(std::string& error, const char* what) {
    if (sc_device_sync() == SC_OK) return true;
    error = std::string(what) + ": " + abi_error();
    return false;
}

OnDevice::OnDevice(int device) {
    int cur = 0;
    if (device >= 0 && sc_get_device(&cur) == SC_OK && cur != device && sc_set_device(device) == SC_OK) previous = cur;
}
OnDevice::~OnDevice() {
    if (previous >= 0) sc_set_device(previous);
}

}  // namespace strata::core::detail

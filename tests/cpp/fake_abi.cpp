// fake_abi.cpp - a host-memory stand-in for libsc_handoff.so's runtime plumbing, for CPU tests of the C++ host
// layer.  TEST INFRASTRUCTURE ONLY: never linked into the product.  It plays the role the reference's
// link-wrapped cudaMemcpy plays in its host-only validation test (src/core/conversation_validation_test.cpp:15-33):
// copies are memcpy, and a countdown can make the Nth copy or synchronization fail, so the control flow of
// "refuse before any write" and "transfer_failed after a write" runs without a GPU.
#include "sc_handoff.h"

#include <cstdlib>
#include <cstring>
#include <string>

namespace fake {
int copy_calls = 0, sync_calls = 0, fail_copy = 0, fail_sync = 0, movers = 0;
size_t copied_bytes = 0;
void reset() { copy_calls = sync_calls = fail_copy = fail_sync = movers = 0; copied_bytes = 0; }
}  // namespace fake

namespace {
thread_local std::string g_error;
int failed(const char* what) { g_error = what; return SC_EHIP; }
int stream_token;
}  // namespace

extern "C" {
const char* sc_last_error(void) { return g_error.c_str(); }
int sc_copy_async(void* dst, const void* src, uint64_t n, void*) {
    if (++fake::copy_calls == fake::fail_copy) return failed("injected copy failure");
    fake::copied_bytes += n;
    std::memcpy(dst, src, n);
    return SC_OK;
}
int sc_stream_create(void** s) { *s = &stream_token; return SC_OK; }
int sc_stream_destroy(void*) { return SC_OK; }
int sc_stream_sync(void*) { return ++fake::sync_calls == fake::fail_sync ? failed("injected sync failure") : SC_OK; }
int sc_device_sync(void) { return ++fake::sync_calls == fake::fail_sync ? failed("injected sync failure") : SC_OK; }
int sc_get_device(int* d) { *d = 0; return SC_OK; }
int sc_set_device(int) { return SC_OK; }
int sc_host_alloc(void**, uint64_t) { return failed("no pinned memory in the fake"); }
int sc_host_free(void*) { return SC_OK; }
int sc_kv_ring_restore(const sc_kv_runs*, int64_t, int64_t, int64_t, void*) { ++fake::movers; return SC_OK; }
int sc_kv_stage_from_host(const sc_kv_runs*, int64_t, void*) { ++fake::movers; return SC_OK; }
int sc_kv_ring_table(int32_t*, int64_t, int64_t, void*) { return SC_OK; }
// the prefill appends are device kernels with no host stand-in: a host-only program that reaches one is refused
int sc_kv_append_async(const float*, const float*, int64_t, int64_t, const int32_t*, int64_t, uint16_t*, uint16_t*,
                       int8_t*, int8_t*, uint16_t*, uint16_t*, void*, const sc_kv_pools*, const sc_kv_pools*) {
    return failed("kv_append runs on the device only");
}
int sc_kv_append_q4_async(uint8_t*, uint8_t*, const int32_t*, int64_t, int64_t, const float*, const float*, int64_t,
                          int64_t, int64_t, void*, const sc_kv_pools*, const sc_kv_pools*) {
    return failed("kv_append_q4 runs on the device only");
}
int sc_kv_stream_reset(int32_t*, int64_t, int32_t*, int32_t*, int32_t*, int64_t, int32_t*, void*) { ++fake::movers; return SC_OK; }
uint64_t sc_kv_block_bytes(int64_t h, int64_t d, int64_t ps, int32_t) { return uint64_t(h * d * ps * 4); }
}

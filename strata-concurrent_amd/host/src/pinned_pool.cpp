// pinned_pool.cpp - pinned host memory for ConversationBuffer segments.
//
// hipHostMalloc is slow (it maps and locks pages), so a park must not call it per segment.  Segments of 1 MiB or
// more take a block from a size class (1, 2, 4, 8 or 16 MiB, the next power of two at or above the segment's
// capacity); a class refills by carving a 64 MiB pinned arena into blocks, and released blocks return to their
// class's free list for the next park.  Arenas live until the process ends.  Smaller segments, and any segment
// when pinned memory cannot be had (no device, or the pool disabled), are heap memory.
#include "strata/core/conversation_buffer.hpp"

#include "sc_handoff.h"

#include <array>
#include <atomic>
#include <cstdlib>
#include <mutex>
#include <new>
#include <vector>

namespace strata::core {
namespace {

constexpr size_t kMinPinned = size_t(1) << 20;
constexpr size_t kMaxPinned = ConversationBuffer::segment_bytes;
constexpr size_t kArenaBytes = size_t(64) << 20;
constexpr int kClasses = 5;   // 1, 2, 4, 8, 16 MiB

int class_of(size_t capacity) {
    int c = 0;
    size_t size = kMinPinned;
    while (size < capacity) { size <<= 1; ++c; }
    return c;
}
size_t class_bytes(int c) { return kMinPinned << c; }

struct Pool {
    std::mutex mutex;
    std::array<std::vector<void*>, kClasses> free;
    size_t held = 0;         // bytes of pinned arenas
    bool broken = false;     // pinned allocation failed once: stop trying
};

Pool& pool() {
    static Pool* p = new Pool();   // never destroyed: blocks may be released during static destruction
    return *p;
}

std::atomic<bool> g_enabled{true};

}  // namespace

void conversation_pinned_segments(bool enabled) { g_enabled.store(enabled); }

size_t conversation_pinned_pool_bytes() {
    Pool& p = pool();
    std::lock_guard<std::mutex> lock(p.mutex);
    return p.held;
}

namespace detail {

void* segment_allocate(size_t capacity, bool& pinned) {
    pinned = false;
    if (capacity >= kMinPinned && capacity <= kMaxPinned && g_enabled.load()) {
        Pool& p = pool();
        std::lock_guard<std::mutex> lock(p.mutex);
        const int c = class_of(capacity);
        if (p.free[c].empty() && !p.broken) {
            void* arena = nullptr;
            if (sc_host_alloc(&arena, kArenaBytes) == SC_OK) {
                p.held += kArenaBytes;
                for (size_t at = 0; at + class_bytes(c) <= kArenaBytes; at += class_bytes(c))
                    p.free[c].push_back(static_cast<uint8_t*>(arena) + at);
            } else {
                p.broken = true;
            }
        }
        if (!p.free[c].empty()) {
            void* block = p.free[c].back();
            p.free[c].pop_back();
            pinned = true;
            return block;
        }
    }
    void* block = std::malloc(capacity);
    if (!block) throw std::bad_alloc();
    return block;
}

void segment_release(void* block, size_t capacity, bool pinned) {
    if (!block) return;
    if (!pinned) {
        std::free(block);
        return;
    }
    Pool& p = pool();
    std::lock_guard<std::mutex> lock(p.mutex);
    p.free[class_of(capacity)].push_back(block);
}

}  // namespace detail
}  // namespace strata::core

// conversation_buffer.hpp - host storage for parked conversation bytes.
//
// Same interface and growth accounting as the reference's ConversationBuffer
// (include/strata/core/conversation_buffer.hpp:16-152): a directory of segments of at most 16 MiB, appends never
// move existing payload, `visit` walks the segments in order and `bytes`/`allocation_peak` report what the RAM
// budget must admit.  The difference is where the segments live: a segment of 1 MiB or more comes from a pool of
// PINNED host memory (hipHostMalloc through the library's C-ABI), so every park and resume copy of a large
// buffer is a DMA at the host link's rate instead of a staged copy through pageable memory.  Small segments,
// and every segment when pinned memory is unavailable, are ordinary heap memory.
#pragma once

#include <algorithm>
#include <cstddef>
#include <cstdint>
#include <cstring>
#include <initializer_list>
#include <utility>
#include <vector>

namespace strata::core {

namespace detail {
// Segment storage (host/src/pinned_pool.cpp).  `pinned` reports where the block came from.
void* segment_allocate(size_t capacity, bool& pinned);
void segment_release(void* block, size_t capacity, bool pinned);
}  // namespace detail

/// Enables or disables pinned segments for buffers created afterwards (enabled by default).
void conversation_pinned_segments(bool enabled);
/// Pinned bytes the segment pool holds (in use plus cached for reuse).
size_t conversation_pinned_pool_bytes();

class ConversationBuffer {
    // One segment: 24 bytes like the std::vector the reference uses, so `bytes()` accounts the same directory.
    class Segment {
    public:
        Segment() = default;
        explicit Segment(size_t capacity) { allocate(capacity); }
        Segment(const Segment& o) {
            allocate(o.size_);
            if (o.size_) std::memcpy(data_, o.data_, o.size_);
            size_ = o.size_;
        }
        Segment& operator=(const Segment& o) {
            if (this != &o) { Segment copy(o); swap(copy); }
            return *this;
        }
        Segment(Segment&& o) noexcept
            : data_(std::exchange(o.data_, nullptr)), size_(std::exchange(o.size_, 0)), cap_(std::exchange(o.cap_, 0)) {}
        Segment& operator=(Segment&& o) noexcept {
            if (this != &o) { release(); data_ = std::exchange(o.data_, nullptr); size_ = std::exchange(o.size_, 0);
                              cap_ = std::exchange(o.cap_, 0); }
            return *this;
        }
        ~Segment() { release(); }

        uint8_t* data() { return data_; }
        const uint8_t* data() const { return data_; }
        size_t size() const { return size_; }
        size_t capacity() const { return cap_ & ~kPinnedBit; }
        bool pinned() const { return (cap_ & kPinnedBit) != 0; }
        // Within the reserved capacity only; growth past it never happens (the buffer adds segments instead).
        void resize(size_t n, uint8_t value) {
            if (n > size_) std::memset(data_ + size_, value, n - size_);
            size_ = n;
        }

    private:
        static constexpr size_t kPinnedBit = size_t(1) << 63;
        void allocate(size_t capacity) {
            if (!capacity) return;
            bool pinned = false;
            data_ = static_cast<uint8_t*>(detail::segment_allocate(capacity, pinned));
            cap_ = capacity | (pinned ? kPinnedBit : 0);
        }
        void release() {
            if (data_) detail::segment_release(data_, capacity(), pinned());
            data_ = nullptr;
            size_ = cap_ = 0;
        }
        void swap(Segment& o) noexcept { std::swap(data_, o.data_); std::swap(size_, o.size_); std::swap(cap_, o.cap_); }

        uint8_t* data_ = nullptr;
        size_t size_ = 0;
        size_t cap_ = 0;
    };
    static_assert(sizeof(Segment) == 24, "a segment costs what a std::vector<uint8_t> costs");

public:
    static constexpr size_t segment_bytes = 16 * 1024 * 1024;

    ConversationBuffer() = default;
    ConversationBuffer(std::initializer_list<uint8_t> values) {
        resize(values.size());
        visit(0, size(), [&](uint8_t* p, size_t n, size_t at) {
            std::memcpy(p, values.begin() + at, n);
            return true;
        });
    }
    ConversationBuffer(const ConversationBuffer&) = default;
    ConversationBuffer& operator=(const ConversationBuffer&) = default;
    ConversationBuffer(ConversationBuffer&& o) noexcept : segments_(std::move(o.segments_)), size_(std::exchange(o.size_, 0)) {}
    ConversationBuffer& operator=(ConversationBuffer&& o) noexcept {
        if (this != &o) { segments_ = std::move(o.segments_); size_ = std::exchange(o.size_, 0); }
        return *this;
    }

    size_t size() const { return size_; }
    bool empty() const { return size_ == 0; }
    /// Host bytes held: the segment directory plus every segment's capacity.
    size_t bytes() const {
        size_t n = segments_.capacity() * sizeof(Segment);
        for (const Segment& s : segments_) n += s.capacity();
        return n;
    }
    /// bytes() after a resize(n), counting the old directory while a larger one is built; SIZE_MAX on overflow
    /// (so an impossible estimate fails admission before anything is allocated).
    size_t allocation_peak(size_t n) const {
        size_t total = bytes();
        if (n <= size_) return total;
        const size_t spare = tail_spare();
        const size_t extra = n - size_ - std::min(n - size_, spare);
        const size_t whole = extra / segment_bytes, rest = extra % segment_bytes;
        if (!add(total, whole * segment_bytes)) return SIZE_MAX;
        const size_t prev = whole ? segment_bytes : segments_.empty() ? 0 : segments_.back().capacity();
        if (rest && !add(total, grow_capacity(rest, prev, size_ != 0))) return SIZE_MAX;
        size_t count = segments_.size();
        if (!add(count, whole + (rest != 0))) return SIZE_MAX;
        if (count > segments_.capacity() &&
            (count > SIZE_MAX / sizeof(Segment) || !add(total, count * sizeof(Segment)))) return SIZE_MAX;
        return total;
    }
    void resize(size_t n, uint8_t value = 0) {
        if (n <= size_) { shrink(n); return; }
        const bool growing = size_ != 0;
        const size_t fill = std::min(n - size_, tail_spare());
        const size_t extra = n - size_ - fill;
        segments_.reserve(segments_.size() + extra / segment_bytes + (extra % segment_bytes != 0));
        if (fill) {
            Segment& last = segments_.back();
            last.resize(last.size() + fill, value);
            size_ += fill;
        }
        while (size_ < n) {
            const size_t count = std::min(segment_bytes, n - size_);
            const size_t prev = segments_.empty() ? 0 : segments_.back().capacity();
            Segment s(grow_capacity(count, prev, growing));
            s.resize(count, value);
            segments_.push_back(std::move(s));
            size_ += count;
        }
    }
    void pop_back() { resize(size_ - 1); }

    /// fn(pointer, count, absolute_offset) over [offset, offset + count) segment by segment; false stops.
    template <class Fn> bool visit(size_t offset, size_t count, Fn fn) { return walk(*this, offset, count, fn); }
    template <class Fn> bool visit(size_t offset, size_t count, Fn fn) const { return walk(*this, offset, count, fn); }

    bool read(void* target, size_t offset, size_t count) const {
        return visit(offset, count, [&](const uint8_t* p, size_t n, size_t at) {
            std::memcpy(static_cast<uint8_t*>(target) + (at - offset), p, n);
            return true;
        });
    }
    /// True when every segment of the buffer is pinned host memory.
    bool pinned() const {
        return std::all_of(segments_.begin(), segments_.end(), [](const Segment& s) { return s.pinned(); });
    }
    bool operator==(const ConversationBuffer& o) const {
        if (size_ != o.size_) return false;
        size_t i = 0, j = 0, x = 0, y = 0;
        while (i < segments_.size() && j < o.segments_.size()) {
            const Segment& a = segments_[i];
            const Segment& b = o.segments_[j];
            const size_t n = std::min(a.size() - x, b.size() - y);
            if (n && std::memcmp(a.data() + x, b.data() + y, n) != 0) return false;
            x += n;
            y += n;
            if (x == a.size()) { ++i; x = 0; }
            if (y == b.size()) { ++j; y = 0; }
        }
        return true;
    }

private:
    // A first capture allocates exactly its payload; later growth reserves geometrically (64 KiB .. 16 MiB), so a
    // conversation that grows by small turns extends its last segment instead of adding a copy per turn.
    static size_t grow_capacity(size_t count, size_t previous, bool growing) {
        if (!growing) return count;
        const size_t doubled = std::min(previous, segment_bytes / 2) * 2;
        return std::max(count, std::min(segment_bytes, std::max<size_t>(65536, doubled)));
    }
    static bool add(size_t& n, size_t extra) {
        if (extra > SIZE_MAX - n) return false;
        n += extra;
        return true;
    }
    size_t tail_spare() const { return segments_.empty() ? 0 : segments_.back().capacity() - segments_.back().size(); }
    void shrink(size_t n) {
        while (!segments_.empty() && size_ - segments_.back().size() >= n) {
            size_ -= segments_.back().size();
            segments_.pop_back();
        }
        if (size_ > n) segments_.back().resize(segments_.back().size() - (size_ - n), 0);
        size_ = n;
    }
    template <class Self, class Fn> static bool walk(Self& self, size_t offset, size_t count, Fn& fn) {
        if (offset > self.size_ || count > self.size_ - offset) return false;
        size_t begin = 0;
        for (auto& s : self.segments_) {
            if (!count) break;
            const size_t end = begin + s.size();
            if (offset < end) {
                const size_t n = std::min(count, end - offset);
                if (!fn(s.data() + (offset - begin), n, offset)) return false;
                offset += n;
                count -= n;
            }
            begin = end;
        }
        return count == 0;
    }

    std::vector<Segment> segments_;
    size_t size_ = 0;
};

}  // namespace strata::core

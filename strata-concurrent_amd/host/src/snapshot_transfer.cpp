// snapshot_transfer.cpp - running capture and restore batches (snapshot_transfer.hpp).
#include "snapshot_transfer.hpp"

#include "strata/kernels/kv_stream.hpp"
#include "transfer.hpp"

#include <algorithm>
#include <cstring>

namespace strata::core::xfer {
namespace {

const char* missing_message(Kind k) { return k == Kind::kv ? "missing state buffer" : "missing running-state buffer"; }
const char* copy_message(Kind k) {
    return k == Kind::kv ? "conversation snapshot copy" : "conversation snapshot running-state copy";
}

bool copy(void* dst, const void* src, size_t n, Kind k, std::string& error) {
    return detail::enqueue_copy(dst, src, n, error, copy_message(k));
}

// After a failure, nothing may still be in flight into a buffer the caller is about to free or reuse.
void drain() {
    std::string ignored;
    detail::finish_transfers(ignored, "");
}

bool enqueue(const CaptureLeg& leg, std::string& error) {
    const size_t n = leg.bytes - leg.from;
    if (!n) return true;
    if (leg.flat) return copy(leg.flat + leg.from, leg.state + leg.from, n, leg.kind, error);
    return leg.segmented->visit(leg.from, n, [&](uint8_t* p, size_t count, size_t at) {
        return copy(p, leg.state + at, count, leg.kind, error);
    });
}

bool enqueue(const RestoreLeg& leg, std::string& error) {
    if (!leg.bytes) return true;
    if (leg.flat) return copy(leg.state, leg.flat, leg.bytes, leg.kind, error);
    return leg.segmented->visit(0, leg.bytes, [&](const uint8_t* p, size_t count, size_t at) {
        return copy(leg.state + at, p, count, leg.kind, error);
    });
}

// A streamed layer (kv_mode 1) restored through its host copy: evict every VRAM slot so the next resolve refills
// from the restored bytes (src/kernels/cuda/kv_stream.cu:173-182).  A ring (kv_mode 2): refill the window - the last
// n_slots pages of the extent - from the host copy (kv_stream.cu:231-242).
void settle(const Residency& r, void* stream) {
    const QsaState& st = *r.layer;
    if (st.kv_mode == 1) strata::kernels::kv_stream_reset(st.map, stream);
    if (st.kv_mode == 2 && r.tokens > 0) {
        strata::kernels::QsaShapes s = strata::kernels::qsa_real_shapes();
        s.n_head_kv = r.n_head_kv;
        s.head_dim = r.head_dim;
        s.page_size = r.page_size;
        const int64_t end = (r.tokens + s.page_size - 1) / s.page_size;
        strata::kernels::kv_ring_restore(qsa_attn_pools(st), st.host, qsa_kv_format(st),
                                         std::max<int64_t>(0, end - st.n_slots), end, st.n_slots, s, stream);
    }
}

template <class Leg>
bool run_batches(const std::vector<Batch<Leg>>& batches, std::string& error) {
    for (const Batch<Leg>& b : batches)
        for (const Leg& leg : b.legs)
            if (leg.bytes > leg.from && !leg.state) return spec::refuse(error, missing_message(leg.kind));
    for (const Batch<Leg>& b : batches) {
        const detail::OnDevice on(b.device);
        if (b.sync_before && !detail::device_synchronize(error, "conversation snapshot synchronize")) return false;
        for (const Leg& leg : b.legs)
            if (!enqueue(leg, error)) {
                drain();
                return false;
            }
        if (!b.residency.empty()) {
            void* stream = detail::transfer_stream();
            for (const Residency& r : b.residency) settle(r, stream);
        }
        if (!detail::finish_transfers(error, "conversation snapshot transfer")) return false;
        if (b.sync_after && !detail::device_synchronize(error, "conversation snapshot synchronize")) return false;
    }
    return true;
}

}  // namespace

bool run(const std::vector<CaptureBatch>& batches, std::string& error) { return run_batches(batches, error); }
bool run(const std::vector<RestoreBatch>& batches, std::string& error) { return run_batches(batches, error); }

bool read_back_equal(const uint8_t* state, const ConversationBuffer& held, size_t offset, size_t bytes, uint64_t* fnv,
                     std::string& error) {
    static constexpr size_t kPiece = 65536;
    std::vector<uint8_t> piece(std::min(kPiece, bytes));
    for (size_t done = 0; done < bytes;) {
        const size_t n = std::min(kPiece, bytes - done);
        if (!detail::enqueue_copy(piece.data(), state + done, n, error, "conversation snapshot copy") ||
            !detail::finish_transfers(error, "conversation snapshot copy"))
            return false;
        const size_t base = offset + done;
        const bool same = held.visit(base, n, [&](const uint8_t* p, size_t count, size_t at) {
            return std::memcmp(p, piece.data() + (at - base), count) == 0;
        });
        if (!same) return spec::refuse(error, "restored K/V bytes differ");
        if (fnv)
            for (size_t i = 0; i < n; ++i) *fnv = (*fnv ^ piece[i]) * 1099511628211ull;
        done += n;
    }
    return true;
}

}  // namespace strata::core::xfer

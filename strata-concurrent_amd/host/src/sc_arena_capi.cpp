// sc_arena_capi.cpp - the C-ABI of include/sc_arena.h over strata::core::HandoffArena and HandoffMover.
#include "sc_arena.h"

#include "strata/core/handoff.hpp"
#include "strata/core/handoff_device.hpp"

#include <algorithm>
#include <array>
#include <cstring>
#include <exception>
#include <string>
#include <vector>

using strata::core::HandoffArena;
using strata::core::HandoffClaim;
using strata::core::HandoffMoveStats;
using strata::core::HandoffMover;
using strata::core::HandoffMoverConfig;
using strata::core::HandoffPayload;
using strata::core::HandoffSizing;
using strata::core::HandoffSlotInfo;
using strata::core::HandoffTierSpec;

struct sc_arena {
    HandoffArena arena;
};
struct sc_mover {
    HandoffMover mover;
};

namespace {

thread_local std::string g_error;

int fail(int code, std::string why) {
    g_error = std::move(why);
    return code;
}

template <class F>
int guarded(F&& f) {
    try {
        return f();
    } catch (const std::exception& e) {
        return fail(SC_ENOMEM, std::string("sc_arena: ") + e.what());
    } catch (...) {
        return fail(SC_ENOMEM, "sc_arena: unknown exception");
    }
}

bool tiers_of(int32_t n, const uint64_t* tokens, const uint64_t* slots, const uint64_t* priced,
              std::vector<HandoffTierSpec>& tiers, std::vector<uint64_t>& bytes) {
    if (n < 0 || n > 64 || (n && (!tokens || !slots || !priced))) return false;
    for (int32_t i = 0; i < n; ++i) {
        tiers.push_back({tokens[i], slots[i]});
        bytes.push_back(priced[i]);
    }
    return true;
}

HandoffClaim claim_of(const sc_arena_claim& c) {
    HandoffClaim h;
    h.index = c.index;
    h.tier = c.tier;
    h.base = c.base;
    h.payload_off = c.payload_off;
    h.capacity = c.capacity;
    h.nonce = c.nonce;
    return h;
}

void slot_out(const HandoffSlotInfo& i, sc_arena_slot* out) {
    if (!out) return;
    out->index = i.index;
    out->state = i.state;
    out->flags = i.flags;
    out->tier = i.tier;
    out->base = i.base;
    out->capacity = i.capacity;
    out->owner_pid = i.owner_pid;
    out->owner_start = i.owner_start;
    out->nonce = i.nonce;
    out->client_id = i.client_id;
    out->request_id = i.request_id;
    out->pack_hash = i.pack_hash;
    out->geom_hash = i.geom_hash;
    out->tokens = i.tokens;
    out->payload_bytes = i.payload_bytes;
    out->payload_hash = i.payload_hash;
    out->claimed_ms = i.claimed_ms;
    out->published_ms = i.published_ms;
    out->seq = i.seq;
}

}  // namespace

extern "C" {

const char* sc_arena_last_error(void) { return g_error.c_str(); }

int sc_arena_size(int32_t n_tiers, const uint64_t* tier_tokens, const uint64_t* tier_slots, const uint64_t* priced,
                  uint64_t* slot_bytes, uint64_t* slot_off, uint64_t* arena_bytes, char* describe,
                  uint64_t describe_cap) {
    return guarded([&] {
        std::vector<HandoffTierSpec> tiers;
        std::vector<uint64_t> bytes;
        if (!tiers_of(n_tiers, tier_tokens, tier_slots, priced, tiers, bytes))
            return fail(SC_EINVAL, "sc_arena: invalid tier table");
        HandoffSizing s;
        std::string err;
        if (!strata::core::handoff_size_arena(tiers, bytes, s, err)) return fail(SC_EINVAL, err);
        for (int32_t i = 0; i < n_tiers; ++i) {
            if (slot_bytes) slot_bytes[i] = s.slot_bytes[(size_t) i];
            if (slot_off) slot_off[i] = s.slot_off[(size_t) i];
        }
        if (arena_bytes) *arena_bytes = s.arena_bytes;
        if (describe && describe_cap) {
            const size_t n = std::min<size_t>(s.describe.size(), (size_t) describe_cap - 1);
            std::memcpy(describe, s.describe.data(), n);
            describe[n] = 0;
        }
        return (int) SC_OK;
    });
}

uint64_t sc_arena_geom_hash(const int64_t* geometry18, const char* split_spec) {
    if (!geometry18) return 0;
    std::array<int64_t, 18> g{};
    for (int i = 0; i < 18; ++i) g[(size_t) i] = geometry18[i];
    return strata::core::handoff_geom_hash(g, split_spec ? split_spec : "");
}

int sc_arena_open_writer(const char* path, int32_t n_tiers, const uint64_t* tier_tokens, const uint64_t* tier_slots,
                         const uint64_t* priced, uint64_t pack_hash, uint64_t geom_hash, int32_t reserve,
                         int64_t lease_ms, sc_arena** out) {
    return guarded([&] {
        if (!path || !out) return fail(SC_EINVAL, "sc_arena: missing path or output");
        *out = nullptr;
        std::vector<HandoffTierSpec> tiers;
        std::vector<uint64_t> bytes;
        if (!tiers_of(n_tiers, tier_tokens, tier_slots, priced, tiers, bytes))
            return fail(SC_EINVAL, "sc_arena: invalid tier table");
        HandoffSizing s;
        std::string err;
        if (!strata::core::handoff_size_arena(tiers, bytes, s, err)) return fail(SC_EINVAL, err);
        auto* a = new sc_arena;
        if (lease_ms >= 0) a->arena.set_lease_ms((uint64_t) lease_ms);
        if (!a->arena.open_writer(path, s, pack_hash, geom_hash, err) || (reserve && !a->arena.reserve(err))) {
            delete a;
            return fail(SC_EINVAL, err);
        }
        *out = a;
        return (int) SC_OK;
    });
}

int sc_arena_open_reader(const char* path, uint64_t pack_hash, uint64_t geom_hash, sc_arena** out) {
    return guarded([&] {
        if (!path || !out) return fail(SC_EINVAL, "sc_arena: missing path or output");
        *out = nullptr;
        auto* a = new sc_arena;
        std::string err;
        if (!a->arena.open_reader(path, pack_hash, geom_hash, err)) {
            delete a;
            return fail(SC_EINVAL, err);
        }
        *out = a;
        return (int) SC_OK;
    });
}

int sc_arena_close(sc_arena* arena) {
    delete arena;
    return SC_OK;
}

int sc_arena_reserve(sc_arena* arena) {
    return guarded([&] {
        if (!arena) return fail(SC_EINVAL, "sc_arena: missing arena");
        std::string err;
        return arena->arena.reserve(err) ? (int) SC_OK : fail(SC_EINVAL, err);
    });
}

int sc_arena_claim_slot(sc_arena* arena, uint32_t tier, uint64_t client_id, uint64_t request_id, sc_arena_claim* out) {
    return guarded([&] {
        if (!arena || !out) return fail(SC_EINVAL, "sc_arena: missing arena or output");
        HandoffClaim c;
        std::string err;
        if (!arena->arena.claim(tier, client_id, request_id, c, err))
            return fail(err.find("no free handoff slot") != std::string::npos ? (int) SC_EBUSY : (int) SC_EINVAL, err);
        out->index = c.index;
        out->tier = c.tier;
        out->base = c.base;
        out->payload_off = c.payload_off;
        out->capacity = c.capacity;
        out->nonce = c.nonce;
        return (int) SC_OK;
    });
}

int sc_arena_write(sc_arena* arena, const sc_arena_claim* claim, uint64_t offset, const void* host, uint64_t bytes) {
    return guarded([&] {
        if (!arena || !claim) return fail(SC_EINVAL, "sc_arena: missing arena or claim");
        std::string err;
        return arena->arena.write_payload(claim_of(*claim), offset, host, bytes, err) ? (int) SC_OK : fail(SC_EINVAL, err);
    });
}

int sc_arena_publish(sc_arena* arena, const sc_arena_claim* claim, uint64_t tokens, uint64_t payload_bytes,
                     uint64_t payload_hash) {
    return guarded([&] {
        if (!arena || !claim) return fail(SC_EINVAL, "sc_arena: missing arena or claim");
        std::string err;
        return arena->arena.publish(claim_of(*claim), tokens, payload_bytes, payload_hash, err) ? (int) SC_OK
                                                                                                : fail(SC_EINVAL, err);
    });
}

int sc_arena_release(sc_arena* arena, int32_t index, uint64_t nonce) {
    return guarded([&] {
        if (!arena) return fail(SC_EINVAL, "sc_arena: missing arena");
        std::string err;
        return arena->arena.release(index, nonce, err) ? (int) SC_OK : fail(SC_EINVAL, err);
    });
}

int sc_arena_abort(sc_arena* arena, int32_t index, uint64_t nonce) {
    return guarded([&] {
        if (!arena) return fail(SC_EINVAL, "sc_arena: missing arena");
        std::string err;
        return arena->arena.abort_claim(index, nonce, err) ? (int) SC_OK : fail(SC_EINVAL, err);
    });
}

int sc_arena_cancel(sc_arena* arena, int32_t index, uint64_t nonce) {
    return guarded([&] {
        if (!arena) return fail(SC_EINVAL, "sc_arena: missing arena");
        std::string err;
        return arena->arena.cancel(index, nonce, err) ? (int) SC_OK : fail(SC_EINVAL, err);
    });
}

int sc_arena_slot_info(sc_arena* arena, int32_t index, sc_arena_slot* out) {
    return guarded([&] {
        if (!arena || !out) return fail(SC_EINVAL, "sc_arena: missing arena or output");
        HandoffSlotInfo i;
        if (!arena->arena.slot_info(index, i)) return fail(SC_EINVAL, "sc_arena: no slot " + std::to_string(index));
        slot_out(i, out);
        return (int) SC_OK;
    });
}

int sc_arena_read_host(sc_arena* arena, int32_t index, uint64_t nonce, uint64_t client_id, void* host, uint64_t capacity,
                       int32_t check_hash, sc_arena_slot* out) {
    return guarded([&] {
        if (!arena) return fail(SC_EINVAL, "sc_arena: missing arena");
        HandoffPayload p;
        std::string err;
        if (!arena->arena.read_slot(index, nonce, client_id, p, err)) return fail(SC_EINVAL, err);
        if (p.payload_bytes > capacity || (p.payload_bytes && !host))
            return fail(SC_EINVAL, "sc_arena: the payload is " + std::to_string(p.payload_bytes) + " B and the buffer holds " +
                                       std::to_string(capacity) + " B");
        if (p.payload_bytes) std::memcpy(host, p.data, (size_t) p.payload_bytes);
        if (check_hash && HandoffArena::payload_hash_of(p) != p.payload_hash)
            return fail(SC_ESTALE, "sc_arena: slot " + std::to_string(index) + " fails its payload hash");
        HandoffSlotInfo i;
        if (out && arena->arena.slot_info(index, i)) slot_out(i, out);
        return (int) SC_OK;
    });
}

int sc_mover_create(uint64_t chunk_bytes, int32_t depth, int32_t threads, sc_mover** out) {
    return guarded([&] {
        if (!out) return fail(SC_EINVAL, "sc_arena: missing output");
        *out = nullptr;
        auto* m = new sc_mover;
        HandoffMoverConfig cfg;
        cfg.chunk_bytes = chunk_bytes;
        cfg.depth = depth;
        cfg.threads = threads;
        std::string err;
        if (!m->mover.init(cfg, err)) {
            delete m;
            return fail(SC_ENOMEM, err);
        }
        *out = m;
        return (int) SC_OK;
    });
}

int sc_mover_destroy(sc_mover* mover) {
    delete mover;
    return SC_OK;
}

// The status of a failed transfer: a device hash that did not complete, a device call's failure, or a refusal.
static int mover_code(const HandoffMoveStats& st) {
    return st.hash_fault ? (int) SC_ETIMEOUT : st.device_error ? (int) SC_EHIP : (int) SC_EINVAL;
}

int sc_mover_write(sc_mover* mover, sc_arena* arena, const sc_arena_claim* claim, const void* device_src,
                   uint64_t bytes, void* stream, uint64_t* hash) {
    return guarded([&] {
        if (!mover || !arena || !claim) return fail(SC_EINVAL, "sc_arena: missing mover, arena or claim");
        std::string err;
        if (mover->mover.write_from_device(arena->arena, claim_of(*claim), device_src, bytes, stream, hash, err))
            return (int) SC_OK;
        return fail(mover_code(mover->mover.last()), err);
    });
}

int sc_mover_publish(sc_mover* mover, sc_arena* arena, const sc_arena_claim* claim, const void* device_src,
                     uint64_t bytes, uint64_t tokens, void* stream) {
    return guarded([&] {
        if (!mover || !arena || !claim) return fail(SC_EINVAL, "sc_arena: missing mover, arena or claim");
        std::string err;
        if (mover->mover.publish_from_device(arena->arena, claim_of(*claim), device_src, bytes, tokens, stream, err))
            return (int) SC_OK;
        return fail(mover_code(mover->mover.last()), err);
    });
}

int sc_mover_read(sc_mover* mover, sc_arena* arena, int32_t index, uint64_t nonce, uint64_t client_id, void* device_dst,
                  uint64_t capacity, void* stream, int32_t verify, sc_arena_slot* out) {
    return guarded([&] {
        if (!mover || !arena) return fail(SC_EINVAL, "sc_arena: missing mover or arena");
        HandoffSlotInfo i;
        std::string err;
        const bool ok =
            mover->mover.read_to_device(arena->arena, index, nonce, client_id, device_dst, capacity, stream, verify != 0, i, err);
        slot_out(i, out);
        if (ok) return (int) SC_OK;
        const auto& st = mover->mover.last();
        return fail(st.hash_fault || st.device_error ? mover_code(st) : st.wrote_device ? (int) SC_ESTALE : (int) SC_EINVAL,
                    err);
    });
}

int sc_mover_last(const sc_mover* mover, uint64_t* bytes, double* ms, double* hash_ms, double* copy_ms, double* wait_ms) {
    if (!mover) return fail(SC_EINVAL, "sc_arena: missing mover");
    const auto& st = mover->mover.last();
    if (bytes) *bytes = st.bytes;
    if (ms) *ms = st.ms;
    if (hash_ms) *hash_ms = st.hash_ms;
    if (copy_ms) *copy_ms = st.copy_ms;
    if (wait_ms) *wait_ms = st.wait_ms;
    return SC_OK;
}

}  // extern "C"

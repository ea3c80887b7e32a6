// sc_wire_capi.cpp - the C-ABI of include/sc_wire.h over the C++ device payload path.
#include "sc_wire.h"

#include "strata/core/conversation_wire_device.hpp"

#include <algorithm>
#include <array>
#include <exception>
#include <new>
#include <string>
#include <type_traits>

using namespace strata::core;

struct sc_wire_encoder {
    WireDeviceEncoder enc;
};
struct sc_wire_decoder {
    WireDeviceDecoder dec;
    SavedConversation image;
    bool restored = false;
    // what it was opened with, for sc_wire_decoder_reopen: own copies of the slot's pointer arrays and segments
    bool reopenable = false, layered = false, segmented = false;
    sc_geometry g{};
    WireExpect expect{};
    sc_decode_slot slot{};
    sc_slot_layers layers{};
    std::vector<uint16_t*> k_pool, v_pool;
    std::vector<const int32_t*> tables;
    std::vector<sc_kv_pools> host, stage;
    std::array<std::vector<void*>, SC_N_BUF> bufs;
    std::vector<void*> seg_ptr;
    uint64_t seg_bytes = 0;

    void remember(const sc_geometry& geo, const sc_decode_slot& s, const sc_segments* segs, const WireExpect& e) {
        const size_t n = size_t(std::max<int64_t>(sc_n_qsa_layers(&geo), 0));
        g = geo;
        expect = e;
        slot = s;
        layered = false;
        k_pool.assign(s.k_pool, s.k_pool + (s.k_pool ? n : 0));
        v_pool.assign(s.v_pool, s.v_pool + (s.v_pool ? n : 0));
        tables.assign(s.page_table, s.page_table + (s.page_table ? n : 0));
        host.assign(s.host, s.host + (s.host ? n : 0));
        stage.assign(s.stage, s.stage + (s.stage ? n : 0));
        slot.k_pool = s.k_pool ? k_pool.data() : nullptr;
        slot.v_pool = s.v_pool ? v_pool.data() : nullptr;
        slot.page_table = s.page_table ? tables.data() : nullptr;
        slot.host = s.host ? host.data() : nullptr;
        slot.stage = s.stage ? stage.data() : nullptr;
        remember_segments(segs);
    }
    void remember(const sc_geometry& geo, const sc_slot_layers& s, const sc_segments* segs, const WireExpect& e) {
        const size_t n = size_t(std::max<int64_t>(sc_n_qsa_layers(&geo), 0));
        g = geo;
        expect = e;
        layers = s;
        layered = true;
        for (int x = 0; x < SC_N_BUF; ++x) {
            bufs[size_t(x)].assign(s.buf[x], s.buf[x] + (s.buf[x] ? n : 0));
            layers.buf[x] = s.buf[x] ? bufs[size_t(x)].data() : nullptr;
        }
        remember_segments(segs);
    }
    void remember_segments(const sc_segments* segs) {
        segmented = segs != nullptr;
        seg_ptr.assign(segs ? segs->ptr : nullptr, segs ? segs->ptr + segs->n : nullptr);
        seg_bytes = segs ? segs->segment_bytes : 0;
        reopenable = true;
    }
};

namespace {

thread_local std::string g_error;

int done() {
    g_error.clear();
    return SC_OK;
}
int failed(int code, const std::string& why) {
    g_error = why;
    return code;
}

template <class F> int guarded(F&& f) {
    try {
        return f();
    } catch (const std::bad_alloc&) {
        return failed(SC_ENOMEM, "conversation wire: host allocation failed");
    } catch (const std::exception& e) {
        return failed(SC_EINVAL, std::string("conversation wire: ") + e.what());
    }
}

}  // namespace

extern "C" {

const char* sc_wire_last_error(void) { return g_error.c_str(); }

extern "C++" {
// The host side of a conversation from its C description; SC_OK or the refusal.
static int conversation_of(const sc_wire_live* live, WireDeviceConversation& conv) {
    if (live->n_ids < 0 || live->n_imgs < 0 || (live->n_ids && !live->ids) ||
        (live->n_imgs && (!live->img_start || !live->img_hash)))
        return failed(SC_EINVAL, "conversation wire: invalid live checkpoint arrays");
    for (int i = 0; i < 18; ++i) conv.geometry[size_t(i)] = live->geometry[i];
    conv.layer_lo = live->layer_lo;
    conv.layer_hi = live->layer_hi;
    conv.cvec = live->cvec != 0;
    conv.idx_dim = live->idx_dim;
    conv.live.ids.assign(live->ids, live->ids + live->n_ids);
    for (int64_t i = 0; i < live->n_imgs; ++i) conv.live.imgs.push_back({live->img_start[i], live->img_hash[i]});
    conv.live.used = live->used;
    std::vector<uint8_t>* small[4] = {&conv.live.ple, &conv.live.tails, &conv.live.dead, &conv.live.block_pos};
    for (int i = 0; i < 4; ++i) {
        if (live->small_bytes[i] && !live->small[i]) return failed(SC_EINVAL, "conversation wire: missing small buffer");
        small[i]->assign(live->small[i], live->small[i] + live->small_bytes[i]);
    }
    if (live->draft_record) conv.trailing_kv.emplace_back();
    return SC_OK;
}

// The stages of a layer split from their C description (the small buffers only when `with_state`).
static int stages_of(const sc_wire_stage* stages, int32_t n, const std::vector<int32_t>& ids, bool with_state,
                     std::vector<WireDeviceStage>& out) {
    if (n < 0 || (n && !stages)) return failed(SC_EINVAL, "conversation wire: invalid stage array");
    out.resize(size_t(n));
    for (int32_t i = 0; i < n; ++i) {
        const sc_wire_stage& in = stages[i];
        WireDeviceStage& st = out[size_t(i)];
        st.geometry = in.geometry;
        st.slot = in.slot;
        st.layer_lo = in.layer_lo;
        st.layer_hi = in.layer_hi;
        if (!with_state) continue;
        st.state.ids = ids;
        std::vector<uint8_t>* small[4] = {&st.state.ple, &st.state.tails, &st.state.dead, &st.state.block_pos};
        for (int k = 0; k < 4; ++k) {
            if (in.small_bytes[k] && !in.small[k]) return failed(SC_EINVAL, "conversation wire: missing stage buffer");
            small[k]->assign(in.small[k], in.small[k] + in.small_bytes[k]);
        }
    }
    return SC_OK;
}

template <class Slot>
static int encoder_create(const sc_geometry* g, const Slot* slot, int64_t tokens, const sc_wire_live* live,
                          const sc_wire_stage* stages, int32_t n_stages, uint64_t geom_hash, uint64_t pack_hash,
                          sc_wire_encoder** out) {
    return guarded([&] {
        if (!g || !slot || !live || !out) return failed(SC_EINVAL, "conversation wire: missing argument");
        WireDeviceConversation conv;
        if (const int rc = conversation_of(live, conv)) return rc;
        auto* e = new sc_wire_encoder();
        std::string err;
        bool planned;
        if constexpr (std::is_same_v<Slot, sc_decode_slot>) {
            std::vector<WireDeviceStage> parts;
            if (const int rc = stages_of(stages, n_stages, conv.live.ids, true, parts)) {
                delete e;
                return rc;
            }
            planned = e->enc.plan(*g, *slot, tokens, conv, parts, WireIdentity{geom_hash, pack_hash}, err);
        } else {
            planned = e->enc.plan(*g, *slot, tokens, conv, WireIdentity{geom_hash, pack_hash}, err);
        }
        if (!planned) {
            delete e;
            return failed(SC_EINVAL, err);
        }
        *out = e;
        return done();
    });
}
}  // extern "C++"

int sc_wire_encoder_create(const sc_geometry* g, const sc_decode_slot* slot, int64_t tokens, const sc_wire_live* live,
                           uint64_t geom_hash, uint64_t pack_hash, sc_wire_encoder** out) {
    return encoder_create(g, slot, tokens, live, nullptr, 0, geom_hash, pack_hash, out);
}

int sc_wire_encoder_create_split(const sc_geometry* g, const sc_decode_slot* slot, int64_t tokens,
                                 const sc_wire_live* live, const sc_wire_stage* stages, int32_t n_stages,
                                 uint64_t geom_hash, uint64_t pack_hash, sc_wire_encoder** out) {
    return encoder_create(g, slot, tokens, live, stages, n_stages, geom_hash, pack_hash, out);
}

int sc_wire_encoder_create_layers(const sc_geometry* g, const sc_slot_layers* slot, int64_t tokens,
                                  const sc_wire_live* live, uint64_t geom_hash, uint64_t pack_hash,
                                  sc_wire_encoder** out) {
    return encoder_create(g, slot, tokens, live, nullptr, 0, geom_hash, pack_hash, out);
}

uint64_t sc_wire_encoder_bytes(const sc_wire_encoder* e) { return e ? e->enc.bytes() : 0; }
uint64_t sc_wire_encoder_pool_offset(const sc_wire_encoder* e) { return e ? e->enc.layout().blob_pool_off : 0; }

int sc_wire_encode_async(sc_wire_encoder* e, void* payload, uint64_t capacity, void* stream, void* gathered) {
    return guarded([&] {
        if (!e) return failed(SC_EINVAL, "conversation wire: missing encoder");
        std::string err;
        return e->enc.encode(payload, capacity, stream, err, gathered) ? done() : failed(SC_EHIP, err);
    });
}

int sc_wire_encode_segments_async(sc_wire_encoder* e, const sc_segments* into, void* stream) {
    return guarded([&] {
        if (!e || !into) return failed(SC_EINVAL, "conversation wire: missing encoder or segments");
        std::string err;
        if (e->enc.encode_segments(*into, stream, err)) return done();
        return failed(err.find("conversation wire") != std::string::npos && err.find("sc_handoff") == std::string::npos
                          ? SC_EINVAL : SC_EHIP, err);
    });
}

// The encoder's and decoder's refusal of a device hash whose kernel's bounded wait ran out.
static bool hash_incomplete(const std::string& err) { return err.find("did not complete") != std::string::npos; }

int sc_wire_encoder_hash(sc_wire_encoder* e, uint64_t* hash) {
    return guarded([&] {
        if (!e || !hash) return failed(SC_EINVAL, "conversation wire: missing argument");
        std::string err;
        if (e->enc.payload_hash(*hash, err)) return done();
        return failed(hash_incomplete(err) ? SC_ETIMEOUT : SC_EHIP, err);
    });
}

int sc_wire_encoder_set_carry(sc_wire_encoder* e, void* carry) {
    if (!e) return failed(SC_EINVAL, "conversation wire: missing encoder");
    e->enc.set_carry(static_cast<uint8_t*>(carry));
    return done();
}

int sc_wire_encoder_destroy(sc_wire_encoder* e) {
    delete e;
    return done();
}

extern "C++" {
template <class Slot>
static int decoder_open(const void* payload, uint64_t bytes, const sc_geometry* g, const Slot* slot,
                        const sc_wire_stage* stages, int32_t n_stages, const int64_t* geometry, uint64_t geom_hash,
                        uint64_t pack_hash, int32_t check_identity, uint64_t payload_hash, int32_t check_hash,
                        sc_wire_decoder** out, const sc_segments* segs = nullptr) {
    return guarded([&] {
        if (!g || !slot || !out) return failed(SC_EINVAL, "conversation wire: missing argument");
        WireExpect expect;
        if (geometry) {
            for (int i = 0; i < 18; ++i) expect.geometry[size_t(i)] = geometry[i];
            expect.check_geometry = true;
        }
        expect.geom_hash = geom_hash;
        expect.pack_hash = pack_hash;
        expect.check_hashes = check_identity != 0;
        expect.payload_hash = payload_hash;
        expect.check_payload_hash = check_hash != 0;
        expect.stage_parts = n_stages;
        auto* d = new sc_wire_decoder();
        std::string err;
        bool opened;
        if constexpr (std::is_same_v<Slot, sc_decode_slot>) {
            std::vector<WireDeviceStage> parts;
            if (const int rc = stages_of(stages, n_stages, {}, false, parts)) {
                delete d;
                return rc;
            }
            opened = segs ? d->dec.open(*segs, bytes, *g, *slot, parts, expect, err)
                          : d->dec.open(payload, bytes, *g, *slot, parts, expect, err);
        } else {
            opened = segs ? d->dec.open(*segs, bytes, *g, *slot, expect, err)
                          : d->dec.open(payload, bytes, *g, *slot, expect, err);
        }
        if (!opened) {
            delete d;
            return failed(SC_EINVAL, err);
        }
        if (n_stages == 0) d->remember(*g, *slot, segs, expect);
        *out = d;
        return done();
    });
}
}  // extern "C++"

int sc_wire_decoder_open(const void* payload, uint64_t bytes, const sc_geometry* g, const sc_decode_slot* slot,
                         const int64_t* geometry, uint64_t geom_hash, uint64_t pack_hash, int32_t check_identity,
                         uint64_t payload_hash, int32_t check_hash, sc_wire_decoder** out) {
    return decoder_open(payload, bytes, g, slot, nullptr, 0, geometry, geom_hash, pack_hash, check_identity, payload_hash,
                        check_hash, out);
}

int sc_wire_decoder_open_split(const void* payload, uint64_t bytes, const sc_geometry* g, const sc_decode_slot* slot,
                               const sc_wire_stage* stages, int32_t n_stages, const int64_t* geometry,
                               uint64_t geom_hash, uint64_t pack_hash, int32_t check_identity, uint64_t payload_hash,
                               int32_t check_hash, sc_wire_decoder** out) {
    return decoder_open(payload, bytes, g, slot, stages, n_stages, geometry, geom_hash, pack_hash, check_identity,
                        payload_hash, check_hash, out);
}

int sc_wire_decoder_open_layers(const void* payload, uint64_t bytes, const sc_geometry* g, const sc_slot_layers* slot,
                                const int64_t* geometry, uint64_t geom_hash, uint64_t pack_hash, int32_t check_identity,
                                uint64_t payload_hash, int32_t check_hash, sc_wire_decoder** out) {
    return decoder_open(payload, bytes, g, slot, nullptr, 0, geometry, geom_hash, pack_hash, check_identity, payload_hash,
                        check_hash, out);
}

int sc_wire_decoder_open_segments(const sc_segments* from, uint64_t bytes, const sc_geometry* g,
                                  const sc_decode_slot* slot, const int64_t* geometry, uint64_t geom_hash,
                                  uint64_t pack_hash, int32_t check_identity, uint64_t payload_hash, int32_t check_hash,
                                  sc_wire_decoder** out) {
    if (!from) return failed(SC_EINVAL, "conversation wire: missing segments");
    return decoder_open(nullptr, bytes, g, slot, nullptr, 0, geometry, geom_hash, pack_hash, check_identity,
                        payload_hash, check_hash, out, from);
}

int sc_wire_decoder_open_layers_segments(const sc_segments* from, uint64_t bytes, const sc_geometry* g,
                                         const sc_slot_layers* slot, const int64_t* geometry, uint64_t geom_hash,
                                         uint64_t pack_hash, int32_t check_identity, uint64_t payload_hash,
                                         int32_t check_hash, sc_wire_decoder** out) {
    if (!from) return failed(SC_EINVAL, "conversation wire: missing segments");
    return decoder_open(nullptr, bytes, g, slot, nullptr, 0, geometry, geom_hash, pack_hash, check_identity,
                        payload_hash, check_hash, out, from);
}

int64_t sc_wire_decoder_tokens(const sc_wire_decoder* d) { return d ? d->dec.tokens() : -1; }

int sc_wire_decoder_reopen(sc_wire_decoder* d, const void* payload, uint64_t bytes, uint64_t payload_hash) {
    return guarded([&] {
        if (!d) return failed(SC_EINVAL, "conversation wire: missing decoder");
        if (!d->reopenable)
            return failed(SC_EINVAL, "conversation wire: a decoder of a layer-split payload is not opened again; open a new one");
        if (d->segmented != (payload == nullptr))
            return failed(SC_EINVAL, d->segmented ? "conversation wire: this decoder reads its payload from its segments "
                                                    "(payload must be NULL)"
                                                  : "conversation wire: missing payload");
        WireExpect expect = d->expect;
        expect.payload_hash = payload_hash;
        d->restored = false;
        d->image = SavedConversation{};
        const sc_segments segs{int32_t(d->seg_ptr.size()), d->seg_bytes, d->seg_ptr.data()};
        std::string err;
        bool opened;
        if (d->layered)
            opened = d->segmented ? d->dec.open(segs, bytes, d->g, d->layers, expect, err)
                                  : d->dec.open(payload, bytes, d->g, d->layers, expect, err);
        else
            opened = d->segmented ? d->dec.open(segs, bytes, d->g, d->slot, {}, expect, err)
                                  : d->dec.open(payload, bytes, d->g, d->slot, expect, err);
        if (!opened) return failed(SC_EINVAL, err);
        d->expect = expect;
        return done();
    });
}

int sc_wire_decoder_set_carry(sc_wire_decoder* d, const void* carry) {
    if (!d) return failed(SC_EINVAL, "conversation wire: missing decoder");
    d->dec.set_carry(static_cast<const uint8_t*>(carry));
    return done();
}

int sc_wire_decoder_restore(sc_wire_decoder* d, void* stream) {
    return guarded([&] {
        if (!d) return failed(SC_EINVAL, "conversation wire: missing decoder");
        std::string err;
        if (!d->dec.restore(stream, d->image, err))   // a timed-out or mismatching hash gated every scatter off
            return failed(hash_incomplete(err) ? SC_ETIMEOUT
                          : err.find("hash mismatch") != std::string::npos || err.find("before a successful") != std::string::npos ||
                                    err.find("its carries") != std::string::npos
                              ? SC_EINVAL : SC_EHIP, err);
        d->restored = true;
        return done();
    });
}

int sc_wire_decoder_live_ids(const sc_wire_decoder* d, int32_t* ids, int64_t cap, int64_t* n) {
    if (!d || !d->restored || !n) return failed(SC_EINVAL, "conversation wire: no restored image");
    const auto& v = d->image.live.ids;
    *n = int64_t(v.size());
    if (cap < int64_t(v.size()) || (!v.empty() && !ids)) return failed(SC_ERANGE, "conversation wire: id buffer too small");
    for (size_t i = 0; i < v.size(); ++i) ids[i] = v[i];
    return done();
}

int sc_wire_decoder_small(const sc_wire_decoder* d, int32_t which, uint8_t* dst, uint64_t cap, uint64_t* n) {
    if (!d || !d->restored || !n || which < 0 || which > 3) return failed(SC_EINVAL, "conversation wire: no such buffer");
    const std::vector<uint8_t>* small[4] = {&d->image.live.ple, &d->image.live.tails, &d->image.live.dead,
                                            &d->image.live.block_pos};
    const auto& v = *small[which];
    *n = v.size();
    if (cap < v.size() || (!v.empty() && !dst)) return failed(SC_ERANGE, "conversation wire: buffer too small");
    for (size_t i = 0; i < v.size(); ++i) dst[i] = v[i];
    return done();
}

int sc_wire_decoder_stage_small(const sc_wire_decoder* d, int32_t stage, int32_t which, uint8_t* dst, uint64_t cap,
                                uint64_t* n) {
    if (!d || !d->restored || !n || which < 0 || which > 3 || stage < 0 ||
        size_t(stage) >= d->image.stage_parts.size())
        return failed(SC_EINVAL, "conversation wire: no such stage buffer");
    const ConversationCheckpoint& st = d->image.stage_parts[size_t(stage)].state;
    const std::vector<uint8_t>* small[4] = {&st.ple, &st.tails, &st.dead, &st.block_pos};
    const auto& v = *small[which];
    *n = v.size();
    if (cap < v.size() || (!v.empty() && !dst)) return failed(SC_ERANGE, "conversation wire: buffer too small");
    for (size_t i = 0; i < v.size(); ++i) dst[i] = v[i];
    return done();
}

int sc_wire_decoder_destroy(sc_wire_decoder* d) {
    delete d;
    return done();
}

}  // extern "C"

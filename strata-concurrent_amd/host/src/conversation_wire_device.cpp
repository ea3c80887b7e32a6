// conversation_wire_device.cpp - device-resident hand-off payloads (see conversation_wire_device.hpp).
#include "strata/core/conversation_wire_device.hpp"

#include "wire_internal.hpp"

#include <algorithm>
#include <cstring>

namespace strata::core {
namespace {

bool refuse(std::string& error, const std::string& why) {
    error = "conversation wire: " + why;
    return false;
}
bool abi(int rc, std::string& error, const char* what) {
    if (rc == SC_OK) return true;
    error = std::string("conversation wire: ") + what + ": " + sc_last_error();
    return false;
}
uint64_t up64(uint64_t n) { return (n + 63) & ~uint64_t(63); }

// The slot-side shape of the payload: per-layer K/V blob bytes and the GDN blob bytes.
// The bytes of a value, appended to the key of a plan (what it was built for).
template <class T>
void put_key(std::vector<uint8_t>& key, const T& v) {
    const auto* p = reinterpret_cast<const uint8_t*>(&v);
    key.insert(key.end(), p, p + sizeof(T));
}

struct SlotShape {
    int64_t n_qsa = 0, n_gdn = 0, cells = 0;
    uint64_t kv_bytes = 0, gdn_bytes = 0;
};

bool slot_shape(const sc_geometry& g, int64_t tokens, SlotShape& s, std::string& error) {
    if (tokens < 0) return refuse(error, "a negative token count");
    s.n_qsa = sc_n_qsa_layers(&g);
    s.n_gdn = sc_n_gdn_layers(&g);
    s.cells = sc_kv_cells(&g, tokens);
    const int64_t row_floats = sc_gdn_row_floats(&g);
    if (s.cells < 0 || (s.n_gdn > 0 && row_floats <= 0)) return refuse(error, "invalid model geometry");
    s.kv_bytes = uint64_t(s.cells) * uint64_t(g.n_head_kv) * uint64_t(g.head_dim) * 2;
    s.gdn_bytes = uint64_t(s.n_gdn) * uint64_t(row_floats) * 4;
    return true;
}

// Copies the bytes of the image buffer `who` (a K/V record's ConversationBuffer or a checkpoint's vector) to `dst`.
bool stage_checkpoint_blob(const ConversationCheckpoint& c, const void* who, uint8_t* dst, uint64_t n) {
    for (const std::vector<uint8_t>* v : {&c.gdn, &c.ple, &c.tails, &c.dead, &c.block_pos})
        if (v == who) {
            std::memcpy(dst, v->data(), size_t(n));
            return true;
        }
    for (const ConversationCheckpoint& part : c.stage_parts)
        if (stage_checkpoint_blob(part, who, dst, n)) return true;
    return false;
}
bool stage_host_blob(const SavedConversation& img, const void* who, uint8_t* dst, uint64_t n) {
    for (const ConversationKv& k : img.kv)
        for (const ConversationBuffer* b : {&k.k, &k.v, &k.k_scale, &k.v_scale, &k.pooled})
            if (b == who) return b->read(dst, 0, size_t(n));
    if (stage_checkpoint_blob(img.live, who, dst, n)) return true;
    for (const ConversationCheckpoint& c : img.checkpoints)
        if (stage_checkpoint_blob(c, who, dst, n)) return true;
    for (const ConversationStageSnapshot& part : img.stage_parts)
        if (stage_checkpoint_blob(part.state, who, dst, n)) return true;
    return false;
}

const detail::WireBlobAt* find(const std::vector<detail::WireBlobAt>& pool, const void* who);

// The K/V records of a slot's f16 layers for `tokens` tokens, sized (not held), appended to `sizes` and `device`.
void size_f16_records(std::vector<ConversationKv>& kv, const sc_geometry& g, const SlotShape& s, int64_t idx_dim,
                      detail::WireSizes& sizes, std::vector<const void*>& device) {
    for (int64_t j = 0; j < s.n_qsa; ++j) {
        ConversationKv& k = kv[size_t(j)];
        k.format = 0;
        k.cells = s.cells;
        k.heads = g.n_head_kv;
        k.head_dim = g.head_dim;
        k.page_size = g.page_size;
        k.pooled_rows = 0;
        k.idx_dim = idx_dim;
        sizes.push_back({&k.k, s.kv_bytes});
        sizes.push_back({&k.v, s.kv_bytes});
        if (s.kv_bytes) { device.push_back(&k.k); device.push_back(&k.v); }
    }
}

// Checks that the first s.n_qsa records of `kv` are a slot's f16 layers for `tokens` tokens, carried as whole K and V
// blobs, and notes where those blobs sit.
bool f16_records(const std::vector<ConversationKv>& kv, const sc_geometry& g, const SlotShape& s, int64_t tokens,
                 const std::vector<detail::WireBlobAt>& blobs, const std::string& whose, std::vector<uint64_t>& k_off,
                 std::vector<uint64_t>& v_off, std::vector<const void*>& device, std::string& error) {
    if (int64_t(kv.size()) < s.n_qsa) return refuse(error, whose + " carries fewer K/V records than its slot has layers");
    k_off.assign(size_t(s.n_qsa), 0);
    v_off.assign(size_t(s.n_qsa), 0);
    for (int64_t j = 0; j < s.n_qsa; ++j) {
        const ConversationKv& k = kv[size_t(j)];
        const std::string rec = whose + " K/V record " + std::to_string(j);
        if (k.format != 0 || k.cells != s.cells || k.heads != g.n_head_kv || k.head_dim != g.head_dim ||
            k.page_size != g.page_size || k.pooled_rows != 0)
            return refuse(error, rec + " is not the slot's f16 layer of " + std::to_string(tokens) + " tokens");
        const detail::WireBlobAt* kb = find(blobs, &k.k);
        const detail::WireBlobAt* vb = find(blobs, &k.v);
        if (s.kv_bytes && (!kb || !vb || kb->bytes != s.kv_bytes || vb->bytes != s.kv_bytes))
            return refuse(error, rec + " does not carry whole K and V blobs");
        if (find(blobs, &k.k_scale) || find(blobs, &k.v_scale) || find(blobs, &k.pooled))
            return refuse(error, rec + " carries scales or indexer rows");
        k_off[size_t(j)] = kb ? kb->offset : 0;
        v_off[size_t(j)] = vb ? vb->offset : 0;
        device.push_back(&k.k);
        device.push_back(&k.v);
    }
    return true;
}

const detail::WireBlobAt* find(const std::vector<detail::WireBlobAt>& pool, const void* who) {
    for (const auto& e : pool)
        if (e.who == who) return &e;
    return nullptr;
}

}  // namespace

// ---- encoder ---------------------------------------------------------------------------------------------------------

WireDeviceEncoder::~WireDeviceEncoder() { release(); }

// Waits for the last encode's launches, before anything they read is destroyed (a freed plan or map must not be in use:
// the library does not rely on the runtime's free waiting for the device).
void WireDeviceEncoder::settle() {
    if (launched_ && done_) (void) sc_event_sync(done_);
    launched_ = false;
}

// Records the encoder's event after an encode's launches (what settle() waits for).
bool WireDeviceEncoder::mark_launched(void* stream, std::string& error) {
    if (!done_ && !abi(sc_event_create(&done_), error, "encode event")) return false;
    if (!abi(sc_event_record(done_, stream), error, "encode event")) return false;
    launched_ = true;
    return true;
}

void WireDeviceEncoder::release() {
    settle();
    last_stream_ = nullptr;
    if (done_) sc_event_destroy(done_);
    done_ = nullptr;
    for (StagePlan& sp : stage_plans_)
        if (sp.plan) sc_plan_destroy(sp.plan);
    stage_plans_.clear();
    if (capture_) sc_plan_destroy(capture_);
    if (copies_) sc_plan_destroy(copies_);
    copies_ = nullptr;
    if (hash_map_) sc_hash_map_destroy(hash_map_);
    hash_map_ = nullptr;
    if (seg_map_) sc_hash_map_destroy(seg_map_);
    seg_map_ = nullptr;
    seg_target_.clear();
    seg_bytes_ = 0;
    if (staged_) sc_host_free(staged_);
    if (staged_dev_) sc_device_free(staged_dev_);
    if (hash_host_) sc_host_free(hash_host_);
    if (hash_ws_) sc_device_free(hash_ws_);
    capture_ = nullptr;
    staged_ = nullptr;
    staged_dev_ = nullptr;
    staged_rows_ = false;
    hash_host_ = nullptr;
    hash_ws_ = nullptr;
    capture_target_ = nullptr;
    uploads_.clear();
}

// The image the wire sees for a slot: geometry and flags from `conv`, `n_qsa` K/V records first (sized, not held), the
// trailing host records after them, then the live checkpoint and the retained checkpoints.
static void slot_image(const WireDeviceConversation& conv, int64_t n_qsa, SavedConversation& img) {
    img.geometry = conv.geometry;
    img.layer_lo = conv.layer_lo;
    img.layer_hi = conv.layer_hi;
    img.cvec = conv.cvec;
    // the K/V vector gets its final length before any buffer's address is taken
    img.kv.resize(size_t(n_qsa));
    img.kv.insert(img.kv.end(), conv.trailing_kv.begin(), conv.trailing_kv.end());
    img.live = conv.live;
    img.checkpoints = conv.checkpoints;
}

static bool check_conversation(const WireDeviceConversation& conv, int64_t tokens, std::string& error) {
    if (int64_t(conv.live.ids.size()) != tokens)
        return refuse(error, "the live checkpoint's id count is not the slot's token count");
    if (!conv.live.gdn.empty()) return refuse(error, "the live checkpoint's gdn blob is the slot's GDN rows; leave it empty");
    return true;
}

bool WireDeviceEncoder::stage(const SavedConversation& img, const std::vector<std::pair<const void*, uint64_t>>& sizes,
                              const std::vector<const void*>& device, const WireIdentity& identity,
                              std::vector<detail::WireBlobAt>& pool, std::string& error) {
    std::vector<uint8_t> head;
    if (!detail::wire_head(img, identity, sizes, head, pool, plan_, error)) return false;
    // Device blobs go to the capture plan; a zero range closes each one up to the next 64-byte boundary.  Host blobs
    // are staged with their own zero padding and copied in.
    zero_.clear();
    for (const void* who : device) {
        const detail::WireBlobAt* e = find(pool, who);
        if (!e) return refuse(error, "internal: a slot blob is missing from the pool");
        const uint64_t end = e->offset + e->bytes, padded = up64(end);
        if (padded > end) { zero_.push_back(end); zero_.push_back(padded - end); }
    }
    std::vector<const detail::WireBlobAt*> host;
    for (const auto& e : pool)
        if (std::find(device.begin(), device.end(), e.who) == device.end()) host.push_back(&e);
    staged_bytes_ = up64(head.size());
    for (const auto* e : host) staged_bytes_ += up64(e->bytes);
    int rc = sc_host_alloc(reinterpret_cast<void**>(&staged_), staged_bytes_ ? staged_bytes_ : 64);
    if (rc == SC_OK) rc = sc_host_alloc(reinterpret_cast<void**>(&hash_host_), 64);
    if (!abi(rc, error, "pinned staging")) return false;
    std::memset(staged_, 0, staged_bytes_);
    std::memcpy(staged_, head.data(), head.size());
    uploads_.push_back({0, head.size(), 0});
    uint64_t at = up64(head.size());
    for (const auto* e : host) {
        if (!stage_host_blob(img, e->who, staged_ + at, e->bytes)) return refuse(error, "internal: a host blob of the pool was not found");
        uploads_.push_back({e->offset, up64(e->bytes), at});
        at += up64(e->bytes);
    }
    // a device copy of the staged bytes, written into each payload by copy rows of the gather (no copy per encode)
    staged_rows_ = std::all_of(uploads_.begin(), uploads_.end(),
                               [](const Upload& u) { return u.offset % 16 == 0 && u.bytes % 16 == 0; });
    if (staged_rows_) {
        rc = sc_device_alloc(reinterpret_cast<void**>(&staged_dev_), staged_bytes_ ? staged_bytes_ : 64);
        if (rc == SC_OK) rc = sc_copy_async(staged_dev_, staged_, staged_bytes_, nullptr);
        if (rc == SC_OK) rc = sc_stream_sync(nullptr);
        if (!abi(rc, error, "device staging")) return false;
    }
    hash_ws_bytes_ = sc_fnv1a64_workspace_bytes(plan_.total_bytes);
    rc = sc_device_alloc(&hash_ws_, hash_ws_bytes_);
    return abi(rc, error, "hash workspace");
}

bool WireDeviceEncoder::plan(const sc_geometry& g, const sc_decode_slot& slot, int64_t tokens,
                             const WireDeviceConversation& conv, const WireIdentity& identity, std::string& error) {
    return plan(g, slot, tokens, conv, {}, identity, error);
}

bool WireDeviceEncoder::plan(const sc_geometry& g, const sc_decode_slot& slot, int64_t tokens,
                             const WireDeviceConversation& conv, const std::vector<WireDeviceStage>& stages,
                             const WireIdentity& identity, std::string& error) {
    release();
    plan_ = WirePlan{};
    SlotShape s;
    if (!slot_shape(g, tokens, s, error) || !check_conversation(conv, tokens, error)) return false;
    // the slot's layers as f16 K/V records whose buffers are sized, not held
    SavedConversation img;
    slot_image(conv, s.n_qsa, img);
    detail::WireSizes sizes;
    std::vector<const void*> device;
    size_f16_records(img.kv, g, s, conv.idx_dim, sizes, device);
    if (s.n_gdn > 0) {
        sizes.push_back({&img.live.gdn, s.gdn_bytes});
        device.push_back(&img.live.gdn);
    }
    // each later stage: a part whose K/V records and GDN rows are its own slot's, the rest its host running state
    std::vector<SlotShape> stage_shapes(stages.size());
    img.stage_parts.resize(stages.size());
    for (size_t i = 0; i < stages.size(); ++i) {
        const WireDeviceStage& st = stages[i];
        SlotShape& ss = stage_shapes[i];
        if (!slot_shape(st.geometry, tokens, ss, error)) return false;
        if (st.state.ids != conv.live.ids) return refuse(error, "a stage part's ids are not the live ids");
        if (!st.state.gdn.empty() || !st.state.imgs.empty() || !st.state.stage_parts.empty())
            return refuse(error, "a stage part's state carries only its small host buffers (its GDN rows are the slot's)");
        // checked before anything is staged: a refusal leaves the encoder without a plan
        if (st.slot.page_table)
            for (int64_t j = 0; j < ss.n_qsa; ++j)
                if (st.slot.page_table[j]) return refuse(error, "a stage slot must use identity page tables");
        ConversationStageSnapshot& part = img.stage_parts[i];
        part.layer_lo = st.layer_lo;
        part.layer_hi = st.layer_hi;
        part.state = st.state;
        part.kv.resize(size_t(ss.n_qsa));
        size_f16_records(part.kv, st.geometry, ss, conv.idx_dim, sizes, device);
        if (ss.n_gdn > 0) {
            sizes.push_back({&part.state.gdn, ss.gdn_bytes});
            device.push_back(&part.state.gdn);
        }
    }
    std::vector<detail::WireBlobAt> pool;
    if (!stage(img, sizes, device, identity, pool, error)) { release(); return false; }
    k_off_.assign(size_t(s.n_qsa), 0);
    v_off_.assign(size_t(s.n_qsa), 0);
    for (int64_t j = 0; j < s.n_qsa && s.kv_bytes; ++j) {
        k_off_[size_t(j)] = find(pool, &img.kv[size_t(j)].k)->offset;
        v_off_[size_t(j)] = find(pool, &img.kv[size_t(j)].v)->offset;
    }
    gdn_off_ = s.n_gdn > 0 ? find(pool, &img.live.gdn)->offset : 0;
    stage_plans_.resize(stages.size());
    for (size_t i = 0; i < stages.size(); ++i) {
        const WireDeviceStage& st = stages[i];
        const SlotShape& ss = stage_shapes[i];
        const ConversationStageSnapshot& part = img.stage_parts[i];
        StagePlan& sp = stage_plans_[i];
        sp.g = st.geometry;
        sp.slot = st.slot;
        // own copies of the stage slot's pointer arrays: the caller's may not outlive the encoder
        sp.k.assign(st.slot.k_pool ? st.slot.k_pool : nullptr, st.slot.k_pool ? st.slot.k_pool + ss.n_qsa : nullptr);
        sp.v.assign(st.slot.v_pool ? st.slot.v_pool : nullptr, st.slot.v_pool ? st.slot.v_pool + ss.n_qsa : nullptr);
        sp.slot.k_pool = st.slot.k_pool ? sp.k.data() : nullptr;
        sp.slot.v_pool = st.slot.v_pool ? sp.v.data() : nullptr;
        sp.slot.page_table = nullptr;
        sp.slot.host = sp.slot.stage = nullptr;
        sp.k_off.assign(size_t(ss.n_qsa), 0);
        sp.v_off.assign(size_t(ss.n_qsa), 0);
        for (int64_t j = 0; j < ss.n_qsa && ss.kv_bytes; ++j) {
            sp.k_off[size_t(j)] = find(pool, &part.kv[size_t(j)].k)->offset;
            sp.v_off[size_t(j)] = find(pool, &part.kv[size_t(j)].v)->offset;
        }
        sp.gdn_off = ss.n_gdn > 0 ? find(pool, &part.state.gdn)->offset : 0;
    }
    layered_ = false;
    g_ = g;
    slot_ = slot;
    tokens_ = tokens;
    return true;
}

bool WireDeviceEncoder::plan(const sc_geometry& g, const sc_slot_layers& slot, int64_t tokens,
                             const WireDeviceConversation& conv, const WireIdentity& identity, std::string& error) {
    release();
    plan_ = WirePlan{};
    SlotShape s;
    if (!slot_shape(g, tokens, s, error) || !check_conversation(conv, tokens, error)) return false;
    uint64_t b[SC_N_BUF];
    if (!abi(sc_layer_blob_bytes(&g, slot.format, slot.with_index, tokens, b), error, "K/V layout")) return false;
    // the slot's layers as K/V records of its format (data, scales, indexer rows) whose buffers are sized, not held
    SavedConversation img;
    slot_image(conv, s.n_qsa, img);
    detail::WireSizes sizes;
    std::vector<const void*> device;
    for (int64_t j = 0; j < s.n_qsa; ++j) {
        ConversationKv& k = img.kv[size_t(j)];
        k.format = slot.format;
        k.cells = s.cells;
        k.heads = g.n_head_kv;
        k.head_dim = g.head_dim;
        k.page_size = g.page_size;
        k.pooled_rows = int64_t(b[SC_BUF_POOLED] / (uint64_t(g.idx_key_dim) * 4));
        k.idx_dim = conv.idx_dim;
        const ConversationBuffer* bufs[SC_N_BUF] = {&k.k, &k.v, &k.k_scale, &k.v_scale, &k.pooled};
        for (int x = 0; x < SC_N_BUF; ++x) {
            sizes.push_back({bufs[x], b[x]});
            if (b[x]) device.push_back(bufs[x]);
        }
    }
    if (s.n_gdn > 0) {
        sizes.push_back({&img.live.gdn, s.gdn_bytes});
        device.push_back(&img.live.gdn);
    }
    std::vector<detail::WireBlobAt> pool;
    if (!stage(img, sizes, device, identity, pool, error)) { release(); return false; }
    lay_off_.assign(size_t(s.n_qsa) * SC_N_BUF + 1, ~uint64_t(0));
    for (int64_t j = 0; j < s.n_qsa; ++j) {
        const ConversationKv& k = img.kv[size_t(j)];
        const ConversationBuffer* bufs[SC_N_BUF] = {&k.k, &k.v, &k.k_scale, &k.v_scale, &k.pooled};
        for (int x = 0; x < SC_N_BUF; ++x)
            if (b[x]) lay_off_[size_t(j) * SC_N_BUF + size_t(x)] = find(pool, bufs[x])->offset;
    }
    if (s.n_gdn > 0) lay_off_.back() = find(pool, &img.live.gdn)->offset;
    // own copies of the slot's pointer arrays: the caller's may not outlive the encoder
    layers_ = slot;
    for (int x = 0; x < SC_N_BUF; ++x) {
        layer_bufs_[size_t(x)].assign(slot.buf[x] ? slot.buf[x] : nullptr, slot.buf[x] ? slot.buf[x] + s.n_qsa : nullptr);
        layers_.buf[x] = slot.buf[x] ? layer_bufs_[size_t(x)].data() : nullptr;
    }
    layered_ = true;
    g_ = g;
    tokens_ = tokens;
    return true;
}

bool WireDeviceEncoder::encode(void* payload, uint64_t capacity, void* stream, std::string& error, void* gathered) {
    if (!staged_) return refuse(error, "encode before a successful plan");
    if (!payload || capacity < plan_.total_bytes)
        return refuse(error, "the payload buffer holds " + std::to_string(capacity) + " bytes and the payload needs " +
                                 std::to_string(plan_.total_bytes));
    if (capture_target_ != payload) {
        settle();
        if (capture_) sc_plan_destroy(capture_);
        capture_ = nullptr;
        if (copies_) sc_plan_destroy(copies_);
        copies_ = nullptr;
        for (StagePlan& sp : stage_plans_) {
            if (sp.plan) sc_plan_destroy(sp.plan);
            sp.plan = nullptr;
        }
        if (hash_map_) sc_hash_map_destroy(hash_map_);
        hash_map_ = nullptr;
        capture_target_ = nullptr;
        std::vector<sc_plan*> plans;
        if (!capture_plans(payload, capacity, plans, error)) return false;
        capture_ = plans[0];
        for (size_t i = 0; i < stage_plans_.size(); ++i) stage_plans_[i].plan = plans[i + 1];
        if (staged_rows_) copies_ = plans.back();
        // the same rows as the sources of the fused gather + hash (with the head and the small host blobs as copy
        // rows, or, when they are not whole 16-byte chunks, copied in first and hashed as the payload holds them)
        if (!abi(sc_hash_map_create(plans.data(), int32_t(plans.size()), payload, plan_.total_bytes, &hash_map_), error,
                 "payload hash map"))
            return false;
        capture_target_ = payload;
    }
    uint8_t* p = static_cast<uint8_t*>(payload);
    if (!staged_rows_)
        for (const Upload& u : uploads_)
            if (!abi(sc_copy_async(p + u.offset, staged_ + u.staged_at, u.bytes, stream), error, "head copy"))
                return false;
    // the hash and its fault word go straight to pinned host memory (the last kernel's stores): no readback copy
    if (!gathered) {
        // one kernel gathers the slot's blobs into the payload and hashes the payload from its registers
        if (!abi(carry_ ? sc_hash_map_launch_carry(hash_map_, kWireHashSeed, hash_host_, hash_fault_host(), carry_,
                                                   hash_ws_, hash_ws_bytes_, stream)
                        : sc_hash_map_launch(hash_map_, kWireHashSeed, hash_host_, hash_fault_host(), hash_ws_,
                                             hash_ws_bytes_, stream),
                 error, "payload gather and hash"))
            return false;
    } else {
        // a caller that copies the payload out as soon as its bytes are in place (a checked park) gets the gather
        // first, the event, then the hash, so the copy overlaps the hash
        if (!abi(sc_plan_launch(capture_, stream), error, "pool gather")) return false;
        for (const StagePlan& sp : stage_plans_)
            if (!abi(sc_plan_launch(sp.plan, stream), error, "stage gather")) return false;
        if (copies_ && !abi(sc_plan_launch(copies_, stream), error, "head copy")) return false;
        if (!abi(sc_event_record(gathered, stream), error, "gather event")) return false;
        if (!abi(carry_ ? sc_fnv1a64_carry_async(payload, plan_.total_bytes, kWireHashSeed, hash_host_,
                                                 hash_fault_host(), carry_, hash_ws_, hash_ws_bytes_, stream)
                        : sc_fnv1a64_async(payload, plan_.total_bytes, kWireHashSeed, hash_host_, hash_fault_host(),
                                           hash_ws_, hash_ws_bytes_, stream),
                 error, "payload hash"))
            return false;
    }
    last_stream_ = stream;
    return mark_launched(stream, error);
}

bool WireDeviceEncoder::capture_plans(void* base, uint64_t capacity, std::vector<sc_plan*>& plans, std::string& error) {
    plans.clear();
    auto undo = [&] {
        for (sc_plan* q : plans) sc_plan_destroy(q);
        plans.clear();
        return false;
    };
    sc_plan* main = nullptr;
    int rc;
    if (layered_) {
        sc_layers_map map{lay_off_.data(), zero_.data(), int64_t(zero_.size() / 2)};
        rc = sc_plan_capture_layers(&g_, &layers_, tokens_, base, capacity, &map, &main);
    } else {
        sc_blob_map map{};
        map.k_off = k_off_.data();
        map.v_off = v_off_.data();
        map.gdn_off = gdn_off_;
        map.zero = zero_.data();
        map.n_zero = int64_t(zero_.size() / 2);
        rc = sc_plan_capture_map(&g_, &slot_, tokens_, base, capacity, &map, &main);
    }
    if (!abi(rc, error, "capture plan")) return false;
    plans.push_back(main);
    for (const StagePlan& sp : stage_plans_) {   // every gap of the pool is cleared by the main plan's zero ranges
        sc_blob_map map{};
        map.k_off = sp.k_off.data();
        map.v_off = sp.v_off.data();
        map.gdn_off = sp.gdn_off;
        sc_plan* q = nullptr;
        if (!abi(sc_plan_capture_map(&sp.g, &sp.slot, tokens_, base, capacity, &map, &q), error, "stage capture plan"))
            return undo();
        plans.push_back(q);
    }
    if (staged_rows_) {   // the head and the small host blobs from their device copy, last
        std::vector<sc_copy> copies;
        for (const Upload& u : uploads_)
            copies.push_back({static_cast<uint8_t*>(base) + u.offset, staged_dev_ + u.staged_at, u.bytes});
        sc_plan* q = nullptr;
        if (!abi(sc_plan_copies(copies.data(), int32_t(copies.size()), &q), error, "head copy plan")) return undo();
        plans.push_back(q);
    }
    return true;
}

bool WireDeviceEncoder::encode_segments(const sc_segments& into, void* stream, std::string& error) {
    if (!staged_) return refuse(error, "encode before a successful plan");
    if (into.n < 1 || !into.ptr || !into.segment_bytes) return refuse(error, "a segmented payload needs its segments");
    std::vector<void*> ptrs(into.ptr, into.ptr + into.n);
    if (!seg_map_ || ptrs != seg_target_ || into.segment_bytes != seg_bytes_) {
        settle();
        if (seg_map_) sc_hash_map_destroy(seg_map_);
        seg_map_ = nullptr;
        seg_target_.clear();
        // the plans are built for a contiguous payload framed at the first segment, never launched: the map takes
        // their rows as payload offsets and writes them into the segments
        std::vector<sc_plan*> plans;
        if (!capture_plans(ptrs[0], plan_.total_bytes, plans, error)) return false;
        const int rc = sc_hash_map_create_segments(plans.data(), int32_t(plans.size()), ptrs[0], plan_.total_bytes, &into,
                                                   &seg_map_);
        for (sc_plan* q : plans) sc_plan_destroy(q);
        if (!abi(rc, error, "segmented payload hash map")) return false;
        seg_target_ = ptrs;
        seg_bytes_ = into.segment_bytes;
    }
    // the head and the small host blobs (when the map does not write them), a piece per segment they touch
    if (!staged_rows_)
        for (const Upload& u : uploads_)
            for (uint64_t o = u.offset, end = u.offset + u.bytes; o < end;) {
                const uint64_t k = o / seg_bytes_, stop = std::min(end, (k + 1) * seg_bytes_);
                if (k >= ptrs.size()) return refuse(error, "the segments are smaller than the payload");
                if (!abi(sc_copy_async(static_cast<uint8_t*>(ptrs[size_t(k)]) + (o - k * seg_bytes_),
                                       staged_ + u.staged_at + (o - u.offset), stop - o, stream),
                         error, "head copy"))
                    return false;
                o = stop;
            }
    if (!abi(carry_ ? sc_hash_map_launch_carry(seg_map_, kWireHashSeed, hash_host_, hash_fault_host(), carry_, hash_ws_,
                                               hash_ws_bytes_, stream)
                    : sc_hash_map_launch(seg_map_, kWireHashSeed, hash_host_, hash_fault_host(), hash_ws_,
                                         hash_ws_bytes_, stream),
             error, "payload gather and hash"))
        return false;
    last_stream_ = stream;
    return mark_launched(stream, error);
}

bool WireDeviceEncoder::payload_hash(uint64_t& hash, std::string& error) {
    if (!hash_host_) return refuse(error, "no encode to read a hash from");
    if (!abi(sc_stream_sync(last_stream_), error, "encode")) return false;
    if (*hash_fault_host())   // a wait of the hash kernel ran out: the word at hash_host_ is not the payload's hash
        return refuse(error, "the payload hash did not complete on the device (a look-back wait ran out); encode again");
    hash = *hash_host_;
    return true;
}

// ---- decoder ---------------------------------------------------------------------------------------------------------

WireDeviceDecoder::~WireDeviceDecoder() { release(); }

void WireDeviceDecoder::drop_open() {
    opened_ = false;
    for (sc_plan* p : stage_scatters_)
        if (p) sc_plan_destroy(p);
    stage_scatters_.clear();
    seg_.clear();
    seg_bytes_ = 0;
    downloads_.clear();
    head_image_ = SavedConversation{};
    carry_ = nullptr;
}

void WireDeviceDecoder::release() {
    drop_open();
    if (scatter_) sc_plan_destroy(scatter_);
    if (read_map_) sc_hash_map_destroy(read_map_);
    read_map_ = nullptr;
    plan_key_.clear();
    map_key_.clear();
    if (hash_ws_) sc_device_free(hash_ws_);
    if (hash_dev_) sc_device_free(hash_dev_);
    if (hash_host_) sc_host_free(hash_host_);
    if (staged_) sc_host_free(staged_);
    if (head_pinned_) sc_host_free(head_pinned_);
    head_pinned_ = nullptr;
    head_cap_ = 0;
    if (ev_start_) sc_event_destroy(ev_start_);
    if (ev_done_) sc_event_destroy(ev_done_);
    if (side_) sc_stream_destroy(side_);
    scatter_ = nullptr;
    hash_ws_ = nullptr;
    hash_ws_bytes_ = 0;
    hash_dev_ = nullptr;
    hash_host_ = nullptr;
    staged_ = nullptr;
    staged_cap_ = 0;
    ev_start_ = ev_done_ = side_ = nullptr;
}

bool WireDeviceDecoder::copy_payload(void* dst, uint64_t off, uint64_t n, void* stream, std::string& error) {
    if (seg_.empty())
        return abi(sc_copy_async(dst, payload_ + off, n, stream), error, "payload read");
    for (uint64_t o = off, end = off + n; o < end;) {
        const uint64_t k = o / seg_bytes_, stop = std::min(end, (k + 1) * seg_bytes_);
        if (k >= seg_.size()) return refuse(error, "the payload runs past its segments");
        if (!abi(sc_copy_async(static_cast<uint8_t*>(dst) + (o - off),
                               static_cast<const uint8_t*>(seg_[size_t(k)]) + (o - k * seg_bytes_), stop - o, stream),
                 error, "payload read"))
            return false;
        o = stop;
    }
    return true;
}

bool WireDeviceDecoder::read_head(const void* payload, const sc_segments* segs, uint64_t bytes,
                                  const WireExpect& expect, std::vector<detail::WireBlobAt>& blobs, std::string& error) {
    drop_open();
    if (segs) {
        if (segs->n < 1 || !segs->ptr || !segs->segment_bytes || !segs->ptr[0])
            return refuse(error, "a segmented payload needs its segments");
        if (uint64_t(segs->n) * segs->segment_bytes < bytes) return refuse(error, "the segments are smaller than the payload");
        seg_.assign(segs->ptr, segs->ptr + segs->n);
        seg_bytes_ = segs->segment_bytes;
        payload = seg_[0];
    }
    payload_ = static_cast<const uint8_t*>(payload);
    if (!payload || bytes < kWireHeaderRecordBytes) return refuse(error, "the payload is shorter than the header record");
    // the payload may still be arriving on another stream: everything enqueued before this call completes first
    if (!abi(sc_device_sync(), error, "wait for the payload")) return false;
    // the head is read into pinned memory kept across opens (plain DMA, no bounce copies)
    auto head_room = [&](uint64_t need) {
        if (head_cap_ >= need) return true;
        if (head_pinned_) sc_host_free(head_pinned_);
        head_pinned_ = nullptr;
        head_cap_ = 0;
        const uint64_t cap = std::max<uint64_t>(need, uint64_t(1) << 20);
        if (!abi(sc_host_alloc(reinterpret_cast<void**>(&head_pinned_), cap), error, "head staging")) return false;
        head_cap_ = cap;
        return true;
    };
    if (!head_room(kWireHeaderRecordBytes)) return false;
    if (!copy_payload(head_pinned_, 0, kWireHeaderRecordBytes, nullptr, error) ||
        !abi(sc_device_sync(), error, "head read"))
        return false;
    WireHeaderRecord h{};
    if (!conversation_wire_peek(head_pinned_, kWireHeaderRecordBytes, h, error)) return false;
    if (h.blob_pool_off > bytes) return refuse(error, "the blob pool starts past the end of the buffer");
    if (!head_room(h.blob_pool_off)) return false;
    if (!copy_payload(head_pinned_, 0, h.blob_pool_off, nullptr, error) || !abi(sc_device_sync(), error, "head read"))
        return false;
    const uint8_t* head_bytes = head_pinned_;
    const uint64_t head_len = h.blob_pool_off;
    // every check of the host decoder, against the real buffer size
    WireExpect bounded = expect;
    if (!bounded.max_payload_bytes || bounded.max_payload_bytes > bytes) bounded.max_payload_bytes = bytes;
    head_image_ = SavedConversation{};
    if (!detail::wire_locate(head_bytes, head_len, head_image_, info_, bounded, blobs, error)) return false;
    tokens_ = info_.live_tokens;
    return true;
}

bool WireDeviceDecoder::finish_open(const void* payload, uint64_t bytes, const WireExpect& expect,
                                    const std::vector<detail::WireBlobAt>& blobs, const std::vector<const void*>& device,
                                    std::string& error) {
    uint64_t staged = 0;
    for (const auto& b : blobs) {
        if (std::find(device.begin(), device.end(), b.who) != device.end()) continue;
        bool buffer = false;
        for (const ConversationKv& k : head_image_.kv)
            for (const ConversationBuffer* x : {&k.k, &k.v, &k.k_scale, &k.v_scale, &k.pooled}) buffer |= x == b.who;
        downloads_.push_back({const_cast<void*>(b.who), buffer, b.offset, b.bytes, staged});
        staged += up64(b.bytes);
    }
    // The host blobs are read into pinned staging on a stream of their own, beside the hash and the scatter (pinned
    // reads are plain DMA; reads into pageable memory would each wait for a bounce copy), and handed out after the
    // verdict is read.
    // the buffers of an earlier open are kept when they are large enough
    int rc = SC_OK;
    const uint64_t need = staged ? staged : 64;
    if (staged_cap_ < need) {
        if (staged_) sc_host_free(staged_);
        staged_ = nullptr;
        staged_cap_ = 0;
        rc = sc_host_alloc(reinterpret_cast<void**>(&staged_), need);
        if (rc == SC_OK) staged_cap_ = need;
    }
    if (rc == SC_OK && !side_) rc = sc_stream_create(&side_);
    if (rc == SC_OK && !ev_start_) rc = sc_event_create(&ev_start_);
    if (rc == SC_OK && !ev_done_) rc = sc_event_create(&ev_done_);
    if (!abi(rc, error, "host blob staging")) { release(); return false; }
    if (expect.check_payload_hash) {
        const uint64_t ws = sc_fnv1a64_workspace_bytes(info_.bytes);
        if (hash_ws_bytes_ < ws) {
            if (hash_ws_) sc_device_free(hash_ws_);
            hash_ws_ = nullptr;
            hash_ws_bytes_ = 0;
            rc = sc_device_alloc(&hash_ws_, ws);
            if (rc == SC_OK) hash_ws_bytes_ = ws;
        }
        if (rc == SC_OK && !hash_dev_) rc = sc_device_alloc(reinterpret_cast<void**>(&hash_dev_), 64);
        if (rc == SC_OK && !hash_host_) rc = sc_host_alloc(reinterpret_cast<void**>(&hash_host_), 64);
        if (rc == SC_OK && !seg_.empty()) {   // a segmented payload is hashed where it lies, in one launch
            std::vector<uint8_t> key;
            put_key(key, seg_bytes_);
            put_key(key, info_.bytes);
            for (void* q : seg_) put_key(key, q);
            if (!read_map_ || key != map_key_) {
                if (read_map_) sc_hash_map_destroy(read_map_);
                read_map_ = nullptr;
                map_key_.clear();
                const sc_segments segs = segments();
                rc = sc_hash_map_create_read(&segs, info_.bytes, &read_map_);
                if (rc == SC_OK) map_key_ = key;
            }
        }
        if (!abi(rc, error, "hash workspace")) { release(); return false; }
    }
    (void) payload;
    bytes_ = bytes;
    expect_ = expect;
    opened_ = true;
    return true;
}

bool WireDeviceDecoder::open(const void* payload, uint64_t bytes, const sc_geometry& g, const sc_decode_slot& slot,
                             const WireExpect& expect, std::string& error) {
    return open_f16(payload, nullptr, bytes, g, slot, {}, expect, error);
}

bool WireDeviceDecoder::open(const void* payload, uint64_t bytes, const sc_geometry& g, const sc_decode_slot& slot,
                             const std::vector<WireDeviceStage>& stages, const WireExpect& expect, std::string& error) {
    return open_f16(payload, nullptr, bytes, g, slot, stages, expect, error);
}

bool WireDeviceDecoder::open(const sc_segments& from, uint64_t bytes, const sc_geometry& g, const sc_decode_slot& slot,
                             const std::vector<WireDeviceStage>& stages, const WireExpect& expect, std::string& error) {
    return open_f16(nullptr, &from, bytes, g, slot, stages, expect, error);
}

bool WireDeviceDecoder::open(const void* payload, uint64_t bytes, const sc_geometry& g, const sc_slot_layers& slot,
                             const WireExpect& expect, std::string& error) {
    return open_layers(payload, nullptr, bytes, g, slot, expect, error);
}

bool WireDeviceDecoder::open(const sc_segments& from, uint64_t bytes, const sc_geometry& g, const sc_slot_layers& slot,
                             const WireExpect& expect, std::string& error) {
    return open_layers(nullptr, &from, bytes, g, slot, expect, error);
}

bool WireDeviceDecoder::open_f16(const void* payload, const sc_segments* segs, uint64_t bytes, const sc_geometry& g,
                                 const sc_decode_slot& slot, const std::vector<WireDeviceStage>& stages,
                                 const WireExpect& expect, std::string& error) {
    std::vector<detail::WireBlobAt> blobs;
    if (!read_head(payload, segs, bytes, expect, blobs, error)) return false;
    payload = payload_;
    if (info_.n_stage_parts != int64_t(stages.size()))
        return refuse(error, stages.empty() ? "a layer-split image cannot be mounted on the device path without its "
                                              "stages' slots"
                                            : "the payload carries " + std::to_string(info_.n_stage_parts) +
                                                  " stage parts and " + std::to_string(stages.size()) +
                                                  " stage slots were given");
    SlotShape s;
    if (!slot_shape(g, tokens_, s, error)) return false;
    std::vector<uint64_t> k_off, v_off;
    std::vector<const void*> device;
    if (!f16_records(head_image_.kv, g, s, tokens_, blobs, "the payload", k_off, v_off, device, error)) return false;
    const detail::WireBlobAt* gb = find(blobs, &head_image_.live.gdn);
    if (s.n_gdn > 0 && (!gb || gb->bytes != s.gdn_bytes))
        return refuse(error, "the live checkpoint does not carry the slot's GDN rows");
    device.push_back(&head_image_.live.gdn);
    // every stage part against its slot, checked before any plan is built
    struct Part { SlotShape shape; std::vector<uint64_t> k_off, v_off; uint64_t gdn_off; };
    std::vector<Part> parts(stages.size());
    for (size_t i = 0; i < stages.size(); ++i) {
        const WireDeviceStage& st = stages[i];
        const ConversationStageSnapshot& part = head_image_.stage_parts[i];
        const std::string whose = "stage part " + std::to_string(i);
        if (part.layer_lo != st.layer_lo || part.layer_hi != st.layer_hi)
            return refuse(error, whose + " covers layers [" + std::to_string(part.layer_lo) + ", " +
                                     std::to_string(part.layer_hi) + "), not its slot's");
        if (!slot_shape(st.geometry, tokens_, parts[i].shape, error)) return false;
        if (int64_t(part.kv.size()) != parts[i].shape.n_qsa)
            return refuse(error, whose + " does not carry one K/V record per layer of its slot");
        if (!f16_records(part.kv, st.geometry, parts[i].shape, tokens_, blobs, whose, parts[i].k_off, parts[i].v_off,
                         device, error))
            return false;
        const detail::WireBlobAt* sg = find(blobs, &part.state.gdn);
        if (parts[i].shape.n_gdn > 0 && (!sg || sg->bytes != parts[i].shape.gdn_bytes))
            return refuse(error, whose + " does not carry its slot's GDN rows");
        parts[i].gdn_off = sg ? sg->offset : 0;
        device.push_back(&part.state.gdn);
    }
    sc_blob_map map{};
    map.k_off = k_off.data();
    map.v_off = v_off.data();
    map.gdn_off = gb ? gb->offset : 0;
    const sc_segments from = segments();
    auto scatter_plan = [&](const sc_geometry& sg, const sc_blob_map& m, const sc_decode_slot& s, sc_plan** out) {
        return seg_.empty() ? sc_plan_scatter_map(&sg, payload, bytes, &m, tokens_, &s, out)
                            : sc_plan_scatter_map_segments(&sg, &from, bytes, &m, tokens_, &s, out);
    };
    // the plan is kept for the next open of the same payload place, slot and blob offsets (no stages)
    std::vector<uint8_t> key;
    if (stages.empty()) {
        put_key(key, int32_t(1));
        put_key(key, g.n_layers);
        put_key(key, g.qsa_interval);
        put_key(key, g.n_head_kv);
        put_key(key, g.head_dim);
        put_key(key, g.page_size);
        put_key(key, g.ssm_state_size);
        put_key(key, g.ssm_k_heads);
        put_key(key, g.ssm_v_heads);
        put_key(key, g.ssm_d_conv);
        put_key(key, g.ssm_conv_channels);
        put_key(key, g.idx_key_dim);
        put_key(key, slot.n_pages);
        put_key(key, slot.max_cells);
        put_key(key, slot.gdn_state);
        for (int64_t j = 0; j < s.n_qsa; ++j) {
            put_key(key, slot.k_pool[j]);
            put_key(key, slot.v_pool[j]);
            put_key(key, slot.page_table ? slot.page_table[j] : nullptr);
            if (slot.host) put_key(key, slot.host[j]);
            if (slot.stage) put_key(key, slot.stage[j]);
        }
        put_key(key, slot.host != nullptr);
        put_key(key, slot.stage != nullptr);
        put_key(key, payload);
        put_key(key, bytes);
        put_key(key, seg_bytes_);
        for (void* q : seg_) put_key(key, q);
        put_key(key, tokens_);
        put_key(key, map.gdn_off);
        for (uint64_t o : k_off) put_key(key, o);
        for (uint64_t o : v_off) put_key(key, o);
    }
    if (key.empty() || !scatter_ || key != plan_key_) {
        if (scatter_) sc_plan_destroy(scatter_);
        scatter_ = nullptr;
        plan_key_.clear();
        if (!abi(scatter_plan(g, map, slot, &scatter_), error, "scatter plan")) {
            release();
            return false;
        }
        plan_key_ = key;
    }
    stage_scatters_.assign(stages.size(), nullptr);
    for (size_t i = 0; i < stages.size(); ++i) {
        sc_blob_map pm{};
        pm.k_off = parts[i].k_off.data();
        pm.v_off = parts[i].v_off.data();
        pm.gdn_off = parts[i].gdn_off;
        if (!abi(scatter_plan(stages[i].geometry, pm, stages[i].slot, &stage_scatters_[i]), error, "stage scatter plan")) {
            release();
            return false;
        }
    }
    return finish_open(payload, bytes, expect, blobs, device, error);
}

bool WireDeviceDecoder::open_layers(const void* payload, const sc_segments* segs, uint64_t bytes, const sc_geometry& g,
                                    const sc_slot_layers& slot, const WireExpect& expect, std::string& error) {
    std::vector<detail::WireBlobAt> blobs;
    if (!read_head(payload, segs, bytes, expect, blobs, error)) return false;
    payload = payload_;
    if (info_.n_stage_parts) return refuse(error, "a layer-split image cannot be mounted into a single layered slot");
    SlotShape s;
    if (!slot_shape(g, tokens_, s, error)) return false;
    uint64_t b[SC_N_BUF];
    if (!abi(sc_layer_blob_bytes(&g, slot.format, slot.with_index, tokens_, b), error, "K/V layout")) return false;
    if (int64_t(head_image_.kv.size()) < s.n_qsa)
        return refuse(error, "the payload carries fewer K/V records than the slot has layers");
    const int64_t pooled_rows = int64_t(b[SC_BUF_POOLED] / (uint64_t(g.idx_key_dim) * 4));
    std::vector<uint64_t> off(size_t(s.n_qsa) * SC_N_BUF + 1, ~uint64_t(0));
    std::vector<const void*> device;
    for (int64_t j = 0; j < s.n_qsa; ++j) {
        const ConversationKv& k = head_image_.kv[size_t(j)];
        if (k.format != slot.format || k.cells != s.cells || k.heads != g.n_head_kv || k.head_dim != g.head_dim ||
            k.page_size != g.page_size || k.pooled_rows != pooled_rows)
            return refuse(error, "K/V record " + std::to_string(j) + " is not the slot's layer (format " +
                                     std::to_string(slot.format) + ", " + std::to_string(tokens_) + " tokens)");
        const ConversationBuffer* bufs[SC_N_BUF] = {&k.k, &k.v, &k.k_scale, &k.v_scale, &k.pooled};
        for (int x = 0; x < SC_N_BUF; ++x) {
            const detail::WireBlobAt* e = find(blobs, bufs[x]);
            if (b[x] ? (!e || e->bytes != b[x]) : e != nullptr)
                return refuse(error, "K/V record " + std::to_string(j) + " does not carry the slot format's blobs");
            if (e) {
                off[size_t(j) * SC_N_BUF + size_t(x)] = e->offset;
                device.push_back(bufs[x]);
            }
        }
    }
    const detail::WireBlobAt* gb = find(blobs, &head_image_.live.gdn);
    if (s.n_gdn > 0 && (!gb || gb->bytes != s.gdn_bytes))
        return refuse(error, "the live checkpoint does not carry the slot's GDN rows");
    if (gb) off.back() = gb->offset;
    device.push_back(&head_image_.live.gdn);
    sc_layers_map map{off.data(), nullptr, 0};
    const sc_segments from = segments();
    // the plan is kept for the next open of the same payload place, slot and blob offsets
    std::vector<uint8_t> key;
    put_key(key, int32_t(2));
    put_key(key, g.n_layers);
    put_key(key, g.qsa_interval);
    put_key(key, g.n_head_kv);
    put_key(key, g.head_dim);
    put_key(key, g.page_size);
    put_key(key, g.ssm_state_size);
    put_key(key, g.ssm_k_heads);
    put_key(key, g.ssm_v_heads);
    put_key(key, g.ssm_d_conv);
    put_key(key, g.ssm_conv_channels);
    put_key(key, g.idx_key_dim);
    put_key(key, slot.format);
    put_key(key, slot.with_index);
    put_key(key, slot.max_cells);
    put_key(key, slot.pooled_capacity);
    put_key(key, slot.gdn_state);
    for (int x = 0; x < SC_N_BUF; ++x)
        for (int64_t j = 0; j < s.n_qsa; ++j) put_key(key, slot.buf[x] ? slot.buf[x][j] : nullptr);
    put_key(key, payload);
    put_key(key, bytes);
    put_key(key, seg_bytes_);
    for (void* q : seg_) put_key(key, q);
    put_key(key, tokens_);
    for (uint64_t o : off) put_key(key, o);
    if (!scatter_ || key != plan_key_) {
        if (scatter_) sc_plan_destroy(scatter_);
        scatter_ = nullptr;
        plan_key_.clear();
        const int rc = seg_.empty() ? sc_plan_scatter_layers(&g, payload, bytes, &map, tokens_, &slot, &scatter_)
                                    : sc_plan_scatter_layers_segments(&g, &from, bytes, &map, tokens_, &slot, &scatter_);
        if (!abi(rc, error, "scatter plan")) {
            release();
            return false;
        }
        plan_key_ = key;
    }
    return finish_open(payload, bytes, expect, blobs, device, error);
}

bool WireDeviceDecoder::restore(void* stream, SavedConversation& image, std::string& error) {
    if (!opened_ || !scatter_) return refuse(error, "restore before a successful open");
    // The payload hash is checked on the device: the hash's last kernel compares it with the expected one and leaves a
    // verdict word that gates the scatter, so a mismatch writes nothing and there is no host round trip before the
    // scatter; the host reads the hash back with the other small blobs, once, at the end.
    uint32_t* verdict = reinterpret_cast<uint32_t*>(hash_dev_ + 1);
    // host blobs are read on the side stream once everything before this call on `stream` (the payload's arrival) is
    // done: the point is marked here, and the side stream is set up after the hash is enqueued (a wait between streams
    // and the first launch after it cost the host ~30 us, the GPU idle meanwhile); with no host blob to read there is
    // no side stream work at all
    const bool side = std::any_of(downloads_.begin(), downloads_.end(), [](const Download& d) { return d.bytes != 0; });
    if (side && !abi(sc_event_record(ev_start_, stream), error, "restore start")) return false;
    // the hash itself goes straight to pinned host memory (the last kernel's store), the verdict stays on the device
    int hrc = SC_OK;
    if (expect_.check_payload_hash) {
        const uint64_t want = expect_.payload_hash;
        if (read_map_)
            hrc = carry_ ? sc_hash_map_check_carried_async(read_map_, kWireHashSeed, want, carry_, hash_host_, verdict,
                                                           hash_fault_host(), hash_ws_, hash_ws_bytes_, stream)
                         : sc_hash_map_check_async(read_map_, kWireHashSeed, want, hash_host_, verdict,
                                                   hash_fault_host(), hash_ws_, hash_ws_bytes_, stream);
        else
            hrc = carry_ ? sc_fnv1a64_check_carried_async(payload_, info_.bytes, kWireHashSeed, want, carry_, hash_host_,
                                                          verdict, hash_fault_host(), hash_ws_, hash_ws_bytes_, stream)
                         : sc_fnv1a64_check_async(payload_, info_.bytes, kWireHashSeed, want, hash_host_, verdict,
                                                  hash_fault_host(), hash_ws_, hash_ws_bytes_, stream);
    }
    if (!abi(hrc, error, "payload hash")) return false;
    if (side) {
        if (!abi(sc_stream_wait_event(side_, ev_start_), error, "restore start")) return false;
        for (const Download& d : downloads_)
            if (d.bytes && !copy_payload(staged_ + d.staged_at, d.offset, d.bytes, side_, error)) return false;
        if (!abi(sc_event_record(ev_done_, side_), error, "blob read")) return false;
    }
    SavedConversation out = head_image_;
    // the same blobs inside the copy: re-point the downloads by position
    auto remap = [&](void* who) -> void* {
        for (size_t i = 0; i < head_image_.kv.size(); ++i) {
            ConversationKv& a = head_image_.kv[i];
            ConversationKv& b = out.kv[i];
            if (who == &a.k) return &b.k;
            if (who == &a.v) return &b.v;
            if (who == &a.k_scale) return &b.k_scale;
            if (who == &a.v_scale) return &b.v_scale;
            if (who == &a.pooled) return &b.pooled;
        }
        std::vector<std::pair<ConversationCheckpoint*, ConversationCheckpoint*>> cps{{&head_image_.live, &out.live}};
        for (size_t i = 0; i < head_image_.checkpoints.size(); ++i)
            cps.push_back({&head_image_.checkpoints[i], &out.checkpoints[i]});
        for (size_t i = 0; i < head_image_.stage_parts.size(); ++i)
            cps.push_back({&head_image_.stage_parts[i].state, &out.stage_parts[i].state});
        for (size_t i = 0; i < cps.size(); ++i)
            for (size_t k = 0; k < cps[i].first->stage_parts.size(); ++k)
                cps.push_back({&cps[i].first->stage_parts[k], &cps[i].second->stage_parts[k]});
        for (auto& [a, b] : cps) {
            if (who == &a->gdn) return &b->gdn;
            if (who == &a->ple) return &b->ple;
            if (who == &a->tails) return &b->tails;
            if (who == &a->dead) return &b->dead;
            if (who == &a->block_pos) return &b->block_pos;
        }
        return nullptr;
    };
    for (sc_plan* p : stage_scatters_) {   // the stages' parts share the main scatter's verdict: all or nothing
        if (expect_.check_payload_hash ? !abi(sc_plan_launch_gated(p, verdict, stream), error, "stage scatter")
                                       : !abi(sc_plan_launch(p, stream), error, "stage scatter"))
            return false;
    }
    if (expect_.check_payload_hash ? !abi(sc_plan_launch_gated(scatter_, verdict, stream), error, "pool scatter")
                                   : !abi(sc_plan_launch(scatter_, stream), error, "pool scatter"))
        return false;
    // the caller's stream covers the whole restore, the side stream's reads included
    if ((side && !abi(sc_stream_wait_event(stream, ev_done_), error, "restore")) ||
        !abi(sc_stream_sync(stream), error, "restore"))
        return false;
    if (expect_.check_payload_hash) {
        // the device verdict that gated the scatters is exactly (hash == expected && no fault); the same two words are
        // in pinned memory, so the host decides as the scatters did, and a 0 verdict means they wrote nothing
        if (*hash_fault_host() & SC_FNV_FAULT_CARRY)
            return refuse(error, "the payload or its carries are not what was hashed (a 64 KiB piece of the payload "
                                 "does not end with its carry); nothing was mounted");
        if (*hash_fault_host())
            return refuse(error, "the payload hash did not complete on the device (a look-back wait ran out); nothing "
                                 "was mounted");
        if (*hash_host_ != expect_.payload_hash)
            return refuse(error, "payload hash mismatch on the device (the bytes are not the bytes that were written)");
        info_.payload_hash = *hash_host_;
    }
    for (const Download& d : downloads_) {
        void* target = remap(d.who);
        if (!target) return refuse(error, "internal: a host blob lost its place");
        const uint8_t* src = staged_ + d.staged_at;
        if (d.buffer) {
            auto* b = static_cast<ConversationBuffer*>(target);
            b->resize(size_t(d.bytes));
            b->visit(0, size_t(d.bytes), [&](uint8_t* p, size_t n, size_t at) {
                std::memcpy(p, src + at, n);
                return true;
            });
        } else {
            auto* v = static_cast<std::vector<uint8_t>*>(target);
            v->resize(size_t(d.bytes));
            if (d.bytes) std::memcpy(v->data(), src, size_t(d.bytes));
        }
    }
    image = std::move(out);
    return true;
}

}  // namespace strata::core

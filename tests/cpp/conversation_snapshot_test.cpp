// conversation_snapshot_test.cpp - park and mount through the C++ host layer on one GPU.
//
// The scenarios of the reference's device test (src/core/conversation_snapshot_test.cpp): real device pools and
// pinned host copies in f16 / int8 / q4_0 / hybrid K8V4 x resident / streamed / ring, a whole session saved as A,
// overwritten as B, a refused restore that must leave B untouched, a restore of A that must read back as A (the
// A/B/A exactness the engine's STRATA_STATE_HASH recipe checks), incremental re-capture after growth and rewind,
// the checkpoint's spare-row rebuild and PLE window, and a two-stage layer split carved on one device.
// Every buffer comes from libsc_handoff.so's C-ABI; every check failure exits non-zero with its label.
#include "strata/core/conversation_snapshot.hpp"
#include "strata/kernels/kv_stream.hpp"

#include "sc_handoff.h"

#include <algorithm>
#include <array>
#include <cstdio>
#include <limits>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

using namespace strata::core;
using namespace strata::kernels;

namespace {

int checks = 0;
void check(bool ok, const std::string& label) {
    ++checks;
    if (!ok) {
        std::fprintf(stderr, "FAIL: %s\n", label.c_str());
        std::exit(1);
    }
}
void abi(int rc, const char* what) {
    if (rc != SC_OK) {
        std::fprintf(stderr, "C-ABI %s: %s\n", what, sc_last_error());
        std::exit(1);
    }
}
void upload(void* dst, const void* src, size_t n) {
    abi(sc_copy_async(dst, src, n, nullptr), "upload");
    abi(sc_device_sync(), "sync");
}
void download(void* dst, const void* src, size_t n) {
    abi(sc_copy_async(dst, src, n, nullptr), "download");
    abi(sc_device_sync(), "sync");
}
void memset_dev(void* p, uint8_t v, size_t n) {
    abi(sc_fill_bytes_async(p, v, n, nullptr), "fill");
    abi(sc_device_sync(), "sync");
}

constexpr int kHybrid = 3;

// One QSA layer's state: slot pools on the device, the authoritative host copy for modes 1 and 2.
struct Layer {
    ModelGeometry g;
    QsaState st;
    std::vector<void*> device, host;
    std::array<void*, 5> sources{};
    std::array<size_t, 5> sizes{};

    template <class T> void alloc(T*& p, size_t n, bool pinned = false) {
        if (!n) return;
        void* raw = nullptr;
        if (pinned) { abi(sc_host_alloc(&raw, n), "host alloc"); host.push_back(raw); }
        else { abi(sc_device_alloc(&raw, n), "device alloc"); device.push_back(raw); }
        p = static_cast<T*>(raw);
    }

    Layer(int fmt, int mode) {
        st.kv_mode = mode;
        st.kv_int8 = fmt == kKvInt8;
        st.kv_q4 = fmt == kKvQ4;
        st.kv_hybrid = fmt == kHybrid;
        st.n_pages = 24;
        st.n_slots = mode ? 4 : st.n_pages;
        st.max_cells = st.n_pages * 4;
        st.idx_pooled_rows = mode == 2 ? 2 : st.max_cells / 4 + 2;
        const size_t per = fmt == kKvQ4 ? kv_q4_bytes_per_head(int(g.head_dim))
                                        : size_t(g.head_dim) * ((st.kv_int8 || st.kv_hybrid) ? 1 : 2);
        const size_t rows = size_t(st.max_cells * g.n_head_kv), slot_rows = size_t(st.n_slots * 4 * g.n_head_kv);
        const size_t scales = rows * size_t(g.head_dim / 64) * 2, slot_scales = slot_rows * size_t(g.head_dim / 64) * 2;
        sizes = {rows * per, rows * per, fmt == kKvInt8 ? scales : 0, fmt == kKvInt8 ? scales : 0,
                 size_t(st.idx_pooled_rows) * size_t(g.idx_key_dim) * 4};
        if (fmt == kHybrid) {
            sizes = {rows * per, rows * kv_q4_bytes_per_head(int(g.head_dim)), scales, 0, sizes[4]};
            alloc(st.k_q, sizes[0]); alloc(st.v_q4, sizes[1]); alloc(st.k_scale, sizes[2]);
            sources = {st.k_q, st.v_q4, st.k_scale, nullptr, nullptr};
        } else if (fmt == kKvQ4) {
            alloc(st.k_q4, slot_rows * per); alloc(st.v_q4, slot_rows * per);
            if (mode) { alloc(st.host.k_q4, sizes[0], true); alloc(st.host.v_q4, sizes[1], true); }
            sources = {mode ? st.host.k_q4 : st.k_q4, mode ? st.host.v_q4 : st.v_q4, nullptr, nullptr, nullptr};
        } else if (fmt == kKvInt8) {
            alloc(st.k_q, slot_rows * per); alloc(st.v_q, slot_rows * per);
            alloc(st.k_scale, slot_scales); alloc(st.v_scale, slot_scales);
            if (mode) {
                alloc(st.host.k_q, sizes[0], true); alloc(st.host.v_q, sizes[1], true);
                alloc(st.host.k_scale, sizes[2], true); alloc(st.host.v_scale, sizes[3], true);
            }
            sources = {mode ? (void*) st.host.k_q : (void*) st.k_q, mode ? (void*) st.host.v_q : (void*) st.v_q,
                       mode ? st.host.k_scale : st.k_scale, mode ? st.host.v_scale : st.v_scale, nullptr};
        } else {
            alloc(st.k_pool, slot_rows * per); alloc(st.v_pool, slot_rows * per);
            if (mode) { alloc(st.host.k_pool, sizes[0], true); alloc(st.host.v_pool, sizes[1], true); }
            sources = {mode ? st.host.k_pool : st.k_pool, mode ? st.host.v_pool : st.v_pool, nullptr, nullptr, nullptr};
        }
        alloc(st.idx_pooled, sizes[4]);
        sources[4] = st.idx_pooled;
        alloc(st.page_table, size_t(st.n_pages) * 4);
        if (mode == 1) {
            auto& m = st.map;
            m.page_table = st.page_table; m.n_blocks = st.n_pages; m.n_slots = st.n_slots;
            alloc(m.slot_block, size_t(st.n_slots) * 4); alloc(m.slot_stamp, size_t(st.n_slots) * 4);
            alloc(m.slot_ref, size_t(st.n_slots) * 4); alloc(m.miss_block, size_t(st.n_slots) * 4);
            alloc(m.miss_slot, size_t(st.n_slots) * 4); alloc(m.ctl, size_t(kKvCtlInts) * 4);
        } else if (mode == 2) {
            kv_ring_table(st.page_table, st.n_pages, st.n_slots, nullptr);
            abi(sc_device_sync(), "sync");
        }
    }
    // A deterministic pattern per buffer and salt; distinct salts give distinct bytes everywhere.
    void fill(uint8_t salt) {
        for (size_t i = 0; i < sources.size(); ++i) {
            std::vector<uint8_t> data(sizes[i]);
            for (size_t j = 0; j < data.size(); ++j) data[j] = uint8_t(salt + i * 31 + j * 7 + j / 257);
            if (!data.empty()) upload(sources[i], data.data(), data.size());
        }
    }
    // Overwrites everything from the page (or indexer row) of `first_dirty` on.
    void fill_after(uint8_t salt, int64_t first_dirty) {
        for (size_t i = 0; i < sources.size(); ++i) {
            const size_t offset = i == 4 ? size_t(first_dirty / 4) * size_t(g.idx_key_dim) * 4
                                         : sizes[i] / size_t(st.max_cells) * size_t(first_dirty / 4 * 4);
            if (sizes[i] > offset) {
                std::vector<uint8_t> data(sizes[i] - offset, salt);
                upload(static_cast<uint8_t*>(sources[i]) + offset, data.data(), data.size());
            }
        }
    }
    ~Layer() {
        for (void* p : device) sc_device_free(p);
        for (void* p : host) sc_host_free(p);
    }
};

bool same(const ConversationKv& a, const ConversationKv& b) {
    return a.k == b.k && a.v == b.v && a.k_scale == b.k_scale && a.v_scale == b.v_scale && a.pooled == b.pooled;
}

// Running state of a session on the device: GDN rows, PLE history, and the indexer's per-layer state.
struct RunningState {
    std::vector<void*> device;
    void* get(size_t n) {
        void* p = nullptr;
        abi(sc_device_alloc(&p, n ? n : 16), "device alloc");
        device.push_back(p);
        return p;
    }
    ~RunningState() { for (void* p : device) sc_device_free(p); }
};

void full_session(int fmt, int mode, int64_t experts) {
    const std::string tag = " [fmt " + std::to_string(fmt) + " mode " + std::to_string(mode) + " experts " +
                            std::to_string(experts) + "]";
    Layer main(fmt, mode), draft(fmt == kHybrid ? int(kKvInt8) : fmt, 2);
    ModelGeometry& g = main.g;
    g.n_layers = 4;
    g.n_expert = experts;
    g.ssm_state_size = 2; g.ssm_v_heads = 2; g.ssm_conv_channels = 8;
    SessionState ss;
    ss.max_cells = 96;
    ss.qsa_states = &main.st;
    ss.layer_hi = g.n_layers; ss.gdn_alloc = g.n_gdn_layers(); ss.qsa_alloc = g.n_qsa_layers();
    std::string err;
    ConversationStateSizes sizes;
    check(conversation_state_sizes(g, sizes, err), "whole-session geometry sizes" + tag);
    RunningState rs;
    ss.gdn_state = static_cast<float*>(rs.get(sizes.gdn));
    ss.ple_hist = static_cast<float*>(rs.get(sizes.ple));
    main.st.idx_tail = static_cast<float*>(rs.get(sizes.tail));
    main.st.idx_dead = static_cast<float*>(rs.get(sizes.dead));
    main.st.idx_block_pos = static_cast<int32_t*>(rs.get(sizes.block_pos));
    std::vector<int32_t> ids(65);
    for (size_t i = 0; i < ids.size(); ++i) ids[i] = int32_t(i) + 1;
    std::vector<ConversationImageKey> images;
    std::vector<ConversationCheckpoint> checkpoints;
    auto fill = [&](uint8_t salt) {
        main.fill(salt);
        draft.fill(salt);
        for (auto [p, n] : std::vector<std::pair<void*, size_t>>{{ss.gdn_state, sizes.gdn}, {ss.ple_hist, sizes.ple},
                 {main.st.idx_tail, sizes.tail}, {main.st.idx_dead, sizes.dead}, {main.st.idx_block_pos, sizes.block_pos}})
            memset_dev(p, salt, n);
        // an indexer keeps its spare pooled row equal to its spare key
        abi(sc_copy_async(main.st.idx_pooled + ids.size() / 4 * size_t(g.idx_key_dim), main.st.idx_dead, sizes.dead,
                          nullptr), "spare row");
        abi(sc_device_sync(), "sync");
    };
    fill(13);
    ConversationCheckpoint checkpoint;
    checkpoint.ids.assign(ids.begin(), ids.begin() + 3);
    check(conversation_checkpoint_save(checkpoint, ss, g, err), "save a running checkpoint" + tag + " " + err);
    checkpoint.used = 17;
    checkpoints.push_back(std::move(checkpoint));
    const ConversationView view{ids, images, checkpoints, true};
    SavedConversation a, b, back;
    check(conversation_snapshot_save(a, view, ss, g, draft.st, err), "capture A" + tag + " " + err);
    check(a.checkpoints[0].used == 17, "the checkpoint LRU stamp survives capture" + tag);
    size_t estimate = 0;
    check(conversation_snapshot_bytes(view, ss, g, draft.st, estimate, err) && a.bytes() <= estimate,
          "the byte estimate admits the capture" + tag);
    fill(177);
    check(conversation_snapshot_save(b, view, ss, g, draft.st, err), "capture B" + tag);
    check(a.live.dead != b.live.dead && !same(a.kv[0], b.kv[0]), "A and B differ" + tag);
    auto bad = a;
    bad.kv.back().k.pop_back();
    check(conversation_snapshot_restore(bad, ss, g, draft.st, err) == ConversationRestore::invalid,
          "a bad draft image is refused before any main-layer write" + tag);
    check(err == "conversation snapshot: invalid K/V payload size", "the refusal names its reason" + tag + ": " + err);
    check(conversation_snapshot_save(back, view, ss, g, draft.st, err), "capture after the refusal" + tag);
    check(back.live.gdn == b.live.gdn && back.live.dead == b.live.dead && same(back.kv[0], b.kv[0]) &&
              same(back.kv[1], b.kv[1]),
          "the refusal left every byte of B" + tag);
    check(conversation_snapshot_restore(a, ss, g, draft.st, err) == ConversationRestore::restored, "restore A" + tag + " " + err);
    check(conversation_snapshot_save(back, view, ss, g, draft.st, err), "capture the restored A" + tag);
    check(back.live.gdn == a.live.gdn && back.live.ple == a.live.ple && back.live.tails == a.live.tails &&
              back.live.dead == a.live.dead && back.live.block_pos == a.live.block_pos && same(back.kv[0], a.kv[0]) &&
              same(back.kv[1], a.kv[1]),
          "A/B/A: the restored session reads back as A, spare key included" + tag);
    check(ss.ple_prev[0] == 64 && ss.ple_prev[1] == 65, "the PLE token window is rebuilt" + tag);
    uint64_t fp = 0;
    check(conversation_kv_verify(a.kv[0], main.st, g, 65, true, fp, err) && fp != 0, "verify the restored layer" + tag);
    for (int64_t dirty : {65, 3, 0}) {
        const std::string dtag = tag + " dirty " + std::to_string(dirty);
        check(conversation_snapshot_restore(a, ss, g, draft.st, err) == ConversationRestore::restored, "restore the base" + dtag);
        ConversationKvReuse reuse{a.kv, 65, dirty};
        const uint8_t* original = nullptr;
        reuse.kv[0].k.visit(0, 1, [&](const uint8_t* p, size_t, size_t) { original = p; return true; });
        main.fill_after(91, dirty);
        draft.fill_after(91, std::max<int64_t>(0, dirty - 1));
        memset_dev(ss.gdn_state, 91, sizes.gdn);
        ids.resize(70);
        for (size_t i = 65; i < ids.size(); ++i) ids[i] = int32_t(i + 1);
        abi(sc_copy_async(main.st.idx_pooled + ids.size() / 4 * size_t(g.idx_key_dim), main.st.idx_dead, sizes.dead,
                          nullptr), "spare row");
        abi(sc_device_sync(), "sync");
        SavedConversation fresh, incremental;
        check(conversation_snapshot_save(fresh, view, ss, g, draft.st, err), "full capture after growth" + dtag);
        size_t peak = 0, reused = 0;
        check(conversation_snapshot_capture_bytes(reuse, view, ss, g, draft.st, peak, err), "admit the incremental peak" + dtag);
        check(conversation_snapshot_save(incremental, view, ss, g, draft.st, err, std::move(reuse), &reused),
              "capture with retained pages" + dtag + " " + err);
        check(incremental.bytes() <= peak, "the incremental capture stays within its admitted bound" + dtag);
        check(incremental.live.gdn == fresh.live.gdn && incremental.live.ple == fresh.live.ple &&
                  incremental.live.dead == fresh.live.dead && same(incremental.kv[0], fresh.kv[0]) &&
                  same(incremental.kv[1], fresh.kv[1]),
              "incremental capture equals a full capture" + dtag);
        check((dirty >= 4) == (reused > 0), "only whole unchanged pages or rows are retained" + dtag);
        incremental.kv[0].k.visit(0, 1, [&](const uint8_t* p, size_t, size_t) {
            check(p == original, "growth never reallocates the retained payload" + dtag);
            return true;
        });
        check(conversation_snapshot_restore(incremental, ss, g, draft.st, err) == ConversationRestore::restored,
              "restore the incremental image" + dtag);
        check(conversation_kv_verify(incremental.kv.back(), draft.st, g, 70, false, fp, err),
              "the draft's authoritative copy and ring read back" + dtag + " " + err);
        ids.resize(65);
    }
    check(conversation_checkpoint_restore(a.checkpoints[0], ss, g, err), "restore the early checkpoint" + tag);
    std::vector<uint8_t> spare(sizes.dead);
    download(spare.data(), main.st.idx_pooled, sizes.dead);
    check(spare == a.checkpoints[0].dead, "the checkpoint rebuilds the spare row over a later completed block" + tag);
    check(ss.ple_prev[0] == 2 && ss.ple_prev[1] == 3, "the checkpoint's PLE window" + tag);
}

void split_session(int fmt, int mode, int64_t experts) {
    const std::string tag = " [split fmt " + std::to_string(fmt) + " mode " + std::to_string(mode) + " experts " +
                            std::to_string(experts) + "]";
    Layer main(fmt, mode), stage(fmt, mode), draft(fmt == kHybrid ? int(kKvInt8) : fmt, 2);
    ModelGeometry& g = main.g;
    g.n_layers = 8;
    g.n_expert = experts;
    g.ssm_state_size = 2; g.ssm_v_heads = 2; g.ssm_conv_channels = 8;
    SessionState ss, st1;
    ss.max_cells = st1.max_cells = 96;
    ss.layer_lo = 0; ss.layer_hi = 4; ss.qsa_ord0 = 0; ss.qsa_alloc = 1; ss.gdn_ord0 = 0; ss.gdn_alloc = 3;
    st1.layer_lo = 4; st1.layer_hi = 8; st1.qsa_ord0 = 1; st1.qsa_alloc = 1; st1.gdn_ord0 = 3; st1.gdn_alloc = 3;
    std::string err;
    ConversationStateSizes whole;
    check(conversation_state_sizes(g, whole, err), "split sizes" + tag);
    const size_t rows = whole.gdn / size_t(g.n_gdn_layers());
    RunningState rs;
    ss.gdn_state = static_cast<float*>(rs.get(rows * 3));
    ss.ple_hist = static_cast<float*>(rs.get(whole.ple));
    st1.gdn_state = static_cast<float*>(rs.get(rows * 3));
    st1.ple_hist = static_cast<float*>(rs.get(whole.ple));
    for (Layer* f : {&main, &stage}) {
        f->st.idx_tail = static_cast<float*>(rs.get(whole.tail));
        f->st.idx_dead = static_cast<float*>(rs.get(whole.dead));
        f->st.idx_block_pos = static_cast<int32_t*>(rs.get(whole.block_pos));
    }
    std::array<QsaState, 2> main_layers{main.st, QsaState{}}, stage_layers{QsaState{}, stage.st};
    ss.qsa_states = main_layers.data();
    st1.qsa_states = stage_layers.data();
    std::vector<int32_t> ids(65);
    for (size_t i = 0; i < ids.size(); ++i) ids[i] = int32_t(i) + 1;
    std::vector<ConversationImageKey> images;
    std::vector<ConversationCheckpoint> checkpoints;
    auto fill = [&](uint8_t salt) {
        main.fill(salt); stage.fill(salt); draft.fill(salt);
        for (auto [p, n] : std::vector<std::pair<void*, size_t>>{{ss.gdn_state, rows * 3}, {ss.ple_hist, whole.ple},
                 {st1.gdn_state, rows * 3}, {st1.ple_hist, whole.ple}, {main.st.idx_tail, whole.tail},
                 {main.st.idx_dead, whole.dead}, {main.st.idx_block_pos, whole.block_pos}, {stage.st.idx_tail, whole.tail},
                 {stage.st.idx_dead, whole.dead}, {stage.st.idx_block_pos, whole.block_pos}})
            memset_dev(p, salt, n);
        for (Layer* f : {&main, &stage})
            abi(sc_copy_async(f->st.idx_pooled + ids.size() / 4 * size_t(g.idx_key_dim), f->st.idx_dead, whole.dead,
                              nullptr), "spare row");
        abi(sc_device_sync(), "sync");
    };
    fill(13);
    ConversationCheckpoint checkpoint;
    checkpoint.ids.assign(ids.begin(), ids.begin() + 3);
    check(conversation_checkpoint_save(checkpoint, ss, g, err), "split: the first stage's checkpoint part" + tag);
    ConversationCheckpoint part;
    part.ids = checkpoint.ids;
    check(conversation_checkpoint_save(part, st1, g, err), "split: the later stage's checkpoint part" + tag);
    checkpoint.stage_parts.push_back(std::move(part));
    checkpoints.push_back(std::move(checkpoint));
    const ConversationView view{ids, images, checkpoints, true};
    const ConversationStage stage_list[]{{&st1, -1}};
    const ConversationStageSet stages{stage_list, 1, -1, -1};
    SavedConversation a, b, back;
    check(conversation_snapshot_save(a, view, ss, stages, g, draft.st, err), "split: capture A" + tag + " " + err);
    check(a.stage_parts.size() == 1 && a.stage_parts[0].kv.size() == 1, "split: one stage part with its K/V" + tag);
    fill(177);
    check(conversation_snapshot_save(b, view, ss, stages, g, draft.st, err), "split: capture B" + tag);
    check(conversation_snapshot_restore(a, ss, g, draft.st, err) == ConversationRestore::invalid,
          "split: a split image is refused without its stages" + tag);
    check(conversation_snapshot_restore(a, ss, stages, g, draft.st, err) == ConversationRestore::restored,
          "split: restore A" + tag + " " + err);
    check(conversation_snapshot_save(back, view, ss, stages, g, draft.st, err), "split: capture the restored A" + tag);
    check(back.live.gdn == a.live.gdn && back.stage_parts[0].state.gdn == a.stage_parts[0].state.gdn &&
              same(back.kv[0], a.kv[0]) && same(back.stage_parts[0].kv[0], a.stage_parts[0].kv[0]) &&
              same(back.kv[1], a.kv[1]),
          "split: A/B/A over both stages and the draft" + tag);
}

// One layer at a time over every extent: A/B/A, the byte estimate, refusals, and the residency after a restore.
void layer_cases(int fmt, int mode) {
    const std::string tag = " [layer fmt " + std::to_string(fmt) + " mode " + std::to_string(mode) + "]";
    Layer f(fmt, mode);
    std::string err;
    if (fmt == kHybrid) {
        ConversationKv invalid;
        for (int unsupported : {1, 2}) {
            f.st.kv_mode = unsupported;
            check(conversation_kv_bytes(f.st, f.g, 9, true) == 0, "hybrid streaming/ring is refused" + tag);
            check(!conversation_kv_save(invalid, f.st, f.g, 9, true, err), "hybrid streaming/ring capture fails" + tag);
        }
        f.st.kv_mode = 0;
    }
    {
        ConversationKv invalid;
        for (const int64_t bad : {int64_t(-1), int64_t(97), std::numeric_limits<int64_t>::max()}) {
            check(!conversation_kv_save(invalid, f.st, f.g, bad, mode != 2, err), "an invalid save extent is refused" + tag);
            check(!conversation_kv_restore(invalid, f.st, f.g, bad, mode != 2, err), "an invalid restore extent is refused" + tag);
            check(conversation_kv_bytes(f.st, f.g, bad, mode != 2) == 0, "an invalid extent has no byte estimate" + tag);
        }
    }
    for (int64_t upto : {0, 1, 3, 4, 5, 63, 64, 65, 96}) {
        const std::string utag = tag + " upto " + std::to_string(upto);
        const bool index = mode != 2;
        f.fill(13);
        ConversationKv a, b, restored;
        check(conversation_kv_save(a, f.st, f.g, upto, index, err), "save A" + utag + " " + err);
        check(a.bytes() == conversation_kv_bytes(f.st, f.g, upto, index), "the byte estimate equals the payload" + utag);
        f.fill(177);
        check(conversation_kv_save(b, f.st, f.g, upto, index, err), "save B" + utag);
        check(upto == 0 || !same(a, b), "the fixture changes state" + utag);
        check(conversation_kv_restore(a, f.st, f.g, upto, index, err), "restore A over B" + utag + " " + err);
        check(conversation_kv_save(restored, f.st, f.g, upto, index, err), "read back the restored A" + utag);
        check(same(a, restored), "A/B/A byte-exact K/V and indexer state" + utag);
        uint64_t fp = 0;
        check(conversation_kv_verify(a, f.st, f.g, upto, index, fp, err), "verify authoritative and resident bytes" + utag);
        if (mode == 1) {
            std::vector<int32_t> table(size_t(f.st.n_pages));
            download(table.data(), f.st.page_table, table.size() * 4);
            check(std::all_of(table.begin(), table.end(), [](int32_t x) { return x == -1; }),
                  "a restore evicts every VRAM page of a streamed layer" + utag);
        }
        if (mode == 2 && upto > 0) {
            const QsaShapes s = qsa_real_shapes();
            const int64_t b1 = (upto + s.page_size - 1) / s.page_size, b0 = std::max<int64_t>(0, b1 - f.st.n_slots);
            const size_t block = size_t(kv_block_bytes(s, fmt)) / 2;
            const size_t code_block = fmt == kKvInt8 ? size_t(s.page_size * s.n_head_kv * s.head_dim) : block;
            const void* slots = fmt == kKvQ4 ? (void*) f.st.k_q4 : fmt == kKvInt8 ? (void*) f.st.k_q : (void*) f.st.k_pool;
            std::vector<uint8_t> got(code_block), want(code_block);
            for (int64_t page = b0; page < b1; ++page) {
                download(got.data(), static_cast<const uint8_t*>(slots) + size_t(page % f.st.n_slots) * code_block, code_block);
                check(a.k.read(want.data(), size_t(page) * code_block, code_block), "read the expected ring page" + utag);
                check(got == want, "the ring holds the restored pages" + utag);
            }
        }
        auto bad = a;
        bad.head_dim++;
        check(!conversation_kv_restore(bad, f.st, f.g, upto, index, err), "an incompatible geometry is refused" + utag);
        if (!a.k.empty()) {
            bad = a;
            bad.k.pop_back();
            check(!conversation_kv_restore(bad, f.st, f.g, upto, index, err), "a malformed payload is refused" + utag);
        }
    }
}

}  // namespace

int main() {
    int devices = 0;
    if (sc_device_count(&devices) != SC_OK || devices < 1) {
        std::fprintf(stderr, "conversation_snapshot_test: no HIP device\n");
        return 2;
    }
    for (int fmt : {int(kKvF16), int(kKvInt8), int(kKvQ4), kHybrid})
        for (int mode : {0, 1, 2}) {
            if (fmt == kHybrid && mode != 0) continue;   // K8V4 is an identity-layout format only
            layer_cases(fmt, mode);
        }
    // Whole sessions: the main layers resident or streamed (a ring is the draft's layout), the draft a ring.
    for (int fmt : {int(kKvF16), int(kKvInt8), int(kKvQ4)})
        for (int mode : {0, 1})
            for (int64_t experts : {256, 512}) {
                full_session(fmt, mode, experts);
                split_session(fmt, mode, experts);
            }
    for (int64_t experts : {256, 512}) {
        full_session(kHybrid, 0, experts);
        split_session(kHybrid, 0, experts);
    }
    std::printf("conversation_snapshot_test: %d checks passed; pinned pool %zu bytes\n", checks,
                conversation_pinned_pool_bytes());
    return 0;
}

// conversation_validation_test.cpp - the C++ host layer's refusals and failure classes, on the CPU.
//
// The reference's host-only validation matrix (src/core/conversation_validation_test.cpp:77-140) restated: pools
// are host memory filled with 0xa5 sentinels, the runtime is tests/cpp/fake_abi.cpp (memcpy copies with an
// injectable failure), and every invalid request must return before the first copy with the sentinels intact,
// while a copy that fails after the first write must be reported as transfer_failed.
#include "strata/core/conversation_snapshot.hpp"

#include <algorithm>
#include <array>
#include <cstdio>
#include <cstdlib>
#include <functional>
#include <string>
#include <vector>

namespace fake {
extern int copy_calls, sync_calls, fail_copy, fail_sync, movers;
extern size_t copied_bytes;
void reset();
}  // namespace fake

using namespace strata::core;

namespace {
int checks = 0;
void check(bool ok, const std::string& label) {
    ++checks;
    if (!ok) {
        std::fprintf(stderr, "FAIL: %s\n", label.c_str());
        std::exit(1);
    }
}

// One QSA layer in host memory: 96 cells, 24 pages, the indexer's pooled rows, tail, spare key, block position.
struct Pools {
    QsaState st;
    std::array<std::vector<uint8_t>, 8> data;
    Pools(const ModelGeometry& g, int format) {
        st.max_cells = 96;
        st.n_pages = st.n_slots = 24;
        st.idx_pooled_rows = 26;
        st.kv_int8 = format == 1;
        st.kv_q4 = format == 2;
        const size_t per = format == 2 ? strata::kernels::kv_q4_bytes_per_head(int(g.head_dim))
                                       : size_t(g.head_dim) * (format == 1 ? 1 : 2);
        data[0].assign(96 * size_t(g.n_head_kv) * per, 0xa5);
        data[1] = data[0];
        data[2].assign(format == 1 ? 96 * size_t(g.n_head_kv) * size_t(g.head_dim / 64) * 2 : 0, 0xa5);
        data[3] = data[2];
        data[4].assign(26 * size_t(g.idx_key_dim) * 4, 0xa5);
        data[5].assign(3 * size_t(g.idx_key_dim) * 4, 0xa5);
        data[6].assign(size_t(g.idx_key_dim) * 4, 0xa5);
        data[7].assign(4, 0xa5);
        if (format == 2) { st.k_q4 = data[0].data(); st.v_q4 = data[1].data(); }
        else if (format == 1) {
            st.k_q = (int8_t*) data[0].data(); st.v_q = (int8_t*) data[1].data();
            st.k_scale = (uint16_t*) data[2].data(); st.v_scale = (uint16_t*) data[3].data();
        } else {
            st.k_pool = (uint16_t*) data[0].data(); st.v_pool = (uint16_t*) data[1].data();
        }
        st.idx_pooled = (float*) data[4].data();
        st.idx_tail = (float*) data[5].data();
        st.idx_dead = (float*) data[6].data();
        st.idx_block_pos = (int32_t*) data[7].data();
    }
    bool untouched() const {
        return std::all_of(data.begin(), data.end(), [](const std::vector<uint8_t>& d) {
            return std::all_of(d.begin(), d.end(), [](uint8_t b) { return b == 0xa5; });
        });
    }
};

void matrix(int format) {
    const std::string tag = " [format " + std::to_string(format) + "]";
    ModelGeometry g;
    g.n_layers = 8;
    g.ssm_state_size = 2; g.ssm_v_heads = 2; g.ssm_conv_channels = 8;
    g.n_head_kv = 1; g.head_dim = 64; g.idx_key_dim = 8;
    std::string err;
    ConversationStateSizes z;
    check(conversation_state_sizes(g, z, err), "sizes" + tag);
    Pools q0(g, format), q1(g, format), draft(g, format);
    draft.st.idx_pooled_rows = 26;
    std::array<QsaState, 2> states{q0.st, q1.st};
    std::vector<uint8_t> gdn(z.gdn, 0xa5), ple(z.ple, 0xa5);
    SessionState ss;
    ss.max_cells = 96;
    ss.qsa_states = states.data();
    ss.layer_hi = g.n_layers; ss.qsa_alloc = 2; ss.gdn_alloc = g.n_gdn_layers();
    ss.gdn_state = (float*) gdn.data();
    ss.ple_hist = (float*) ple.data();
    std::vector<int32_t> ids(9);
    for (size_t i = 0; i < ids.size(); ++i) ids[i] = int32_t(i) + 1;
    std::vector<ConversationImageKey> images;
    std::vector<ConversationCheckpoint> checkpoints;
    const ConversationView view{ids, images, checkpoints, true};
    // A valid image: captured from fresh pools (the sentinels), then the pools are reset to sentinels.
    SavedConversation good;
    fake::reset();
    check(conversation_snapshot_save(good, view, ss, g, draft.st, err), "capture a valid image" + tag + " " + err);
    check(fake::copy_calls > 0, "capture copies" + tag);
    auto untouched = [&] {
        return q0.untouched() && q1.untouched() && draft.untouched() &&
               std::all_of(gdn.begin(), gdn.end(), [](uint8_t b) { return b == 0xa5; }) &&
               std::all_of(ple.begin(), ple.end(), [](uint8_t b) { return b == 0xa5; });
    };
    // Every malformed image is refused with no copy at all and every sentinel intact.
    const std::vector<std::pair<const char*, std::function<void(SavedConversation&)>>> mutations = {
        {"geometry key", [](SavedConversation& s) { s.geometry[3]++; }},
        {"layer range", [](SavedConversation& s) { s.layer_hi++; }},
        {"K/V layer count", [](SavedConversation& s) { s.kv.pop_back(); }},
        {"first layer K size", [](SavedConversation& s) { s.kv[0].k.pop_back(); }},
        {"last layer V size", [](SavedConversation& s) { s.kv[1].v.resize(s.kv[1].v.size() + 1); }},
        {"draft payload", [](SavedConversation& s) { s.kv.back().k.pop_back(); }},
        {"draft geometry", [](SavedConversation& s) { s.kv.back().head_dim++; }},
        {"pooled rows", [](SavedConversation& s) { s.kv[0].pooled_rows++; }},
        {"format", [](SavedConversation& s) { s.kv[1].format ^= 1; }},
        {"GDN payload", [](SavedConversation& s) { s.live.gdn.pop_back(); }},
        {"PLE payload", [](SavedConversation& s) { s.live.ple.clear(); }},
        {"indexer tails", [](SavedConversation& s) { s.live.tails.push_back(0); }},
        {"no live tokens", [](SavedConversation& s) { s.live.ids.clear(); }},
        {"negative token", [](SavedConversation& s) { s.live.ids[0] = -1; }},
        {"stage part on one GPU", [](SavedConversation& s) { s.stage_parts.resize(1); }},
        {"checkpoint not a prefix", [](SavedConversation& s) {
             ConversationCheckpoint c; c.ids = {99}; s.checkpoints.push_back(c); }},
    };
    for (const auto& [name, mutate] : mutations) {
        SavedConversation bad = good;
        mutate(bad);
        fake::reset();
        const auto r = conversation_snapshot_restore(bad, ss, g, draft.st, err);
        check(r == ConversationRestore::invalid, std::string("refuse ") + name + tag);
        check(err.rfind("conversation snapshot: ", 0) == 0, std::string("refusal message ") + name + tag + ": " + err);
        check(fake::copy_calls == 0 && fake::sync_calls == 0 && fake::movers == 0,
              std::string("no copy, sync or mover before refusing ") + name + tag);
        check(untouched(), std::string("every sentinel intact after refusing ") + name + tag);
    }
    // A failure at any copy after the first is transfer_failed, never restored and never invalid.
    fake::reset();
    check(conversation_snapshot_restore(good, ss, g, draft.st, err) == ConversationRestore::restored, "restore" + tag);
    const int copies = fake::copy_calls;
    check(copies > 2, "a restore copies" + tag);
    for (int n : {1, 2, copies / 2, copies}) {
        fake::reset();
        fake::fail_copy = n;
        check(conversation_snapshot_restore(good, ss, g, draft.st, err) == ConversationRestore::transfer_failed,
              "a failed copy " + std::to_string(n) + " is transfer_failed" + tag);
    }
    fake::reset();
    fake::fail_sync = 1;
    check(conversation_snapshot_restore(good, ss, g, draft.st, err) == ConversationRestore::transfer_failed,
          "a failed synchronization is transfer_failed" + tag);
    // A save that fails publishes nothing: the target image keeps its previous content.
    SavedConversation target = good;
    fake::reset();
    fake::fail_copy = 3;
    check(!conversation_snapshot_save(target, view, ss, g, draft.st, err), "a failed capture reports failure" + tag);
    check(target.kv.size() == good.kv.size() && target.kv[0].k == good.kv[0].k, "a failed capture publishes nothing" + tag);
}

}  // namespace

int main() {
    strata::core::conversation_pinned_segments(false);
    for (int format : {0, 1, 2}) matrix(format);
    std::printf("conversation_validation_test: %d checks passed\n", checks);
    return 0;
}

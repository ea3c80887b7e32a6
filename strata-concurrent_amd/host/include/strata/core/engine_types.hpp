// engine_types.hpp - the engine structs the handoff reads and writes, as this library sees them.
//
// These are the members of the reference engine's ModelGeometry, QsaState and SessionState that the
// conversation-state path uses, with the same names, types and meaning:
//   ModelGeometry  include/strata/core/layout.hpp:27-59   (all 18 fields: they form the image's geometry key)
//   QsaState       include/strata/core/layer.hpp:203-261  (K/V pools, page table, streaming/ring mode, indexer)
//   SessionState   include/strata/core/session.hpp:30-88  (GDN rows, QSA states, the layer carve, PLE state)
//   KvHostPools / KvStreamMap  include/strata/kernels/kv_stream.hpp:32-59
// An engine that links this library in place of its own conversation_snapshot.cpp / conversation_state.cpp
// builds these translation units against its own headers (the members used here all exist there); a standalone
// build uses the definitions below.  Everything else of the engine's structs is irrelevant to the handoff.
#pragma once

#include <cstdint>
#include <cstdio>
#include <cstdlib>

namespace strata::kernels {

enum KvFormat : int { kKvF16 = 0, kKvInt8 = 1, kKvQ4 = 2 };

inline constexpr int KV_Q8_GROUP = 64;   // int8 K/V: one f16 scale per 64 values (kv_q8.hpp:22)
inline constexpr int QK4_0 = 32;         // q4_0: blocks of 32 values, 18 bytes each (kv_q4.hpp:33)
inline constexpr int kQ4BlockBytes = 18;
inline uint64_t kv_q4_bytes_per_head(int head_dim) { return uint64_t(head_dim / QK4_0) * kQ4BlockBytes; }

// The QSA granules the snapshot depends on (qsa.hpp:110-114): one page = one indexer block = 4 cells.
struct QsaGranules {
    int64_t page_size = 4;
    int64_t idx_block = 4;
};
inline QsaGranules qsa_granules() { return {}; }

// The PLE history is NG_HIST rows of NG_HC_DIM floats (ngram.hpp:39-40).
inline constexpr int NG_HC_DIM = 10240;
inline constexpr int NG_HIST = 9;

struct KvHostPools {
    uint16_t* k_pool = nullptr;
    uint16_t* v_pool = nullptr;
    int8_t* k_q = nullptr;
    int8_t* v_q = nullptr;
    uint16_t* k_scale = nullptr;
    uint16_t* v_scale = nullptr;
    uint8_t* k_q4 = nullptr;
    uint8_t* v_q4 = nullptr;
    bool present() const { return k_pool != nullptr || k_q != nullptr || k_q4 != nullptr; }
};

inline constexpr int kKvCtlInts = 16;

struct KvStreamMap {
    int32_t* page_table = nullptr;
    int32_t* slot_block = nullptr;
    int32_t* slot_stamp = nullptr;
    int32_t* slot_ref = nullptr;
    int32_t* ctl = nullptr;
    int32_t* miss_block = nullptr;
    int32_t* miss_slot = nullptr;
    int64_t n_blocks = 0;
    int64_t n_slots = 0;
};

}  // namespace strata::kernels

namespace strata::core {

struct ModelGeometry {
    int64_t n_embd = 2560;
    int64_t n_layers = 48;
    int64_t qsa_interval = 4;
    int64_t ssm_state_size = 128;
    int64_t ssm_k_heads = 16;
    int64_t ssm_v_heads = 48;
    int64_t ssm_d_conv = 4;
    int64_t ssm_conv_channels = 10240;
    int64_t ssm_value_dim = 6144;
    int64_t n_head = 24;
    int64_t n_head_kv = 2;
    int64_t head_dim = 256;
    int64_t idx_q_heads = 4;
    int64_t idx_key_dim = 128;
    int64_t hc = 4;
    int64_t hc_lr = 320;
    int64_t n_expert = 512;
    int64_t n_ff = 640;

    int64_t n_qsa_layers() const { return n_layers / qsa_interval; }
    int64_t n_gdn_layers() const { return n_layers - n_qsa_layers(); }
};

struct QsaState {
    uint16_t* k_pool = nullptr;   // [page][kv_head][page_size][head_dim] f16
    uint16_t* v_pool = nullptr;
    bool kv_int8 = false;
    int8_t* k_q = nullptr;
    int8_t* v_q = nullptr;
    uint16_t* k_scale = nullptr;
    uint16_t* v_scale = nullptr;
    bool kv_q4 = false;
    uint8_t* k_q4 = nullptr;
    uint8_t* v_q4 = nullptr;
    bool kv_hybrid = false;
    int32_t* page_table = nullptr;
    int64_t n_pages = 0;
    int64_t max_cells = 0;
    int kv_mode = 0;              // 0 resident, 1 streamed (authoritative host copy), 2 ring (draft)
    int64_t n_slots = 0;
    strata::kernels::KvHostPools host;
    strata::kernels::KvStreamMap map;
    int64_t idx_pooled_rows = 0;
    float* idx_tail = nullptr;
    float* idx_dead = nullptr;
    float* idx_pooled = nullptr;
    int32_t* idx_block_pos = nullptr;
};

struct SessionState {
    int64_t max_cells = 0;
    float* gdn_state = nullptr;            // (gdn_alloc, gdn row floats)
    QsaState* qsa_states = nullptr;        // global QSA ordinals; [qsa_ord0, qsa_ord0 + qsa_alloc) are owned
    int64_t layer_lo = 0, layer_hi = 0;
    int64_t qsa_ord0 = 0, qsa_alloc = 0;
    int64_t gdn_ord0 = 0, gdn_alloc = 0;
    int32_t ple_prev[2] = {-1, -1};
    float* ple_hist = nullptr;
};

// The block-mover format of a state (layer.hpp:275-284).  A hybrid K8V4 state never reaches the block movers;
// asking for its format is a programming error and stops the process, as the reference does.
inline int qsa_kv_format(const QsaState& st) {
    if (st.kv_hybrid) {
        std::fprintf(stderr, "strata: qsa_kv_format: a hybrid K8V4 state must never reach the block movers\n");
        std::exit(1);
    }
    return st.kv_q4 ? strata::kernels::kKvQ4 : st.kv_int8 ? strata::kernels::kKvInt8 : strata::kernels::kKvF16;
}

}  // namespace strata::core

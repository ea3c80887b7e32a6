// kv_stream.cpp - the block movers and the prefill K/V appends over libsc_handoff.so (see strata/kernels/kv_stream.hpp,
// strata/kernels/kv_q4.hpp and strata/prefill/kernels.hpp).
#include "strata/kernels/kv_stream.hpp"

#include "sc_handoff.h"
#include "strata/kernels/kv_q4.hpp"
#include "strata/prefill/kernels.hpp"

#include <type_traits>

#include <cstdio>
#include <cstdlib>

namespace strata::kernels {
namespace {

void check(int rc, const char* what) {
    if (rc != SC_OK) {
        std::fprintf(stderr, "kv_stream: %s: %s\n", what, sc_last_error());
        std::exit(1);
    }
}

// The per-block runs of the format's pool arrays (kv_stream.cu:33-55): rows = n_head_kv * page_size per block.
sc_kv_runs runs_of(const QsaAttnPools& slots, const KvHostPools& host, int fmt, const QsaShapes& s) {
    const uint64_t rows = uint64_t(s.n_head_kv * s.page_size);
    sc_kv_runs r{};
    auto put = [&](const void* src, const void* dst, uint64_t len) {
        r.src[r.n] = src;
        r.dst[r.n] = const_cast<void*>(dst);
        r.len[r.n] = len;
        ++r.n;
    };
    if (fmt == kKvQ4) {
        const uint64_t bytes = rows * kv_q4_bytes_per_head(int(s.head_dim));
        put(host.k_q4, slots.k_q4, bytes);
        put(host.v_q4, slots.v_q4, bytes);
    } else if (fmt == kKvInt8) {
        const uint64_t codes = rows * uint64_t(s.head_dim), scales = rows * uint64_t(s.head_dim / KV_Q8_GROUP) * 2;
        put(host.k_q, slots.k_q, codes);
        put(host.v_q, slots.v_q, codes);
        put(host.k_scale, slots.k_scale, scales);
        put(host.v_scale, slots.v_scale, scales);
    } else {
        const uint64_t bytes = rows * uint64_t(s.head_dim) * 2;
        put(host.k_pool, slots.k_pool, bytes);
        put(host.v_pool, slots.v_pool, bytes);
    }
    return r;
}

// KvHostPools as the C-ABI's sc_kv_pools (the same eight pointers; null stays null).
static_assert(std::is_standard_layout_v<KvHostPools> && sizeof(KvHostPools) == sizeof(sc_kv_pools),
              "KvHostPools and sc_kv_pools hold the same eight pointers");
const sc_kv_pools* c_pools(const KvHostPools* p, sc_kv_pools& out) {
    if (!p) return nullptr;
    out = sc_kv_pools{p->k_pool, p->v_pool, p->k_q, p->v_q, p->k_scale, p->v_scale, p->k_q4, p->v_q4};
    return &out;
}

}  // namespace

void kv_append_q4(uint8_t* k_q4, uint8_t* v_q4, const int32_t* page_table, int64_t pos0, int64_t T, const float* K,
                  const float* V, const QsaShapes& s, void* stream, const KvHostPools* host,
                  const KvHostPools* stage) {
    sc_kv_pools h{}, st{};
    check(sc_kv_append_q4_async(k_q4, v_q4, page_table, pos0, T, K, V, s.n_head_kv, s.head_dim, s.page_size, stream,
                                c_pools(host, h), c_pools(stage, st)),
          "kv_append_q4");
}

void kv_stream_reset(const KvStreamMap& m, void* stream) {
    check(sc_kv_stream_reset(m.page_table, m.n_blocks, m.slot_block, m.slot_stamp, m.slot_ref, m.n_slots, m.ctl, stream),
          "reset");
}

void kv_ring_table(int32_t* page_table, int64_t n_blocks, int64_t n_slots, void* stream) {
    check(sc_kv_ring_table(page_table, n_blocks, n_slots, stream), "ring table");
}

void kv_ring_restore(const QsaAttnPools& slots, const KvHostPools& host, int fmt, int64_t b0, int64_t b1,
                     int64_t n_slots, const QsaShapes& s, void* stream) {
    if (b1 <= b0) return;
    const sc_kv_runs r = runs_of(slots, host, fmt, s);
    check(sc_kv_ring_restore(&r, b0, b1, n_slots, stream), "ring restore");
}

void kv_stage_from_host(const QsaAttnPools& stage, const KvHostPools& host, int fmt, int64_t n_blocks,
                        const QsaShapes& s, void* stream) {
    if (n_blocks <= 0) return;
    const sc_kv_runs r = runs_of(stage, host, fmt, s);
    check(sc_kv_stage_from_host(&r, n_blocks, stream), "stage");
}

uint64_t kv_block_bytes(const QsaShapes& s, int fmt) {
    return sc_kv_block_bytes(s.n_head_kv, s.head_dim, s.page_size, fmt);
}

}  // namespace strata::kernels

namespace strata::core {
strata::kernels::QsaAttnPools qsa_attn_pools(const QsaState& st) {
    strata::kernels::QsaAttnPools p;
    p.page_table = st.page_table;
    if (st.kv_hybrid) { p.k_q = st.k_q; p.k_scale = st.k_scale; p.v_q4 = st.v_q4; }
    else if (st.kv_q4) { p.k_q4 = st.k_q4; p.v_q4 = st.v_q4; }
    else if (st.kv_int8) { p.k_q = st.k_q; p.v_q = st.v_q; p.k_scale = st.k_scale; p.v_scale = st.v_scale; }
    else { p.k_pool = st.k_pool; p.v_pool = st.v_pool; }
    return p;
}
}  // namespace strata::core

namespace strata::prefill {

void kv_append(const float* K, const float* V, int64_t T, int64_t pos0, const int32_t* page_table, int64_t page_size,
               uint16_t* k_pool, uint16_t* v_pool, int8_t* k_q, int8_t* v_q, uint16_t* k_scale, uint16_t* v_scale,
               void* stream, const strata::kernels::KvHostPools* host, const strata::kernels::KvHostPools* stage) {
    sc_kv_pools h{}, st{};
    const int rc = sc_kv_append_async(K, V, T, pos0, page_table, page_size, k_pool, v_pool, k_q, v_q, k_scale, v_scale,
                                      stream, strata::kernels::c_pools(host, h), strata::kernels::c_pools(stage, st));
    if (rc != SC_OK) {
        std::fprintf(stderr, "kv_append: %s\n", sc_last_error());
        std::exit(1);
    }
}

}  // namespace strata::prefill

// kv_stream.hpp - the block movers of streamed and ring K/V layers, over libsc_handoff.so.
//
// The reference's kv_ring_table / kv_ring_restore / kv_stage_from_host / kv_stream_reset / kv_block_bytes
// (include/strata/kernels/kv_stream.hpp:65-96) with the same arguments.  As there, these wrappers return nothing
// and stop the process on a launch failure (src/kernels/cuda/kv_stream.cu:15-21).
#pragma once

#include "strata/core/engine_types.hpp"
#include "strata/kernels/qsa.hpp"

#include <cstdint>

namespace strata::kernels {

/// The pools a reader sees (include/strata/kernels/qsa_decode_attn.hpp:23-33).
struct QsaAttnPools {
    const uint16_t* k_pool = nullptr;
    const uint16_t* v_pool = nullptr;
    const int8_t* k_q = nullptr;
    const int8_t* v_q = nullptr;
    const uint16_t* k_scale = nullptr;
    const uint16_t* v_scale = nullptr;
    const uint8_t* k_q4 = nullptr;
    const uint8_t* v_q4 = nullptr;
    const int32_t* page_table = nullptr;
};

void kv_stream_reset(const KvStreamMap& m, void* stream);
void kv_ring_table(int32_t* page_table, int64_t n_blocks, int64_t n_slots, void* stream);
void kv_ring_restore(const QsaAttnPools& slots, const KvHostPools& host, int fmt, int64_t b0, int64_t b1,
                     int64_t n_slots, const QsaShapes& s, void* stream);
void kv_stage_from_host(const QsaAttnPools& stage, const KvHostPools& host, int fmt, int64_t n_blocks,
                        const QsaShapes& s, void* stream);
uint64_t kv_block_bytes(const QsaShapes& s, int fmt);

}  // namespace strata::kernels

namespace strata::core {
/// The reader's view of a state's pools (src/core/layer.cpp:710-718).
strata::kernels::QsaAttnPools qsa_attn_pools(const QsaState& st);
}  // namespace strata::core

// kv_q4.hpp - the q4_0 K/V storage facts the snapshot path sizes its buffers with, at the reference's include path
// (include/strata/kernels/kv_q4.hpp:21-38): blocks of 32 values, each an f16 scale and 16 bytes of 4-bit codes
// (value j in the low nibble of byte j, value j + 16 in the high one), 144 B per KV head per cell at head_dim 256.
// The decode-side q4_0 kernels declared beside them there (the Hadamard rotation, the per-step append, the gather)
// belong to attention, not to the hand-off; the prefill-side append is sc_plan_carve_quant (include/sc_handoff.h).
#pragma once

#include "strata/core/engine_types.hpp"
#include "strata/kernels/qsa.hpp"

#include <cstdint>

namespace strata::kernels {

#pragma pack(push, 1)
struct block_q4_0 {
    uint16_t d;             // scale (f16 bits)
    uint8_t qs[QK4_0 / 2];  // 32 codes, two per byte
};
#pragma pack(pop)
static_assert(sizeof(block_q4_0) == kQ4BlockBytes, "a q4_0 block is 18 bytes");

/// Bytes per cell (one token of one layer): K and V of every KV head.
inline uint64_t kv_q4_bytes_per_cell(const QsaShapes& s) {
    return uint64_t(s.n_head_kv) * kv_q4_bytes_per_head(int(s.head_dim)) * 2;
}

}  // namespace strata::kernels

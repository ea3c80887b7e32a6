// kv_q4.hpp - the q4_0 K/V storage facts the snapshot path sizes its buffers with, at the reference's include path
// (include/strata/kernels/kv_q4.hpp:21-38): blocks of 32 values, each an f16 scale and 16 bytes of 4-bit codes
// (value j in the low nibble of byte j, value j + 16 in the high one), 144 B per KV head per cell at head_dim 256,
// and the prompt path's append (kv_append_q4).  The decode-side q4_0 kernels declared beside them there (the Hadamard
// rotation, the per-step append, the gather) belong to attention, not to the hand-off.
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

/// The prompt path (include/strata/kernels/kv_q4.hpp:50-54): T consecutive already-rotated cells from pos0, K and V
/// f32 [T, n_head_kv, 256], into the q4_0 pools through page_table (negative entries skip the pool), and into
/// host->k_q4 / stage->k_q4 (identity layout) when given.  One launch; head_dim must be 256, and a refused argument
/// or a failed launch prints the reason and ends the process, as the reference does.
void kv_append_q4(uint8_t* k_q4, uint8_t* v_q4, const int32_t* page_table, int64_t pos0, int64_t T, const float* K,
                  const float* V, const QsaShapes& s, void* stream, const KvHostPools* host = nullptr,
                  const KvHostPools* stage = nullptr);

}  // namespace strata::kernels

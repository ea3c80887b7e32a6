// kernels.hpp - the prefill-side writer of the decode K/V layout, at the reference's include path and with its
// arguments (include/strata/prefill/kernels.hpp:78-83), over libsc_handoff.so.  The reference's other prefill
// kernels (RoPE, the gates, the activation conversions) are model compute, not part of the hand-off.
#pragma once

#include "strata/kernels/kv_stream.hpp"

#include <cstdint>

namespace strata::prefill {

/// K and V of T consecutive cells (positions pos0 .. pos0 + T - 1), f32 [T, 2, 256], into the paged pools: f16
/// (`k_pool` / `v_pool`, round to nearest even) or, when k_pool is null, int8 codes + an f16 scale per 64 values
/// (`k_q`...).  Cells whose page entry is negative are not resident and skip the pool; the host copy and the staging
/// pool (identity layout) take every cell when given.  One launch on `stream`; a refused argument or a failed launch
/// prints the reason and ends the process, as the reference's kernel wrappers do (src/kernels/cuda/kv_stream.cu:15-21).
void kv_append(const float* K, const float* V, int64_t T, int64_t pos0, const int32_t* page_table, int64_t page_size,
               uint16_t* k_pool, uint16_t* v_pool, int8_t* k_q, int8_t* v_q, uint16_t* k_scale, uint16_t* v_scale,
               void* stream, const strata::kernels::KvHostPools* host = nullptr,
               const strata::kernels::KvHostPools* stage = nullptr);

}  // namespace strata::prefill

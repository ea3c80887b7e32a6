// qsa.hpp - the shape of one QSA layer, at the reference's include path and with the reference's field order
// (include/strata/kernels/qsa.hpp:96-117), so a caller's QsaShapes passes to the block movers (kv_stream.hpp)
// unchanged.  Only the shape facts live here; the attention kernels declared beside them there are not part of the
// hand-off.
#pragma once

#include <cstdint>

namespace strata::kernels {

/// Geometry of one QSA layer.  The real artifact: n_head 24, n_head_kv 2, head_dim 256, n_rot 64, idx_n_head 4,
/// idx_dim 128, idx_block 4, idx_top_k 2048, page_size 4.
struct QsaShapes {
    int64_t n_head = 0;      ///< query heads
    int64_t n_head_kv = 0;   ///< key/value heads
    int64_t head_dim = 0;    ///< a multiple of 4 (256)
    int64_t n_rot = 0;       ///< rotated dims of head_dim
    int64_t idx_n_head = 0;  ///< indexer query heads
    int64_t idx_dim = 0;     ///< indexer key width
    int64_t idx_block = 0;   ///< cells per pooled indexer key
    int64_t idx_top_k = 0;   ///< cells of selection budget
    int64_t page_size = 0;   ///< K/V page granule in cells
};
static_assert(sizeof(QsaShapes) == 9 * sizeof(int64_t), "QsaShapes is nine int64 fields, as the reference's");

/// The real artifact's shapes (one page = one indexer block = 4 cells).
inline QsaShapes qsa_real_shapes() {
    QsaShapes s;
    s.n_head = 24;
    s.n_head_kv = 2;
    s.head_dim = 256;
    s.n_rot = 64;
    s.idx_n_head = 4;
    s.idx_dim = 128;
    s.idx_block = 4;
    s.idx_top_k = 2048;
    s.page_size = 4;
    return s;
}

}  // namespace strata::kernels

/* sc_handoff.h - the C-ABI of the MI355X prefill->decode cache handoff.
 *
 * One shared library, libsc_handoff.so, built for gfx950.  Every entry point is `extern "C"`, takes plain
 * pointers and sizes, returns an int status (SC_OK == 0) and never lets a C++ exception cross the ABI; the
 * message of the last failure on the calling thread is `sc_last_error()`.
 *
 * Status classes follow the reference's restore contract (include/strata/core/conversation_snapshot.hpp:103-108):
 *   SC_EINVAL  the request was refused BEFORE any device work was enqueued; nothing was written
 *              (the reference's `ConversationRestore::invalid`, conversation_state.cpp:474);
 *   SC_EHIP    a HIP call failed after work may have been enqueued: destination state is undefined
 *              (the reference's `transfer_failed`, conversation_state.cpp:478-504; fatal to that slot).
 *
 * Layouts (all device memory unless a name says host):
 *   prefill K/V   [T][n_head_kv][head_dim]         f16 (or f32, rounded RNE to f16 as kv_append does)
 *   prefill rec   [HV][S][S] f32                  head-major recurrent state of one GDN layer
 *   prefill conv  [rows][C] f32 (row stride ld)   the conv input rows; the history is the last 3 rows
 *   decode K/V    [page][n_head_kv][page_size][head_dim] f16 through a page table
 *                 (include/strata/core/layer.hpp:204-205; identity when the table is NULL = kv_mode 0)
 *   decode GDN    one row per GDN layer: (S, HV, S) f32 recurrence then [C][d_conv-1] f32 history
 *                 (src/core/session.cpp:156-162, src/kernels/cuda/gdn.cu:75)
 *   image         the park image / transfer buffer: the blobs of a SavedConversation in the wire codec's
 *                 blob-pool order, each 64-byte aligned (src/core/conversation_wire.cpp:400-437):
 *                 for each QSA layer K then V (the first ceil(T/page_size)*page_size cells, as
 *                 conversation_kv_save copies them, src/core/conversation_snapshot.cpp:40-49,157-171),
 *                 then the GDN rows (conversation_checkpoint_save, src/core/conversation_state.cpp:233-235).
 */
#ifndef SC_HANDOFF_H
#define SC_HANDOFF_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    SC_OK = 0,
    SC_EINVAL = 1,   /* refused before any write */
    SC_EHIP = 2,     /* HIP failure after work may have been enqueued (transfer_failed) */
    SC_ENOMEM = 3,   /* an allocation the call needed failed; nothing was written */
    SC_ERANGE = 4,   /* a size is beyond what the entry point supports; nothing was written */
    /* 5 and 6 are sc_arena.h's SC_EBUSY and SC_ESTALE */
    SC_ETIMEOUT = 7  /* a bounded wait on the device ran out: the launch ended, its result is not to be used */
};

enum { SC_DTYPE_F16 = 0, SC_DTYPE_F32 = 1 };

/* Blob kinds of the image (one row each in the image layout). */
enum { SC_BLOB_K = 1, SC_BLOB_V = 2, SC_BLOB_GDN = 3 };

/* The subset of strata::core::ModelGeometry (include/strata/core/layout.hpp:27-59) the path depends on, plus
 * the page granule of strata::kernels::QsaShapes (include/strata/kernels/qsa.hpp:113, page_size = 4). */
typedef struct sc_geometry {
    int64_t n_layers;          /* layout.hpp:29 */
    int64_t qsa_interval;      /* layout.hpp:30: layer % qsa_interval == qsa_interval - 1 is full attention */
    int64_t n_head_kv;         /* layout.hpp:42 */
    int64_t head_dim;          /* layout.hpp:43; a multiple of 8 (16-byte rows) */
    int64_t page_size;         /* qsa.hpp:113 */
    int64_t ssm_state_size;    /* S, layout.hpp:33 */
    int64_t ssm_k_heads;       /* layout.hpp:34 */
    int64_t ssm_v_heads;       /* HV, layout.hpp:35 */
    int64_t ssm_d_conv;        /* layout.hpp:36: the history keeps d_conv - 1 = 3 rows */
    int64_t ssm_conv_channels; /* C, layout.hpp:37 */
    int64_t idx_key_dim;       /* layout.hpp:45 */
} sc_geometry;

/* The carve source: one prefilled sequence (or one appended chunk of it) in the prefill layout.
 * The pointer arrays are HOST arrays of DEVICE pointers, one entry per QSA / GDN layer in layer order. */
typedef struct sc_prefill_view {
    int64_t tokens;               /* T: prefill token t lands in decode cell pos0 + t */
    int64_t pos0;                 /* first decode cell written (kv_append's pos0, src/prefill/kernels.cu:570-573) */
    int32_t kv_dtype;             /* SC_DTYPE_F16 (a pure permutation) or SC_DTYPE_F32 (RNE to f16) */
    int32_t with_gdn;             /* 0: K/V only (an appended chunk); 1: carve the GDN state too */
    const void* const* k;         /* [n_qsa] -> [T][n_head_kv][head_dim] */
    const void* const* v;         /* [n_qsa] */
    const float* const* rec;      /* [n_gdn] -> [HV][S][S] */
    const float* const* conv;     /* [n_gdn] -> [conv_rows][C] conv input rows (row stride conv_ld floats) */
    int64_t conv_rows;            /* rows in each conv source; fewer than 3 keeps older history rows
                                     (gdn_conv_hist_kernel, src/prefill/kernels.cu:219-228) */
    int64_t conv_ld;              /* row stride of the conv source in floats (>= C) */
} sc_prefill_view;

/* strata::kernels::KvHostPools (include/strata/kernels/kv_stream.hpp:30-39), member for member: one layer's host
 * copy (device-mapped pinned memory) or staging pool, identity layout [block][kv_head][page_size][row]. */
typedef struct sc_kv_pools {
    uint16_t* k_pool;   /* f16 rows */
    uint16_t* v_pool;
    int8_t* k_q;        /* int8 codes */
    int8_t* v_q;
    uint16_t* k_scale;  /* int8: one f16 scale per 64 values */
    uint16_t* v_scale;
    uint8_t* k_q4;      /* q4_0 blocks, 144 bytes per cell and head */
    uint8_t* v_q4;
} sc_kv_pools;

/* The decode slot: the device pointers of a strata::core::SessionState's state for one sequence
 * (include/strata/core/session.hpp:30-60 and QsaState, include/strata/core/layer.hpp:203-225). */
typedef struct sc_decode_slot {
    int64_t n_pages;                    /* physical pages in each K/V pool */
    int64_t max_cells;                  /* logical capacity in cells (n_pages * page_size for identity) */
    uint16_t* const* k_pool;            /* [n_qsa] -> [n_pages][n_head_kv][page_size][head_dim] f16 */
    uint16_t* const* v_pool;            /* [n_qsa] */
    const int32_t* const* page_table;   /* NULL, or [n_qsa] device tables logical page -> physical page;
                                           a NULL entry is the identity table (kv_mode 0) */
    float* gdn_state;                   /* n_gdn rows of sc_gdn_row_floats() floats (session.hpp:34) */
    /* A streamed layer's authoritative host copy and the prompt path's staging pool: NULL, or host arrays [n_qsa] of
     * sc_kv_pools in the identity layout [logical page][n_head_kv][page_size][row] holding max_cells cells (the host
     * copy is device-mapped pinned memory, the staging pool device memory).  An entry whose pools of the slot's
     * format are NULL is skipped.  The kernels write a host copy straight into host memory, so one that is not
     * pinned memory mapped for the device is refused when the plan is built (sc_host_range_mapped).  A carve writes every cell it carves into each given pool as well, resident in the
     * paged pool or not, in the same launch (kv_append, src/prefill/kernels.cu:574-577,587-600;
     * kv_append_q4, src/kernels/cuda/kv_q4.cu:124-128). */
    const sc_kv_pools* host;
    const sc_kv_pools* stage;
} sc_decode_slot;

/* One row of an image layout. */
typedef struct sc_image_blob {
    int32_t kind;     /* SC_BLOB_K, SC_BLOB_V, SC_BLOB_GDN */
    int32_t layer;    /* QSA ordinal for K/V, -1 for the GDN blob */
    uint64_t offset;  /* from the image start, a multiple of 64 */
    uint64_t bytes;
} sc_image_blob;

typedef struct sc_plan sc_plan;   /* a device-resident handoff table plus its launch shape */
typedef struct sc_hash_map sc_hash_map;   /* capture plans' rows as the sources of a payload, for the fused hash */
/* A payload held in segments rather than one allocation (the same-GPU hand-off's exported segments, each its own
 * allocation of at most SC_IPC_MAX_SEGMENT bytes): payload byte o lives at ptr[o / segment_bytes] + o % segment_bytes,
 * every segment but the last holding segment_bytes (a multiple of 64 KiB), the last the rest. */
typedef struct sc_segments {
    int32_t n;                /* segments, 1 .. SC_IPC_MAX_SEGMENTS */
    uint64_t segment_bytes;   /* bytes of each segment but the last */
    void* const* ptr;         /* [n] 16-byte aligned device pointers, host array */
} sc_segments;

/* ---- errors ---------------------------------------------------------------------------------------------- */

/* The message of the last failure on this thread ("" after a success).  Messages of refusals carry the
 * reference's prefix "conversation snapshot: " where the reference has the same refusal
 * (src/core/conversation_state.cpp:21-24). */
const char* sc_last_error(void);
/* Library version, e.g. "sc_handoff 0.1 gfx950". */
const char* sc_version(void);

/* ---- geometry and layout arithmetic (host only, no HIP call) ----------------------------------------------- */

/* QSA and GDN layer counts: n_layers / qsa_interval and the rest (layout.hpp:57-58). */
int64_t sc_n_qsa_layers(const sc_geometry* g);
int64_t sc_n_gdn_layers(const sc_geometry* g);
/* Floats of one GDN row: S*HV*S + C*(d_conv-1) (conversation_state.cpp:186-189, session.cpp:160-161). */
int64_t sc_gdn_row_floats(const sc_geometry* g);
/* Cells a park copies for `tokens`: ceil(tokens/page_size)*page_size (conversation_snapshot.cpp:40). */
int64_t sc_kv_cells(const sc_geometry* g, int64_t tokens);
/* Payload bytes of one handoff of `tokens` tokens: K+V of every QSA layer over sc_kv_cells() cells plus every
 * GDN row.  The figure behind the bench's GB/s. */
uint64_t sc_payload_bytes(const sc_geometry* g, int64_t tokens);
/* The image layout for `tokens`.  With blobs == NULL only *n_blobs and *total_bytes are written.
 * Replaces the byte accounting of conversation_kv_bytes / conversation_snapshot_bytes
 * (include/strata/core/conversation_snapshot.hpp:13,87-88) for the K/V + GDN payload. */
int sc_image_layout(const sc_geometry* g, int64_t tokens, sc_image_blob* blobs, int64_t* n_blobs,
                    uint64_t* total_bytes);

/* ---- plans: the device-resident handoff table ---------------------------------------------------------------- */

/* Fused carve -> scatter: prefill layout straight into the decode slot, one launch for every layer.
 * Replaces kv_append (include/strata/prefill/kernels.hpp:81-83, src/prefill/kernels.cu:560-625) and
 * gdn_conv_hist (src/prefill/kernels.cu:219-228) as the writers of the decode layout, plus the GDN row
 * placement of src/prefill/prefill.cpp:1282-1283.  Validates extents against the slot first. */
int sc_plan_carve(const sc_geometry* g, const sc_prefill_view* src, const sc_decode_slot* dst, sc_plan** out);
/* Re-points a carve plan at another prefill view of the same slot - new K/V, recurrence and conv pointers, token count,
 * pos0, dtype, with or without the GDN rows - without allocating and without waiting on the device: the new table rows
 * go through pinned staging the plan owns, and a small kernel on `stream` copies them into the plan's device table and
 * rebuilds its tile map before the next launch on that stream.  So a serving engine builds one plan per decode slot and
 * pays a few microseconds per hand-off instead of a table build (device allocations and blocking uploads); the
 * reference's per-layer writer likewise takes every pointer as an argument per call (src/prefill/kernels.cu:618-625,
 * src/prefill/prefill.cpp:1327-1340).  The view must fit what the plan was built with: its rows and tiles at most the
 * build's (build the plan with the largest view it will carve, e.g. the slot's capacity), the GDN rows only if the build
 * carved them; otherwise SC_ERANGE and the plan is unchanged, as it is after any refusal (SC_EINVAL).  Retargets and
 * launches of one plan must be issued on one stream (or ordered by events); the host-side fields change at once, so a
 * launch enqueued after the call carves the new view.  Only plans from sc_plan_carve can be retargeted. */
int sc_plan_retarget(sc_plan* plan, const sc_prefill_view* src, void* stream);
/* Quantized K/V storage of the decode pools (include/strata/kernels/kv_stream.hpp:44-46 KvFormat, plus the K8V4
 * hybrid of src/core/conversation_snapshot.cpp's format 3): int8 codes with one f16 scale per 64 values (kv_q8.hpp),
 * q4_0 blocks of 32 values, 18 bytes each (kv_q4.hpp:21-28), or int8 K with q4_0 V. */
enum { SC_KV_F16 = 0, SC_KV_INT8 = 1, SC_KV_Q4 = 2, SC_KV_K8V4 = 3 };

/* A decode slot whose K/V pools are quantized (QsaState::k_q / v_q / k_scale / v_scale / k_q4 / v_q4,
 * include/strata/core/layer.hpp:206-215).  Pools are indexed by pool row (page * H + h) * page_size + cell % page_size:
 * int8 codes 256 bytes per row, int8 scales 4 f16 (8 bytes) per row, q4_0 8 blocks (144 bytes) per row. */
typedef struct sc_quant_slot {
    int64_t n_pages;
    int64_t max_cells;
    int32_t format;                     /* SC_KV_INT8, SC_KV_Q4 or SC_KV_K8V4 */
    void* const* k_codes;               /* [n_qsa]: int8 codes (INT8, K8V4) or q4_0 blocks (Q4) */
    void* const* v_codes;               /* [n_qsa]: int8 codes (INT8) or q4_0 blocks (Q4, K8V4) */
    uint16_t* const* k_scale;           /* [n_qsa] f16 scales of K (INT8, K8V4), else NULL */
    uint16_t* const* v_scale;           /* [n_qsa] f16 scales of V (INT8), else NULL */
    const int32_t* const* page_table;   /* as sc_decode_slot */
    float* gdn_state;
    const sc_kv_pools* host;            /* as sc_decode_slot: int8 codes + scales, or q4_0 blocks (not for K8V4, which */
    const sc_kv_pools* stage;           /* is resident only, conversation_snapshot.cpp's hybrid rule) */
} sc_quant_slot;

/* The quantizing carve: f32 prefill K/V rows [T][H][256] (q4_0 rows already rotated, as the reference rotates before
 * kv_append_q4) into quantized decode pools, plus the GDN state, in one launch.  Replaces the int8 path of kv_append
 * (src/prefill/kernels.cu:578-600) and kv_append_q4 (src/kernels/cuda/kv_q4.cu:111-129, launched from
 * src/prefill/prefill.cpp).  src->kv_dtype must be SC_DTYPE_F32 and head_dim 256.  sc_plan_payload_bytes() of the
 * plan counts the bytes it reads plus the bytes it writes. */
int sc_plan_carve_quant(const sc_geometry* g, const sc_prefill_view* src, const sc_quant_slot* dst, sc_plan** out);
/* ---- kv_append: the per-layer prefill writers, with the reference's arguments ---------------------------------
 * One launch per call, nothing allocated, like the reference's own (the plans above build a whole slot in one launch
 * instead).  Every entry point returns before its launch when T <= 0, and refuses (SC_EINVAL, nothing launched)
 * missing or misaligned buffers and impossible extents; pools are not bounded, the caller sized them, as there.  A
 * host copy is written by the kernel straight into host memory: the pages a call writes must be pinned memory mapped
 * for the device, which is checked before the launch (SC_EINVAL otherwise). */


/* kv_append (include/strata/prefill/kernels.hpp:78-83, src/prefill/kernels.cu:558-625): K and V, f32 [T][2][256]
 * (positions pos0 .. pos0 + T - 1), into the paged pool - f16 rows (RNE) when k_pool is given, else int8 codes with an
 * f16 scale per 64 values - through page_table (NULL: identity), skipping cells whose page entry is negative; also
 * into the host copy and the staging pool (identity layout, every cell) when `host` / `stage` name pools of the same
 * format.  K8V4's K-only call (K == V, k_q == v_q) is allowed.  Pool alignment: f16 16 bytes, int8 codes 4, scales 8. */
int sc_kv_append_async(const float* K, const float* V, int64_t T, int64_t pos0, const int32_t* page_table,
                       int64_t page_size, uint16_t* k_pool, uint16_t* v_pool, int8_t* k_q, int8_t* v_q,
                       uint16_t* k_scale, uint16_t* v_scale, void* stream, const sc_kv_pools* host,
                       const sc_kv_pools* stage);
/* kv_append_q4 (include/strata/kernels/kv_q4.hpp:50-54, src/kernels/cuda/kv_q4.cu:110-135,205-215): already rotated
 * K and V, f32 [T][n_head_kv][256], into q4_0 pools through page_table, and into host->k_q4 / stage->k_q4 (identity)
 * when given.  head_dim must be 256. */
int sc_kv_append_q4_async(uint8_t* k_q4, uint8_t* v_q4, const int32_t* page_table, int64_t pos0, int64_t T,
                          const float* K, const float* V, int64_t n_head_kv, int64_t head_dim, int64_t page_size,
                          void* stream, const sc_kv_pools* host, const sc_kv_pools* stage);

/* Pass 1 of the two-pass handoff: carve into a transfer buffer laid out as the image for src->tokens
 * (pos0 must be 0).  The transfer buffer is what a park writes and what crosses to another instance. */
int sc_plan_gather(const sc_geometry* g, const sc_prefill_view* src, void* image, uint64_t image_bytes,
                   sc_plan** out);
/* Pass 2: an image of `tokens` tokens into a decode slot through its page tables.  With identity tables it
 * is the device-side twin of conversation_kv_restore + conversation_checkpoint_restore's GDN copy
 * (conversation_snapshot.cpp:196-204, conversation_state.cpp:251), and of kv_stage_from_host
 * (src/kernels/cuda/kv_stream.cu:244-252) for paged pools. */
int sc_plan_scatter(const sc_geometry* g, const void* image, uint64_t image_bytes, int64_t tokens,
                    const sc_decode_slot* dst, sc_plan** out);
/* The inverse: a decode slot's first sc_kv_cells(tokens) cells and its GDN rows into an image, through the
 * page tables.  The device half of conversation_kv_save (conversation_snapshot.cpp:139-173) for paged pools. */
int sc_plan_capture(const sc_geometry* g, const sc_decode_slot* src, int64_t tokens, void* image,
                    uint64_t image_bytes, sc_plan** out);
/* Where the blobs of a capture or scatter sit in a caller-laid-out buffer, e.g. the blob pool of a wire payload
 * (include/strata/core/conversation_wire.hpp:24-81: the pool of a K/V + running-state image holds each QSA layer's K
 * then V blob, then the GDN rows, each 64-byte aligned, with other entries - the draft layer, the small checkpoint
 * buffers - between or after them).  Offsets are bytes from the buffer start, 16-byte aligned; blobs must not overlap. */
typedef struct sc_blob_map {
    const uint64_t* k_off;   /* [n_qsa] the K blob of QSA layer j: its first sc_kv_cells(tokens) cells, identity layout */
    const uint64_t* v_off;   /* [n_qsa] the V blob */
    uint64_t gdn_off;        /* every GDN row (ignored without GDN layers) */
    const uint64_t* zero;    /* [2 * n_zero] (offset, bytes) ranges a capture zero-fills: whole 16-byte chunks */
    int64_t n_zero;
} sc_blob_map;
/* A slot's first sc_kv_cells(tokens) cells (through its page tables) and GDN rows into the blobs `map` places in
 * `dst`, and the zero ranges cleared, in one launch: the device half of writing a payload's pool straight from the
 * slot (the reference fills the pool from host copies, src/core/conversation_wire.cpp:400-437). */
int sc_plan_capture_map(const sc_geometry* g, const sc_decode_slot* src, int64_t tokens, void* dst, uint64_t dst_bytes,
                        const sc_blob_map* map, sc_plan** out);
/* The inverse: the blobs `map` places in `src` into the slot, in one launch (the device half of mounting a decoded
 * payload, the reference's Decoder::blobref + conversation_kv_restore, conversation_wire.cpp:694-754 and
 * src/core/conversation_snapshot.cpp:196-204). */
int sc_plan_scatter_map(const sc_geometry* g, const void* src, uint64_t src_bytes, const sc_blob_map* map,
                        int64_t tokens, const sc_decode_slot* dst, sc_plan** out);
/* ---- slot images in every K/V format ------------------------------------------------------------------------------
 * A slot's per-layer buffers as conversation_kv_save takes them (src/core/conversation_snapshot.cpp:69-78, pools()):
 * the K and V data, the K and V int8 scales and the indexer's pooled rows, each in the identity layout (kv_mode 0, the
 * layout a snapshot copies a prefix of), plus the GDN rows. */
enum { SC_BUF_K = 0, SC_BUF_V = 1, SC_BUF_K_SCALE = 2, SC_BUF_V_SCALE = 3, SC_BUF_POOLED = 4, SC_N_BUF = 5 };
/* The indexer pools one key per 4 cells (include/strata/kernels/qsa.hpp:103,112: idx_block). */
enum { SC_IDX_BLOCK = 4 };
typedef struct sc_slot_layers {
    int32_t format;               /* SC_KV_F16, SC_KV_INT8, SC_KV_Q4 or SC_KV_K8V4 */
    int32_t with_index;           /* 1: the indexer's pooled rows belong to the image (include_index) */
    int64_t max_cells;            /* cells every K/V buffer holds (QsaState::max_cells) */
    int64_t pooled_capacity;      /* rows every pooled buffer holds (QsaState::idx_pooled_rows) */
    void* const* buf[SC_N_BUF];   /* host arrays of [n_qsa] device pointers, by SC_BUF_*; NULL where the format or
                                     with_index has no such buffer */
    float* gdn_state;             /* the n_gdn GDN rows (NULL without GDN layers) */
} sc_slot_layers;
/* Bytes of one QSA layer's five blobs for `tokens` tokens, by conversation_snapshot.cpp:27-66 (layout()): cells =
 * sc_kv_cells(tokens); K and V data cells*H*(2D f16, D int8, D/32*18 q4_0; K8V4: D for K, D/32*18 for V); int8 scales
 * cells*H*(D/64)*2 (K8V4: K only); pooled rows (tokens/SC_IDX_BLOCK + 1)*idx_key_dim*4 when with_index and tokens > 0.
 * Refuses a head_dim the format cannot hold (int8 needs D % 64 == 0, q4_0 D % 32 == 0). */
int sc_layer_blob_bytes(const sc_geometry* g, int32_t format, int32_t with_index, int64_t tokens, uint64_t* bytes);
/* The image of a slot in any format: for each QSA layer its nonempty blobs in SC_BUF order, then the GDN rows, each
 * on a 64-byte boundary (the wire codec's pool order, src/core/conversation_wire.cpp:400-437).  offsets (may be NULL)
 * gets n_qsa*SC_N_BUF + 1 entries: blob b of layer j at [j*SC_N_BUF + b], the GDN rows last; UINT64_MAX marks an
 * empty blob.  For SC_KV_F16 without the index it is sc_image_layout. */
int sc_image_layout_layers(const sc_geometry* g, int32_t format, int32_t with_index, int64_t tokens, uint64_t* offsets,
                           uint64_t* total_bytes);
/* Where a capture or scatter of sc_slot_layers puts each blob in a caller-laid-out buffer (a wire payload's pool):
 * `off` as sc_image_layout_layers writes it (16-byte aligned, UINT64_MAX for an empty blob), and zero ranges as in
 * sc_blob_map.  A NULL map means the image layout of sc_image_layout_layers with its gaps zeroed. */
typedef struct sc_layers_map {
    const uint64_t* off;     /* [n_qsa*SC_N_BUF + 1] */
    const uint64_t* zero;    /* [2*n_zero] (offset, bytes) ranges a capture zero-fills: whole 16-byte chunks */
    int64_t n_zero;
} sc_layers_map;
/* The slot's blob prefixes and GDN rows into `dst`, in one launch: the device half of conversation_kv_save for every
 * format (conversation_snapshot.cpp:139-173) and of conversation_checkpoint_save's GDN copy (conversation_state.cpp:235).
 * Every blob must be whole 16-byte chunks (SC_ERANGE otherwise). */
int sc_plan_capture_layers(const sc_geometry* g, const sc_slot_layers* src, int64_t tokens, void* dst,
                           uint64_t dst_bytes, const sc_layers_map* map, sc_plan** out);
/* The inverse, in one launch: conversation_kv_restore for every format (conversation_snapshot.cpp:196-204) and the GDN
 * restore (conversation_state.cpp:251).  Bytes of the slot past the image's cells and rows are left as they are. */
int sc_plan_scatter_layers(const sc_geometry* g, const void* src, uint64_t src_bytes, const sc_layers_map* map,
                           int64_t tokens, const sc_slot_layers* dst, sc_plan** out);
/* The scatters of sc_plan_scatter_map / sc_plan_scatter_layers from a segmented payload (a payload mounted straight
 * from another process's exported segments): the blob map's offsets are payload offsets, and a blob a segment boundary
 * cuts is read from both segments (the page-scatter rows of its pieces keep their place in its pages). */
int sc_plan_scatter_map_segments(const sc_geometry* g, const sc_segments* src, uint64_t src_bytes,
                                 const sc_blob_map* map, int64_t tokens, const sc_decode_slot* dst, sc_plan** out);
int sc_plan_scatter_layers_segments(const sc_geometry* g, const sc_segments* src, uint64_t src_bytes,
                                    const sc_layers_map* map, int64_t tokens, const sc_slot_layers* dst,
                                    sc_plan** out);
/* Park / resume of a slot in any format to / from a pinned host image of sc_image_layout_layers, one hipMemcpyAsync per
 * blob on `stream`, `done` recorded after the last (as sc_park_async / sc_resume_async for f16 slots). */
int sc_park_layers_async(const sc_geometry* g, const sc_slot_layers* slot, int64_t tokens, void* host_image,
                         uint64_t image_bytes, void* stream, void* done);
int sc_resume_layers_async(const sc_geometry* g, const void* host_image, uint64_t image_bytes, int64_t tokens,
                           const sc_slot_layers* slot, void* stream, void* done);
/* A plan of plain device-to-device copies: `n` copies of `bytes` each (whole 16-byte chunks, both addresses 16-byte
 * aligned, no two destinations overlapping), moved by one launch.  Its use is as a row source of a hash map
 * (sc_hash_map_create, _segments): bytes staged in device memory once, such as a payload's head built on the host,
 * are then written by the fused gather + hash itself instead of copied in before it.  No counterpart in the reference
 * (its encoder writes the head and the pool with one host walk, src/core/conversation_wire.cpp:400-480). */
typedef struct sc_copy {
    void* dst;
    const void* src;
    uint64_t bytes;
} sc_copy;
int sc_plan_copies(const sc_copy* copies, int32_t n, sc_plan** out);
/* Enqueue the plan on `stream` (a hipStream_t; NULL is the null stream).  Asynchronous. */
int sc_plan_launch(const sc_plan* plan, void* stream);
/* sc_plan_launch that moves nothing unless the 32-bit word at `gate` (device memory, written by earlier work on the
 * same stream, e.g. the verdict of sc_fnv1a64_check_async) is nonzero when the launch runs.  Every workgroup reads the
 * same word, so the launch writes all of the plan's bytes or none: a mount that checks its payload hash on the device
 * and scatters without a host round trip (the reference compares the hash on the host before it mounts,
 * src/core/conversation_wire.cpp:1069-1071).  Not for batched plans (SC_EINVAL). */
int sc_plan_launch_gated(const sc_plan* plan, const uint32_t* gate, void* stream);
/* Algorithmic payload bytes the plan moves (each read once and written once). */
uint64_t sc_plan_payload_bytes(const sc_plan* plan);
/* Workgroups the launch uses, for launch-shape sweeps; 0 restores the grid the plan was built with. */
int sc_plan_set_grid(sc_plan* plan, int64_t workgroups);
/* Destination order (no reference counterpart: a launch-shape choice of this build).  Rows that write through a page
 * table (K/V carves into a paged slot, image pages scattered into one) visit their pages in the order of the
 * physical pages, so the writes of a launch form one ascending run of the pool; the order is rebuilt on the device by
 * three small kernels before every launch of the plan (the table may change between launches), in the plan's own
 * workspace - so launches of one such plan on different streams must not overlap.  A table gets the order when it
 * covers at least `pages` logical pages in a pool of at most 8 times as many physical pages.  Library-wide, for plans
 * built afterwards; pages <= 0 turns it off.  Returns the previous value (default 2048).  A table must name each
 * physical page at most once: in source order two logical pages on one physical page race (as the reference's
 * kv_append does), and in destination order that page receives one of them whole. */
int64_t sc_set_order_min_pages(int64_t pages);
/* How many page tables of the plan are visited in destination order (0: every row follows its source). */
int sc_plan_order_groups(const sc_plan* plan);
/* Frees the device table.  The caller must not destroy a plan whose launch has not completed. */
int sc_plan_destroy(sc_plan* plan);

/* ---- batched ragged resume + append (many slots, one launch) ---------------------------------------------------- */

/* The multi-slot decode layout: every QSA layer has one shared page arena [arena_pages][H][ps][D] f16, each slot
 * reads it through its own page table, and each slot has its own GDN rows.  There is no reference counterpart:
 * the reference keeps one live session (docs/STAGE3-CONCURRENCY.md:182) and designs batching with a shared K/V
 * arena plus per-sequence page tables (docs/STAGE4-BATCH-DECODE.md:474-518), which is this layout.  Parity rule:
 * each slot read through its table equals the single-slot handoff of that slot's sequence. */
typedef struct sc_batch_desc {
    int32_t n_slots;               /* 1..64 */
    const int64_t* lens;           /* device [n_slots]: parked tokens L_i, read when the launch runs */
    int64_t max_tokens;            /* bound on every L_i; a slot outside [0, max_tokens] refuses the whole batch */
    const void* staging;           /* device: the parked images back to back (sc_batch_staging_layout) */
    uint64_t staging_bytes;
    int64_t chunk_tokens;          /* the fresh prefill chunk appended to every slot at cell L_i */
    const void* const* chunk_k;    /* host array [n_slots * n_qsa] of device [chunk_tokens][H][D] f16, slot-major */
    const void* const* chunk_v;
    uint16_t* const* arena_k;      /* host array [n_qsa] of device page arenas */
    uint16_t* const* arena_v;
    int64_t arena_pages;
    const int32_t* const* tables;  /* host array [n_slots] of device page tables, logical page -> arena page */
    int64_t table_pages;           /* entries per table, >= ceil((max_tokens + chunk_tokens) / page_size) */
    float* const* gdn;             /* host array [n_slots] of device GDN rows (n_gdn rows each) */
    int64_t* lens_out;             /* device [n_slots] or NULL: L_i + chunk_tokens, or -1 for a skipped slot */
} sc_batch_desc;

/* Where slot i's parked image of lens[i] tokens sits in the staging buffer: images back to back, each padded to
 * 256 bytes (an exclusive prefix sum of the padded image sizes).  The launch recomputes the same offsets on the
 * device from the device-resident lengths with a wave-level scan; this host twin places the H2D copies. */
int sc_batch_staging_layout(const sc_geometry* g, const int64_t* lens, int32_t n_slots, uint64_t* offsets,
                            uint64_t* total_bytes);
/* One launch for every slot: its parked K/V prefix and its GDN rows from the staging buffer into the arena through
 * its table, and its chunk's K/V at cells [L_i, L_i + chunk) (kv_append's mapping, src/prefill/kernels.cu:567-573,
 * including a start in the middle of a page).  A small pre-pass reads the lengths: the staging offsets are a
 * wave-level exclusive scan over the slots (the device analogue of the reference's block_scan,
 * src/kernels/cuda/kv_stream.cu:58-80), and the arena pages the slots' tables name are put in ascending arena order;
 * the move then assembles each arena page once, in that order (parked cells from the image, chunk cells from the
 * chunk), so no two workgroups write the same bytes and the arena is written as one ascending run.  If any length is
 * outside [0, max_tokens] or any image would run past the staging buffer, nothing is written and every lens_out
 * entry is -1.  The slots' tables must name disjoint arena pages (an arena page named twice receives one of its
 * logical pages).  The pre-pass uses the plan's workspace: launches of one plan on different streams must not
 * overlap. */
int sc_plan_resume_append(const sc_geometry* g, const sc_batch_desc* desc, sc_plan** out);

/* ---- park / resume: slot <-> pinned host image ----------------------------------------------------------------- */

/* Park: copy a decode slot into a pinned host image of sc_image_layout(tokens) on `stream`; records `done` (a
 * hipEvent_t, may be NULL) after the last copy.  An identity-layout slot takes one hipMemcpyAsync per blob; a paged
 * slot (any non-null page table) has its K/V pages gathered through the tables straight into the pinned image by a
 * kernel that writes the host memory itself (no staging copy in HBM, nothing allocated; 32 layers per launch), then
 * its GDN rows by one copy; a page whose entry is negative or past the pool (not resident) is skipped, and its bytes
 * of the image are left as they were.  A paged slot's image must be pinned memory mapped for the device (sc_host_alloc,
 * hipHostMalloc), which is checked before anything is enqueued (SC_EINVAL otherwise, see sc_host_range_mapped); an
 * identity slot's image may be any host memory hipMemcpyAsync accepts.  Replaces conversation_kv_save's synchronous
 * per-16-MiB cudaMemcpy loop
 * (conversation_snapshot.cpp:105-113, 160-171) and conversation_checkpoint_save's GDN copy (conversation_state.cpp:235). */
int sc_park_async(const sc_geometry* g, const sc_decode_slot* slot, int64_t tokens, void* host_image,
                  uint64_t image_bytes, void* stream, void* done);
/* Resume: the inverse, H2D (a paged slot's pages scattered through its tables by a kernel that reads the pinned
 * image itself).  Replaces conversation_kv_restore (conversation_snapshot.cpp:196-204) and
 * conversation_checkpoint_restore's GDN copy (conversation_state.cpp:251). */
int sc_resume_async(const sc_geometry* g, const void* host_image, uint64_t image_bytes, int64_t tokens,
                    const sc_decode_slot* slot, void* stream, void* done);

/* ---- block movers of streamed and ring K/V layers ---------------------------------------------------------------- */

/* The per-block byte runs of up to four pool arrays: block b of array i is bytes [b*len[i], (b+1)*len[i]) of
 * src[i] (the host copy, a device-mapped pinned pointer) and of dst[i] (the VRAM slots).  The reference's `Runs`
 * (src/kernels/cuda/kv_stream.cu:26-55): f16 K and V; int8 codes and scales; q4 codes. */
typedef struct sc_kv_runs {
    const void* src[4];
    void* dst[4];
    uint64_t len[4];
    int32_t n;
} sc_kv_runs;

/* Blocks [b0, b1) of the host copy into ring slots b % n_slots, as hipMemcpyAsync runs up to the ring's end.
 * Replaces kv_ring_restore (include/strata/kernels/kv_stream.hpp:78-81, src/kernels/cuda/kv_stream.cu:231-242). */
int sc_kv_ring_restore(const sc_kv_runs* runs, int64_t b0, int64_t b1, int64_t n_slots, void* stream);
/* The first n_blocks blocks of the host copy into an identity-layout pool.  Replaces kv_stage_from_host
 * (kv_stream.hpp:83-86, kv_stream.cu:244-252). */
int sc_kv_stage_from_host(const sc_kv_runs* runs, int64_t n_blocks, void* stream);
/* The static ring table block -> block % n_slots.  Replaces kv_ring_table (kv_stream.hpp:75-76, kv_stream.cu:226-229). */
int sc_kv_ring_table(int32_t* page_table, int64_t n_blocks, int64_t n_slots, void* stream);
/* Evicts every block of a streamed layer: page table -1, slots free (block -1, stamp -1, ref 0), the 16 control
 * ints zero.  Replaces kv_stream_reset (kv_stream.hpp:65-66, kv_stream.cu:173-182,199-202). */
int sc_kv_stream_reset(int32_t* page_table, int64_t n_blocks, int32_t* slot_block, int32_t* slot_stamp,
                       int32_t* slot_ref, int64_t n_slots, int32_t* ctl, void* stream);
/* Bytes of one block (page) of K and V together.  Replaces kv_block_bytes (kv_stream.hpp:95-96). */
uint64_t sc_kv_block_bytes(int64_t n_head_kv, int64_t head_dim, int64_t page_size, int32_t format);

/* ---- FNV-1a 64 of device bytes ------------------------------------------------------------------------------------ */

/* The engine's content hash - for every byte h = (h ^ b) * 1099511628211 mod 2^64 from `seed` - of `bytes` bytes of
 * device memory, bit-identical to the reference's byte loop fnv1a64 (src/core/pinned.cu:594-601; the payload hash of
 * conversation_wire_payload_hash, src/core/conversation_wire.cpp:1069-1071, and of HandoffArena::payload_hash_of,
 * src/core/handoff.cpp:1133-1136), computed in parallel on the device in one read of the input: the low byte of the
 * state is resolved a few bit planes at a time by xor prefixes and a look-back across workgroups, after which the hash
 * is a sum of independent per-segment terms.  The reference seeds every call with 1469598103934665603
 * (conversation_wire.hpp:196). */
/* Device workspace the asynchronous form needs for `bytes` bytes of input (about bytes / 3000, at least 512 bytes). */
uint64_t sc_fnv1a64_workspace_bytes(uint64_t bytes);
/* Enqueue the hash on `stream`; the result lands as one u64 at `out`, and the launch's status as one u32 at `fault`:
 * 0, or 1 when one of the kernel's bounded look-back waits ran out (never in a correct launch on a GPU that runs its
 * waves; sc_fnv1a64_set_spin_limit forces it), in which case the u64 at `out` is not the hash and must not be used.
 * `out` and `fault` (required, 4-byte aligned) may be device memory or pinned host memory mapped for the device.
 * `data` may have any alignment (16-byte aligned input takes the vector path); `workspace` is 16-byte aligned device
 * memory of at least sc_fnv1a64_workspace_bytes(bytes); nothing is allocated. */
int sc_fnv1a64_async(const void* data, uint64_t bytes, uint64_t seed, uint64_t* out, uint32_t* fault, void* workspace,
                     uint64_t workspace_bytes, void* stream);
/* sc_fnv1a64_async that also writes, at `verdict` (4-byte aligned device memory), 1 when the hash equals `expected` and
 * no wait ran out, and 0 otherwise: the gate of sc_plan_launch_gated.  `fault` is optional here (NULL: the verdict
 * alone carries the fault), with the meaning it has in sc_fnv1a64_async. */
int sc_fnv1a64_check_async(const void* data, uint64_t bytes, uint64_t seed, uint64_t expected, uint64_t* out,
                           uint32_t* verdict, uint32_t* fault, void* workspace, uint64_t workspace_bytes, void* stream);
/* The same hash continued over one more piece: the running hash is the u64 at `state` in device memory (the seed
 * before the first piece), read when the piece's kernels run on `stream` and replaced by the hash of everything so
 * far.  Hashing a buffer piece by piece in order, each call after the one before it on the same stream, gives the
 * one-shot hash of the whole buffer: fnv1a64 is a left fold, and the reference chains it the same way through its
 * seed argument (src/core/conversation_wire.cpp:135,679-683).  This lets a copy into device memory be verified piece
 * by piece while later pieces are still in flight.  `state` is 8-byte aligned; the workspace rules are those of
 * sc_fnv1a64_async for `bytes`.  `fault` (required, 4-byte aligned) is sticky across a chain: a piece whose wait ran
 * out sets it to 1 and a piece without a fault leaves it as it is, so the caller clears it (0) with the seed before
 * the first piece and reads it with the final state; 1 means the state is not the hash.  Nothing is allocated. */
int sc_fnv1a64_chain_async(const void* data, uint64_t bytes, uint64_t* state, uint32_t* fault, void* workspace,
                           uint64_t workspace_bytes, void* stream);
/* Synchronous convenience: allocates its workspace, runs on the null stream, waits, and returns the hash in *hash
 * (SC_ETIMEOUT, and *hash untouched, when a wait of the kernel ran out). */
int sc_fnv1a64_device(const void* data, uint64_t bytes, uint64_t seed, uint64_t* hash);
/* sc_fnv1a64_async without a workspace argument and without any allocation.  No counterpart in the reference: it is
 * for callers that cannot allocate (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  The workspace is a static device array the library holds on each GPU until the process ends, sized for
 * inputs of at most SC_FNV_NOALLOC_MAX_BYTES (larger inputs are refused with SC_ERANGE before anything is enqueued).
 * Each call clears what it uses of the array with a kernel of its own first.  `out` and `fault` are as in
 * sc_fnv1a64_async.  Calls ordered on one stream are safe; calls that overlap on one GPU (on different streams) race
 * on the shared array and must not be issued. */
#define SC_FNV_NOALLOC_MAX_BYTES (4ull << 30)
int sc_fnv1a64_noalloc_async(const void* data, uint64_t bytes, uint64_t seed, uint64_t* out, uint32_t* fault,
                             void* stream);
/* The capture fused with its hash.  A capture plan (sc_plan_capture*, sc_plan_gather: page gathers, copies and zero
 * fills into the payload) writes the payload from the slot, and the payload hash then reads it all again; the encode of
 * a hand-off payload (conversation_wire_encode's walk and hash, src/core/conversation_wire.cpp:400-480, 1069-1071) is
 * both.  sc_hash_map_create reads the rows of `n_plans` capture plans writing into `payload` (16-byte aligned, `bytes`
 * a multiple of 16, every row inside it and no two rows on the same bytes; the bytes no row writes are taken as the
 * payload holds them when the launch runs, e.g. a head copied in before it) and uploads them as a map of the payload
 * once (this allocates); sc_hash_map_launch then gathers every row's bytes into the payload and hashes the whole payload
 * in one kernel that reads each source byte once, with the result and fault word of sc_fnv1a64_async.  The payload
 * afterwards holds exactly what launching the plans would write.  Nothing is allocated per launch; the plans may be
 * destroyed after the map is made, their sources and the payload must stay where they were. */
int sc_hash_map_create(const sc_plan* const* plans, int32_t n_plans, void* payload, uint64_t bytes, sc_hash_map** out);
int sc_hash_map_launch(const sc_hash_map* map, uint64_t seed, uint64_t* out, uint32_t* fault, void* workspace,
                       uint64_t workspace_bytes, void* stream);
/* sc_hash_map_create for a segmented payload: the plans were built for a contiguous payload at `frame` (any 16-byte
 * aligned address: they are never launched, and may be destroyed once the map exists), and the map writes their rows'
 * bytes into the segments of `into` instead, at the same payload offsets. */
int sc_hash_map_create_segments(const sc_plan* const* plans, int32_t n_plans, const void* frame, uint64_t bytes,
                                const sc_segments* into, sc_hash_map** out);
/* A map that only hashes a segmented payload where it lies (nothing is written): the hash of a payload spread over
 * imported segments, in one launch. */
int sc_hash_map_create_read(const sc_segments* from, uint64_t bytes, sc_hash_map** out);
/* sc_hash_map_launch that also leaves the verdict of sc_fnv1a64_check_async at `verdict` (the gate of
 * sc_plan_launch_gated); `fault` is optional here. */
int sc_hash_map_check_async(const sc_hash_map* map, uint64_t seed, uint64_t expected, uint64_t* out, uint32_t* verdict,
                            uint32_t* fault, void* workspace, uint64_t workspace_bytes, void* stream);
/* The carries of a hashed input: the low byte of the running hash after each whole 64 KiB of the input whose end lies
 * strictly inside it - sc_fnv1a64_carry_bytes(bytes) bytes, one per boundary, in order.  No counterpart in the
 * reference: they are what lets a consumer check a payload's hash without the kernel's serial look-back across
 * workgroups.  The hash kernel resolves the low byte of the state at every 64 KiB boundary anyway; a producer writes
 * those bytes out beside the hash (sc_fnv1a64_carry_async, sc_hash_map_launch_carry: the same launch, one byte store per
 * 64 KiB), ships them with the payload, and a consumer's check given them (sc_fnv1a64_check_carried_async,
 * sc_hash_map_check_carried_async) starts every 64 KiB workgroup from the carry before it instead of waiting for its
 * predecessors, and checks that it ends with the carry after it.  The check stays exact: if every workgroup ends with
 * the carry after it, every carry is the true state (by induction from the seed), so the hash computed is the
 * payload's FNV-1a; if any does not, the payload or its carries are not what was hashed, the fault word gets
 * SC_FNV_FAULT_CARRY and the verdict is 0 (nothing gated by it runs).  A mismatch is refused, never repaired: hash
 * again without carries to tell a corrupted payload from corrupted carries.  `carry_out` / `carry` are device memory
 * (or pinned host memory mapped for the device); the other arguments are those of the forms without carries. */
#define SC_FNV_FAULT_WAIT 1u    /* a look-back wait ran out (the launch still ended) */
#define SC_FNV_FAULT_CARRY 2u   /* a check given carries: a workgroup did not end with the carry after it */
uint64_t sc_fnv1a64_carry_bytes(uint64_t bytes);
int sc_fnv1a64_carry_async(const void* data, uint64_t bytes, uint64_t seed, uint64_t* out, uint32_t* fault,
                           uint8_t* carry_out, void* workspace, uint64_t workspace_bytes, void* stream);
int sc_fnv1a64_check_carried_async(const void* data, uint64_t bytes, uint64_t seed, uint64_t expected,
                                   const uint8_t* carry, uint64_t* out, uint32_t* verdict, uint32_t* fault,
                                   void* workspace, uint64_t workspace_bytes, void* stream);
int sc_hash_map_launch_carry(const sc_hash_map* map, uint64_t seed, uint64_t* out, uint32_t* fault, uint8_t* carry_out,
                             void* workspace, uint64_t workspace_bytes, void* stream);
/* A read map only (sc_hash_map_create_read: a payload hashed where its segments hold it). */
int sc_hash_map_check_carried_async(const sc_hash_map* map, uint64_t seed, uint64_t expected, const uint8_t* carry,
                                    uint64_t* out, uint32_t* verdict, uint32_t* fault, void* workspace,
                                    uint64_t workspace_bytes, void* stream);
int sc_hash_map_destroy(sc_hash_map* map);
/* The bound on each of the hash kernel's look-back waits, in reads of its window (0 restores the default, 65536, about
 * 0.2 s).  No counterpart in the reference: a workgroup only waits on workgroups that are running or done, so a
 * correct launch never reaches the bound; tests lower it to force a wait to run out, which must set the fault word of
 * every form and fail the verdict of sc_fnv1a64_check_async (the launch still ends, and the hash is not to be used).
 * SC_FNV_FORCE_FAULT makes every wait run out at once (any input past the first workgroup's 64 KiB then faults, which
 * makes the failure paths of the callers testable deterministically).  Applies to launches enqueued after the call,
 * in this process. */
#define SC_FNV_FORCE_FAULT 0xFFFFFFFFu
int sc_fnv1a64_set_spin_limit(uint32_t reads);

/* ---- runtime plumbing the C++ host layer calls instead of HIP ---------------------------------------------------- */

/* Number of visible HIP devices (0 and SC_EHIP when the runtime finds none). */
int sc_device_count(int* count);
/* The calling thread's current device, and making one current (hipGetDevice / hipSetDevice): what a layer-split
 * caller's OnDevice scope (include/strata/core/on_device.hpp:10-20) needs. */
int sc_get_device(int* device);
int sc_set_device(int device);
int sc_device_alloc(void** ptr, uint64_t bytes);
int sc_device_free(void* ptr);
/* Pinned host memory (hipHostMalloc): the park pool. */
int sc_host_alloc(void** ptr, uint64_t bytes);
int sc_host_free(void* ptr);
/* *mapped = 1 when [host, host + bytes) is pinned host memory mapped for the device (its first and last byte in one
 * mapping), else 0: what a paged slot's park or resume checks before its kernel touches the image. */
int sc_host_range_mapped(const void* host, uint64_t bytes, int32_t* mapped);
/* hipMemcpyAsync(hipMemcpyDefault) on `stream`. */
int sc_copy_async(void* dst, const void* src, uint64_t bytes, void* stream);
/* A device-side fill of `bytes` bytes with `value` by a small kernel (never a memset node). */
int sc_fill_bytes_async(void* dst, uint8_t value, uint64_t bytes, void* stream);
int sc_stream_create(void** stream);     /* non-blocking, default priority */
int sc_stream_destroy(void* stream);
int sc_stream_sync(void* stream);
int sc_device_sync(void);
int sc_event_create(void** event);
int sc_event_destroy(void* event);
int sc_event_record(void* event, void* stream);
int sc_event_sync(void* event);
int sc_event_elapsed_ms(void* start, void* end, float* ms);
/* The stream waits for the event (hipStreamWaitEvent). */
int sc_stream_wait_event(void* stream, void* event);

/* Host-link probe: pinned `bytes` x `iters` hipMemcpyAsync per direction, after one warm-up copy; the method of
 * probe_pcie_h2d_gbps (src/program/generate.cpp:1133-1161) applied to both directions. */
int sc_probe_link(uint64_t bytes, int iters, double* h2d_gbps, double* d2h_gbps);

/* A device-to-device copy by a shader kernel (16-byte vectors when both pointers share their alignment modulo 16), for
 * sources the runtime's own copy might hand to a copy engine (memory of another process mapped by a handle). */
int sc_copy_device_async(void* dst, const void* src, uint64_t bytes, void* stream);

/* ---- same-GPU hand-off between processes (hipIpcMemHandle) --------------------------------------------------------
 *
 * No counterpart in the reference: its prefill and decode instances hand a payload over only through the tmpfs arena
 * (include/strata/core/handoff.hpp:432-551), through host memory and the host link twice.  When both instances run on
 * one GPU the payload can stay in HBM: the exporter (prefill) allocates device segments once, exports a memory handle
 * for each, and stages every payload into them with one device copy; the importer (decode) opens the handles once and
 * copies the payload out into its own buffer with one device copy, after which the exporter may reuse the segments.
 * Which payload is in the segments, and when the importer is done with it, travel on the caller's own channel (a
 * socket line, or an arena slot).  Every segment is its own allocation of at most SC_IPC_MAX_SEGMENT bytes. */
#define SC_IPC_HANDLE_BYTES 64
#define SC_IPC_MAX_SEGMENT (1ull << 30)
#define SC_IPC_MAX_SEGMENTS 64
typedef struct sc_ipc_segment {
    uint8_t handle[SC_IPC_HANDLE_BYTES];   /* hipIpcMemHandle_t of the segment's allocation */
    uint64_t bytes;                        /* the segment's size */
} sc_ipc_segment;
typedef struct sc_ipc_export sc_ipc_export;
typedef struct sc_ipc_import sc_ipc_import;

/* Segments of `segment_bytes` (a multiple of 4 KiB, at most SC_IPC_MAX_SEGMENT; the last one holds the remainder)
 * covering `capacity` bytes, on the current device, each exported. */
int sc_ipc_export_create(uint64_t capacity, uint64_t segment_bytes, sc_ipc_export** out);
int32_t sc_ipc_export_count(const sc_ipc_export* ex);
/* The segments' handles and sizes, in payload order (`max_segments` entries of room). */
int sc_ipc_export_segments(const sc_ipc_export* ex, sc_ipc_segment* segments, int32_t max_segments);
/* Stage `bytes` of device memory into the segments, on `stream` (ordered after the work already on it). */
int sc_ipc_export_stage(sc_ipc_export* ex, const void* device_payload, uint64_t bytes, void* stream);
int sc_ipc_export_destroy(sc_ipc_export* ex);

/* Map another process's segments into this one (refused, before any handle is opened, when a segment is larger than
 * SC_IPC_MAX_SEGMENT or there are more than SC_IPC_MAX_SEGMENTS). */
int sc_ipc_import_open(const sc_ipc_segment* segments, int32_t n_segments, sc_ipc_import** out);
/* Copy the first `bytes` of the segments into `device_dst`, on `stream`. */
int sc_ipc_import_fetch(sc_ipc_import* im, void* device_dst, uint64_t bytes, void* stream);
/* The zero-copy form of the hand-off: the segments' device addresses in payload order (`ptr`, room for `max_segments`)
 * and the size of every segment but the last, which is an sc_segments over them, for sc_wire_encode_segments_async
 * on the exporter's side and sc_wire_decoder_open_segments on the importer's.  The encode then writes the payload
 * straight into the exported segments and the mount hashes and scatters it straight out of the imported ones: neither
 * sc_ipc_export_stage nor sc_ipc_import_fetch runs.  (The hash needs segment_bytes to be a multiple of 64 KiB, as
 * SC_IPC_MAX_SEGMENT is.) */
int sc_ipc_export_layout(const sc_ipc_export* ex, void** ptr, int32_t max_segments, int32_t* n, uint64_t* segment_bytes);
int sc_ipc_import_layout(const sc_ipc_import* im, void** ptr, int32_t max_segments, int32_t* n, uint64_t* segment_bytes);
/* Unmap the segments (before the exporter frees them). */
int sc_ipc_import_close(sc_ipc_import* im);

/* ---- synthetic inputs (bench and tests; not on the handoff path) ---------------------------------------------- */

/* Counter-based fills, bit-identical to the host generator of the test oracle:
 *   element i of stream s under seed: u64 = mix(seed, s, i) (SplitMix64 finaliser, see the source);
 *   uniform f16:  u = (u64 >> 40) * 2^-24;  x = lo + (hi - lo) * u  in f32, then RNE to f16;
 *   normal f32:   (sum of twelve 24-bit uniforms) - 6, an Irwin-Hall(12) value with mean 0 and variance 1,
 *                 formed in integers so host and device produce the same bits. */
int sc_fill_uniform_f16(uint16_t* dst, uint64_t n, float lo, float hi, uint64_t seed, uint64_t stream_id,
                        void* stream);
int sc_fill_uniform_f32(float* dst, uint64_t n, float lo, float hi, uint64_t seed, uint64_t stream_id,
                        void* stream);
int sc_fill_normal_f32(float* dst, uint64_t n, uint64_t seed, uint64_t stream_id, void* stream);

/* A synthetic decode step for overlap measurements: every workgroup reads its share of `n_bytes` bytes of K/V
 * at `kv` and folds them into one u32 per workgroup in `sink` (so the reads cannot be elided).  It stands in
 * for the attention reading the slot that keeps decoding while others park or resume. */
int sc_decode_probe(const void* kv, uint64_t n_bytes, uint32_t* sink, int64_t workgroups, void* stream);
/* Long work that always ends: one wave holds `stream` for `microseconds` (at most 2 s) of the device's constant-rate
 * wall clock.  Queued ahead of a transfer, it shows that event-gated work on another stream waits for that transfer. */
int sc_delay_async(uint32_t microseconds, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* SC_HANDOFF_H */

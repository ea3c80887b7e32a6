/* sc_wire.h - a C-ABI over the device hand-off payload path of libsc_core.so.
 *
 * The C++ engine interface is strata/core/conversation_wire.hpp (the reference's codec API) and
 * strata/core/conversation_wire_device.hpp (payloads written from and mounted into a decode slot on the device).
 * These entry points expose the device path to callers that bind C (tests, the bench, a Python or cgo host): plain
 * pointers and sizes, an int status (SC_OK == 0, the codes of sc_handoff.h) and the message of the last failure in
 * sc_wire_last_error().  Every refusal happens before anything is written to the slot.
 *
 * The payload is the reference's wire format (include/strata/core/conversation_wire.hpp:24-81), byte for byte: a
 * payload written here decodes with conversation_wire_decode, and a reference payload of a slot's f16 K/V + GDN rows
 * mounts here.
 */
#ifndef SC_WIRE_H
#define SC_WIRE_H

#include <stddef.h>
#include <stdint.h>

#include "sc_handoff.h"

#ifdef __cplusplus
extern "C" {
#endif

/* The host side of the conversation a device payload carries: the SavedConversation fields that are not the slot's
 * K/V and GDN rows (include/strata/core/conversation_cache.hpp:51-162).  Arrays are host memory, read during
 * sc_wire_encoder_create only. */
typedef struct sc_wire_live {
    int64_t geometry[18];          /* SavedConversation::geometry */
    int64_t layer_lo, layer_hi;
    int32_t cvec;
    int32_t draft_record;          /* 1: an empty K/V record follows the slot's layers (the draft layer's place) */
    int64_t idx_dim;               /* the K/V records' idx_dim */
    const int32_t* ids;            /* the live checkpoint's token ids; n_ids must equal the slot's token count */
    int64_t n_ids;
    const int64_t* img_start;      /* the live checkpoint's image keys */
    const uint64_t* img_hash;
    int64_t n_imgs;
    uint64_t used;
    const uint8_t* small[4];       /* ple, tails, dead, block_pos (host bytes, may be NULL when empty) */
    uint64_t small_bytes[4];
} sc_wire_live;

/* One later stage of a layer split (ConversationStageSnapshot, include/strata/core/conversation_cache.hpp): its own f16
 * decode slot, laid out by its own geometry (the QSA layers and GDN rows the stage owns; identity page tables), its
 * layer range, and - when encoding - its running state's small host buffers (the part's ids are the live ids). */
typedef struct sc_wire_stage {
    sc_geometry geometry;
    sc_decode_slot slot;
    int64_t layer_lo, layer_hi;
    const uint8_t* small[4];       /* ple, tails, dead, block_pos (host bytes, may be NULL when empty; encode only) */
    uint64_t small_bytes[4];
} sc_wire_stage;

typedef struct sc_wire_encoder sc_wire_encoder;
typedef struct sc_wire_decoder sc_wire_decoder;

/* The message of the last failure on this thread. */
const char* sc_wire_last_error(void);

/* Lays out the payload of `live` carrying the slot's first `tokens` tokens of f16 K/V (through its page tables) and its
 * GDN rows.  Replaces conversation_wire_plan (src/core/conversation_wire.cpp:988-1004) for slot-resident state. */
int sc_wire_encoder_create(const sc_geometry* g, const sc_decode_slot* slot, int64_t tokens, const sc_wire_live* live,
                           uint64_t geom_hash, uint64_t pack_hash, sc_wire_encoder** out);
/* The same with a layer split (the reference's conversation_snapshot_save, src/core/conversation_state.cpp:397-413):
 * `slot` holds the main session's layers, each of `stages` a later stage's, and the payload carries one stage part
 * per stage, in order, its K/V records and GDN rows gathered from the stage's slot by a launch of its own. */
int sc_wire_encoder_create_split(const sc_geometry* g, const sc_decode_slot* slot, int64_t tokens,
                                 const sc_wire_live* live, const sc_wire_stage* stages, int32_t n_stages,
                                 uint64_t geom_hash, uint64_t pack_hash, sc_wire_encoder** out);
/* The same for a slot in any K/V format (sc_slot_layers, include/sc_handoff.h): its layers become K/V records of
 * slot->format carrying data, int8 scales and, with slot->with_index, the indexer's pooled rows, all gathered from the
 * slot's identity pools by one launch (conversation_kv_save's five buffers, src/core/conversation_snapshot.cpp:69-78). */
int sc_wire_encoder_create_layers(const sc_geometry* g, const sc_slot_layers* slot, int64_t tokens,
                                  const sc_wire_live* live, uint64_t geom_hash, uint64_t pack_hash,
                                  sc_wire_encoder** out);
/* The payload's total size (WirePlan::total_bytes) and where its blob pool starts. */
uint64_t sc_wire_encoder_bytes(const sc_wire_encoder* e);
uint64_t sc_wire_encoder_pool_offset(const sc_wire_encoder* e);
/* Enqueues the encode on `stream` into 16-byte aligned device memory `payload`: one kernel that gathers the pool's
 * blobs from the slot, and the head and small host blobs from their device copy (staged once by
 * sc_wire_encoder_create), and hashes the whole payload as it writes it (sc_hash_map_launch: the slot is read once and
 * the payload never re-read).  With `gathered` (a hipEvent_t) the gather runs first on its own,
 * the event is recorded when every payload byte is in place, then the hash: a park on another stream can wait on the
 * event and overlap the hash.  Replaces conversation_wire_encode's walk and byte-serial hash
 * (src/core/conversation_wire.cpp:400-480, 1006-1025). */
int sc_wire_encode_async(sc_wire_encoder* e, void* payload, uint64_t capacity, void* stream, void* gathered);
/* The encode into a payload held in segments (`into`, sc_handoff.h: the same-GPU hand-off's exported segments, each at
 * most SC_IPC_MAX_SEGMENT bytes, segment_bytes a multiple of 64 KiB): the head, the small blobs and the slot's blobs
 * written into them by the fused gather + hash, cut wherever a segment ends.  The bytes are
 * exactly sc_wire_encode_async's, and no contiguous copy of the payload exists at any point. */
int sc_wire_encode_segments_async(sc_wire_encoder* e, const sc_segments* into, void* stream);
/* The payload hash of the last encode (waits for it): WireEncoded::payload_hash.  SC_ETIMEOUT, and no hash, when the
 * device hash did not complete (a bounded wait of its kernel ran out, sc_fnv1a64_async): encode again. */
int sc_wire_encoder_hash(sc_wire_encoder* e, uint64_t* hash);
/* Later encodes also write the payload's carries at `carry` (device memory of sc_fnv1a64_carry_bytes(
 * sc_wire_encoder_bytes(e)) bytes, sc_handoff.h): the low byte of the running payload hash after every 64 KiB, from the
 * same launch.  A consumer that receives them with the payload checks its hash without the look-back across the
 * payload (sc_wire_decoder_set_carry).  NULL stops writing them.  No counterpart in the reference (its hash is the
 * byte-serial loop). */
int sc_wire_encoder_set_carry(sc_wire_encoder* e, void* carry);
int sc_wire_encoder_destroy(sc_wire_encoder* e);

/* Reads and checks the head of a device payload against the slot: magic, version, flags, sizes, every record, the
 * geometry (when `geometry` is not NULL), the identity hashes (when check_identity), and that the first K/V records
 * are the slot's f16 layers.  Replaces the checks of conversation_wire_decode (src/core/conversation_wire.cpp:
 * 560-880) for a payload bound for a slot. */
int sc_wire_decoder_open(const void* payload, uint64_t bytes, const sc_geometry* g, const sc_decode_slot* slot,
                         const int64_t* geometry, uint64_t geom_hash, uint64_t pack_hash, int32_t check_identity,
                         uint64_t payload_hash, int32_t check_hash, sc_wire_decoder** out);
/* The same for a layer-split payload (the reference's conversation_snapshot_restore of stage parts,
 * src/core/conversation_state.cpp:497-509): exactly n_stages stage parts, each with its stage's layer range and the
 * shape of its slot; the restore scatters every part into its stage's slot, gated by the same device hash check as the
 * main slot (all or nothing). */
int sc_wire_decoder_open_split(const void* payload, uint64_t bytes, const sc_geometry* g, const sc_decode_slot* slot,
                               const sc_wire_stage* stages, int32_t n_stages, const int64_t* geometry,
                               uint64_t geom_hash, uint64_t pack_hash, int32_t check_identity, uint64_t payload_hash,
                               int32_t check_hash, sc_wire_decoder** out);
/* The same for a slot in any K/V format: the first K/V records must be the slot's layers in slot->format, with the
 * indexer's rows exactly when slot->with_index. */
int sc_wire_decoder_open_layers(const void* payload, uint64_t bytes, const sc_geometry* g, const sc_slot_layers* slot,
                                const int64_t* geometry, uint64_t geom_hash, uint64_t pack_hash, int32_t check_identity,
                                uint64_t payload_hash, int32_t check_hash, sc_wire_decoder** out);
/* sc_wire_decoder_open / _open_layers for a payload held in segments (another process's exported segments, imported
 * with sc_ipc_import_open): the head is read from them, the restore hashes the payload where it lies (one launch) and
 * scatters every blob straight from them, so nothing is fetched into a contiguous buffer first. */
int sc_wire_decoder_open_segments(const sc_segments* from, uint64_t bytes, const sc_geometry* g,
                                  const sc_decode_slot* slot, const int64_t* geometry, uint64_t geom_hash,
                                  uint64_t pack_hash, int32_t check_identity, uint64_t payload_hash, int32_t check_hash,
                                  sc_wire_decoder** out);
int sc_wire_decoder_open_layers_segments(const sc_segments* from, uint64_t bytes, const sc_geometry* g,
                                         const sc_slot_layers* slot, const int64_t* geometry, uint64_t geom_hash,
                                         uint64_t pack_hash, int32_t check_identity, uint64_t payload_hash,
                                         int32_t check_hash, sc_wire_decoder** out);
/* Tokens the payload carries (its live token count). */
int64_t sc_wire_decoder_tokens(const sc_wire_decoder* d);
/* Verifies the payload hash on the device (when asked), then scatters the K/V and GDN rows into the slot in one launch
 * and copies the host-side blobs out.  Synchronous; on a refusal the slot is untouched (the reference's "invalid: no
 * write", include/strata/core/conversation_snapshot.hpp:103-108): SC_EINVAL for a hash that differs, SC_ETIMEOUT for a
 * device hash that did not complete (its verdict gated every scatter off, as for a mismatch). */
int sc_wire_decoder_restore(sc_wire_decoder* d, void* stream);
/* Opens `d` again for the next payload, with the geometry, slot, identity checks and kind of payload place it was
 * opened with (not for a decoder of a layer-split payload): `payload` is the next payload's device memory, or NULL for
 * a decoder opened on segments (the next payload lies in the same segments), `bytes` its size and `payload_hash` its
 * expected hash.  The decoder keeps its staging, streams, events and hash words, and keeps its scatter plan when the
 * payload's place, the slot and the blob offsets are unchanged (the next hand-off of a same-shaped conversation), so
 * an engine that holds one decoder per slot opens each such hand-off without allocating device memory.  Carries set for the previous
 * payload are dropped.  A refusal leaves the decoder to be opened again or destroyed.  No counterpart in the reference
 * (its decoder is a function over a host buffer). */
int sc_wire_decoder_reopen(sc_wire_decoder* d, const void* payload, uint64_t bytes, uint64_t payload_hash);
/* The payload's carries as its encoder wrote them (device memory; sc_wire_encoder_set_carry), for the next restore of
 * this opened decoder: the payload hash is then checked starting every 64 KiB from its carry, with the same verdict -
 * a payload or carries that are not what was hashed are refused with SC_EINVAL and nothing is mounted.  NULL checks
 * without them.  No counterpart in the reference. */
int sc_wire_decoder_set_carry(sc_wire_decoder* d, const void* carry);
/* After a restore: the live checkpoint's ids (n written to *n; needs cap >= tokens) and its small buffers
 * (which: 0 ple, 1 tails, 2 dead, 3 block_pos). */
int sc_wire_decoder_live_ids(const sc_wire_decoder* d, int32_t* ids, int64_t cap, int64_t* n);
int sc_wire_decoder_small(const sc_wire_decoder* d, int32_t which, uint8_t* dst, uint64_t cap, uint64_t* n);
/* After a restore of a layer-split payload: stage part `stage`'s small buffers (which as above). */
int sc_wire_decoder_stage_small(const sc_wire_decoder* d, int32_t stage, int32_t which, uint8_t* dst, uint64_t cap,
                                uint64_t* n);
int sc_wire_decoder_destroy(sc_wire_decoder* d);

#ifdef __cplusplus
}
#endif
#endif /* SC_WIRE_H */

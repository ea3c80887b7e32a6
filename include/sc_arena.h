/* sc_arena.h - a C-ABI over the hand-off arena and its device movers in libsc_core.so.
 *
 * The C++ engine interface is strata/core/handoff.hpp (the reference's HandoffArena, include/strata/core/handoff.hpp:
 * 432-551, same API and same file format) and strata/core/handoff_device.hpp (HBM <-> slot movers).  These entry points
 * expose both to callers that bind C (tests, the bench, a Python or cgo host): plain pointers and sizes, an int status
 * (SC_OK == 0, the codes of sc_handoff.h) and the message of the last failure in sc_arena_last_error().
 */
#ifndef SC_ARENA_H
#define SC_ARENA_H

#include <stddef.h>
#include <stdint.h>

#include "sc_handoff.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct sc_arena sc_arena;
typedef struct sc_mover sc_mover;

/* Status codes beyond sc_handoff.h's. */
enum {
    SC_EBUSY = 5,    /* no free slot of the tier or above: temporary, queue the job; nothing was written */
    SC_ESTALE = 6    /* the payload was copied to the device and then failed its re-check (slot released or
                        reclaimed meanwhile, or the hash differs): the destination holds those bytes, do not mount */
};

/* A claimed slot (HandoffClaim, include/strata/core/handoff.hpp:384-391). */
typedef struct sc_arena_claim {
    int32_t index;
    uint32_t tier;
    uint64_t base, payload_off, capacity, nonce;
} sc_arena_claim;

/* One slot header as read (HandoffSlotInfo, include/strata/core/handoff.hpp:369-381). */
typedef struct sc_arena_slot {
    int32_t index;
    uint32_t state, flags, tier;
    uint64_t base, capacity, owner_pid, owner_start, nonce, client_id, request_id, pack_hash, geom_hash;
    uint64_t tokens, payload_bytes, payload_hash, claimed_ms, published_ms, seq;
} sc_arena_slot;

/* The message of the last failure on this thread. */
const char* sc_arena_last_error(void);

/* handoff_size_arena (src/core/handoff.cpp:164-231): per tier its slot bytes and group offset, and the file size.
 * `describe` (may be NULL) receives the start-up figure, NUL-terminated, truncated to describe_cap bytes. */
int sc_arena_size(int32_t n_tiers, const uint64_t* tier_tokens, const uint64_t* tier_slots, const uint64_t* priced,
                  uint64_t* slot_bytes, uint64_t* slot_off, uint64_t* arena_bytes, char* describe, uint64_t describe_cap);
/* handoff_geom_hash (src/core/handoff.cpp:132-138) of the 18 geometry words and a split spec. */
uint64_t sc_arena_geom_hash(const int64_t* geometry18, const char* split_spec);

/* HandoffArena::open_writer (src/core/handoff.cpp:453-622) with the sizing of the tier table; `reserve` != 0 also
 * commits every page of the file and maps it (HandoffArena::reserve).  `lease_ms` < 0 keeps the default lease. */
int sc_arena_open_writer(const char* path, int32_t n_tiers, const uint64_t* tier_tokens, const uint64_t* tier_slots,
                         const uint64_t* priced, uint64_t pack_hash, uint64_t geom_hash, int32_t reserve,
                         int64_t lease_ms, sc_arena** out);
/* HandoffArena::open_reader (src/core/handoff.cpp:978-1018). */
int sc_arena_open_reader(const char* path, uint64_t pack_hash, uint64_t geom_hash, sc_arena** out);
int sc_arena_close(sc_arena* arena);
/* HandoffArena::reserve: a writer commits every page of the file and maps it populated; a reader maps it read-only
 * populated (this library's addition, for the device movers; a start-up cost paid once per arena). */
int sc_arena_reserve(sc_arena* arena);

/* HandoffArena::claim / write_payload / publish / release / abort_claim / cancel (src/core/handoff.cpp:729-976).
 * sc_arena_claim_slot answers SC_EBUSY (not an error: queue the job) when no slot of the tier or above is free. */
int sc_arena_claim_slot(sc_arena* arena, uint32_t tier, uint64_t client_id, uint64_t request_id, sc_arena_claim* out);
int sc_arena_write(sc_arena* arena, const sc_arena_claim* claim, uint64_t offset, const void* host, uint64_t bytes);
int sc_arena_publish(sc_arena* arena, const sc_arena_claim* claim, uint64_t tokens, uint64_t payload_bytes,
                     uint64_t payload_hash);
int sc_arena_release(sc_arena* arena, int32_t index, uint64_t nonce);
int sc_arena_abort(sc_arena* arena, int32_t index, uint64_t nonce);
int sc_arena_cancel(sc_arena* arena, int32_t index, uint64_t nonce);
/* HandoffArena::slot_info (src/core/handoff.cpp:1020-1051). */
int sc_arena_slot_info(sc_arena* arena, int32_t index, sc_arena_slot* out);
/* The reference's reader path on the host: read_slot (every check), a copy of the payload into `host` (room for
 * `capacity` bytes) and, with `check_hash`, HandoffArena::payload_hash_of against the slot's record
 * (src/core/handoff.cpp:1053-1136).  `out` (may be NULL) receives the slot as read. */
int sc_arena_read_host(sc_arena* arena, int32_t index, uint64_t nonce, uint64_t client_id, void* host, uint64_t capacity,
                       int32_t check_hash, sc_arena_slot* out);

/* ---- HBM <-> slot (strata/core/handoff_device.hpp); no counterpart in the reference, whose payloads reach the
 * arena from host memory ---- */

/* Pinned staging of `depth` buffers of `chunk_bytes`, `threads` host copy threads, on the current device. */
int sc_mover_create(uint64_t chunk_bytes, int32_t depth, int32_t threads, sc_mover** out);
int sc_mover_destroy(sc_mover* mover);
/* `bytes` of device memory into the claimed slot (after the work on `stream`); with `hash` != NULL also the payload's
 * FNV-1a, computed on the device.  SC_ETIMEOUT when that hash did not complete (a bounded wait of its kernel ran out,
 * sc_fnv1a64_async): the slot holds the bytes, no hash is returned, and nothing is published. */
int sc_mover_write(sc_mover* mover, sc_arena* arena, const sc_arena_claim* claim, const void* device_src,
                   uint64_t bytes, void* stream, uint64_t* hash);
/* sc_mover_write with the device hash, then sc_arena_publish. */
int sc_mover_publish(sc_mover* mover, sc_arena* arena, const sc_arena_claim* claim, const void* device_src,
                     uint64_t bytes, uint64_t tokens, void* stream);
/* A READY slot (every check of read_slot) into device memory, re-checked after the copy, and with `verify` its
 * FNV-1a on the device against the slot's record.  Nothing is written to `device_dst` when the slot is refused before
 * the copy.  SC_ETIMEOUT when the device hash did not complete: the destination holds the bytes, unverified, and is
 * not to be mounted. */
int sc_mover_read(sc_mover* mover, sc_arena* arena, int32_t index, uint64_t nonce, uint64_t client_id, void* device_dst,
                  uint64_t capacity, void* stream, int32_t verify, sc_arena_slot* out);
/* The last transfer's host wall-clock time, the part spent on the hash (a verified read), in host copies between
 * staging and the slot, and waiting for DMA.  Any output may be NULL. */
int sc_mover_last(const sc_mover* mover, uint64_t* bytes, double* ms, double* hash_ms, double* copy_ms, double* wait_ms);

#ifdef __cplusplus
}
#endif

#endif /* SC_ARENA_H */

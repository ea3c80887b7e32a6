// conversation_wire.cpp - the hand-off payload codec (format: include/strata/core/conversation_wire.hpp).
//
// Encoding is three steps over one fixed traversal order (K/V records, live, retained checkpoints, stage parts):
//   1. collect the pool - every non-empty buffer in BLOBREF order with its 64-aligned offset inside the pool;
//   2. size the record stream in closed form, which fixes where the pool starts;
//   3. write header, records, padding and pool through a bounded staging buffer, hashing every byte as it leaves.
// The writer re-derives each BLOBREF from the collected list and checks the sizes agree, so the two walks cannot drift
// apart silently.  Decoding validates each field before it is used to size anything, builds into a local image and
// moves it out only when the whole payload parsed.
#include "strata/core/conversation_wire.hpp"

#include "wire_internal.hpp"

#include <algorithm>
#include <cerrno>
#include <cstdio>
#include <cstring>
#include <limits>

#include <unistd.h>

namespace strata::core {

uint64_t fnv1a64(const uint8_t* data, uint64_t bytes, uint64_t seed) {
    uint64_t h = seed;
    for (uint64_t i = 0; i < bytes; ++i) {
        h ^= data[i];
        h *= 1099511628211ull;
    }
    return h;
}

namespace {

constexpr uint64_t kKvBodyBytes = 8 + 6 * 8 + 5 * 16;   // format + pad, six extents, five BLOBREFs = 136
constexpr uint64_t kStagingBytes = 64 * 1024;
constexpr uint64_t kU64Max = std::numeric_limits<uint64_t>::max();

bool refuse(std::string& error, const std::string& why) {
    error = "conversation wire: " + why;
    return false;
}
std::string hex64(uint64_t v) {
    char b[24];
    std::snprintf(b, sizeof b, "%016llx", static_cast<unsigned long long>(v));
    return b;
}
std::string num(uint64_t v) { return std::to_string(v); }
uint64_t up64(uint64_t n) { return (n + 63) & ~uint64_t(63); }

// The wire format is little-endian: on a little-endian host an array of 32-bit ids is its own wire image, moved with
// one copy (a byte loop per id, which the compiler cannot merge through the byte buffer, took 0.3-0.5 ms for a 128K
// checkpoint each way).
constexpr bool kHostLittleEndian = __BYTE_ORDER__ == __ORDER_LITTLE_ENDIAN__;

template <class T> void put_le(uint8_t* p, T value) {
    const uint64_t v = static_cast<uint64_t>(value);
    for (size_t i = 0; i < sizeof(T); ++i) p[i] = static_cast<uint8_t>(v >> (8 * i));
}
template <class T> T get_le(const uint8_t* p) {
    uint64_t v = 0;
    for (size_t i = 0; i < sizeof(T); ++i) v |= uint64_t(p[i]) << (8 * i);
    return static_cast<T>(v);
}

// Checked arithmetic for sizes derived from an image (a corrupt in-memory image must not wrap a size).
struct Size {
    uint64_t v = 0;
    bool ok = true;
    Size& add(uint64_t x) {
        if (x > kU64Max - v) ok = false; else v += x;
        return *this;
    }
    Size& add_mul(uint64_t a, uint64_t b) {
        if (a && b > kU64Max / a) ok = false; else add(a * b);
        return *this;
    }
};

uint64_t ids_pad(uint64_t n_ids) { return (n_ids & 1) ? 4 : 0; }   // the id array is padded to 8 bytes

// Body bytes of a CHECKPOINT record: ids, image keys, five BLOBREFs, `used`, the part count, the nested parts.
bool checkpoint_body(const ConversationCheckpoint& c, int depth, int max_depth, uint64_t& out, std::string& error) {
    if (depth > max_depth) return refuse(error, "checkpoint stage_parts nesting exceeds the bound");
    Size s;
    s.add(8).add_mul(c.ids.size(), 4).add(ids_pad(c.ids.size())).add(8).add_mul(c.imgs.size(), 16).add(5 * 16 + 16);
    for (const ConversationCheckpoint& part : c.stage_parts) {
        uint64_t sub = 0;
        if (!checkpoint_body(part, depth + 1, max_depth, sub, error)) return false;
        s.add(kWireRecordHeaderBytes).add(sub);
    }
    if (!s.ok) return refuse(error, "byte count overflow");
    out = s.v;
    return true;
}

bool stage_body(const ConversationStageSnapshot& st, int max_depth, uint64_t& out, std::string& error) {
    uint64_t cp = 0;
    if (!checkpoint_body(st.state, 0, max_depth, cp, error)) return false;
    Size s;
    s.add(16).add(kWireRecordHeaderBytes).add(cp).add(8).add_mul(st.kv.size(), kWireRecordHeaderBytes + kKvBodyBytes);
    if (!s.ok) return refuse(error, "byte count overflow");
    out = s.v;
    return true;
}

// One pool entry: a ConversationKv buffer (segmented) or a checkpoint vector (contiguous).
struct PoolEntry {
    const ConversationBuffer* buf = nullptr;
    const std::vector<uint8_t>* vec = nullptr;
    uint64_t bytes = 0;
    uint64_t rel = 0;   // offset inside the pool
};

// The traversal both passes share, as a visitor over (buffer | vector) in BLOBREF order.
template <class Fn> void each_checkpoint_buffer(const ConversationCheckpoint& c, Fn& fn) {
    for (const std::vector<uint8_t>* v : {&c.gdn, &c.ple, &c.tails, &c.dead, &c.block_pos}) fn(nullptr, v);
    for (const ConversationCheckpoint& part : c.stage_parts) each_checkpoint_buffer(part, fn);
}
template <class Fn> void each_kv_buffer(const ConversationKv& k, Fn& fn) {
    for (const ConversationBuffer* b : {&k.k, &k.v, &k.k_scale, &k.v_scale, &k.pooled}) fn(b, nullptr);
}
template <class Fn> void each_buffer(const SavedConversation& img, Fn&& fn) {
    for (const ConversationKv& k : img.kv) each_kv_buffer(k, fn);
    each_checkpoint_buffer(img.live, fn);
    for (const ConversationCheckpoint& c : img.checkpoints) each_checkpoint_buffer(c, fn);
    for (const ConversationStageSnapshot& st : img.stage_parts) {
        each_checkpoint_buffer(st.state, fn);
        for (const ConversationKv& k : st.kv) each_kv_buffer(k, fn);
    }
}

struct Layout {
    std::vector<PoolEntry> pool;
    uint64_t pool_used = 0;     // end of the last entry, pool-relative
    WirePlan plan;
    const detail::WireSizes* sizes = nullptr;   // buffers laid out at a given size whatever they hold

    uint64_t size_of(const void* who, uint64_t held) const {
        if (sizes)
            for (const auto& s : *sizes)
                if (s.first == who) return s.second;
        return held;
    }
};

bool lay_out(const SavedConversation& img, int max_depth, Layout& lay, std::string& error) {
    if (!img.live.stage_parts.empty())
        return refuse(error, "a parked image keeps its layer-split state in stage_parts, not in the live checkpoint");
    bool overflow = false;
    each_buffer(img, [&](const ConversationBuffer* b, const std::vector<uint8_t>* v) {
        const uint64_t n = b ? lay.size_of(b, b->size()) : lay.size_of(v, v->size());
        if (!n) return;
        const uint64_t at = up64(lay.pool_used);
        if (at < lay.pool_used || n > kU64Max - at) overflow = true;
        lay.pool.push_back(PoolEntry{b, v, n, at});
        lay.pool_used = at + n;
    });
    Size records;
    records.add_mul(img.kv.size(), kWireRecordHeaderBytes + kKvBodyBytes);
    uint64_t body = 0;
    if (!checkpoint_body(img.live, 0, max_depth, body, error)) return false;
    records.add(kWireRecordHeaderBytes).add(body);
    for (const ConversationCheckpoint& c : img.checkpoints) {
        if (!checkpoint_body(c, 0, max_depth, body, error)) return false;
        records.add(kWireRecordHeaderBytes).add(body);
    }
    for (const ConversationStageSnapshot& st : img.stage_parts) {
        if (!stage_body(st, max_depth, body, error)) return false;
        records.add(kWireRecordHeaderBytes).add(body);
    }
    records.add(kWireRecordHeaderBytes);   // END
    if (overflow || !records.ok || records.v > kU64Max - 2 * kWireHeaderRecordBytes) return refuse(error, "byte count overflow");
    WirePlan& p = lay.plan;
    p.body_bytes = records.v;
    p.blob_pool_off = up64(kWireHeaderRecordBytes + records.v);
    p.blob_pool_bytes = lay.pool.empty() ? 0 : up64(lay.pool_used);
    if (p.blob_pool_bytes > kU64Max - p.blob_pool_off) return refuse(error, "byte count overflow");
    p.total_bytes = p.blob_pool_off + p.blob_pool_bytes;
    p.n_kv = int64_t(img.kv.size());
    p.n_checkpoints = int64_t(img.checkpoints.size());
    p.n_stage_parts = int64_t(img.stage_parts.size());
    p.live_tokens = int64_t(img.live.ids.size());
    p.flags = uint16_t((img.cvec ? kWireFlagCvec : 0) | (img.stage_parts.empty() ? 0 : kWireFlagHasStageParts));
    p.blobs = lay.pool.size();
    return true;
}

// The write pass: bytes go through a bounded staging buffer into the sink, and every byte is hashed on its way out.
class Writer {
public:
    // `hashing` false: the bytes are not hashed as they are written (a head whose payload is hashed elsewhere, e.g. on
    // the device with the pool; the byte-serial hash was most of a 128K head's write time)
    Writer(WireSink& sink, const Layout& lay, std::string& error, bool hashing = true)
        : sink_(sink), lay_(lay), error_(error), hashing_(hashing) {
        staging_.reserve(kStagingBytes);
    }

    bool put(const void* p, uint64_t n) {
        const uint8_t* b = static_cast<const uint8_t*>(p);
        while (n) {
            if (staging_.size() == kStagingBytes && !flush()) return false;
            const uint64_t k = std::min<uint64_t>(n, kStagingBytes - staging_.size());
            staging_.insert(staging_.end(), b, b + k);
            b += k;
            n -= k;
        }
        return true;
    }
    bool u32(uint32_t v) { uint8_t b[4]; put_le(b, v); return put(b, 4); }
    bool u64(uint64_t v) { uint8_t b[8]; put_le(b, v); return put(b, 8); }
    bool zeros(uint64_t n) {
        static const uint8_t z[4096] = {};
        while (n) {
            const uint64_t k = std::min<uint64_t>(n, sizeof z);
            if (!put(z, k)) return false;
            n -= k;
        }
        return true;
    }
    // Each record starts a new sink write (the staged bytes before it go out first), so a sink sees the head as one
    // write per record, as the reference's encoder writes it (src/core/conversation_wire.cpp:293-396).
    bool record(uint32_t kind, uint64_t body) { return flush() && u32(kind) && u32(0) && u64(body); }
    // The BLOBREF of `who` (a buffer of the image): {bytes, absolute offset} of the next pool entry, or {0, 0}.
    bool blobref_of(const void* who, uint64_t held) { return blobref(lay_.size_of(who, held)); }
    // The next BLOBREF: {bytes, absolute offset} of the next pool entry, or {0, 0} for an empty buffer.
    bool blobref(uint64_t bytes) {
        if (!bytes) return u64(0) && u64(0);
        if (next_ >= lay_.pool.size() || lay_.pool[next_].bytes != bytes)
            return refuse(error_, "internal: the pool order changed between the layout and the write");
        return u64(bytes) && u64(lay_.plan.blob_pool_off + lay_.pool[next_++].rel);
    }
    // Large contiguous runs bypass the staging buffer (after flushing it) in pieces of at most kWireChunkBytes.
    bool bulk(const uint8_t* p, uint64_t n) {
        if (n < kStagingBytes) return put(p, n);
        if (!flush()) return false;
        while (n) {
            const uint64_t k = std::min<uint64_t>(n, kWireChunkBytes);
            if (!emit(p, k)) return false;
            p += k;
            n -= k;
        }
        return true;
    }
    // A ConversationBuffer's segment run goes to the sink as one write (after flushing the staging buffer), as the
    // reference hands each visited segment to its sink (src/core/conversation_wire.cpp:421-427): a 20 MiB buffer is
    // written as a 16 MiB and a 4 MiB write, straight from the segments' own memory.
    bool segment(const uint8_t* p, uint64_t n) {
        if (n < kStagingBytes) return put(p, n);
        return flush() && emit(p, n);
    }
    bool flush() {
        if (staging_.empty()) return true;
        const bool ok = emit(staging_.data(), staging_.size());
        staging_.clear();
        return ok;
    }
    uint64_t written() const { return written_; }
    uint64_t hash() const { return hash_; }
    size_t refs_written() const { return next_; }

private:
    bool emit(const uint8_t* p, uint64_t n) {
        if (hashing_) hash_ = fnv1a64(p, n, hash_);
        if (!sink_.write(p, size_t(n))) {
            std::string why = "the sink refused the payload at byte " + num(written_);
            const std::string sink_why = sink_.refusal();
            if (!sink_why.empty()) why += ": " + sink_why;
            return refuse(error_, why);
        }
        written_ += n;
        return true;
    }

    WireSink& sink_;
    const Layout& lay_;
    std::string& error_;
    std::vector<uint8_t> staging_;
    uint64_t written_ = 0;
    bool hashing_ = true;
    uint64_t hash_ = kWireHashSeed;
    size_t next_ = 0;
};

bool write_kv(Writer& w, const ConversationKv& k) {
    if (!w.record(kWireRecordKv, kKvBodyBytes) || !w.u32(uint32_t(int32_t(k.format))) || !w.u32(0)) return false;
    for (int64_t v : {k.cells, k.heads, k.head_dim, k.page_size, k.pooled_rows, k.idx_dim})
        if (!w.u64(uint64_t(v))) return false;
    for (const ConversationBuffer* b : {&k.k, &k.v, &k.k_scale, &k.v_scale, &k.pooled})
        if (!w.blobref_of(b, b->size())) return false;
    return true;
}

bool write_checkpoint(Writer& w, const ConversationCheckpoint& c, int depth, int max_depth, std::string& error) {
    uint64_t body = 0;
    if (!checkpoint_body(c, depth, max_depth, body, error)) return false;
    if (!w.record(kWireRecordCheckpoint, body) || !w.u64(c.ids.size())) return false;
    if constexpr (kHostLittleEndian) {
        if (!w.put(reinterpret_cast<const uint8_t*>(c.ids.data()), 4 * uint64_t(c.ids.size()))) return false;
    } else {
        uint8_t buf[4 * 1024];
        for (size_t i = 0; i < c.ids.size();) {
            const size_t n = std::min<size_t>(sizeof buf / 4, c.ids.size() - i);
            for (size_t j = 0; j < n; ++j) put_le(buf + 4 * j, uint32_t(c.ids[i + j]));
            if (!w.put(buf, 4 * n)) return false;
            i += n;
        }
    }
    if (!w.zeros(ids_pad(c.ids.size())) || !w.u64(c.imgs.size())) return false;
    for (const ConversationImageKey& key : c.imgs)
        if (!w.u64(uint64_t(key.start)) || !w.u64(key.hash)) return false;
    for (const std::vector<uint8_t>* v : {&c.gdn, &c.ple, &c.tails, &c.dead, &c.block_pos})
        if (!w.blobref_of(v, v->size())) return false;
    if (!w.u64(c.used) || !w.u64(c.stage_parts.size())) return false;
    for (const ConversationCheckpoint& part : c.stage_parts)
        if (!write_checkpoint(w, part, depth + 1, max_depth, error)) return false;
    return true;
}

bool write_payload(const SavedConversation& img, const WireIdentity& id, const Layout& lay, int max_depth, Writer& w,
                   std::string& error, bool head_only = false) {
    const WirePlan& p = lay.plan;
    uint8_t h[kWireHeaderRecordBytes] = {};
    put_le(h + 0, kWireMagic);
    put_le(h + 4, kWireFormatVersion);
    put_le(h + 6, p.flags);
    for (size_t i = 0; i < 18; ++i) put_le(h + 8 + 8 * i, uint64_t(img.geometry[i]));
    put_le(h + 152, uint64_t(img.layer_lo));
    put_le(h + 160, uint64_t(img.layer_hi));
    put_le(h + 168, uint64_t(p.n_kv));
    put_le(h + 176, uint64_t(p.n_checkpoints));
    put_le(h + 184, uint64_t(p.n_stage_parts));
    put_le(h + 192, uint64_t(p.live_tokens));
    put_le(h + 200, p.blob_pool_off);
    put_le(h + 208, p.blob_pool_bytes);
    put_le(h + 216, id.geom_hash);
    put_le(h + 224, id.pack_hash);
    put_le(h + 232, p.total_bytes);
    if (!w.put(h, sizeof h)) return false;
    for (const ConversationKv& k : img.kv)
        if (!write_kv(w, k)) return false;
    if (!write_checkpoint(w, img.live, 0, max_depth, error)) return false;
    for (const ConversationCheckpoint& c : img.checkpoints)
        if (!write_checkpoint(w, c, 0, max_depth, error)) return false;
    for (const ConversationStageSnapshot& st : img.stage_parts) {
        uint64_t body = 0;
        if (!stage_body(st, max_depth, body, error)) return false;
        if (!w.record(kWireRecordStage, body) || !w.u64(uint64_t(st.layer_lo)) || !w.u64(uint64_t(st.layer_hi)))
            return false;
        if (!write_checkpoint(w, st.state, 0, max_depth, error) || !w.u64(st.kv.size())) return false;
        for (const ConversationKv& k : st.kv)
            if (!write_kv(w, k)) return false;
    }
    if (!w.record(kWireRecordEnd, 0)) return false;
    if (w.refs_written() != lay.pool.size()) return refuse(error, "internal: not every pool entry was referenced");
    // zero pad to the pool, then the entries with zero gaps, then the pool's own tail pad
    uint64_t at = kWireHeaderRecordBytes + p.body_bytes;
    if (!w.zeros(p.blob_pool_off - at)) return false;
    if (head_only) return w.flush();
    uint64_t rel = 0;
    for (const PoolEntry& e : lay.pool) {
        if (!w.zeros(e.rel - rel)) return false;
        if (e.vec) {
            if (!w.bulk(e.vec->data(), e.bytes)) return false;
        } else {
            bool ok = true;
            e.buf->visit(0, size_t(e.bytes), [&](const uint8_t* q, size_t n, size_t) { return ok = w.segment(q, n); });
            if (!ok) return false;
        }
        rel = e.rel + e.bytes;
    }
    if (!w.zeros(p.blob_pool_bytes - rel) || !w.flush()) return false;
    if (w.written() != p.total_bytes) return refuse(error, "internal: the written bytes disagree with the plan");
    return true;
}

// ---- decode -----------------------------------------------------------------------------------------------------------

// A bounded cursor: every read checks the room left before it happens.
class Cursor {
public:
    Cursor(const WireSource& src, uint64_t begin, uint64_t end, std::string& error)
        : src_(src), pos_(begin), end_(end), error_(error) {}
    uint64_t pos() const { return pos_; }
    uint64_t room() const { return end_ - pos_; }
    bool bytes(uint8_t* dst, uint64_t n) {
        if (n > room()) return refuse(error_, "the payload is shorter than its records claim");
        if (n && !src_.read(dst, pos_, size_t(n))) return refuse(error_, "the source refused a read");
        pos_ += n;
        return true;
    }
    bool u32(uint32_t& v) { uint8_t b[4]; if (!bytes(b, 4)) return false; v = get_le<uint32_t>(b); return true; }
    bool u64(uint64_t& v) { uint8_t b[8]; if (!bytes(b, 8)) return false; v = get_le<uint64_t>(b); return true; }
    bool i64(int64_t& v) { uint64_t u = 0; if (!u64(u)) return false; v = int64_t(u); return true; }
    bool zeros(uint64_t n) {
        uint8_t b[64];
        while (n) {
            const uint64_t k = std::min<uint64_t>(n, sizeof b);
            if (!bytes(b, k)) return false;
            for (uint64_t i = 0; i < k; ++i)
                if (b[i]) return refuse(error_, "a reserved field is not zero");
            n -= k;
        }
        return true;
    }
    bool record_header(uint32_t& kind, uint32_t& flags, uint64_t& body) { return u32(kind) && u32(flags) && u64(body); }

private:
    const WireSource& src_;
    uint64_t pos_, end_;
    std::string& error_;
};

// A count read from the payload must be non-negative, under its structural cap, and fit the bytes left for it.
bool count_ok(int64_t n, int64_t cap, const char* what, uint64_t room, uint64_t element, std::string& error) {
    if (n < 0) return refuse(error, std::string(what) + " is negative");
    if (n > cap) return refuse(error, std::string(what) + " " + num(uint64_t(n)) + " exceeds its bound " + num(uint64_t(cap)));
    if (element && uint64_t(n) > room / element)
        return refuse(error, std::string(what) + " " + num(uint64_t(n)) + " does not fit the record's remaining bytes");
    return true;
}

WireHeaderRecord parse_header(const uint8_t* p) {
    WireHeaderRecord h{};
    h.magic = get_le<uint32_t>(p);
    h.fmt_version = get_le<uint16_t>(p + 4);
    h.flags = get_le<uint16_t>(p + 6);
    for (size_t i = 0; i < 18; ++i) h.geometry[i] = get_le<uint64_t>(p + 8 + 8 * i);
    h.layer_lo = get_le<uint64_t>(p + 152);
    h.layer_hi = get_le<uint64_t>(p + 160);
    h.n_kv = get_le<int64_t>(p + 168);
    h.n_checkpoints = get_le<int64_t>(p + 176);
    h.n_stage_parts = get_le<int64_t>(p + 184);
    h.live_tokens = get_le<int64_t>(p + 192);
    h.blob_pool_off = get_le<uint64_t>(p + 200);
    h.blob_pool_bytes = get_le<uint64_t>(p + 208);
    h.geom_hash = get_le<uint64_t>(p + 216);
    h.pack_hash = get_le<uint64_t>(p + 224);
    h.payload_bytes = get_le<uint64_t>(p + 232);
    h.payload_hash = get_le<uint64_t>(p + 240);
    h.reserved = get_le<uint64_t>(p + 248);
    return h;
}

class Parser {
public:
    Parser(const WireSource& src, const WireExpect& expect, std::string& error) : src_(src), expect_(expect), error_(error) {}
    /// Locate mode: blobs are validated and reported here, never read (the buffers stay empty), and the payload hash
    /// is left to whoever holds the bytes.
    void locate_into(std::vector<detail::WireBlobAt>* out) { located_ = out; }

    bool run(SavedConversation& out, WireDecoded& info) {
        if (!header(info) || !check_hash(info)) return false;
        Cursor c(src_, kWireHeaderRecordBytes, pool_begin_, error_);
        // Normally the image is built aside and moved out only on success.  In locate mode the blob addresses must
        // be those of the caller's image, so it is built in place (the caller discards it on a refusal).
        SavedConversation local;
        SavedConversation& img = located_ ? out : local;
        img = SavedConversation{};
        for (size_t i = 0; i < 18; ++i) img.geometry[i] = int64_t(h_.geometry[i]);
        img.layer_lo = int64_t(h_.layer_lo);
        img.layer_hi = int64_t(h_.layer_hi);
        img.cvec = (h_.flags & kWireFlagCvec) != 0;
        img.owner = kNoOwner;   // the receiver claims an image when it stores it, never from the wire
        img.kv.resize(size_t(h_.n_kv));
        for (ConversationKv& k : img.kv)
            if (!kv_record(c, k, "KV array")) return false;
        if (!checkpoint(c, img.live, 0)) return false;
        img.checkpoints.resize(size_t(h_.n_checkpoints));
        for (ConversationCheckpoint& cp : img.checkpoints)
            if (!checkpoint(c, cp, 0)) return false;
        img.stage_parts.resize(size_t(h_.n_stage_parts));
        for (ConversationStageSnapshot& st : img.stage_parts)
            if (!stage(c, st)) return false;
        uint32_t kind = 0, flags = 0;
        uint64_t body = 0;
        if (!c.record_header(kind, flags, body)) return refuse(error_, "the record stream has no END marker");
        if (kind != kWireRecordEnd || flags || body) return refuse(error_, "the END marker is malformed");
        if (!c.zeros(pool_begin_ - c.pos())) return false;   // the pad between END and the pool is defined: zero
        if (h_.live_tokens != int64_t(img.live.ids.size()))
            return refuse(error_, "live_tokens disagrees with the live checkpoint's id count");
        info.blobs = blobs_;
        if (!located_) out = std::move(img);
        return true;
    }

private:
    bool header(WireDecoded& info) {
        if (src_.size() < kWireHeaderRecordBytes) return refuse(error_, "the payload is shorter than the header record");
        uint8_t raw[kWireHeaderRecordBytes];
        if (!src_.read(raw, 0, sizeof raw)) return refuse(error_, "the source refused the header");
        h_ = parse_header(raw);
        if (h_.magic != kWireMagic) return refuse(error_, "not a hand-off payload (magic " + hex64(h_.magic) + ")");
        if (h_.fmt_version != kWireFormatVersion)
            return refuse(error_, "payload format version " + num(h_.fmt_version) + ", this codec speaks " +
                                      num(kWireFormatVersion));
        if (h_.flags & kWireFlagPartial) return refuse(error_, "the payload says it is partial");
        if (h_.flags & uint16_t(~kWireFlagKnown)) return refuse(error_, "unknown header flag bits");
        if (h_.payload_hash) return refuse(error_, "the header's payload_hash word is not zero");
        if (h_.reserved) return refuse(error_, "the header's reserved word is not zero");
        if (h_.payload_bytes < kWireHeaderRecordBytes) return refuse(error_, "the declared payload size is absurd");
        if (expect_.max_payload_bytes && h_.payload_bytes > expect_.max_payload_bytes)
            return refuse(error_, "the payload declares " + num(h_.payload_bytes) + " bytes, more than its " +
                                      num(expect_.max_payload_bytes) + "-byte slot");
        if (h_.payload_bytes > src_.size())
            return refuse(error_, "the payload declares " + num(h_.payload_bytes) + " bytes but " + num(src_.size()) +
                                      " are present (truncated)");
        if (h_.blob_pool_off < kWireHeaderRecordBytes || h_.blob_pool_off % kWireBlobAlign)
            return refuse(error_, "the blob pool does not start on a 64-byte boundary");
        if (h_.blob_pool_bytes > h_.payload_bytes - h_.blob_pool_off)
            return refuse(error_, "the blob pool runs past the end of the payload");
        pool_begin_ = h_.blob_pool_off;
        pool_end_ = h_.blob_pool_off + h_.blob_pool_bytes;
        const bool flagged = (h_.flags & kWireFlagHasStageParts) != 0;
        if (flagged ? h_.n_stage_parts <= 0 : h_.n_stage_parts > 0)
            return refuse(error_, "the stage-parts flag and the stage-parts count disagree");
        if (expect_.check_geometry)
            for (size_t i = 0; i < 18; ++i)
                if (h_.geometry[i] != uint64_t(expect_.geometry[i]))
                    return refuse(error_, "incompatible runtime geometry - " + conversation_wire_describe(h_));
        if (expect_.check_hashes && h_.geom_hash != expect_.geom_hash)
            return refuse(error_, "geometry hash " + hex64(h_.geom_hash) + " != " + hex64(expect_.geom_hash));
        if (expect_.check_hashes && h_.pack_hash != expect_.pack_hash)
            return refuse(error_, "pack hash " + hex64(h_.pack_hash) + " != " + hex64(expect_.pack_hash));
        if (expect_.stage_parts >= 0 && h_.n_stage_parts != expect_.stage_parts)
            return refuse(error_, "the payload carries " + num(uint64_t(h_.n_stage_parts)) +
                                      " stage parts and this instance has " + num(uint64_t(expect_.stage_parts)));
        if (!count_ok(h_.n_kv, kWireMaxKvRecords, "n_kv", 0, 0, error_) ||
            !count_ok(h_.n_checkpoints, kWireMaxCheckpoints, "n_checkpoints", 0, 0, error_) ||
            !count_ok(h_.n_stage_parts, kWireMaxStageParts, "n_stage_parts", 0, 0, error_))
            return false;
        if (h_.live_tokens < 0) return refuse(error_, "live_tokens is negative");
        info.bytes = h_.payload_bytes;
        info.geom_hash = h_.geom_hash;
        info.pack_hash = h_.pack_hash;
        for (size_t i = 0; i < 18; ++i) info.geometry[i] = int64_t(h_.geometry[i]);
        info.layer_lo = int64_t(h_.layer_lo);
        info.layer_hi = int64_t(h_.layer_hi);
        info.n_kv = h_.n_kv;
        info.n_checkpoints = h_.n_checkpoints;
        info.n_stage_parts = h_.n_stage_parts;
        info.live_tokens = h_.live_tokens;
        info.flags = h_.flags;
        info.cvec = (h_.flags & kWireFlagCvec) != 0;
        info.blob_pool_off = h_.blob_pool_off;
        info.blob_pool_bytes = h_.blob_pool_bytes;
        return true;
    }

    bool check_hash(WireDecoded& info) {
        if (!expect_.check_payload_hash || located_) return true;
        uint64_t h = kWireHashSeed;
        std::vector<uint8_t> chunk;
        for (uint64_t at = 0; at < h_.payload_bytes; at += kWireChunkBytes) {
            const size_t n = size_t(std::min<uint64_t>(kWireChunkBytes, h_.payload_bytes - at));
            if (const uint8_t* p = src_.span(at, n)) {
                h = fnv1a64(p, n, h);
                continue;
            }
            chunk.resize(n);
            if (!src_.read(chunk.data(), at, n)) return refuse(error_, "the source refused a read");
            h = fnv1a64(chunk.data(), n, h);
        }
        if (h != expect_.payload_hash)
            return refuse(error_, "payload hash " + hex64(h) + " != " + hex64(expect_.payload_hash) +
                                      " (the bytes are not the bytes that were written)");
        info.payload_hash = h;
        return true;
    }

    // A BLOBREF: {0, 0} or a 64-aligned run inside the pool.  Returns the run through `bytes` / `offset`.
    bool blobref(Cursor& c, uint64_t& bytes, uint64_t& offset) {
        if (!c.u64(bytes) || !c.u64(offset)) return false;
        if (!bytes) return offset == 0 || refuse(error_, "a zero-length blob must be referenced as {0,0}");
        ++blobs_;
        if (offset < pool_begin_ || offset % kWireBlobAlign)
            return refuse(error_, "a blob reference is not on a 64-byte boundary inside the pool");
        if (offset > pool_end_ || bytes > pool_end_ - offset) return refuse(error_, "a blob reference runs past the end of the pool");
        return true;
    }
    bool read_into(uint8_t* dst, uint64_t offset, uint64_t n) {
        for (uint64_t at = 0; at < n; at += kWireChunkBytes) {
            const size_t k = size_t(std::min<uint64_t>(kWireChunkBytes, n - at));
            if (const uint8_t* p = src_.span(offset + at, k)) std::memcpy(dst + at, p, k);
            else if (!src_.read(dst + at, offset + at, k)) return refuse(error_, "the source refused a blob read");
        }
        return true;
    }
    bool blob(Cursor& c, ConversationBuffer& b) {
        uint64_t bytes = 0, offset = 0;
        if (!blobref(c, bytes, offset)) return false;
        if (!bytes) return true;
        if (located_) { located_->push_back({&b, offset, bytes}); return true; }
        b.resize(size_t(bytes));   // bounded: the run lies inside the pool, inside the payload
        bool ok = true;
        b.visit(0, size_t(bytes), [&](uint8_t* p, size_t n, size_t at) { return ok = read_into(p, offset + at, n); });
        return ok;
    }
    bool blob(Cursor& c, std::vector<uint8_t>& v) {
        uint64_t bytes = 0, offset = 0;
        if (!blobref(c, bytes, offset)) return false;
        if (!bytes) return true;
        if (located_) { located_->push_back({&v, offset, bytes}); return true; }
        v.resize(size_t(bytes));
        return read_into(v.data(), offset, bytes);
    }

    bool kv_record(Cursor& c, ConversationKv& k, const char* where) {
        uint32_t kind = 0, flags = 0;
        uint64_t body = 0;
        if (!c.record_header(kind, flags, body)) return false;
        if (kind != kWireRecordKv || flags || body != kKvBodyBytes)
            return refuse(error_, std::string("the ") + where + " does not hold plain KV records (kind " + hex64(kind) +
                                      ", flags " + num(flags) + ", " + num(body) + " body bytes)");
        uint32_t fmt = 0;
        if (!c.u32(fmt) || !c.zeros(4)) return false;
        k.format = int(int32_t(fmt));
        for (int64_t* f : {&k.cells, &k.heads, &k.head_dim, &k.page_size, &k.pooled_rows, &k.idx_dim})
            if (!c.i64(*f)) return false;
        for (ConversationBuffer* b : {&k.k, &k.v, &k.k_scale, &k.v_scale, &k.pooled})
            if (!blob(c, *b)) return false;
        return true;
    }

    bool checkpoint(Cursor& c, ConversationCheckpoint& cp, int depth) {
        if (depth > expect_.max_checkpoint_depth)
            return refuse(error_, "stage_parts nested " + num(uint64_t(depth) + 1) + " deep, past the bound " +
                                      num(uint64_t(expect_.max_checkpoint_depth)));
        uint32_t kind = 0, flags = 0;
        uint64_t body = 0;
        if (!c.record_header(kind, flags, body)) return false;
        if (kind != kWireRecordCheckpoint) return refuse(error_, "expected a CHECKPOINT record, found kind " + hex64(kind));
        if (flags) return refuse(error_, "a record's flags field is not zero");
        if (body > c.room()) return refuse(error_, "a record declares more bytes than the payload has");
        const uint64_t end = c.pos() + body;
        int64_t n = 0;
        if (!c.i64(n) || !count_ok(n, std::numeric_limits<int64_t>::max() / 8, "n_ids", end - c.pos(), 4, error_))
            return false;
        cp.ids.resize(size_t(n));
        if constexpr (kHostLittleEndian) {
            if (!c.bytes(reinterpret_cast<uint8_t*>(cp.ids.data()), 4 * uint64_t(n))) return false;
        } else {
            uint8_t buf[4 * 2048];
            for (size_t i = 0; i < cp.ids.size();) {
                const size_t k = std::min<size_t>(2048, cp.ids.size() - i);
                if (!c.bytes(buf, 4 * k)) return false;
                for (size_t j = 0; j < k; ++j) cp.ids[i + j] = int32_t(get_le<uint32_t>(buf + 4 * j));
                i += k;
            }
        }
        if (!c.zeros(ids_pad(uint64_t(n))) || !c.i64(n) || !count_ok(n, kWireMaxImages, "n_imgs", end - c.pos(), 16, error_))
            return false;
        cp.imgs.resize(size_t(n));
        for (ConversationImageKey& key : cp.imgs)
            if (!c.i64(key.start) || !c.u64(key.hash)) return false;
        for (std::vector<uint8_t>* v : {&cp.gdn, &cp.ple, &cp.tails, &cp.dead, &cp.block_pos})
            if (!blob(c, *v)) return false;
        if (!c.u64(cp.used) || !c.i64(n) ||
            !count_ok(n, kWireMaxStageParts, "checkpoint stage_parts", end - c.pos(), kWireRecordHeaderBytes, error_))
            return false;
        cp.stage_parts.resize(size_t(n));
        for (ConversationCheckpoint& part : cp.stage_parts)
            if (!checkpoint(c, part, depth + 1)) return false;
        if (c.pos() != end) return refuse(error_, "a CHECKPOINT record's body does not end where its header said");
        return true;
    }

    bool stage(Cursor& c, ConversationStageSnapshot& st) {
        uint32_t kind = 0, flags = 0;
        uint64_t body = 0;
        if (!c.record_header(kind, flags, body)) return false;
        if (kind != kWireRecordStage) return refuse(error_, "expected a STAGE record, found kind " + hex64(kind));
        if (flags) return refuse(error_, "a record's flags field is not zero");
        if (body > c.room()) return refuse(error_, "a record declares more bytes than the payload has");
        const uint64_t end = c.pos() + body;
        int64_t n = 0;
        if (!c.i64(st.layer_lo) || !c.i64(st.layer_hi) || !checkpoint(c, st.state, 0) || !c.i64(n) ||
            !count_ok(n, kWireMaxKvRecords, "stage n_kv", end - c.pos(), kWireRecordHeaderBytes + kKvBodyBytes, error_))
            return false;
        st.kv.resize(size_t(n));
        for (ConversationKv& k : st.kv)
            if (!kv_record(c, k, "stage's K/V array")) return false;
        if (c.pos() != end) return refuse(error_, "a STAGE record's body does not end where its header said");
        return true;
    }

    const WireSource& src_;
    const WireExpect& expect_;
    std::string& error_;
    WireHeaderRecord h_{};
    uint64_t pool_begin_ = 0, pool_end_ = 0;
    size_t blobs_ = 0;
    std::vector<detail::WireBlobAt>* located_ = nullptr;
};

// The head of a payload (bytes [0, blob_pool_off)) standing in for a whole payload of `total` bytes.
class HeadSource final : public WireSource {
public:
    HeadSource(const uint8_t* head, uint64_t head_bytes, uint64_t total) : p_(head), n_(head_bytes), total_(total) {}
    uint64_t size() const override { return total_; }
    bool read(uint8_t* dst, uint64_t offset, size_t bytes) const override {
        if (offset > n_ || bytes > n_ - offset) return false;
        if (bytes) std::memcpy(dst, p_ + offset, bytes);
        return true;
    }
    const uint8_t* span(uint64_t offset, size_t bytes) const override {
        return offset <= n_ && bytes <= n_ - offset ? p_ + offset : nullptr;
    }

private:
    const uint8_t* p_;
    uint64_t n_, total_;
};

}  // namespace

// ---- sinks and sources --------------------------------------------------------------------------------------------------

bool VectorWireSink::write(const uint8_t* data, size_t bytes) {
    if (!bytes) return true;
    if (!data) return false;
    bytes_.insert(bytes_.end(), data, data + bytes);
    return true;
}

SlotWireSink::SlotWireSink(int fd, uint64_t offset, uint64_t capacity) : fd_(fd), base_(offset), capacity_(capacity) {}
SlotWireSink::SlotWireSink(uint8_t* mapping, uint64_t capacity) : map_(mapping), capacity_(capacity) {}

bool SlotWireSink::write(const uint8_t* data, size_t bytes) {
    if (!bytes) return true;
    if (pos_ > capacity_ || bytes > capacity_ - pos_) {
        error_ = "conversation wire: the payload needs " + num(pos_ + bytes) + " bytes and the slot holds " +
                 num(capacity_) + " (claim a larger tier)";
        return false;
    }
    if (map_) {
        std::memcpy(map_ + pos_, data, bytes);
        pos_ += bytes;
        return true;
    }
    while (bytes) {
        const ssize_t n = ::pwrite(fd_, data, bytes, off_t(base_ + pos_));
        if (n < 0 && errno == EINTR) continue;
        if (n <= 0) {
            error_ = std::string("conversation wire: pwrite into the slot failed: ") + (n < 0 ? std::strerror(errno) : "no progress");
            return false;
        }
        data += n;
        bytes -= size_t(n);
        pos_ += uint64_t(n);
    }
    return true;
}

bool SpanWireSource::read(uint8_t* dst, uint64_t offset, size_t bytes) const {
    const uint8_t* p = span(offset, bytes);
    if (!p && bytes) return false;
    if (bytes) std::memcpy(dst, p, bytes);
    return true;
}
const uint8_t* SpanWireSource::span(uint64_t offset, size_t bytes) const {
    if (!p_ || offset > n_ || bytes > n_ - offset) return nullptr;
    return p_ + offset;
}

bool FileWireSource::read(uint8_t* dst, uint64_t offset, size_t bytes) const {
    if (offset > n_ || bytes > n_ - offset) return false;
    while (bytes) {
        const ssize_t n = ::pread(fd_, dst, bytes, off_t(base_ + offset));
        if (n < 0 && errno == EINTR) continue;
        if (n <= 0) return false;
        dst += n;
        offset += uint64_t(n);
        bytes -= size_t(n);
    }
    return true;
}

// ---- entry points -------------------------------------------------------------------------------------------------------

bool conversation_wire_plan(const SavedConversation& image, WirePlan& plan, std::string& error) {
    return conversation_wire_plan(image, kWireMaxCheckpointDepth, plan, error);
}

bool conversation_wire_plan(const SavedConversation& image, int max_checkpoint_depth, WirePlan& plan, std::string& error) {
    plan = WirePlan{};
    Layout lay;
    if (!lay_out(image, std::max(1, max_checkpoint_depth), lay, error)) return false;
    plan = lay.plan;
    return true;
}

bool conversation_wire_encode(const SavedConversation& image, WireSink& sink, const WireIdentity& identity,
                              WireEncoded& out, std::string& error) {
    WirePlan plan;
    return conversation_wire_encode(image, sink, identity, kWireMaxCheckpointDepth, plan, out, error);
}

bool conversation_wire_encode(const SavedConversation& image, WireSink& sink, const WireIdentity& identity,
                              int max_checkpoint_depth, WirePlan& plan, WireEncoded& out, std::string& error) {
    out = WireEncoded{};
    plan = WirePlan{};
    const int depth = std::max(1, max_checkpoint_depth);
    Layout lay;
    if (!lay_out(image, depth, lay, error)) return false;
    plan = lay.plan;
    Writer w(sink, lay, error);
    if (!write_payload(image, identity, lay, depth, w, error)) return false;
    out.bytes = w.written();
    out.payload_hash = w.hash();
    out.blob_pool_bytes = plan.blob_pool_bytes;
    out.blobs = plan.blobs;
    return true;
}

bool conversation_wire_decode(const WireSource& source, SavedConversation& image, WireDecoded& info,
                              const WireExpect& expect, std::string& error) {
    info = WireDecoded{};
    Parser p(source, expect, error);
    return p.run(image, info);
}

bool conversation_wire_decode(const uint8_t* data, uint64_t bytes, SavedConversation& image, WireDecoded& info,
                              const WireExpect& expect, std::string& error) {
    const SpanWireSource src(data, bytes);
    return conversation_wire_decode(src, image, info, expect, error);
}

bool conversation_wire_peek(const uint8_t* data, uint64_t bytes, WireHeaderRecord& header, std::string& error) {
    if (!data || bytes < kWireHeaderRecordBytes) return refuse(error, "the payload is shorter than the header record");
    header = parse_header(data);
    if (header.magic != kWireMagic) return refuse(error, "not a hand-off payload");
    if (header.fmt_version != kWireFormatVersion) return refuse(error, "payload format version mismatch");
    if (header.flags & uint16_t(~kWireFlagKnown)) return refuse(error, "unknown header flag bits");
    if (header.payload_bytes < kWireHeaderRecordBytes) return refuse(error, "the declared payload size is absurd");
    if (header.blob_pool_off < kWireHeaderRecordBytes || header.blob_pool_off % kWireBlobAlign)
        return refuse(error, "the blob pool does not start on a 64-byte boundary");
    if (header.blob_pool_bytes > header.payload_bytes - header.blob_pool_off)
        return refuse(error, "the blob pool runs past the end of the payload");
    return true;
}

uint64_t conversation_wire_payload_hash(const uint8_t* data, uint64_t bytes) { return fnv1a64(data, bytes, kWireHashSeed); }

namespace detail {

bool wire_head(const SavedConversation& image, const WireIdentity& identity, const WireSizes& sizes,
               std::vector<uint8_t>& head, std::vector<WireBlobAt>& pool, WirePlan& plan, std::string& error) {
    Layout lay;
    lay.sizes = &sizes;
    if (!lay_out(image, kWireMaxCheckpointDepth, lay, error)) return false;
    plan = lay.plan;
    VectorWireSink sink(size_t(plan.blob_pool_off));
    Writer w(sink, lay, error, false);   // the device hashes the whole payload, head included
    if (!write_payload(image, identity, lay, kWireMaxCheckpointDepth, w, error, true)) return false;
    if (w.written() != plan.blob_pool_off) return refuse(error, "internal: the head is not the bytes before the pool");
    head = std::move(sink.data());
    pool.clear();
    for (const PoolEntry& e : lay.pool)
        pool.push_back({e.buf ? static_cast<const void*>(e.buf) : static_cast<const void*>(e.vec),
                        plan.blob_pool_off + e.rel, e.bytes});
    return true;
}

bool wire_locate(const uint8_t* head, uint64_t head_bytes, SavedConversation& image, WireDecoded& info,
                 const WireExpect& expect, std::vector<WireBlobAt>& blobs, std::string& error) {
    if (!head || head_bytes < kWireHeaderRecordBytes) return refuse(error, "the payload is shorter than the header record");
    const uint64_t total = get_le<uint64_t>(head + 232);
    if (get_le<uint64_t>(head + 200) > head_bytes)
        return refuse(error, "the head given does not reach the blob pool");
    const HeadSource src(head, head_bytes, std::max(total, head_bytes));
    info = WireDecoded{};
    blobs.clear();
    Parser p(src, expect, error);
    p.locate_into(&blobs);
    return p.run(image, info);
}

}  // namespace detail

std::string conversation_wire_describe(const WireHeaderRecord& h) {
    std::string s = "geometry [";
    for (size_t i = 0; i < 18; ++i) s += (i ? "," : "") + std::to_string(int64_t(h.geometry[i]));
    s += "] layers [" + std::to_string(int64_t(h.layer_lo)) + "," + std::to_string(int64_t(h.layer_hi)) + ") kv " +
         std::to_string(h.n_kv) + " checkpoints " + std::to_string(h.n_checkpoints) + " stages " +
         std::to_string(h.n_stage_parts) + " tokens " + std::to_string(h.live_tokens) + " geom " + hex64(h.geom_hash) +
         " pack " + hex64(h.pack_hash);
    return s;
}

}  // namespace strata::core

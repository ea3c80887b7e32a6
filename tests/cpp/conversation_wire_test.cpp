// conversation_wire_test.cpp - host-only checks of the payload codec (host/src/conversation_wire.cpp) that need
// images built in C++: the scenarios of the reference's codec test (src/core/saved_conv_wire_test.cpp) restated -
// round trips through every source and sink shape, a buffer spanning 16 MiB segments written as its own segments and
// read back through a source that serves small pieces, the claim never travelling, plan and encode agreeing, the
// depth bound, all-or-nothing decoding, and peek.  Byte-level parity with the reference codec is checked separately
// (tests/test_wire_codec.py runs this library's build of oracle/ref_wire_driver.cpp against the golden manifest).
#include "strata/core/conversation_wire.hpp"

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

using namespace strata::core;

namespace {

int checks = 0, failures = 0;
void check(bool ok, const char* what) {
    ++checks;
    if (!ok) {
        ++failures;
        std::printf("FAIL: %s\n", what);
    }
}
void check_ok(bool ok, const std::string& err, const char* what) {
    ++checks;
    if (!ok) {
        ++failures;
        std::printf("FAIL: %s: %s\n", what, err.c_str());
    }
}

uint8_t pattern(uint64_t salt, uint64_t i) { return uint8_t((salt * 131 + i * 31 + (i >> 8) * 7) & 0xFF); }

void fill(ConversationBuffer& b, size_t n, uint64_t salt) {
    b.resize(n);
    b.visit(0, n, [&](uint8_t* p, size_t k, size_t at) {
        for (size_t i = 0; i < k; ++i) p[i] = pattern(salt, at + i);
        return true;
    });
}
std::vector<uint8_t> vec(size_t n, uint64_t salt) {
    std::vector<uint8_t> v(n);
    for (size_t i = 0; i < n; ++i) v[i] = pattern(salt, i);
    return v;
}

ConversationKv make_kv(int64_t cells, uint64_t salt, size_t extra = 0) {
    ConversationKv k;
    k.cells = cells;
    k.heads = 2;
    k.head_dim = 16;
    k.page_size = 4;
    fill(k.k, size_t(cells) * 2 * 16 * 2 + extra, salt);
    fill(k.v, size_t(cells) * 2 * 16 * 2, salt + 1);
    return k;
}

ConversationCheckpoint make_cp(size_t ids, uint64_t salt) {
    ConversationCheckpoint c;
    for (size_t i = 0; i < ids; ++i) c.ids.push_back(int32_t(salt * 7 + i));
    c.imgs = {{4, salt}, {8, salt * 3}};
    c.gdn = vec(300 + salt, salt);
    c.ple = vec(40, salt + 9);
    c.tails = vec(8, salt + 10);
    c.used = salt;
    return c;
}

SavedConversation make_image(int layers, size_t ids, uint64_t salt) {
    SavedConversation s;
    for (size_t i = 0; i < 18; ++i) s.geometry[i] = int64_t(i * 3 + salt);
    s.layer_lo = 0;
    s.layer_hi = layers;
    for (int j = 0; j < layers / 4; ++j) s.kv.push_back(make_kv(int64_t(ids + 3) / 4 * 4, salt + j * 2));
    s.kv.emplace_back();   // the draft layer, empty
    s.live = make_cp(ids, salt);
    s.checkpoints.push_back(make_cp(ids / 2, salt + 50));
    return s;
}

bool same_cp(const ConversationCheckpoint& a, const ConversationCheckpoint& b) {
    if (a.ids != b.ids || a.imgs.size() != b.imgs.size() || a.gdn != b.gdn || a.ple != b.ple || a.tails != b.tails ||
        a.dead != b.dead || a.block_pos != b.block_pos || a.used != b.used || a.stage_parts.size() != b.stage_parts.size())
        return false;
    for (size_t i = 0; i < a.imgs.size(); ++i)
        if (!(a.imgs[i] == b.imgs[i])) return false;
    for (size_t i = 0; i < a.stage_parts.size(); ++i)
        if (!same_cp(a.stage_parts[i], b.stage_parts[i])) return false;
    return true;
}
bool same_kv(const ConversationKv& a, const ConversationKv& b) {
    return a.format == b.format && a.cells == b.cells && a.heads == b.heads && a.head_dim == b.head_dim &&
           a.page_size == b.page_size && a.pooled_rows == b.pooled_rows && a.idx_dim == b.idx_dim && a.k == b.k &&
           a.v == b.v && a.k_scale == b.k_scale && a.v_scale == b.v_scale && a.pooled == b.pooled;
}
bool same_image(const SavedConversation& a, const SavedConversation& b) {
    if (a.geometry != b.geometry || a.layer_lo != b.layer_lo || a.layer_hi != b.layer_hi || a.cvec != b.cvec ||
        a.kv.size() != b.kv.size() || a.checkpoints.size() != b.checkpoints.size() ||
        a.stage_parts.size() != b.stage_parts.size() || !same_cp(a.live, b.live))
        return false;
    for (size_t i = 0; i < a.kv.size(); ++i)
        if (!same_kv(a.kv[i], b.kv[i])) return false;
    for (size_t i = 0; i < a.checkpoints.size(); ++i)
        if (!same_cp(a.checkpoints[i], b.checkpoints[i])) return false;
    for (size_t i = 0; i < a.stage_parts.size(); ++i) {
        const auto &x = a.stage_parts[i], &y = b.stage_parts[i];
        if (x.layer_lo != y.layer_lo || x.layer_hi != y.layer_hi || !same_cp(x.state, y.state) || x.kv.size() != y.kv.size())
            return false;
        for (size_t j = 0; j < x.kv.size(); ++j)
            if (!same_kv(x.kv[j], y.kv[j])) return false;
    }
    return true;
}

WireExpect expect_for(const SavedConversation& s, uint64_t geom, uint64_t pack) {
    WireExpect e;
    e.geometry = s.geometry;
    e.check_geometry = true;
    e.geom_hash = geom;
    e.pack_hash = pack;
    e.check_hashes = true;
    return e;
}

// A sink that records the largest single write and how many there were.
struct CountingSink final : WireSink {
    std::vector<uint8_t> bytes;
    size_t writes = 0, max_write = 0;
    bool write(const uint8_t* d, size_t n) override {
        ++writes;
        max_write = std::max(max_write, n);
        bytes.insert(bytes.end(), d, d + n);
        return true;
    }
};
// A source with no span() that serves reads of at most `piece` bytes by splitting them.
struct ChunkySource final : WireSource {
    const std::vector<uint8_t>& d;
    size_t piece;
    mutable size_t reads = 0;
    ChunkySource(const std::vector<uint8_t>& data, size_t p) : d(data), piece(p) {}
    uint64_t size() const override { return d.size(); }
    bool read(uint8_t* dst, uint64_t off, size_t n) const override {
        ++reads;
        if (off > d.size() || n > d.size() - off) return false;
        for (size_t at = 0; at < n; at += piece) std::memcpy(dst + at, d.data() + off + at, std::min(piece, n - at));
        return true;
    }
};
// A sink that stops accepting after `cap` bytes.
struct ShortSink final : WireSink {
    size_t cap, got = 0;
    explicit ShortSink(size_t c) : cap(c) {}
    bool write(const uint8_t*, size_t n) override {
        if (got + n > cap) return false;
        got += n;
        return true;
    }
    std::string refusal() const override { return "the test sink is full"; }
};

void test_round_trips() {
    const SavedConversation s = make_image(16, 37, 3);
    WirePlan plan;
    std::string err;
    check_ok(conversation_wire_plan(s, plan, err), err, "plan");
    VectorWireSink sink;
    WireEncoded enc;
    check_ok(conversation_wire_encode(s, sink, {0x11, 0x22}, enc, err), err, "encode");
    check(enc.bytes == plan.total_bytes && sink.data().size() == plan.total_bytes, "plan and encode agree on the size");
    check(enc.payload_hash == conversation_wire_payload_hash(sink.data().data(), sink.data().size()),
          "the streamed hash is the hash of the bytes written");
    check(plan.blob_pool_off % kWireBlobAlign == 0 && plan.total_bytes == plan.blob_pool_off + plan.blob_pool_bytes,
          "the pool is 64-aligned and ends the payload");
    SavedConversation out;
    WireDecoded info;
    WireExpect e = expect_for(s, 0x11, 0x22);
    e.payload_hash = enc.payload_hash;
    e.check_payload_hash = true;
    check_ok(conversation_wire_decode(sink.data().data(), sink.data().size(), out, info, e, err), err, "decode");
    check(same_image(s, out), "decode(encode(x)) == x");
    check(info.blobs == plan.blobs && info.live_tokens == 37 && info.n_kv == int64_t(s.kv.size()), "decoded info");
    VectorWireSink again;
    check_ok(conversation_wire_encode(out, again, {0x11, 0x22}, enc, err), err, "re-encode");
    check(again.data() == sink.data(), "encode(decode(p)) == p byte for byte");
    ChunkySource src(sink.data(), 100);
    SavedConversation out2;
    check_ok(conversation_wire_decode(src, out2, info, e, err), err, "decode from a source without spans");
    check(same_image(s, out2) && src.reads > 10, "the read path reproduces the image");
    WireHeaderRecord h{};
    check_ok(conversation_wire_peek(sink.data().data(), sink.data().size(), h, err), err, "peek");
    check(h.payload_bytes == plan.total_bytes && h.live_tokens == 37 && h.geom_hash == 0x11, "peek reads the header");
    check(!conversation_wire_peek(sink.data().data(), kWireHeaderRecordBytes - 1, h, err), "peek refuses a short header");
}

void test_segments() {
    // a K buffer of 20 MiB + 3 bytes spans two 16 MiB segments; the writer hands the segments over as they are
    SavedConversation s = make_image(4, 8, 5);
    fill(s.kv[0].k, (20u << 20) + 3, 77);
    CountingSink sink;
    WireEncoded enc;
    std::string err;
    check_ok(conversation_wire_encode(s, sink, {1, 2}, enc, err), err, "big encode");
    check(sink.max_write == ConversationBuffer::segment_bytes,
          "each segment goes out as one write, straight from the segment (none larger)");
    check(sink.writes > 8, "the payload went out record by record and segment by segment, never staged whole");
    ChunkySource src(sink.bytes, 4096);
    SavedConversation out;
    WireDecoded info;
    check_ok(conversation_wire_decode(src, out, info, expect_for(s, 1, 2), err), err, "big decode");
    check(same_image(s, out) && out.kv[0].k.size() == (20u << 20) + 3, "the spanning buffer comes back byte for byte");
}

void test_claim_and_all_or_nothing() {
    SavedConversation s = make_image(8, 9, 7);
    s.owner = 4242;
    VectorWireSink sink;
    WireEncoded enc;
    std::string err;
    check_ok(conversation_wire_encode(s, sink, {5, 6}, enc, err), err, "owner encode");
    SavedConversation out;
    out.owner = 777;
    WireDecoded info;
    check_ok(conversation_wire_decode(sink.data().data(), sink.data().size(), out, info, expect_for(s, 5, 6), err), err,
             "owner decode");
    check(out.owner == kNoOwner, "a claim never travels on the wire");
    // a refused decode leaves the caller's image exactly as it was
    SavedConversation untouched = make_image(4, 3, 9);
    const SavedConversation before = untouched;
    std::vector<uint8_t> bad = sink.data();
    bad[bad.size() - 1] ^= 1;
    WireExpect e = expect_for(s, 5, 6);
    e.payload_hash = enc.payload_hash;
    e.check_payload_hash = true;
    check(!conversation_wire_decode(bad.data(), bad.size(), untouched, info, e, err), "a corrupt payload is refused");
    check(err.find("payload hash") != std::string::npos, "by its content hash");
    check(same_image(untouched, before), "a refused decode writes nothing into the target");
    e.geom_hash = 99;
    check(!conversation_wire_decode(sink.data().data(), sink.data().size(), untouched, info, e, err) &&
              same_image(untouched, before), "an identity mismatch writes nothing either");
}

void test_depth_and_live_parts() {
    SavedConversation deep = make_image(4, 5, 3);
    ConversationCheckpoint* at = &deep.checkpoints[0];
    for (int i = 0; i < 40; ++i) {
        at->stage_parts.emplace_back();
        at = &at->stage_parts.back();
        at->ids = {1, 2, 3};
    }
    WirePlan plan;
    std::string err;
    check(!conversation_wire_plan(deep, plan, err), "plan refuses an over-deep chain");
    VectorWireSink sink;
    WireEncoded enc;
    check_ok(conversation_wire_encode(deep, sink, {1, 2}, 64, plan, enc, err), err, "a raised bound encodes it");
    SavedConversation out;
    WireDecoded info;
    WireExpect e = expect_for(deep, 1, 2);
    check(!conversation_wire_decode(sink.data().data(), sink.data().size(), out, info, e, err), "decode refuses it");
    check(err.find("nested") != std::string::npos, "and says it is nested too deep");
    e.max_checkpoint_depth = 64;
    check_ok(conversation_wire_decode(sink.data().data(), sink.data().size(), out, info, e, err), err, "raised bound");
    check(same_image(deep, out), "the deep chain round-trips under the raised bound");
    SavedConversation bad = make_image(4, 5, 3);
    bad.live.stage_parts.emplace_back();
    check(!conversation_wire_plan(bad, plan, err), "stage parts inside the live checkpoint are refused");
    check(!conversation_wire_encode(bad, sink, {1, 2}, enc, err), "by encode too");
}

void test_sinks() {
    const SavedConversation s = make_image(8, 21, 11);
    WirePlan plan;
    std::string err;
    check_ok(conversation_wire_plan(s, plan, err), err, "plan");
    ShortSink tiny(plan.total_bytes / 2);
    WireEncoded enc;
    check(!conversation_wire_encode(s, tiny, {1, 2}, enc, err), "a sink that runs out refuses the encode");
    check(err.find("the test sink is full") != std::string::npos, "and its own reason reaches the message");
    std::vector<uint8_t> slot(plan.total_bytes + 100, 0xEE);
    SlotWireSink mapped(slot.data(), plan.total_bytes);
    check_ok(conversation_wire_encode(s, mapped, {1, 2}, enc, err), err, "mapped slot sink");
    VectorWireSink ref;
    check_ok(conversation_wire_encode(s, ref, {1, 2}, enc, err), err, "vector sink");
    check(std::equal(ref.data().begin(), ref.data().end(), slot.begin()) && slot[plan.total_bytes] == 0xEE,
          "the mapped slot holds the payload and nothing past it");
    SlotWireSink small(slot.data(), plan.total_bytes - 1);
    check(!conversation_wire_encode(s, small, {1, 2}, enc, err), "a slot one byte short refuses");
    FILE* f = std::tmpfile();
    if (f) {
        SlotWireSink file(fileno(f), 4096, plan.total_bytes);
        check_ok(conversation_wire_encode(s, file, {1, 2}, enc, err), err, "file slot sink");
        FileWireSource src(fileno(f), 4096, plan.total_bytes);
        SavedConversation out;
        WireDecoded info;
        check_ok(conversation_wire_decode(src, out, info, expect_for(s, 1, 2), err), err, "file source");
        check(same_image(s, out), "a payload written through pwrite reads back through pread");
        std::fclose(f);
    }
}

}  // namespace

int main() {
    test_round_trips();
    test_segments();
    test_claim_and_all_or_nothing();
    test_depth_and_live_parts();
    test_sinks();
    std::printf("conversation_wire_test: %d/%d checks passed\n", checks - failures, checks);
    return failures ? 1 : 0;
}

// ref_wire_driver.cpp - drives the REFERENCE's own payload codec (src/core/conversation_wire.cpp, compiled from the
// reference's sources by oracle/Makefile.ref into oracle/_ref/ref_wire) to write golden payloads and refusal verdicts.
//
// TEST INFRASTRUCTURE ONLY.  Used in this container by tests/golden/make_wire_vectors.py (fixtures) and by the CPU
// tests when the reference build exists; nothing in the product links or runs it.
//
// An image is described by a "wire spec": whitespace-separated integers (grammar below), and every byte of every
// buffer comes from a fixed fill rule, so the same spec gives the same SavedConversation here, in the Python oracle
// (oracle/sc_wire.py) and in the C++ codec's test (tests/cpp/conversation_wire_test.cpp):
//
//   spec       := geom_hash pack_hash geometry[18] layer_lo layer_hi cvec n_kv kv{n_kv} checkpoint
//                 n_checkpoints checkpoint{n_checkpoints} n_stage stage{n_stage}
//   kv         := format cells heads head_dim page_size pooled_rows idx_dim len_k len_v len_k_scale len_v_scale len_pooled
//   checkpoint := n_ids n_imgs len_gdn len_ple len_tails len_dead len_block_pos used n_parts checkpoint{n_parts}
//   stage      := layer_lo layer_hi checkpoint n_kv kv{n_kv}
//
// Fill rule: a counter `salt` starts at 1 and is taken (then incremented) by every array in traversal order - for a
// kv: k, v, k_scale, v_scale, pooled; for a checkpoint: ids, imgs, gdn, ple, tails, dead, block_pos, then its parts.
//   byte i    = (salt*131 + i*31 + (i>>8)*7 + (i>>16)*3) & 0xFF
//   ids[i]    = int32(uint32(salt*2654435761 + i*40503))
//   imgs[i]   = {start = 4*i + salt, hash = splitmix64 finaliser of (salt*1000003 + i)}
//
// Usage:
//   ref_wire time SPEC REPS        the CPU baseline of the codec: build the image (untimed), then REPS times encode it
//                                  into memory (payload hash included) and decode it back with the payload hash
//                                  checked; print "bytes=<n> encode_s=<best> decode_s=<best>"
//   ref_wire encode SPEC OUT       write the payload; print "<bytes> <payload_hash hex>"
//   ref_wire decode PAYLOAD GEOM_HASH PACK_HASH PAYLOAD_HASH|- [STAGE_PARTS [MAX_PAYLOAD_BYTES]]
//                                  decode with those expectations (a '-' hash is not checked); print
//                                  "ok <re-encode equal 0|1>" or "refused <message>"
#include "strata/core/conversation_wire.hpp"

#include <algorithm>
#include <chrono>
#include <cinttypes>
#include <cstdio>
#include <cstdlib>
#include <fstream>
#include <iterator>
#include <sstream>
#include <string>
#include <vector>

using namespace strata::core;

namespace {

struct Reader {
    std::vector<long long> v;
    size_t at = 0;
    long long next() {
        if (at >= v.size()) { std::fprintf(stderr, "spec ends early\n"); std::exit(2); }
        return v[at++];
    }
};

uint64_t salt_counter = 1;

uint8_t pattern(uint64_t salt, uint64_t i) {
    return uint8_t((salt * 131 + i * 31 + (i >> 8) * 7 + (i >> 16) * 3) & 0xFF);
}
uint64_t mix(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

void fill_buffer(ConversationBuffer& b, uint64_t n) {
    const uint64_t salt = salt_counter++;
    b.resize((size_t) n);
    b.visit(0, (size_t) n, [&](uint8_t* p, size_t cnt, size_t at) {
        for (size_t i = 0; i < cnt; ++i) p[i] = pattern(salt, at + i);
        return true;
    });
}
void fill_vector(std::vector<uint8_t>& b, uint64_t n) {
    const uint64_t salt = salt_counter++;
    b.resize((size_t) n);
    for (uint64_t i = 0; i < n; ++i) b[(size_t) i] = pattern(salt, i);
}

void read_kv(Reader& r, ConversationKv& k) {
    k.format = (int) r.next();
    k.cells = r.next();
    k.heads = r.next();
    k.head_dim = r.next();
    k.page_size = r.next();
    k.pooled_rows = r.next();
    k.idx_dim = r.next();
    const uint64_t lk = (uint64_t) r.next(), lv = (uint64_t) r.next(), lks = (uint64_t) r.next(),
                   lvs = (uint64_t) r.next(), lp = (uint64_t) r.next();
    fill_buffer(k.k, lk);
    fill_buffer(k.v, lv);
    fill_buffer(k.k_scale, lks);
    fill_buffer(k.v_scale, lvs);
    fill_buffer(k.pooled, lp);
}

void read_checkpoint(Reader& r, ConversationCheckpoint& c) {
    const long long n_ids = r.next(), n_imgs = r.next();
    const uint64_t lg = (uint64_t) r.next(), lp = (uint64_t) r.next(), lt = (uint64_t) r.next(),
                   ld = (uint64_t) r.next(), lb = (uint64_t) r.next();
    c.used = (uint64_t) r.next();
    const long long n_parts = r.next();
    {
        const uint64_t salt = salt_counter++;
        c.ids.resize((size_t) n_ids);
        for (long long i = 0; i < n_ids; ++i) c.ids[(size_t) i] = (int32_t) (uint32_t) (salt * 2654435761ull + (uint64_t) i * 40503ull);
    }
    {
        const uint64_t salt = salt_counter++;
        c.imgs.resize((size_t) n_imgs);
        for (long long i = 0; i < n_imgs; ++i) {
            c.imgs[(size_t) i].start = 4 * i + (long long) salt;
            c.imgs[(size_t) i].hash = mix(salt * 1000003ull + (uint64_t) i);
        }
    }
    fill_vector(c.gdn, lg);
    fill_vector(c.ple, lp);
    fill_vector(c.tails, lt);
    fill_vector(c.dead, ld);
    fill_vector(c.block_pos, lb);
    c.stage_parts.resize((size_t) n_parts);
    for (auto& p : c.stage_parts) read_checkpoint(r, p);
}

SavedConversation read_spec(const std::string& path, WireIdentity& id) {
    std::ifstream f(path);
    Reader r;
    long long x;
    while (f >> x) r.v.push_back(x);
    id.geom_hash = (uint64_t) r.next();
    id.pack_hash = (uint64_t) r.next();
    SavedConversation img;
    for (auto& g : img.geometry) g = r.next();
    img.layer_lo = r.next();
    img.layer_hi = r.next();
    img.cvec = r.next() != 0;
    img.kv.resize((size_t) r.next());
    for (auto& k : img.kv) read_kv(r, k);
    read_checkpoint(r, img.live);
    img.checkpoints.resize((size_t) r.next());
    for (auto& c : img.checkpoints) read_checkpoint(r, c);
    img.stage_parts.resize((size_t) r.next());
    for (auto& s : img.stage_parts) {
        s.layer_lo = r.next();
        s.layer_hi = r.next();
        read_checkpoint(r, s.state);
        s.kv.resize((size_t) r.next());
        for (auto& k : s.kv) read_kv(r, k);
    }
    return img;
}

std::vector<uint8_t> slurp(const std::string& path) {
    std::ifstream f(path, std::ios::binary);
    return std::vector<uint8_t>((std::istreambuf_iterator<char>(f)), std::istreambuf_iterator<char>());
}

}  // namespace

int main(int argc, char** argv) {
    if (argc >= 4 && std::string(argv[1]) == "time") {
        WireIdentity id;
        const SavedConversation img = read_spec(argv[2], id);
        const int reps = std::atoi(argv[3]) > 0 ? std::atoi(argv[3]) : 1;
        double best_enc = 1e30, best_dec = 1e30;
        uint64_t bytes = 0;
        std::string err;
        for (int r = 0; r < reps; ++r) {
            VectorWireSink sink;
            WireEncoded enc;
            auto t0 = std::chrono::steady_clock::now();
            if (!conversation_wire_encode(img, sink, id, enc, err)) {
                std::printf("refused %s\n", err.c_str());
                return 1;
            }
            auto t1 = std::chrono::steady_clock::now();
            WireExpect expect;
            expect.geom_hash = id.geom_hash;
            expect.pack_hash = id.pack_hash;
            expect.check_hashes = true;
            expect.check_payload_hash = true;
            expect.payload_hash = enc.payload_hash;
            SavedConversation back;
            WireDecoded info;
            if (!conversation_wire_decode(sink.data().data(), sink.data().size(), back, info, expect, err)) {
                std::printf("refused %s\n", err.c_str());
                return 1;
            }
            auto t2 = std::chrono::steady_clock::now();
            bytes = sink.data().size();
            best_enc = std::min(best_enc, std::chrono::duration<double>(t1 - t0).count());
            best_dec = std::min(best_dec, std::chrono::duration<double>(t2 - t1).count());
        }
        std::printf("bytes=%" PRIu64 " encode_s=%.6f decode_s=%.6f\n", bytes, best_enc, best_dec);
        return 0;
    }
    if (argc >= 4 && std::string(argv[1]) == "encode") {
        WireIdentity id;
        SavedConversation img = read_spec(argv[2], id);
        VectorWireSink sink;
        WireEncoded enc;
        std::string err;
        if (!conversation_wire_encode(img, sink, id, enc, err)) {
            std::printf("refused %s\n", err.c_str());
            return 0;
        }
        std::ofstream out(argv[3], std::ios::binary);
        out.write(reinterpret_cast<const char*>(sink.data().data()), (std::streamsize) sink.data().size());
        std::printf("%zu %016" PRIx64 "\n", sink.data().size(), enc.payload_hash);
        return 0;
    }
    if (argc >= 6 && std::string(argv[1]) == "decode") {
        const std::vector<uint8_t> payload = slurp(argv[2]);
        WireExpect expect;
        expect.geom_hash = std::strtoull(argv[3], nullptr, 0);
        expect.pack_hash = std::strtoull(argv[4], nullptr, 0);
        expect.check_hashes = true;
        expect.check_payload_hash = std::string(argv[5]) != "-";
        if (expect.check_payload_hash) expect.payload_hash = std::strtoull(argv[5], nullptr, 0);
        if (argc >= 7) expect.stage_parts = std::strtoll(argv[6], nullptr, 0);
        if (argc >= 8) expect.max_payload_bytes = std::strtoull(argv[7], nullptr, 0);
        SavedConversation img;
        WireDecoded info;
        std::string err;
        if (!conversation_wire_decode(payload.data(), payload.size(), img, info, expect, err)) {
            std::printf("refused %s\n", err.c_str());
            return 0;
        }
        VectorWireSink sink;
        WireEncoded enc;
        const bool again = conversation_wire_encode(img, sink, WireIdentity{info.geom_hash, info.pack_hash}, enc, err);
        std::printf("ok %d\n", again && sink.data() == payload ? 1 : 0);
        return 0;
    }
    std::fprintf(stderr, "usage: ref_wire encode SPEC OUT | decode PAYLOAD GEOM PACK HASH\n");
    return 2;
}

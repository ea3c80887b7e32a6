// ref_arena_driver.cpp - one command-line driver over the hand-off arena API (include/strata/core/handoff.hpp), compiled
// twice: against the REFERENCE's implementation (src/core/handoff.cpp, built in place by oracle/Makefile.ref into
// oracle/_ref/ref_arena) and against this library's (tests/cpp/bin/arena_driver).  The CPU tests run the two on the
// same arena files: one implementation writes and publishes, the other reads; both size, hash and dump the same way.
//
// TEST INFRASTRUCTURE ONLY: nothing in the product links or runs it.
//
// Every command prints "key=value" words on one line per step.  TIERS is "max_tokens:slots,..."; PRICED is the
// priced payload bytes of each tier, "b0,b1,...".  Payload byte i of a given seed is (i*131 + seed*17 + (i>>9)) & 255.
//
//   geom-hash SPEC G0 .. G17                    hash=<16 hex>
//   split-spec MAIN_LO MAIN_HI DRAFT_LAST [LO HI]...  spec=<spec>
//   path DIR PACK16 SPEC INSTANCE               path=<path>
//   size TIERS PRICED                           one line per tier (slot_bytes, slot_off), then arena/total/describe
//   create PATH PACK16 GEOM16 TIERS PRICED       open_writer, print describe, exit
//   hold PATH PACK16 GEOM16 TIERS PRICED         open_writer, print "HELD pid=<pid>", wait for a line on stdin, exit
//   write PATH PACK16 GEOM16 TIERS PRICED TIER CLIENT REQUEST BYTES SEED TOKENS ALLOW
//                                               open_writer(allow_existing_writer = ALLOW), claim, write, publish
//   read PATH PACK16 GEOM16 SLOT NONCE16 CLIENT SEED
//                                               open_reader, read_slot, check every byte and the hash
//   info PATH PACK16 GEOM16 SLOT                 slot_info of one slot, every field
//   time PATH PACK16 GEOM16 TIERS PRICED BYTES REPS
//                                               the CPU baseline of the hand-off: REPS times claim, write_payload
//                                               (one call), fnv1a64, publish (the writer's leg), then read_slot and
//                                               payload_hash_of (the reader's leg), release; print the best of each
#include "strata/core/handoff.hpp"

#include <algorithm>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include <unistd.h>

using namespace strata::core;

namespace {

uint8_t pattern(uint64_t i, uint64_t seed) { return (uint8_t) ((i * 131u + seed * 17u + (i >> 9)) & 0xFF); }

uint64_t hexarg(const char* s) { return std::strtoull(s, nullptr, 16); }
uint64_t decarg(const char* s) { return std::strtoull(s, nullptr, 10); }

std::vector<uint64_t> list(const char* s) {
    std::vector<uint64_t> out;
    const char* p = s;
    while (*p) {
        char* end = nullptr;
        out.push_back(std::strtoull(p, &end, 10));
        p = end;
        if (*p == ',' || *p == ':') ++p;
    }
    return out;
}

bool sizing(const char* tiers_arg, const char* priced_arg, HandoffSizing& s, std::string& err) {
    const std::vector<uint64_t> flat = list(tiers_arg);
    std::vector<HandoffTierSpec> tiers;
    for (size_t i = 0; i + 1 < flat.size(); i += 2) tiers.push_back({flat[i], flat[i + 1]});
    return handoff_size_arena(tiers, list(priced_arg), s, err);
}

int fail(const char* what, const std::string& err) {
    std::printf("%s ok=0 err=%s\n", what, err.c_str());
    return 0;
}

}  // namespace

int main(int argc, char** argv) {
    if (argc < 2) return 2;
    const std::string cmd = argv[1];
    std::string err;

    if (cmd == "geom-hash" && argc == 21) {
        std::array<int64_t, 18> g{};
        for (int i = 0; i < 18; ++i) g[(size_t) i] = std::strtoll(argv[3 + i], nullptr, 10);
        std::printf("hash=%016llx\n", (unsigned long long) handoff_geom_hash(g, argv[2]));
        return 0;
    }
    if (cmd == "split-spec" && argc >= 5 && (argc - 5) % 2 == 0) {
        HandoffSplit s;
        s.main_lo = std::strtoll(argv[2], nullptr, 10);
        s.main_hi = std::strtoll(argv[3], nullptr, 10);
        s.draft_on_last = std::atoi(argv[4]) != 0;
        for (int i = 5; i + 1 < argc; i += 2)
            s.stages.push_back({std::strtoll(argv[i], nullptr, 10), std::strtoll(argv[i + 1], nullptr, 10)});
        std::printf("spec=%s\n", handoff_split_spec(s).c_str());
        return 0;
    }
    if (cmd == "path" && argc == 6) {
        std::printf("path=%s\n", handoff_arena_path(argv[2], hexarg(argv[3]), argv[4], argv[5]).c_str());
        return 0;
    }
    if (cmd == "size" && argc == 4) {
        HandoffSizing s;
        if (!sizing(argv[2], argv[3], s, err)) return fail("SIZE", err);
        for (size_t i = 0; i < s.tiers.size(); ++i)
            std::printf("tier=%zu payload=%llu slot_bytes=%llu slot_off=%llu\n", i,
                        (unsigned long long) s.payload_bytes[i], (unsigned long long) s.slot_bytes[i],
                        (unsigned long long) s.slot_off[i]);
        std::printf("SIZE ok=1 arena=%llu total=%llu max=%llu describe=%s\n", (unsigned long long) s.arena_bytes,
                    (unsigned long long) s.slot_total, (unsigned long long) s.max_tokens, s.describe.c_str());
        return 0;
    }
    if ((cmd == "create" || cmd == "hold") && argc == 7) {
        HandoffSizing s;
        if (!sizing(argv[5], argv[6], s, err)) return fail("SIZE", err);
        HandoffArena a;
        if (!a.open_writer(argv[2], s, hexarg(argv[3]), hexarg(argv[4]), err)) return fail("OPEN", err);
        std::printf("OPEN ok=1 free=%s describe=%s\n", a.free_slots().c_str(), a.describe().c_str());
        if (cmd == "hold") {
            std::printf("HELD pid=%d\n", (int) getpid());
            std::fflush(stdout);
            char line[64];
            if (!std::fgets(line, sizeof line, stdin)) {}
        }
        return 0;
    }
    if (cmd == "write" && argc == 14) {
        HandoffSizing s;
        if (!sizing(argv[5], argv[6], s, err)) return fail("SIZE", err);
        HandoffArena a;
        a.set_lease_ms(600000);
        if (!a.open_writer(argv[2], s, hexarg(argv[3]), hexarg(argv[4]), err, std::atoi(argv[13]) != 0))
            return fail("OPEN", err);
        std::printf("OPEN ok=1\n");
        HandoffClaim c;
        if (!a.claim((uint32_t) decarg(argv[7]), decarg(argv[8]), decarg(argv[9]), c, err)) return fail("CLAIM", err);
        std::printf("CLAIM ok=1 slot=%d tier=%u nonce=%016llx base=%llu capacity=%llu\n", c.index, c.tier,
                    (unsigned long long) c.nonce, (unsigned long long) c.base, (unsigned long long) c.capacity);
        const uint64_t bytes = decarg(argv[10]), seed = decarg(argv[11]);
        std::vector<uint8_t> payload(bytes);
        for (uint64_t i = 0; i < bytes; ++i) payload[i] = pattern(i, seed);
        // in pieces, so a payload crosses several write calls as a producer's would
        const uint64_t piece = (1u << 20) + 7;
        for (uint64_t off = 0; off < bytes; off += piece) {
            const uint64_t n = bytes - off < piece ? bytes - off : piece;
            if (!a.write_payload(c, off, payload.data() + off, n, err)) return fail("WRITE", err);
        }
        const uint64_t h = fnv1a64(payload.data(), bytes);
        if (!a.publish(c, decarg(argv[12]), bytes, h, err)) return fail("PUBLISH", err);
        std::printf("PUBLISH ok=1 hash=%016llx\n", (unsigned long long) h);
        return 0;
    }
    if (cmd == "read" && argc == 9) {
        HandoffArena r;
        if (!r.open_reader(argv[2], hexarg(argv[3]), hexarg(argv[4]), err)) return fail("OPEN", err);
        HandoffPayload p;
        if (!r.read_slot(std::atoi(argv[5]), hexarg(argv[6]), decarg(argv[7]), p, err)) return fail("READ", err);
        const uint64_t seed = decarg(argv[8]);
        bool same = true;
        for (uint64_t i = 0; i < p.payload_bytes && same; ++i) same = p.data[i] == pattern(i, seed);
        const uint64_t h = HandoffArena::payload_hash_of(p);
        std::printf("READ ok=1 bytes=%llu tokens=%llu request=%llu tier=%u hash=%016llx recorded=%016llx pattern=%d\n",
                    (unsigned long long) p.payload_bytes, (unsigned long long) p.tokens,
                    (unsigned long long) p.request_id, p.tier, (unsigned long long) h,
                    (unsigned long long) p.payload_hash, (int) same);
        return 0;
    }
    if (cmd == "time" && argc == 9) {
        HandoffSizing s;
        if (!sizing(argv[5], argv[6], s, err)) return fail("SIZE", err);
        HandoffArena a, r;
        a.set_lease_ms(600000);
        if (!a.open_writer(argv[2], s, hexarg(argv[3]), hexarg(argv[4]), err)) return fail("OPEN", err);
        if (!r.open_reader(argv[2], hexarg(argv[3]), hexarg(argv[4]), err)) return fail("OPEN", err);
        const uint64_t bytes = decarg(argv[7]);
        const int reps = std::atoi(argv[8]) > 0 ? std::atoi(argv[8]) : 1;
        std::vector<uint8_t> payload(bytes);
        for (uint64_t i = 0; i < bytes; ++i) payload[i] = pattern(i, 3);
        double best_w = 1e30, best_r = 1e30;
        for (int rep = 0; rep < reps; ++rep) {
            HandoffClaim c;
            if (!a.claim(0, 1, uint64_t(rep), c, err)) return fail("CLAIM", err);
            const auto t0 = std::chrono::steady_clock::now();
            if (!a.write_payload(c, 0, payload.data(), bytes, err)) return fail("WRITE", err);
            const uint64_t h = fnv1a64(payload.data(), bytes);
            if (!a.publish(c, 1, bytes, h, err)) return fail("PUBLISH", err);
            const auto t1 = std::chrono::steady_clock::now();
            HandoffPayload p;
            if (!r.read_slot(c.index, c.nonce, 1, p, err)) return fail("READ", err);
            const uint64_t got = HandoffArena::payload_hash_of(p);
            const auto t2 = std::chrono::steady_clock::now();
            if (got != h) return fail("READ", "hash mismatch");
            if (!a.release(c.index, c.nonce, err)) return fail("RELEASE", err);
            best_w = std::min(best_w, std::chrono::duration<double>(t1 - t0).count());
            best_r = std::min(best_r, std::chrono::duration<double>(t2 - t1).count());
        }
        std::printf("TIME ok=1 bytes=%llu write_s=%.6f read_s=%.6f\n", (unsigned long long) bytes, best_w, best_r);
        return 0;
    }
    if (cmd == "info" && argc == 6) {
        HandoffArena r;
        if (!r.open_reader(argv[2], hexarg(argv[3]), hexarg(argv[4]), err)) return fail("OPEN", err);
        HandoffSlotInfo i;
        if (!r.slot_info(std::atoi(argv[5]), i)) return fail("INFO", "no such slot");
        std::printf("INFO ok=1 base=%llu capacity=%llu state=%u flags=%u tier=%u client=%llu request=%llu "
                    "pack=%016llx geom=%016llx tokens=%llu bytes=%llu hash=%016llx seq=%llu owner=%llu nonce=%016llx\n",
                    (unsigned long long) i.base, (unsigned long long) i.capacity, i.state, i.flags, i.tier,
                    (unsigned long long) i.client_id, (unsigned long long) i.request_id,
                    (unsigned long long) i.pack_hash, (unsigned long long) i.geom_hash, (unsigned long long) i.tokens,
                    (unsigned long long) i.payload_bytes, (unsigned long long) i.payload_hash,
                    (unsigned long long) i.seq, (unsigned long long) i.owner_pid, (unsigned long long) i.nonce);
        return 0;
    }
    std::fprintf(stderr, "usage: see the header of ref_arena_driver.cpp\n");
    return 2;
}

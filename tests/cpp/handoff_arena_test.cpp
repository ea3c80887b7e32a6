// handoff_arena_test.cpp - CPU test of the hand-off arena (strata-concurrent_amd/host/src/handoff.cpp).
//
// The scenarios are the ones the reference's own test covers (src/core/handoff_arena_test.cpp: the file layout, the
// identity helpers, sizing, the slot life cycle, the publish order under a racing reader, tier preference, ownership,
// dead and recycled claimers, leases, refusals, a slot's own identity, the free-space check, several processes, a
// slot over 1 GiB, a restarted writer), written here with fork()ed children instead of re-executing the binary, plus
// this library's additions (the writer's mapped window and reserve()).  The layout table below restates every offset
// from the protocol's description, independently of handoff.hpp's constants.
//
// Arenas live under /dev/shm/sc-handoff-test-<pid>/, which this program creates and removes; nothing else is touched.
#include "strata/core/handoff.hpp"

#include <atomic>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <filesystem>
#include <string>
#include <thread>
#include <vector>

#include <fcntl.h>
#include <sys/file.h>
#include <sys/stat.h>
#include <sys/statvfs.h>
#include <sys/wait.h>
#include <unistd.h>

using namespace strata::core;

namespace {

int g_checks = 0, g_failed = 0;

void expect(bool ok, const std::string& what, const std::string& detail = "") {
    ++g_checks;
    if (!ok) ++g_failed;
    std::printf("  %s %s%s%s\n", ok ? "ok  " : "FAIL", what.c_str(), detail.empty() ? "" : " :: ", detail.c_str());
}

bool has(const std::string& s, const std::string& part) { return s.find(part) != std::string::npos; }

std::string hex(uint64_t v) {
    char b[20];
    std::snprintf(b, sizeof b, "%016llx", (unsigned long long) v);
    return b;
}

std::string g_root;
std::string arena(const std::string& tag) { return g_root + "/" + tag + "/arena"; }
void drop(const std::string& path) {
    std::error_code ec;
    std::filesystem::remove_all(std::filesystem::path(path).parent_path(), ec);
}

/// The payload size a tier is priced at: a fixed part plus a per-token part (the shape of the engine's pricing).
bool pricer(uint64_t tokens, uint64_t& bytes, std::string& err) {
    if (tokens == 0) { err = "a tier of 0 tokens"; return false; }
    bytes = (200ull << 20) + tokens * 20000ull + 5;   // + 5: the rounding to 64 bytes must show
    return true;
}

HandoffSizing sized(const std::vector<HandoffTierSpec>& tiers) {
    HandoffSizing s;
    std::string err;
    if (!handoff_size_arena(tiers, pricer, s, err)) {
        std::fprintf(stderr, "sizing failed: %s\n", err.c_str());
        std::exit(2);
    }
    return s;
}
HandoffSizing three_by_two() { return sized({{1024, 2}, {4096, 2}, {16384, 2}}); }
HandoffSizing one_slot() { return sized({{1024, 1}}); }

bool poke(const std::string& path, uint64_t off, const void* data, uint64_t n) {
    const int fd = ::open(path.c_str(), O_RDWR);
    if (fd < 0) return false;
    const bool ok = ::pwrite(fd, data, n, (off_t) off) == (ssize_t) n;
    ::close(fd);
    return ok;
}

/// A slot header the API cannot produce, written straight into the file (what a crash leaves behind).
void forge(const std::string& path, uint64_t base, uint32_t state, uint64_t pid, uint64_t start, uint64_t nonce,
           uint64_t client, uint64_t pack, uint64_t geom, uint64_t bytes, uint64_t seq) {
    HandoffSlotHeader h{};
    std::memcpy(h.magic, "STRATA-HSLOT-V1", 16);
    h.version = 1;
    h.header_bytes = 4096;
    h.state = state;
    h.owner_pid = pid;
    h.owner_start = start;
    h.nonce = nonce;
    h.client_id = client;
    h.pack_hash = pack;
    h.geom_hash = geom;
    h.payload_bytes = bytes;
    h.claimed_ms = h.published_ms = handoff_now_ms();
    h.seq = seq;
    poke(path, base, &h, sizeof h);
}

uint64_t reaped_pid() {
    const pid_t p = ::fork();
    if (p == 0) _exit(0);
    int st = 0;
    ::waitpid(p, &st, 0);
    return (uint64_t) p;
}

/// Runs `fn` in a forked child and returns what it wrote to the pipe (the child exits when fn returns).
template <class F>
std::string in_child(F fn) {
    int fds[2];
    if (::pipe(fds) != 0) return "pipe failed";
    std::fflush(stdout);
    const pid_t p = ::fork();
    if (p == 0) {
        ::close(fds[0]);
        const std::string out = fn();
        if (::write(fds[1], out.data(), out.size()) < 0) {}
        ::close(fds[1]);
        _exit(0);
    }
    ::close(fds[1]);
    std::string out;
    char buf[512];
    ssize_t n;
    while ((n = ::read(fds[0], buf, sizeof buf)) > 0) out.append(buf, (size_t) n);
    ::close(fds[0]);
    int st = 0;
    ::waitpid(p, &st, 0);
    return out;
}

const uint64_t kPack = 0x0A1B2C3D4E5F6071ull;

}  // namespace

int main() {
    char root[96];
    std::snprintf(root, sizeof root, "/dev/shm/sc-handoff-test-%d", (int) getpid());
    g_root = root;
    std::filesystem::create_directories(g_root);
    std::array<int64_t, 18> key{};
    for (int i = 0; i < 18; ++i) key[(size_t) i] = 10 + 3 * i;
    const uint64_t geom = handoff_geom_hash(key, "main=0..48||n=1|draft=main");

    std::printf("layout\n");
    {
        // the protocol's table, restated: name, offset in the file, offset as the struct lays it out
        struct Row { const char* name; uint64_t doc, have; };
        const Row rows[] = {
            {"arena.version", 16, offsetof(HandoffArenaHeader, version)},
            {"arena.header_bytes", 20, offsetof(HandoffArenaHeader, header_bytes)},
            {"arena.tier_count", 24, offsetof(HandoffArenaHeader, tier_count)},
            {"arena.slot_total", 32, offsetof(HandoffArenaHeader, slot_total)},
            {"arena.arena_bytes", 40, offsetof(HandoffArenaHeader, arena_bytes)},
            {"arena.pack_hash", 48, offsetof(HandoffArenaHeader, pack_hash)},
            {"arena.geom_hash", 56, offsetof(HandoffArenaHeader, geom_hash)},
            {"arena.created_pid", 64, offsetof(HandoffArenaHeader, created_pid)},
            {"arena.created_start", 72, offsetof(HandoffArenaHeader, created_start)},
            {"arena.tier_max_tokens", 80, offsetof(HandoffArenaHeader, tier_max_tokens)},
            {"arena.tier_slot_count", 144, offsetof(HandoffArenaHeader, tier_slot_count)},
            {"arena.tier_slot_bytes", 208, offsetof(HandoffArenaHeader, tier_slot_bytes)},
            {"arena.tier_slot_off", 272, offsetof(HandoffArenaHeader, tier_slot_off)},
            {"arena.reserved", 336, offsetof(HandoffArenaHeader, reserved)},
            {"slot.version", 16, offsetof(HandoffSlotHeader, version)},
            {"slot.header_bytes", 20, offsetof(HandoffSlotHeader, header_bytes)},
            {"slot.state", 24, offsetof(HandoffSlotHeader, state)},
            {"slot.flags", 28, offsetof(HandoffSlotHeader, flags)},
            {"slot.tier", 32, offsetof(HandoffSlotHeader, tier)},
            {"slot.owner_pid", 40, offsetof(HandoffSlotHeader, owner_pid)},
            {"slot.owner_start", 48, offsetof(HandoffSlotHeader, owner_start)},
            {"slot.nonce", 56, offsetof(HandoffSlotHeader, nonce)},
            {"slot.client_id", 64, offsetof(HandoffSlotHeader, client_id)},
            {"slot.request_id", 72, offsetof(HandoffSlotHeader, request_id)},
            {"slot.pack_hash", 80, offsetof(HandoffSlotHeader, pack_hash)},
            {"slot.geom_hash", 88, offsetof(HandoffSlotHeader, geom_hash)},
            {"slot.tokens", 96, offsetof(HandoffSlotHeader, tokens)},
            {"slot.payload_bytes", 104, offsetof(HandoffSlotHeader, payload_bytes)},
            {"slot.payload_hash", 112, offsetof(HandoffSlotHeader, payload_hash)},
            {"slot.claimed_ms", 120, offsetof(HandoffSlotHeader, claimed_ms)},
            {"slot.published_ms", 128, offsetof(HandoffSlotHeader, published_ms)},
            {"slot.seq", 136, offsetof(HandoffSlotHeader, seq)},
            {"slot.reserved", 144, offsetof(HandoffSlotHeader, reserved)},
        };
        std::string bad;
        for (const Row& r : rows)
            if (r.doc != r.have) bad += std::string(r.name) + " ";
        expect(bad.empty(), "every header field sits at the protocol's offset", bad);
        expect(kSlotStateOffset == 24 && kSlotFlagsOffset == 28 && kSlotPublishStateBytes == 8,
               "the publish point is the 8 bytes of state and flags at 24");
        expect(kSlotPublishBlockOffset == 96 && kSlotPublishBlockBytes == 48, "the payload record is [96,144)");
        expect(kHandoffFree == 0 && kHandoffClaimed == 1 && kHandoffReady == 2 && kHandoffFlagCancelled == 1 &&
                   kHandoffFlagAbandoned == 2 && kHandoffFlagPartial == 4,
               "states 0/1/2 and flag bits 1/2/4");
        expect(kHandoffSlackBytes == 64ull << 20 && kHandoffDefaultLeaseMs == 300000 && kHandoffMaxTiers == 8,
               "64 MiB slack, 300 s lease, 8 tiers");
    }

    std::printf("identity\n");
    {
        HandoffSplit whole;
        whole.main_hi = 48;
        expect(handoff_split_spec(whole) == "main=0..48||n=1|draft=main", "no split", handoff_split_spec(whole));
        HandoffSplit three;
        three.main_hi = 16;
        three.stages = {{16, 34}, {34, 48}};
        expect(handoff_split_spec(three) == "main=0..16|16..34,34..48|n=3|draft=last", "a three-way split",
               handoff_split_spec(three));
        three.draft_on_last = false;
        expect(handoff_split_spec(three) == "main=0..16|16..34,34..48|n=3|draft=main", "the draft on the main stage");
        // the hash is FNV-1a from the engine seed over the salt, 18 little-endian words and the spec, in one stream
        std::vector<uint8_t> stream;
        const char* salt = "strata-handoff-geom-v1";
        stream.insert(stream.end(), salt, salt + std::strlen(salt));
        for (int64_t v : key)
            for (int b = 0; b < 8; ++b) stream.push_back((uint8_t) ((uint64_t) v >> (8 * b)));
        const std::string spec = "main=0..48||n=1|draft=main";
        stream.insert(stream.end(), spec.begin(), spec.end());
        expect(geom == fnv1a64(stream.data(), stream.size()), "the geometry hash is one FNV-1a stream");
        std::array<int64_t, 18> other = key;
        other[11] += 1;
        expect(handoff_geom_hash(other, spec) != geom && handoff_geom_hash(key, spec + "x") != geom,
               "a different geometry word or split gives a different hash");
        const std::string p = handoff_arena_path("/dev/shm/h/", 0xABCull, "main=0..48||n=1|draft=main", "pf-0");
        expect(p == "/dev/shm/h/0000000000000abc-main=0..48||n=1|draft=main/pf-0/arena", "the arena path", p);
        expect(handoff_arena_path("d", 1, "s", "") == "d/0000000000000001-s/arena", "no instance component");
    }

    std::printf("sizing\n");
    {
        const HandoffSizing s = three_by_two();
        uint64_t off = 4096;
        bool ok = true;
        for (size_t i = 0; i < 3; ++i) {
            const uint64_t priced = (200ull << 20) + s.tiers[i].max_tokens * 20000ull + 5;
            ok = ok && s.payload_bytes[i] == priced && s.slot_bytes[i] == ((priced + 63) / 64) * 64 + (64ull << 20) &&
                 s.slot_off[i] == off;
            off += 2 * (4096 + s.slot_bytes[i]);
        }
        expect(ok, "payload, slot bytes (64-byte rounding + 64 MiB) and group offsets");
        expect(s.arena_bytes == off && s.slot_total == 6 && s.max_tokens == 16384, "arena bytes, slot total, max");
        expect(has(s.describe, "slots 2,2,2 (tiers 1024,4096,16384), max 16384 tokens, arena ") &&
                   has(s.describe, "(" + std::to_string(s.arena_bytes) + " B)"),
               "the start-up figure", s.describe);
        HandoffSizing bad;
        std::string err;
        expect(!handoff_size_arena({}, pricer, bad, err) && has(err, "no tiers"), "no tiers", err);
        expect(!handoff_size_arena({{4096, 1}, {1024, 1}}, pricer, bad, err) && has(err, "ascend"), "descending", err);
        expect(!handoff_size_arena({{4096, 1}, {4096, 1}}, pricer, bad, err) && has(err, "ascend"), "a repeated tier", err);
        expect(!handoff_size_arena({{1024, 0}}, pricer, bad, err) && has(err, "0 slots"), "a tier of 0 slots", err);
        expect(!handoff_size_arena({{0, 1}}, pricer, bad, err) && has(err, "0 tokens"), "a tier of 0 tokens", err);
        std::vector<HandoffTierSpec> nine;
        for (uint64_t i = 1; i <= 9; ++i) nine.push_back({i * 100, 1});
        expect(!handoff_size_arena(nine, pricer, bad, err) && has(err, "9 tiers"), "nine tiers", err);
        expect(!handoff_size_arena({{1024, 1}}, std::vector<uint64_t>{}, bad, err) && has(err, "priced"),
               "a priced list of the wrong length", err);
        expect(!handoff_size_arena({{1024, 1}}, [](uint64_t, uint64_t&, std::string& e) { e = "pricer broke"; return false; },
                                   bad, err) && has(err, "pricer broke"),
               "the pricer's own reason", err);
        expect(!handoff_size_arena({{1024, 1}}, std::vector<uint64_t>{UINT64_MAX - 10}, bad, err), "a size that overflows");
    }

    const std::string main_path = arena("main");
    std::printf("create\n");
    {
        const HandoffSizing s = three_by_two();
        HandoffArena a;
        std::string err;
        expect(a.open_writer(main_path, s, kPack, geom, err), "the writer creates the arena", err);
        struct stat st {};
        expect(::stat(main_path.c_str(), &st) == 0 && (uint64_t) st.st_size == s.arena_bytes, "the file is arena_bytes");
        expect(a.is_writer() && a.tier_count() == 3 && a.slot_total() == 6 && a.max_tokens() == 16384 &&
                   a.tier_slot_off(1) == s.slot_off[1] && a.tier_slot_bytes(2) == s.slot_bytes[2] &&
                   a.tier_slot_count(0) == 2 && a.tier_max_tokens(1) == 4096,
               "the header's tables");
        expect(a.header().created_pid == (uint64_t) getpid() && a.header().created_start != 0, "the creator and its start");
        expect(has(a.describe(), hex(kPack)) && has(a.describe(), hex(geom)), "describe names both hashes", a.describe());
        expect(a.free_slots() == "6/6", "every slot free");
        HandoffSlotInfo i, none;
        expect(a.slot_info(3, i) && i.tier == 1 && i.state == kHandoffFree && i.base == s.slot_off[1] + 4096 + s.slot_bytes[1],
               "slot 3 is the second slot of group 1");
        expect(!a.slot_info(6, none) && !a.slot_info(-1, none), "no slot 6, no slot -1");
        // the raw file: magic bytes, and a FREE slot header with its tier
        char magic[16];
        const int fd = ::open(main_path.c_str(), O_RDONLY);
        expect(::pread(fd, magic, 16, 0) == 16 && std::memcmp(magic, "STRATA-HARENA-V1", 16) == 0, "the arena magic");
        HandoffSlotHeader sh{};
        expect(::pread(fd, &sh, sizeof sh, (off_t) i.base) == sizeof sh && std::memcmp(sh.magic, "STRATA-HSLOT-V1", 16) == 0 &&
                   sh.version == 1 && sh.header_bytes == 4096 && sh.tier == 1,
               "a slot header as the protocol writes it");
        ::close(fd);
        // a live foreign creator: our parent process
        const uint64_t ppid = (uint64_t) getppid(), pstart = handoff_proc_start_time(ppid);
        poke(main_path, kArenaCreatedPidOffset, &ppid, 8);
        poke(main_path, kArenaCreatedStartOffset, &pstart, 8);
        HandoffArena second;
        expect(!second.open_writer(main_path, s, kPack, geom, err) && has(err, "one arena per prefill instance") &&
                   has(err, std::to_string(ppid)),
               "a second writer beside a live creator is refused", err);
        const uint64_t me = (uint64_t) getpid(), mstart = handoff_proc_start_time(me);
        poke(main_path, kArenaCreatedPidOffset, &me, 8);
        poke(main_path, kArenaCreatedStartOffset, &mstart, 8);
        const HandoffSizing other = sized({{1024, 3}, {4096, 2}, {16384, 2}});
        HandoffArena resized;
        expect(!resized.open_writer(main_path, other, kPack, geom, err) && has(err, std::to_string(other.arena_bytes)) &&
                   has(err, std::to_string(s.arena_bytes)),
               "a different size names both sizes", err);
        expect(!a.open_writer(main_path, s, 0, geom, err) && has(err, "pack hash") && !a.valid(), "pack hash 0", err);
        expect(!a.open_writer(main_path, s, kPack, 0, err) && has(err, "geometry hash"), "geometry hash 0", err);
    }

    std::printf("lifecycle\n");
    {
        const HandoffSizing s = three_by_two();
        HandoffArena a;
        std::string err;
        expect(a.open_writer(main_path, s, kPack, geom, err), "this process re-opens its own arena", err);
        HandoffClaim c;
        expect(a.claim(0, 0x51, 9, c, err) && c.index == 0 && c.tier == 0 && c.base == s.slot_off[0] &&
                   c.payload_off == c.base + 4096 && c.capacity == s.slot_bytes[0] && c.nonce != 0,
               "a tier-0 claim takes slot 0", err);
        HandoffSlotInfo i;
        expect(a.slot_info(0, i) && i.state == kHandoffClaimed && i.owner_pid == (uint64_t) getpid() && i.owner_start != 0 &&
                   i.client_id == 0x51 && i.request_id == 9 && i.pack_hash == kPack && i.geom_hash == geom &&
                   i.payload_bytes == 0 && i.published_ms == 0 && i.nonce == c.nonce && i.claimed_ms != 0,
               "the claim's header");
        std::vector<uint8_t> body(3u << 20);
        for (size_t k = 0; k < body.size(); ++k) body[k] = (uint8_t) (k * 29u + (k >> 11));
        expect(a.write_payload(c, 0, body.data(), body.size() / 2, err) &&
                   a.write_payload(c, body.size() / 2, body.data() + body.size() / 2, body.size() - body.size() / 2, err),
               "the payload in two writes", err);
        HandoffArena r;
        expect(r.open_reader(main_path, kPack, geom, err) && !r.is_writer(), "a reader opens", err);
        HandoffPayload p;
        expect(!r.read_slot(0, c.nonce, 0x51, p, err) && has(err, "CLAIMED") && !p.valid(), "an unpublished slot", err);
        const uint64_t h = fnv1a64(body.data(), body.size());
        expect(a.publish(c, 777, body.size(), h, err), "publish", err);
        expect(a.slot_info(0, i) && i.state == kHandoffReady && i.tokens == 777 && i.payload_bytes == body.size() &&
                   i.payload_hash == h && i.seq == 1 && i.published_ms >= i.claimed_ms && i.flags == 0,
               "the published header");
        expect(r.read_slot(0, c.nonce, 0x51, p, err) && p.valid() && p.payload_bytes == body.size() &&
                   std::memcmp(p.data, body.data(), body.size()) == 0 && HandoffArena::payload_hash_of(p) == h &&
                   p.tokens == 777 && p.request_id == 9 && p.nonce == c.nonce && p.tier == 0 && p.seq == 1,
               "the reader maps the payload", err);
        HandoffPayload q;
        expect(!r.read_slot(0, c.nonce, 0x52, q, err) && has(err, "addressed to client"), "another client", err);
        expect(!r.read_slot(0, c.nonce + 1, 0x51, q, err) && has(err, "nonce"), "another nonce", err);
        expect(!r.read_slot(1, c.nonce, 0x51, q, err) && has(err, "FREE"), "another slot", err);
        HandoffPayload moved = std::move(p);
        expect(moved.valid() && !p.valid() && moved.data[5] == body[5], "a payload moves");
        expect(a.release(0, c.nonce, err), "the ACK releases", err);
        expect(a.slot_info(0, i) && i.state == kHandoffFree && i.owner_pid == 0 && i.owner_start == 0 && i.nonce == 0 &&
                   i.client_id == 0 && i.payload_bytes == 0 && i.flags == 0,
               "release clears the claim");
        expect(moved.data[5] == body[5], "the body stays where it was after release (a mapping still reads it)");
        expect(!a.release(0, c.nonce, err) && has(err, "nonce"), "a stale release", err);
        expect(a.free_slots() == "6/6", "all free again");
    }

    std::printf("publish-order\n");
    {
        const std::string path = arena("race");
        HandoffArena a;
        std::string err;
        expect(a.open_writer(path, one_slot(), kPack, geom, err), "a one-slot arena", err);
        std::atomic<int> bad{0}, seen{0};
        int published = 0;
        std::vector<uint8_t> body(8192);
        for (uint64_t round = 0; round < 120; ++round) {
            for (size_t k = 0; k < body.size(); ++k) body[k] = (uint8_t) (k ^ (round * 13));
            const uint64_t h = fnv1a64(body.data(), body.size());
            HandoffClaim c;
            if (!a.claim(0, 7, round, c, err) || !a.write_payload(c, 0, body.data(), body.size(), err)) break;
            std::atomic<bool> stop{false};
            std::thread reader([&] {
                HandoffArena r;
                std::string e;
                if (!r.open_reader(path, kPack, geom, e)) { ++bad; return; }
                while (!stop.load()) {
                    HandoffPayload p;
                    if (!r.read_slot(c.index, c.nonce, 7, p, e)) continue;
                    ++seen;
                    if (p.tokens != round + 5 || p.payload_bytes != body.size() || p.payload_hash != h ||
                        HandoffArena::payload_hash_of(p) != h)
                        ++bad;
                }
            });
            std::this_thread::sleep_for(std::chrono::microseconds(100));
            const int before = seen.load();
            if (a.publish(c, round + 5, body.size(), h, err)) ++published;
            // let the reader see the READY slot at least once (a loaded machine may not schedule it for a while)
            const auto t_pub = std::chrono::steady_clock::now();
            while (seen.load() == before && std::chrono::steady_clock::now() - t_pub < std::chrono::seconds(2))
                std::this_thread::sleep_for(std::chrono::microseconds(50));
            std::this_thread::sleep_for(std::chrono::microseconds(200));
            stop = true;
            reader.join();
            a.release(c.index, c.nonce, err);
        }
        expect(published == 120, "every round published");
        expect(seen.load() >= 120, "the racing reader saw every round's READY slot", std::to_string(seen.load()) + " reads");
        expect(bad.load() == 0, "no read saw READY with a stale record or body");
        drop(path);
    }

    std::printf("tiers\n");
    {
        const HandoffSizing s = three_by_two();
        HandoffArena a;
        std::string err;
        a.open_writer(main_path, s, kPack, geom, err);
        HandoffClaim b1, b2, none, c[4];
        expect(a.claim(2, 1, 1, b1, err) && a.claim(2, 1, 2, b2, err) && b1.index == 4 && b2.index == 5 && b2.tier == 2,
               "tier-2 jobs take group 2");
        expect(!a.claim(2, 1, 3, none, err) && has(err, "no free handoff slot") && has(err, "4/6") && none.index == -1 &&
                   none.nonce == 0,
               "a tier-2 job never takes a smaller group", err);
        const int want_index[4] = {0, 1, 2, 3};
        const uint32_t want_tier[4] = {0, 0, 1, 1};
        bool ok = true;
        for (int k = 0; k < 4; ++k)
            ok = ok && a.claim(0, 1, 10 + k, c[k], err) && c[k].index == want_index[k] && c[k].tier == want_tier[k] &&
                 c[k].capacity == s.slot_bytes[want_tier[k]];
        expect(ok, "tier-0 jobs fill group 0, then the smallest larger group", err);
        expect(!a.claim(0, 1, 20, none, err) && has(err, "0/6"), "a full arena", err);
        ok = true;
        for (HandoffClaim* x : {&c[0], &c[1], &c[2], &c[3], &b1, &b2}) ok = ok && a.release(x->index, x->nonce, err);
        expect(ok && a.free_slots() == "6/6", "every claim releases");
        expect(!a.claim(3, 1, 1, none, err) && has(err, "not in this arena"), "tier 3 of 3", err);
    }

    std::printf("ownership\n");
    {
        HandoffArena a;
        std::string err;
        a.open_writer(main_path, three_by_two(), kPack, geom, err);
        HandoffClaim c, d;
        expect(a.claim(0, 1, 1, c, err) && a.cancel(c.index, c.nonce, err), "claim and cancel", err);
        expect(!a.publish(c, 1, 16, 1, err) && has(err, "cancelled"), "a cancelled job does not publish", err);
        HandoffSlotInfo i;
        expect(a.abort_claim(c.index, c.nonce, err) && a.slot_info(c.index, i) && i.state == kHandoffFree &&
                   (i.flags & kHandoffFlagPartial),
               "abort frees the slot with the partial flag", err);
        expect(!a.abort_claim(c.index, c.nonce, err), "a FREE slot cannot be aborted");
        expect(a.claim(0, 1, 2, d, err), "claim again", err);
        HandoffClaim stale = d;
        stale.nonce ^= 0x77;
        expect(!a.publish(stale, 1, 16, 1, err) && has(err, "claim is gone"), "a stale nonce does not publish", err);
        expect(!a.cancel(stale.index, stale.nonce, err) && !a.release(stale.index, stale.nonce, err), "nor cancel or release");
        std::vector<uint8_t> blob(4096, 1);
        expect(!a.write_payload(d, d.capacity - 100, blob.data(), blob.size(), err) && has(err, std::to_string(d.capacity)) &&
                   has(err, std::to_string(d.capacity - 100 + 4096)),
               "a write past the slot names both numbers", err);
        expect(!a.publish(d, 1, d.capacity + 1, 1, err) && has(err, std::to_string(d.capacity)), "a payload past the slot", err);
        HandoffClaim forged = d;
        forged.base += 64;
        expect(!a.write_payload(forged, 0, blob.data(), 16, err) && has(err, "slot table"), "a claim that is not a slot", err);
        a.abort_claim(d.index, d.nonce, err);
        HandoffArena r;
        r.open_reader(main_path, kPack, geom, err);
        HandoffClaim rc;
        expect(!r.claim(0, 1, 1, rc, err) && has(err, "reader never claims"), "a reader does not claim", err);
        expect(!r.write_payload(d, 0, blob.data(), 16, err) && !r.publish(d, 1, 16, 1, err) && !r.release(0, 1, err) &&
                   !r.abort_claim(0, 1, err) && !r.cancel(0, 1, err) && !r.claim_window(d, err),
               "nor write, publish, release, abort, cancel or map a claim");
        HandoffPayload p;
        expect(!a.read_slot(0, 1, 1, p, err) && has(err, "as a reader"), "a writer does not read slots", err);
    }

    std::printf("dead-owner\n");
    {
        const HandoffSizing s = three_by_two();
        HandoffArena a;
        std::string err;
        a.open_writer(main_path, s, kPack, geom, err);
        forge(main_path, s.slot_off[0], kHandoffClaimed, reaped_pid(), 0, 0x99, 5, kPack, geom, 0, 0);
        expect(a.free_slots() == "5/6", "a dead claim is not free");
        const auto took = a.reclaim(&err);
        expect(took.size() == 1 && took[0].index == 0 && took[0].was_state == kHandoffClaimed && has(took[0].why, "gone") &&
                   took[0].nonce == 0x99,
               "reclaim takes it and says why", took.empty() ? "" : took[0].why);
        HandoffSlotInfo i;
        expect(a.slot_info(0, i) && i.state == kHandoffFree && (i.flags & kHandoffFlagAbandoned), "FREE, flagged abandoned");
        HandoffClaim live, other, over;
        expect(a.claim(0, 1, 1, live, err) && a.reclaim(&err).empty(), "a live claim is left alone");
        expect(a.claim(0, 1, 2, other, err) && other.index != live.index, "and is never taken by another claim");
        forge(main_path, s.slot_off[0] + 4096 + s.slot_bytes[0], kHandoffClaimed, reaped_pid(), 0, 0x98, 5, kPack, geom, 0, 0);
        expect(a.claim(0, 1, 3, over, err) && over.index == 1 && over.nonce != 0x98, "claim takes over a dead claim itself", err);
        for (HandoffClaim* x : {&live, &over}) a.release(x->index, x->nonce, err);
    }

    std::printf("recycled-pid\n");
    {
        const HandoffSizing s = three_by_two();
        HandoffArena a;
        std::string err;
        a.open_writer(main_path, s, kPack, geom, err);
        const uint64_t me = (uint64_t) getpid(), start = handoff_proc_start_time(me);
        expect(handoff_pid_alive(me) && start != 0 && handoff_claim_alive(me, start) && !handoff_claim_alive(me, start + 1) &&
                   handoff_claim_alive(me, 0),
               "liveness: pid plus start time, unknown start means alive");
        expect(!handoff_pid_alive(0) && handoff_proc_start_time(0) == 0 && !handoff_pid_alive(1ull << 40), "pid 0 and absurd pids");
        expect(!handoff_pid_alive(reaped_pid()), "a reaped child is dead");
        forge(main_path, s.slot_off[1], kHandoffClaimed, me, start ^ 0x5A5A, 0x97, 5, kPack, geom, 0, 0);
        const auto took = a.reclaim(&err);
        expect(took.size() == 1 && took[0].index == 2 && has(took[0].why, "gone"), "a recycled pid is a dead claimer");
        forge(main_path, s.slot_off[1], kHandoffClaimed, me, 0, 0x96, 5, kPack, geom, 0, 0);
        expect(a.reclaim(&err).empty(), "an unknown start time is alive");
        a.abort_claim(2, 0x96, err);
    }

    std::printf("leases\n");
    {
        HandoffArena a;
        std::string err;
        a.open_writer(main_path, three_by_two(), kPack, geom, err);
        // a lease long enough that claim -> publish -> reclaim fits in it on a loaded machine
        a.set_lease_ms(400);
        std::vector<uint8_t> body(1000, 3);
        const uint64_t h = fnv1a64(body.data(), body.size());
        HandoffClaim c;
        expect(a.claim(1, 0xA, 1, c, err) && a.write_payload(c, 0, body.data(), body.size(), err) &&
                   a.publish(c, 1, body.size(), h, err) && a.reclaim(&err).empty(),
               "a fresh READY slot survives a reclaim");
        std::this_thread::sleep_for(std::chrono::milliseconds(480));
        auto took = a.reclaim(&err);
        expect(took.size() == 1 && took[0].was_state == kHandoffReady && has(took[0].why, "lease") && took[0].age_ms >= 400,
               "an unread READY slot is reclaimed at the lease", took.empty() ? "" : took[0].why);
        expect(a.claim(1, 0xA, 2, c, err), "claim again");
        std::this_thread::sleep_for(std::chrono::milliseconds(480));
        took = a.reclaim(&err);
        expect(took.size() == 1 && took[0].was_state == kHandoffClaimed && has(took[0].why, "lease"), "so is a stuck claim");
        a.set_lease_ms(1000000);
        a.note_client_pid(0xB, reaped_pid());
        a.note_client_pid(0xC, (uint64_t) getpid());
        HandoffClaim d, e;
        // both claimed before either is published: claim() itself reclaims, and would take the first one
        expect(a.claim(1, 0xB, 3, d, err) && a.claim(1, 0xC, 4, e, err) && a.publish(d, 1, 0, fnv1a64(nullptr, 0), err) &&
                   a.publish(e, 1, 0, fnv1a64(nullptr, 0), err),
               "two READY slots, one for a dead reader and one for a live one", err);
        took = a.reclaim(&err);
        expect(took.size() == 1 && took[0].client_id == 0xB && has(took[0].why, "reader"), "the dead reader's is reclaimed at once",
               took.empty() ? "" : took[0].why);
        a.release(e.index, e.nonce, err);
        a.set_lease_ms(0);
        HandoffClaim f;
        expect(a.claim(0, 1, 5, f, err) && a.reclaim(&err).size() == 1, "a lease of 0 reclaims at once");
        HandoffArena closed;
        std::string cerr;
        expect(closed.reclaim(&cerr).empty() && has(cerr, "not open"), "reclaim on a closed arena reports");
        ::setenv("STRATA_HANDOFF_LEASE_MS", "1234", 1);
        HandoffArena env;
        expect(env.lease_ms() == 1234, "STRATA_HANDOFF_LEASE_MS sets the default lease");
        ::unsetenv("STRATA_HANDOFF_LEASE_MS");
        HandoffArena dflt;
        expect(dflt.lease_ms() == kHandoffDefaultLeaseMs, "and without it the lease is 300 s");
    }

    std::printf("refusal\n");
    {
        const HandoffSizing s = three_by_two();
        HandoffArena r, w;
        std::string err;
        const uint64_t wrong = kPack ^ 0x1111;
        expect(!r.open_reader(main_path, wrong, geom, err) && has(err, "pack hash") && has(err, hex(kPack)) && has(err, hex(wrong)),
               "a reader's pack mismatch names both hashes", err);
        expect(!r.open_reader(main_path, kPack, geom ^ 4, err) && has(err, "geometry hash") && has(err, hex(geom)) &&
                   has(err, hex(geom ^ 4)),
               "a reader's geometry mismatch names both", err);
        expect(!r.open_reader(g_root + "/absent/arena", kPack, geom, err) && has(err, "cannot open"), "a missing arena", err);
        expect(!w.open_writer(main_path, s, wrong, geom, err) && has(err, "pack hash") && has(err, hex(kPack)), "a writer's pack", err);
        expect(!w.open_writer(main_path, s, kPack, geom ^ 4, err) && has(err, "geometry hash"), "a writer's geometry", err);
        const uint64_t low = s.arena_bytes - 4096;
        poke(main_path, kArenaBytesOffset, &low, 8);
        expect(!r.open_reader(main_path, kPack, geom, err) && has(err, "but its header says"), "a header that disagrees with the file",
               err);
        poke(main_path, kArenaBytesOffset, &s.arena_bytes, 8);
        expect(r.open_reader(main_path, kPack, geom, err), "and reads once it agrees", err);
        HandoffSizing broken = s;
        broken.arena_bytes += 64;
        expect(!w.open_writer(arena("broken"), broken, kPack, geom, err) && has(err, "does not add up") && !w.valid(),
               "a sizing that does not add up", err);
        broken = s;
        broken.slot_off[2] += 4096;
        expect(!w.open_writer(arena("broken"), broken, kPack, geom, err) && has(err, "the layout says"), "a shifted tier", err);
        const std::string vpath = arena("version");
        HandoffArena v;
        expect(v.open_writer(vpath, s, kPack, geom, err), "a second arena");
        const uint32_t two = 2, half = 2048, seven = 9;
        poke(vpath, kArenaVersionOffset, &two, 4);
        expect(!r.open_reader(vpath, kPack, geom, err) && has(err, "version"), "a future version", err);
        const uint32_t one = 1;
        poke(vpath, kArenaVersionOffset, &one, 4);
        poke(vpath, kArenaHeaderBytesOffset, &half, 4);
        expect(!r.open_reader(vpath, kPack, geom, err) && has(err, "header_bytes"), "a 2048-byte header", err);
        const uint32_t full = 4096;
        poke(vpath, kArenaHeaderBytesOffset, &full, 4);
        poke(vpath, kArenaTierCountOffset, &seven, 4);
        expect(!r.open_reader(vpath, kPack, geom, err) && has(err, "9 tiers"), "nine tiers in the header", err);
        poke(vpath, 0, "NOT-AN-ARENA-AT-ALL", 16);
        expect(!r.open_reader(vpath, kPack, geom, err) && has(err, "magic"), "a foreign file", err);
        expect(!v.open_writer(vpath, s, kPack, geom, err) && has(err, "magic"), "the writer does not reuse it either", err);
        drop(vpath);
        drop(arena("broken"));
    }

    std::printf("slot-identity\n");
    {
        const HandoffSizing s = three_by_two();
        HandoffArena a, r;
        std::string err;
        a.open_writer(main_path, s, kPack, geom, err);
        HandoffClaim c;
        std::vector<uint8_t> body(512, 9);
        a.claim(0, 0x77, 1, c, err);
        a.write_payload(c, 0, body.data(), body.size(), err);
        a.publish(c, 1, body.size(), fnv1a64(body.data(), body.size()), err);
        r.open_reader(main_path, kPack, geom, err);
        HandoffPayload p;
        expect(r.read_slot(c.index, c.nonce, 0x77, p, err), "the honest slot reads", err);
        p = HandoffPayload{};
        struct Case { uint64_t pack, geom, bytes, seq; const char* word; const char* what; };
        const Case cases[] = {{kPack ^ 1, geom, 512, 1, "was written for pack", "another pack"},
                              {kPack, geom ^ 1, 512, 1, "geometry", "another geometry"},
                              {kPack, geom, 512, 2, "seq", "seq 2"},
                              {kPack, geom, c.capacity + 1, 1, "in a", "more bytes than the slot holds"}};
        for (const Case& k : cases) {
            forge(main_path, c.base, kHandoffReady, (uint64_t) getpid(), 0, c.nonce, 0x77, k.pack, k.geom, k.bytes, k.seq);
            expect(!r.read_slot(c.index, c.nonce, 0x77, p, err) && has(err, k.word) && !p.valid(), k.what, err);
        }
        poke(main_path, c.base, "NOT-A-SLOT-AT-ALL", 16);
        expect(!r.read_slot(c.index, c.nonce, 0x77, p, err) && has(err, "incompatible header"), "a slot without its magic", err);
        forge(main_path, c.base, kHandoffFree, 0, 0, 0, 0, kPack, geom, 0, 0);
    }

    std::printf("statvfs\n");
    {
        const std::string path = arena("too-big");
        HandoffSizing huge;
        std::string err;
        expect(handoff_size_arena({{131072, 8}}, std::vector<uint64_t>{1ull << 40}, huge, err), "an 8 TiB arena on paper");
        HandoffArena a;
        expect(!a.open_writer(path, huge, kPack, geom, err) && has(err, std::to_string(huge.arena_bytes)) && has(err, "free") &&
                   !std::filesystem::exists(path) && !a.valid(),
               "is refused before any file exists, with both numbers", err);
        expect(a.open_writer(path, one_slot(), kPack, geom, err), "the same path at a sane size", err);
        drop(path);
    }

    std::printf("processes\n");
    {
        const HandoffSizing s = three_by_two();
        std::string err;
        {
            const int f1 = ::open(main_path.c_str(), O_RDONLY), f2 = ::open(main_path.c_str(), O_RDONLY);
            const bool ex = ::flock(f1, LOCK_EX) == 0;
            const bool blocked = ::flock(f2, LOCK_SH | LOCK_NB) != 0;
            ::flock(f1, LOCK_UN);
            ::close(f1);
            ::close(f2);
            expect(ex && blocked, "flock excludes a second open file description");
        }
        // two processes race for the only slot of an arena a third (this one) created
        const std::string cpath = arena("contention");
        HandoffArena owner;
        owner.open_writer(cpath, one_slot(), kPack, geom, err);
        auto racer = [&](uint64_t request) {
            return in_child([&, request] {
                HandoffArena w;
                std::string e;
                if (!w.open_writer(cpath, one_slot(), kPack, geom, e, true)) return "OPEN " + e;
                HandoffClaim c;
                if (!w.claim(0, 42, request, c, e)) return "LOST " + e;
                std::vector<uint8_t> body(4096, (uint8_t) request);
                w.write_payload(c, 0, body.data(), body.size(), e);
                return std::string(w.publish(c, 1, body.size(), fnv1a64(body.data(), body.size()), e) ? "WON " : "PUBFAIL ") +
                       std::to_string(c.index) + " " + hex(c.nonce);
            });
        };
        const std::string r1 = racer(1), r2 = racer(2);
        expect((r1.rfind("WON 0", 0) == 0) != (r2.rfind("WON 0", 0) == 0), "exactly one process gets the only slot",
               "[" + r1 + "] [" + r2 + "]");
        expect(has(r1.rfind("WON", 0) == 0 ? r2 : r1, "no free handoff slot"), "the other is told to wait");
        drop(cpath);
        // a child writes and publishes; this process reads it through the file; a child reads it too
        HandoffArena a;
        a.open_writer(main_path, s, kPack, geom, err);
        const std::string out = in_child([&] {
            HandoffArena w;
            std::string e;
            if (!w.open_writer(main_path, three_by_two(), kPack, geom, e, true)) return "OPEN " + e;
            HandoffClaim c;
            if (!w.claim(1, 314, 15, c, e)) return "CLAIM " + e;
            std::vector<uint8_t> body(100000);
            for (size_t k = 0; k < body.size(); ++k) body[k] = (uint8_t) (k * 7 + 15);
            w.write_payload(c, 0, body.data(), body.size(), e);
            w.publish(c, 2718, body.size(), fnv1a64(body.data(), body.size()), e);
            return std::to_string(c.index) + " " + hex(c.nonce) + " " + hex(fnv1a64(body.data(), body.size()));
        });
        int slot = -1;
        unsigned long long nonce = 0, h = 0;
        expect(std::sscanf(out.c_str(), "%d %llx %llx", &slot, &nonce, &h) == 3 && slot == 2, "a child published in group 1", out);
        HandoffArena r;
        HandoffPayload p;
        bool pattern = r.open_reader(main_path, kPack, geom, err) && r.read_slot(slot, nonce, 314, p, err) && p.tokens == 2718;
        for (uint64_t k = 0; pattern && k < p.payload_bytes; ++k) pattern = p.data[k] == (uint8_t) (k * 7 + 15);
        expect(pattern && HandoffArena::payload_hash_of(p) == h, "this process reads the child's bytes and hash", err);
        const std::string child_read = in_child([&] {
            HandoffArena rr;
            HandoffPayload pp;
            std::string e;
            const bool ok = rr.open_reader(main_path, kPack, geom, e) && rr.read_slot(slot, nonce, 314, pp, e);
            const bool wrong = rr.read_slot(slot, nonce ^ 1, 314, pp, e) || rr.read_slot(slot, nonce, 315, pp, e);
            return std::string(ok ? "READ1 " : "READ0 ") + (wrong ? "WRONG1" : "WRONG0");
        });
        expect(child_read == "READ1 WRONG0", "a reader process reads it and refuses the wrong nonce and client", child_read);
        expect(a.release(slot, nonce, err), "the writer releases a slot another process published", err);
        // a live child's claim is not reclaimed by this writer
        int sync[2];
        if (::pipe(sync) != 0) return 2;
        std::fflush(stdout);
        const pid_t holder = ::fork();
        if (holder == 0) {
            ::close(sync[0]);
            HandoffArena w;
            std::string e;
            HandoffClaim c;
            const bool ok = w.open_writer(main_path, three_by_two(), kPack, geom, e, true) && w.claim(2, 1, 1, c, e);
            const char msg = ok ? (char) ('0' + c.index) : 'x';
            if (::write(sync[1], &msg, 1) < 0) {}
            std::this_thread::sleep_for(std::chrono::milliseconds(800));
            _exit(0);
        }
        ::close(sync[1]);
        char held = 'x';
        if (::read(sync[0], &held, 1) != 1) held = 'x';
        ::close(sync[0]);
        HandoffSlotInfo i;
        expect(held == '4' && a.reclaim(&err).empty() && a.slot_info(4, i) && i.state == kHandoffClaimed &&
                   i.owner_pid == (uint64_t) holder,
               "a live process's claim survives this writer's reclaim");
        int st = 0;
        ::waitpid(holder, &st, 0);
        const auto took = a.reclaim(&err);
        expect(took.size() == 1 && took[0].index == 4 && has(took[0].why, "gone"), "and is reclaimed once it exits");
        // a claim waits for a lock held by another process
        int ready[2];
        if (::pipe(ready) != 0) return 2;
        std::fflush(stdout);
        const pid_t locker = ::fork();
        if (locker == 0) {
            ::close(ready[0]);
            const int fd = ::open(main_path.c_str(), O_RDONLY);
            ::flock(fd, LOCK_EX);
            if (::write(ready[1], "L", 1) < 0) {}
            std::this_thread::sleep_for(std::chrono::milliseconds(400));
            ::flock(fd, LOCK_UN);
            _exit(0);
        }
        ::close(ready[1]);
        char l = 0;
        if (::read(ready[0], &l, 1) != 1) l = 0;
        ::close(ready[0]);
        const uint64_t t0 = handoff_now_ms();
        HandoffClaim waited;
        const bool got = a.claim(0, 1, 1, waited, err);
        const uint64_t dt = handoff_now_ms() - t0;
        ::waitpid(locker, &st, 0);
        expect(l == 'L' && got && dt >= 300, "a claim waits for another process's lock", std::to_string(dt) + " ms");
        a.release(waited.index, waited.nonce, err);
    }

    std::printf("window\n");
    {
        // this library's additions: the writer's mapped window into a claimed slot, and reserve()
        const std::string path = arena("window");
        HandoffArena a, r;
        std::string err;
        const HandoffSizing s = sized({{1024, 2}, {65536, 1}});
        expect(a.open_writer(path, s, kPack, geom, err) && a.reserve(err), "create and reserve", err);
        struct stat st {};
        expect(::stat(path.c_str(), &st) == 0 && (uint64_t) st.st_blocks * 512 >= s.arena_bytes, "every page is committed",
               std::to_string((uint64_t) st.st_blocks * 512) + " of " + std::to_string(s.arena_bytes));
        HandoffClaim c;
        a.claim(1, 5, 6, c, err);
        uint8_t* win = a.claim_window(c, err);
        expect(win != nullptr, "the claim's window", err);
        const uint64_t n = 96ull << 20;
        std::vector<std::thread> fill;
        for (int t = 0; t < 4; ++t)
            fill.emplace_back([&, t] {
                for (uint64_t k = (uint64_t) t * n / 4; k < (uint64_t) (t + 1) * n / 4; ++k) win[k] = (uint8_t) (k * 11 + (k >> 13));
            });
        for (auto& t : fill) t.join();
        uint64_t h = 1469598103934665603ull;
        std::vector<uint8_t> chunk(1 << 20);
        for (uint64_t off = 0; off < n; off += chunk.size()) {
            for (size_t k = 0; k < chunk.size(); ++k) chunk[k] = (uint8_t) ((off + k) * 11 + ((off + k) >> 13));
            h = fnv1a64(chunk.data(), chunk.size(), h);
        }
        expect(a.publish(c, 65536, n, h, err), "publish what four threads wrote through the window", err);
        HandoffPayload p;
        expect(r.open_reader(path, kPack, geom, err) && r.read_slot(c.index, c.nonce, 5, p, err) &&
                   HandoffArena::payload_hash_of(p) == h,
               "a reader sees it through the file", err);
        HandoffClaim fake = c;
        fake.payload_off += 64;
        expect(a.claim_window(fake, err) == nullptr && has(err, "slot table"), "a window only for a real claim", err);
        // the reader's window: the same checks as read_slot, the same bytes, one mapping for every read
        HandoffSlotInfo wi;
        expect(r.reserve(err), "a reader maps the arena read-only, populated", err);
        const uint8_t* rw = r.read_window(c.index, c.nonce, 5, wi, err);
        expect(rw != nullptr && wi.payload_bytes == n && wi.payload_hash == h && wi.tokens == 65536 && wi.nonce == c.nonce &&
                   fnv1a64(rw, n) == h,
               "read_window gives the published bytes and the checked header", err);
        expect(r.read_window(c.index, c.nonce, 5, wi, err) == rw, "and the same mapping on the next read");
        expect(r.read_window(c.index, c.nonce ^ 1, 5, wi, err) == nullptr && has(err, "nonce"), "another nonce", err);
        expect(r.read_window(c.index, c.nonce, 6, wi, err) == nullptr && has(err, "addressed to client"), "another client",
               err);
        expect(r.read_window(0, c.nonce, 5, wi, err) == nullptr && has(err, "not READY"), "a FREE slot", err);
        expect(a.read_window(c.index, c.nonce, 5, wi, err) == nullptr && has(err, "as a reader"), "a writer has no read window",
               err);
        HandoffArena moved = std::move(a);
        expect(moved.valid() && !a.valid() && moved.claim_window(c, err) == win, "the window moves with the arena");
        expect(moved.release(c.index, c.nonce, err), "release", err);
        drop(path);
    }

    std::printf("big-slot\n");
    {
        struct statvfs sv {};
        ::statvfs("/dev/shm", &sv);
        const uint64_t avail = (uint64_t) sv.f_bavail * sv.f_frsize;
        const HandoffSizing s = sized({{1024, 1}, {100000, 1}});   // a 2.2 GiB slot
        if (avail < s.arena_bytes + (1ull << 30)) {
            std::printf("  skip: /dev/shm has %llu MiB free\n", (unsigned long long) (avail >> 20));
        } else {
            const std::string path = arena("big");
            HandoffArena a, r;
            std::string err;
            a.open_writer(path, s, kPack, geom, err);
            HandoffClaim c;
            a.claim(1, 8, 8, c, err);
            const uint64_t total = (2ull << 30) + 3;   // over the ~2 GiB a single write moves
            std::vector<uint8_t> body(total);
            for (uint64_t k = 0; k < total; ++k) body[k] = (uint8_t) (k * 3 + (k >> 20));
            expect(a.write_payload(c, 0, body.data(), total, err), "one write of 2 GiB + 3 B", err);
            const uint64_t h = fnv1a64(body.data(), total);
            body = std::vector<uint8_t>();
            expect(a.publish(c, 1, total, h, err), "publish");
            HandoffPayload p;
            expect(r.open_reader(path, kPack, geom, err) && r.read_slot(c.index, c.nonce, 8, p, err) &&
                       p.payload_bytes == total && p.data[total - 1] == (uint8_t) ((total - 1) * 3 + ((total - 1) >> 20)) &&
                       HandoffArena::payload_hash_of(p) == h,
                   "read back whole, hash equal", err);
            drop(path);
        }
    }

    std::printf("restart\n");
    {
        const std::string path = arena("restart");
        std::string err;
        const std::string out = in_child([&] {
            HandoffArena w;
            std::string e;
            HandoffClaim c;
            std::vector<uint8_t> body(64, 1);
            if (!w.open_writer(path, three_by_two(), kPack, geom, e) || !w.claim(2, 9, 9, c, e) ||
                !w.publish(c, 1, body.size(), fnv1a64(body.data(), body.size()), e))
                return "FAIL " + e;
            return hex(c.nonce);
        });
        const uint64_t nonce = std::strtoull(out.c_str(), nullptr, 16);
        HandoffArena r;
        HandoffPayload p;
        expect(r.open_reader(path, kPack, geom, err) && r.read_slot(4, nonce, 9, p, err), "a dead writer's slot is readable", err);
        p = HandoffPayload{};
        HandoffArena fresh;
        expect(fresh.open_writer(path, three_by_two(), kPack, geom, err) && fresh.header().created_pid == (uint64_t) getpid() &&
                   fresh.free_slots() == "6/6",
               "a new writer rebuilds a dead creator's slot table", err);
        expect(!r.read_slot(4, nonce, 9, p, err) && has(err, "FREE"), "and the old payload is gone", err);
        drop(path);
    }

    std::error_code ec;
    std::filesystem::remove_all(g_root, ec);
    std::printf("handoff_arena_test: %d checks, %d failed\n", g_checks, g_failed);
    return g_failed ? 1 : 0;
}

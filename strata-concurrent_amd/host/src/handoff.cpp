// handoff.cpp - the hand-off arena (the reference's src/core/handoff.cpp: same protocol, same file, this library's
// code).  Host only: a file, two kinds of 4 KiB header, an advisory lock and mappings.
//
// Decisions about slots are taken with the process mutex and the file's flock both held (FileLock below); payload
// bytes move without either.  Every header store goes through the file descriptor (pwrite), and publish orders its two
// stores with a release fence between them, so a reader that sees READY also sees the payload record and the bytes
// written before it.
#include "strata/core/handoff.hpp"

#include <algorithm>
#include <atomic>
#include <cerrno>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <ctime>
#include <filesystem>
#include <system_error>
#include <thread>

#include <fcntl.h>
#include <sys/file.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <sys/statvfs.h>
#include <unistd.h>

namespace strata::core {

namespace {

/// Both magics are compared as 16 raw bytes.  The arena's fills all 16 (no terminator); the slot's is 15 characters
/// and a zero (src/core/handoff.cpp:42-45).
constexpr char kArenaMagic[16] = {'S', 'T', 'R', 'A', 'T', 'A', '-', 'H', 'A', 'R', 'E', 'N', 'A', '-', 'V', '1'};
constexpr char kSlotMagic[16] = "STRATA-HSLOT-V1";

/// The flock is held for microseconds; one still held after 10 s is a foreign lock, reported instead of waited out
/// (retry every 20 ms, src/core/handoff.cpp:50).
constexpr int kLockRetryMs = 20;
constexpr int kLockGiveUpMs = 10000;

uint64_t self_pid() { return (uint64_t) (uint32_t) getpid(); }

std::string hex16(uint64_t v) {
    char b[20];
    std::snprintf(b, sizeof b, "%016llx", (unsigned long long) v);
    return b;
}

std::string gib(uint64_t bytes) {
    char b[32];
    std::snprintf(b, sizeof b, "%.2f GiB", (double) bytes / (double) (1ull << 30));
    return b;
}

std::string num(uint64_t v) { return std::to_string((unsigned long long) v); }

/// A nonce must not repeat on this machine within a pid's lifetime: the monotonic clock, the pid and a per-process
/// counter, through the splitmix64 finaliser.  Never 0.
uint64_t fresh_nonce() {
    static std::atomic<uint64_t> counter{0};
    uint64_t z = (uint64_t) std::chrono::steady_clock::now().time_since_epoch().count();
    z += (self_pid() << 40) + 0x9E3779B97F4A7C15ull * (counter.fetch_add(1) + 1);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    z ^= z >> 31;
    return z ? z : 1;
}

/// pread/pwrite of exactly n bytes (a single call moves at most ~2 GiB on Linux, and may be interrupted).
bool read_at(int fd, void* dst, uint64_t n, uint64_t off) {
    auto* p = static_cast<uint8_t*>(dst);
    while (n) {
        const ssize_t got = ::pread(fd, p, (size_t) std::min<uint64_t>(n, 1ull << 30), (off_t) off);
        if (got < 0 && errno == EINTR) continue;
        if (got <= 0) return false;
        p += got;
        off += (uint64_t) got;
        n -= (uint64_t) got;
    }
    return true;
}

bool write_at(int fd, const void* src, uint64_t n, uint64_t off, uint64_t* done = nullptr) {
    const auto* p = static_cast<const uint8_t*>(src);
    uint64_t moved = 0;
    bool ok = true;
    while (moved < n) {
        const ssize_t put = ::pwrite(fd, p + moved, (size_t) std::min<uint64_t>(n - moved, 1ull << 30),
                                     (off_t) (off + moved));
        if (put < 0 && errno == EINTR) continue;
        if (put <= 0) { ok = false; break; }
        moved += (uint64_t) put;
    }
    if (done) *done = moved;
    return ok;
}

/// The file's advisory lock for one decision, retried every 20 ms for up to 10 s.
class FileLock {
  public:
    FileLock(int fd, bool exclusive) : fd_(fd) {
        const int op = (exclusive ? LOCK_EX : LOCK_SH) | LOCK_NB;
        for (int waited = 0;; waited += kLockRetryMs) {
            if (::flock(fd_, op) == 0) { held_ = true; return; }
            if (errno != EWOULDBLOCK && errno != EAGAIN && errno != EINTR) {
                error_ = std::string("cannot lock the handoff arena: ") + std::strerror(errno);
                return;
            }
            if (waited >= kLockGiveUpMs) {
                error_ = "the handoff arena has been locked by another process for over " +
                         num(kLockGiveUpMs / 1000) + " s; not acting on a slot table that cannot be read";
                return;
            }
            std::this_thread::sleep_for(std::chrono::milliseconds(kLockRetryMs));
        }
    }
    ~FileLock() { release(); }
    FileLock(const FileLock&) = delete;
    FileLock& operator=(const FileLock&) = delete;
    void release() {
        if (held_) ::flock(fd_, LOCK_UN);
        held_ = false;
    }
    bool held() const { return held_; }
    const std::string& error() const { return error_; }

  private:
    int fd_;
    bool held_ = false;
    std::string error_;
};

/// statvfs of the directory that will hold `path`: false (with both numbers) only when the filesystem reports less
/// room than `bytes`; a check that cannot be made does not refuse (src/core/handoff.cpp:88-110).
bool room_for(const std::string& path, uint64_t bytes, std::string& why) {
    const std::filesystem::path p(path);
    const std::filesystem::path dir = p.has_parent_path() ? p.parent_path() : std::filesystem::path(".");
    struct statvfs sv {};
    if (::statvfs(dir.c_str(), &sv) != 0) return true;
    const uint64_t avail = (uint64_t) sv.f_bavail * (uint64_t) (sv.f_frsize ? sv.f_frsize : sv.f_bsize);
    if (avail >= bytes) return true;
    why = dir.string() + " has " + num(avail) + " B free";
    return false;
}

void put_u32(uint8_t* rec, uint64_t off, uint32_t v) { std::memcpy(rec + off, &v, 4); }
void put_u64(uint8_t* rec, uint64_t off, uint64_t v) { std::memcpy(rec + off, &v, 8); }

}  // namespace

// ================================ identity ================================

std::string handoff_split_spec(const HandoffSplit& split) {
    // src/core/handoff.cpp:115-130
    std::string later;
    for (const HandoffSplitStage& st : split.stages) {
        if (!later.empty()) later += ',';
        later += std::to_string(st.layer_lo) + ".." + std::to_string(st.layer_hi);
    }
    const bool draft_last = split.draft_on_last && !split.stages.empty();
    return "main=" + std::to_string(split.main_lo) + ".." + std::to_string(split.main_hi) + "|" + later +
           "|n=" + std::to_string(split.stages.size() + 1) + "|draft=" + (draft_last ? "last" : "main");
}

uint64_t handoff_geom_hash(const std::array<int64_t, 18>& geometry, const std::string& split_spec) {
    // src/core/handoff.cpp:132-138: the salt, the 18 words little-endian, the spec; 0 is reserved for "unset".
    static const char kSalt[] = "strata-handoff-geom-v1";
    uint8_t words[18 * 8];
    for (int i = 0; i < 18; ++i)
        for (int b = 0; b < 8; ++b) words[i * 8 + b] = (uint8_t) ((uint64_t) geometry[(size_t) i] >> (8 * b));
    uint64_t h = fnv1a64(reinterpret_cast<const uint8_t*>(kSalt), sizeof kSalt - 1);
    h = fnv1a64(words, sizeof words, h);
    h = fnv1a64(reinterpret_cast<const uint8_t*>(split_spec.data()), split_spec.size(), h);
    return h ? h : 1;
}

std::string handoff_arena_path(const std::string& handoff_dir, uint64_t pack_hash, const std::string& split_spec,
                               const std::string& instance) {
    std::string p = handoff_dir;
    if (!p.empty() && p.back() != '/') p += '/';
    p += hex16(pack_hash) + "-" + split_spec;
    if (!instance.empty()) p += "/" + instance;
    return p + "/arena";
}

// ================================ sizing ================================

bool handoff_size_arena(const std::vector<HandoffTierSpec>& tiers, const HandoffPricer& pricer, HandoffSizing& out,
                        std::string& err) {
    std::vector<uint64_t> priced;
    priced.reserve(tiers.size());
    for (const HandoffTierSpec& t : tiers) {
        uint64_t bytes = 0;
        std::string why;
        if (!pricer || !pricer(t.max_tokens, bytes, why)) {
            err = "handoff sizing, tier " + num(t.max_tokens) + " tokens: " + (pricer ? why : "no pricer");
            return false;
        }
        priced.push_back(bytes);
    }
    return handoff_size_arena(tiers, priced, out, err);
}

bool handoff_size_arena(const std::vector<HandoffTierSpec>& tiers, const std::vector<uint64_t>& payload_bytes,
                        HandoffSizing& out, std::string& err) {
    // src/core/handoff.cpp:164-231
    out = HandoffSizing{};
    if (tiers.empty()) { err = "handoff sizing: no tiers"; return false; }
    if (tiers.size() > (size_t) kHandoffMaxTiers) {
        err = "handoff sizing: " + num(tiers.size()) + " tiers, the arena header has room for " + num(kHandoffMaxTiers);
        return false;
    }
    if (payload_bytes.size() != tiers.size()) {
        err = "handoff sizing: " + num(payload_bytes.size()) + " priced sizes for " + num(tiers.size()) + " tiers";
        return false;
    }
    HandoffSizing s;
    s.tiers = tiers;
    s.payload_bytes = payload_bytes;
    uint64_t off = kHandoffHeaderBytes;
    std::string slots, tokens;
    for (size_t i = 0; i < tiers.size(); ++i) {
        const HandoffTierSpec& t = tiers[i];
        if (t.max_tokens == 0) { err = "handoff sizing: tier " + num(i) + " has 0 tokens"; return false; }
        if (i && t.max_tokens <= tiers[i - 1].max_tokens) {
            err = "handoff sizing: tiers must ascend by token count (" + num(tiers[i - 1].max_tokens) + " then " +
                  num(t.max_tokens) + ")";
            return false;
        }
        if (t.slot_count == 0) { err = "handoff sizing: tier " + num(t.max_tokens) + " has 0 slots"; return false; }
        if (payload_bytes[i] > UINT64_MAX - 63 - kHandoffSlackBytes - kHandoffHeaderBytes) {
            err = "handoff sizing: tier " + num(t.max_tokens) + " is too big to size";
            return false;
        }
        const uint64_t slot = handoff_round_up_64(payload_bytes[i]) + kHandoffSlackBytes;
        const uint64_t stride = kHandoffHeaderBytes + slot;
        if (t.slot_count > (UINT64_MAX - off) / stride) { err = "handoff sizing: the arena offset overflows"; return false; }
        s.slot_bytes.push_back(slot);
        s.slot_off.push_back(off);
        off += t.slot_count * stride;
        s.slot_total += t.slot_count;
        s.max_tokens = std::max(s.max_tokens, t.max_tokens);
        slots += (i ? "," : "") + num(t.slot_count);
        tokens += (i ? "," : "") + num(t.max_tokens);
    }
    s.arena_bytes = off;
    s.describe = "slots " + slots + " (tiers " + tokens + "), max " + num(s.max_tokens) + " tokens, arena " +
                 gib(s.arena_bytes) + " (" + num(s.arena_bytes) + " B)";
    out = std::move(s);
    return true;
}

// ================================ liveness and clock ================================

bool handoff_pid_alive(uint64_t pid) {
    // /proc/<pid> needs no signal permission; with no /proc at all the answer is "alive" (src/core/handoff.cpp:237-247).
    if (pid == 0 || pid > (uint64_t) INT32_MAX) return false;
    struct stat st {};
    if (::stat(("/proc/" + num(pid)).c_str(), &st) == 0) return true;
    return ::stat("/proc", &st) != 0;
}

uint64_t handoff_proc_start_time(uint64_t pid) {
    // /proc/<pid>/stat: "pid (comm) state ..." where comm may hold spaces and parentheses; starttime is field 22,
    // i.e. the 20th space-separated token after the LAST ')' (src/core/handoff.cpp:249-270).
    if (pid == 0 || pid > (uint64_t) INT32_MAX) return 0;
    FILE* f = std::fopen(("/proc/" + num(pid) + "/stat").c_str(), "rb");
    if (!f) return 0;
    char buf[4096];
    const size_t n = std::fread(buf, 1, sizeof buf - 1, f);
    std::fclose(f);
    buf[n] = 0;
    const char* p = std::strrchr(buf, ')');
    if (!p) return 0;
    ++p;
    for (int token = 0; token < 20; ++token) {
        while (*p == ' ') ++p;
        if (!*p) return 0;
        if (token == 19) return std::strtoull(p, nullptr, 10);
        while (*p && *p != ' ') ++p;
    }
    return 0;
}

bool handoff_claim_alive(uint64_t pid, uint64_t start_time) {
    if (!handoff_pid_alive(pid)) return false;
    if (start_time == 0) return true;                 // unknown never means dead
    const uint64_t now = handoff_proc_start_time(pid);
    return now == 0 || now == start_time;
}

uint64_t handoff_now_ms() {
    struct timespec ts {};
    if (::clock_gettime(CLOCK_MONOTONIC, &ts) != 0) return 0;
    return (uint64_t) ts.tv_sec * 1000ull + (uint64_t) ts.tv_nsec / 1000000ull;
}

// ================================ HandoffPayload ================================

HandoffPayload::~HandoffPayload() { unbind(); }

void HandoffPayload::bind_mapping(void* map, uint64_t map_bytes, const uint8_t* d, uint64_t payload) {
    unbind();
    map_ = map;
    map_bytes_ = map_bytes;
    data = d;
    bytes = payload;
}

void HandoffPayload::unbind() {
    if (map_) ::munmap(map_, (size_t) map_bytes_);
    map_ = nullptr;
    map_bytes_ = 0;
    data = nullptr;
    bytes = 0;
}

HandoffPayload::HandoffPayload(HandoffPayload&& o) noexcept { *this = std::move(o); }

HandoffPayload& HandoffPayload::operator=(HandoffPayload&& o) noexcept {
    if (this == &o) return *this;
    unbind();
    data = o.data;
    bytes = o.bytes;
    index = o.index;
    tier = o.tier;
    nonce = o.nonce;
    client_id = o.client_id;
    request_id = o.request_id;
    tokens = o.tokens;
    payload_bytes = o.payload_bytes;
    payload_hash = o.payload_hash;
    seq = o.seq;
    map_ = o.map_;
    map_bytes_ = o.map_bytes_;
    o.map_ = nullptr;
    o.map_bytes_ = 0;
    o.data = nullptr;
    o.bytes = 0;
    return *this;
}

// ================================ HandoffArena: plumbing ================================

HandoffArena::HandoffArena() {
    const char* v = std::getenv("STRATA_HANDOFF_LEASE_MS");
    if (v && *v) lease_ms_ = std::strtoull(v, nullptr, 10);
}

HandoffArena::~HandoffArena() { close_(); }

HandoffArena::HandoffArena(HandoffArena&& o) noexcept { *this = std::move(o); }

HandoffArena& HandoffArena::operator=(HandoffArena&& o) noexcept {
    if (this == &o) return *this;
    close_();
    fd_ = o.fd_;
    writer_ = o.writer_;
    map_ = o.map_;
    map_bytes_ = o.map_bytes_;
    path_ = std::move(o.path_);
    hdr_ = o.hdr_;
    places_ = std::move(o.places_);
    lease_ms_ = o.lease_ms_;
    client_pids_ = std::move(o.client_pids_);
    o.fd_ = -1;
    o.writer_ = false;
    o.map_ = nullptr;
    o.map_bytes_ = 0;
    o.hdr_ = HandoffArenaHeader{};
    return *this;
}

void HandoffArena::close_() {
    if (map_) ::munmap(map_, (size_t) map_bytes_);
    map_ = nullptr;
    map_bytes_ = 0;
    if (fd_ >= 0) ::close(fd_);
    fd_ = -1;
    writer_ = false;
    path_.clear();
    hdr_ = HandoffArenaHeader{};
    places_.clear();
    client_pids_.clear();
}

bool HandoffArena::store_(uint64_t off, const void* data, uint64_t n) const { return write_at(fd_, data, n, off); }

/// Check a header read from the file and adopt it: the identity fields first (nothing else means anything in a file
/// that is not an arena), then the file's size against the header's (when `file_bytes` is given), then the tier
/// table, whose every slot must lie inside the file the header describes.
bool HandoffArena::adopt_header_(const HandoffArenaHeader& h, uint64_t file_bytes, std::string& err) {
    if (std::memcmp(h.magic, kArenaMagic, sizeof kArenaMagic) != 0) {
        err = "handoff arena " + path_ + " is not a Strata handoff arena (its magic does not match)";
        return false;
    }
    if (h.version != kHandoffVersion) {
        err = "handoff arena " + path_ + " speaks protocol version " + num(h.version) + "; this library speaks " +
              num(kHandoffVersion);
        return false;
    }
    if (h.header_bytes != kHandoffHeaderBytes) {
        err = "handoff arena " + path_ + " declares header_bytes " + num(h.header_bytes) + ", expected " +
              num(kHandoffHeaderBytes);
        return false;
    }
    if (file_bytes && file_bytes != h.arena_bytes) {
        err = "handoff arena " + path_ + " is " + num(file_bytes) + " B but its header says " + num(h.arena_bytes) + " B";
        return false;
    }
    if (h.tier_count == 0 || h.tier_count > (uint32_t) kHandoffMaxTiers) {
        err = "handoff arena " + path_ + " declares " + num(h.tier_count) + " tiers";
        return false;
    }
    std::vector<Place> places;
    for (uint32_t t = 0; t < h.tier_count; ++t) {
        const uint64_t stride = kHandoffHeaderBytes + h.tier_slot_bytes[t];
        for (uint64_t k = 0; k < h.tier_slot_count[t]; ++k) {
            Place p;
            p.base = h.tier_slot_off[t] + k * stride;
            p.capacity = h.tier_slot_bytes[t];
            p.tier = t;
            if (p.base < kHandoffHeaderBytes || p.base + kHandoffHeaderBytes + p.capacity > h.arena_bytes ||
                places.size() >= (1u << 20)) {
                err = "handoff arena " + path_ + " has a slot table that runs past its " + num(h.arena_bytes) + " B";
                return false;
            }
            places.push_back(p);
        }
    }
    if (places.size() != h.slot_total) {
        err = "handoff arena " + path_ + " lists " + num(places.size()) + " slots but its header says " +
              num(h.slot_total);
        return false;
    }
    hdr_ = h;
    places_ = std::move(places);
    return true;
}

bool HandoffArena::place_(int index, Place& p) const {
    if (index < 0 || (size_t) index >= places_.size()) return false;
    p = places_[(size_t) index];
    return true;
}

bool HandoffArena::load_slot_(int index, HandoffSlotHeader& s, Place& p) const {
    return place_(index, p) && read_at(fd_, &s, sizeof s, p.base);
}

bool HandoffArena::lease_over_(uint64_t stamp_ms) const {
    if (lease_ms_ == 0 || stamp_ms == 0) return true;
    const uint64_t now = handoff_now_ms();
    return now >= stamp_ms && now - stamp_ms >= lease_ms_;
}

bool HandoffArena::reader_gone_(uint64_t client_id) const {
    if (client_id == 0) return false;
    for (const auto& cp : client_pids_)
        if (cp.first == client_id) return !handoff_pid_alive(cp.second);
    return false;   // an unregistered reader is reclaimed by the lease alone
}

uint64_t HandoffArena::tier_max_tokens(uint32_t t) const { return t < (uint32_t) kHandoffMaxTiers ? hdr_.tier_max_tokens[t] : 0; }
uint64_t HandoffArena::tier_slot_bytes(uint32_t t) const { return t < (uint32_t) kHandoffMaxTiers ? hdr_.tier_slot_bytes[t] : 0; }
uint64_t HandoffArena::tier_slot_count(uint32_t t) const { return t < (uint32_t) kHandoffMaxTiers ? hdr_.tier_slot_count[t] : 0; }
uint64_t HandoffArena::tier_slot_off(uint32_t t) const { return t < (uint32_t) kHandoffMaxTiers ? hdr_.tier_slot_off[t] : 0; }

std::string HandoffArena::describe() const {
    std::string slots, tokens;
    for (uint32_t t = 0; t < hdr_.tier_count && t < (uint32_t) kHandoffMaxTiers; ++t) {
        slots += (t ? "," : "") + num(hdr_.tier_slot_count[t]);
        tokens += (t ? "," : "") + num(hdr_.tier_max_tokens[t]);
    }
    return "slots " + slots + " (tiers " + tokens + "), max " + num(max_tokens()) + " tokens, arena " +
           gib(hdr_.arena_bytes) + ", pack hash " + hex16(hdr_.pack_hash) + ", geometry hash " + hex16(hdr_.geom_hash);
}

// ================================ the writer ================================

/// Write a fresh header and every slot header FREE (the caller holds the exclusive lock).
bool HandoffArena::format_(const HandoffSizing& sizing, uint64_t pack_hash, uint64_t geom_hash, std::string& err) {
    HandoffArenaHeader h{};
    std::memcpy(h.magic, kArenaMagic, sizeof kArenaMagic);
    h.version = kHandoffVersion;
    h.header_bytes = (uint32_t) kHandoffHeaderBytes;
    h.tier_count = (uint32_t) sizing.tiers.size();
    h.slot_total = sizing.slot_total;
    h.arena_bytes = sizing.arena_bytes;
    h.pack_hash = pack_hash;
    h.geom_hash = geom_hash;
    h.created_pid = self_pid();
    h.created_start = handoff_proc_start_time(h.created_pid);
    for (size_t i = 0; i < sizing.tiers.size(); ++i) {
        h.tier_max_tokens[i] = sizing.tiers[i].max_tokens;
        h.tier_slot_count[i] = sizing.tiers[i].slot_count;
        h.tier_slot_bytes[i] = sizing.slot_bytes[i];
        h.tier_slot_off[i] = sizing.slot_off[i];
    }
    uint8_t page[kHandoffHeaderBytes] = {};
    std::memcpy(page, &h, sizeof h);
    if (!store_(0, page, sizeof page)) {
        err = "cannot write the handoff arena header of " + path_ + ": " + std::strerror(errno);
        return false;
    }
    if (!adopt_header_(h, 0, err)) return false;
    std::memset(page, 0, sizeof page);
    std::memcpy(page + kSlotMagicOffset, kSlotMagic, sizeof kSlotMagic);
    put_u32(page, kSlotVersionOffset, kHandoffVersion);
    put_u32(page, kSlotHeaderBytesOffset, (uint32_t) kHandoffHeaderBytes);
    put_u32(page, kSlotStateOffset, kHandoffFree);
    for (const Place& p : places_) {
        put_u32(page, kSlotTierOffset, p.tier);
        if (!store_(p.base, page, sizeof page)) {
            err = "cannot initialise the handoff slot at offset " + num(p.base) + " of " + path_;
            return false;
        }
    }
    return true;
}

bool HandoffArena::open_writer(const std::string& path, const HandoffSizing& sizing, uint64_t pack_hash,
                               uint64_t geom_hash, std::string& err, bool allow_existing_writer) {
    // src/core/handoff.cpp:453-622
    std::lock_guard<std::mutex> guard(mu_);
    close_();
    err.clear();
    if (pack_hash == 0) { err = "a handoff arena needs a nonzero pack hash"; return false; }
    if (geom_hash == 0) { err = "a handoff arena needs a nonzero geometry hash"; return false; }
    const size_t nt = sizing.tiers.size();
    if (nt == 0 || nt > (size_t) kHandoffMaxTiers || sizing.arena_bytes == 0 || sizing.slot_bytes.size() != nt ||
        sizing.slot_off.size() != nt) {
        err = "handoff arena: the sizing is empty, inconsistent or has more than " + num(kHandoffMaxTiers) + " tiers";
        return false;
    }
    // the sizing must describe the layout it claims before it sizes a file
    uint64_t walk = kHandoffHeaderBytes, slots = 0;
    for (size_t i = 0; i < nt; ++i) {
        if (sizing.slot_off[i] != walk) {
            err = "handoff arena: tier " + num(i) + " starts at " + num(sizing.slot_off[i]) + " but the layout says " +
                  num(walk);
            return false;
        }
        walk += sizing.tiers[i].slot_count * (kHandoffHeaderBytes + sizing.slot_bytes[i]);
        slots += sizing.tiers[i].slot_count;
    }
    if (walk != sizing.arena_bytes || slots != sizing.slot_total) {
        err = "handoff arena: the sizing does not add up (" + num(sizing.arena_bytes) + " B and " +
              num(sizing.slot_total) + " slots claimed, " + num(walk) + " B and " + num(slots) + " slots laid out)";
        return false;
    }

    const std::filesystem::path p(path);
    if (p.has_parent_path()) {
        std::error_code ec;
        std::filesystem::create_directories(p.parent_path(), ec);
        if (ec) {
            err = "cannot create the handoff directory " + p.parent_path().string() + ": " + ec.message();
            return false;
        }
    }
    // A sparse file on a tmpfs that cannot back it is created without complaint and kills the writer with SIGBUS
    // later, so the room is checked before the file exists (an existing sized file already holds its room).
    struct stat st {};
    if (::stat(path.c_str(), &st) != 0 || st.st_size == 0) {
        std::string why;
        if (!room_for(path, sizing.arena_bytes, why)) {
            err = "the handoff arena " + path + " needs " + num(sizing.arena_bytes) + " B (" + gib(sizing.arena_bytes) +
                  ") but " + why + "; use fewer slots per tier, fewer tiers, or a filesystem with more room";
            return false;
        }
    }
    const int fd = ::open(path.c_str(), O_RDWR | O_CREAT | O_CLOEXEC, 0600);
    if (fd < 0) {
        err = "cannot open the handoff arena " + path + ": " + std::strerror(errno);
        return false;
    }
    fd_ = fd;
    path_ = path;
    writer_ = true;

    FileLock lock(fd_, true);
    if (!lock.held()) {
        err = lock.error();
        lock.release();
        close_();
        return false;
    }
    auto fail = [&](std::string why) {
        err = std::move(why);
        lock.release();
        close_();
        return false;
    };
    if (::fstat(fd_, &st) != 0) return fail("cannot stat the handoff arena " + path + ": " + std::strerror(errno));

    bool format = false;
    if (st.st_size == 0) {
        if (::ftruncate(fd_, (off_t) sizing.arena_bytes) != 0)
            return fail("cannot size the handoff arena " + path + ": " + std::strerror(errno));
        format = true;
    } else if ((uint64_t) st.st_size != sizing.arena_bytes) {
        return fail("handoff arena " + path + " is " + num((uint64_t) st.st_size) + " B and this instance needs " +
                    num(sizing.arena_bytes) + " B (its tier table differs)");
    } else {
        HandoffArenaHeader h{};
        if (!read_at(fd_, &h, sizeof h, 0)) return fail("handoff arena " + path + ": cannot read its header");
        std::string why;
        if (!adopt_header_(h, (uint64_t) st.st_size, why)) return fail(why);
        if (h.pack_hash != pack_hash)
            return fail("handoff arena " + path + " was written for pack hash " + hex16(h.pack_hash) + ", expected " +
                        hex16(pack_hash));
        if (h.geom_hash != geom_hash)
            return fail("handoff arena " + path + " was written for geometry hash " + hex16(h.geom_hash) +
                        ", expected " + hex16(geom_hash) + " (a different geometry or layer split)");
        bool same_table = h.tier_count == nt && h.slot_total == sizing.slot_total;
        for (size_t i = 0; same_table && i < nt; ++i)
            same_table = h.tier_max_tokens[i] == sizing.tiers[i].max_tokens &&
                         h.tier_slot_count[i] == sizing.tiers[i].slot_count &&
                         h.tier_slot_bytes[i] == sizing.slot_bytes[i] && h.tier_slot_off[i] == sizing.slot_off[i];
        if (!same_table)
            return fail("handoff arena " + path + " has the size this instance needs but a different tier table (" +
                        describe() + ")");
        if (h.created_pid != self_pid()) {
            if (handoff_claim_alive(h.created_pid, h.created_start)) {
                // one arena, one writer; the flag exists only for the tests' two-process contention case
                if (!allow_existing_writer)
                    return fail("handoff arena " + path + " is already being written by pid " + num(h.created_pid) +
                                "; one arena per prefill instance");
            } else if (!allow_existing_writer) {
                format = true;   // its creator is gone: no payload of a dead process survives a restart
            }
        }
        // else: this process re-opens its own arena and keeps its slots (a job may be in flight)
    }
    if (format && !format_(sizing, pack_hash, geom_hash, err)) {
        std::string why = err;
        return fail(why);
    }
    return true;
}

void HandoffArena::note_client_pid(uint64_t client_id, uint64_t pid) {
    std::lock_guard<std::mutex> guard(mu_);
    for (auto& cp : client_pids_) {
        if (cp.first == client_id) { cp.second = pid; return; }
    }
    client_pids_.emplace_back(client_id, pid);
}

std::vector<HandoffReclaim> HandoffArena::sweep_(std::string* err) {
    // src/core/handoff.cpp:662-715: CLAIMED slots of dead claimers or past the lease, READY slots of dead readers or
    // past the lease; the abandoned flag is stored before the state goes FREE.
    std::vector<HandoffReclaim> took;
    for (int i = 0; i < (int) places_.size(); ++i) {
        HandoffSlotHeader s{};
        Place p;
        if (!load_slot_(i, s, p) || s.state == kHandoffFree) continue;
        const uint64_t stamp = s.state == kHandoffReady ? s.published_ms : s.claimed_ms;
        std::string why;
        if (s.state == kHandoffClaimed) {
            if (!handoff_claim_alive(s.owner_pid, s.owner_start))
                why = "the claiming writer (pid " + num(s.owner_pid) + ") is gone";
            else if (lease_over_(s.claimed_ms))
                why = "its CLAIMED lease ran out after " + num(handoff_now_ms() - std::min(stamp, handoff_now_ms())) + " ms";
        } else if (s.state == kHandoffReady) {
            if (reader_gone_(s.client_id))
                why = "its reader (client " + hex16(s.client_id) + ") is gone";
            else if (lease_over_(s.published_ms))
                why = "nobody read it within the " + num(lease_ms_) + " ms lease";
        }
        if (why.empty()) continue;
        const uint32_t flags = s.flags | kHandoffFlagAbandoned;
        const uint32_t free_state = kHandoffFree;
        if (!store_(p.base + kSlotFlagsOffset, &flags, 4) || !store_(p.base + kSlotStateOffset, &free_state, 4)) {
            if (err) *err = "cannot reclaim the handoff slot at offset " + num(p.base);
            continue;
        }
        HandoffReclaim r;
        r.index = i;
        r.was_state = s.state;
        r.flags = flags;
        r.owner_pid = s.owner_pid;
        r.client_id = s.client_id;
        r.nonce = s.nonce;
        r.payload_bytes = s.payload_bytes;
        const uint64_t now = handoff_now_ms();
        r.age_ms = stamp && now >= stamp ? now - stamp : 0;
        r.why = std::move(why);
        took.push_back(std::move(r));
    }
    return took;
}

std::vector<HandoffReclaim> HandoffArena::reclaim(std::string* err) {
    std::lock_guard<std::mutex> guard(mu_);
    if (fd_ < 0) { if (err) *err = "the handoff arena is not open"; return {}; }
    if (!writer_) { if (err) *err = "a reader never reclaims handoff slots"; return {}; }
    FileLock lock(fd_, true);
    if (!lock.held()) { if (err) *err = lock.error(); return {}; }
    return sweep_(err);
}

uint64_t HandoffArena::count_free_() const {
    uint64_t n = 0;
    for (int i = 0; i < (int) places_.size(); ++i) {
        HandoffSlotHeader s{};
        Place p;
        if (load_slot_(i, s, p) && s.state == kHandoffFree) ++n;
    }
    return n;
}

bool HandoffArena::claim(uint32_t tier, uint64_t client_id, uint64_t request_id, HandoffClaim& out, std::string& err) {
    // src/core/handoff.cpp:729-818: the smallest group >= tier with a FREE slot (or a dead claimer's), one 4 KiB store
    std::lock_guard<std::mutex> guard(mu_);
    out = HandoffClaim{};
    err.clear();
    if (fd_ < 0) { err = "the handoff arena is not open"; return false; }
    if (!writer_) { err = "a reader never claims a handoff slot"; return false; }
    if (tier >= hdr_.tier_count) {
        err = "handoff tier " + num(tier) + " is not in this arena (" + num(hdr_.tier_count) + " tiers)";
        return false;
    }
    FileLock lock(fd_, true);
    if (!lock.held()) { err = lock.error(); return false; }
    sweep_(nullptr);
    for (int i = 0; i < (int) places_.size(); ++i) {
        const Place& p = places_[(size_t) i];
        if (p.tier < tier) continue;   // places_ ascend by tier, so the first usable slot is in the smallest group
        HandoffSlotHeader s{};
        Place at;
        if (!load_slot_(i, s, at)) { err = "cannot read the handoff slot header at index " + num(i); return false; }
        const bool usable = s.state == kHandoffFree ||
                            (s.state == kHandoffClaimed && !handoff_claim_alive(s.owner_pid, s.owner_start));
        if (!usable) continue;
        const uint64_t nonce = fresh_nonce();
        uint8_t rec[kHandoffHeaderBytes] = {};
        std::memcpy(rec + kSlotMagicOffset, kSlotMagic, sizeof kSlotMagic);
        put_u32(rec, kSlotVersionOffset, kHandoffVersion);
        put_u32(rec, kSlotHeaderBytesOffset, (uint32_t) kHandoffHeaderBytes);
        put_u32(rec, kSlotStateOffset, kHandoffClaimed);
        put_u32(rec, kSlotTierOffset, p.tier);
        put_u64(rec, kSlotOwnerOffset, self_pid());
        put_u64(rec, kSlotOwnerStartOffset, handoff_proc_start_time(self_pid()));
        put_u64(rec, kSlotNonceOffset, nonce);
        put_u64(rec, kSlotClientOffset, client_id);
        put_u64(rec, kSlotRequestOffset, request_id);
        put_u64(rec, kSlotPackHashOffset, hdr_.pack_hash);
        put_u64(rec, kSlotGeomHashOffset, hdr_.geom_hash);
        put_u64(rec, kSlotClaimedMsOffset, handoff_now_ms());
        if (!store_(p.base, rec, sizeof rec)) { err = "cannot claim the handoff slot at index " + num(i); return false; }
        out.index = i;
        out.base = p.base;
        out.payload_off = p.base + kHandoffHeaderBytes;
        out.capacity = p.capacity;
        out.tier = p.tier;
        out.nonce = nonce;
        return true;
    }
    // temporary: the caller queues the job
    err = "no free handoff slot for tier " + num(tier) + " or above (" + num(count_free_()) + "/" +
          num(hdr_.slot_total) + " free)";
    return false;
}

bool HandoffArena::write_payload(const HandoffClaim& c, uint64_t offset, const void* data, uint64_t bytes,
                                 std::string& err) {
    if (fd_ < 0) { err = "the handoff arena is not open"; return false; }
    if (!writer_) { err = "a reader never writes a handoff slot"; return false; }
    if (data == nullptr && bytes != 0) { err = "a handoff payload write with no data"; return false; }
    if (offset > c.capacity || bytes > c.capacity - offset) {
        err = "handoff slot " + num(c.index) + " holds " + num(c.capacity) + " B and this write reaches " +
              num(offset + bytes) + " B";
        return false;
    }
    Place p;
    if (!place_(c.index, p) || p.base != c.base || p.capacity != c.capacity) {
        err = "handoff claim of slot " + num(c.index) + " does not match this arena's slot table";
        return false;
    }
    uint64_t done = 0;
    if (!write_at(fd_, data, bytes, c.payload_off + offset, &done)) {
        err = "short handoff payload write in slot " + num(c.index) + ": wrote " + num(done) + " of " + num(bytes) +
              " B: " + std::strerror(errno);
        return false;
    }
    return true;
}

bool HandoffArena::publish(const HandoffClaim& c, uint64_t tokens, uint64_t payload_bytes, uint64_t payload_hash,
                           std::string& err) {
    // src/core/handoff.cpp:843-901: ownership checked under the lock; then the 48-byte record, a release fence and
    // the 8-byte state+flags store that is the publish point.
    std::lock_guard<std::mutex> guard(mu_);
    if (fd_ < 0) { err = "the handoff arena is not open"; return false; }
    if (!writer_) { err = "a reader never publishes a handoff slot"; return false; }
    if (payload_bytes > c.capacity) {
        err = "handoff slot " + num(c.index) + " holds " + num(c.capacity) + " B and the payload is " +
              num(payload_bytes) + " B";
        return false;
    }
    FileLock lock(fd_, true);
    if (!lock.held()) { err = lock.error(); return false; }
    HandoffSlotHeader s{};
    Place p;
    const bool readable = load_slot_(c.index, s, p) && p.base == c.base;
    if (!readable || s.state != kHandoffClaimed || s.nonce != c.nonce) {
        err = "the handoff slot " + num(c.index) + " claim is gone (state " + (readable ? num(s.state) : "?") +
              ", nonce " + (readable ? hex16(s.nonce) : "?") + ", ours " + hex16(c.nonce) + ")";
        return false;
    }
    if (s.flags & kHandoffFlagCancelled) {
        err = "the handoff slot " + num(c.index) + " job was cancelled";
        return false;
    }
    const uint64_t record[6] = {tokens, payload_bytes, payload_hash, s.claimed_ms, handoff_now_ms(), 1};
    static_assert(sizeof record == kSlotPublishBlockBytes);
    if (!store_(p.base + kSlotPublishBlockOffset, record, sizeof record)) {
        err = "cannot write the payload record of handoff slot " + num(c.index);
        return false;
    }
    std::atomic_thread_fence(std::memory_order_release);
    const uint32_t state_flags[2] = {kHandoffReady, s.flags & ~kHandoffFlagPartial};
    static_assert(sizeof state_flags == kSlotPublishStateBytes);
    if (!store_(p.base + kSlotStateOffset, state_flags, sizeof state_flags)) {
        err = "cannot publish handoff slot " + num(c.index);
        return false;
    }
    return true;
}

bool HandoffArena::release(int index, uint64_t nonce, std::string& err) {
    // src/core/handoff.cpp:903-932: the claim's identity cleared, then FREE; the body stays as it is
    std::lock_guard<std::mutex> guard(mu_);
    if (fd_ < 0) { err = "the handoff arena is not open"; return false; }
    if (!writer_) { err = "a reader never releases a handoff slot"; return false; }
    FileLock lock(fd_, true);
    if (!lock.held()) { err = lock.error(); return false; }
    HandoffSlotHeader s{};
    Place p;
    if (!load_slot_(index, s, p) || s.nonce != nonce) {
        err = "handoff slot " + num(index) + " is not the one nonce " + hex16(nonce) + " refers to";
        return false;
    }
    const uint64_t ids[4] = {0, 0, 0, 0};   // owner_pid, owner_start, nonce, client_id
    const uint64_t none = 0;
    const uint32_t state_flags[2] = {kHandoffFree, 0};
    const bool ok = store_(p.base + kSlotOwnerOffset, ids, sizeof ids) &&
                    store_(p.base + kSlotPayloadBytesOffset, &none, sizeof none) &&
                    store_(p.base + kSlotStateOffset, state_flags, sizeof state_flags);
    if (!ok) err = "cannot release handoff slot " + num(index);
    return ok;
}

bool HandoffArena::abort_claim(int index, uint64_t nonce, std::string& err) {
    std::lock_guard<std::mutex> guard(mu_);
    if (fd_ < 0) { err = "the handoff arena is not open"; return false; }
    if (!writer_) { err = "a reader never aborts a handoff claim"; return false; }
    FileLock lock(fd_, true);
    if (!lock.held()) { err = lock.error(); return false; }
    HandoffSlotHeader s{};
    Place p;
    if (!load_slot_(index, s, p) || s.nonce != nonce || s.state != kHandoffClaimed) {
        err = "handoff slot " + num(index) + " is not a claim of nonce " + hex16(nonce);
        return false;
    }
    const uint32_t flags = s.flags | kHandoffFlagPartial;
    const uint32_t free_state = kHandoffFree;
    const bool ok = store_(p.base + kSlotFlagsOffset, &flags, 4) && store_(p.base + kSlotStateOffset, &free_state, 4);
    if (!ok) err = "cannot abort handoff slot " + num(index);
    return ok;
}

bool HandoffArena::cancel(int index, uint64_t nonce, std::string& err) {
    std::lock_guard<std::mutex> guard(mu_);
    if (fd_ < 0) { err = "the handoff arena is not open"; return false; }
    if (!writer_) { err = "a reader never cancels a handoff job"; return false; }
    FileLock lock(fd_, true);
    if (!lock.held()) { err = lock.error(); return false; }
    HandoffSlotHeader s{};
    Place p;
    if (!load_slot_(index, s, p) || s.nonce != nonce) {
        err = "handoff slot " + num(index) + " is not the one nonce " + hex16(nonce) + " refers to";
        return false;
    }
    const uint32_t flags = s.flags | kHandoffFlagCancelled;
    if (!store_(p.base + kSlotFlagsOffset, &flags, 4)) {
        err = "cannot cancel handoff slot " + num(index);
        return false;
    }
    return true;
}

bool HandoffArena::map_all_(bool populate, std::string& err) {
    if (map_) return true;
    // the writer's mapping is writable; a reader's is read-only (its descriptor is too)
    void* m = ::mmap(nullptr, (size_t) hdr_.arena_bytes, writer_ ? PROT_READ | PROT_WRITE : PROT_READ,
                     MAP_SHARED | (populate ? MAP_POPULATE : 0), fd_, 0);
    if (m == MAP_FAILED) {
        err = "cannot map the handoff arena " + path_ + ": " + std::strerror(errno);
        return false;
    }
    map_ = static_cast<uint8_t*>(m);
    map_bytes_ = hdr_.arena_bytes;
    return true;
}

uint8_t* HandoffArena::claim_window(const HandoffClaim& c, std::string& err) {
    std::lock_guard<std::mutex> guard(mu_);
    if (fd_ < 0) { err = "the handoff arena is not open"; return nullptr; }
    if (!writer_) { err = "a reader never writes a handoff slot"; return nullptr; }
    Place p;
    if (!place_(c.index, p) || p.base != c.base || p.capacity != c.capacity ||
        c.payload_off != c.base + kHandoffHeaderBytes) {
        err = "handoff claim of slot " + num(c.index) + " does not match this arena's slot table";
        return nullptr;
    }
    if (!map_all_(false, err)) return nullptr;
    return map_ + c.payload_off;
}

bool HandoffArena::reserve(std::string& err) {
    std::lock_guard<std::mutex> guard(mu_);
    if (fd_ < 0) { err = "the handoff arena is not open"; return false; }
    if (!writer_) {
        // a reader commits nothing: it maps the file read-only with its page tables populated
        if (map_) {
            ::munmap(map_, (size_t) map_bytes_);
            map_ = nullptr;
        }
        return map_all_(true, err);
    }
    const int rc = ::posix_fallocate(fd_, 0, (off_t) hdr_.arena_bytes);
    if (rc != 0) {
        err = "cannot commit the " + num(hdr_.arena_bytes) + " B of handoff arena " + path_ + ": " + std::strerror(rc);
        return false;
    }
    if (map_) {
        ::munmap(map_, (size_t) map_bytes_);
        map_ = nullptr;
    }
    return map_all_(true, err);
}

// ================================ the reader ================================

bool HandoffArena::open_reader(const std::string& path, uint64_t pack_hash, uint64_t geom_hash, std::string& err) {
    // src/core/handoff.cpp:978-1018
    std::lock_guard<std::mutex> guard(mu_);
    close_();
    err.clear();
    const int fd = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
    if (fd < 0) {
        err = "cannot open the handoff arena " + path + ": " + std::strerror(errno);
        return false;
    }
    fd_ = fd;
    path_ = path;
    writer_ = false;
    std::string why;
    {
        FileLock lock(fd_, false);
        if (!lock.held()) {
            why = lock.error();
        } else {
            struct stat st {};
            HandoffArenaHeader h{};
            if (::fstat(fd_, &st) != 0 || !read_at(fd_, &h, sizeof h, 0)) {
                why = "handoff arena " + path + ": cannot read its header";
            } else if (adopt_header_(h, (uint64_t) st.st_size, why)) {
                if (h.pack_hash != pack_hash)
                    why = "handoff arena " + path + " was written for pack hash " + hex16(h.pack_hash) +
                          ", this instance is " + hex16(pack_hash);
                else if (h.geom_hash != geom_hash)
                    why = "handoff arena " + path + " was written for geometry hash " + hex16(h.geom_hash) +
                          ", this instance is " + hex16(geom_hash) + " (a different geometry or layer split)";
            }
        }
    }
    if (!why.empty()) {
        err = why;
        close_();
        return false;
    }
    return true;
}

bool HandoffArena::slot_info(int index, HandoffSlotInfo& out) const {
    std::lock_guard<std::mutex> guard(mu_);
    out = HandoffSlotInfo{};
    if (fd_ < 0) return false;
    HandoffSlotHeader s{};
    Place p;
    {
        FileLock lock(fd_, false);
        if (!lock.held() || !load_slot_(index, s, p)) return false;
    }
    out.index = index;
    out.base = p.base;
    out.capacity = p.capacity;
    out.state = s.state;
    out.flags = s.flags;
    out.tier = s.tier;
    out.owner_pid = s.owner_pid;
    out.owner_start = s.owner_start;
    out.nonce = s.nonce;
    out.client_id = s.client_id;
    out.request_id = s.request_id;
    out.pack_hash = s.pack_hash;
    out.geom_hash = s.geom_hash;
    out.tokens = s.tokens;
    out.payload_bytes = s.payload_bytes;
    out.payload_hash = s.payload_hash;
    out.claimed_ms = s.claimed_ms;
    out.published_ms = s.published_ms;
    out.seq = s.seq;
    return true;
}

/// The slot header under a shared lock and every check a reader makes before it copies a byte
/// (src/core/handoff.cpp:1053-1111).  The caller holds mu_.
bool HandoffArena::ready_slot_(int index, uint64_t expect_nonce, uint64_t client_id, HandoffSlotHeader& s, Place& p,
                               std::string& err) const {
    if (fd_ < 0) { err = "the handoff arena is not open"; return false; }
    if (writer_) { err = "open the arena as a reader to read a handoff slot"; return false; }
    {
        FileLock lock(fd_, false);
        if (!lock.held()) { err = lock.error(); return false; }
        if (!load_slot_(index, s, p)) {
            err = "cannot read the handoff slot header at index " + num(index);
            return false;
        }
    }
    const std::string slot = "handoff slot " + num(index);
    if (std::memcmp(s.magic, kSlotMagic, sizeof kSlotMagic) != 0 || s.version != kHandoffVersion ||
        s.header_bytes != kHandoffHeaderBytes) {
        err = slot + " has an incompatible header";
        return false;
    }
    if (s.state != kHandoffReady) {
        err = slot + " is " + (s.state == kHandoffClaimed ? "CLAIMED (its writer has not published it)" :
                               s.state == kHandoffFree ? "FREE" : "in state " + num(s.state)) + ", not READY";
        return false;
    }
    if (s.nonce != expect_nonce) {
        err = slot + " holds nonce " + hex16(s.nonce) + ", not the expected nonce " + hex16(expect_nonce);
        return false;
    }
    if (s.client_id != client_id) {
        err = slot + " is addressed to client " + hex16(s.client_id) + ", not " + hex16(client_id);
        return false;
    }
    if (s.pack_hash != hdr_.pack_hash || s.geom_hash != hdr_.geom_hash) {
        err = slot + " was written for pack " + hex16(s.pack_hash) + " / geometry " + hex16(s.geom_hash) +
              ", this arena is " + hex16(hdr_.pack_hash) + " / " + hex16(hdr_.geom_hash);
        return false;
    }
    if (s.payload_bytes > p.capacity) {
        err = slot + " claims " + num(s.payload_bytes) + " B in a " + num(p.capacity) + " B slot";
        return false;
    }
    if (s.seq != 1) {
        err = slot + " has seq " + num(s.seq) + "; this protocol version reads seq 1 only";
        return false;
    }
    return true;
}

bool HandoffArena::read_slot(int index, uint64_t expect_nonce, uint64_t client_id, HandoffPayload& out,
                             std::string& err) {
    // src/core/handoff.cpp:1053-1131: every check, then a PROT_READ mapping of the payload region only (from the
    // page holding its first byte)
    std::lock_guard<std::mutex> guard(mu_);
    out = HandoffPayload{};
    HandoffSlotHeader s{};
    Place p;
    if (!ready_slot_(index, expect_nonce, client_id, s, p, err)) return false;
    const uint64_t first = p.base + kHandoffHeaderBytes;
    const long ps = ::sysconf(_SC_PAGESIZE);
    const uint64_t page = ps > 0 ? (uint64_t) ps : 4096;
    const uint64_t lead = first % page;
    const uint64_t span = lead + std::max<uint64_t>(s.payload_bytes, 1);
    void* m = ::mmap(nullptr, (size_t) span, PROT_READ, MAP_SHARED, fd_, (off_t) (first - lead));
    if (m == MAP_FAILED) {
        err = "cannot map handoff slot " + num(index) + ": " + std::strerror(errno);
        return false;
    }
    out.bind_mapping(m, span, static_cast<const uint8_t*>(m) + lead, s.payload_bytes);
    out.index = index;
    out.tier = s.tier;
    out.nonce = s.nonce;
    out.client_id = s.client_id;
    out.request_id = s.request_id;
    out.tokens = s.tokens;
    out.payload_bytes = s.payload_bytes;
    out.payload_hash = s.payload_hash;
    out.seq = s.seq;
    return true;
}

const uint8_t* HandoffArena::read_window(int index, uint64_t expect_nonce, uint64_t client_id, HandoffSlotInfo& info,
                                         std::string& err) {
    std::lock_guard<std::mutex> guard(mu_);
    info = HandoffSlotInfo{};
    HandoffSlotHeader s{};
    Place p;
    if (!ready_slot_(index, expect_nonce, client_id, s, p, err)) return nullptr;
    if (!map_all_(false, err)) return nullptr;
    info.index = index;
    info.base = p.base;
    info.capacity = p.capacity;
    info.state = s.state;
    info.flags = s.flags;
    info.tier = s.tier;
    info.owner_pid = s.owner_pid;
    info.owner_start = s.owner_start;
    info.nonce = s.nonce;
    info.client_id = s.client_id;
    info.request_id = s.request_id;
    info.pack_hash = s.pack_hash;
    info.geom_hash = s.geom_hash;
    info.tokens = s.tokens;
    info.payload_bytes = s.payload_bytes;
    info.payload_hash = s.payload_hash;
    info.claimed_ms = s.claimed_ms;
    info.published_ms = s.published_ms;
    info.seq = s.seq;
    return map_ + p.base + kHandoffHeaderBytes;
}

uint64_t HandoffArena::payload_hash_of(const HandoffPayload& p) {
    return p.data ? fnv1a64(p.data, p.payload_bytes) : fnv1a64(nullptr, 0);
}

std::string HandoffArena::free_slots(std::string* err) const {
    std::lock_guard<std::mutex> guard(mu_);
    if (fd_ < 0) { if (err) *err = "the handoff arena is not open"; return "0/0"; }
    FileLock lock(fd_, false);
    if (!lock.held()) { if (err) *err = lock.error(); return "0/0"; }
    return num(count_free_()) + "/" + num(hdr_.slot_total);
}

}  // namespace strata::core

// Host page manager of the paged path: content-addressed, reference-counted physical KV
// pages with LRU eviction of idle immutable prefixes (src/inference/page_cache.rs:48-304),
// the prefix key chain (src/prefix_cache.rs:61-70) and the scheduler's per-step row
// construction (src/server/paged/schedule.rs:5-60).
//
// The reference scans the whole pool on every allocation and availability query.  Here the
// pool keeps two ordered indexes - idle pages without a key (by page id) and idle pages
// with a key (by last use) - plus an idle counter, so allocation is O(log pages) and picks
// exactly the page the reference's scan would: the lowest-numbered idle unkeyed page, else
// the least recently used idle keyed page (ages are unique, so ties cannot occur).
#include <array>
#include <cstring>
#include <map>
#include <set>
#include <utility>
#include <vector>

#include "../../include/lia_hip.h"

namespace {

// ------------------------------------------------------------------ SHA-256 (FIPS 180-4)

struct Sha256 {
    uint32_t h[8] = {0x6a09e667u, 0xbb67ae85u, 0x3c6ef372u, 0xa54ff53au,
                     0x510e527fu, 0x9b05688cu, 0x1f83d9abu, 0x5be0cd19u};
    uint8_t block[64];
    size_t used = 0;
    uint64_t length = 0;

    static uint32_t rotr(uint32_t x, int n) { return (x >> n) | (x << (32 - n)); }

    void compress(const uint8_t *p) {
        static const uint32_t k[64] = {
            0x428a2f98u, 0x71374491u, 0xb5c0fbcfu, 0xe9b5dba5u, 0x3956c25bu, 0x59f111f1u, 0x923f82a4u,
            0xab1c5ed5u, 0xd807aa98u, 0x12835b01u, 0x243185beu, 0x550c7dc3u, 0x72be5d74u, 0x80deb1feu,
            0x9bdc06a7u, 0xc19bf174u, 0xe49b69c1u, 0xefbe4786u, 0x0fc19dc6u, 0x240ca1ccu, 0x2de92c6fu,
            0x4a7484aau, 0x5cb0a9dcu, 0x76f988dau, 0x983e5152u, 0xa831c66du, 0xb00327c8u, 0xbf597fc7u,
            0xc6e00bf3u, 0xd5a79147u, 0x06ca6351u, 0x14292967u, 0x27b70a85u, 0x2e1b2138u, 0x4d2c6dfcu,
            0x53380d13u, 0x650a7354u, 0x766a0abbu, 0x81c2c92eu, 0x92722c85u, 0xa2bfe8a1u, 0xa81a664bu,
            0xc24b8b70u, 0xc76c51a3u, 0xd192e819u, 0xd6990624u, 0xf40e3585u, 0x106aa070u, 0x19a4c116u,
            0x1e376c08u, 0x2748774cu, 0x34b0bcb5u, 0x391c0cb3u, 0x4ed8aa4au, 0x5b9cca4fu, 0x682e6ff3u,
            0x748f82eeu, 0x78a5636fu, 0x84c87814u, 0x8cc70208u, 0x90befffau, 0xa4506cebu, 0xbef9a3f7u,
            0xc67178f2u};
        uint32_t w[64];
        for (int i = 0; i < 16; i++)
            w[i] = (uint32_t)p[4 * i] << 24 | (uint32_t)p[4 * i + 1] << 16 | (uint32_t)p[4 * i + 2] << 8 |
                   p[4 * i + 3];
        for (int i = 16; i < 64; i++) {
            const uint32_t s0 = rotr(w[i - 15], 7) ^ rotr(w[i - 15], 18) ^ (w[i - 15] >> 3);
            const uint32_t s1 = rotr(w[i - 2], 17) ^ rotr(w[i - 2], 19) ^ (w[i - 2] >> 10);
            w[i] = w[i - 16] + s0 + w[i - 7] + s1;
        }
        uint32_t a = h[0], b = h[1], c = h[2], d = h[3], e = h[4], f = h[5], g = h[6], hh = h[7];
        for (int i = 0; i < 64; i++) {
            const uint32_t t1 = hh + (rotr(e, 6) ^ rotr(e, 11) ^ rotr(e, 25)) + ((e & f) ^ (~e & g)) + k[i] + w[i];
            const uint32_t t2 = (rotr(a, 2) ^ rotr(a, 13) ^ rotr(a, 22)) + ((a & b) ^ (a & c) ^ (b & c));
            hh = g; g = f; f = e; e = d + t1; d = c; c = b; b = a; a = t1 + t2;
        }
        h[0] += a; h[1] += b; h[2] += c; h[3] += d; h[4] += e; h[5] += f; h[6] += g; h[7] += hh;
    }

    void update(const void *data, size_t n) {
        const uint8_t *p = (const uint8_t *)data;
        length += n;
        while (n) {
            const size_t take = std::min(n, 64 - used);
            memcpy(block + used, p, take);
            used += take; p += take; n -= take;
            if (used == 64) { compress(block); used = 0; }
        }
    }

    void finish(uint8_t out[32]) {
        const uint64_t bits = length * 8;
        const uint8_t one = 0x80, zero = 0;
        update(&one, 1);
        while (used != 56) update(&zero, 1);
        uint8_t be[8];
        for (int i = 0; i < 8; i++) be[i] = (uint8_t)(bits >> (56 - 8 * i));
        update(be, 8);
        for (int i = 0; i < 8; i++)
            for (int j = 0; j < 4; j++) out[4 * i + j] = (uint8_t)(h[i] >> (24 - 8 * j));
    }
};

using Key = std::array<uint8_t, 32>;

// Key::prefix (src/prefix_cache.rs:61-70): SHA-256 of the domain tag, the parent key, the
// token count as a little-endian u64 and the tokens as little-endian u32s.
Key prefix_key(const Key &parent, const uint32_t *tokens, size_t n) {
    static const char tag[] = "lia-kv-prefix-v1";
    Sha256 s;
    s.update(tag, sizeof(tag) - 1);
    s.update(parent.data(), 32);
    uint8_t le[8];
    for (int i = 0; i < 8; i++) le[i] = (uint8_t)((uint64_t)n >> (8 * i));
    s.update(le, 8);
    for (size_t i = 0; i < n; i++) {
        uint8_t t[4] = {(uint8_t)tokens[i], (uint8_t)(tokens[i] >> 8), (uint8_t)(tokens[i] >> 16),
                        (uint8_t)(tokens[i] >> 24)};
        s.update(t, 4);
    }
    Key out;
    s.finish(out.data());
    return out;
}

constexpr uint32_t kWindow = 16; // pages restored per transfer (the KV transfer window)

} // namespace

struct lia_sequence {
    std::vector<uint32_t> pages;
    std::vector<Key> keys;
};

struct lia_page_cache {
    struct Page {
        Key key;
        bool keyed = false;
        uint32_t users = 0;
        uint64_t age = 0;
    };
    Key ns;
    uint32_t page_size;
    lia_page_io io;
    std::vector<Page> pages;
    std::map<Key, uint32_t> prefixes;
    std::set<uint32_t> idle_unkeyed;                       // users == 0, no key
    std::set<std::pair<uint64_t, uint32_t>> idle_keyed;    // users == 0, key: (age, page)
    uint64_t clock = 0, gpu_hits = 0, evictions = 0;
    std::vector<uint8_t> scratch;                          // one page payload (eviction)

    // Index maintenance around every change of users / key / age of a page.
    void unindex(uint32_t p) {
        const Page &e = pages[p];
        if (e.users) return;
        if (e.keyed) idle_keyed.erase({e.age, p});
        else idle_unkeyed.erase(p);
    }
    void index(uint32_t p) {
        const Page &e = pages[p];
        if (e.users) return;
        if (e.keyed) idle_keyed.insert({e.age, p});
        else idle_unkeyed.insert(p);
    }
    size_t available() const { return idle_unkeyed.size() + idle_keyed.size(); }

    void touch(uint32_t p) {
        unindex(p);
        pages[p].age = ++clock;
        index(p);
    }
    void retain(uint32_t p) {
        unindex(p);
        pages[p].users++;
    }
    int release_page(uint32_t p) {
        if (pages[p].users == 0) return LIA_E_PAGE_UNDERFLOW;
        pages[p].users--;
        index(p);
        return LIA_OK;
    }
    void set_key(uint32_t p, const Key &k) {
        unindex(p);
        pages[p].key = k;
        pages[p].keyed = true;
        index(p);
        prefixes[k] = p;
    }

    // PageCache::evict (page_cache.rs:275-287): an idle keyed page goes to the store.
    int evict(uint32_t p) {
        if (pages[p].users) return LIA_E_ACTIVE_EVICT;
        if (!pages[p].keyed) return LIA_OK;
        if (io.put) {
            if (!io.read_page) return LIA_E_ARG;
            scratch.resize(io.page_bytes);
            int st = io.read_page(io.ctx, p, scratch.data());
            if (st) return st < 0 ? st : LIA_E_STORE;
            st = io.put(io.ctx, pages[p].key.data(), scratch.data());
            if (st) return st < 0 ? st : LIA_E_STORE;
        }
        prefixes.erase(pages[p].key);
        unindex(p);
        pages[p].keyed = false;
        index(p);
        evictions++;
        return LIA_OK;
    }

    // PageCache::allocate (page_cache.rs:250-273).  Returns 1 with *out set, 0 when every
    // page is in use, or a negative status.
    int allocate(uint32_t *out) {
        uint32_t p;
        if (!idle_unkeyed.empty()) p = *idle_unkeyed.begin();
        else if (!idle_keyed.empty()) p = idle_keyed.begin()->second;
        else return 0;
        if (pages[p].keyed) {
            const int st = evict(p);
            if (st) return st;
        }
        unindex(p);
        pages[p].users = 1;
        touch(p);
        *out = p;
        return 1;
    }

    void keys_of(const uint32_t *tokens, size_t n, std::vector<Key> &keys) const {
        const size_t count = n ? (n - 1) / page_size : 0;
        Key parent = ns;
        keys.clear();
        for (size_t b = 0; b < count; b++) {
            parent = prefix_key(parent, tokens + b * page_size, page_size);
            keys.push_back(parent);
        }
    }

    int release_all(lia_sequence *s) {
        int first = LIA_OK;
        for (uint32_t p : s->pages) {
            const int st = release_page(p);
            if (st && !first) first = st;
        }
        s->pages.clear();
        s->keys.clear();
        return first;
    }

    // PageCache::attach (page_cache.rs:48-157).
    int attach(const uint32_t *tokens, size_t n, lia_sequence *seq, size_t *cached) {
        std::vector<Key> keys;
        keys_of(tokens, n, keys);
        // Retain every resident match before allocating, so restoring an early hole can
        // never evict a later page of the same prefix.
        std::vector<int64_t> retained(keys.size(), -1);
        for (size_t i = 0; i < keys.size(); i++) {
            auto it = prefixes.find(keys[i]);
            if (it != prefixes.end()) {
                retain(it->second);
                retained[i] = it->second;
            }
        }
        int status = LIA_OK;
        std::vector<const void *> staged(kWindow);
        for (size_t w0 = 0; w0 < keys.size() && status == LIA_OK; w0 += kWindow) {
            const size_t w1 = std::min(keys.size(), w0 + kWindow);
            for (size_t i = w0; i < w1; i++) {
                staged[i - w0] = nullptr;
                if (retained[i] >= 0 || !io.load) continue;
                const int hit = io.load(io.ctx, keys[i].data(), &staged[i - w0]);
                if (hit < 0) { status = hit; break; }
                if (hit == 0) staged[i - w0] = nullptr;
            }
            if (status) break;
            std::vector<uint32_t> restored_pages;
            std::vector<const void *> restored_data;
            std::vector<Key> restored_keys;
            bool stop = false;
            for (size_t i = w0; i < w1; i++) {
                uint32_t page;
                if (retained[i] >= 0) {
                    page = (uint32_t)retained[i];
                    retained[i] = -1;
                    gpu_hits++;
                } else {
                    if (!staged[i - w0]) { stop = true; break; }
                    const int got = allocate(&page);
                    if (got < 0) { status = got; break; }
                    if (got == 0) { stop = true; break; }
                    restored_pages.push_back(page);
                    restored_data.push_back(staged[i - w0]);
                    restored_keys.push_back(keys[i]);
                }
                touch(page);
                seq->pages.push_back(page);
                seq->keys.push_back(keys[i]);
            }
            if (status == LIA_OK && !restored_pages.empty()) {
                if (!io.write_pages) status = LIA_E_ARG;
                else {
                    const int st = io.write_pages(io.ctx, (uint32_t)restored_pages.size(),
                                                  restored_pages.data(), restored_data.data());
                    if (st) status = st < 0 ? st : LIA_E_STORE;
                }
                if (status == LIA_OK)
                    for (size_t j = 0; j < restored_pages.size(); j++)
                        set_key(restored_pages[j], restored_keys[j]);
            }
            if (stop) break;
        }
        for (int64_t p : retained)
            if (p >= 0) release_page((uint32_t)p);
        if (status) {
            release_all(seq);
            return status;
        }
        *cached = seq->pages.size() * (size_t)page_size;
        return LIA_OK;
    }

    // PageCache::can_fit (page_cache.rs:163-180).
    bool can_fit(const uint32_t *tokens, size_t n) const {
        std::vector<Key> keys;
        keys_of(tokens, n, keys);
        size_t shared = 0;
        for (const Key &k : keys) {
            auto it = prefixes.find(k);
            if (it != prefixes.end() && pages[it->second].users > 0) shared++;
        }
        return (n + page_size - 1) / page_size <= available() + shared;
    }

    // PageCache::ensure_position (page_cache.rs:183-206): 1, 0 (pool occupied) or < 0.
    int ensure_position(lia_sequence *s, size_t position) {
        const size_t need = position / page_size + 1;
        if (need <= s->pages.size()) return 1;
        if (need - s->pages.size() > available()) return 0;
        while (s->pages.size() < need) {
            uint32_t p;
            const int got = allocate(&p);
            if (got <= 0) return got;
            s->pages.push_back(p);
        }
        return 1;
    }

    // PageCache::seal (page_cache.rs:208-237).
    int seal(lia_sequence *s, const uint32_t *tokens, size_t n, size_t computed) {
        if (computed > n || (computed + page_size - 1) / page_size > s->pages.size())
            return LIA_E_PREFIX_EXTENT;
        while (s->keys.size() < computed / page_size) {
            const size_t b = s->keys.size();
            const Key k = prefix_key(s->keys.empty() ? ns : s->keys.back(), tokens + b * page_size,
                                     page_size);
            const uint32_t current = s->pages[b];
            auto it = prefixes.find(k);
            if (it != prefixes.end()) {
                const uint32_t shared = it->second;
                if (shared != current) {
                    const int st = release_page(current);
                    if (st) return st;
                    retain(shared);
                    s->pages[b] = shared;
                }
            } else {
                if (pages[current].keyed) return LIA_E_IMMUTABLE_PAGE;
                set_key(current, k);
            }
            touch(s->pages[b]);
            s->keys.push_back(k);
        }
        return LIA_OK;
    }
};

// ------------------------------------------------------------------ C ABI

extern "C" int lia_prefix_key(const uint8_t parent[32], const uint32_t *tokens, size_t n_tokens,
                              uint8_t out[32]) {
    if (!parent || !out || (n_tokens && !tokens)) return LIA_E_ARG;
    Key p;
    memcpy(p.data(), parent, 32);
    const Key k = prefix_key(p, tokens, n_tokens);
    memcpy(out, k.data(), 32);
    return LIA_OK;
}

extern "C" int lia_page_cache_create(const uint8_t ns[32], uint32_t n_pages, uint32_t page_size,
                                     const lia_page_io *io, lia_page_cache **out) {
    if (!ns || !out || page_size == 0) return LIA_E_ARG;
    if (n_pages == 0) return LIA_E_CONFIG; // "empty KV page pool" (page_cache.rs:30)
    auto *pc = new lia_page_cache();
    memcpy(pc->ns.data(), ns, 32);
    pc->page_size = page_size;
    pc->io = io ? *io : lia_page_io{};
    pc->pages.resize(n_pages);
    for (uint32_t p = 0; p < n_pages; p++) pc->idle_unkeyed.insert(pc->idle_unkeyed.end(), p);
    *out = pc;
    return LIA_OK;
}

extern "C" void lia_page_cache_destroy(lia_page_cache *pc) { delete pc; }

extern "C" int lia_page_cache_attach(lia_page_cache *pc, const uint32_t *tokens, size_t n_tokens,
                                     lia_sequence **sequence, size_t *cached) {
    if (!pc || !sequence || !cached || (n_tokens && !tokens)) return LIA_E_ARG;
    auto *s = new lia_sequence();
    const int st = pc->attach(tokens, n_tokens, s, cached);
    if (st) {
        delete s;
        *sequence = nullptr;
        return st;
    }
    *sequence = s;
    return LIA_OK;
}

extern "C" int lia_page_cache_can_fit(const lia_page_cache *pc, const uint32_t *tokens,
                                      size_t n_tokens) {
    if (!pc || (n_tokens && !tokens)) return LIA_E_ARG;
    return pc->can_fit(tokens, n_tokens) ? 1 : 0;
}

extern "C" size_t lia_page_cache_available(const lia_page_cache *pc) {
    return pc ? pc->available() : 0;
}

extern "C" int lia_page_cache_ensure_position(lia_page_cache *pc, lia_sequence *sequence,
                                              size_t position) {
    if (!pc || !sequence) return LIA_E_ARG;
    return pc->ensure_position(sequence, position);
}

extern "C" int lia_page_cache_seal(lia_page_cache *pc, lia_sequence *sequence,
                                   const uint32_t *tokens, size_t n_tokens, size_t computed) {
    if (!pc || !sequence || (n_tokens && !tokens)) return LIA_E_ARG;
    return pc->seal(sequence, tokens, n_tokens, computed);
}

extern "C" int lia_page_cache_release(lia_page_cache *pc, lia_sequence *sequence) {
    if (!pc) return LIA_E_ARG;
    if (!sequence) return LIA_OK;
    const int st = pc->release_all(sequence);
    delete sequence;
    return st;
}

extern "C" int lia_page_cache_evict_idle(lia_page_cache *pc) {
    if (!pc) return LIA_E_ARG;
    for (uint32_t p = 0; p < pc->pages.size(); p++)
        if (pc->pages[p].users == 0 && pc->pages[p].keyed) {
            const int st = pc->evict(p);
            if (st) return st;
        }
    return LIA_OK;
}

extern "C" void lia_page_cache_stats(const lia_page_cache *pc, uint64_t *gpu_hits,
                                     uint64_t *evictions) {
    if (gpu_hits) *gpu_hits = pc ? pc->gpu_hits : 0;
    if (evictions) *evictions = pc ? pc->evictions : 0;
}

extern "C" uint32_t lia_sequence_pages(const lia_sequence *sequence, const uint32_t **pages) {
    if (!sequence) {
        if (pages) *pages = nullptr;
        return 0;
    }
    if (pages) *pages = sequence->pages.data();
    return (uint32_t)sequence->pages.size();
}

// Runtime::step's row construction (src/server/paged/schedule.rs:5-60): every active
// request gets prefill_batch / active rows (at least one) starting at its computed
// position, each row's page ensured first; a request stops at the first position the pool
// cannot hold.  A request whose last token is scheduled produces an output row.
extern "C" int lia_schedule_rows(lia_page_cache *pc, uint32_t n_slots, lia_request *requests,
                                 uint32_t prefill_batch, lia_paged_row *rows, uint32_t max_rows,
                                 uint32_t *n_rows, uint32_t *outputs, uint32_t *n_outputs,
                                 lia_update *updates, uint32_t *n_updates) {
    if (!pc || (n_slots && !requests) || !n_rows || !n_outputs || !n_updates) return LIA_E_ARG;
    *n_rows = *n_outputs = *n_updates = 0;
    uint32_t count = 0;
    for (uint32_t i = 0; i < n_slots; i++) count += requests[i].active != 0;
    if (count == 0) return LIA_OK;
    const size_t allowance = std::max<size_t>(prefill_batch / count, 1);
    for (uint32_t slot = 0; slot < n_slots; slot++) {
        lia_request &r = requests[slot];
        if (!r.active) continue;
        if (r.closed) {
            r.done = 1;
            continue;
        }
        if (!r.sequence || (r.n_tokens && !r.tokens) || r.computed > r.n_tokens) return LIA_E_ARG;
        const size_t end = std::min(r.computed + allowance, r.n_tokens);
        size_t computed = r.computed;
        for (size_t pos = r.computed; pos < end; pos++) {
            const int st = pc->ensure_position(r.sequence, pos);
            if (st < 0) return st;
            if (st == 0) break;
            if (*n_rows >= max_rows || !rows) return LIA_E_ROWS;
            rows[*n_rows] = lia_paged_row{r.tokens[pos], (uint32_t)pos, slot};
            ++*n_rows;
            computed++;
        }
        if (computed > r.computed) {
            const bool output = computed == r.n_tokens;
            if (output) {
                if (!outputs) return LIA_E_ARG;
                outputs[(*n_outputs)++] = *n_rows - 1;
            }
            if (!updates) return LIA_E_ARG;
            updates[(*n_updates)++] = lia_update{slot, (uint64_t)computed, output ? 1u : 0u};
        }
    }
    return LIA_OK;
}

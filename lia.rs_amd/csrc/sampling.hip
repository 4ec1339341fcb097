// Sparse sampling after the paged step (gfx950): the candidates kernel and the host-side
// sampler of Engine::forward_paged_sampled (src/inference/paged_sampling.rs:7-76).
//
// The kernel (llama_nucleus_candidates, src/gpu/kernels/llama_nucleus.rs:18-117) gives one
// wavefront to each (row, part of 1024 vocabulary entries): lane l holds entries
// part*1024 + l + 64j (j < 16), so every load instruction reads 256 contiguous bytes.  It
// writes the part's 21 largest entries by the total order of their f32 bits (ties: larger
// id first) as (id << 32 | bits) words, then the part's maximum and the f64 softmax mass
// sum exp((x - max) / T) (NaN when the part holds a NaN or +inf).  The host reduces the
// parts to one candidate list per row (src/gpu/nucleus.rs:103-143) and samples it: top-k
// from the candidates, nucleus only when the candidates prove the cutoff
// (checked_nucleus), else from the full logit row read back from the device.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <vector>

#include "common.hpp"
#include "launch.hpp"

// Every product and sum below is rounded on its own, as in the reference (no FMA contraction).
#pragma clang fp contract(off)

namespace lia {

constexpr uint32_t kSlots = 21;   // 20 candidates + the omitted-tail bound (nucleus.rs:4)
constexpr uint32_t kPart = 1024;
constexpr uint32_t kPerLane = kPart / 64;

// f32::total_cmp as a signed key: negative values have their magnitude bits flipped.
__host__ __device__ __forceinline__ int32_t total_key(uint32_t bits) {
    const int32_t s = (int32_t)bits;
    return s ^ (int32_t)((uint32_t)(s >> 31) >> 1);
}

__device__ __forceinline__ bool better(int32_t key, uint32_t id, int32_t bkey, uint32_t bid) {
    return key > bkey || (key == bkey && id > bid);
}

// Number of (lane, j) entries of the wave with pred(j) true: one ballot and one scalar bit
// count per register.
template <typename Pred>
__device__ __forceinline__ uint32_t wave_count(Pred pred) {
    uint32_t n = 0;
#pragma unroll
    for (uint32_t j = 0; j < kPerLane; j++) n += __builtin_popcountll(__ballot(pred(j)));
    return n;
}

// One wavefront per (row, part).  The k = min(21, visible) best entries are found without
// k serial argmax rounds (keys biased to unsigned: u = key ^ 0x80000000):
//  - the 21st largest lane maximum tau is a lower bound of the 21st largest entry (the 21
//    largest lane maxima are 21 distinct entries), so the entries >= tau - usually a few
//    dozen - contain the answer: when at most 64 survive they are ranked directly;
//  - otherwise (mass ties) a bit-by-bit search with ballot counts finds the k-th largest key
//    T, and a second search over the in-part offset settles ties at T (larger ids first).
// The selected entries are compacted into LDS and each lands at its rank.  "Visible" entries are the reference's selectable ones:
// inside the vocabulary and with a key above INT32_MIN (an all-ones NaN is never taken by
// its rounds).  Slots past k hold the reference's empty word (0xFFFFFFFF id, -inf bits).
__global__ __launch_bounds__(256) void nucleus_candidates_kernel(
        uint32_t vocab, uint32_t parts, uint32_t groups, const double *__restrict__ temperatures,
        const float *__restrict__ logits, uint64_t *__restrict__ candidates,
        double *__restrict__ normalizers) {
    __shared__ uint32_t stage_u[4][64], stage_off[4][64];
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t group = blockIdx.x * 4 + wave;
    if (group >= groups) return;                       // whole waves leave together
    const uint32_t row = group / parts, part = group % parts;
    const uint32_t base = part * kPart;
    const uint32_t live = min(vocab - base, kPart);
    // Bounded loads: entries past the part's live range read as 0 without touching memory,
    // so all 16 loads are issued back to back with no branch.
    const auto rsrc = make_rsrc(logits + (size_t)row * vocab + base, live * 4);
    float v[kPerLane];
#pragma unroll
    for (uint32_t j = 0; j < kPerLane; j++)
        v[j] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rsrc, (int)((lane + 64 * j) * 4), 0, 0));
    float mx = -INFINITY;
    bool invalid = false;
    uint32_t u[kPerLane];                               // biased order keys, 0 = not visible
#pragma unroll
    for (uint32_t j = 0; j < kPerLane; j++) {
        const bool in = lane + 64 * j < live;
        v[j] = in ? v[j] : -INFINITY;
        mx = fmaxf(mx, v[j]);                           // ignores NaN, as f32::max does
        invalid |= in && ((v[j] != v[j]) || v[j] == INFINITY);
        u[j] = in ? (uint32_t)total_key(__float_as_uint(v[j])) ^ 0x80000000u : 0u;
    }
#pragma unroll
    for (int o = 32; o; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
    double sum = 0.0;
    const double t = temperatures[row];
    if (t > 0.0 && isfinite(mx)) {
#pragma unroll
        for (uint32_t j = 0; j < kPerLane; j++) {
            const double e = exp(((double)v[j] - (double)mx) / t);
            sum += isfinite(v[j]) ? e : 0.0;
        }
    }
    if (__any(invalid)) sum = NAN;
#pragma unroll
    for (int o = 32; o; o >>= 1) sum += __shfl_xor(sum, o);
    if (lane == 0) {
        normalizers[2 * (size_t)group] = (double)mx;
        normalizers[2 * (size_t)group + 1] = sum;
    }

    const uint32_t visible = wave_count([&](uint32_t j) { return u[j] != 0; });
    const uint32_t k = min(visible, kSlots);
    // selection: u >= lo, and at u == lo only offsets >= I
    uint32_t lo = 1, I = 0, n_sel = k;
    if (k == kSlots) {
        uint32_t lm = 0;
#pragma unroll
        for (uint32_t j = 0; j < kPerLane; j++) lm = max(lm, u[j]);
        uint32_t tau = 0;                               // 21st largest lane maximum
        for (int bit = 31; bit >= 0; bit--) {
            const uint32_t c = tau | (1u << bit);
            if ((uint32_t)__builtin_popcountll(__ballot(lm >= c)) >= kSlots) tau = c;
        }
        const uint32_t n_s = tau ? wave_count([&](uint32_t j) { return u[j] >= tau; }) : 1024u;
        if (n_s <= 64) {
            lo = tau;
            n_sel = n_s;
        } else {
            uint32_t T = 0;                             // largest T with count(u >= T) >= 21
            for (int bit = 31; bit >= 0; bit--) {
                const uint32_t c = T | (1u << bit);
                if (wave_count([&](uint32_t j) { return u[j] >= c; }) >= kSlots) T = c;
            }
            const uint32_t r = kSlots - wave_count([&](uint32_t j) { return u[j] > T; });
            for (int bit = 9; bit >= 0; bit--) {        // the r largest offsets among u == T
                const uint32_t c = I | (1u << bit);
                if (wave_count([&](uint32_t j) { return u[j] == T && lane + 64 * j >= c; }) >= r) I = c;
            }
            lo = T;
        }
    }
    // compact the n_sel selected entries into LDS (any order), then rank them
    uint32_t at = 0;
#pragma unroll
    for (uint32_t j = 0; j < kPerLane; j++) {
        const uint32_t off = lane + 64 * j;
        const bool sel = k && (u[j] > lo || (u[j] == lo && off >= I));
        const uint64_t m = __ballot(sel);
        if (sel) {
            const uint32_t pos = at + __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32),
                                                               __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0));
            stage_u[wave][pos] = u[j];
            stage_off[wave][pos] = off;
        }
        at += __builtin_popcountll(m);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    uint64_t word = (uint64_t)0xFFFFFFFFu << 32 | __float_as_uint(-INFINITY);
    uint32_t rank = lane;                               // lanes k..20: empty slots
    if (lane < n_sel) {
        const uint32_t mu = stage_u[wave][lane], mo = stage_off[wave][lane];
        rank = 0;
        for (uint32_t m = 0; m < n_sel; m++) {
            const uint32_t ou = stage_u[wave][m], oo = stage_off[wave][m];
            rank += ou > mu || (ou == mu && oo > mo);
        }
        const uint32_t bits = (uint32_t)total_key(mu ^ 0x80000000u);   // the key map is an involution
        word = (uint64_t)(base + mo) << 32 | bits;
    }
    if (rank < kSlots) candidates[(size_t)group * kSlots + rank] = word;
}

// ------------------------------------------------------------------ host sampler

// MT19937 and the reference sampler's two-word canonical double (src/sampling/random.rs).
struct Mt19937 {
    uint32_t w[624];
    uint32_t index = 624;
    explicit Mt19937(uint32_t seed) {
        w[0] = seed;
        for (uint32_t i = 1; i < 624; i++) w[i] = 1812433253u * (w[i - 1] ^ (w[i - 1] >> 30)) + i;
    }
    uint32_t next() {
        if (index == 624) {
            for (uint32_t i = 0; i < 624; i++) {
                const uint32_t mixed = (w[i] & 0x80000000u) | (w[(i + 1) % 624] & 0x7fffffffu);
                w[i] = w[(i + 397) % 624] ^ (mixed >> 1) ^ ((mixed & 1) ? 0x9908b0dfu : 0u);
            }
            index = 0;
        }
        uint32_t v = w[index++];
        v ^= v >> 11;
        v ^= (v << 7) & 0x9d2c5680u;
        v ^= (v << 15) & 0xefc60000u;
        return v ^ (v >> 18);
    }
    double uniform() {
        const double low = next(), high = next();
        return std::min((low + high * 4294967296.0) / 18446744073709551616.0, std::nextafter(1.0, 0.0));
    }
};

// Position-keyed Gumbel-max draw (src/sampling/gumbel.rs): MurmurHash3 mixing of
// (seed lo, seed hi, position lo, token), a 32-bit uniform, and -ln(-ln(1-u)) with a
// series for small u.
static uint32_t rotl(uint32_t x, int r) { return (x << r) | (x >> (32 - r)); }
static uint32_t gumbel_hash(uint64_t seed, uint64_t position, uint32_t token) {
    uint32_t h = 0;
    const uint32_t words[4] = {(uint32_t)seed, (uint32_t)(seed >> 32), (uint32_t)position, token};
    for (uint32_t word : words) {
        const uint32_t k = rotl(word * 0xcc9e2d51u, 15) * 0x1b873593u;
        h = rotl(h ^ k, 13) * 5u + 0xe6546b64u;
    }
    h ^= 16;
    h ^= h >> 16;
    h *= 0x85ebca6bu;
    h ^= h >> 13;
    h *= 0xc2b2ae35u;
    return h ^ (h >> 16);
}
static float gumbel_uniform(uint32_t word) {
    return (float)(word >> 16) * (1.0f / 65536.0f) + ((float)(word & 65535) + 0.5f) * (1.0f / 4294967296.0f);
}
static float gumbel_noise(float u) {
    float negative_log;
    if (u < 0.25f) {
        float poly = 1.0f / 8.0f;
        for (int d = 7; d >= 1; d--) poly = fmaf(u, poly, 1.0f / (float)d);
        negative_log = u * poly;
    } else {
        negative_log = -logf(std::max(1.0f - u, 1.0f / 16777216.0f));
    }
    return -logf(negative_log);
}

using Cand = std::pair<uint32_t, float>;   // (token id, logit)
using Entry = std::pair<uint32_t, double>; // (token id, probability)

static int32_t key_of(float x) {
    uint32_t b;
    memcpy(&b, &x, 4);
    return total_key(b);
}
// The reference's candidate order: descending total order of the logit, then descending id.
static bool before(const Cand &a, const Cand &b) {
    const int32_t ka = key_of(a.second), kb = key_of(b.second);
    return ka != kb ? ka > kb : a.first > b.first;
}

} // namespace lia

using namespace lia;

struct lia_sampler {
    double temperature, top_p;
    uint32_t top_k;
    uint64_t seed;
    bool keyed;
    uint64_t position;
    Mt19937 random;
    lia_sampler(double t, uint32_t k, double p, uint64_t s, bool keyed)
        : temperature(t), top_p(p), top_k(k), seed(s), keyed(keyed), position(0), random((uint32_t)s) {}

    double weight(float v, double maximum) const { return std::exp(((double)v - maximum) / temperature); }

    // Sampling::distribution (src/sampling.rs:82-128).
    int distribution(std::vector<Cand> c, std::vector<Entry> &out) const {
        for (const Cand &x : c)
            if (std::isnan(x.second) || x.second == INFINITY) return LIA_E_SAMPLING_LOGITS;
        c.erase(std::remove_if(c.begin(), c.end(), [](const Cand &x) { return x.second == -INFINITY; }),
                c.end());
        if (top_k && c.size() > top_k) {
            std::nth_element(c.begin(), c.begin() + top_k, c.end(), before);
            c.resize(top_k);
        }
        std::sort(c.begin(), c.end(), before);
        if (c.empty()) return LIA_E_EMPTY_DISTRIBUTION;
        {
            std::vector<uint32_t> ids(c.size());
            for (size_t i = 0; i < c.size(); i++) ids[i] = c[i].first;
            std::sort(ids.begin(), ids.end());
            if (std::adjacent_find(ids.begin(), ids.end()) != ids.end()) return LIA_E_DUPLICATE_CANDIDATE;
        }
        const double mx = c[0].second;
        out.resize(c.size());
        double total = 0.0;
        for (size_t i = 0; i < c.size(); i++) {
            out[i] = {c[i].first, std::exp(((double)c[i].second - mx) / temperature)};
        }
        for (const Entry &e : out) total += e.second;
        double mass = 0.0;
        size_t keep = out.size();
        for (size_t i = 0; i < out.size(); i++) {
            mass += out[i].second;
            if (mass >= top_p * total) {
                keep = i + 1;
                break;
            }
        }
        out.resize(keep);
        total = 0.0;
        for (const Entry &e : out) total += e.second;
        for (Entry &e : out) e.second /= total;
        return LIA_OK;
    }

    // select_nucleus (src/sampling/nucleus.rs:96-124); leaves c's retained prefix sorted.
    int select_nucleus(std::vector<Cand> &c, double maximum, double total, std::vector<Entry> &out) const {
        if (c.empty()) return LIA_E_EMPTY_DISTRIBUTION;
        const double target = top_p * total;
        size_t count = std::min<size_t>(c.size(), 128);
        for (;;) {
            if (count < c.size()) {
                std::nth_element(c.begin(), c.begin() + count, c.end(), before);
                std::sort(c.begin(), c.begin() + count, before);
            }
            double mass = 0.0;
            for (size_t i = 0; i < count; i++) mass += weight(c[i].second, maximum);
            if (mass >= target || count == c.size()) break;
            count = std::min(count * 2, c.size());
        }
        std::sort(c.begin(), c.begin() + count, before);
        double mass = 0.0;
        out.clear();
        for (size_t i = 0; i < count; i++) {
            const double w = weight(c[i].second, maximum);
            mass += w;
            out.push_back({c[i].first, w});
            if (mass >= target) break;
        }
        if (!std::isfinite(mass) || !(mass > 0.0)) return LIA_E_NUCLEUS;
        for (Entry &e : out) e.second /= mass;
        return LIA_OK;
    }

    // distribution_logits (nucleus.rs:9-46): the full-row fallback.
    int distribution_logits(const float *logits, uint32_t vocab, std::vector<Entry> &out) const {
        std::vector<Cand> c;
        c.reserve(vocab);
        if (top_k != 0 || top_p == 1.0) {
            for (uint32_t i = 0; i < vocab; i++) c.push_back({i, logits[i]});
            return distribution(std::move(c), out);
        }
        for (uint32_t i = 0; i < vocab; i++)
            if (std::isnan(logits[i]) || logits[i] == INFINITY) return LIA_E_SAMPLING_LOGITS;
        for (uint32_t i = 0; i < vocab; i++)
            if (logits[i] != -INFINITY) c.push_back({i, logits[i]});
        if (c.empty()) return LIA_E_EMPTY_DISTRIBUTION;
        float mx = c[0].second;
        for (const Cand &x : c)
            if (key_of(x.second) > key_of(mx)) mx = x.second;
        double total = 0.0;
        for (const Cand &x : c) total += weight(x.second, (double)mx);
        return select_nucleus(c, (double)mx, total, out);
    }

    // checked_nucleus (nucleus.rs:49-93): 1 with out set, 0 when the sparse candidates cannot
    // prove the cutoff (the caller falls back to the full row), or a negative status.
    int checked_nucleus(std::vector<Cand> c, double maximum, double total, float omitted,
                        std::vector<Entry> &out) const {
        if (!std::isfinite(total) || !(total > 0.0) || !std::isfinite(maximum)) return LIA_E_NUCLEUS;
        if (top_p == 1.0) return 0;
        const int st = select_nucleus(c, maximum, total, out);
        if (st) return st;
        if (out.empty()) return 0;
        const size_t keep = out.size();
        if (c[keep - 1].first != out.back().first) return LIA_E_NUCLEUS;
        if (!(key_of(c[keep - 1].second) > key_of(omitted))) return 0;
        const double target = top_p * total;
        double through = 0.0;
        for (size_t i = 0; i < keep; i++) through += weight(c[i].second, maximum);
        const double before_last = through - weight(c[keep - 1].second, maximum);
        const double uncertainty = std::fabs(total) * 1e-10;
        if (before_last >= target - uncertainty || through <= target + uncertainty) return 0;
        return 1;
    }

    // Sampling::draw (src/sampling.rs:134-146).
    uint32_t draw(const std::vector<Entry> &d) {
        if (keyed) {
            const uint64_t pos = position++;
            uint32_t best = d[0].first;
            float best_score = 0.0f;
            bool have = false;
            for (const Entry &e : d) {
                const float score = (float)std::log(e.second) + gumbel_noise(gumbel_uniform(gumbel_hash(seed, pos, e.first)));
                const int32_t k = key_of(score), bk = key_of(best_score);
                if (!have || k > bk || (k == bk && e.first < best)) {
                    best = e.first;
                    best_score = score;
                    have = true;
                }
            }
            return best;
        }
        if (d.size() == 1) return d[0].first;
        const double sample = random.uniform();
        double cumulative = 0.0;
        for (const Entry &e : d) {
            cumulative += e.second;
            if (sample < cumulative) return e.first;
        }
        return d.back().first;
    }
};

extern "C" int lia_sampler_create(double temperature, uint32_t top_k, double top_p, uint64_t seed,
                                  int32_t position_keyed, lia_sampler **out) {
    if (!out) return LIA_E_ARG;
    if (!std::isfinite(temperature) || !(temperature > 0.0) || top_k > 20 || !std::isfinite(top_p) ||
        !(top_p > 0.0) || top_p > 1.0)
        return LIA_E_SAMPLER_SETTINGS; // Sampling::new (src/sampling.rs:33-58)
    *out = new lia_sampler(temperature, top_k, top_p, seed, position_keyed != 0);
    return LIA_OK;
}

extern "C" void lia_sampler_destroy(lia_sampler *s) { delete s; }

extern "C" void lia_sampler_set_position(lia_sampler *s, uint64_t position) {
    if (s && s->keyed) s->position = position;
}

extern "C" int lia_sampler_distribution(const lia_sampler *s, uint32_t n, const uint32_t *ids,
                                        const float *logits, uint32_t *out_ids, double *out_probs,
                                        uint32_t *n_out) {
    if (!s || !n_out || (n && (!ids || !logits || !out_ids || !out_probs))) return LIA_E_ARG;
    std::vector<Cand> c(n);
    for (uint32_t i = 0; i < n; i++) c[i] = {ids[i], logits[i]};
    std::vector<Entry> d;
    const int st = s->distribution(std::move(c), d);
    if (st) return st;
    for (size_t i = 0; i < d.size(); i++) {
        out_ids[i] = d[i].first;
        out_probs[i] = d[i].second;
    }
    *n_out = (uint32_t)d.size();
    return LIA_OK;
}

extern "C" int lia_sampler_draw(lia_sampler *s, uint32_t n, const uint32_t *ids, const double *probs,
                                uint32_t *token) {
    if (!s || !token || n == 0 || !ids || !probs) return LIA_E_ARG;
    std::vector<Entry> d(n);
    for (uint32_t i = 0; i < n; i++) d[i] = {ids[i], probs[i]};
    *token = s->draw(d);
    return LIA_OK;
}

static uint32_t nucleus_parts(uint32_t vocab) { return (vocab + kPart - 1) / kPart; }
static size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

extern "C" size_t lia_nucleus_workspace_bytes(uint32_t vocab, uint32_t rows) {
    const size_t g = (size_t)rows * nucleus_parts(vocab);
    return align_up(g * kSlots * 8, 256) + align_up(g * 16, 256) + align_up((size_t)rows * 8, 256);
}

extern "C" size_t lia_nucleus_host_bytes(uint32_t vocab, uint32_t rows) {
    return lia_nucleus_workspace_bytes(vocab, rows) + (size_t)vocab * 4;
}

extern "C" int lia_nucleus_candidates(uint32_t vocab, uint32_t rows, const double *temperatures,
                                      const float *logits, uint64_t *candidates,
                                      double *normalizers, lia_stream_t stream) {
    if (vocab == 0 || !temperatures || !logits || !candidates || !normalizers) return LIA_E_ARG;
    if (rows == 0) return LIA_OK;
    const uint64_t groups = (uint64_t)rows * nucleus_parts(vocab);
    if (groups > 0x3FFFFFFFu || (uint64_t)rows * vocab > 0xFFFFFFFFull) return LIA_E_ARG;
    const hipError_t e = launch<nucleus_candidates_kernel>(
        dim3((uint32_t)((groups + 3) / 4)), dim3(256), 0, (hipStream_t)stream, vocab,
        nucleus_parts(vocab), (uint32_t)groups, temperatures, logits, candidates, normalizers);
    return e == hipSuccess ? LIA_OK : LIA_E_HIP;
}

// Workspace::read's reduction and the per-row sampling of forward_paged_sampled, on host
// records.  `fetch_row(i, dst)` provides output row i's full logits for a fallback.
template <typename Fetch>
static int sample_records(uint32_t vocab, uint32_t n, lia_sampler *const *samplers,
                          const double *temps, const uint64_t *cand, const double *norm,
                          uint32_t *tokens, uint64_t *fallbacks, Fetch fetch_row) {
    const uint32_t parts = nucleus_parts(vocab);
    std::vector<Cand> c;
    std::vector<Entry> d;
    std::vector<float> row;
    for (uint32_t r = 0; r < n; r++) {
        const double *ns = norm + (size_t)r * parts * 2;
        double maximum = -INFINITY;
        for (uint32_t p = 0; p < parts; p++) {
            if (!std::isfinite(ns[2 * p + 1])) return LIA_E_SAMPLING_LOGITS;
            if (ns[2 * p] > maximum) maximum = ns[2 * p];
        }
        double total = 0.0;
        if (temps[r] > 0.0)
            for (uint32_t p = 0; p < parts; p++)
                if (ns[2 * p + 1] > 0.0) total += ns[2 * p + 1] * std::exp((ns[2 * p] - maximum) / temps[r]);
        c.clear();
        float omitted = -INFINITY;
        for (uint32_t p = 0; p < parts; p++) {
            const uint64_t *words = cand + ((size_t)r * parts + p) * kSlots;
            for (uint32_t rank = 0; rank < kSlots; rank++) {
                const uint32_t id = (uint32_t)(words[rank] >> 32);
                const uint32_t bits = (uint32_t)words[rank];
                float v;
                memcpy(&v, &bits, 4);
                if (id == 0xFFFFFFFFu || !std::isfinite(v)) continue;
                if (id >= vocab) return LIA_E_NUCLEUS;
                if (rank < kSlots - 1) c.push_back({id, v});
                else omitted = std::max(omitted, v);
            }
        }
        lia_sampler *s = samplers ? samplers[r] : nullptr;
        if (s) {
            int st;
            if (s->top_k != 0) {
                st = s->distribution(c, d);
            } else {
                st = s->checked_nucleus(c, maximum, total, omitted, d);
                if (st == 0) {
                    if (fallbacks) ++*fallbacks;
                    row.resize(vocab);
                    st = fetch_row(r, row.data());
                    if (st == LIA_OK) st = s->distribution_logits(row.data(), vocab, d);
                } else if (st == 1) {
                    st = LIA_OK;
                }
            }
            if (st) return st;
            tokens[r] = s->draw(d);
        } else {
            if (c.empty()) return LIA_E_EMPTY_DISTRIBUTION;
            Cand best = c[0];
            for (const Cand &x : c) {
                const int32_t k = key_of(x.second), bk = key_of(best.second);
                if (k > bk || (k == bk && x.first > best.first)) best = x;
            }
            tokens[r] = best.first;
        }
    }
    return LIA_OK;
}

static void temperatures_for(uint32_t n, lia_sampler *const *samplers, double *t) {
    for (uint32_t i = 0; i < n; i++) {
        const lia_sampler *s = samplers ? samplers[i] : nullptr;
        t[i] = s ? (s->top_k == 0 ? s->temperature : 0.0) : 0.0;
    }
}

extern "C" int lia_sample_host(uint32_t vocab, uint32_t n, lia_sampler *const *samplers,
                               const uint32_t *positions, const uint64_t *candidates,
                               const double *normalizers, const float *logits, uint32_t *tokens,
                               uint64_t *fallbacks) {
    if (vocab == 0 || (n && (!candidates || !normalizers || !tokens))) return LIA_E_ARG;
    for (uint32_t i = 0; i < n; i++)
        if (samplers && samplers[i] && positions) lia_sampler_set_position(samplers[i], positions[i]);
    std::vector<double> t(n);
    temperatures_for(n, samplers, t.data());
    return sample_records(vocab, n, samplers, t.data(), candidates, normalizers, tokens, fallbacks,
                          [&](uint32_t r, float *dst) {
                              if (!logits) return LIA_E_ARG;
                              memcpy(dst, logits + (size_t)r * vocab, (size_t)vocab * 4);
                              return LIA_OK;
                          });
}

extern "C" int lia_sample_paged(uint32_t vocab, uint32_t n, lia_sampler *const *samplers,
                                const uint32_t *positions, const float *logits, void *workspace,
                                size_t workspace_bytes, void *host, size_t host_bytes,
                                uint32_t *tokens, uint64_t *fallbacks, lia_stream_t stream) {
    if (vocab == 0 || !tokens || !logits || !workspace || !host) return LIA_E_ARG;
    if (n == 0) return LIA_OK;
    if (workspace_bytes < lia_nucleus_workspace_bytes(vocab, n) ||
        host_bytes < lia_nucleus_host_bytes(vocab, n))
        return LIA_E_WORKSPACE;
    const size_t g = (size_t)n * nucleus_parts(vocab);
    const size_t cand_bytes = align_up(g * kSlots * 8, 256), norm_bytes = align_up(g * 16, 256);
    uint8_t *ws = (uint8_t *)workspace, *hb = (uint8_t *)host;
    uint64_t *cand = (uint64_t *)ws;
    double *norm = (double *)(ws + cand_bytes);
    double *temps = (double *)(ws + cand_bytes + norm_bytes);
    double *htemps = (double *)(hb + cand_bytes + norm_bytes);
    float *hrow = (float *)(hb + lia_nucleus_workspace_bytes(vocab, n));
    for (uint32_t i = 0; i < n; i++)
        if (samplers && samplers[i] && positions) lia_sampler_set_position(samplers[i], positions[i]);
    temperatures_for(n, samplers, htemps);
    hipStream_t s = (hipStream_t)stream;
    if (hipMemcpyAsync(temps, htemps, (size_t)n * 8, hipMemcpyHostToDevice, s) != hipSuccess)
        return LIA_E_HIP;
    int st = lia_nucleus_candidates(vocab, n, temps, logits, cand, norm, stream);
    if (st) {
        (void)hipStreamSynchronize(s);
        return st;
    }
    if (hipMemcpyAsync(hb, ws, cand_bytes + norm_bytes, hipMemcpyDeviceToHost, s) != hipSuccess ||
        hipStreamSynchronize(s) != hipSuccess)
        return LIA_E_HIP;
    return sample_records(vocab, n, samplers, htemps, (const uint64_t *)hb,
                          (const double *)(hb + cand_bytes), tokens, fallbacks,
                          [&](uint32_t r, float *dst) {
                              if (hipMemcpyAsync(hrow, logits + (size_t)r * vocab, (size_t)vocab * 4,
                                                 hipMemcpyDeviceToHost, s) != hipSuccess ||
                                  hipStreamSynchronize(s) != hipSuccess)
                                  return LIA_E_HIP;
                              memcpy(dst, hrow, (size_t)vocab * 4);
                              return LIA_OK;
                          });
}

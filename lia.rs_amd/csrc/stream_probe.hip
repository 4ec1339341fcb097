// Streaming-rate probe for the paged decode pattern (measurement tool for bench.py; not
// part of the library).
//
// Reads the K and V planes of a paged pool the way a decode layer does - every live token
// of every (sequence, KV head) once - with loads that do nothing but fold the data into a
// register, so the time is the memory system's alone.  Five access patterns, the paged
// ones also with the non-temporal cache policy (`_nt`):
//   contiguous  both planes read front to back (the pool's bytes, no paging): the practical
//               read ceiling for a transfer of this size;
//   contiguous_1gib  one launch reading 1 GiB front to back: the sustained rate, without the
//               ramp and tail a launch of a few tens of microseconds pays;
//   slices      per-wave 64-byte d slices (the decode kernel's mapping on FP8 pools): a
//               4-wave workgroup per block range of a (sequence, KV head) unit, wave w
//               loading bytes [64w, 64w+64) of each token's head row (one load = 16 tokens x
//               64 bytes);
//   head_rows   whole head rows: one load = 64*16/(2D) tokens x 2D bytes, the waves of a
//               workgroup taking consecutive tokens of each 32-token chunk;
//   token_rows  whole token rows (every KV head): units are sequences.
// The pool is allocated `copies` times and the launches rotate over the copies, so no copy
// is still cache-resident when it is read again (MI355X has a 256 MB last-level cache).
//
// usage: stream_probe page_size hkv head_dim copies ctx0 [ctx1 ...]
// prints one JSON line per pattern: {"pattern", "us", "GBps", "bytes", "workgroups"}.
#include <hip/hip_runtime.h>
#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <random>
#include <vector>
#include <type_traits>

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

#define CHECK(x)                                                                         \
    do {                                                                                 \
        hipError_t e_ = (x);                                                             \
        if (e_ != hipSuccess) {                                                          \
            fprintf(stderr, "%s:%d %s: %s\n", __FILE__, __LINE__, #x, hipGetErrorString(e_)); \
            exit(1);                                                                     \
        }                                                                                \
    } while (0)

// AUX: cache policy of the load (0 default, 2 non-temporal)
template <int AUX = 0>
__device__ __forceinline__ u32x4 load16(const void *base, uint32_t bytes, uint32_t off) {
    const __amdgpu_buffer_rsrc_t r =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, bytes, 0x00020000);
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, AUX));
}

struct Range {
    uint32_t seq, head, c0, c1; // 32-token chunks [c0, c1) of (seq, head)
};

struct Pool {
    const uint8_t *k, *v;
    const uint32_t *table; // [seq][stride] physical pages
    const uint32_t *ctx;   // live tokens per sequence
    uint32_t stride, page_shift, row_bytes, head_bytes;
};

constexpr uint32_t kMaxPages = 4096; // per sequence (checked on the host)

enum { SLICES = 0, HEAD_ROWS = 1, TOKEN_ROWS = 2 };

// One workgroup of 256 threads per range, the next chunk's loads issued before the current
// chunk is folded.  NLP: loads per plane per wave and chunk (a 32-token chunk of S-byte
// spans is 32*S/1024 loads per plane; slots past it are bounded to nothing).
template <int MODE, int NLP, int AUX>
__global__ __launch_bounds__(256) void paged_read(Pool p, const Range *ranges, uint32_t *sink) {
    __shared__ uint32_t pages[kMaxPages];
    const Range w = ranges[blockIdx.x];
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t ctx = p.ctx[w.seq];
    const uint32_t P = 1u << p.page_shift;
    const uint32_t first_page = (32 * w.c0) >> p.page_shift;
    const uint32_t last_page = min((32 * w.c1 + P - 1) >> p.page_shift, (ctx + P - 1) >> p.page_shift);
    for (uint32_t i = first_page + threadIdx.x; i < last_page; i += blockDim.x)
        pages[i - first_page] = p.table[(size_t)w.seq * p.stride + i];
    __syncthreads();
    const uint32_t span = MODE == TOKEN_ROWS ? p.row_bytes : p.head_bytes;   // bytes read per token
    const uint32_t pieces = span / 16;                                       // 16-byte pieces per token
    const uint32_t tpi = MODE == SLICES ? 16 : 64 / pieces;                  // tokens per load
    const uint32_t base_off = MODE == TOKEN_ROWS ? 0 : w.head * p.head_bytes;
    u32x4 acc = {0, 0, 0, 0};
    constexpr int NL = 2 * NLP; // loads per wave and chunk (K then V)
    auto load = [&](u32x4 (&b)[NL], uint32_t c) {
#pragma unroll
        for (int i = 0; i < NL; i++) {
            const bool isv = i >= NLP;
            const uint32_t q = i % NLP;
            uint32_t tok, byte;
            if (MODE == SLICES) { // q = 16-token tile (NLP = 2)
                if (!isv) { tok = 16 * q + (lane & 15); byte = 64 * wave + 16 * (lane >> 4); }
                else { tok = 16 * q + (lane >> 2); byte = 64 * wave + 16 * (lane & 3); }
            } else {
                const uint32_t slot = q * 4 + wave; // load slot of the plane
                tok = slot * tpi + lane / pieces;
                byte = 16 * (lane % pieces);
            }
            const uint32_t tt = 32 * c + tok;
            const bool live = tok < 32 && byte < span && tt < ctx; // (slices at D 64: waves 0-1)
            const uint32_t page = live ? pages[(tt >> p.page_shift) - first_page] : 0u;
            const uint8_t *base = (isv ? p.v : p.k) + (size_t)page * P * p.row_bytes;
            b[i] = load16<AUX>(base, live ? P * p.row_bytes : 0u,
                          (tt & (P - 1)) * p.row_bytes + base_off + byte);
        }
    };
    u32x4 b0[NL], b1[NL];
    uint32_t c = w.c0;
    if (c < w.c1) load(b0, c);
    for (; c < w.c1; c += 2) {
        if (c + 1 < w.c1) load(b1, c + 1);
#pragma unroll
        for (int i = 0; i < NL; i++) acc ^= b0[i];
        if (c + 1 >= w.c1) break;
        if (c + 2 < w.c1) load(b0, c + 2);
#pragma unroll
        for (int i = 0; i < NL; i++) acc ^= b1[i];
    }
    sink[blockIdx.x * 256 + threadIdx.x] = acc.x ^ acc.y ^ acc.z ^ acc.w;
}

// Both planes front to back: workgroup i reads an equal share of each.
__global__ __launch_bounds__(256) void contiguous_read(const u32x4 *k, const u32x4 *v, uint32_t n16,
                                                       uint32_t *sink) {
    const uint32_t per = (n16 + gridDim.x - 1) / gridDim.x;
    const uint32_t lo = blockIdx.x * per, hi = min(n16, lo + per);
    u32x4 acc = {0, 0, 0, 0};
    for (uint32_t i = lo + threadIdx.x; i < hi; i += 4 * 256) {
        u32x4 x[8];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint32_t q = i + j * 256;
            x[j] = q < hi ? k[q] : u32x4{0, 0, 0, 0};
            x[4 + j] = q < hi ? v[q] : u32x4{0, 0, 0, 0};
        }
#pragma unroll
        for (int j = 0; j < 8; j++) acc ^= x[j];
    }
    sink[blockIdx.x * 256 + threadIdx.x] = acc.x ^ acc.y ^ acc.z ^ acc.w;
}

int main(int argc, char **argv) {
    if (argc < 6) {
        fprintf(stderr, "usage: %s page_size hkv head_dim copies ctx0 [ctx1 ...]\n", argv[0]);
        return 2;
    }
    const uint32_t P = atoi(argv[1]), hkv = atoi(argv[2]), D = atoi(argv[3]), copies = atoi(argv[4]);
    std::vector<uint32_t> ctx;
    for (int i = 5; i < argc; i++) ctx.push_back(atoi(argv[i]));
    uint32_t shift = 0;
    while ((1u << shift) < P) shift++;
    if ((1u << shift) != P || P < 16 || (D != 64 && D != 128) || copies < 1 || copies > 64) {
        fprintf(stderr, "unsupported shape\n");
        return 2;
    }
    const uint32_t nseq = ctx.size(), head_bytes = 2 * D, row_bytes = hkv * head_bytes;
    uint32_t pages = 0, maxp = 0;
    for (uint32_t c : ctx) {
        const uint32_t n = (c + P - 1) / P;
        pages += n;
        maxp = std::max(maxp, n);
    }
    if (maxp > kMaxPages) {
        fprintf(stderr, "a sequence has more than %u pages\n", kMaxPages);
        return 2;
    }
    const uint32_t stride = maxp;
    // loads per plane per wave of a whole-token-row chunk: 32 rows x row_bytes / (1 KB x 4 waves)
    const uint32_t nlp_rows = std::max(1u, 32 * row_bytes / 4096);
    if (nlp_rows > 8 || 32 * head_bytes / 4096 > 2) {
        fprintf(stderr, "unsupported row size\n");
        return 2;
    }
    // pages of all sequences scattered by a seeded permutation of the pool
    std::vector<uint32_t> perm(pages), table((size_t)nseq * stride, 0);
    for (uint32_t i = 0; i < pages; i++) perm[i] = i;
    std::mt19937 rng(0);
    std::shuffle(perm.begin(), perm.end(), rng);
    for (uint32_t s = 0, at = 0; s < nseq; s++)
        for (uint32_t i = 0; i < (ctx[s] + P - 1) / P; i++) table[(size_t)s * stride + i] = perm[at++];
    const size_t plane = (size_t)pages * P * row_bytes;
    std::vector<uint8_t *> kp(copies), vp(copies);
    for (uint32_t c = 0; c < copies; c++) {
        CHECK(hipMalloc(&kp[c], plane));
        CHECK(hipMalloc(&vp[c], plane));
        CHECK(hipMemset(kp[c], 0x11, plane));
        CHECK(hipMemset(vp[c], 0x22, plane));
    }
    uint32_t *dtable, *dctx, *sink;
    Range *dranges;
    const uint32_t max_wg = 4096;
    CHECK(hipMalloc(&dtable, table.size() * 4));
    CHECK(hipMemcpy(dtable, table.data(), table.size() * 4, hipMemcpyHostToDevice));
    CHECK(hipMalloc(&dctx, nseq * 4));
    CHECK(hipMemcpy(dctx, ctx.data(), nseq * 4, hipMemcpyHostToDevice));
    CHECK(hipMalloc(&sink, (size_t)max_wg * 256 * 4));
    CHECK(hipMalloc(&dranges, max_wg * sizeof(Range)));
    int cus = 0;
    CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, 0));
    double live_bytes = 0; // K and V of every live token, every head
    for (uint32_t c : ctx) live_bytes += 2.0 * c * row_bytes;
    const int reps = 50;
    auto timed = [&](auto launch) {
        for (uint32_t i = 0; i < 2 * copies; i++) launch(i % copies);
        hipEvent_t e0, e1;
        CHECK(hipEventCreate(&e0));
        CHECK(hipEventCreate(&e1));
        CHECK(hipEventRecord(e0));
        for (int i = 0; i < reps; i++) launch(i % copies);
        CHECK(hipEventRecord(e1));
        CHECK(hipEventSynchronize(e1));
        float ms = 0;
        CHECK(hipEventElapsedTime(&ms, e0, e1));
        CHECK(hipGetLastError());
        return ms * 1e3 / reps;
    };
    // contiguous
    {
        const uint32_t n16 = (uint32_t)(plane / 16), wgs = 3 * cus;
        const double us = timed([&](uint32_t c) {
            contiguous_read<<<wgs, 256>>>((const u32x4 *)kp[c], (const u32x4 *)vp[c], n16, sink);
        });
        printf("{\"pattern\": \"contiguous\", \"us\": %.3f, \"GBps\": %.1f, \"bytes\": %.0f, \"workgroups\": %u}\n",
               us, 2.0 * plane / us / 1e3, 2.0 * plane, wgs);
    }
    {
        const size_t big = (size_t)1 << 30; // 512 MiB per plane
        uint8_t *bk, *bv;
        CHECK(hipMalloc(&bk, big / 2));
        CHECK(hipMalloc(&bv, big / 2));
        CHECK(hipMemset(bk, 0x11, big / 2));
        CHECK(hipMemset(bv, 0x22, big / 2));
        const uint32_t n16 = (uint32_t)(big / 2 / 16), wgs = 3 * cus;
        const double us = timed([&](uint32_t) {
            contiguous_read<<<wgs, 256>>>((const u32x4 *)bk, (const u32x4 *)bv, n16, sink);
        });
        printf("{\"pattern\": \"contiguous_1gib\", \"us\": %.3f, \"GBps\": %.1f, \"bytes\": %.0f, \"workgroups\": %u}\n",
               us, (double)big / us / 1e3, (double)big, wgs);
        CHECK(hipFree(bk));
        CHECK(hipFree(bv));
    }
    // paged patterns: units' chunks laid end to end, cut into equal ranges (3 workgroups per
    // CU, as the decode kernel runs), split where a range crosses units
    auto paged = [&](int mode, bool nt, const char *name) {
        const bool rows = mode == TOKEN_ROWS;
        std::vector<Range> rs;
        std::vector<std::pair<uint32_t, uint32_t>> units; // (seq, head)
        std::vector<uint32_t> nch;
        uint32_t total = 0;
        for (uint32_t s = 0; s < nseq; s++)
            for (uint32_t h = 0; h < (rows ? 1u : hkv); h++) {
                units.push_back({s, h});
                nch.push_back((ctx[s] + 31) / 32);
                total += nch.back();
            }
        const uint32_t n = std::min<uint32_t>(3 * cus / (rows ? hkv : 1), total);
        for (uint32_t i = 0; i < n; i++) {
            const uint32_t b0 = (uint64_t)total * i / n, b1 = (uint64_t)total * (i + 1) / n;
            for (uint32_t u = 0, base = 0; u < units.size(); base += nch[u], u++) {
                const uint32_t lo = std::max(b0, base), hi = std::min(b1, base + nch[u]);
                if (lo < hi) rs.push_back({units[u].first, units[u].second, lo - base, hi - base});
            }
        }
        if (rs.size() > max_wg) {
            fprintf(stderr, "too many ranges\n");
            exit(2);
        }
        CHECK(hipMemcpy(dranges, rs.data(), rs.size() * sizeof(Range), hipMemcpyHostToDevice));
        const uint32_t wgs = rs.size();
        const double us = timed([&](uint32_t c) {
            const Pool pool{kp[c], vp[c], dtable, dctx, stride, shift, row_bytes, head_bytes};
            auto launch = [&](auto aux) {
                constexpr int A = decltype(aux)::value;
                if (mode == SLICES) paged_read<SLICES, 2, A><<<wgs, 256>>>(pool, dranges, sink);
                else if (mode == HEAD_ROWS) paged_read<HEAD_ROWS, 2, A><<<wgs, 256>>>(pool, dranges, sink);
                else if (nlp_rows <= 2) paged_read<TOKEN_ROWS, 2, A><<<wgs, 256>>>(pool, dranges, sink);
                else if (nlp_rows <= 4) paged_read<TOKEN_ROWS, 4, A><<<wgs, 256>>>(pool, dranges, sink);
                else paged_read<TOKEN_ROWS, 8, A><<<wgs, 256>>>(pool, dranges, sink);
            };
            if (nt) launch(std::integral_constant<int, 2>{});
            else launch(std::integral_constant<int, 0>{});
        });
        printf("{\"pattern\": \"%s\", \"us\": %.3f, \"GBps\": %.1f, \"bytes\": %.0f, \"workgroups\": %u}\n",
               name, us, live_bytes / us / 1e3, live_bytes, wgs);
    };
    paged(SLICES, false, "slices");
    paged(HEAD_ROWS, false, "head_rows");
    paged(TOKEN_ROWS, false, "token_rows");
    paged(SLICES, true, "slices_nt");
    paged(HEAD_ROWS, true, "head_rows_nt");
    paged(TOKEN_ROWS, true, "token_rows_nt");
    CHECK(hipDeviceSynchronize());
    return 0;
}

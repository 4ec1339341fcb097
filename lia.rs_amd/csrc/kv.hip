// Packing, slot mapping and KV-append scatter for the paged KV pool (gfx950).
#include "common.hpp"
#include "launch.hpp"

namespace lia {

// FP8 page scale for an append.  A page appended to before it was ever quantised holds
// scale 0; it takes scale 1, which the appending threads record (every writer stores the
// same value, and readers after the append see 1).
__device__ __forceinline__ float append_scale(float *scales, size_t at) {
    float s = scales[at];
    if (s == 0.0f) {
        s = 1.0f;
        scales[at] = 1.0f;
    }
    return s;
}

// Per-step packing on the device.  One workgroup scans the per-sequence new-token counts
// into cu_seqlens and then every thread fills rows: position = cached + i, sequence =
// table row, slot = pages[seq * stride + pos / P] * P + pos % P (the slot rule of
// src/inference/paging.rs:163-166 and src/gpu/kernels/llama.rs:174-177).
//
// Row checks, as Engine::run_paged makes them on the host (paging.rs:152-172), the lowest
// failing row first: position >= context (LIA_E_POSITION), the row's page missing
// (LIA_E_MISSING_PAGE), its slot written by an earlier row (LIA_E_DUPLICATE_SLOT).
// Positions within a sequence are consecutive by construction.  The table checks, which the
// reference makes ahead of the rows (paging.rs:137-144), are table_check_kernel's, launched
// right after.  On failure cu_seqlens is written all zero and all max_rows slots as "no
// slot", so a plan built from them schedules no work, no append writes the pool and the
// attention output is left untouched.
constexpr uint32_t kPackHash = 8192;  // LDS slot hash (open addressing, load <= 1/2 per pass)
constexpr uint32_t kPackPass = kPackHash / 2;

// Home bucket of a slot: the 16 slots of an aligned 16-slot group (the consecutive rows of a
// page) take the 16 buckets of one bucket group, chosen by a multiplicative hash of the group
// index, so they never collide with each other and their LDS accesses hit distinct banks.  A
// probe steps 17 buckets - the next group, the next offset - which visits every bucket.
__device__ __forceinline__ uint32_t slot_hash(uint32_t s) {
    return ((((s >> 4) * 2654435761u) >> 23) << 4) | (s & 15u); // 13 bits
}
constexpr uint32_t kPackProbe = 17;

// K independent upper-bound searches over arr[0 .. n) (n <= 1024, ascending): out[k] = the
// smallest index whose value exceeds v[k].  Branchless and with a fixed step count, so the K
// searches advance together instead of waiting on each other's LDS reads.
template <int K>
__device__ __forceinline__ void upper_many(const uint32_t *arr, uint32_t n, const uint32_t (&v)[K],
                                           uint32_t (&out)[K]) {
#pragma unroll
    for (int k = 0; k < K; k++) out[k] = 0;
    for (uint32_t step = 512; step; step >>= 1) {
        if (step > n) continue;  // uniform
        uint32_t x[K];
#pragma unroll
        for (int k = 0; k < K; k++) x[k] = arr[min(out[k] + step, n) - 1]; // every read issued
#pragma unroll
        for (int k = 0; k < K; k++) {
            const uint32_t at = out[k] + step; // candidate count of entries <= v
            out[k] = (at <= n && x[k] <= v[k]) ? at : out[k];
        }
    }
}

__global__ __launch_bounds__(1024) void pack_kernel(uint32_t n_seqs, const uint32_t *seq_slots,
                                                    const uint32_t *q_lens, const uint32_t *cached,
                                                    const uint32_t *pages, uint32_t stride,
                                                    uint32_t page_shift, uint32_t pool_pages,
                                                    uint32_t context, uint32_t max_rows,
                                                    uint32_t *cu, uint32_t *positions,
                                                    uint32_t *sequences, uint32_t *slot_mapping,
                                                    uint32_t *status) {
    __shared__ uint32_t scan[1024], s_slot[1024], s_c0[1024];
    __shared__ uint32_t h_key[kPackHash], h_row[kPackHash];
    __shared__ uint32_t w_a[16], w_b[16];
    // error: (row << 4) | code of the failing row with the lowest index, so the status is the
    // first failure in row order whatever the thread timing (codes are below 16)
    // dup: some insert found its slot already present (only then can a row fail the check)
    __shared__ uint32_t carry, error, dup;
    const uint32_t t = threadIdx.x;
    if (t == 0) { carry = 0; error = 0xFFFFFFFFu; dup = 0; }
    for (uint32_t i = t; i < kPackHash; i += 1024) { h_key[i] = kNone; h_row[i] = kNone; }
    const uint32_t P = 1u << page_shift;
    auto upper = [&](const uint32_t *arr, uint32_t n, uint32_t v) { // smallest b with arr[b] > v
        uint32_t a = 0, e = n;
        while (a < e) {
            const uint32_t mid = (a + e) >> 1;
            if (arr[mid] > v) e = mid; else a = mid + 1;
        }
        return a;
    };
    for (uint32_t base = 0; base < n_seqs; base += 1024) {
        const uint32_t b = base + t;
        const uint32_t n = b < n_seqs ? q_lens[b] : 0;
        const uint32_t slot = b < n_seqs ? seq_slots[b] : 0u, c0 = b < n_seqs ? cached[b] : 0u;
        uint32_t sc = n, unused = 0;
        block_scan2(sc, unused, w_a, w_b);
        s_slot[t] = slot;
        s_c0[t] = c0;
        scan[t] = sc;
        const uint32_t start = carry + sc - n;
        if (b < n_seqs) {
            cu[b] = start;
            if (b == n_seqs - 1) cu[n_seqs] = start + n;
        }
        lds_barrier();
        if (t == 1023) carry += scan[1023];
        lds_barrier();
    }
    const uint32_t total = carry;
    // rejects the batch: no sequence has rows, no row has a slot (all max_rows slots, so a
    // launch given more rows than the batch holds finds none either)
    auto reject = [&](uint32_t code) {
        for (uint32_t b = t; b <= n_seqs; b += 1024) cu[b] = 0;
        for (uint32_t r = t; r < max_rows; r += 1024) slot_mapping[r] = kNone;
        if (t == 0) *status = code;
    };
    if (total > max_rows) {
        __syncthreads(); // the cu stores above land before the rejection overwrites them
        reject((uint32_t)(-LIA_E_ROWS));
        return;
    }
    // Duplicate slots: slots are hashed keeping the lowest row per slot; a row whose slot has a
    // lower row fails.  Up to kPackPass rows take one pass, inserted while the rows are filled;
    // larger batches take one pass per hash class of slots (slot % passes), reading the slots
    // back.
    const uint32_t passes = (total + kPackPass - 1) / kPackPass;
    auto insert = [&](uint32_t s, uint32_t r) {
        uint32_t h = slot_hash(s), probes = 0;
        for (; probes < kPackHash; probes++) {
            const uint32_t k = atomicCAS(&h_key[h], kNone, s);
            if (k == s) dup = 1;
            if (k == kNone || k == s) { atomicMin(&h_row[h], r); break; }
            h = (h + kPackProbe) & (kPackHash - 1);
        }
        if (probes == kPackHash) { // table full (a pathological slot pattern): scan the rows
            for (uint32_t q = 0; q < r; q++)
                if (slot_mapping[q] == s) { atomicMin(&error, (r << 4) | (uint32_t)(-LIA_E_DUPLICATE_SLOT)); break; }
        }
    };
    auto lookup = [&](uint32_t s, uint32_t r) {
        uint32_t h = slot_hash(s);
        for (uint32_t probes = 0; probes < kPackHash; probes++) {
            const uint32_t k = h_key[h];
            if (k == s) {
                if (h_row[h] < r) atomicMin(&error, (r << 4) | (uint32_t)(-LIA_E_DUPLICATE_SLOT));
                return;
            }
            if (k == kNone) return;
            h = (h + kPackProbe) & (kPackHash - 1);
        }
    };
    // the row's slot from its page (loaded by the caller), with the row checks
    auto finish = [&](uint32_t r, uint32_t pos, uint32_t slot, uint32_t page) {
        uint32_t s = kNone;
        if (pos >= context) atomicMin(&error, (r << 4) | (uint32_t)(-LIA_E_POSITION));
        else if (page >= pool_pages) atomicMin(&error, (r << 4) | (uint32_t)(-LIA_E_MISSING_PAGE));
        else s = page * P + (pos & (P - 1));
        positions[r] = pos;
        sequences[r] = slot;
        slot_mapping[r] = s;
        return s;
    };
    auto page_of = [&](uint32_t pos, uint32_t slot) {
        return pos < context ? pages[(size_t)slot * stride + (pos >> page_shift)] : kNone;
    };
    if (n_seqs <= 1024 && passes <= 1) {
        // Rows in parallel (at most 4 per thread, slots kept in registers): row r belongs to
        // the first sequence whose inclusive prefix sum exceeds r.  The rows' page loads are
        // issued together with the table check's.
        constexpr uint32_t RPT = kPackPass / 1024;
        uint32_t mine[RPT], pos[RPT], sl[RPT], pg[RPT];
        auto rows = [&] {
            uint32_t rr[RPT], seq[RPT];
#pragma unroll
            for (uint32_t k = 0; k < RPT; k++) rr[k] = min(t + k * 1024, total ? total - 1 : 0u);
            upper_many<RPT>(scan, n_seqs, rr, seq);
#pragma unroll
            for (uint32_t k = 0; k < RPT; k++) {
                const uint32_t r = t + k * 1024, a = seq[k];
                pos[k] = s_c0[a] + r - (a ? scan[a - 1] : 0u);
                sl[k] = s_slot[a];
                pg[k] = r < total ? page_of(pos[k], sl[k]) : kNone;
            }
        };
        rows();
#pragma unroll
        for (uint32_t k = 0; k < RPT; k++) {
            const uint32_t r = t + k * 1024;
            mine[k] = kNone;
            if (r < total) {
                mine[k] = finish(r, pos[k], sl[k], pg[k]);
                if (mine[k] != kNone) insert(mine[k], r);
            }
        }
        lds_barrier(); // the hash (LDS); the rows' global stores need not have landed
        if (dup) { // uniform; with no slot inserted twice no row can fail
#pragma unroll
            for (uint32_t k = 0; k < RPT; k++)
                if (mine[k] != kNone) lookup(mine[k], t + k * 1024);
        }
    } else {
        if (n_seqs <= 1024) {
            for (uint32_t r = t; r < total; r += 1024) {
                const uint32_t a = upper(scan, n_seqs, r);
                const uint32_t p = s_c0[a] + r - (a ? scan[a - 1] : 0u);
                finish(r, p, s_slot[a], page_of(p, s_slot[a]));
            }
        } else {
            // more sequences than the LDS copies hold: walk sequences, threads stride over each
            // sequence's rows
            for (uint32_t b = 0; b < n_seqs; b++) {
                const uint32_t start = cu[b], n = q_lens[b], slot = seq_slots[b], c0 = cached[b];
                for (uint32_t i = t; i < n; i += 1024) finish(start + i, c0 + i, slot, page_of(c0 + i, slot));
            }
        }
        __threadfence_block(); // this workgroup's slot_mapping writes, read back below
        __syncthreads();
        for (uint32_t pass = 0; pass < passes; pass++) {
            if (pass) {
                for (uint32_t i = t; i < kPackHash; i += 1024) { h_key[i] = kNone; h_row[i] = kNone; }
                __syncthreads();
            }
            for (uint32_t r = t; r < total; r += 1024) {
                const uint32_t s = slot_mapping[r];
                if (s != kNone && s % passes == pass) insert(s, r);
            }
            __syncthreads();
            if (dup) { // uniform
                for (uint32_t r = t; r < total; r += 1024) {
                    const uint32_t s = slot_mapping[r];
                    if (s != kNone && s % passes == pass) lookup(s, r);
                }
            }
            __syncthreads();
        }
    }
    lds_barrier();
    const uint32_t code = error == 0xFFFFFFFFu ? 0u : (error & 15u); // uniform
    if (code) {
        // nothing downstream may run on a rejected batch; every row store of the workgroup
        // lands before the rejection overwrites it
        __syncthreads();
        reject(code);
    } else if (t == 0) {
        *status = 0;
    }
}

// Table checks of a packed step, launched right after pack_kernel.  The reference checks the
// tables ahead of the rows (paging.rs:137-144): every entry a sequence with rows attends
// (logical pages 0 .. ceil((cached + q_len) / P) - 1, within its row) that is neither a pool
// page nor "no page" is LIA_E_PAGE_RANGE; "no page" wholly below the cached length is
// LIA_E_MISSING_PAGE (the reference's tables cannot hold one; the attention kernels would read
// it).  Both take precedence over the row checks (PAGE_RANGE over MISSING_PAGE) and yield to a
// row-count failure, which the reference checks first.  A failing batch is rejected as
// pack_kernel rejects one.  The workgroups split the flattened entries (16-byte quads when
// table rows are 16-byte aligned); each builds the per-sequence prefix sums it searches
// itself, 256 sequences at a time.
constexpr uint32_t kCheckThreads = 256, kCheckGroups = 64;

__global__ __launch_bounds__(kCheckThreads) void table_check_kernel(
    uint32_t n_seqs, const uint32_t *seq_slots, const uint32_t *q_lens, const uint32_t *cached,
    const uint32_t *pages, uint32_t stride, uint32_t page_shift, uint32_t pool_pages,
    uint32_t context, uint32_t max_rows, uint32_t *cu, uint32_t *slot_mapping, uint32_t *status) {
    __shared__ uint32_t iscan[kCheckThreads], s_slot[kCheckThreads], s_c0[kCheckThreads],
        s_npg[kCheckThreads], w_a[16], w_b[16];
    __shared__ uint32_t found; // bit 0: a page outside the pool, bit 1: a missing cached page
    const uint32_t t = threadIdx.x, P = 1u << page_shift;
    if (t == 0) found = 0;
    const bool quads = (stride & 3) == 0 && ((uintptr_t)pages & 15) == 0;
    const uint32_t per = quads ? 4u : 1u;
    constexpr int K = 4; // items in flight per thread
    for (uint32_t base = 0; base < n_seqs; base += kCheckThreads) {
        const uint32_t b = base + t;
        const uint32_t n = b < n_seqs ? q_lens[b] : 0u, c0 = b < n_seqs ? cached[b] : 0u;
        const uint32_t keys = min(c0 + n, context);
        const uint32_t npg = n ? min((keys + P - 1) >> page_shift, stride) : 0u;
        uint32_t items = (npg + per - 1) / per, unused = 0;
        s_slot[t] = b < n_seqs ? seq_slots[b] : 0u;
        s_c0[t] = c0;
        s_npg[t] = npg;
        block_scan2(items, unused, w_a, w_b);
        iscan[t] = items;
        __syncthreads();
        const uint32_t cnt = min(n_seqs - base, kCheckThreads), total = iscan[cnt - 1];
        const uint32_t step = gridDim.x * kCheckThreads;
        for (uint32_t e0 = blockIdx.x * kCheckThreads + t; e0 < total; e0 += K * step) {
            uint32_t e[K], bl[K];
#pragma unroll
            for (int k = 0; k < K; k++) e[k] = min(e0 + k * step, total - 1);
            upper_many<K>(iscan, cnt, e, bl);
            u32x4 v[K];
#pragma unroll
            for (int k = 0; k < K; k++) {
                const uint32_t lp = (e[k] - (bl[k] ? iscan[bl[k] - 1] : 0u)) * per;
                const uint32_t *row = pages + (size_t)s_slot[bl[k]] * stride + lp;
                v[k] = quads ? *(const u32x4 *)row : u32x4{*row, kNone, kNone, kNone};
            }
            uint32_t bits = 0;
#pragma unroll
            for (int k = 0; k < K; k++) {
                if (e0 + k * step >= total) break;
                const uint32_t lp = (e[k] - (bl[k] ? iscan[bl[k] - 1] : 0u)) * per;
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const uint32_t lpq = lp + q, x = v[k][q];
                    if (q >= (int)per || lpq >= s_npg[bl[k]]) break;
                    if (x != kNone && x >= pool_pages) bits |= 1;
                    if (x == kNone && (lpq + 1) * P <= s_c0[bl[k]]) bits |= 2;
                }
            }
            if (bits) atomicOr(&found, bits);
        }
        __syncthreads(); // the LDS arrays are rewritten by the next chunk of sequences
    }
    if (!found) return;
    for (uint32_t b = t; b <= n_seqs; b += kCheckThreads) cu[b] = 0;
    for (uint32_t r = t; r < max_rows; r += kCheckThreads) slot_mapping[r] = kNone;
    if (t == 0) {
        const uint32_t want = (found & 1) ? (uint32_t)(-LIA_E_PAGE_RANGE) : (uint32_t)(-LIA_E_MISSING_PAGE);
        uint32_t old = __hip_atomic_load(status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        while (old != (uint32_t)(-LIA_E_ROWS) && old != (uint32_t)(-LIA_E_PAGE_RANGE) && old != want) {
            const uint32_t prev = atomicCAS(status, old, want);
            if (prev == old) break;
            old = prev;
        }
    }
}

// Slot of append row r (slot_mapping[r], or the table's page of its position); kNone for
// "no slot" and for any slot outside the pool, whose row is then not written.
__device__ __forceinline__ uint32_t row_slot(uint32_t r, const uint32_t *slot_mapping,
                                             const uint32_t *positions, const uint32_t *sequences,
                                             const uint32_t *pages, uint32_t stride,
                                             uint32_t page_shift, uint32_t pool_pages) {
    if (slot_mapping) {
        const uint32_t slot = slot_mapping[r];
        return (slot >> page_shift) < pool_pages ? slot : kNone;
    }
    const uint32_t pos = positions[r];
    const uint32_t page = pages[(size_t)sequences[r] * stride + (pos >> page_shift)];
    return page < pool_pages ? page * (1u << page_shift) + (pos & ((1u << page_shift) - 1)) : kNone;
}

template <typename SRC>
__device__ __forceinline__ float load_src(const SRC *p, size_t i);
template <>
__device__ __forceinline__ float load_src<float>(const float *p, size_t i) { return p[i]; }
template <>
__device__ __forceinline__ float load_src<uint16_t>(const uint16_t *p, size_t i) {
    return bf16_to_f32(p[i]);
}

// KV append: one thread per (row, 4 consecutive elements).  Mirrors llama_cache_paged
// (src/gpu/kernels/llama.rs:162-183) for any head count / head_dim / page size and the
// three pool element types.  src_kind: 0 = f32, 1 = f16, 2 = bf16.
template <int KVT>
__global__ __launch_bounds__(256) void append_kernel(uint32_t rows, uint32_t width, uint32_t hd,
                                                     uint32_t hkv, const uint32_t *positions,
                                                     const uint32_t *sequences,
                                                     const uint32_t *pages, uint32_t stride,
                                                     uint32_t page_shift, uint32_t pool_pages,
                                                     const uint32_t *slot_mapping, int src_kind,
                                                     const void *k, const void *v, void *kc,
                                                     void *vc, float *k_scales,
                                                     float *v_scales) {
    const size_t i = ((size_t)blockIdx.x * 256 + threadIdx.x);
    const uint32_t quads = width / 4;
    if (i >= (size_t)rows * quads) return;
    const uint32_t r = (uint32_t)(i / quads), e0 = (uint32_t)(i % quads) * 4;
    const uint32_t slot = row_slot(r, slot_mapping, positions, sequences, pages, stride, page_shift, pool_pages);
    if (slot == kNone) return;
    float kx[4], vx[4];
    size_t src = (size_t)r * width + e0;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        if (src_kind == 0) {
            kx[j] = ((const float *)k)[src + j];
            vx[j] = ((const float *)v)[src + j];
        } else if (src_kind == 1) {
            kx[j] = f16_to_f32(((const uint16_t *)k)[src + j]);
            vx[j] = f16_to_f32(((const uint16_t *)v)[src + j]);
        } else {
            kx[j] = bf16_to_f32(((const uint16_t *)k)[src + j]);
            vx[j] = bf16_to_f32(((const uint16_t *)v)[src + j]);
        }
    }
    size_t dst = (size_t)slot * width + e0;
    if constexpr (KVT == LIA_FP8_E4M3) {
        uint32_t page = slot >> page_shift, h = e0 / hd;
        const float ks = append_scale(k_scales, (size_t)page * hkv + h);
        const float vs = append_scale(v_scales, (size_t)page * hkv + h);
        uint32_t kw = 0, vw = 0;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            kw |= (uint32_t)f32_to_e4m3(kx[j] / ks) << (8 * j);
            vw |= (uint32_t)f32_to_e4m3(vx[j] / vs) << (8 * j);
        }
        *(uint32_t *)((uint8_t *)kc + dst) = kw;
        *(uint32_t *)((uint8_t *)vc + dst) = vw;
    } else {
        uint16_t kh[4], vh[4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            kh[j] = KVT == LIA_BF16 ? f32_to_bf16(kx[j]) : f32_to_f16(kx[j]);
            vh[j] = KVT == LIA_BF16 ? f32_to_bf16(vx[j]) : f32_to_f16(vx[j]);
        }
        u32x2 kq = u32x2{(uint32_t)kh[0] | ((uint32_t)kh[1] << 16), (uint32_t)kh[2] | ((uint32_t)kh[3] << 16)};
        u32x2 vq = u32x2{(uint32_t)vh[0] | ((uint32_t)vh[1] << 16), (uint32_t)vh[2] | ((uint32_t)vh[3] << 16)};
        *(u32x2 *)((uint16_t *)kc + dst) = kq;
        *(u32x2 *)((uint16_t *)vc + dst) = vq;
    }
}

// FP8 page quantisation: one workgroup per (page, kv head, plane).  The scale is the
// page's absolute maximum over that head / 448, 1 for an all-zero page.
__global__ __launch_bounds__(256) void quantize_kernel(uint32_t P, uint32_t hkv, uint32_t hd,
                                                       const uint32_t *page_ids, int src_kind,
                                                       const void *k, const void *v, void *kc,
                                                       void *vc, float *k_scales,
                                                       float *v_scales) {
    __shared__ float red[256];
    const uint32_t n = blockIdx.x, h = blockIdx.y, plane = blockIdx.z, t = threadIdx.x;
    const void *src = plane ? v : k;
    uint8_t *dst = (uint8_t *)(plane ? vc : kc);
    float *scales = plane ? v_scales : k_scales;
    const uint32_t page = page_ids[n];
    const uint32_t count = P * hd;
    auto at = [&](uint32_t e) -> size_t {
        uint32_t tok = e / hd, d = e % hd;
        return (((size_t)n * P + tok) * hkv + h) * hd + d;
    };
    auto val = [&](size_t i) -> float {
        if (src_kind == 0) return ((const float *)src)[i];
        if (src_kind == 1) return f16_to_f32(((const uint16_t *)src)[i]);
        return bf16_to_f32(((const uint16_t *)src)[i]);
    };
    float amax = 0.0f;
    for (uint32_t e = t; e < count; e += 256) amax = fmaxf(amax, fabsf(val(at(e))));
    red[t] = amax;
    __syncthreads();
    for (uint32_t off = 128; off > 0; off >>= 1) {
        if (t < off) red[t] = fmaxf(red[t], red[t + off]);
        __syncthreads();
    }
    float s = red[0] > 0.0f ? red[0] / 448.0f : 1.0f;
    if (t == 0) scales[(size_t)page * hkv + h] = s;
    for (uint32_t e = t; e < count; e += 256) {
        uint32_t tok = e / hd, d = e % hd;
        dst[(((size_t)page * P + tok) * hkv + h) * hd + d] = f32_to_e4m3(val(at(e)) / s);
    }
}

// RoPE coefficient table [rows][head_dim/2][2] = {cos, sin}(position * inv_i) with
// inv_i = f32(1 / f32(base^(2i/head_dim))), the rounded steps of coefficients
// (src/gpu/kernels/llama_position.rs:36-47).  pow, cos and sin are evaluated in double and
// rounded once to f32.
__global__ __launch_bounds__(256) void rope_coefficients_kernel(uint32_t rows, uint32_t head_dim,
                                                                float base,
                                                                const uint32_t *positions,
                                                                float *out) {
    const uint32_t half = head_dim / 2;
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    if (i >= rows * half) return;
    const float e = 2.0f * (float)(i % half) / (float)head_dim;
    const float p = (float)pow((double)base, (double)e);
    const float inv = 1.0f / p;
    const float angle = (float)positions[i / half] * inv;
    float2 cs;
    cs.x = (float)cos((double)angle);
    cs.y = (float)sin((double)angle);
    ((float2 *)out)[i] = cs;
}

template <int KVT>
__device__ __forceinline__ void store_pool4(void *pool, size_t at, float4 x, float scale) {
    if constexpr (KVT == LIA_FP8_E4M3) {
        const uint32_t w = (uint32_t)f32_to_e4m3(x.x / scale) | ((uint32_t)f32_to_e4m3(x.y / scale) << 8) |
                           ((uint32_t)f32_to_e4m3(x.z / scale) << 16) | ((uint32_t)f32_to_e4m3(x.w / scale) << 24);
        *(uint32_t *)((uint8_t *)pool + at) = w;
    } else {
        auto cv = [](float f) -> uint32_t { return KVT == LIA_BF16 ? f32_to_bf16(f) : f32_to_f16(f); };
        *(u32x2 *)((uint16_t *)pool + at) = u32x2{cv(x.x) | (cv(x.y) << 16), cv(x.z) | (cv(x.w) << 16)};
    }
}

// Fused RoPE + KV append: generalises rotary_cache (src/gpu/kernels/llama_position.rs:49-118)
// to any head counts, head_dim 64 / 128, the three pool types and slot-mapping or table
// addressing.  Input rows [rows][(hq + 2 hkv) * d] = q heads | k heads | v heads.  For
// d' < d/2 with {c, s} = coefficients[row][d']: x'[d'] = fma(x[d'], c, -(x[d'+d/2] * s)),
// x'[d'+d/2] = fma(x[d'+d/2], c, x[d'] * s), the products rounded (contraction off).  One
// thread per (row, head, 4 consecutive d' < d/2).
template <int KVT>
__global__ __launch_bounds__(256) void rope_append_kernel(
    uint32_t rows, uint32_t hq, uint32_t hkv, uint32_t d, const uint32_t *positions,
    const uint32_t *sequences, const uint32_t *pages, uint32_t stride, uint32_t page_shift,
    uint32_t pool_pages, const uint32_t *slot_mapping, const float *coefficients, const float *input, void *query,
    int query_bf16, void *kc, void *vc, float *k_scales, float *v_scales) {
#pragma clang fp contract(off)
    const uint32_t half = d / 2, quads = half / 4, heads = hq + hkv;
    const uint32_t i = blockIdx.x * 256 + threadIdx.x; // the host bounds the grid to 32 bits
    if (i >= rows * heads * quads) return;
    const uint32_t r = i / (heads * quads);
    const uint32_t h = i / quads % heads, d0 = 4 * (i % quads);
    const float4 *cs = (const float4 *)(coefficients + ((size_t)r * half + d0) * 2);
    const float4 c01 = cs[0], c23 = cs[1]; // {c0, s0, c1, s1}, {c2, s2, c3, s3}
    const float c[4] = {c01.x, c01.z, c23.x, c23.z}, sn[4] = {c01.y, c01.w, c23.y, c23.w};
    const size_t width = (size_t)(hq + 2 * hkv) * d;
    const float *x = input + r * width + (size_t)h * d;
    const float4 l4 = *(const float4 *)(x + d0), r4 = *(const float4 *)(x + half + d0);
    const float l[4] = {l4.x, l4.y, l4.z, l4.w}, rr[4] = {r4.x, r4.y, r4.z, r4.w};
    float a[4], b[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const float rs = rr[k] * sn[k], ls = l[k] * sn[k];
        a[k] = __builtin_fmaf(l[k], c[k], -rs);
        b[k] = __builtin_fmaf(rr[k], c[k], ls);
    }
    const float4 av = make_float4(a[0], a[1], a[2], a[3]), bv = make_float4(b[0], b[1], b[2], b[3]);
    if (h < hq) {
        const size_t at = ((size_t)r * hq + h) * d + d0;
        if (query_bf16) {
            store_pool4<LIA_BF16>(query, at, av, 1.0f);
            store_pool4<LIA_BF16>(query, at + half, bv, 1.0f);
        } else {
            *(float4 *)((float *)query + at) = av;
            *(float4 *)((float *)query + at + half) = bv;
        }
        return;
    }
    const uint32_t kh = h - hq;
    const uint32_t slot = row_slot(r, slot_mapping, positions, sequences, pages, stride, page_shift, pool_pages);
    if (slot == kNone) return;
    float ks = 1.0f, vs = 1.0f;
    if constexpr (KVT == LIA_FP8_E4M3) {
        const size_t ps = (size_t)(slot >> page_shift) * hkv + kh;
        ks = append_scale(k_scales, ps);
        vs = append_scale(v_scales, ps);
    }
    const size_t at = ((size_t)slot * hkv + kh) * d + d0;
    const float *v = input + r * width + (size_t)(hq + hkv + kh) * d;
    store_pool4<KVT>(kc, at, av, ks);
    store_pool4<KVT>(kc, at + half, bv, ks);
    store_pool4<KVT>(vc, at, *(const float4 *)(v + d0), vs);
    store_pool4<KVT>(vc, at + half, *(const float4 *)(v + half + d0), vs);
}

// Output-row gather: dst row i = src row indices[i], rows of `width` 32-bit words.
// Generalises llama_gather_hidden (src/gpu/kernels/llama.rs:186-198, width 2048 f32).
// One thread per 16 bytes when rows are a multiple of 4 words and 16-byte aligned.
template <bool VEC>
__global__ __launch_bounds__(256) void gather_kernel(uint32_t count, uint32_t width,
                                                     const uint32_t *indices, const void *src,
                                                     void *dst) {
    const uint32_t per = VEC ? width / 4 : width;
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    if (i >= count * per) return;
    const uint32_t row = i / per, e = i % per;
    const size_t from = (size_t)indices[row] * per + e;
    if constexpr (VEC) ((u32x4 *)dst)[i] = ((const u32x4 *)src)[from];
    else ((uint32_t *)dst)[i] = ((const uint32_t *)src)[from];
}

} // namespace lia

using namespace lia;

extern "C" int lia_gather_rows(uint32_t count, uint32_t width, const uint32_t *indices,
                               const void *src, void *dst, lia_stream_t stream) {
    if (!indices || !src || !dst || width == 0) return LIA_E_ARG;
    if (count == 0) return LIA_OK;
    if ((uint64_t)count * width >= (1ull << 32) - 256) return LIA_E_ARG;
    const bool vec = width % 4 == 0 && (((uintptr_t)src | (uintptr_t)dst) & 15) == 0;
    const uint32_t n = count * (vec ? width / 4 : width);
    hipStream_t s = (hipStream_t)stream;
    const dim3 grid((n + 255) / 256);
    const hipError_t e = vec ? launch<gather_kernel<true>>(grid, dim3(256), 0, s, count, width, indices, src, dst)
                             : launch<gather_kernel<false>>(grid, dim3(256), 0, s, count, width, indices, src, dst);
    return e == hipSuccess ? LIA_OK : LIA_E_HIP;
}

extern "C" int lia_rope_coefficients(uint32_t rows, uint32_t head_dim, float base,
                                     const uint32_t *positions, float *coefficients,
                                     lia_stream_t stream) {
    if (!positions || !coefficients) return LIA_E_ARG;
    if (head_dim != 64 && head_dim != 128) return LIA_E_UNSUPPORTED;
    if (((uintptr_t)coefficients & 7) != 0) return LIA_E_ALIGN;
    if (rows == 0) return LIA_OK;
    const uint32_t n = rows * (head_dim / 2);
    const hipError_t e = launch<rope_coefficients_kernel>(dim3((n + 255) / 256), dim3(256), 0,
                                                          (hipStream_t)stream, rows, head_dim, base,
                                                          positions, coefficients);
    return e == hipSuccess ? LIA_OK : LIA_E_HIP;
}

extern "C" int lia_rope_kv_append(const lia_kv_layout *L, uint32_t num_q_heads, uint32_t rows,
                                  const uint32_t *positions, const uint32_t *sequences,
                                  const uint32_t *pages, uint32_t stride,
                                  const uint32_t *slot_mapping, const float *coefficients,
                                  const float *input, void *query, int32_t query_dtype, void *kc,
                                  void *vc, float *k_scales, float *v_scales,
                                  lia_stream_t stream) {
    if (!L || !coefficients || !input || !query || !kc || !vc) return LIA_E_ARG;
    if (L->head_dim != 64 && L->head_dim != 128) return LIA_E_UNSUPPORTED;
    if (query_dtype != LIA_F32 && query_dtype != LIA_BF16) return LIA_E_UNSUPPORTED;
    if (L->num_kv_heads == 0 || num_q_heads == 0) return LIA_E_ARG;
    if (L->page_size == 0 || (L->page_size & (L->page_size - 1))) return LIA_E_ARG;
    if (!slot_mapping && (!positions || !sequences || !pages || stride == 0)) return LIA_E_ARG;
    if (L->dtype == LIA_FP8_E4M3 && (!k_scales || !v_scales)) return LIA_E_ARG;
    if (((uintptr_t)coefficients | (uintptr_t)input | (uintptr_t)query) & 15) return LIA_E_ALIGN;
    if (rows == 0) return LIA_OK;
    const size_t n = (size_t)rows * (num_q_heads + L->num_kv_heads) * (L->head_dim / 8);
    if (n >= (1ull << 32) - 256) return LIA_E_ARG;
    const dim3 grid((uint32_t)((n + 255) / 256));
    const uint32_t shift = (uint32_t)__builtin_ctz(L->page_size);
    hipStream_t s = (hipStream_t)stream;
    const int qb = query_dtype == LIA_BF16;
    hipError_t e;
#define LIA_ROPE(KVT)                                                                              \
    e = launch<rope_append_kernel<KVT>>(grid, dim3(256), 0, s, rows, num_q_heads, L->num_kv_heads, \
                                        L->head_dim, positions, sequences, pages, stride, shift,   \
                                        L->pool_pages, slot_mapping, coefficients, input, query,   \
                                        qb, kc, vc, k_scales, v_scales)
    switch (L->dtype) {
    case LIA_F16: LIA_ROPE(LIA_F16); break;
    case LIA_BF16: LIA_ROPE(LIA_BF16); break;
    case LIA_FP8_E4M3: LIA_ROPE(LIA_FP8_E4M3); break;
    default: return LIA_E_UNSUPPORTED;
    }
#undef LIA_ROPE
    return e == hipSuccess ? LIA_OK : LIA_E_HIP;
}

static int src_kind_of(int32_t dtype) {
    return dtype == LIA_F32 ? 0 : dtype == LIA_F16 ? 1 : dtype == LIA_BF16 ? 2 : -1;
}

extern "C" int lia_pack_device(uint32_t n_seqs, const uint32_t *seq_slots, const uint32_t *q_lens,
                               const uint32_t *cached, const uint32_t *pages, uint32_t stride,
                               uint32_t page_size, uint32_t pool_pages, uint32_t context,
                               uint32_t max_rows, uint32_t *cu_seqlens, uint32_t *positions,
                               uint32_t *sequences, uint32_t *slot_mapping, uint32_t *status,
                               lia_stream_t stream) {
    if (n_seqs == 0 || !seq_slots || !q_lens || !cached || !pages || !cu_seqlens || !positions ||
        !sequences || !slot_mapping || !status || stride == 0)
        return LIA_E_ARG;
    if (page_size == 0 || (page_size & (page_size - 1))) return LIA_E_ARG;
    hipStream_t s = (hipStream_t)stream;
    const uint32_t shift = (uint32_t)__builtin_ctz(page_size);
    if (launch<pack_kernel>(dim3(1), dim3(1024), 0, s, n_seqs, seq_slots, q_lens, cached, pages,
                            stride, shift, pool_pages, context, max_rows, cu_seqlens, positions,
                            sequences, slot_mapping, status) != hipSuccess)
        return LIA_E_HIP;
    const hipError_t e = launch<table_check_kernel>(dim3(kCheckGroups), dim3(kCheckThreads), 0, s,
                                                    n_seqs, seq_slots, q_lens, cached, pages, stride,
                                                    shift, pool_pages, context, max_rows, cu_seqlens,
                                                    slot_mapping, status);
    return e == hipSuccess ? LIA_OK : LIA_E_HIP;
}

extern "C" int lia_kv_append(const lia_kv_layout *L, uint32_t rows, const uint32_t *positions,
                             const uint32_t *sequences, const uint32_t *pages, uint32_t stride,
                             const uint32_t *slot_mapping, int32_t src_dtype, const void *k,
                             const void *v, void *kc, void *vc, float *k_scales,
                             float *v_scales, lia_stream_t stream) {
    if (!L || !k || !v || !kc || !vc) return LIA_E_ARG;
    if (rows == 0) return LIA_OK;
    if (!slot_mapping && (!positions || !sequences || !pages || stride == 0)) return LIA_E_ARG;
    if (L->page_size == 0 || (L->page_size & (L->page_size - 1))) return LIA_E_ARG;
    if (L->num_kv_heads == 0 || L->head_dim == 0 || L->head_dim % 4) return LIA_E_ARG;
    int kind = src_kind_of(src_dtype);
    if (kind < 0) return LIA_E_UNSUPPORTED;
    if (L->dtype == LIA_FP8_E4M3 && (!k_scales || !v_scales)) return LIA_E_ARG;
    uint32_t width = L->num_kv_heads * L->head_dim;
    size_t threads = (size_t)rows * (width / 4);
    dim3 grid((uint32_t)((threads + 255) / 256));
    uint32_t shift = (uint32_t)__builtin_ctz(L->page_size);
    hipStream_t s = (hipStream_t)stream;
    hipError_t e;
#define LIA_APPEND(KVT)                                                                            \
    e = launch<append_kernel<KVT>>(grid, dim3(256), 0, s, rows, width, L->head_dim,                \
                                   L->num_kv_heads, positions, sequences, pages, stride, shift,    \
                                   L->pool_pages, slot_mapping, kind, k, v, kc, vc, k_scales,      \
                                   v_scales)
    switch (L->dtype) {
    case LIA_F16: LIA_APPEND(LIA_F16); break;
    case LIA_BF16: LIA_APPEND(LIA_BF16); break;
    case LIA_FP8_E4M3: LIA_APPEND(LIA_FP8_E4M3); break;
    default: return LIA_E_UNSUPPORTED;
    }
#undef LIA_APPEND
    return e == hipSuccess ? LIA_OK : LIA_E_HIP;
}

extern "C" int lia_kv_quantize_pages(const lia_kv_layout *L, uint32_t n_pages,
                                     const uint32_t *page_ids, int32_t src_dtype, const void *k,
                                     const void *v, void *kc, void *vc, float *k_scales,
                                     float *v_scales, lia_stream_t stream) {
    if (!L || !page_ids || !k || !v || !kc || !vc || !k_scales || !v_scales) return LIA_E_ARG;
    if (L->dtype != LIA_FP8_E4M3) return LIA_E_UNSUPPORTED;
    if (n_pages == 0) return LIA_OK;
    int kind = src_kind_of(src_dtype);
    if (kind < 0) return LIA_E_UNSUPPORTED;
    const hipError_t e = launch<quantize_kernel>(dim3(n_pages, L->num_kv_heads, 2), dim3(256), 0,
                                                 (hipStream_t)stream, L->page_size, L->num_kv_heads,
                                                 L->head_dim, page_ids, kind, k, v, kc, vc, k_scales,
                                                 v_scales);
    return e == hipSuccess ? LIA_OK : LIA_E_HIP;
}

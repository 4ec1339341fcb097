// Per-step device packing shared by kv.hip (lia_pack_device) and attention.hip
// (lia_pack_plan_device, which packs and plans in one launch): the pack workgroup and the
// table-check workgroups as device functions of a workgroup.
#pragma once

#include "common.hpp"

namespace lia {

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

// One 1024-thread workgroup packs the batch.  `verdict` (may be null): a copy of the status this
// workgroup writes, for callers that read it from elsewhere (the attention workspace header).
__device__ void pack_rows_block(uint32_t n_seqs, const uint32_t *seq_slots, const uint32_t *q_lens,
                                const uint32_t *cached, const uint32_t *pages, uint32_t stride,
                                uint32_t page_shift, uint32_t pool_pages, uint32_t context,
                                uint32_t max_rows, uint32_t *cu, uint32_t *positions,
                                uint32_t *sequences, uint32_t *slot_mapping, uint32_t *status,
                                uint32_t *verdict) {
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
        if (t == 0) {
            *status = code;
            if (verdict) *verdict = code;
        }
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
        if (verdict) *verdict = 0;
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

// The table checks of workgroup grp of ngrp (T threads each): failure bits found in its share
// of the entries (bit 0: a page outside the pool, bit 1: a missing cached page), uniform over
// the workgroup.
template <uint32_t T>
__device__ uint32_t table_check_scan(uint32_t grp, uint32_t ngrp, uint32_t n_seqs,
                                     const uint32_t *seq_slots, const uint32_t *q_lens,
                                     const uint32_t *cached, const uint32_t *pages, uint32_t stride,
                                     uint32_t page_shift, uint32_t pool_pages, uint32_t context) {
    __shared__ uint32_t iscan[T], s_slot[T], s_c0[T], s_npg[T], w_a[16], w_b[16];
    __shared__ uint32_t found;
    const uint32_t t = threadIdx.x, P = 1u << page_shift;
    if (t == 0) found = 0;
    const bool quads = (stride & 3) == 0 && ((uintptr_t)pages & 15) == 0;
    const uint32_t per = quads ? 4u : 1u;
    constexpr int K = 4; // items in flight per thread
    for (uint32_t base = 0; base < n_seqs; base += T) {
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
        const uint32_t cnt = min(n_seqs - base, T), total = iscan[cnt - 1];
        const uint32_t step = ngrp * T;
        for (uint32_t e0 = grp * T + t; e0 < total; e0 += K * step) {
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
    return found;
}

// Status of the table-check failure bits: a page outside the pool outranks a missing page.
__device__ __forceinline__ uint32_t table_failure(uint32_t bits) {
    return (bits & 1) ? (uint32_t)(-LIA_E_PAGE_RANGE) : (bits & 2) ? (uint32_t)(-LIA_E_MISSING_PAGE) : 0u;
}

// table_check_kernel's workgroup: the checks, and on a failure the batch rejected as the
// packing rejects one and the status raised to it unless it holds a failure the reference
// checks earlier.
__device__ void table_check_block(uint32_t grp, uint32_t ngrp, uint32_t n_seqs,
                                  const uint32_t *seq_slots, const uint32_t *q_lens,
                                  const uint32_t *cached, const uint32_t *pages, uint32_t stride,
                                  uint32_t page_shift, uint32_t pool_pages, uint32_t context,
                                  uint32_t max_rows, uint32_t *cu, uint32_t *slot_mapping,
                                  uint32_t *status) {
    const uint32_t found = table_check_scan<kCheckThreads>(grp, ngrp, n_seqs, seq_slots, q_lens, cached,
                                                           pages, stride, page_shift, pool_pages, context);
    if (!found) return;
    const uint32_t t = threadIdx.x;
    for (uint32_t b = t; b <= n_seqs; b += kCheckThreads) cu[b] = 0;
    for (uint32_t r = t; r < max_rows; r += kCheckThreads) slot_mapping[r] = kNone;
    if (t == 0) {
        const uint32_t want = table_failure(found);
        uint32_t old = __hip_atomic_load(status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        while (old != (uint32_t)(-LIA_E_ROWS) && old != (uint32_t)(-LIA_E_PAGE_RANGE) && old != want) {
            const uint32_t prev = atomicCAS(status, old, want);
            if (prev == old) break;
            old = prev;
        }
    }
}

} // namespace lia

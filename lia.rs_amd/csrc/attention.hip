// Paged causal GQA attention over a ragged packed batch for gfx950 (CDNA4).
//
// Work decomposition ("units"): for batch sequence b, its query rows are cut into column
// blocks of `rpc` rows; each (sequence, column block, KV head) is one unit whose MFMA
// columns are the rpc*group (row, query head) pairs that share that KV head.  A unit
// attends keys 0 .. positions[last row of the block], tiled in 32-token blocks.
//
// Scheduling is balanced over workgroups rather than over units: the key blocks of all
// units are laid end to end and workgroup w of N takes blocks [w*B/N, (w+1)*B/N).  In the
// decode kernel the waves of a workgroup split head_dim and walk the same 32-token chunks,
// summing their partial scores through LDS; in the prefill kernel (wide_kernel) each wave
// owns 16 of a unit's 128 columns and all waves share each chunk's K/V staged in LDS.  A
// unit covered by one workgroup is written normalised straight to `out`; a unit split
// across workgroups leaves one partial record per workgroup (O, reference max, mass) and
// the combine kernels merge them - the reference's split-K partial + merge
// (src/gpu/kernels/llama_flash_kernel.rs:321-376, src/gpu/kernels/llama_merge.rs:10-76)
// with splits chosen for load balance instead of a batch-uniform span.
//
// Keys of a unit come from two sources: the keys cached before this step, [0, kcache), are
// read through the block table from the pool, and the keys of this step's own rows,
// [kcache, kend), are blocked separately.  The plain entry points read both from the pool
// (the rows were appended first); the fused-append entry point reads the new keys straight
// from the caller's new K/V rows and scatters those rows into the pool in the same launch,
// so no work of the launch ever reads a slot the launch writes.
//
// Per 32-token chunk a wave computes S^T = K * Q^T with K straight from HBM (bounded
// buffer loads) as the MFMA A operand (16 tokens x 32 dims per instruction) and Q^T
// resident in registers, runs the online softmax in the log2 domain per column, stages V
// through LDS in its natural token-major layout and reads it back transposed
// (ds_read_b64_tr_b16) as the A operand of O^T += V^T * P^T.  Causal masking is per
// column: row r sees keys <= positions[r] (src/gpu/kernels/llama_flash_kernel.rs:145-175).
#include <mutex>

#include "common.hpp"
#include "launch.hpp"
#include "pack.hpp"

namespace lia {


// Unit descriptor written by the plan kernel (32 bytes).  Rows of a sequence have
// consecutive positions (validated by packing), so positions[rowbeg] = kend - nrows and
// the sequence's first packed row is rowbeg - (positions[rowbeg] - kcache).
struct UnitDesc {
    uint32_t block_start; // first block in the flattened block order
    uint32_t nblocks;     // cblocks + ceil((kend - kcache) / 32)
    uint32_t cblocks;     // ceil(kcache / 32): blocks of the keys cached before this step
    uint32_t rowbeg;      // first packed row of the column block
    uint32_t nrows_hk;    // rows in the column block | KV head << 16
    uint32_t kend;        // keys attended by the last row (positions[last] + 1)
    uint32_t table_row;   // block-table row of the sequence
    uint32_t kcache;      // position of the sequence's first packed row
};

__device__ __forceinline__ uint32_t unit_rows(const UnitDesc &u) { return u.nrows_hk & 0xffffu; }
__device__ __forceinline__ uint32_t unit_head(const UnitDesc &u) { return u.nrows_hk >> 16; }

// Per-workgroup work descriptor (64 bytes): the block range, a copy of the descriptor of
// the range's first unit and the physical pages of the first four logical pages the range
// reads, so a workgroup issues its first K/V loads one dependent load after launch.
constexpr uint32_t kPrePages = 4;
struct WorkDesc {
    uint32_t unit;            // first unit of the range
    uint32_t lo, hi;          // block range [lo, hi)
    uint32_t flags;           // bit 0: pre[] valid; bits 8-31: range index (record base)
    UnitDesc first;           // units[unit]
    uint4 pre;                // pages of logical pages (32 * (lo - first.block_start)) / P + 0..3
};

// Per-unit merge descriptor (16 bytes): the records the combine reads, n = 0 when one
// workgroup wrote the unit directly (or the unit does not exist in this plan).
struct MergeDesc {
    uint32_t rec0, n;     // records rec0 .. rec0 + n - 1
    uint32_t rowbeg;      // as in UnitDesc
    uint32_t nrows_hk;
};

// Word of the workspace header holding the step's verdict: 0, or the failure (a positive
// lia_status) of the packing that lia_pack_plan_device ran beside the plan, whose table checks
// then empty the plan (every work range and merge descriptor), so the attention and combine
// kernels do nothing for a rejected step.
constexpr uint32_t kVerdict = 4;

struct AttnParams {
    const void *q;
    const void *kc;
    const void *vc;
    const float *k_scales;
    const float *v_scales;
    const uint32_t *cu;
    const uint32_t *positions;
    const uint32_t *sequences;
    const uint32_t *pages;
    void *out;
    const UnitDesc *units;   // [U + 1]; units[U].block_start = B
    const WorkDesc *work;    // per launched workgroup (empty ranges past the planned count)
    const MergeDesc *merge;  // per unit slot of the workspace
    const uint32_t *header;  // {U, B, N (workgroups with work), overflow}
    float *part_o;           // [records][cols][D]
    float *part_ml;          // [records][cols][2]
    uint32_t hq, hkv, group, stride, page_shift, n_wg, rpc, pool_pages;
    float scale_log2;        // softmax scale * log2(e)
    int q_f32, out_f32;
    // fused append (null when the new rows are already in the pool)
    const void *newk;        // [n_rows][hkv][D] in the pool dtype
    const void *newv;
    const uint32_t *slots;   // slot_mapping[n_rows]
    void *kc_w, *vc_w;       // the pool planes, written by the append
    uint32_t n_rows;
    uint32_t round_wg;       // workgroups per dispatch round (one per CU)
};

// ------------------------------------------------------------------ plan

// One workgroup builds the unit list of a step and the block range of every attention
// workgroup.  Positions within a sequence are consecutive (validated by packing,
// src/inference/paging.rs:167-172), so the key count of a column block follows from the
// position of its first row.  A unit's keys are blocked in two runs: the keys cached before
// the step, [0, kcache) with kcache the position of the sequence's first row, then the
// keys of the step's own rows, [kcache, kend).
__device__ __forceinline__ uint32_t unit_blocks(uint32_t p0, uint32_t new_keys) {
    return (p0 + 31) / 32 + (new_keys + 31) / 32;
}

// sum_{i=0}^{n-1} floor((a*i + b) / m) (the standard floor-sum reduction, O(log) steps),
// for the plan's small operands: 32-bit divisions, 64-bit sum.
__device__ __forceinline__ uint64_t floor_sum(uint32_t n, uint32_t m, uint32_t a, uint32_t b) {
    uint64_t ans = 0;
    while (true) {
        if (a >= m) {
            ans += (uint64_t)n * (n - 1) / 2 * (a / m);
            a %= m;
        }
        if (b >= m) {
            ans += (uint64_t)n * (b / m);
            b %= m;
        }
        const uint32_t y = a * n + b;
        if (y < m) break;
        n = y / m;
        b = y % m;
        const uint32_t tmp = m;
        m = a;
        a = tmp;
    }
    return ans;
}

// New-key blocks of column blocks 0 .. m-1 of a sequence in one KV head: sum over c = 1..m
// of ceil(c * rpc / 32) (column block c-1 ends at row c * rpc, before the last block).
// Power-of-two rpc (every batch shape the launches choose) in closed form with k = 32/rpc:
// k*q*(q+1)/2 + r*(q+1), q = m / k, r = m % k.
__device__ __forceinline__ uint32_t new_blocks_before(uint32_t m, uint32_t rpc) {
    if (!m) return 0;
    if ((rpc & (rpc - 1)) == 0) {
        if (rpc >= 32) return (rpc >> 5) * (m * (m + 1) / 2);
        const uint32_t lk = 5 - (31 - __builtin_clz(rpc)), k = 1u << lk; // k = 32 / rpc
        const uint32_t q = m >> lk, r = m & (k - 1);
        return k * q * (q + 1) / 2 + r * (q + 1);
    }
    return (uint32_t)floor_sum(m, 32, rpc, rpc + 31);
}

constexpr uint32_t kPlanSeqs = 1024; // sequences the plan keeps in LDS (one per thread)
constexpr uint32_t kPlanThreads = 1024;
// Workgroups of plan_lds_kernel: each computes the per-sequence extents and then writes an
// interleaved share of the descriptors (one workgroup issued them all at 16 waves on one CU).
constexpr uint32_t kPlanGroups = 8;
// Cost of starting a unit, in 32-key blocks, that the balanced partition charges each unit: a
// range crossing into a unit loads its queries, unit descriptor and page window before its first
// keys.  Measured best: 8 for the prefill kernel (config 3 step 303 -> 246 us against no charge;
// re-swept with XCD-major ranges: 40-layer step 210.5-210.6 us per layer at 8, 212.8-212.9 at 12,
// 262.5-262.6 at 4),
// 4 for the decode kernel (config 2 8,320 -> 8,540 tokens/s; configs 4 and 5 lose beyond 4;
// re-swept with XCD-major ranges: 2 is 1 % slower on config 2 and 2 % on config 4, 6 and 8
// within 0.5 % of 4 on every decode configuration).
constexpr uint32_t kUnitCostWide = 8, kUnitCostDecode = 4;
// Weight lag (of 256) of the workgroups that share a CU with an older one.  Measured per
// workgroup on the prefill kernel (two per CU): with equal shares the CU's first workgroup
// finished in 183 us and the second in 216 us, the older waves being issued first.  Lag 56
// (22 %) gave the best step (lags 24-96 measured).  The decode kernel loses with any lag (16-64
// measured 1.5-2.5 % slower on config 2): its first-round workgroups do finish earlier, but more
// blocks for them leave the other rounds' end unchanged, since the chip's aggregate rate while
// every workgroup runs is the cap.
// Re-measured with XCD-major ranges (every decode launch at lag 40, or FP8 and two-tile launches
// only): 40-layer steps per layer config 5 156.1-156.5 us against 158.3-158.4 and config 4
// 55.64-55.72 against 55.97-56.04, but the weighted plan's searches lengthen every step by about
// 3 us (config 4 one-layer step 67.8 against 64.4-64.8) and config 2 loses 1 % at any lag: 0 kept.
constexpr uint32_t kLagWide = 56, kLagDecode = 0;

// The plan for up to kPlanSeqs sequences, one thread each (kPlanThreads): per-sequence extents
// in LDS (a shuffle scan with one barrier) and every unit in closed form (unit (h, cb) of
// sequence b starts at block b0 + h*nbh + cb*cblocks + new_blocks_before(cb)), so units, merge
// descriptors and the work list are each written in parallel with no serial per-sequence loop
// and no reads of the units just written.  Workgroups get shares of cost - the blocks plus
// unit_cost per unit (its start) - equal, or weighted by dispatch round (round_wg, lag).
//
// Per-sequence extents come from the packed metadata (cu_seqlens, positions, sequences), or,
// with `raw` set, from the packing's own inputs (raw->q_lens, cached, seq_slots), so the plan
// can run beside the packing in one launch; a raw batch whose rows differ from raw->n_rows is
// planned empty.  The workgroup is `grp` of `ngrp` sharing the descriptor loops.
struct RawSeqs {
    const uint32_t *q_lens, *cached, *seq_slots;
    uint32_t n_rows;
};

__device__ void plan_lds(uint32_t n_seqs, const uint32_t *cu, const uint32_t *positions,
                         const uint32_t *sequences, const RawSeqs *raw, const uint32_t *pages,
                         uint32_t stride, uint32_t page_shift, uint32_t rpc, uint32_t hkv,
                         uint32_t max_units, uint32_t n_wg, uint32_t unit_cost, uint32_t round_wg,
                         uint32_t lag, uint32_t xcd, uint32_t grp, uint32_t ngrp, UnitDesc *units,
                         WorkDesc *work, MergeDesc *merge, uint32_t *header) {
    __shared__ uint32_t s_r0[kPlanSeqs], s_nr[kPlanSeqs], s_p0[kPlanSeqs], s_trow[kPlanSeqs];
    __shared__ uint32_t s_u0[kPlanSeqs + 1], s_b0[kPlanSeqs + 1], s_c0[kPlanSeqs + 1];
    __shared__ uint32_t w_s[4][kPlanThreads / 64];
    __shared__ uint32_t carry_units, carry_blocks, carry_rows, raw_bad;
    __shared__ uint64_t s_rlo[kPlanThreads + 1];
    // Threads exchange only LDS data (nothing written to global memory is read back), so the
    // barriers need not wait for the descriptor stores in flight.
    constexpr uint32_t T = kPlanThreads;
    const uint32_t t = threadIdx.x;
    // the workgroups of the launch share the descriptor loops; each computes the per-sequence
    // extents and range starts itself (they live in its LDS)
    const uint32_t g0 = t * ngrp + grp, GT = ngrp * T; // interleaved shares
    // up to 64 sequences: the scans stay in wave 0, with no barrier of their own
    const bool one_wave = n_seqs <= 64;
    const uint32_t last = one_wave ? 63 : T - 1; // the thread holding the totals
    {
        const uint32_t b = t;
        uint32_t nu = 0, nb = 0, r0 = 0, nr = 0, p0 = 0, trow = 0;
        if (b < n_seqs) {
            if (raw) {
                // the packing's inputs; the rows before this sequence are a scan of the
                // new-token counts, below
                nr = raw->q_lens[b];
                p0 = raw->cached[b];
                trow = raw->seq_slots[b];
            } else {
                r0 = cu[b];
                nr = cu[b + 1] - r0;
                if (nr > 0) {
                    p0 = positions[r0];
                    trow = sequences[r0];
                }
            }
            if (nr > 0) {
                const uint32_t ncb = (nr + rpc - 1) / rpc;
                nu = ncb * hkv;
                nb = (ncb * ((p0 + 31) / 32) + new_blocks_before(ncb - 1, rpc) + (nr + 31) / 32) * hkv;
            }
        }
        // inclusive scans of the units and blocks, and on raw inputs of the rows and of the
        // sequences whose keys pass their table row.  The packing beside a raw plan has not
        // validated its inputs: such a sequence makes the plan empty, so no table read leaves
        // the row.
        uint32_t v[4] = {nu, nb, nr,
                         raw && (uint64_t)p0 + nr > ((uint64_t)stride << page_shift) ? 1u : 0u};
        if (raw) block_scan_n<4>(v, w_s, one_wave);
        else block_scan_n<2>(v, w_s, one_wave);
        if (raw) r0 = v[2] - nr;
        if (b < n_seqs) {
            s_r0[b] = r0; s_nr[b] = nr; s_p0[b] = p0; s_trow[b] = trow;
            s_u0[b] = v[0] - nu;
            s_b0[b] = v[1] - nb;
            s_c0[b] = v[1] - nb + unit_cost * (v[0] - nu);
        }
        if (t == last) {
            carry_units = v[0]; carry_blocks = v[1];
            if (raw) { carry_rows = v[2]; raw_bad = v[3]; }
        }
        lds_barrier();
    }
    const bool overflow = carry_units > max_units || (raw && (carry_rows != raw->n_rows || raw_bad));
    const uint32_t U = overflow ? 0 : carry_units, B = overflow ? 0 : carry_blocks;
    const uint32_t N = min(n_wg, B);
    if (t == 0) {
        s_u0[n_seqs] = carry_units;
        s_b0[n_seqs] = carry_blocks;
        s_c0[n_seqs] = carry_blocks + unit_cost * carry_units;
        if (grp == 0) {
            units[U] = UnitDesc{B, 0, 0, 0, 0, 0, 0, 0};
            header[0] = U;
            header[1] = B;
            header[2] = N;
            header[3] = overflow;
            // the batch verdict: a plan of packed metadata is never of a rejected batch (its
            // rejection empties cu_seqlens); the packing beside a raw plan writes it instead
            if (!raw) header[kVerdict] = 0;
        }
    }
    lds_barrier();
    // last sequence b with arr[b] <= v (empty sequences share their offset with the next
    // one, so this is the sequence that owns v)
    auto seq_of = [&](const uint32_t *arr, uint32_t v) {
        uint32_t a = 0, e = n_seqs;
        while (a + 1 < e) {
            const uint32_t mid = (a + e) >> 1;
            if (arr[mid] <= v) a = mid; else e = mid;
        }
        return a;
    };
    auto make_unit = [&](uint32_t b, uint32_t h, uint32_t cb) {
        const uint32_t nr = s_nr[b], p0 = s_p0[b], cblocks = (p0 + 31) / 32;
        const uint32_t nbh = (s_b0[b + 1] - s_b0[b]) / hkv;
        const uint32_t rows = min(rpc, nr - cb * rpc), kend = p0 + cb * rpc + rows;
        const uint32_t blk = s_b0[b] + h * nbh + cb * cblocks + new_blocks_before(cb, rpc);
        return UnitDesc{blk, unit_blocks(p0, kend - p0), cblocks, s_r0[b] + cb * rpc, rows | (h << 16),
                        kend, s_trow[b], p0};
    };
    auto unit_by_index = [&](uint32_t u) {
        const uint32_t b = seq_of(s_u0, u), ncb = (s_nr[b] + rpc - 1) / rpc, i = u - s_u0[b];
        return make_unit(b, i / ncb, i % ncb);
    };
    const uint32_t P = 1u << page_shift;
    for (uint32_t w = N + g0; w < n_wg; w += GT) { // launched workgroups without work
        WorkDesc d = {};
        work[w] = d;
    }
    // Work is split in cost: each unit's blocks are preceded by unit_cost virtual blocks (the
    // cost of starting a unit), so a range that crosses into a unit is shorter by that much and a
    // boundary falling in a unit's lead-in moves to the unit's start.
    const uint64_t TC = (uint64_t)B + (uint64_t)unit_cost * U;
    const bool xcd_major = xcd && N == n_wg && N % 8 == 0;
    const uint32_t per = N / 8;
    // Ranges in cost order r = 0 .. N-1 run on workgroup w(r): r itself, or XCD-major when xcd is
    // set and the grid allows (range r on workgroup (r % per) * 8 + r / per, so the workgroups of
    // one XCD - workgroup i runs on XCD i % 8 - take contiguous ranges).
    // A workgroup dispatched after the first round_wg shares its CU with an older one, which the
    // hardware issues first, so its range is weighted (256 - lag) / 256 against 1 for the first
    // round (lag 0: equal shares).  F(r) = sum of the weights of ranges before r, times 256.
    auto late_before = [&](uint32_t r) -> uint32_t { // ranges before r on workgroups w >= round_wg
        uint32_t late = 0;
        if (xcd_major) {
            const uint32_t X = r / per, I = r % per;
            for (uint32_t x = 0; x <= X && x < 8; x++) {
                const uint32_t cx = round_wg > x ? min(per, (round_wg - x + 7) / 8) : 0u;
                late += x < X ? per - cx : (I > cx ? I - cx : 0u);
            }
        } else {
            late = r > round_wg ? r - round_wg : 0u;
        }
        return late;
    };
    // Weights only when every range still spans at least one block of cost: a range weighted w
    // of 256 spans TC * w / F(N) >= TC * (256 - lag) / F(N), so with that at least 1 each start
    // lies at least one block after the previous one.  A range empty in blocks inside a unit
    // would be counted among the unit's records without writing one.
    const bool skew = lag && round_wg && round_wg < N &&
                      TC * (256 - lag) >= 256ull * N - (uint64_t)lag * late_before(N);
    auto weight_before = [&](uint32_t r) -> uint64_t {
        return 256ull * r - (skew ? (uint64_t)lag * late_before(r) : 0ull);
    };
    // Equal weights: range r starts at cost r*TC/N, and cost c lies in range ((c+1)*N-1)/TC.
    // Weighted: the start cost of every range is tabulated once (one division per range) and
    // searched.
    if (skew) {
        const uint64_t FN = weight_before(N);
        for (uint32_t r = t; r <= N; r += T) s_rlo[r] = weight_before(r) * TC / FN;
        lds_barrier();
    }
    // equal shares in 32-bit arithmetic when TC * N fits (every batch up to 2^32 / n_wg
    // blocks): a 64-bit division is a long software sequence on the plan's critical path
    const bool narrow = TC * N < (1ull << 32);
    auto range_lo = [&](uint32_t r) -> uint64_t {
        if (skew) return s_rlo[r];
        return narrow ? r * (uint32_t)TC / N : (uint64_t)r * TC / N;
    };
    // the last range starting at or before cost c
    auto range_of = [&](uint64_t c) {
        if (!skew) return narrow ? ((uint32_t)c * N + N - 1) / (uint32_t)TC : (uint32_t)(((c + 1) * N - 1) / TC);
        uint32_t a = 0, e = N;
        while (a + 1 < e) {
            const uint32_t mid = (a + e) >> 1;
            if (s_rlo[mid] <= c) a = mid; else e = mid;
        }
        return a;
    };
    // each unit's descriptor, and its merge descriptor from it
    for (uint32_t u = g0; u < max_units; u += GT) {
        MergeDesc m = {0, 0, 0, 0};
        if (u < U) {
            const UnitDesc ud = unit_by_index(u);
            units[u] = ud;
            const uint64_t cu0 = (uint64_t)ud.block_start + unit_cost * (u + 1); // cost of its first block
            const uint32_t wf = range_of(cu0), wl = range_of(cu0 + ud.nblocks - 1);
            if (wf != wl) m = MergeDesc{wf + u, wl - wf + 1, ud.rowbeg, ud.nrows_hk};
        }
        merge[u] = m;
    }
    // The block at cost c, and its unit (sequence ub, KV head uh, column block ucb): in cost,
    // sequence b starts at s_c0[b], a KV head's units span nbh + unit_cost * ncb, and a unit's
    // blocks follow its unit_cost lead-in; a cost inside a lead-in maps to the unit's first block.
    auto block_of_cost = [&](uint64_t c, uint32_t &ub, uint32_t &uh, uint32_t &ucb) {
        if (c >= TC) { ub = n_seqs; return B; }
        const uint32_t cc = (uint32_t)c;
        const uint32_t b = seq_of(s_c0, cc);
        const uint32_t ncb = (s_nr[b] + rpc - 1) / rpc, cblocks = (s_p0[b] + 31) / 32;
        const uint32_t nbh = (s_b0[b + 1] - s_b0[b]) / hkv;
        const uint32_t hsp = nbh + unit_cost * ncb, co = cc - s_c0[b];
        const uint32_t h = co / hsp, co2 = co - h * hsp;
        uint32_t cb = 0, e = ncb; // last cb whose cost start <= co2
        while (cb + 1 < e) {
            const uint32_t mid = (cb + e) >> 1;
            if (mid * cblocks + new_blocks_before(mid, rpc) + unit_cost * mid <= co2) cb = mid; else e = mid;
        }
        const uint32_t ustart = cb * cblocks + new_blocks_before(cb, rpc);
        const uint32_t off = co2 - (ustart + unit_cost * cb);
        ub = b; uh = h; ucb = cb;
        return s_b0[b] + h * nbh + ustart + (off < unit_cost ? 0u : off - unit_cost);
    };
    // One work descriptor per thread and pass (unconditional page-table loads: an entry not
    // needed reads a word the plan reads anyway - cu[0], or q_lens[0] of a raw plan, whose
    // cu is null - and is replaced by 0).
    const uint32_t *dummy = raw ? raw->q_lens : cu;
    // the work descriptors from the last threads, so that their chain (searches, divisions,
    // table loads) runs beside the units' on other waves
    for (uint32_t w0 = (T - 1 - t) * ngrp + grp; w0 < N; w0 += GT) {
        WorkDesc d[1];
        uint32_t v[1][kPrePages];
        {
            constexpr int k = 0;
            const uint32_t w = w0;
            const uint32_t r = xcd_major ? (w % 8) * per + w / 8 : w;
            uint32_t b, h, c, b2, h2, c2;
            const uint32_t lo = block_of_cost(range_lo(r), b, h, c);
            const uint32_t hi = block_of_cost(range_lo(r + 1), b2, h2, c2);
            if (b >= n_seqs) { b = 0; h = 0; c = 0; } // empty range at the end
            const uint32_t ncb = (s_nr[b] + rpc - 1) / rpc;
            d[k].unit = s_u0[b] + h * ncb + c;
            d[k].first = make_unit(b, h, c);
            d[k].flags = r << 8;
            d[k].lo = lo;
            d[k].hi = hi;
            // logical pages the range starts with, when it starts in the cached keys
            const uint32_t rel = lo - d[k].first.block_start;
            const bool pre = pages && rel < d[k].first.cblocks;
            const uint32_t lp = (32 * rel) >> page_shift;
            const uint32_t lend = (d[k].first.kend + P - 1) >> page_shift;
#pragma unroll
            for (uint32_t i = 0; i < kPrePages; i++) {
                const bool use = pre && lp + i < lend;
                const uint32_t *src = use ? pages + (size_t)d[k].first.table_row * stride + lp + i : dummy;
                v[k][i] = *src;
                v[k][i] = use ? v[k][i] : 0u;
            }
            if (pre) d[k].flags |= 1;
        }
        d[0].pre = make_uint4(v[0][0], v[0][1], v[0][2], v[0][3]);
        work[w0] = d[0];
    }
}

__global__ __launch_bounds__(kPlanThreads) void plan_lds_kernel(
    uint32_t n_seqs, const uint32_t *cu, const uint32_t *positions, const uint32_t *sequences,
    const uint32_t *pages, uint32_t stride, uint32_t page_shift, uint32_t rpc, uint32_t hkv,
    uint32_t max_units, uint32_t n_wg, uint32_t unit_cost, uint32_t round_wg, uint32_t lag,
    uint32_t xcd, UnitDesc *units, WorkDesc *work, MergeDesc *merge, uint32_t *header) {
    plan_lds(n_seqs, cu, positions, sequences, nullptr, pages, stride, page_shift, rpc, hkv, max_units,
             n_wg, unit_cost, round_wg, lag, xcd, blockIdx.x, gridDim.x, units, work, merge, header);
}

struct PackArgs {
    const uint32_t *seq_slots, *q_lens, *cached, *pages;
    uint32_t stride, page_shift, pool_pages, context, max_rows;
    uint32_t *cu, *positions, *sequences, *slot_mapping, *status;
};

// Workgroups of lia_pack_plan_device's first launch that check the block tables (1024 threads
// each, as many threads as table_check_kernel's 64 x 256); each writes its failure bits to
// header[kFoundWords + its index] on every call, so no word needs clearing first.
constexpr uint32_t kSetupChecks = 16, kFoundWords = 16;

// lia_pack_plan_device's first launch (1024-thread workgroups): 0 .. kPlanGroups-1 plan the step
// from the packing's inputs, kPlanGroups packs it (its status also to the header's verdict
// word), and the kSetupChecks after it check the block tables.
__global__ __launch_bounds__(kPlanThreads) void pack_plan_kernel(
    uint32_t n_seqs, PackArgs pk, RawSeqs raw, uint32_t rpc, uint32_t hkv, uint32_t max_units,
    uint32_t n_wg, uint32_t unit_cost, uint32_t round_wg, uint32_t lag, uint32_t xcd, UnitDesc *units,
    WorkDesc *work, MergeDesc *merge, uint32_t *header) {
    const uint32_t bid = blockIdx.x;
    if (bid < kPlanGroups) {
        plan_lds(n_seqs, nullptr, nullptr, nullptr, &raw, pk.pages, pk.stride, pk.page_shift, rpc, hkv,
                 max_units, n_wg, unit_cost, round_wg, lag, xcd, bid, kPlanGroups, units, work, merge,
                 header);
    } else if (bid == kPlanGroups) {
        pack_rows_block(n_seqs, pk.seq_slots, pk.q_lens, pk.cached, pk.pages, pk.stride, pk.page_shift,
                        pk.pool_pages, pk.context, pk.max_rows, pk.cu, pk.positions, pk.sequences,
                        pk.slot_mapping, pk.status, header + kVerdict);
    } else {
        const uint32_t grp = bid - kPlanGroups - 1;
        const uint32_t found = table_check_scan<kPlanThreads>(grp, kSetupChecks, n_seqs, pk.seq_slots,
                                                              pk.q_lens, pk.cached, pk.pages, pk.stride,
                                                              pk.page_shift, pk.pool_pages, pk.context);
        if (threadIdx.x == 0) header[kFoundWords + grp] = found;
    }
}

// lia_pack_plan_device's second launch (one workgroup): the step's status from the packing's
// (header[kVerdict]) and the table checks' bits, in the reference's order of checks (the row
// count, then the tables, then the rows: paging.rs:120-172), written to status and to the
// verdict word.  A table failure rejects the rows as the packing rejects its own; any failure
// empties the plan, so the attention and combine kernels do nothing for the step.
__global__ __launch_bounds__(kPlanThreads) void setup_verdict_kernel(
    uint32_t n_seqs, uint32_t max_rows, uint32_t *cu, uint32_t *slot_mapping, uint32_t *status,
    uint32_t *header, WorkDesc *work, uint32_t n_wg, MergeDesc *merge, uint32_t max_units) {
    const uint32_t t = threadIdx.x;
    const uint32_t packing = header[kVerdict];
    uint32_t bits = 0;
#pragma unroll
    for (uint32_t i = 0; i < kSetupChecks; i++) bits |= header[kFoundWords + i];
    const uint32_t verdict = packing == (uint32_t)(-LIA_E_ROWS) ? packing : bits ? table_failure(bits) : packing;
    if (verdict == 0) {
        if (t == 0) *status = 0;
        return;
    }
    if (verdict != packing) { // a table failure: the packing wrote the rows
        for (uint32_t b = t; b <= n_seqs; b += kPlanThreads) cu[b] = 0;
        for (uint32_t r = t; r < max_rows; r += kPlanThreads) slot_mapping[r] = kNone;
    }
    for (uint32_t w = t; w < n_wg; w += kPlanThreads) work[w] = WorkDesc{};
    for (uint32_t u = t; u < max_units; u += kPlanThreads) merge[u] = MergeDesc{0, 0, 0, 0};
    if (t == 0) {
        *status = verdict;
        header[kVerdict] = verdict;
    }
}

// The plan for more sequences than plan_lds_kernel holds: units written by a serial walk of
// each thread's sequences.
__global__ __launch_bounds__(256) void plan_kernel(uint32_t n_seqs, const uint32_t *cu,
                                                   const uint32_t *positions,
                                                   const uint32_t *sequences, const uint32_t *pages,
                                                   uint32_t stride, uint32_t page_shift, uint32_t rpc,
                                                   uint32_t hkv, uint32_t max_units,
                                                   uint32_t n_wg, uint32_t xcd, UnitDesc *units,
                                                   WorkDesc *work, MergeDesc *merge,
                                                   uint32_t *header) {
    __shared__ uint32_t s_units[256], s_blocks[256];
    __shared__ uint32_t carry_units, carry_blocks, overflow;
    const uint32_t t = threadIdx.x;
    if (t == 0) { carry_units = 0; carry_blocks = 0; overflow = 0; }
    __syncthreads();
    for (uint32_t base = 0; base < n_seqs; base += 256) {
        uint32_t b = base + t;
        uint32_t nu = 0, nb = 0, r0 = 0, nr = 0, p0 = 0, trow = 0;
        if (b < n_seqs) {
            r0 = cu[b];
            nr = cu[b + 1] - r0;
            if (nr > 0) {
                p0 = positions[r0];
                trow = sequences[r0];
                uint32_t ncb = (nr + rpc - 1) / rpc;
                nu = ncb * hkv;
                for (uint32_t cb = 0; cb < ncb; cb++) nb += unit_blocks(p0, min((cb + 1) * rpc, nr));
                nb *= hkv;
            }
        }
        s_units[t] = nu;
        s_blocks[t] = nb;
        __syncthreads();
        for (uint32_t off = 1; off < 256; off <<= 1) { // inclusive Hillis-Steele scan
            uint32_t a = t >= off ? s_units[t - off] : 0, c = t >= off ? s_blocks[t - off] : 0;
            __syncthreads();
            s_units[t] += a;
            s_blocks[t] += c;
            __syncthreads();
        }
        uint32_t u = carry_units + s_units[t] - nu;
        uint32_t blk = carry_blocks + s_blocks[t] - nb;
        if (nu && u + nu > max_units) overflow = 1;
        if (nu && u + nu <= max_units) {
            uint32_t ncb = nu / hkv;
            const uint32_t cblocks = (p0 + 31) / 32;
            // KV head outermost: consecutive units (and the block ranges over them) stream
            // the same keys
            for (uint32_t h = 0; h < hkv; h++) {
                for (uint32_t cb = 0; cb < ncb; cb++) {
                    uint32_t rows = min(rpc, nr - cb * rpc);
                    uint32_t kend = p0 + cb * rpc + rows;
                    uint32_t blocks = unit_blocks(p0, kend - p0);
                    units[u++] = UnitDesc{blk, blocks, cblocks, r0 + cb * rpc, rows | (h << 16),
                                          kend, trow, p0};
                    blk += blocks;
                }
            }
        }
        __syncthreads();
        if (t == 255) { carry_units += s_units[255]; carry_blocks += s_blocks[255]; }
        __syncthreads();
    }
    const uint32_t U = overflow ? 0 : carry_units, B = overflow ? 0 : carry_blocks;
    const uint32_t N = min(n_wg, B);
    if (t == 0) {
        units[U] = UnitDesc{B, 0, 0, 0, 0, 0, 0, 0};
        header[0] = U;
        header[1] = B;
        header[2] = N;
        header[3] = overflow;
        header[kVerdict] = 0;
    }
    __threadfence();
    __syncthreads();
    const uint32_t P = 1u << page_shift;
    for (uint32_t w = N + t; w < n_wg; w += 256) { // launched workgroups without work
        WorkDesc d = {};
        work[w] = d;
    }
    for (uint32_t u = t; u < max_units; u += 256) {
        MergeDesc m = {0, 0, 0, 0};
        if (u < U) {
            const UnitDesc ud = units[u];
            const uint32_t wf = (uint32_t)((((uint64_t)ud.block_start + 1) * N - 1) / B);
            const uint32_t wl = (uint32_t)((((uint64_t)ud.block_start + ud.nblocks) * N - 1) / B);
            if (wf != wl) m = MergeDesc{wf + u, wl - wf + 1, ud.rowbeg, ud.nrows_hk};
        }
        merge[u] = m;
    }
    auto range_lo = [&](uint32_t w) { return (uint32_t)((uint64_t)w * B / N); };
    // Range r of the flat block order runs on workgroup r, or (xcd) on workgroup
    // (r % per) * 8 + r / per, so the workgroups of one XCD (workgroup i runs on XCD i % 8) take
    // contiguous ranges.  Records are indexed by range.
    const bool xcd_major = xcd && N == n_wg && N % 8 == 0;
    const uint32_t per = N / 8;
    for (uint32_t w = t; w < N; w += 256) {
        const uint32_t r = xcd_major ? (w % 8) * per + w / 8 : w;
        uint32_t lo = range_lo(r), hi = range_lo(r + 1);
        uint32_t a = 0, e = U; // last unit whose first block <= lo
        while (a + 1 < e) {
            uint32_t mid = (a + e) >> 1;
            if (units[mid].block_start <= lo) a = mid; else e = mid;
        }
        while (a + 1 < U && units[a].block_start + units[a].nblocks <= lo) a++;
        WorkDesc d;
        d.unit = a;
        d.first = units[a];
        d.flags = r << 8;
        d.lo = lo;
        d.hi = hi;
        d.pre = make_uint4(0, 0, 0, 0);
        const uint32_t rel = lo - d.first.block_start;
        if (pages && rel < d.first.cblocks) {
            // logical pages the range starts with; the unfused launch reads a range that
            // begins in the cached keys on into the new keys from the same table, so the
            // pages of every attended key qualify
            const uint32_t lp = (32 * rel) >> page_shift;
            const uint32_t lend = (d.first.kend + P - 1) >> page_shift;
            const uint32_t *row = pages + (size_t)d.first.table_row * stride;
            uint32_t v[kPrePages];
            for (uint32_t i = 0; i < kPrePages; i++) v[i] = lp + i < lend ? row[lp + i] : 0u;
            d.pre = make_uint4(v[0], v[1], v[2], v[3]);
            d.flags |= 1;
        }
        work[w] = d;
    }
}

// ------------------------------------------------------------------ the attention kernel
//
// A workgroup has D/SW wavefronts; wave w owns head_dim slice [SW w, SW w + SW) (SW = 64
// dims on 16-bit and FP8 pools).  Every wave walks every 32-token chunk of the workgroup's
// block range: it loads its slice of K (registers, MFMA A operand) and V (direct-to-LDS on
// 16-bit pools, through registers on FP8 pools), computes its partial S^T = K_w Q_w^T with
// SW/32 MFMAs per 16-token tile, and the partial scores are summed across the waves
// through LDS (one barrier per chunk).  Each wave then runs the same online softmax on the
// same scores and accumulates O^T for its own d slice.  Work inside a workgroup is
// therefore split evenly whatever the segment lengths, and no end-of-segment merge is
// needed: each wave writes its own slice of the output or of the split record.

// Cache policy of the K/V loads: 2 (non-temporal; every key is read once).  On FP8 pools the V
// loads read whole 128-byte head rows per wave; the K loads of the two waves share each line
// (64-byte slices).  Measured on config 5 (one-layer step): V as whole rows with the default
// policy 197.3 -> 196.6 us, non-temporal 183.5 us, and non-temporal K as well 179.1 us (with V
// still in 64-byte slices the non-temporal policy had cost 5 %).

template <int D, int KVT>
struct Cfg {
    static constexpr bool FP8 = KVT == LIA_FP8_E4M3;
    static constexpr bool MBF16 = KVT == LIA_BF16;  // MFMA operand type (f16 for f16 and FP8)
    static constexpr int EB = FP8 ? 1 : 2;          // bytes per stored KV element
    // Each wave owns a head_dim slice of SW dims for P.V: 64 dims of a 16-bit pool (128 bytes
    // of a token; its K in two loads per tile of 8 tokens x 128 bytes each), 64 dims of an FP8
    // pool (64 bytes; with two waves each K load reads 8 tokens' whole 128-byte rows, KROW,
    // and with one wave 16 tokens x 64 bytes).  A lane loads 16 contiguous bytes of a token
    // per load.
    static constexpr int SW = 64;
    static constexpr int AUX = 2;           // cache policy of the K loads and FP8 V loads (nt)
    static constexpr int WAVES = D / SW;            // one wave per slice
    static constexpr int KS = SW / 32;              // k-steps of S^T = K Q^T per tile
    static constexpr int DTW = SW / 16;             // 16-dim tiles of O per wave
    static constexpr int THREADS = WAVES * 64;
    static constexpr int STAGE = 32 * SW;           // staged V per wave: [32 tokens][SW] 16-bit
    static constexpr int KL = FP8 ? 1 : KS;         // K loads per tile (16 bytes each)
    static constexpr int KW = 4 * KL;               // K words per tile and lane
    static constexpr int CPR = SW / 8;              // 16-byte chunks of a staged V row
    static constexpr int VRPI = 64 / CPR;           // staged V rows per direct-to-LDS load
    static constexpr int NV = FP8 ? 2 : 32 / VRPI;  // V loads per chunk
    static constexpr int CPT = D * EB / 16;         // FP8: 16-byte chunks of a head's row
    static constexpr int TPI = 64 / CPT;            // FP8: tokens per V load (whole rows)
    static_assert(!FP8 || TPI * WAVES == 16, "the waves' V loads cover a 16-token tile");
    // FP8 pools with two waves: K is loaded as whole 128-byte head rows too, wave w taking
    // tokens 8w .. 8w+7 of each tile, and each wave forms the full scores of its own 16 tokens
    // of the chunk (QS query operands: both halves of head_dim)
    static constexpr bool KROW = FP8 && WAVES == 2;
    static constexpr int QS = KROW ? 4 : KS;        // query operands per column tile
};

// Staged V rows hold 64 16-bit values (8 chunks of 16 bytes); chunk c of row r sits in slot
// c ^ vswz(r), which flips the chunk pair by row bit 2 so rows r and r + 4 of a transpose
// read (the same banks otherwise) land on distinct banks.
__device__ __forceinline__ uint32_t vswz(uint32_t row) { return 2 * ((row >> 2) & 1); }

template <int D, int KVT>
struct Chunk {
    uint32_t k[2][Cfg<D, KVT>::KW]; // per 16-token tile: this lane's K bytes (A-operand k slots)
    u32x4 v[2];       // FP8 only: this lane's 16 bytes of V per tile, staged later
    float ks[2], vs[2];
};

// Page ids of a key range live in the lanes of the wave: lane i holds the physical page of
// logical page base + i, so the chunk loop gets page ids with v_readlane and issues no
// metadata loads.  A range over the new rows of the step uses identity pages (logical page
// i of the rows is "page" i of a base pointer at the sequence's first new row).
struct PageWindow {
    uint32_t base;  // first logical page covered (wave-uniform)
    uint32_t valid; // page ids below this are readable (pool_pages; no bound for new rows)
    uint32_t page;  // per lane: physical page of logical page base + lane (0 past the end)
    float ks, vs;   // per lane: FP8 scales of that page
};

// Unconditional bounded loads (entries past `limit` read as zero): a load under a branch
// would be waited for at the branch's join, ahead of the first K/V loads.
template <bool FP8>
__device__ __forceinline__ void window_load(const AttnParams &p, PageWindow &w,
                                            const uint32_t *table, uint32_t first, uint32_t limit,
                                            uint32_t hk) {
    const uint32_t idx = first + lane_id();
    w.base = first;
    if (!table) { // identity pages of the new rows
        w.valid = kNone;
        w.page = idx;
        w.ks = w.vs = 1.0f;
        return;
    }
    w.valid = p.pool_pages;
    w.page = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(make_rsrc(table, limit * 4), (int)(idx * 4), 0, 0);
    if constexpr (FP8) {
        const uint32_t n = p.pool_pages * p.hkv * 4;
        const uint32_t off = idx < limit ? (w.page * p.hkv + hk) * 4 : 0x80000000u;
        w.ks = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(make_rsrc(p.k_scales, n), (int)off, 0, 0));
        w.vs = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(make_rsrc(p.v_scales, n), (int)off, 0, 0));
    }
}

// Physical page, live-token count and FP8 scales of the two 16-token tiles of chunk t
// (pages hold >= 16 tokens, so a tile lies in one page).  Tokens at or past tlim are not
// live: their loads return zeros and move no data.  A table entry outside the pool (a stale
// or corrupt block table; packing reports it) has no live tokens either, so no load is
// ever based outside the pool: its keys read as zeros.
struct TilePages {
    uint32_t page[2], live[2];
    float ks[2], vs[2];
};

template <bool FP8>
__device__ __forceinline__ TilePages tile_pages(const PageWindow &w, uint32_t t, uint32_t shift,
                                                uint32_t tlim) {
    TilePages tp;
    const uint32_t P = 1u << shift;
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const uint32_t t0 = t + 16 * j;
        const uint32_t rel = (t0 >> shift) - w.base;
        tp.page[j] = (uint32_t)__builtin_amdgcn_readlane((int)w.page, (int)(rel & 63));
        const uint32_t pstart = t0 & ~(P - 1);
        tp.live[j] = (rel < 64 && tlim > t0 && tp.page[j] < w.valid) ? min(tlim - pstart, P) : 0u;
        if constexpr (FP8) {
            tp.ks[j] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, w.ks), (int)(rel & 63)));
            tp.vs[j] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, w.vs), (int)(rel & 63)));
        } else {
            tp.ks[j] = tp.vs[j] = 1.0f;
        }
    }
    return tp;
}

// The same from pages preloaded by the plan: pre[i] is the page of logical page lp0 + i
// (wave-uniform values, selected without indexing).
__device__ __forceinline__ TilePages tile_pages_pre(uint4 pre, uint32_t lp0, uint32_t t,
                                                    uint32_t shift, uint32_t tlim, uint32_t valid) {
    TilePages tp;
    const uint32_t P = 1u << shift;
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const uint32_t t0 = t + 16 * j;
        const uint32_t rel = (t0 >> shift) - lp0;
        const uint32_t pstart = t0 & ~(P - 1);
        tp.page[j] = rel == 0 ? pre.x : rel == 1 ? pre.y : rel == 2 ? pre.z : pre.w;
        tp.live[j] = (rel < kPrePages && tlim > t0 && tp.page[j] < valid) ? min(tlim - pstart, P) : 0u;
        tp.ks[j] = tp.vs[j] = 1.0f;
    }
    return tp;
}

// Wait until at most `n` vector-memory operations of this wave are outstanding.
template <int n>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(n >= 0 && n < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((n & 0xF) | ((n >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// Vector-memory operations one load_chunk issues (the pipeline waits on this count).
template <int D, int KVT>
constexpr int kLoadsPerChunk = 2 * Cfg<D, KVT>::KL + Cfg<D, KVT>::NV; // K loads + V loads

// Per-lane byte offsets of the chunk loads within their 16-token tile (constant over a key
// range; the tile's position in its page goes into the scalar buffer base).
template <int D, int KVT>
struct DecLanes {
    uint32_t k[Cfg<D, KVT>::KL];                     // K: tile row li, this lane's 16 bytes
    uint32_t v[Cfg<D, KVT>::FP8 ? 1 : Cfg<D, KVT>::NV]; // V: FP8 whole-row load, or each staged load
};

template <int D, int KVT>
__device__ __forceinline__ DecLanes<D, KVT> dec_lanes(uint32_t hk, uint32_t wave, uint32_t row_bytes) {
    using C = Cfg<D, KVT>;
    const uint32_t lane = lane_id(), g = lane >> 4, li = lane & 15;
    const uint32_t slice_off = (hk * D + C::SW * wave) * C::EB;
    DecLanes<D, KVT> r;
    if constexpr (C::FP8) {
        // K: lane (g, li) of a tile reads token li, bytes 16g .. 16g+15 of the wave's 64-byte
        // slice: dims 64w + 16g .. +15 (k slots 8g..8g+7 of k-step s hold dims 64w + 16g + 8s
        // .. +7, and Q is loaded to match)
        r.k[0] = li * row_bytes + slice_off + 16 * g;
        if constexpr (C::KROW) {
            // whole head rows: lane (g, li) reads token 8w + li%8, bytes 16(g + 4(li/8)) .. +15
            // of the head's 128-byte row (dims 64h + 16g .. +15 with h = li/8)
            r.k[0] = (8 * wave + (li & 7)) * row_bytes + hk * D + 16 * (g + 4 * (li >> 3));
        }
    } else {
        // K of a 16-bit pool (128-byte slices, two loads per tile): load q reads tokens
        // 8q .. 8q+7 of the tile as whole slices, lane (g, li) token 8q + li%8, bytes
        // 16(g + 4(li/8)) .. +15, so every load instruction reads whole lines; k_operand()
        // moves the halves into the MFMA layout (token li, dims 32s + 8g .. +7 for k-step s)
#pragma unroll
        for (int q = 0; q < C::KL; q++)
            r.k[q] = (8 * q + (li & 7)) * row_bytes + slice_off + 16 * (g + 4 * (li >> 3));
    }
    if constexpr (C::FP8) {
        // V as whole head rows: wave w reads tokens TPI*w .. +TPI-1 of each tile (lane l:
        // token TPI*w + l/CPT, bytes 16(l%CPT) .. +15 of the head's row)
        r.v[0] = (C::TPI * wave + lane / C::CPT) * row_bytes + hk * D * C::EB + 16 * (lane % C::CPT);
    } else {
        // staged V: load s fills rows VRPI*s .. +VRPI-1, lane l writes slot l%CPR of row
        // VRPI*s + l/CPR with the swizzled chunk
#pragma unroll
        for (int s = 0; s < C::NV; s++) {
            const uint32_t row = C::VRPI * s + lane / C::CPR;
            const uint32_t chunk = (lane % C::CPR) ^ vswz(row);
            r.v[s] = (row & 15) * row_bytes + slice_off + 16 * chunk;
        }
    }
    return r;
}

// Byte span of 16-token tile j of chunk t within a plane: it starts at the tile's first
// token and holds the live tokens from there (a tile with live tokens starts before the
// range end, tile_pages), so loads past them read zeros without touching memory.  Scalar
// arithmetic only; the K and V descriptors of the tile share it.
struct TileSpan {
    uint64_t off;
    uint32_t bytes;
};

__device__ __forceinline__ TileSpan tile_span(const TilePages &tp, int j, uint32_t t, uint32_t shift,
                                              uint32_t row_bytes) {
    const uint32_t P = 1u << shift;
    const uint32_t pb = P * row_bytes; // bytes of a page (all KV heads)
    const uint32_t pg = tp.page[j];
    const uint32_t sh = ((t + 16 * j) & (P - 1)) * row_bytes;
    const uint32_t live = tp.live[j] * row_bytes;
    TileSpan r;
    r.off = (((uint64_t)__umulhi(pg, pb) << 32) | (uint32_t)(pg * pb)) + sh;
    r.bytes = live ? live - sh : 0u;
    return r;
}

// Cache policy of the direct-to-LDS V loads of a 16-bit pool for NT column tiles: non-temporal
// (every key is read once) for single-row units (decode) and two-tile units (MTP verify, short
// chunks) alike.  Measured with every launch on its own layer's pool: config 4 attention 53.6 ->
// 51.0-51.4 us against the default policy, which costs config 2 5 %.  (The default policy had
// measured 1.7 % faster on config 4 when one layer's 274 MB pool was replayed, partly from the
// last-level cache.)
template <int NT>
constexpr int kVAux = 2;

// Loads chunk t (32 tokens, t a multiple of 32) of this wave's d slice from the planes at
// kbase / vbase (the pool, or the step's new rows).  Every load is issued unconditionally:
// tiles past the live keys have empty descriptors, and masked V rows are zero.
template <int D, int KVT, int VAUX>
__device__ __forceinline__ void load_chunk(const AttnParams &p, Chunk<D, KVT> &c, uint32_t t,
                                           const TilePages &tp, const uint8_t *kbase,
                                           const uint8_t *vbase, const DecLanes<D, KVT> &ln,
                                           uint16_t *stage) {
    using C = Cfg<D, KVT>;
    const uint32_t row_bytes = p.hkv * D * C::EB; // bytes per slot (all KV heads)
    TileSpan sp[2];
#pragma unroll
    for (int j = 0; j < 2; j++) {
        sp[j] = tile_span(tp, j, t, p.page_shift, row_bytes);
        if constexpr (C::FP8) {
            c.ks[j] = tp.ks[j];
            c.vs[j] = tp.vs[j];
        }
        const __amdgpu_buffer_rsrc_t r = make_rsrc(kbase + sp[j].off, sp[j].bytes);
#pragma unroll
        for (int q = 0; q < C::KL; q++) {
            u32x4 x = buffer_load16_p<C::AUX>(r, (uint32_t)ln.k[q]);
            c.k[j][4 * q] = x.x; c.k[j][4 * q + 1] = x.y; c.k[j][4 * q + 2] = x.z; c.k[j][4 * q + 3] = x.w;
        }
    }
    if constexpr (C::FP8) {
        // V into registers as whole head rows, so every load reads whole lines; each wave
        // stages both halves of its rows for the wave that owns those dims
#pragma unroll
        for (int j = 0; j < 2; j++)
            c.v[j] = buffer_load16_p<C::AUX>(make_rsrc(vbase + sp[j].off, sp[j].bytes), (uint32_t)ln.v[0]);
    } else {
        // V slice straight to this wave's LDS stage
        __builtin_amdgcn_s_waitcnt(0xC07F); // lgkmcnt(0): earlier reads of this stage are done
#pragma unroll
        for (int s = 0; s < C::NV; s++) {
            const int j = (C::VRPI * s) / 16; // the load's 16-token tile
            const __amdgpu_buffer_rsrc_t vr = make_rsrc(vbase + sp[j].off, sp[j].bytes);
            auto *dst = (__attribute__((address_space(3))) void *)(stage + s * 512);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(vr, dst, 16, (int)ln.v[s], 0, 0, VAUX);
        }
    }
    __builtin_amdgcn_sched_barrier(0);
}

// Query operand of one 16-column tile for this wave's d slice, k-step s: lane (g, col) holds
// q[col][SW*w + (SW/4)*g + 8s .. +7] - the dims the K loads put in the same k slots.
// Padding columns load from an out-of-range offset (zeros) so the loads are unconditional.
template <int D, int KVT>
__device__ __forceinline__ u32x4 load_q(const AttnParams &p, uint32_t row, uint32_t head,
                                        bool valid, uint32_t wave, uint32_t s) {
    using C = Cfg<D, KVT>;
    const uint32_t g = lane_id() >> 4;
    // FP8: a lane's 16 bytes hold dims 16g .. 16g+15 (k-steps 0, 1) of the wave's slice, or
    // with whole-row K (KROW) operand s = 2h + k holds dims 64h + 16g + 8k .. +7 of the head;
    // 16-bit: load s holds dims 32s + 8g .. +7 of the wave's slice
    const uint32_t at = (row * p.hq + head) * D +
                        (C::KROW ? 64 * (s >> 1) + 16 * g + 8 * (s & 1)
                                 : C::SW * wave + (C::FP8 ? 16 * g + 8 * s : 32 * s + 8 * g));
    const uint32_t qb = p.q_f32 ? 4 : 2;
    const __amdgpu_buffer_rsrc_t r = make_rsrc(p.q, p.n_rows * p.hq * D * qb);
    const uint32_t off = valid ? at * qb : 0x80000000u;
    float x[8];
    if (p.q_f32) {
        // Cast the whole vector: with this toolchain, bit-casting single elements of a
        // 128-bit buffer load to float narrows the load to its first dword.
        const f32x4 a = __builtin_bit_cast(f32x4, buffer_load16(r, off));
        const f32x4 b = __builtin_bit_cast(f32x4, buffer_load16(r, off + 16));
        x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
        x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
    } else {
        const u32x4 w = buffer_load16(r, off);
        if constexpr (C::MBF16) return w;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            x[2 * e] = bf16_to_f32(w[e] & 0xffffu);
            x[2 * e + 1] = bf16_to_f32(w[e] >> 16);
        }
    }
    return u32x4{pack2<C::MBF16>(x[0], x[1]), pack2<C::MBF16>(x[2], x[3]),
                 pack2<C::MBF16>(x[4], x[5]), pack2<C::MBF16>(x[6], x[7])};
}

template <int D, int NT, int KVT>
struct State {
    u32x4 qr[NT][Cfg<D, KVT>::QS];
    uint32_t lo;       // first key of the current range (wave-uniform)
    uint32_t lim[NT];  // per column: live keys of the range, counted from lo
    uint32_t free_lo, free_hi; // keys live for every valid column of the unit (wave-uniform)
    // per column: reference maximum of the scaled scores in the log2 domain (0 before the
    // first live key) and the exponent above which it is raised (-inf before the first live
    // key, then 2^8)
    float m[NT], thr[NT];
    // the mass: every row of an MFMA tile against ones on 16-bit pools; on FP8 pools (whose
    // weights carry the V page scale) element 0 holds this lane's share, summed across lanes
    // at the end
    f32x4 l[NT];
    f32x4 o[NT][Cfg<D, KVT>::DTW];
    uint32_t fold;    // read-only variant: XOR of the K words this lane loaded of keys in
    uint32_t fold_hi; // [lo, fold_hi), the range (a chunk starts at a 32-key boundary, so a
                      // range's first chunk also loads keys of the range before it)
};

// K operand of k-step ks of a 16-bit tile from the two whole-line loads L0 (tokens 0-7) and L1
// (tokens 8-15): lane (g, li) of L0 holds token li%8, dims 8g .. +7 (li < 8) or 32 + 8g .. +7
// (li >= 8), and L1 the same for tokens 8-15.  The operand wants token li, dims 32ks + 8g .. +7
// in lane (g, li): k-step 0 keeps L0 in lanes li < 8 and takes L1 from lane li - 8 in the
// others; k-step 1 keeps L1 in lanes li >= 8 and takes L0 from lane li + 8 in the others
// (a row rotation by 8 written to half the banks of each row).
template <int KS>
__device__ __forceinline__ u32x4 k_operand(const uint32_t *k) {
    constexpr int keep = KS == 0 ? 0 : 4, take = KS == 0 ? 4 : 0;
    constexpr int banks = KS == 0 ? 0xC : 0x3; // lanes 8-15 / 0-7 of each row take the rotation
    u32x4 a;
#pragma unroll
    for (int w = 0; w < 4; w++)
        a[w] = (uint32_t)__builtin_amdgcn_update_dpp((int)k[keep + w], (int)k[take + w], 0x128 /* row_ror:8 */,
                                                     0xF, banks, false);
    return a;
}

// One chunk: partial scores for this wave's d slice, cross-wave sum through LDS, online
// softmax (identical in every wave), O^T += V^T P^T for the wave's two 16-dim tiles.
template <int D, int NT, int KVT, int VW = kLoadsPerChunk<D, KVT>>
__device__ __forceinline__ void compute_chunk(const AttnParams &p, const Chunk<D, KVT> &c,
                                              uint32_t t, State<D, NT, KVT> &st,
                                              uint16_t *stage, f32x4 *sx, uint32_t wave) {
    using C = Cfg<D, KVT>;
    const uint32_t lane = lane_id(), g = lane >> 4, li = lane & 15;
    if constexpr (C::FP8) {
        // convert this lane's FP8 V (16 values per tile) to f16 and stage it: lane l of tile j
        // holds dims 16(l%CPT) .. +15 of token 16j + TPI*w + l/CPT, i.e. 8-value chunks c0 and
        // c0 + 1 (c0 = 2(l%CPT)) of the head's row, which belong to the stage of the wave owning
        // dims 64(c0/8) .. (staging is double-buffered by chunk and read after the barrier)
        uint16_t *base = stage - wave * C::STAGE;
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const uint32_t row = 16 * j + C::TPI * wave + lane / C::CPT, c0 = 2 * (lane % C::CPT);
            const u32x2 a = e4m3x4_to_f16x4_scaled(c.v[j].x), b = e4m3x4_to_f16x4_scaled(c.v[j].y);
            const u32x2 e = e4m3x4_to_f16x4_scaled(c.v[j].z), f = e4m3x4_to_f16x4_scaled(c.v[j].w);
            uint16_t *dst = base + (c0 / 8) * C::STAGE + row * C::SW;
            const uint32_t cc = c0 % 8;
            *(u32x4 *)(dst + ((cc ^ vswz(row)) * 8)) = u32x4{a.x, a.y, b.x, b.y};
            *(u32x4 *)(dst + (((cc + 1) ^ vswz(row)) * 8)) = u32x4{e.x, e.y, f.x, f.y};
        }
    } else {
        wait_vmcnt<VW>(); // this chunk's V is in LDS (VW = memory ops issued after its loads)
    }
    float kscale[2] = {p.scale_log2, p.scale_log2};
    float vscale[2] = {1.0f, 1.0f};
    if constexpr (C::FP8) {
#pragma unroll
        for (int j = 0; j < 2; j++) {
            // the staged f16 V holds value * 2^-8 and O carries that factor until the unit
            // ends (kFp8VUnscale), so a weight x * vs (x <= 2^8) stays finite in f16 for every
            // page scale below 256
            kscale[j] = p.scale_log2 * c.ks[j] * 256.0f;
            vscale[j] = c.vs[j];
        }
    }
    if constexpr (C::KROW) {
        // Whole-row K: lane (g, li) of tile j holds token 8w + li%8, dims 64h + 16g .. +15 with
        // h = li/8.  One row rotation by 8 (written to half the banks of each 16-lane row) makes
        // operand h hold half h of this wave's 16 tokens of the chunk: rows 0-7 tile 0's, rows
        // 8-15 tile 1's.  Against the queries' half h they sum to the full scores of those
        // tokens, one tile per wave.
        uint32_t kh[2][4];
#pragma unroll
        for (int w = 0; w < 4; w++) {
            kh[0][w] = (uint32_t)__builtin_amdgcn_update_dpp((int)c.k[0][w], (int)c.k[1][w], 0x128 /* row_ror:8 */,
                                                             0xF, 0xC, false);
            kh[1][w] = (uint32_t)__builtin_amdgcn_update_dpp((int)c.k[1][w], (int)c.k[0][w], 0x128 /* row_ror:8 */,
                                                             0xF, 0x3, false);
        }
        u32x4 a[2][2]; // [half][k-step]: bytes 8k .. 8k+7 of the lane's 16 as f16
#pragma unroll
        for (int h = 0; h < 2; h++)
#pragma unroll
            for (int k = 0; k < 2; k++) {
                const u32x2 x0 = e4m3x4_to_f16x4_scaled(kh[h][2 * k]), x1 = e4m3x4_to_f16x4_scaled(kh[h][2 * k + 1]);
                a[h][k] = u32x4{x0.x, x0.y, x1.x, x1.y};
            }
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
            f32x4 sp = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int h = 0; h < 2; h++)
#pragma unroll
                for (int k = 0; k < 2; k++) sp = mfma16x16x32<C::MBF16>(a[h][k], st.qr[nt][2 * h + k], sp);
            sx[(wave * NT + nt) * 64 + lane] = sp;
        }
    } else {
        // partial scores of this wave's slice -> LDS
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
#pragma unroll
            for (int j = 0; j < 2; j++) {
                f32x4 sp = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int ks = 0; ks < C::KS; ks++) {
                    u32x4 a;
                    if constexpr (C::FP8) {
                        // k-step ks: bytes 8ks .. 8ks+7 of the lane's 16
                        u32x2 x0 = e4m3x4_to_f16x4_scaled(c.k[j][2 * ks]);
                        u32x2 x1 = e4m3x4_to_f16x4_scaled(c.k[j][2 * ks + 1]);
                        a = u32x4{x0.x, x0.y, x1.x, x1.y};
                    } else {
                        a = ks == 0 ? k_operand<0>(c.k[j]) : k_operand<1>(c.k[j]);
                    }
                    sp = mfma16x16x32<C::MBF16>(a, st.qr[nt][ks], sp);
                }
                sx[((wave * NT + nt) * 2 + j) * 64 + lane] = sp;
            }
        }
    }
    // Only the LDS score exchange needs ordering (a full __syncthreads would also drain the
    // prefetch loads).
    lds_barrier();
    // Online softmax per column nt*16 + li over tokens t + 16j + 4g + i (live when lo <= token
    // < lo + lim): masked only when the chunk leaves [free_lo, free_hi); the exponent of a
    // score is one fma against a lazily raised reference, which only a ballot of lanes above
    // its threshold (2^8 once the column has a live key, any live key before) makes the wave
    // reduce across lanes and rescale.  Numerator and denominator share the reference, so the
    // normalised result is unchanged.
    const bool masked = !(t >= st.free_lo && t + 32 <= st.free_hi);
#pragma unroll
    for (int nt = 0; nt < NT; nt++) {
        f32x4 s[2];
#pragma unroll
        for (int j = 0; j < 2; j++) {
            if constexpr (C::KROW) {
                // rows 4g .. 4g+3 of tile j are tokens 4g .. of wave g/2, rows 8j + 4(g%2) ..
                // of its tile: lane 16(2j + g%2) + li
                const uint32_t g = lane >> 4;
                s[j] = sx[((g >> 1) * NT + nt) * 64 + 16 * (2 * j + (g & 1)) + (lane & 15)];
                continue;
            }
            s[j] = sx[((0 * NT + nt) * 2 + j) * 64 + lane];
#pragma unroll
            for (int w = 1; w < C::WAVES; w++) s[j] += sx[((w * NT + nt) * 2 + j) * 64 + lane];
        }
        float e[2][4];
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int i = 0; i < 4; i++) e[j][i] = __builtin_fmaf(s[j][i], kscale[j], -st.m[nt]);
        // masked after the scaling: a tile with no live key has scale 0 on FP8 pools
        if (masked) {
#pragma unroll
            for (int j = 0; j < 2; j++)
#pragma unroll
                for (int i = 0; i < 4; i++)
                    if (t + 16 * j + 4 * g + i - st.lo >= st.lim[nt]) e[j][i] = -INFINITY;
        }
        float mx = fmaxf(fmaxf(fmaxf(e[0][0], e[0][1]), fmaxf(e[0][2], e[0][3])),
                         fmaxf(fmaxf(e[1][0], e[1][1]), fmaxf(e[1][2], e[1][3])));
        if (__builtin_amdgcn_ballot_w64(mx > st.thr[nt])) { // wave-uniform: rare after the first chunk
            mx = rows_max(mx);
            if (mx > st.thr[nt]) { // the same in the 4 lanes of the column
                const float factor = fast_exp2(-mx); // 0 before the column's first live key
                st.l[nt] *= factor;
#pragma unroll
                for (int n = 0; n < C::DTW; n++) st.o[nt][n] *= factor;
                st.m[nt] += mx;
                st.thr[nt] = 8.0f;
#pragma unroll
                for (int j = 0; j < 2; j++)
#pragma unroll
                    for (int i = 0; i < 4; i++) e[j][i] -= mx;
            }
        }
        float pr[2][4];
        float sum = 0.0f;
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float x = fast_exp2(e[j][i]);
                if constexpr (C::FP8) {
                    sum += x;
                    pr[j][i] = x * vscale[j];
                } else {
                    pr[j][i] = x;
                }
            }
        if constexpr (C::FP8) st.l[nt][0] += sum;
        const u32x4 pb = u32x4{pack2<C::MBF16>(pr[0][0], pr[0][1]), pack2<C::MBF16>(pr[0][2], pr[0][3]),
                               pack2<C::MBF16>(pr[1][0], pr[1][1]), pack2<C::MBF16>(pr[1][2], pr[1][3])};
#pragma unroll
        for (int n = 0; n < C::DTW; n++) {
            // V^T operand: d rows 16n .. 16n+15 of the slice, k slots = tokens
            // {4g..4g+3, 16+4g..16+4g+3} (transpose reads of the staged rows).
            const uint32_t row0 = 4 * g + li / 4, ch = 2 * n + ((li & 3) >> 1);
            const uint16_t *r0 = stage + row0 * C::SW + ((ch ^ vswz(row0)) * 8) + (li & 1) * 4;
            const uint16_t *r1 = r0 + 16 * C::SW; // row0 + 16 has the same swizzle
            s16x4 a0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (__attribute__((address_space(3))) s16x4 *)(r0));
            s16x4 a1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (__attribute__((address_space(3))) s16x4 *)(r1));
            u32x2 b0 = __builtin_bit_cast(u32x2, a0), b1 = __builtin_bit_cast(u32x2, a1);
            st.o[nt][n] = mfma16x16x32<C::MBF16>(u32x4{b0.x, b0.y, b1.x, b1.y}, pb, st.o[nt][n]);
        }
        if constexpr (!C::FP8) {
            // the mass: the column's sum of this chunk's (rounded) weights, in every tile row
            constexpr uint32_t one2 = C::MBF16 ? 0x3F803F80u : 0x3C003C00u;
            st.l[nt] = mfma16x16x32<C::MBF16>(u32x4{one2, one2, one2, one2}, pb, st.l[nt]);
        }
    }
}

// The read-only variant's chunk t: wait for the chunk's loads as compute_chunk does, pass the
// per-chunk barrier that keeps the workgroup's waves in step (on FP8 pools the two waves' K
// slices share each 128-byte line: without it the waves drift apart and a line is fetched
// twice), and fold the loaded words of its keys inside the range, with no attention arithmetic
// or score exchange.  Lane (g, li) holds K of key t + 16j + li of tile j on FP8 pools, and of
// keys t + 16j + li%8 and t + 16j + 8 + li%8 (one per load) on 16-bit pools; on FP8 pools, whose V
// comes through registers, it also holds V of key t + 16j + TPI * wave + lane / CPT (16-bit
// pools load V straight into LDS, which nothing reads here).
template <int D, int NT, int KVT, int VW = kLoadsPerChunk<D, KVT>>
__device__ __forceinline__ void fold_chunk(const Chunk<D, KVT> &c, uint32_t t, State<D, NT, KVT> &st,
                                           uint32_t wave) {
    using C = Cfg<D, KVT>;
    if constexpr (!C::FP8) wait_vmcnt<VW>(); // V in LDS; register loads are waited for on use
    lds_barrier();
    const uint32_t lane = lane_id(), li = lane & 15;
    auto in = [&](uint32_t key) { return key >= st.lo && key < st.fold_hi; };
#pragma unroll
    for (int j = 0; j < 2; j++) {
        if constexpr (C::FP8) {
            uint32_t x = 0;
#pragma unroll
            for (int w = 0; w < C::KW; w++) x ^= c.k[j][w];
            st.fold ^= in(t + 16 * j + (C::KROW ? 8 * wave + (li & 7) : li)) ? x : 0u;
        } else {
            // load q holds token 8q + li%8 of the tile
#pragma unroll
            for (int q = 0; q < C::KL; q++) {
                const uint32_t x = c.k[j][4 * q] ^ c.k[j][4 * q + 1] ^ c.k[j][4 * q + 2] ^ c.k[j][4 * q + 3];
                st.fold ^= in(t + 16 * j + 8 * q + (li & 7)) ? x : 0u;
            }
        }
        if constexpr (C::FP8) {
            const uint32_t y = c.v[j].x ^ c.v[j].y ^ c.v[j].z ^ c.v[j].w;
            st.fold ^= in(t + 16 * j + C::TPI * wave + lane / C::CPT) ? y : 0u;
        }
    }
}

// One pipeline step: issue the loads of chunk `tn` into stage `sn` (registers cn), then
// compute chunk `tc` from stage `sc` (registers cc).  The two stages are restrict
// parameters: the transpose reads of `sc` are then known not to alias the direct-to-LDS
// loads still in flight into `sn`, so no full vmcnt drain is needed before them.
template <int D, int NT, int KVT, bool RO = false, int VW = kLoadsPerChunk<D, KVT>>
__device__ __forceinline__ void pipeline_step(const AttnParams &p, Chunk<D, KVT> &cn, uint32_t tn,
                                              const TilePages &tpn, uint16_t *__restrict__ sn,
                                              const Chunk<D, KVT> &cc, uint32_t tc,
                                              uint16_t *__restrict__ sc, const uint8_t *kbase,
                                              const uint8_t *vbase, const DecLanes<D, KVT> &ln,
                                              uint32_t wave, State<D, NT, KVT> &st, f32x4 *sx) {
    load_chunk<D, KVT, kVAux<NT>>(p, cn, tn, tpn, kbase, vbase, ln, sn);
    if constexpr (RO) fold_chunk<D, NT, KVT, VW>(cc, tc, st, wave);
    else compute_chunk<D, NT, KVT, VW>(p, cc, tc, st, sc, sx, wave);
}

// Attends keys [s_lo, s_hi) of one source (coordinates of that source: token index in the
// pool, or new-row index) into the running state.  Windows of at most 64 pages; the
// first two chunks of the workgroup's first range take their pages from the plan.  While
// q_pending is set (single-tile units only), qload() loads the unit's queries right after the
// first chunk's K/V loads and before the second's, so the stream starts without waiting for
// the query addressing and the first chunk's wait covers the queries.
template <int D, int NT, int KVT, bool RO = false, class QL>
__device__ __forceinline__ void run_range(const AttnParams &p, const uint8_t *kbase,
                                          const uint8_t *vbase, const uint32_t *table,
                                          uint32_t s_lo, uint32_t s_hi, bool use_pre,
                                          uint4 pre, uint32_t hk, uint32_t wave, State<D, NT, KVT> &st,
                                          uint16_t *stage0, uint16_t *stage1, f32x4 *sxb,
                                          uint32_t &parity, bool &q_pending, const QL &qload) {
    using C = Cfg<D, KVT>;
    constexpr uint32_t SX = C::WAVES * NT * 2 * 64;
    const uint32_t shift = p.page_shift;
    const uint32_t page_limit = (s_hi + (1u << shift) - 1) >> shift;
    const DecLanes<D, KVT> ln = dec_lanes<D, KVT>(hk, wave, p.hkv * D * C::EB);
    // wave-uniform bases, so the descriptors are built by scalar instructions
    kbase = uniform_ptr(kbase);
    vbase = uniform_ptr(vbase);
    for (uint32_t wbeg = s_lo & ~31u; wbeg < s_hi;) {
        const uint32_t wend = min(s_hi, ((wbeg >> shift) + 64) << shift);
        PageWindow win;
        Chunk<D, KVT> c0, c1;
        // prologue: chunks wbeg and wbeg + 32 in flight, chunk wbeg computed
        bool reorder = false; // single-tile units on 16-bit pools (two-tile units spill with both forms)
        if constexpr (NT == 1 && !C::FP8) reorder = use_pre && table != nullptr;
        if (reorder) {
            // the first two chunks' pages come from the plan: their loads (and the queries) go
            // out first and the window's table load after them, before the second chunk's, so
            // the first chunk's wait counts one more operation after its own
            const TilePages tp0 = tile_pages_pre(pre, wbeg >> shift, wbeg, shift, wend, p.pool_pages);
            const TilePages tp1 = tile_pages_pre(pre, wbeg >> shift, wbeg + 32, shift, wend, p.pool_pages);
            use_pre = false;
            load_chunk<D, KVT, kVAux<NT>>(p, c0, wbeg, tp0, kbase, vbase, ln, stage0);
            if (q_pending) {
                qload();
                q_pending = false;
            }
            window_load<C::FP8>(p, win, table, wbeg >> shift, page_limit, hk);
            pipeline_step<D, NT, KVT, RO, kLoadsPerChunk<D, KVT> + 1>(p, c1, wbeg + 32, tp1, stage1, c0, wbeg,
                                                                      stage0, kbase, vbase, ln, wave, st,
                                                                      sxb + parity * SX);
        } else {
            window_load<C::FP8>(p, win, table, wbeg >> shift, page_limit, hk);
            TilePages tp0, tp1;
            if (!C::FP8 && use_pre) {
                tp0 = tile_pages_pre(pre, wbeg >> shift, wbeg, shift, wend, p.pool_pages);
                tp1 = tile_pages_pre(pre, wbeg >> shift, wbeg + 32, shift, wend, p.pool_pages);
                use_pre = false;
            } else {
                tp0 = tile_pages<C::FP8>(win, wbeg, shift, wend);
                tp1 = tile_pages<C::FP8>(win, wbeg + 32, shift, wend);
            }
            load_chunk<D, KVT, kVAux<NT>>(p, c0, wbeg, tp0, kbase, vbase, ln, stage0);
            if constexpr (NT == 1) {
                if (q_pending) {
                    qload();
                    q_pending = false;
                }
            }
            pipeline_step<D, NT, KVT, RO>(p, c1, wbeg + 32, tp1, stage1, c0, wbeg, stage0, kbase, vbase, ln,
                                          wave, st, sxb + parity * SX);
        }
        parity ^= 1;
        if (wbeg + 32 < wend) {
            for (uint32_t t = wbeg + 32;; t += 64) {
                // loads past wend carry no traffic
                pipeline_step<D, NT, KVT, RO>(p, c0, t + 32, tile_pages<C::FP8>(win, t + 32, shift, wend),
                                              stage0, c1, t, stage1, kbase, vbase, ln, wave, st,
                                              sxb + parity * SX);
                parity ^= 1;
                if (t + 32 >= wend) break;
                pipeline_step<D, NT, KVT, RO>(p, c1, t + 64, tile_pages<C::FP8>(win, t + 64, shift, wend),
                                              stage1, c0, t + 32, stage0, kbase, vbase, ln, wave, st,
                                              sxb + parity * SX);
                parity ^= 1;
                if (t + 64 >= wend) break;
            }
        }
        wait_vmcnt<0>(); // the trailing (empty) loads target a stage about to be reused
        wbeg = wend;
    }
}

// Canonical NaN of a 16-bit pool element, as a round trip through f32 produces it (the
// append converts every element src -> f32 -> pool dtype with round-to-nearest-even).
template <int KVT>
__device__ __forceinline__ uint32_t canon16x2(uint32_t w) {
    uint32_t r = 0;
#pragma unroll
    for (int h = 0; h < 2; h++) {
        const uint32_t x = (w >> (16 * h)) & 0xffffu;
        uint32_t y = x;
        if constexpr (KVT == LIA_BF16) {
            if ((x & 0x7fffu) > 0x7f80u) y = (x & 0x8000u) | 0x7fc0u;
        } else {
            if ((x & 0x7fffu) > 0x7c00u) y = (x & 0x8000u) | 0x7e00u;
        }
        r |= y << (16 * h);
    }
    return r;
}

// Fused append: scatter the step's new K/V rows into the pool (16-byte pieces spread over
// the launch's workgroups).  No workgroup of the launch reads these slots: every range over
// the new keys reads the caller's rows.
template <int D, int KVT>
__device__ __forceinline__ void append_rows(const AttnParams &p, uint32_t wg, uint32_t N) {
    using C = Cfg<D, KVT>;
    const uint32_t row_bytes = p.hkv * D * C::EB;
    const uint32_t pieces = row_bytes / 16;
    const uint32_t total = p.n_rows * pieces * 2;
    for (uint32_t i = wg * blockDim.x + threadIdx.x; i < total; i += N * blockDim.x) {
        const uint32_t plane = i / (p.n_rows * pieces), rem = i % (p.n_rows * pieces);
        const uint32_t r = rem / pieces, k = rem % pieces;
        const uint32_t slot = p.slots[r];
        if (slot == kNone || (slot >> p.page_shift) >= p.pool_pages) continue; // outside the pool
        const u32x4 *src = (const u32x4 *)((const uint8_t *)(plane ? p.newv : p.newk) + (size_t)r * row_bytes) + k;
        u32x4 *dst = (u32x4 *)((uint8_t *)(plane ? p.vc_w : p.kc_w) + (size_t)slot * row_bytes) + k;
        u32x4 x = *src;
        *dst = u32x4{canon16x2<KVT>(x.x), canon16x2<KVT>(x.y), canon16x2<KVT>(x.z), canon16x2<KVT>(x.w)};
    }
}

// Four values of a normalised 16-bit split record row in the pool's type.  O / l is a convex
// combination of V rows up to the rounding of the MFMA's 16-bit weights, so it can pass
// max |V| by a rounding step: f16 rows saturate finite values to +-65504 instead of
// rounding them to infinity.
template <int KVT>
__device__ __forceinline__ u32x2 record_pack(f32x4 v) {
    if constexpr (KVT == LIA_F16) {
#pragma unroll
        for (int i = 0; i < 4; i++)
            if (fabsf(v[i]) > 65504.0f && fabsf(v[i]) < INFINITY) v[i] = copysignf(65504.0f, v[i]);
    }
    return u32x2{pack2<KVT == LIA_BF16>(v.x, v.y), pack2<KVT == LIA_BF16>(v.z, v.w)};
}

// One column's split record for this wave's d slice (SW dims), with the reference max and
// mass.  With a 16-bit output, record rows of 16-bit pools hold O / l in the pool's type
// (half the record traffic of f32; the rounding is within a bf16 output's).  Rows for f32
// outputs, and rows of FP8 pools, whose values carry a page scale, are unnormalised f32.
template <int KVT>
constexpr bool kRecord16 = KVT != LIA_FP8_E4M3;

template <int D, int SW, int KVT>
__device__ __forceinline__ void store_record(const AttnParams &p, size_t rb, const f32x4 (&o)[SW / 16],
                                             float m, float l, uint32_t wave) {
    const uint32_t g = lane_id() >> 4;
    if (kRecord16<KVT> && !p.out_f32) {
        uint16_t *po = (uint16_t *)p.part_o + rb * D + SW * wave + 4 * g;
        const float inv = l > 0.0f ? 1.0f / l : 0.0f;
#pragma unroll
        for (int n = 0; n < SW / 16; n++) *(u32x2 *)(po + 16 * n) = record_pack<KVT>(o[n] * inv);
    } else {
        float *po = p.part_o + rb * D + SW * wave + 4 * g;
#pragma unroll
        for (int n = 0; n < SW / 16; n++) *(f32x4 *)(po + 16 * n) = o[n];
    }
    if (wave == 0 && g == 0) {
        p.part_ml[rb * 2] = m;
        p.part_ml[rb * 2 + 1] = l;
    }
}

// FP8 pools stage V as value * 2^-8 (e4m3x4_to_f16x4_scaled); O is scaled back when a unit ends.
constexpr float kFp8VUnscale = 256.0f;

// At most 6 (16-bit pools) or 8 (FP8) decode waves run per CU, so the kernel may use the
// registers of 3 (168) or 2 (256) waves per SIMD instead of squeezing into 4's (128).
template <int KVT>
constexpr int kMinWavesPerEU = KVT == LIA_FP8_E4M3 ? 2 : 3;

// The workgroup-size bound (D/32 waves) is looser than the D/SW waves launched: the
// exact bound changes register allocation and measured 1 % slower on a batch-8 bf16 decode.
//
// RO (lia_paged_read): the same plan, ranges, loads, pipeline, waits and per-chunk barrier with
// the attention arithmetic, the score exchange and every store but one left out - each wave folds the K words
// it loaded and writes the fold to ((uint32_t *)p.out)[wg * waves + wave].  It times the
// kernel's own memory access on its own.
template <int D, int NT, int KVT, bool RO = false>
__global__ __launch_bounds__(D / 32 * 64, kMinWavesPerEU<KVT>) void attention_kernel(AttnParams p) {
    using C = Cfg<D, KVT>;
    constexpr uint32_t COLS = 16 * NT;
    // Two distinct LDS objects for the two V stages, so the compiler can tell a transpose
    // read of one stage from the direct-to-LDS loads in flight into the other; partial
    // scores are exchanged through two alternating buffers (one barrier per chunk).
    __shared__ __attribute__((aligned(16))) uint16_t vst0[C::WAVES * C::STAGE];
    __shared__ __attribute__((aligned(16))) uint16_t vst1[C::WAVES * C::STAGE];
    __shared__ f32x4 sxb[2 * C::WAVES * NT * 2 * 64];
    const uint32_t wg = blockIdx.x;
    const WorkDesc wd = p.work[wg]; // the only load before the first K/V loads
    if constexpr (!RO) {
        // The hardware already issues the waves of a CU's oldest workgroup first; raising the
        // first dispatch round's waves to priority 2 and the second's to 1 (the third keeps 0)
        // makes that order firm: config 2 18.54-18.63 us against 18.67-18.74, and 9,244-9,257
        // against 9,208-9,233 tokens/s (equal priorities for the rounds in reverse: 1 % slower).
        const uint32_t round = wg / p.round_wg;
        if (round == 0) __builtin_amdgcn_s_setprio(2);
        else if (round == 1) __builtin_amdgcn_s_setprio(1);
    }
    const uint32_t tid = threadIdx.x, lane = tid & 63;
    const uint32_t wave = (uint32_t)__builtin_amdgcn_readfirstlane((int)(tid >> 6)); // SGPR
    const uint32_t g = lane >> 4, li = lane & 15;
    uint16_t *stage0 = vst0 + wave * C::STAGE;
    uint16_t *stage1 = vst1 + wave * C::STAGE;
    uint32_t u = wd.unit, lo = wd.lo;
    const uint32_t hi = wd.hi;
    const bool fused = p.newk != nullptr;
    const uint32_t row_bytes = p.hkv * D * C::EB;
    uint32_t parity = 0; // alternates the score-exchange buffer across all chunks
    bool first = true;
    uint32_t fold = 0;

    // the plan guarantees a unit covers every block of a non-empty range
    while (lo < hi) {
        UnitDesc ud;
        if (first) ud = wd.first;
        else ud = p.units[u];
        const bool use_pre = first && (wd.flags & 1);
        first = false;
        const uint32_t bs = ud.block_start, uend = bs + ud.nblocks;
        if (uend <= lo) { u++; continue; }
        const uint32_t seg_end = min(hi, uend);
        const uint32_t hk = unit_head(ud), nrows = unit_rows(ud);
        const uint32_t *table = p.pages + (size_t)ud.table_row * p.stride;
        const uint32_t kend = ud.kend, kcache = ud.kcache, cb = ud.cblocks;
        const uint32_t pos0 = kend - nrows;
        const uint32_t ncols = nrows * p.group;

        State<D, NT, KVT> st;
        st.fold = 0;
        uint32_t climit[NT]; // per column: keys it attends (causal limit), 0 for padding
        // the unit's queries: on single-tile units (decode) 16-bit queries are loaded by the first
        // range after its first chunk's K/V loads (config 2: 19.3-19.6 -> 19.0-19.2 us); f32
        // queries here, since their conversion waits for their loads (and would then wait for the
        // first chunk's too), and on two-tile units too, where the deferred operands' registers
        // made the kernel spill (config 4: 52.9 -> 57.3 us)
        bool q_pending = NT == 1;
        auto qload = [&]() {
#pragma unroll
            for (int nt = 0; nt < NT; nt++) {
                const uint32_t col = nt * 16 + li;
                const bool valid = col < ncols;
                const uint32_t ri = valid ? col / p.group : 0;
#pragma unroll
                for (int ks = 0; ks < C::QS; ks++)
                    st.qr[nt][ks] = load_q<D, KVT>(p, ud.rowbeg + ri, hk * p.group + col % p.group, valid, wave, ks);
            }
        };
        if (!q_pending || p.q_f32) {
            qload();
            q_pending = false;
        }
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
            const uint32_t col = nt * 16 + li;
            const bool valid = col < ncols;
            const uint32_t ri = valid ? col / p.group : 0;
            climit[nt] = valid ? pos0 + ri + 1 : 0;
            st.m[nt] = 0.0f;
            st.thr[nt] = -INFINITY;
            st.l[nt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int n = 0; n < C::DTW; n++) st.o[nt][n] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        }
        // Block i of the unit covers keys [32i, 32i+32) of the cached run for i < cb and
        // [kcache + 32(i-cb), ...) of the new run otherwise.
        const uint32_t a = lo - bs, e = seg_end - bs;
        auto key_of = [&](uint32_t i) { return i < cb ? 32 * i : min(kcache + 32 * (i - cb), kend); };
        auto set_limits = [&](uint32_t r_lo, uint32_t r_hi, uint32_t origin) {
            st.lo = r_lo;
#pragma unroll
            for (int nt = 0; nt < NT; nt++) {
                const int w = (int)min(climit[nt] - origin, r_hi) - (int)r_lo;
                st.lim[nt] = climit[nt] && w > 0 ? (uint32_t)w : 0u;
            }
            // keys live for every valid column: those of the unit's first row
            const int w0 = (int)min(pos0 + 1 - origin, r_hi) - (int)r_lo;
            st.free_lo = r_lo;
            st.free_hi = r_lo + (w0 > 0 ? (uint32_t)w0 : 0u);
            st.fold_hi = r_hi;
        };
        const uint8_t *kpool = (const uint8_t *)p.kc, *vpool = (const uint8_t *)p.vc;
        if (!fused) {
            // both runs from the pool: one contiguous key range
            const uint32_t r_lo = key_of(a), r_hi = min(key_of(e), kend);
            set_limits(r_lo, r_hi, 0);
            run_range<D, NT, KVT, RO>(p, kpool, vpool, table, r_lo, r_hi, use_pre, wd.pre, hk, wave, st,
                                      stage0, stage1, sxb, parity, q_pending, qload);
        } else {
            if (a < cb) {
                const uint32_t r_lo = 32 * a, r_hi = min(32 * min(e, cb), kcache);
                set_limits(r_lo, r_hi, 0);
                run_range<D, NT, KVT, RO>(p, kpool, vpool, table, r_lo, r_hi, use_pre, wd.pre, hk, wave,
                                          st, stage0, stage1, sxb, parity, q_pending, qload);
            }
            if (e > cb) {
                // new keys: row kcache + i of the sequence is packed row r0 + i
                const uint32_t r0 = ud.rowbeg - (pos0 - kcache);
                const uint32_t r_lo = 32 * (max(a, cb) - cb), r_hi = min(32 * (e - cb), kend - kcache);
                set_limits(r_lo, r_hi, kcache);
                run_range<D, NT, KVT, RO>(p, (const uint8_t *)p.newk + (size_t)r0 * row_bytes,
                                          (const uint8_t *)p.newv + (size_t)r0 * row_bytes, nullptr,
                                          r_lo, r_hi, false, wd.pre, hk, wave, st, stage0, stage1, sxb,
                                          parity, q_pending, qload);
            }
        }

        if constexpr (RO) {
            fold ^= st.fold;
            lo = seg_end;
            u++;
            continue;
        }
        // Finalise this wave's d slice: normalised output or a split record.
        const bool whole = lo == bs && seg_end == uend;
        const uint32_t rec = (wd.flags >> 8) + u;
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
            const float lt = C::FP8 ? rows_sum(st.l[nt][0]) : st.l[nt][0];
            const uint32_t col = nt * 16 + li;
            if (col >= ncols) continue;
            const uint32_t row = ud.rowbeg + col / p.group;
            const uint32_t head = hk * p.group + col % p.group;
            if constexpr (C::FP8) {
#pragma unroll
                for (int n = 0; n < C::DTW; n++) st.o[nt][n] *= kFp8VUnscale;
            }
            if (whole) {
                const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
                const size_t base = ((size_t)row * p.hq + head) * D + C::SW * wave + 4 * g;
#pragma unroll
                for (int n = 0; n < C::DTW; n++) {
                    const f32x4 v = st.o[nt][n] * inv;
                    if (p.out_f32) {
                        *(f32x4 *)((float *)p.out + base + 16 * n) = v;
                    } else {
                        *(u32x2 *)((uint16_t *)p.out + base + 16 * n) =
                            u32x2{pack2<true>(v.x, v.y), pack2<true>(v.z, v.w)};
                    }
                }
            } else {
                store_record<D, C::SW, KVT>(p, (size_t)rec * COLS + col, st.o[nt], st.m[nt], lt, wave);
            }
        }
        lo = seg_end;
        u++;
    }
    if constexpr (RO) {
#pragma unroll
        for (int m = 32; m >= 1; m >>= 1) fold ^= (uint32_t)__shfl_xor((int)fold, m, 64);
        if (lane == 0) ((uint32_t *)p.out)[wg * C::WAVES + wave] = fold;
        return;
    }
    if constexpr (!C::FP8) {
        if (fused) append_rows<D, KVT>(p, wg, gridDim.x);
    }
}

// ------------------------------------------------------------------ the prefill kernel
//
// Long query chunks (prefill, chunked prefill, prefix-cache hits) share each key across many
// rows, so the decode kernel's split over head_dim - every wave reading its own slice of K
// and V, 16-32 columns per workgroup - would re-read the K/V of a prefix once per 4 rows.
// Here a workgroup covers 128 columns ((row, query head) pairs of one KV head: 16 rows x 8
// heads at GQA 8) and each of its 4 waves owns two 16-column tiles over the full head_dim.
// Each K and V operand read from LDS then feeds two MFMAs: LDS reads are the kernel's largest
// single cost, and 4 x 32 at 2 waves per SIMD (199 VGPRs) beats 8 x 16 at 4 (measured 3 %
// on a mixed prefill step; 4 x 32 held to 3 waves per SIMD spills and is 8 % slower).  Every
// 32-token chunk of K and V is staged once in LDS with direct-to-LDS loads (spread over the
// waves) and read by all of them: K as the A operand of S^T = K Q^T (one
// 16-byte read per lane per 16 tokens x 32 dims; chunk positions XOR-swizzled by token so
// the 16 rows of a read hit distinct banks), V through transpose reads as the A operand of
// O^T += V^T P^T (swizzled so the 4 rows of a transpose read hit distinct banks).  Three
// stages with one barrier per chunk: the barrier both publishes chunk i and retires chunk
// i - 1, whose stage then receives chunk i + 2.  Work units, block ranges, the two key runs
// (cached keys, this step's keys), the fused append and the split records are the decode
// kernel's; records hold 128 columns.
template <int D>
struct WCfg {
    static constexpr int WAVES = 4;
    static constexpr int NTW = 2;               // 16-column tiles per wave
    static constexpr int THREADS = 64 * WAVES;
    static constexpr int COLS = 16 * NTW * WAVES;
    static constexpr int ROWB = 2 * D;          // bytes of one token's head (16-bit KV)
    static constexpr int CH = ROWB / 16;        // 16-byte chunks per token
    static constexpr int RPI = 1024 / ROWB;     // tokens per direct-to-LDS instruction
    static constexpr int NI = 32 / RPI;         // instructions per plane and chunk
    static constexpr int PER = (NI + WAVES - 1) / WAVES; // at most, per wave
    static constexpr int STAGE = 32 * D;        // 16-bit elements of one K or V stage
    static constexpr int KT = D / 32;           // k steps of S^T = K Q^T
    static constexpr int DT = D / 16;           // 16-dim tiles of O
};

// LDS chunk position of chunk c of token t: K rows are swizzled over all positions (the 16
// rows of an A-operand read), V rows over the 8 rows a transpose read serves per clock (32
// lanes: measured 1.4-1.6 clocks per wave instruction against 2.1 with a 4-row swizzle).
template <int D>
__device__ __forceinline__ uint32_t swz_k(uint32_t t) { return t & (WCfg<D>::CH - 1); }
template <int D>
__device__ __forceinline__ uint32_t swz_v(uint32_t t) {
    return D == 128 ? 2 * (t & 7) : 2 * ((t >> 1) & 1);
}

// Page data of a window of up to 64 logical pages for the wide kernel, one page per lane, so
// that a chunk's tile costs three v_readlane: lane i holds the byte offset of logical page
// base + i in its plane (64-bit) and the bytes of it that are live keys of the range (0 for a
// page wholly past the range end, and for a table entry outside the pool: no load is based
// outside the pool).
struct WideWindow {
    uint32_t base;          // first logical page covered (wave-uniform)
    uint32_t off_lo, off_hi; // per lane
    uint32_t bytes;         // per lane
    float ks, vs;           // per lane, FP8 pools: the page's K and V scales (1 for a dead page)
};

// The 16-token tile a load reads: its page's byte offset and live bytes (0: the loads move
// no data and return zeros).
struct WideTile {
    uint64_t off;
    uint32_t bytes;
};

__device__ __forceinline__ void wide_window(const AttnParams &p, WideWindow &w,
                                            const uint32_t *table, uint32_t first,
                                            uint32_t limit, uint32_t tlim, uint32_t row_bytes,
                                            uint32_t *page_out = nullptr) {
    const uint32_t shift = p.page_shift, P = 1u << shift;
    const uint32_t idx = first + lane_id();
    uint32_t page = idx;
    bool in_pool = true;
    if (table) {
        page = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(make_rsrc(table, limit * 4), (int)(idx * 4), 0, 0);
        in_pool = page < p.pool_pages;
    }
    const uint32_t pstart = idx << shift;
    const uint64_t off = (uint64_t)page * ((uint64_t)P * row_bytes);
    w.base = first;
    w.off_lo = (uint32_t)off;
    w.off_hi = (uint32_t)(off >> 32);
    w.bytes = in_pool && tlim > pstart ? min(tlim - pstart, P) * row_bytes : 0u;
    if (page_out) *page_out = page;
}

// The same with the page's FP8 scales of KV head hk.  A page without live keys (past the
// range, or a table entry outside the pool) takes scale 1: its scores are masked to -inf
// after the scaling, which a scale of 0 would turn into NaN.
__device__ __forceinline__ void wide_window_fp8(const AttnParams &p, WideWindow &w,
                                                const uint32_t *table, uint32_t first,
                                                uint32_t limit, uint32_t tlim, uint32_t row_bytes,
                                                uint32_t hk) {
    uint32_t page = 0;
    wide_window(p, w, table, first, limit, tlim, row_bytes, &page);
    const uint32_t sb = p.pool_pages * p.hkv * 4;
    const uint32_t at = w.bytes ? (page * p.hkv + hk) * 4 : sb; // past the end: reads 0
    const float ks = __builtin_bit_cast(float, (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(
                                                   make_rsrc(p.k_scales, sb), (int)at, 0, 0));
    const float vs = __builtin_bit_cast(float, (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(
                                                   make_rsrc(p.v_scales, sb), (int)at, 0, 0));
    w.ks = w.bytes ? ks : 1.0f;
    w.vs = w.bytes ? vs : 1.0f;
}

// Tile at key t0 of a window whose range ends at tlim (t0 past it: no live keys; before it
// the tile's page lies inside the window).
__device__ __forceinline__ WideTile wide_tile(const WideWindow &w, uint32_t t0, uint32_t shift,
                                              uint32_t tlim) {
    const int rel = (int)(((t0 >> shift) - w.base) & 63);
    WideTile r;
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)w.off_lo, rel);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)w.off_hi, rel);
    r.off = ((uint64_t)hi << 32) | lo;
    r.bytes = t0 < tlim ? (uint32_t)__builtin_amdgcn_readlane((int)w.bytes, rel) : 0u;
    return r;
}

// The tile of chunk t that this wave's k-th load reads (each load reads RPI consecutive
// tokens of one 16-token tile).
template <int D>
__device__ __forceinline__ uint32_t wide_tile_key(uint32_t t, uint32_t wave, int k) {
    return t + 16 * (((wave + k * WCfg<D>::WAVES) * WCfg<D>::RPI) / 16);
}

// Per-lane byte offsets of this wave's direct-to-LDS loads within the 16-token tile each load
// reads (constant over a range: the tile's position in its page goes into the scalar base).
template <int D>
struct WideLanes {
    uint32_t k[WCfg<D>::PER], v[WCfg<D>::PER];
};

template <int D>
__device__ __forceinline__ WideLanes<D> wide_lanes(uint32_t wave, uint32_t hk, uint32_t row_bytes) {
    using W = WCfg<D>;
    const uint32_t lane = lane_id();
    WideLanes<D> r;
#pragma unroll
    for (int k = 0; k < W::PER; k++) {
        const uint32_t q = wave + k * W::WAVES;            // instruction: tokens q*RPI .. +RPI-1
        const uint32_t tl = q * W::RPI + lane / W::CH;      // token within the chunk
        const uint32_t tt = (q * W::RPI) % 16 + lane / W::CH; // token within its 16-token tile
        const uint32_t pos = lane % W::CH;
        const uint32_t rowoff = tt * row_bytes + hk * W::ROWB;
        r.k[k] = rowoff + (pos ^ swz_k<D>(tl)) * 16;
        r.v[k] = rowoff + (pos ^ swz_v<D>(tl)) * 16;
    }
    return r;
}

// This wave's quarter of chunk t of K and V (from the pool or the step's rows) into LDS, from
// the wave's tile (wide_tile_key).  The tile's first token lies (ts mod P) tokens into its
// page: the descriptor starts there and keeps the page's remaining live bytes, so the lane
// offsets stay constant and the per-chunk address arithmetic is scalar.
template <int D>
__device__ __forceinline__ void wide_load(const AttnParams &p, uint32_t t,
                                          const WideTile (&tile)[WCfg<D>::PER], const uint8_t *kbase,
                                          const uint8_t *vbase, const WideLanes<D> &ln, uint32_t wave,
                                          uint16_t *kst, uint16_t *vst) {
    using W = WCfg<D>;
    const uint32_t P = 1u << p.page_shift;
    const uint32_t row_bytes = p.hkv * W::ROWB;
    __builtin_amdgcn_s_waitcnt(0xC07F); // lgkmcnt(0): this wave's reads of the stage are done
#pragma unroll
    for (int k = 0; k < W::PER; k++) {
        const uint32_t q = wave + k * W::WAVES;        // instruction: tokens q*RPI .. +RPI-1
        if (W::NI % W::WAVES == 0 || q < W::NI) {      // waves past the last instruction load nothing
            const uint32_t sh = (wide_tile_key<D>(t, wave, k) & (P - 1)) * row_bytes;
            // a tile with live bytes starts before the range end, so they exceed sh
            const uint32_t nb = tile[k].bytes ? tile[k].bytes - sh : 0u;
            const __amdgpu_buffer_rsrc_t rk = make_rsrc(kbase + tile[k].off + sh, nb);
            const __amdgpu_buffer_rsrc_t rv = make_rsrc(vbase + tile[k].off + sh, nb);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rk, (__attribute__((address_space(3))) void *)(kst + q * 512), 16, (int)ln.k[k], 0, 0, 0);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rv, (__attribute__((address_space(3))) void *)(vst + q * 512), 16, (int)ln.v[k], 0, 0, 0);
        }
    }
    __builtin_amdgcn_sched_barrier(0);
}

// The tiles of chunk t that this wave's loads read.
template <int D>
__device__ __forceinline__ void wide_tiles(const WideWindow &w, uint32_t t, uint32_t wave,
                                           uint32_t shift, uint32_t tlim,
                                           WideTile (&out)[WCfg<D>::PER]) {
#pragma unroll
    for (int k = 0; k < WCfg<D>::PER; k++) out[k] = wide_tile(w, wide_tile_key<D>(t, wave, k), shift, tlim);
}

// FP8 pools: each lane's share of a chunk comes through registers instead of direct-to-LDS
// loads.  The staged stages keep the 16-bit layout (the same swizzles, the same operand reads
// and f16 MFMAs): lane L of the wave's k-th share fills LDS slot L of that share's 1 KB, the 16
// bytes of f16 dims [8c, 8c + 8) of its token with c its swizzled chunk, from the 8 FP8 bytes
// [8c, 8c + 8) of the token's head row, converted exactly to f16 by the hardware conversion
// (every e4m3 code is an f16 value; the scales are applied to the scores and to the weights).
template <int D>
__device__ __forceinline__ WideLanes<D> wide_lanes_fp8(uint32_t wave, uint32_t hk, uint32_t row_bytes) {
    using W = WCfg<D>;
    const uint32_t lane = lane_id();
    WideLanes<D> r;
#pragma unroll
    for (int k = 0; k < W::PER; k++) {
        const uint32_t q = wave + k * W::WAVES;
        const uint32_t tl = q * W::RPI + lane / W::CH;
        const uint32_t tt = (q * W::RPI) % 16 + lane / W::CH;
        const uint32_t pos = lane % W::CH;
        const uint32_t rowoff = tt * row_bytes + hk * D;
        r.k[k] = rowoff + (pos ^ swz_k<D>(tl)) * 8;
        r.v[k] = rowoff + (pos ^ swz_v<D>(tl)) * 8;
    }
    return r;
}

// Eight e4m3 bytes (byte i of the pair's dwords in order) -> eight f16, exactly.
__device__ __forceinline__ u32x4 e4m3x8_to_f16x8(u32x2 w) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    const h2 a = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w.x, 1.0f, false);
    const h2 b = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w.x, 1.0f, true);
    const h2 c = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w.y, 1.0f, false);
    const h2 d = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w.y, 1.0f, true);
    return u32x4{__builtin_bit_cast(uint32_t, a), __builtin_bit_cast(uint32_t, b),
                 __builtin_bit_cast(uint32_t, c), __builtin_bit_cast(uint32_t, d)};
}

template <int D>
struct Fp8Share {
    u32x2 k[WCfg<D>::PER], v[WCfg<D>::PER];
};

// Issue this wave's FP8 loads of chunk t (the tiles as wide_load takes them).
template <int D>
__device__ __forceinline__ void wide_issue_fp8(const AttnParams &p, uint32_t t,
                                               const WideTile (&tile)[WCfg<D>::PER],
                                               const uint8_t *kbase, const uint8_t *vbase,
                                               const WideLanes<D> &ln, uint32_t wave,
                                               Fp8Share<D> &r) {
    using W = WCfg<D>;
    const uint32_t P = 1u << p.page_shift;
    const uint32_t row_bytes = p.hkv * D;
#pragma unroll
    for (int k = 0; k < W::PER; k++) {
        const uint32_t q = wave + k * W::WAVES;
        if (W::NI % W::WAVES == 0 || q < W::NI) {
            const uint32_t sh = (wide_tile_key<D>(t, wave, k) & (P - 1)) * row_bytes;
            const uint32_t nb = tile[k].bytes ? tile[k].bytes - sh : 0u;
            r.k[k] = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(
                                                   make_rsrc(kbase + tile[k].off + sh, nb), (int)ln.k[k], 0, 0));
            r.v[k] = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(
                                                   make_rsrc(vbase + tile[k].off + sh, nb), (int)ln.v[k], 0, 0));
        }
    }
}

// Convert the loaded share and write it into the stage (after the loads have landed).
template <int D>
__device__ __forceinline__ void wide_commit_fp8(const Fp8Share<D> &r, uint32_t wave, uint16_t *kst,
                                                uint16_t *vst) {
    using W = WCfg<D>;
    const uint32_t lane = lane_id();
#pragma unroll
    for (int k = 0; k < W::PER; k++) {
        const uint32_t q = wave + k * W::WAVES;
        if (W::NI % W::WAVES == 0 || q < W::NI) {
            *(u32x4 *)(kst + q * 512 + lane * 8) = e4m3x8_to_f16x8(r.k[k]);
            *(u32x4 *)(vst + q * 512 + lane * 8) = e4m3x8_to_f16x8(r.v[k]);
        }
    }
}

template <int D>
constexpr int kWideLoads = 2 * WCfg<D>::PER; // memory operations of one wide_load

template <int D, int KVT>
struct WState {
    u32x4 qr[WCfg<D>::NTW][WCfg<D>::KT]; // Q^T operands of the wave's column tiles
    uint32_t lo, lim[WCfg<D>::NTW];
    // per column: reference maximum of the scaled scores in the log2 domain (0 before the
    // first live key) and the exponent above which it is raised (-inf before the first live
    // key, then 2^8)
    float m[WCfg<D>::NTW], thr[WCfg<D>::NTW];
    f32x4 l[WCfg<D>::NTW];               // the mass, every row of the tile (MFMA against ones)
    f32x4 o[WCfg<D>::NTW][WCfg<D>::DT];
};

// Full-head_dim query operand of one 16-column tile: lane (g, col) holds q[col][32ks + 8g .. +7].
template <int D, int KVT>
__device__ __forceinline__ void load_q_full(const AttnParams &p, uint32_t row, uint32_t head,
                                            bool valid, u32x4 (&qr)[WCfg<D>::KT]) {
    constexpr bool MB = KVT == LIA_BF16;
    const uint32_t g = lane_id() >> 4;
    const uint32_t qb = p.q_f32 ? 4 : 2;
    const __amdgpu_buffer_rsrc_t r = make_rsrc(p.q, p.n_rows * p.hq * D * qb);
#pragma unroll
    for (int ks = 0; ks < WCfg<D>::KT; ks++) {
        const uint32_t at = (row * p.hq + head) * D + 32 * ks + 8 * g;
        const uint32_t off = valid ? at * qb : 0x80000000u;
        float x[8];
        if (p.q_f32) {
            const f32x4 a = __builtin_bit_cast(f32x4, buffer_load16(r, off));
            const f32x4 b = __builtin_bit_cast(f32x4, buffer_load16(r, off + 16));
            x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
            x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
        } else {
            const u32x4 w = buffer_load16(r, off);
            if constexpr (MB) {
                qr[ks] = w;
                continue;
            }
#pragma unroll
            for (int e = 0; e < 4; e++) {
                x[2 * e] = bf16_to_f32(w[e] & 0xffffu);
                x[2 * e + 1] = bf16_to_f32(w[e] >> 16);
            }
        }
        qr[ks] = u32x4{pack2<MB>(x[0], x[1]), pack2<MB>(x[2], x[3]), pack2<MB>(x[4], x[5]),
                       pack2<MB>(x[6], x[7])};
    }
}

// One chunk (32 tokens at t) for this wave's 16 * NTW columns, from stages kst / vst.  `masked`: some
// key of the chunk is outside some column's live range (the range's unaligned start, the
// causal diagonal, the range end); only then are the scores masked, in a branch of their
// own.  Otherwise every key is live for every valid column (padding columns attend zero
// queries and are never written out).
//
// Online softmax in the log2 domain with a lazily raised reference m per column: the
// exponent of a score s is e = s * scale_log2 - m (one fma), and the reference is raised only
// when some lane of the wave holds an e above its column's threshold - 2^8 once the column
// has a live key, any live key before - so the exponentials stay <= 2^8.  Only then does the
// wave reduce the maxima across lanes and rescale O and the mass.  The mass is accumulated by
// the matrix unit: an MFMA of a ones operand against P^T sums each column over the chunk's
// keys, with the same rounded weights as O.
//
// FP8 pools: the staged values are the codes' values in f16; ksc[j] (the score scale times the
// K scale of tile j's page) scales the scores of tile j, and vsc[j] (its V scale) its weights for
// P.V, while the mass sums the unscaled weights.
template <int D, int KVT>
__device__ __forceinline__ void wide_compute(const AttnParams &p, uint32_t t, WState<D, KVT> &st,
                                             const uint16_t *kst, const uint16_t *vst, bool masked,
                                             const float (&ksc)[2], const float (&vsc)[2]) {
    constexpr bool FP8 = KVT == LIA_FP8_E4M3;
    using W = WCfg<D>;
    constexpr bool MB = KVT == LIA_BF16;
    const uint32_t lane = lane_id(), g = lane >> 4, li = lane & 15;
    // S^T tiles: tokens 16j + (rows), columns 16nt + li
    constexpr int NTW = W::NTW;
    // LDS byte offsets of the operand reads.  K: token row 16j + li, 16-byte chunk 4ks + g at
    // position (4ks + g) ^ s, s = li % chunks-per-row (the staging swizzle) - i.e. kb ^ 64 ks
    // with the row and the ks-independent bits in kb (row 16 + li swizzles like row li).  The
    // XOR form keeps one address register per operand and the stage base an immediate.
    const uint32_t sk = swz_k<D>(li);
    const uint32_t kb = li * 2 * D + 64 * (sk >> 2) + 16 * (g ^ (sk & 3));
    // every operand of the chunk is read from LDS at its start (K first, then V), so the
    // reads' latency passes under the S^T MFMAs and the softmax instead of stalling the wave
    auto kread = [&](int i) { // i = 2 ks + j: the two token tiles' chains alternate
        return *(const u32x4 *)((const uint8_t *)kst + (kb ^ (64 * (i / 2))) + (i % 2) * 32 * D);
    };
    // O^T += V^T P^T: V^T rows 16n .. 16n+15, k slots = tokens {4g..4g+3, 16+4g..16+4g+3}.
    // The transpose read of row r0 = 4g + li/4, chunk 2n + b at position (2n + b) ^ swz_v(r0),
    // is at vb ^ 32 n (row r0 + 16 swizzles like r0).
    const uint32_t r0 = 4 * g + li / 4;
    const uint32_t vb = r0 * 2 * D + 16 * ((li & 3) >> 1) + 8 * (li & 1) + 16 * swz_v<D>(r0);
    auto vread = [&](int n) {
        const uint8_t *a0p = (const uint8_t *)vst + (vb ^ (32 * n));
        const uint8_t *a1p = a0p + 32 * D; // row r0 + 16
        const s16x4 a0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4 *)(a0p));
        const s16x4 a1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4 *)(a1p));
        const u32x2 b0 = __builtin_bit_cast(u32x2, a0), b1 = __builtin_bit_cast(u32x2, a1);
        return u32x4{b0.x, b0.y, b1.x, b1.y};
    };
    u32x4 ka[2 * W::KT], vt[W::DT];
#pragma unroll
    for (int i = 0; i < 2 * W::KT; i++) ka[i] = kread(i);
#pragma unroll
    for (int n = 0; n < W::DT; n++) vt[n] = vread(n);
    f32x4 acc[2][NTW];
#pragma unroll
    for (int j = 0; j < 2; j++)
#pragma unroll
        for (int nt = 0; nt < NTW; nt++) acc[j][nt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int i = 0; i < 2 * W::KT; i++) {
        const int j = i % 2, ks = i / 2;
#pragma unroll
        for (int nt = 0; nt < NTW; nt++) acc[j][nt] = mfma16x16x32<MB>(ka[i], st.qr[nt][ks], acc[j][nt]);
    }
    if (masked) {
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int nt = 0; nt < NTW; nt++)
#pragma unroll
                for (int i = 0; i < 4; i++)
                    if (t + 16 * j + 4 * g + i - st.lo >= st.lim[nt]) acc[j][nt][i] = -INFINITY;
    }
    u32x4 pb[NTW], pv[NTW]; // weights (the mass), and for FP8 pools the V-scaled ones (P.V)
#pragma unroll
    for (int nt = 0; nt < NTW; nt++) {
        float e[2][4];
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int i = 0; i < 4; i++)
                e[j][i] = __builtin_fmaf(acc[j][nt][i], FP8 ? ksc[j] : p.scale_log2, -st.m[nt]);
        float mx = fmaxf(fmaxf(fmaxf(e[0][0], e[0][1]), fmaxf(e[0][2], e[0][3])),
                         fmaxf(fmaxf(e[1][0], e[1][1]), fmaxf(e[1][2], e[1][3])));
        if (__builtin_amdgcn_ballot_w64(mx > st.thr[nt])) { // wave-uniform: rare after the first chunk
            mx = rows_max(mx);
            if (mx > st.thr[nt]) { // the same in the 4 lanes of the column
                const float factor = fast_exp2(-mx); // 0 before the column's first live key
                st.l[nt] *= factor;
#pragma unroll
                for (int n = 0; n < W::DT; n++) st.o[nt][n] *= factor;
                st.m[nt] += mx;
                st.thr[nt] = 8.0f;
#pragma unroll
                for (int j = 0; j < 2; j++)
#pragma unroll
                    for (int i = 0; i < 4; i++) e[j][i] -= mx;
            }
        }
        float pr[2][4];
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int i = 0; i < 4; i++) pr[j][i] = fast_exp2(e[j][i]);
        pb[nt] = u32x4{pack2<MB>(pr[0][0], pr[0][1]), pack2<MB>(pr[0][2], pr[0][3]),
                       pack2<MB>(pr[1][0], pr[1][1]), pack2<MB>(pr[1][2], pr[1][3])};
        if constexpr (FP8) {
#pragma unroll
            for (int j = 0; j < 2; j++)
#pragma unroll
                for (int i = 0; i < 4; i++) pr[j][i] *= vsc[j];
            pv[nt] = u32x4{pack2<MB>(pr[0][0], pr[0][1]), pack2<MB>(pr[0][2], pr[0][3]),
                           pack2<MB>(pr[1][0], pr[1][1]), pack2<MB>(pr[1][2], pr[1][3])};
        }
    }
#pragma unroll
    for (int n = 0; n < W::DT; n++)
#pragma unroll
        for (int nt = 0; nt < NTW; nt++)
            st.o[nt][n] = mfma16x16x32<MB>(vt[n], FP8 ? pv[nt] : pb[nt], st.o[nt][n]);
    // the mass: every row of the ones tile is the column's sum of this chunk's weights
    constexpr uint32_t one2 = MB ? 0x3F803F80u : 0x3C003C00u;
    const u32x4 ones = u32x4{one2, one2, one2, one2};
#pragma unroll
    for (int nt = 0; nt < NTW; nt++) st.l[nt] = mfma16x16x32<MB>(ones, pb[nt], st.l[nt]);
}

// One step: wait for chunk i (this wave's loads; the next chunk's loads stay in flight),
// the barrier, the loads of chunk i + 2 into the stage chunk i - 1 used, then chunk i.
// Restrict stages: the compiler may keep the new loads in flight across the reads.
// Three stages (measured: four are 1 % slower on a mixed prefill step).
constexpr int kWideStages = 3;

// Chunk t needs the causal / range mask unless [t, t + 32) lies in [free_lo, free_hi), the
// keys live for every valid column of the unit.
template <int D, int KVT>
__device__ __forceinline__ void wide_step(const AttnParams &p, uint32_t tn,
                                          const WideTile (&tpn)[WCfg<D>::PER],
                                          uint16_t *__restrict__ kn, uint16_t *__restrict__ vn,
                                          uint32_t tc, const uint16_t *__restrict__ kc,
                                          const uint16_t *__restrict__ vc, const uint8_t *kbase,
                                          const uint8_t *vbase, const WideLanes<D> &ln, uint32_t wave,
                                          bool active, WState<D, KVT> &st, uint32_t free_lo,
                                          uint32_t free_hi) {
    wait_vmcnt<(kWideStages - 2) * kWideLoads<D>>(); // the later chunks' loads stay in flight
    lds_barrier();
    wide_load<D>(p, tn, tpn, kbase, vbase, ln, wave, kn, vn);
    const float one[2] = {1.0f, 1.0f};
    if (active) wide_compute<D, KVT>(p, tc, st, kc, vc, !(tc >= free_lo && tc + 32 <= free_hi), one, one);
}

// Keys [s_lo, s_hi) of one source into the running state (windows of at most 64 pages), through
// a ring of kWideStages LDS stages (st_k / st_v).
template <int D, int KVT>
__device__ __forceinline__ void wide_range(const AttnParams &p, const uint8_t *kbase,
                                           const uint8_t *vbase, const uint32_t *table,
                                           uint32_t s_lo, uint32_t s_hi, bool use_pre, uint4 pre,
                                           uint32_t hk, uint32_t wave, bool active,
                                           WState<D, KVT> &st, uint16_t *const (&st_k)[4],
                                           uint16_t *const (&st_v)[4], uint32_t free_lo,
                                           uint32_t free_hi) {
    constexpr int NS = kWideStages;
    const uint32_t shift = p.page_shift;
    const uint32_t page_limit = (s_hi + (1u << shift) - 1) >> shift;
    const uint32_t row_bytes = p.hkv * WCfg<D>::ROWB;
    using W = WCfg<D>;
    const WideLanes<D> ln = wide_lanes<D>(wave, hk, row_bytes);
    // wave-uniform bases, so the descriptors are built by scalar instructions
    kbase = uniform_ptr(kbase);
    vbase = uniform_ptr(vbase);
    for (uint32_t wbeg = s_lo & ~31u; wbeg < s_hi;) {
        const uint32_t wend = min(s_hi, ((wbeg >> shift) + 64) << shift);
        WideWindow win;
        wide_window(p, win, table, wbeg >> shift, page_limit, wend, row_bytes);
        WideTile tp[NS - 1][W::PER], tpn[W::PER];
        // the first two chunks from the plan's first pages when it preloaded them (no wait for
        // the table load; they cover the kPrePages pages of two chunks at the smallest page size)
#pragma unroll
        for (int c = 0; c < NS - 1; c++) {
            if (use_pre && c < 2) {
                const uint64_t pb = (uint64_t)(1u << shift) * row_bytes;
#pragma unroll
                for (int k = 0; k < W::PER; k++) {
                    const uint32_t key = wide_tile_key<D>(wbeg + 32 * c, wave, k);
                    const TilePages a = tile_pages_pre(pre, wbeg >> shift, key, shift, wend, p.pool_pages);
                    // no live bytes for a tile at or past the range end (wide_load relies on it)
                    tp[c][k] = WideTile{a.page[0] * pb, key < wend ? a.live[0] * row_bytes : 0u};
                }
            } else {
                wide_tiles<D>(win, wbeg + 32 * c, wave, shift, wend, tp[c]);
            }
        }
        use_pre = false;
        // every wave finished the previous window's chunks before their stages are refilled
        lds_barrier();
#pragma unroll
        for (int c = 0; c < NS - 1; c++) wide_load<D>(p, wbeg + 32 * c, tp[c], kbase, vbase, ln, wave, st_k[c], st_v[c]);
        for (uint32_t t = wbeg;; t += 32 * NS) {
            // loads past wend carry no traffic
#pragma unroll
            for (int c = 0; c < NS; c++) {
                const uint32_t tn = t + 32 * (c + NS - 1);
                wide_tiles<D>(win, tn, wave, shift, wend, tpn);
                wide_step<D, KVT>(p, tn, tpn, st_k[(c + NS - 1) % NS], st_v[(c + NS - 1) % NS],
                                  t + 32 * c, st_k[c], st_v[c], kbase, vbase, ln, wave, active, st,
                                  free_lo, free_hi);
                if (t + 32 * (c + 1) >= wend) goto window_done;
            }
        }
    window_done:
        wait_vmcnt<0>(); // the trailing (empty) loads target stages about to be reused
        wbeg = wend;
    }
}

// Keys [s_lo, s_hi) of an FP8 pool into the running state.  A chunk's FP8 bytes are loaded into
// registers one step before they are converted into its stage, right after the barrier that
// retires the stage's previous chunk, and the next barrier publishes them: one chunk is computed
// while the next is converted and the one after is loaded.
template <int D>
__device__ __forceinline__ void wide_range_fp8(const AttnParams &p, const uint8_t *kbase,
                                               const uint8_t *vbase, const uint32_t *table,
                                               uint32_t s_lo, uint32_t s_hi, uint32_t hk,
                                               uint32_t wave, bool active,
                                               WState<D, LIA_FP8_E4M3> &st,
                                               uint16_t *const (&st_k)[4],
                                               uint16_t *const (&st_v)[4], uint32_t free_lo,
                                               uint32_t free_hi) {
    constexpr int NS = kWideStages;
    using W = WCfg<D>;
    const uint32_t shift = p.page_shift;
    const uint32_t page_limit = (s_hi + (1u << shift) - 1) >> shift;
    const uint32_t row_bytes = p.hkv * D; // one byte per element
    const WideLanes<D> ln = wide_lanes_fp8<D>(wave, hk, row_bytes);
    kbase = uniform_ptr(kbase);
    vbase = uniform_ptr(vbase);
    const float sl = p.scale_log2;
    for (uint32_t wbeg = s_lo & ~31u; wbeg < s_hi;) {
        const uint32_t wend = min(s_hi, ((wbeg >> shift) + 64) << shift);
        WideWindow win;
        wide_window_fp8(p, win, table, wbeg >> shift, page_limit, wend, row_bytes, hk);
        WideTile tp[W::PER];
        Fp8Share<D> r;
        // every wave finished the previous window's chunks before their stages are refilled
        lds_barrier();
        wide_tiles<D>(win, wbeg, wave, shift, wend, tp);
        wide_issue_fp8<D>(p, wbeg, tp, kbase, vbase, ln, wave, r);
        wait_vmcnt<0>();
        wide_commit_fp8<D>(r, wave, st_k[0], st_v[0]);
        wide_tiles<D>(win, wbeg + 32, wave, shift, wend, tp);
        wide_issue_fp8<D>(p, wbeg + 32, tp, kbase, vbase, ln, wave, r);
        for (uint32_t t = wbeg;; t += 32 * NS) {
#pragma unroll
            for (int c = 0; c < NS; c++) {
                const uint32_t tc = t + 32 * c;
                lds_barrier(); // chunk tc is in its stage; chunk tc - 32 is retired
                wait_vmcnt<0>();
                wide_commit_fp8<D>(r, wave, st_k[(c + 1) % NS], st_v[(c + 1) % NS]); // chunk tc + 32
                wide_tiles<D>(win, tc + 64, wave, shift, wend, tp);
                wide_issue_fp8<D>(p, tc + 64, tp, kbase, vbase, ln, wave, r);
                if (active) {
                    float ksc[2], vsc[2];
#pragma unroll
                    for (int j = 0; j < 2; j++) {
                        const int rel = (int)((((tc + 16 * j) >> shift) - win.base) & 63);
                        ksc[j] = sl * __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, win.ks), rel));
                        vsc[j] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, win.vs), rel));
                    }
                    wide_compute<D, LIA_FP8_E4M3>(p, tc, st, st_k[c], st_v[c],
                                                  !(tc >= free_lo && tc + 32 <= free_hi), ksc, vsc);
                }
                if (tc + 32 >= wend) goto window_done;
            }
        }
    window_done:
        wait_vmcnt<0>(); // the trailing (empty) loads
        wbeg = wend;
    }
}

template <int D, int KVT>
__global__ __launch_bounds__(WCfg<D>::THREADS, 2) void wide_kernel(AttnParams p) {
    using W = WCfg<D>;
    constexpr uint32_t COLS = W::COLS;
    // one object per stage, so that the compiler sees a stage's reads and the loads in flight
    // into the other stages as independent (with one array and variable offsets into it, it
    // waits for every load before each read)
    static_assert(kWideStages == 3 || kWideStages == 4, "three or four stages");
    constexpr int S4 = kWideStages == 4 ? W::STAGE : 1;
    __shared__ __attribute__((aligned(16))) uint16_t k0[W::STAGE], k1[W::STAGE], k2[W::STAGE], k3[S4];
    __shared__ __attribute__((aligned(16))) uint16_t v0[W::STAGE], v1[W::STAGE], v2[W::STAGE], v3[S4];
    uint16_t *const st_k[4] = {k0, k1, k2, k3}, *const st_v[4] = {v0, v1, v2, v3};
    const uint32_t wg = blockIdx.x;
    const WorkDesc wd = p.work[wg];
    const uint32_t tid = threadIdx.x, lane = tid & 63;
    const uint32_t wave = (uint32_t)__builtin_amdgcn_readfirstlane((int)(tid >> 6));
    const uint32_t g = lane >> 4, li = lane & 15;
    uint32_t u = wd.unit, lo = wd.lo;
    const uint32_t hi = wd.hi;
    const bool fused = p.newk != nullptr;
    const uint32_t row_bytes = p.hkv * W::ROWB;
    bool first = true;
    // the plan guarantees a unit covers every block of a non-empty range
    while (lo < hi) {
        UnitDesc ud;
        if (first) ud = wd.first;
        else ud = p.units[u];
        const bool use_pre = first && (wd.flags & 1);
        first = false;
        const uint32_t bs = ud.block_start, uend = bs + ud.nblocks;
        if (uend <= lo) { u++; continue; }
        const uint32_t seg_end = min(hi, uend);
        const uint32_t hk = unit_head(ud), nrows = unit_rows(ud);
        const uint32_t *table = p.pages + (size_t)ud.table_row * p.stride;
        const uint32_t kend = ud.kend, kcache = ud.kcache, cb = ud.cblocks;
        const uint32_t pos0 = kend - nrows;
        const uint32_t ncols = nrows * p.group;
        constexpr int NTW = W::NTW;
        const bool active = 16 * NTW * wave < ncols; // waves without valid columns only load

        WState<D, KVT> st;
        uint32_t climit[NTW];
#pragma unroll
        for (int nt = 0; nt < NTW; nt++) {
            const uint32_t col = 16 * NTW * wave + 16 * nt + li;
            const bool valid = col < ncols;
            const uint32_t ri = valid ? col / p.group : 0;
            climit[nt] = valid ? pos0 + ri + 1 : 0;
            load_q_full<D, KVT>(p, ud.rowbeg + ri, hk * p.group + col % p.group, valid, st.qr[nt]);
            st.m[nt] = 0.0f;
            st.thr[nt] = -INFINITY;
            st.l[nt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int n = 0; n < W::DT; n++) st.o[nt][n] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        }
        const uint32_t a = lo - bs, e = seg_end - bs;
        auto key_of = [&](uint32_t i) { return i < cb ? 32 * i : min(kcache + 32 * (i - cb), kend); };
        // per column the live keys of [r_lo, r_hi); keys [r_lo, free_hi) are live for every
        // valid column (those of the unit's first row, whose causal limit is the lowest)
        uint32_t free_hi = 0;
        auto set_limits = [&](uint32_t r_lo, uint32_t r_hi, uint32_t origin) {
            st.lo = r_lo;
#pragma unroll
            for (int nt = 0; nt < NTW; nt++) {
                const int w = (int)min(climit[nt] - origin, r_hi) - (int)r_lo;
                st.lim[nt] = climit[nt] && w > 0 ? (uint32_t)w : 0u;
            }
            const int w0 = (int)min(pos0 + 1 - origin, r_hi) - (int)r_lo;
            free_hi = r_lo + (w0 > 0 ? (uint32_t)w0 : 0u);
        };
        const uint8_t *kpool = (const uint8_t *)p.kc, *vpool = (const uint8_t *)p.vc;
        if constexpr (KVT == LIA_FP8_E4M3) {
            // FP8 pools: the step's rows are appended by a launch of their own first
            const uint32_t r_lo = key_of(a), r_hi = min(key_of(e), kend);
            set_limits(r_lo, r_hi, 0);
            wide_range_fp8<D>(p, kpool, vpool, table, r_lo, r_hi, hk, wave, active, st, st_k, st_v,
                              r_lo, free_hi);
        } else if (!fused) {
            const uint32_t r_lo = key_of(a), r_hi = min(key_of(e), kend);
            set_limits(r_lo, r_hi, 0);
            wide_range<D, KVT>(p, kpool, vpool, table, r_lo, r_hi, use_pre, wd.pre, hk, wave, active,
                               st, st_k, st_v, r_lo, free_hi);
        } else {
            if (a < cb) {
                const uint32_t r_lo = 32 * a, r_hi = min(32 * min(e, cb), kcache);
                set_limits(r_lo, r_hi, 0);
                wide_range<D, KVT>(p, kpool, vpool, table, r_lo, r_hi, use_pre, wd.pre, hk, wave,
                                   active, st, st_k, st_v, r_lo, free_hi);
            }
            if (e > cb) {
                const uint32_t r0 = ud.rowbeg - (pos0 - kcache);
                const uint32_t r_lo = 32 * (max(a, cb) - cb), r_hi = min(32 * (e - cb), kend - kcache);
                set_limits(r_lo, r_hi, kcache);
                wide_range<D, KVT>(p, (const uint8_t *)p.newk + (size_t)r0 * row_bytes,
                                   (const uint8_t *)p.newv + (size_t)r0 * row_bytes, nullptr, r_lo,
                                   r_hi, false, wd.pre, hk, wave, active, st, st_k, st_v,
                                   r_lo, free_hi);
            }
        }

        const bool whole = lo == bs && seg_end == uend;
        const uint32_t rec = (wd.flags >> 8) + u;
#pragma unroll
        for (int nt = 0; nt < NTW; nt++) {
            const float lt = st.l[nt][0];
            const uint32_t col = 16 * NTW * wave + 16 * nt + li;
            if (col >= ncols) continue;
            const uint32_t row = ud.rowbeg + col / p.group;
            const uint32_t head = hk * p.group + col % p.group;
            if (whole) {
                const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
                const size_t base = ((size_t)row * p.hq + head) * D + 4 * g;
#pragma unroll
                for (int n = 0; n < W::DT; n++) {
                    const f32x4 v = st.o[nt][n] * inv;
                    if (p.out_f32) {
                        *(f32x4 *)((float *)p.out + base + 16 * n) = v;
                    } else {
                        *(u32x2 *)((uint16_t *)p.out + base + 16 * n) =
                            u32x2{pack2<true>(v.x, v.y), pack2<true>(v.z, v.w)};
                    }
                }
            } else {
                // split record: O normalised by its own mass, in the pool's 16-bit type for a
                // 16-bit output (relative error 2^-11 in f16, 2^-9 in bf16, the rounding of a
                // bf16 output; half the record traffic of f32) or in f32 for an f32 output,
                // with the mass and maximum in f32
                const size_t rb = (size_t)rec * COLS + col;
                const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
                if (p.out_f32 || KVT == LIA_FP8_E4M3) { // the combine reads f32 rows for both
                    float *po = p.part_o + rb * D + 4 * g;
#pragma unroll
                    for (int n = 0; n < W::DT; n++) *(f32x4 *)(po + 16 * n) = st.o[nt][n] * inv;
                } else {
                    uint16_t *po = (uint16_t *)p.part_o + rb * D + 4 * g;
#pragma unroll
                    for (int n = 0; n < W::DT; n++) *(u32x2 *)(po + 16 * n) = record_pack<KVT>(st.o[nt][n] * inv);
                }
                if (g == 0) {
                    p.part_ml[rb * 2] = st.m[nt];
                    p.part_ml[rb * 2 + 1] = lt;
                }
            }
        }
        lo = seg_end;
        u++;
    }
    if (fused) append_rows<D, KVT>(p, wg, gridDim.x);
}

// Merge the partial records of every unit that was split across workgroups.  Weights
// follow the reference merge: a record with zero mass contributes nothing, the others
// are scaled by 2^(m_r - M) (m in the log2 domain here), out = sum w o / sum w l
// (src/gpu/kernels/llama.rs:201-290).  One workgroup per (unit, column), or per half of its
// row (SPLIT = 2, blockIdx.z): D/4/SPLIT lanes cover the workgroup's share of a record's row
// as float4 quads, so 256 threads hold 1024*SPLIT/D records per pass, and a batch of
// kCombinePasses passes is loaded at once (every load independent of the weights).  Each
// thread merges its records against its own running reference maximum; the record groups
// sharing a quad are then merged pairwise (max, rescale both, add) by lane shuffles within
// a wave and through LDS across the waves, with one barrier.
constexpr uint32_t kCombineThreads = 256;
constexpr uint32_t kCombinePasses = 8;
constexpr uint32_t kCombineWaveCols = kCombineThreads / 64;
// Units expected to hold at most this many records merge one column per wave.
constexpr uint32_t kWaveColRecords = 16;
constexpr uint32_t kWideNTDev = 8; // 16-column tiles of a prefill unit

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, shfl_xor(v, m));
    return v;
}

// REC: record rows in f32 unnormalised (0), or normalised in f16 (1) or bf16 (2).
template <int D, int NT, int SPLIT, int REC>
__global__ __launch_bounds__(kCombineThreads) void combine_kernel(AttnParams p) {
    // SPLIT = 0: one wave per column (kCombineWaveCols columns per workgroup), for units with
    // few records: no LDS and no barrier
    constexpr bool WC = SPLIT == 0;
    constexpr uint32_t QF = D / 4;                 // float4 quads per record row
    constexpr uint32_t Q = QF / (WC ? 1 : SPLIT);  // quads of this workgroup's share (blockIdx.z)
    const uint32_t qoff = WC ? 0 : blockIdx.z * Q;
    constexpr uint32_t TPC = WC ? 64 : kCombineThreads; // threads per column
    constexpr uint32_t RPP = TPC / Q;              // records per pass
    constexpr uint32_t COLS = 16 * NT;
    constexpr uint32_t WAVES = kCombineThreads / 64;
    static_assert(Q <= 64 && 64 % Q == 0, "a wave holds whole record rows");
    __shared__ float4 s_num[WC ? 1 : WAVES][Q];
    __shared__ float s_den[WC ? 1 : WAVES][Q], s_m[WC ? 1 : WAVES][Q];
    const uint32_t u = blockIdx.x, t = threadIdx.x;
    const uint32_t col = WC ? blockIdx.y * kCombineWaveCols + (t >> 6) : blockIdx.y;
    const MergeDesc md = p.merge[u];
    if (md.n == 0) return; // written directly by its only workgroup, or no such unit
    if (col >= (md.nrows_hk & 0xffffu) * p.group) return;
    const uint32_t n = md.n, rec0 = md.rec0;
    const uint32_t q = t % Q, rg = (t % TPC) / Q;
    const float4 *po = (const float4 *)p.part_o;
    // per thread: its records merged against its own reference maximum M
    float M = -INFINITY, den = 0.0f;
    float4 num = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    for (uint32_t base = 0; base < n; base += RPP * kCombinePasses) {
        float4 o[kCombinePasses];
        float m[kCombinePasses], l[kCombinePasses];
#pragma unroll
        for (uint32_t k = 0; k < kCombinePasses; k++) {
            // unconditional loads (a clamped index past the end, weighted zero): loads under
            // a branch would each be waited for at the branch's join
            const uint32_t r = base + k * RPP + rg;
            const size_t rb = (size_t)(rec0 + min(r, n - 1)) * COLS + col;
            if constexpr (REC == 0) {
                o[k] = po[rb * QF + qoff + q];
            } else {
                const u32x2 h = ((const u32x2 *)p.part_o)[rb * QF + qoff + q];
                if constexpr (REC == 2)
                    o[k] = make_float4(bf16_to_f32(h.x & 0xffffu), bf16_to_f32(h.x >> 16),
                                       bf16_to_f32(h.y & 0xffffu), bf16_to_f32(h.y >> 16));
                else
                    o[k] = make_float4(f16_to_f32(h.x & 0xffffu), f16_to_f32(h.x >> 16),
                                       f16_to_f32(h.y & 0xffffu), f16_to_f32(h.y >> 16));
            }
            const float2 ml = ((const float2 *)p.part_ml)[rb];
            m[k] = ml.x;
            l[k] = r < n ? ml.y : 0.0f;
        }
        float bm = M;
#pragma unroll
        for (uint32_t k = 0; k < kCombinePasses; k++)
            if (l[k] > 0.0f) bm = fmaxf(bm, m[k]);
        if (bm != M) {
            const float f = M == -INFINITY ? 0.0f : fast_exp2(M - bm);
            num.x *= f; num.y *= f; num.z *= f; num.w *= f;
            den *= f;
            M = bm;
        }
#pragma unroll
        for (uint32_t k = 0; k < kCombinePasses; k++) {
            // normalised rows weigh by their mass too
            const float w = l[k] > 0.0f ? fast_exp2(m[k] - M) * (REC ? l[k] : 1.0f) : 0.0f;
            num.x = fmaf(w, o[k].x, num.x);
            num.y = fmaf(w, o[k].y, num.y);
            num.z = fmaf(w, o[k].z, num.z);
            num.w = fmaf(w, o[k].w, num.w);
            den = REC ? den + w : fmaf(w, l[k], den);
        }
    }
    // merge (M, num, den) of the record groups that share the quad q: lanes Q apart within a
    // wave by shuffles, then the waves through LDS (a group without records holds M = -inf
    // and zeros, and weighs zero)
    auto merge = [&](float mo, float4 no, float dn) {
        const float nm = fmaxf(M, mo);
        const float a = M == -INFINITY ? 0.0f : fast_exp2(M - nm);
        const float b = mo == -INFINITY ? 0.0f : fast_exp2(mo - nm);
        num.x = num.x * a + no.x * b;
        num.y = num.y * a + no.y * b;
        num.z = num.z * a + no.z * b;
        num.w = num.w * a + no.w * b;
        den = den * a + dn * b;
        M = nm;
    };
#pragma unroll
    for (uint32_t sh = Q; sh < 64; sh <<= 1) {
        const float mo = shfl_xor(M, sh), dn = shfl_xor(den, sh);
        const float4 no = make_float4(shfl_xor(num.x, sh), shfl_xor(num.y, sh), shfl_xor(num.z, sh),
                                      shfl_xor(num.w, sh));
        merge(mo, no, dn);
    }
    if constexpr (WC) {
        if ((t & 63) >= Q) return;
    } else {
        const uint32_t w = t >> 6;
        if ((t & 63) < Q) {
            s_num[w][q] = num;
            s_den[w][q] = den;
            s_m[w][q] = M;
        }
        __syncthreads();
        if (t >= Q) return;
#pragma unroll
        for (uint32_t v = 1; v < WAVES; v++) merge(s_m[v][q], s_num[v][q], s_den[v][q]);
    }
    const float inv = den > 0.0f ? 1.0f / den : 0.0f;
    const uint32_t row = md.rowbeg + col / p.group, head = (md.nrows_hk >> 16) * p.group + col % p.group;
    const size_t at = ((size_t)row * p.hq + head) * D + 4 * (qoff + q);
    if (p.out_f32) {
        *(float4 *)((float *)p.out + at) = make_float4(num.x * inv, num.y * inv, num.z * inv, num.w * inv);
    } else {
        *(u32x2 *)((uint16_t *)p.out + at) =
            u32x2{(uint32_t)f32_to_bf16(num.x * inv) | ((uint32_t)f32_to_bf16(num.y * inv) << 16),
                  (uint32_t)f32_to_bf16(num.z * inv) | ((uint32_t)f32_to_bf16(num.w * inv) << 16)};
    }
}

// Merge for the prefill kernel's 128-column units, which are split over few workgroups
// (2-3 records each): one wave per column, four columns per workgroup.  Lanes hold a
// record's row as float4 quads (64 / (D/4) records per pass); the record groups are summed
// with lane shuffles.  Same merge rule as combine_kernel.
// Columns merged by one wave of combine_wide_kernel, and record passes loaded per batch.
constexpr uint32_t kWideCombineCols = 4;
constexpr uint32_t kWideCombinePasses = 2;

// REC: record rows normalised in f32 (0), f16 (1) or bf16 (2).
template <int D, int REC>
__global__ __launch_bounds__(256) void combine_wide_kernel(AttnParams p) {
    constexpr uint32_t Q = D / 4, RPP = 64 / Q, COLS = 16 * kWideNTDev;
    constexpr uint32_t CW = kWideCombineCols, KP = kWideCombinePasses;
    const uint32_t u = blockIdx.x, lane = threadIdx.x & 63;
    const uint32_t wave = (uint32_t)__builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const uint32_t col0 = (blockIdx.y * 4 + wave) * CW; // this wave's first column
    const MergeDesc md = p.merge[u];
    const uint32_t ncols = (md.nrows_hk & 0xffffu) * p.group;
    if (md.n == 0 || col0 >= ncols) return;
    const uint32_t n = md.n, rec0 = md.rec0, q = lane % Q, rg = lane / Q;
    // records hold O / l (f32, f16 or bf16 per REC), four values per quad, so a record
    // weighs w * l
    const u32x2 *po = (const u32x2 *)p.part_o;
    const float4 *pf = (const float4 *)p.part_o;
    float M[CW], den[CW];
    float4 num[CW];
#pragma unroll
    for (uint32_t c = 0; c < CW; c++) {
        M[c] = -INFINITY;
        den[c] = 0.0f;
        num[c] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
    for (uint32_t base = 0; base < n; base += RPP * KP) {
        // every load of the batch (all CW columns) before any use: unconditional, records
        // past n clamped to the last and weighted zero, columns past the unit's to its last
        float4 o[CW][KP];
        float m[CW][KP], l[CW][KP];
#pragma unroll
        for (uint32_t c = 0; c < CW; c++)
#pragma unroll
            for (uint32_t k = 0; k < KP; k++) {
                const uint32_t r = base + k * RPP + rg;
                const size_t rb = (size_t)(rec0 + min(r, n - 1)) * COLS + min(col0 + c, ncols - 1);
                if constexpr (REC == 0) {
                    o[c][k] = pf[rb * Q + q];
                } else {
                    const u32x2 h = po[rb * Q + q];
                    if constexpr (REC == 2)
                        o[c][k] = make_float4(bf16_to_f32(h.x & 0xffffu), bf16_to_f32(h.x >> 16),
                                              bf16_to_f32(h.y & 0xffffu), bf16_to_f32(h.y >> 16));
                    else
                        o[c][k] = make_float4(f16_to_f32(h.x & 0xffffu), f16_to_f32(h.x >> 16),
                                              f16_to_f32(h.y & 0xffffu), f16_to_f32(h.y >> 16));
                }
                const float2 ml = ((const float2 *)p.part_ml)[rb];
                m[c][k] = ml.x;
                l[c][k] = r < n ? ml.y : 0.0f;
            }
#pragma unroll
        for (uint32_t c = 0; c < CW; c++) {
            float bm = -INFINITY;
#pragma unroll
            for (uint32_t k = 0; k < KP; k++)
                if (l[c][k] > 0.0f) bm = fmaxf(bm, m[c][k]);
            bm = wave_max(bm);
            const float nm = fmaxf(M[c], bm);
            if (nm != M[c]) {
                const float f = M[c] == -INFINITY ? 0.0f : fast_exp2(M[c] - nm);
                num[c].x *= f; num[c].y *= f; num[c].z *= f; num[c].w *= f;
                den[c] *= f;
                M[c] = nm;
            }
#pragma unroll
            for (uint32_t k = 0; k < KP; k++) {
                const float w = l[c][k] > 0.0f ? fast_exp2(m[c][k] - M[c]) * l[c][k] : 0.0f;
                num[c].x = fmaf(w, o[c][k].x, num[c].x);
                num[c].y = fmaf(w, o[c][k].y, num[c].y);
                num[c].z = fmaf(w, o[c][k].z, num[c].z);
                num[c].w = fmaf(w, o[c][k].w, num[c].w);
                den[c] += w;
            }
        }
    }
#pragma unroll
    for (uint32_t c = 0; c < CW; c++) {
        const uint32_t col = col0 + c;
        float4 x = num[c];
        float dn = den[c];
#pragma unroll
        for (uint32_t off = Q; off < 64; off <<= 1) {
            x.x += shfl_xor(x.x, off);
            x.y += shfl_xor(x.y, off);
            x.z += shfl_xor(x.z, off);
            x.w += shfl_xor(x.w, off);
            dn += shfl_xor(dn, off);
        }
        if (rg != 0 || col >= ncols) continue;
        const float inv = dn > 0.0f ? 1.0f / dn : 0.0f;
        const uint32_t row = md.rowbeg + col / p.group, head = (md.nrows_hk >> 16) * p.group + col % p.group;
        const size_t at = ((size_t)row * p.hq + head) * D + 4 * q;
        if (p.out_f32) {
            *(float4 *)((float *)p.out + at) = make_float4(x.x * inv, x.y * inv, x.z * inv, x.w * inv);
        } else {
            *(u32x2 *)((uint16_t *)p.out + at) =
                u32x2{(uint32_t)f32_to_bf16(x.x * inv) | ((uint32_t)f32_to_bf16(x.y * inv) << 16),
                      (uint32_t)f32_to_bf16(x.z * inv) | ((uint32_t)f32_to_bf16(x.w * inv) << 16)};
        }
    }
}

// ------------------------------------------------------------------ host side

struct Layout {
    size_t header, units, work, merge, part_ml, part_o, total;
    uint32_t max_units, max_records;
};

// Columns per unit / 16.  Decode-only batches (one row per sequence) use one 16-column tile
// and batches with multi-row sequences (MTP verify, short chunks) two, in the decode kernel;
// batches averaging 16 or more rows per sequence (prefill chunks) use the prefill kernel's
// 128 columns (on FP8 pools with the rows staged through registers).
constexpr uint32_t kWideNT = kWideNTDev;
static inline uint32_t nt_for(uint32_t n_rows, uint32_t n_seqs, uint32_t group, int kv_dtype) {
    if (n_rows >= 16 * n_seqs && group <= 32) return kWideNT;
    return (n_rows > n_seqs || group > 16) ? 2 : 1;
}

template <int D, int NT, int REC>
static hipError_t launch_combine(uint32_t split, dim3 grid, const AttnParams &p, hipStream_t s) {
    const dim3 block(kCombineThreads);
    if (split == 4) return launch<combine_kernel<D, NT, 4, REC>>(grid, block, 0, s, p);
    if (split == 2) return launch<combine_kernel<D, NT, 2, REC>>(grid, block, 0, s, p);
    if (split == 0) {
        const dim3 g(grid.x, (grid.y + kCombineWaveCols - 1) / kCombineWaveCols);
        return launch<combine_kernel<D, NT, 0, REC>>(g, block, 0, s, p);
    }
    return launch<combine_kernel<D, NT, 1, REC>>(grid, block, 0, s, p);
}

static Layout layout_for(const lia_attention_config *c, uint32_t n_wg) {
    Layout L;
    uint32_t group = c->num_q_heads / c->num_kv_heads;
    uint32_t rpc1 = group <= 16 ? 16 / group : 1; // smallest rows-per-block over NT choices
    L.max_units = (c->max_rows / rpc1 + c->max_seqs + 1) * c->num_kv_heads;
    L.max_records = n_wg + L.max_units;
    size_t off = 0;
    L.header = off; off += 256;
    L.units = off; off += ((size_t)L.max_units + 1) * sizeof(UnitDesc);
    off = (off + 255) & ~(size_t)255;
    L.work = off; off += (size_t)n_wg * sizeof(WorkDesc);
    off = (off + 255) & ~(size_t)255;
    L.merge = off; off += (size_t)L.max_units * sizeof(MergeDesc);
    off = (off + 255) & ~(size_t)255;
    // record columns: 16 per tile, up to the prefill kernel's kWideNT
    const size_t rec_cols = 16 * kWideNT;
    L.part_ml = off; off += (size_t)L.max_records * rec_cols * 2 * sizeof(float);
    off = (off + 255) & ~(size_t)255;
    L.part_o = off; off += (size_t)L.max_records * rec_cols * c->head_dim * sizeof(float);
    L.total = off;
    return L;
}

} // namespace lia

using namespace lia;


// Workspace of lia_paged_attention_static: a file-scope device array, so that entry point
// allocates nothing.  Each device the library runs on holds its own copy until the process
// ends; its address is looked up once per device (hipGetSymbolAddress with the device
// current) and only that address is handed to kernels - the array's name in host code is a
// host-side stand-in, not a device address.  Every call on one device shares the array:
// calls that overlap on a device race.  Nothing in it needs to start at zero (the plan writes
// every descriptor the other kernels read, the attention kernel every record the merge reads).
constexpr size_t kStaticWorkspaceBytes = 64ull << 20;
static __device__ __align__(256) uint8_t scratch[kStaticWorkspaceBytes];
constexpr int kMaxDevices = 64;
static void *g_scratch[kMaxDevices];
static std::mutex g_scratch_mutex;

static int scratch_of_current_device(void **out) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return LIA_E_HIP;
    if (dev < 0 || dev >= kMaxDevices) return LIA_E_UNSUPPORTED;
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (!g_scratch[dev]) {
        void *p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return LIA_E_HIP;
        g_scratch[dev] = p;
    }
    *out = g_scratch[dev];
    return LIA_OK;
}

extern "C" int lia_init(int device) {
    if (hipSetDevice(device) != hipSuccess) {
        (void)hipGetLastError(); // leave no pending error for the caller's next runtime call
        return LIA_E_HIP;
    }
    void *ws = nullptr;
    if (const int e = scratch_of_current_device(&ws)) return e;
    if (!device_cus()) return LIA_E_HIP;
    return resolve_kernels();
}

extern "C" uint32_t lia_device_cus(void) { return device_cus(); }

// Prefill kernel: resident 8-wave workgroups per CU at most.  Decode kernel: at most this
// many waves per CU (three 2-wave workgroups measured best on 16-bit pools at head_dim 128,
// four 2-wave workgroups on FP8 pools).  Fewer, longer splits also shrink the combine.
constexpr uint32_t kMaxPerCU = 3;
constexpr uint32_t kMaxWavesPerCU = 6;
constexpr uint32_t kMaxWavesPerCU8 = 8;
static uint32_t max_waves(int kv) { return kv == LIA_FP8_E4M3 ? kMaxWavesPerCU8 : kMaxWavesPerCU; }

static uint32_t decode_waves(uint32_t d, int) { return d / 64; } // one wave per 64-dim slice

// Resident workgroups per CU allowed for a launch of NT column tiles.
static uint32_t max_per_cu(uint32_t d, uint32_t nt, int kv) {
    return nt == kWideNT ? kMaxPerCU : max_waves(kv) / decode_waves(d, kv);
}

// Upper bound on attention workgroups per launch of a configuration: sizes the plan and
// the record area.
static uint32_t max_workgroups(const lia_attention_config *c) {
    uint32_t cus = lia_device_cus();
    if (!cus) cus = 256;
    const uint32_t per = max(kMaxPerCU, max_waves(c->kv_dtype) / decode_waves(c->head_dim, c->kv_dtype));
    return cus * per;
}

template <int D, int NT, int KVT>
static uint32_t resident_workgroups() {
    // workgroups of this instantiation that fit on one CU at once (registers and LDS)
    static uint32_t cached = 0;
    if (!cached) {
        int per_cu = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
                &per_cu, reinterpret_cast<const void *>(&attention_kernel<D, NT, KVT>),
                Cfg<D, KVT>::THREADS, 0) !=
                hipSuccess || per_cu < 1)
            per_cu = 1;
        cached = (uint32_t)per_cu;
    }
    return cached;
}

template <int D, int KVT>
static uint32_t resident_wide() {
    static uint32_t cached = 0;
    if (!cached) {
        int per_cu = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
                &per_cu, reinterpret_cast<const void *>(&wide_kernel<D, KVT>), WCfg<D>::THREADS, 0) != hipSuccess ||
            per_cu < 1)
            per_cu = 1;
        cached = (uint32_t)per_cu;
    }
    return cached;
}

template <int D, int NT>
static uint32_t resident_kv(int kv) {
    if constexpr (NT == kWideNT) {
        return kv == LIA_BF16 ? resident_wide<D, LIA_BF16>()
               : kv == LIA_F16 ? resident_wide<D, LIA_F16>() : resident_wide<D, LIA_FP8_E4M3>();
    } else {
        if (kv == LIA_BF16) return resident_workgroups<D, NT, LIA_BF16>();
        if (kv == LIA_F16) return resident_workgroups<D, NT, LIA_F16>();
        return resident_workgroups<D, NT, LIA_FP8_E4M3>();
    }
}

// Workgroups of one launch: every CU filled once with resident workgroups.
static uint32_t workgroups_for(const lia_attention_config *c, uint32_t nt) {
    const uint32_t d = c->head_dim;
    const int kv = c->kv_dtype;
    uint32_t cus = lia_device_cus();
    if (!cus) cus = 256;
    uint32_t per = d == 128 ? (nt == 1 ? resident_kv<128, 1>(kv)
                               : nt == 2 ? resident_kv<128, 2>(kv) : resident_kv<128, kWideNT>(kv))
                            : (nt == 1 ? resident_kv<64, 1>(kv)
                               : nt == 2 ? resident_kv<64, 2>(kv) : resident_kv<64, kWideNT>(kv));
    if (per > max_per_cu(d, nt, kv)) per = max_per_cu(d, nt, kv);
    uint32_t n = cus * per;
    uint32_t cap = max_workgroups(c);
    return n < cap ? n : cap;
}

extern "C" size_t lia_attention_workspace_bytes(const lia_attention_config *c) {
    if (!c || !c->num_kv_heads) return 0;
    return layout_for(c, max_workgroups(c)).total;
}

static int validate(const lia_attention_config *c) {
    if (!c) return LIA_E_ARG;
    if (c->num_kv_heads == 0 || c->num_q_heads == 0 || c->num_q_heads % c->num_kv_heads)
        return LIA_E_ARG;
    uint32_t group = c->num_q_heads / c->num_kv_heads;
    if (group > 32) return LIA_E_UNSUPPORTED;
    if (c->head_dim != 64 && c->head_dim != 128) return LIA_E_UNSUPPORTED;
    if (c->page_size < 16 || (c->page_size & (c->page_size - 1))) return LIA_E_UNSUPPORTED;
    if (c->q_dtype != LIA_F32 && c->q_dtype != LIA_BF16) return LIA_E_UNSUPPORTED;
    if (c->out_dtype != LIA_F32 && c->out_dtype != LIA_BF16) return LIA_E_UNSUPPORTED;
    if (c->kv_dtype != LIA_F16 && c->kv_dtype != LIA_BF16 && c->kv_dtype != LIA_FP8_E4M3)
        return LIA_E_UNSUPPORTED;
    if (c->stride == 0 || c->max_seqs == 0 || c->max_rows == 0) return LIA_E_ARG;
    if (!(c->scale > 0.0f) || !(c->scale < INFINITY)) return LIA_E_ARG; // the kernels rely on scale > 0
    return LIA_OK;
}

template <int D, int NT, int KVT, bool RO = false>
static hipError_t launch_partial(const AttnParams &p, uint32_t n_wg, hipStream_t s) {
    return launch<attention_kernel<D, NT, KVT, RO>>(dim3(n_wg), dim3(Cfg<D, KVT>::THREADS), 0, s, p);
}

template <int D>
static hipError_t launch_wide(int kv, const AttnParams &p, uint32_t n_wg, hipStream_t s) {
    const dim3 block(WCfg<D>::THREADS);
    if (kv == LIA_BF16) return launch<wide_kernel<D, LIA_BF16>>(dim3(n_wg), block, 0, s, p);
    if (kv == LIA_F16) return launch<wide_kernel<D, LIA_F16>>(dim3(n_wg), block, 0, s, p);
    return launch<wide_kernel<D, LIA_FP8_E4M3>>(dim3(n_wg), block, 0, s, p);
}

template <int D, int NT, bool RO = false>
static hipError_t launch_partial_kv(int kv, const AttnParams &p, uint32_t n_wg, hipStream_t s) {
    if (kv == LIA_BF16) return launch_partial<D, NT, LIA_BF16, RO>(p, n_wg, s);
    if (kv == LIA_F16) return launch_partial<D, NT, LIA_F16, RO>(p, n_wg, s);
    return launch_partial<D, NT, LIA_FP8_E4M3, RO>(p, n_wg, s);
}

enum Stage { kPlan = 1, kPartial = 2, kMerge = 4, kRead = 8 };

// New rows appended by the attention launch itself (lia_attention_partial_append).
struct FusedAppend {
    const void *k, *v;
    const uint32_t *slots;
};

static int run_stages(int stages, const lia_attention_config *c, uint32_t n_seqs, uint32_t n_rows,
                      const uint32_t *cu_seqlens, const uint32_t *positions,
                      const uint32_t *sequences, const uint32_t *pages, const void *q,
                      const void *kc, const void *vc, const float *k_scales,
                      const float *v_scales, void *workspace, size_t workspace_bytes, void *out,
                      lia_stream_t stream, const FusedAppend *fa = nullptr, bool enqueue = true,
                      const PackArgs *pk = nullptr) {
    int st = validate(c);
    if (st) return st;
    if (n_seqs == 0 || n_seqs > c->max_seqs || n_rows == 0 || n_rows > c->max_rows) return LIA_E_ARG;
    if (!cu_seqlens || !positions || !workspace) return LIA_E_ARG;
    if ((stages & kPlan) && !sequences) return LIA_E_ARG;
    if (stages & (kPartial | kMerge)) {
        if (!out) return LIA_E_ARG;
        if ((uintptr_t)out & 15) return LIA_E_ALIGN;
    }
    if (fa) {
        if (c->kv_dtype == LIA_FP8_E4M3) return LIA_E_UNSUPPORTED;
        if (!fa->k || !fa->v || !fa->slots) return LIA_E_ARG;
        if (((uintptr_t)fa->k | (uintptr_t)fa->v) & 15) return LIA_E_ALIGN;
    }
    if (stages & kRead) {
        if (!out) return LIA_E_ARG;
        if ((uintptr_t)out & 3) return LIA_E_ALIGN;
    }
    if (stages & (kPartial | kRead)) {
        if (!pages || !q || !kc || !vc) return LIA_E_ARG;
        if (c->kv_dtype == LIA_FP8_E4M3 && (!k_scales || !v_scales)) return LIA_E_ARG;
        if (((uintptr_t)q | (uintptr_t)kc | (uintptr_t)vc) & 15) return LIA_E_ALIGN;
    }
    // q and the FP8 scale arrays are read through 32-bit buffer ranges
    if ((uint64_t)c->max_rows * c->num_q_heads * c->head_dim * 4 >= (1ull << 31) ||
        (uint64_t)c->pool_pages * c->num_kv_heads * 4 >= (1ull << 31))
        return LIA_E_UNSUPPORTED;
    Layout L = layout_for(c, max_workgroups(c));
    if (workspace_bytes < L.total) return LIA_E_WORKSPACE;
    if ((uintptr_t)workspace & 255) return LIA_E_ALIGN;
    if (!enqueue) return LIA_OK; // validation only
    const uint32_t group = c->num_q_heads / c->num_kv_heads;
    const uint32_t NT = nt_for(n_rows, n_seqs, group, c->kv_dtype);
    const uint32_t n_wg = workgroups_for(c, NT);
    // rows per column block; with as many rows as sequences (decode, possibly with some
    // sequences adding no rows and others several) one row per block, so every unit has
    // `group` columns and there are n_rows units per KV head (the merge grid below relies
    // on both)
    const uint32_t rpc = (NT == 1 && n_rows == n_seqs) ? 1 : (16 * NT) / group;
    uint8_t *ws = (uint8_t *)workspace;
    AttnParams p;
    p.q = q; p.kc = kc; p.vc = vc; p.k_scales = k_scales; p.v_scales = v_scales;
    p.cu = cu_seqlens; p.positions = positions; p.sequences = sequences; p.pages = pages;
    p.out = out;
    p.units = (const UnitDesc *)(ws + L.units);
    p.work = (const WorkDesc *)(ws + L.work);
    p.merge = (const MergeDesc *)(ws + L.merge);
    p.header = (const uint32_t *)(ws + L.header);
    p.part_o = (float *)(ws + L.part_o);
    p.part_ml = (float *)(ws + L.part_ml);
    p.hq = c->num_q_heads; p.hkv = c->num_kv_heads; p.group = group; p.stride = c->stride;
    p.page_shift = (uint32_t)__builtin_ctz(c->page_size);
    p.pool_pages = c->pool_pages;
    p.n_wg = n_wg;
    p.rpc = rpc;
    p.scale_log2 = c->scale * 1.4426950408889634f;
    p.q_f32 = c->q_dtype == LIA_F32;
    p.out_f32 = c->out_dtype == LIA_F32;
    p.newk = fa ? fa->k : nullptr;
    p.newv = fa ? fa->v : nullptr;
    p.slots = fa ? fa->slots : nullptr;
    p.kc_w = const_cast<void *>(kc);
    p.vc_w = const_cast<void *>(vc);
    p.n_rows = n_rows;
    p.round_wg = lia_device_cus() ? lia_device_cus() : 256;
    hipStream_t s = (hipStream_t)stream;
    hipError_t e = hipSuccess;
    if (stages & kPlan) {
        UnitDesc *units = (UnitDesc *)(ws + L.units);
        WorkDesc *work = (WorkDesc *)(ws + L.work);
        MergeDesc *merge = (MergeDesc *)(ws + L.merge);
        uint32_t *header = (uint32_t *)(ws + L.header);
        // Block ranges XCD-major (each XCD a contiguous share).  Measured against launch order:
        // the config-2 step 1.3-1.4 % faster (its attention launch alone 0.15 us slower), the
        // config-3 prefill kernel 3 % faster, config 5 2 us shorter, config 4 unchanged.
        const uint32_t xcd = 1;
        const uint32_t cost = NT == kWideNT ? kUnitCostWide : kUnitCostDecode;
        const uint32_t lag = NT == kWideNT ? kLagWide : kLagDecode;
        if (pk && n_seqs <= kPlanSeqs && n_wg <= kPlanThreads) {
            // the packing, the plan (from the packing's inputs) and the table checks in one
            // launch, then the step's verdict
            const RawSeqs raw{pk->q_lens, pk->cached, pk->seq_slots, n_rows};
            e = launch<pack_plan_kernel>(dim3(kPlanGroups + 1 + kSetupChecks), dim3(kPlanThreads), 0, s,
                                         n_seqs, *pk, raw, rpc, c->num_kv_heads, L.max_units, n_wg, cost,
                                         lia_device_cus(), lag, xcd, units, work, merge, header);
            if (e == hipSuccess)
                e = launch<setup_verdict_kernel>(dim3(1), dim3(kPlanThreads), 0, s, n_seqs, pk->max_rows,
                                                 pk->cu, pk->slot_mapping, pk->status, header, work, n_wg,
                                                 merge, L.max_units);
        } else {
            if (pk) { // too many sequences or workgroups for the one-launch form: pack first
                const int ps = lia_pack_device(n_seqs, pk->seq_slots, pk->q_lens, pk->cached, pk->pages,
                                               pk->stride, 1u << pk->page_shift, pk->pool_pages,
                                               pk->context, pk->max_rows, pk->cu, pk->positions,
                                               pk->sequences, pk->slot_mapping, pk->status, stream);
                if (ps) return ps;
            }
            if (n_seqs <= kPlanSeqs && n_wg <= kPlanThreads)
            e = launch<plan_lds_kernel>(dim3(kPlanGroups), dim3(kPlanThreads), 0, s, n_seqs, cu_seqlens,
                                        positions, sequences, pages, c->stride, p.page_shift, rpc,
                                        c->num_kv_heads, L.max_units, n_wg,
                                        NT == kWideNT ? kUnitCostWide : kUnitCostDecode,
                                        lia_device_cus(), NT == kWideNT ? kLagWide : kLagDecode,
                                        xcd, units, work, merge, header);
            else
            e = launch<plan_kernel>(dim3(1), dim3(256), 0, s, n_seqs, cu_seqlens, positions,
                                    sequences, pages, c->stride, p.page_shift, rpc, c->num_kv_heads,
                                    L.max_units, n_wg, xcd, units, work, merge, header);
        }
    }
    if (e == hipSuccess && (stages & kPartial)) {
        if (c->head_dim == 128) {
            if (NT == 1) e = launch_partial_kv<128, 1>(c->kv_dtype, p, n_wg, s);
            else if (NT == 2) e = launch_partial_kv<128, 2>(c->kv_dtype, p, n_wg, s);
            else e = launch_wide<128>(c->kv_dtype, p, n_wg, s);
        } else {
            if (NT == 1) e = launch_partial_kv<64, 1>(c->kv_dtype, p, n_wg, s);
            else if (NT == 2) e = launch_partial_kv<64, 2>(c->kv_dtype, p, n_wg, s);
            else e = launch_wide<64>(c->kv_dtype, p, n_wg, s);
        }
    }
    if (e == hipSuccess && (stages & kRead)) {
        // the decode kernel's loads alone (lia_paged_read): 16-bit pools, decode tiles
        if (c->head_dim == 128) {
            if (NT == 1) e = launch_partial_kv<128, 1, true>(c->kv_dtype, p, n_wg, s);
            else e = launch_partial_kv<128, 2, true>(c->kv_dtype, p, n_wg, s);
        } else {
            if (NT == 1) e = launch_partial_kv<64, 1, true>(c->kv_dtype, p, n_wg, s);
            else e = launch_partial_kv<64, 2, true>(c->kv_dtype, p, n_wg, s);
        }
    }
    if (e == hipSuccess && (stages & kMerge)) {
        // units this NT can produce: rows in blocks of rpc per sequence and KV head
        // (sum over sequences of ceil(rows / rpc) <= n_rows / rpc + n_seqs)
        uint32_t units_nt = (n_rows / (rpc ? rpc : 1) + n_seqs + 1) * c->num_kv_heads;
        uint32_t cols = 16 * NT;
        if (NT == 1 && n_rows == n_seqs) {
            // one row per column block (rpc = 1): n_rows units per KV head, `group` columns
            units_nt = n_seqs * c->num_kv_heads;
            cols = group < cols ? group : cols;
        }
        dim3 grid(units_nt < L.max_units ? units_nt : L.max_units, cols);
        // a small merge (few units, as in a decode batch of a few long sequences) splits each
        // record row over two workgroups (measured 0.6 us faster per layer at 128 workgroups,
        // slower on grids of hundreds or thousands), and over four when units hold hundreds of
        // records (one or two long sequences: a batch of 256 records per pass instead of 128)
        // record rows: f32 for f32 outputs and FP8 pools, else the pool's 16-bit type
        const int rec = p.out_f32 ? 0 : c->kv_dtype == LIA_BF16 ? 2 : c->kv_dtype == LIA_F16 ? 1 : 0;
        const uint32_t est_units = max((n_rows + rpc - 1) / rpc, n_seqs) * c->num_kv_heads;
        const uint32_t per_unit = n_wg / est_units; // records per unit, roughly
        const uint32_t split = per_unit >= 128 ? 4 : grid.x * grid.y < 256 ? 2 : per_unit <= kWaveColRecords ? 0 : 1;
        grid.z = split;
#define LIA_COMBINE(DD, NN)                                                                      \
    do {                                                                                         \
        if (rec == 1) e = launch_combine<DD, NN, 1>(split, grid, p, s);                           \
        else if (rec == 2) e = launch_combine<DD, NN, 2>(split, grid, p, s);                      \
        else e = launch_combine<DD, NN, 0>(split, grid, p, s);                                    \
    } while (0)
        const dim3 wgrid(grid.x, 16 * kWideNT / (4 * kWideCombineCols));
        if (c->head_dim == 128) {
            if (NT == 1) LIA_COMBINE(128, 1);
            else if (NT == 2) LIA_COMBINE(128, 2);
            else if (rec == 0) e = launch<combine_wide_kernel<128, 0>>(wgrid, dim3(256), 0, s, p);
            else if (rec == 2) e = launch<combine_wide_kernel<128, 2>>(wgrid, dim3(256), 0, s, p);
            else e = launch<combine_wide_kernel<128, 1>>(wgrid, dim3(256), 0, s, p);
        } else {
            if (NT == 1) LIA_COMBINE(64, 1);
            else if (NT == 2) LIA_COMBINE(64, 2);
            else if (rec == 0) e = launch<combine_wide_kernel<64, 0>>(wgrid, dim3(256), 0, s, p);
            else if (rec == 2) e = launch<combine_wide_kernel<64, 2>>(wgrid, dim3(256), 0, s, p);
            else e = launch<combine_wide_kernel<64, 1>>(wgrid, dim3(256), 0, s, p);
        }
#undef LIA_COMBINE
    }
    return e == hipSuccess ? LIA_OK : LIA_E_HIP;
}

extern "C" int lia_paged_attention(const lia_attention_config *c, uint32_t n_seqs, uint32_t n_rows,
                                   const uint32_t *cu_seqlens, const uint32_t *positions,
                                   const uint32_t *sequences, const uint32_t *pages, const void *q,
                                   const void *kc, const void *vc, const float *k_scales,
                                   const float *v_scales, void *workspace, size_t workspace_bytes,
                                   void *out, lia_stream_t stream) {
    return run_stages(kPlan | kPartial | kMerge, c, n_seqs, n_rows, cu_seqlens, positions,
                      sequences, pages, q, kc, vc, k_scales, v_scales, workspace, workspace_bytes,
                      out, stream);
}

extern "C" int lia_attention_plan(const lia_attention_config *c, uint32_t n_seqs, uint32_t n_rows,
                                  const uint32_t *cu_seqlens, const uint32_t *positions,
                                  const uint32_t *sequences, const uint32_t *pages,
                                  void *workspace, size_t workspace_bytes, lia_stream_t stream) {
    return run_stages(kPlan, c, n_seqs, n_rows, cu_seqlens, positions, sequences, pages,
                      nullptr, nullptr, nullptr, nullptr, nullptr, workspace, workspace_bytes,
                      nullptr, stream);
}

extern "C" int lia_pack_plan_device(const lia_attention_config *c, uint32_t n_seqs, uint32_t n_rows,
                                    const uint32_t *seq_slots, const uint32_t *q_lens,
                                    const uint32_t *cached, const uint32_t *pages, uint32_t context,
                                    uint32_t *cu_seqlens, uint32_t *positions, uint32_t *sequences,
                                    uint32_t *slot_mapping, uint32_t *status, void *workspace,
                                    size_t workspace_bytes, lia_stream_t stream) {
    if (!c || !seq_slots || !q_lens || !cached || !pages || !cu_seqlens || !positions || !sequences ||
        !slot_mapping || !status)
        return LIA_E_ARG;
    // every check of the plan stage before anything is enqueued
    int st = run_stages(kPlan, c, n_seqs, n_rows, cu_seqlens, positions, sequences, pages, nullptr,
                        nullptr, nullptr, nullptr, nullptr, workspace, workspace_bytes, nullptr, stream,
                        nullptr, false);
    if (st) return st;
    const PackArgs pk{seq_slots, q_lens, cached, pages, c->stride, (uint32_t)__builtin_ctz(c->page_size),
                      c->pool_pages, context, c->max_rows, cu_seqlens, positions, sequences,
                      slot_mapping, status};
    return run_stages(kPlan, c, n_seqs, n_rows, cu_seqlens, positions, sequences, pages, nullptr,
                      nullptr, nullptr, nullptr, nullptr, workspace, workspace_bytes, nullptr, stream,
                      nullptr, true, &pk);
}

extern "C" int lia_attention_partial(const lia_attention_config *c, uint32_t n_seqs,
                                     uint32_t n_rows, const uint32_t *pages, const void *q,
                                     const void *kc, const void *vc, const float *k_scales,
                                     const float *v_scales, void *workspace,
                                     size_t workspace_bytes, void *out, lia_stream_t stream) {
    // the plan carries the per-row metadata; cu_seqlens / positions are not re-read
    static const uint32_t dummy = 0;
    return run_stages(kPartial, c, n_seqs, n_rows, &dummy, &dummy, nullptr, pages, q, kc, vc,
                      k_scales, v_scales, workspace, workspace_bytes, out, stream);
}

extern "C" int lia_attention_partial_append(const lia_attention_config *c, uint32_t n_seqs,
                                            uint32_t n_rows, const uint32_t *pages,
                                            const uint32_t *slot_mapping, const void *q,
                                            const void *new_k, const void *new_v, void *kc,
                                            void *vc, void *workspace, size_t workspace_bytes,
                                            void *out, lia_stream_t stream) {
    static const uint32_t dummy = 0;
    const FusedAppend fa{new_k, new_v, slot_mapping};
    return run_stages(kPartial, c, n_seqs, n_rows, &dummy, &dummy, nullptr, pages, q, kc, vc,
                      nullptr, nullptr, workspace, workspace_bytes, out, stream, &fa);
}

// FP8 pools: the quantising append (lia_kv_append of bf16 rows through the slot mapping) and
// the attention kernel over the pool, as two launches.  Quantising the new rows inside the
// attention launch instead was measured slower on the config-5 decode step (the e4m3
// conversions and divisions sit on the critical path of every unit's last workgroup).
extern "C" int lia_attention_partial_append_fp8(const lia_attention_config *c, uint32_t n_seqs,
                                                uint32_t n_rows, const uint32_t *pages,
                                                const uint32_t *slot_mapping, const void *q,
                                                const void *new_k, const void *new_v, void *kc,
                                                void *vc, float *k_scales, float *v_scales,
                                                void *workspace, size_t workspace_bytes, void *out,
                                                lia_stream_t stream) {
    static const uint32_t dummy = 0;
    if (!c) return LIA_E_ARG;
    if (c->kv_dtype != LIA_FP8_E4M3) return LIA_E_UNSUPPORTED;
    if (!new_k || !new_v || !slot_mapping) return LIA_E_ARG;
    if (((uintptr_t)new_k | (uintptr_t)new_v) & 15) return LIA_E_ALIGN;
    // every check of both launches before either is issued
    int st = run_stages(kPartial, c, n_seqs, n_rows, &dummy, &dummy, nullptr, pages, q, kc, vc,
                        k_scales, v_scales, workspace, workspace_bytes, out, stream, nullptr, false);
    if (st) return st;
    const lia_kv_layout layout{c->num_kv_heads, c->head_dim, c->page_size, c->pool_pages, LIA_FP8_E4M3};
    st = lia_kv_append(&layout, n_rows, nullptr, nullptr, nullptr, 0, slot_mapping, LIA_BF16, new_k,
                       new_v, kc, vc, k_scales, v_scales, stream);
    if (st) return st;
    return run_stages(kPartial, c, n_seqs, n_rows, &dummy, &dummy, nullptr, pages, q, kc, vc,
                      k_scales, v_scales, workspace, workspace_bytes, out, stream);
}

// The memory access of one lia_attention_partial launch on its own: the plan in `workspace`, the
// same workgroups, block ranges, loads and pipeline waits, without the attention arithmetic.
// Each wave writes the XOR of the words it loaded to sink[workgroup * waves + wave]: the XOR of
// all sink words is the XOR of every attended key's K words (and V words on FP8 pools).
// Batches the decode kernel serves only.
extern "C" int lia_paged_read(const lia_attention_config *c, uint32_t n_seqs, uint32_t n_rows,
                              const uint32_t *pages, const void *q, const void *kc, const void *vc,
                              const float *k_scales, const float *v_scales, void *workspace,
                              size_t workspace_bytes, uint32_t *sink, size_t sink_words,
                              lia_stream_t stream) {
    static const uint32_t dummy = 0;
    int st = validate(c);
    if (st) return st;
    if (n_seqs == 0 || n_seqs > c->max_seqs || n_rows == 0 || n_rows > c->max_rows) return LIA_E_ARG;
    const uint32_t group = c->num_q_heads / c->num_kv_heads;
    if (nt_for(n_rows, n_seqs, group, c->kv_dtype) == kWideNT) return LIA_E_UNSUPPORTED;
    if (!sink) return LIA_E_ARG;
    if (sink_words < lia_paged_read_sink_words(c)) return LIA_E_ARG;
    return run_stages(kRead, c, n_seqs, n_rows, &dummy, &dummy, nullptr, pages, q, kc, vc, k_scales,
                      v_scales, workspace, workspace_bytes, sink, stream);
}

extern "C" size_t lia_paged_read_sink_words(const lia_attention_config *c) {
    if (!c || validate(c)) return 0;
    return (size_t)max_workgroups(c) * (c->head_dim / 64);
}

extern "C" int lia_attention_merge(const lia_attention_config *c, uint32_t n_seqs, uint32_t n_rows,
                                   void *workspace, size_t workspace_bytes, void *out,
                                   lia_stream_t stream) {
    static const uint32_t dummy = 0;
    return run_stages(kMerge, c, n_seqs, n_rows, &dummy, &dummy, nullptr, nullptr, nullptr,
                      nullptr, nullptr, nullptr, nullptr, workspace, workspace_bytes, out, stream);
}

extern "C" size_t lia_static_workspace_bytes(void) { return kStaticWorkspaceBytes; }

extern "C" int lia_paged_attention_static(const lia_attention_config *c, uint32_t n_seqs,
                                          uint32_t n_rows, const uint32_t *cu_seqlens,
                                          const uint32_t *positions, const uint32_t *sequences,
                                          const uint32_t *pages, const void *q, const void *kc,
                                          const void *vc, const float *k_scales,
                                          const float *v_scales, void *out, lia_stream_t stream) {
    int st = validate(c);
    if (st) return st;
    if (lia_attention_workspace_bytes(c) > kStaticWorkspaceBytes) return LIA_E_WORKSPACE;
    void *ws = nullptr;
    st = scratch_of_current_device(&ws);
    if (st) return st;
    return run_stages(kPlan | kPartial | kMerge, c, n_seqs, n_rows, cu_seqlens, positions,
                      sequences, pages, q, kc, vc, k_scales, v_scales, ws, kStaticWorkspaceBytes,
                      out, stream);
}

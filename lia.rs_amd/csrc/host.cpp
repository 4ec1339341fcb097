// Host packing and validation of one continuous-batching step.
// Replaces the host section of Engine::run_paged (src/inference/paging.rs:118-201): the
// same checks in the same order with the same outcomes, producing the flat block table,
// the query groups (cu_seqlens) and the per-row slot mapping that the device kernels read.
#include <stdint.h>
#include <string.h>

#include <unordered_map>
#include <unordered_set>
#include <vector>

#include "../../include/lia_hip.h"

extern "C" uint32_t lia_decode_span(uint32_t tokens) {
    // src/inference/llama.rs:15-26 (the LIA_LLAMA_DECODE_SPAN override is not mirrored)
    if (tokens <= 2048) return 32;
    if (tokens <= 8192) return 64;
    return 160;
}

extern "C" uint32_t lia_decode_parts(uint32_t tokens, uint32_t span) {
    // src/inference/llama.rs:28-35
    if (span == 0) return 0;
    uint32_t count = (tokens + span - 1) / span;
    if (count <= 16) {
        uint32_t p = 1;
        while (p < count) p <<= 1;
        return p;
    }
    return (count + 15) / 16 * 16;
}

extern "C" int lia_pack_rows(const lia_paging_limits *lim, const lia_paged_row *rows,
                             uint32_t n_rows, const uint32_t *table_data,
                             const uint32_t *table_lens, uint32_t n_tables,
                             const uint32_t *outputs, uint32_t n_outputs, uint32_t *positions,
                             uint32_t *sequences, uint32_t *flat_pages, lia_group *groups,
                             uint32_t *cu_seqlens, uint32_t *slot_mapping, lia_pack_info *info) {
    if (!lim || !info || lim->page_size == 0) return LIA_E_ARG;
    const uint32_t P = lim->page_size;
    const uint32_t stride = (lim->context + P - 1) / P; // paging.rs:63
    // paging.rs:120-135
    if (n_rows == 0 || n_rows > lim->prefill_batch) return LIA_E_ROWS;
    if (n_outputs > lim->max_sequences) return LIA_E_OUTPUT_COUNT;
    for (uint32_t i = 0; i < n_outputs; i++)
        if (outputs[i] >= n_rows) return LIA_E_OUTPUT_ROW;
    if (n_tables > lim->max_sequences) return LIA_E_TABLES;
    // paging.rs:136-147
    const size_t flat_len = (size_t)lim->max_sequences * stride;
    for (size_t i = 0; i < flat_len; i++) flat_pages[i] = 0xffffffffu;
    std::vector<size_t> starts(n_tables);
    size_t offset = 0;
    for (uint32_t s = 0; s < n_tables; s++) {
        starts[s] = offset;
        if (table_lens[s] > stride) return LIA_E_TABLE_LEN;
        for (uint32_t p = 0; p < table_lens[s]; p++)
            if (table_data[offset + p] >= lim->pool_pages) return LIA_E_PAGE_RANGE;
        memcpy(flat_pages + (size_t)s * stride, table_data + offset, sizeof(uint32_t) * table_lens[s]);
        offset += table_lens[s];
    }
    // paging.rs:148-186
    std::unordered_set<uint64_t> writes;
    writes.reserve(n_rows * 2);
    std::unordered_map<uint32_t, uint32_t> ordered;
    uint32_t maximum = 0, n_groups = 0;
    bool have_previous = false;
    uint32_t previous_sequence = 0;
    for (uint32_t r = 0; r < n_rows; r++) {
        const uint32_t position = rows[r].position, seq = rows[r].sequence;
        if (rows[r].token >= lim->vocabulary) return LIA_E_TOKEN;
        if (position >= lim->context) return LIA_E_POSITION;
        if (seq >= n_tables) return LIA_E_MISSING_TABLE;
        if (position / P >= table_lens[seq]) return LIA_E_MISSING_PAGE;
        const uint32_t page = table_data[starts[seq] + position / P];
        const uint64_t slot = (uint64_t)page * P + position % P;
        if (!writes.insert(slot).second) return LIA_E_DUPLICATE_SLOT;
        auto found = ordered.find(seq);
        if (found != ordered.end()) {
            if (position != found->second + 1) return LIA_E_NONCONSECUTIVE;
            found->second = position;
        } else {
            ordered.emplace(seq, position);
        }
        if (position + 1 > maximum) maximum = position + 1;
        if (have_previous && previous_sequence == seq) {
            groups[n_groups - 1].count++;
            groups[n_groups - 1].maximum = position + 1;
        } else {
            groups[n_groups].start = r;
            groups[n_groups].count = 1;
            groups[n_groups].maximum = position + 1;
            n_groups++;
            previous_sequence = seq;
            have_previous = true;
        }
        positions[r] = position;
        sequences[r] = seq;
        slot_mapping[r] = (uint32_t)slot;
    }
    for (uint32_t g = 0; g < n_groups; g++) cu_seqlens[g] = groups[g].start;
    cu_seqlens[n_groups] = n_rows;
    // paging.rs:187-201
    bool decoding = n_rows <= 8 && n_outputs == n_rows;
    for (uint32_t i = 0; decoding && i < n_outputs; i++)
        if (outputs[i] != i) decoding = false;
    const uint32_t span = decoding ? lia_decode_span(maximum) : 256;
    info->stride = stride;
    info->maximum = maximum;
    info->decoding = decoding ? 1 : 0;
    info->span = span;
    info->parts = decoding ? lia_decode_parts(maximum, span) : (maximum + span - 1) / span;
    info->n_groups = n_groups;
    return LIA_OK;
}

/* C11 consumer of include/lia_hip.h: prints sizeof and offsetof of every struct the header
 * declares (one "struct field offset size" line each, "struct - 0 sizeof" for the whole), and,
 * when run with an argument, calls a few host entry points of liblia_hip.so linked from C.
 * tests/test_abi_c.py compiles it with gcc -std=c11 -Wall -Werror and compares the printout
 * with the ctypes structures of the Python binding and the Rust #[repr(C)] block. */
#include <stddef.h>
#include <stdio.h>
#include <string.h>

#include "lia_hip.h"

#define F(S, f) printf("%s %s %zu %zu\n", #S, #f, offsetof(S, f), sizeof(((S *)0)->f))
#define WHOLE(S) printf("%s - 0 %zu\n", #S, sizeof(S))

static void layouts(void) {
    F(lia_paged_row, token); F(lia_paged_row, position); F(lia_paged_row, sequence);
    WHOLE(lia_paged_row);
    F(lia_group, start); F(lia_group, count); F(lia_group, maximum);
    WHOLE(lia_group);
    F(lia_paging_limits, max_sequences); F(lia_paging_limits, context);
    F(lia_paging_limits, page_size); F(lia_paging_limits, pool_pages);
    F(lia_paging_limits, vocabulary); F(lia_paging_limits, prefill_batch);
    WHOLE(lia_paging_limits);
    F(lia_pack_info, stride); F(lia_pack_info, maximum); F(lia_pack_info, decoding);
    F(lia_pack_info, span); F(lia_pack_info, parts); F(lia_pack_info, n_groups);
    WHOLE(lia_pack_info);
    F(lia_kv_layout, num_kv_heads); F(lia_kv_layout, head_dim); F(lia_kv_layout, page_size);
    F(lia_kv_layout, pool_pages); F(lia_kv_layout, dtype);
    WHOLE(lia_kv_layout);
    F(lia_kv_planes, n_layers); F(lia_kv_planes, k); F(lia_kv_planes, v);
    F(lia_kv_planes, k_scales); F(lia_kv_planes, v_scales);
    WHOLE(lia_kv_planes);
    F(lia_attention_config, num_q_heads); F(lia_attention_config, num_kv_heads);
    F(lia_attention_config, head_dim); F(lia_attention_config, page_size);
    F(lia_attention_config, pool_pages); F(lia_attention_config, stride);
    F(lia_attention_config, q_dtype); F(lia_attention_config, kv_dtype);
    F(lia_attention_config, out_dtype); F(lia_attention_config, scale);
    F(lia_attention_config, max_seqs); F(lia_attention_config, max_rows);
    F(lia_attention_config, max_context);
    WHOLE(lia_attention_config);
    F(lia_page_io, ctx); F(lia_page_io, page_bytes); F(lia_page_io, load); F(lia_page_io, put);
    F(lia_page_io, read_page); F(lia_page_io, write_pages);
    WHOLE(lia_page_io);
    F(lia_request, tokens); F(lia_request, n_tokens); F(lia_request, computed);
    F(lia_request, sequence); F(lia_request, active); F(lia_request, closed);
    F(lia_request, done); F(lia_request, reserved);
    WHOLE(lia_request);
    F(lia_update, slot); F(lia_update, computed); F(lia_update, output);
    WHOLE(lia_update);
}

/* Host calls through the C ABI (no GPU needed): pack two sequences, size a workspace and hit
 * one validation error of the attention entry point. */
static int calls(void) {
    const lia_paging_limits lim = {4, 64, 16, 8, 1000, 16};
    const lia_paged_row rows[3] = {{5, 16, 0}, {6, 17, 0}, {7, 3, 1}};
    const uint32_t table[3] = {2, 6, 4}; /* sequence 0: pages 2, 6; sequence 1: page 4 */
    const uint32_t lens[2] = {2, 1};
    const uint32_t outputs[2] = {1, 2};
    uint32_t positions[3], sequences[3], flat[16], cu[3], slots[3]; /* flat: max_sequences * stride */
    lia_group groups[3];
    lia_pack_info info;
    memset(&info, 0, sizeof info);
    int st = lia_pack_rows(&lim, rows, 3, table, lens, 2, outputs, 2, positions, sequences, flat,
                           groups, cu, slots, &info);
    printf("pack %d cu %u %u %u slots %u %u %u stride %u groups %u\n", st, cu[0], cu[1], cu[2],
           slots[0], slots[1], slots[2], info.stride, info.n_groups);
    lia_attention_config c = {16, 2, 128, 16, 64, 4, LIA_BF16, LIA_BF16, LIA_BF16, 0.088f, 8, 8, 64};
    printf("workspace %zu\n", lia_attention_workspace_bytes(&c));
    printf("sink_words %zu\n", lia_paged_read_sink_words(&c));
    {
        uint32_t sink = 0;
        printf("read_no_sink %d\n", lia_paged_read(&c, 1, 1, flat, NULL, NULL, NULL, NULL, NULL, NULL, 0,
                                                   NULL, 0, NULL));
        printf("read_short_sink %d\n", lia_paged_read(&c, 1, 1, flat, NULL, NULL, NULL, NULL, NULL, NULL, 0,
                                                      &sink, 1, NULL));
    }
    c.head_dim = 96; /* no kernel for this geometry */
    printf("unsupported %d\n", lia_paged_attention(&c, 1, 1, cu, positions, sequences, flat, NULL,
                                                   NULL, NULL, NULL, NULL, NULL, 0, NULL, NULL));
    printf("null_config %d\n", lia_paged_attention(NULL, 1, 1, cu, positions, sequences, flat, NULL,
                                                   NULL, NULL, NULL, NULL, NULL, 0, NULL, NULL));
    return 0;
}

int main(int argc, char **argv) {
    (void)argv;
    if (argc > 1) return calls();
    layouts();
    return 0;
}

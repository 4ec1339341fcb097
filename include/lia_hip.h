/*
 * lia_hip.h - C ABI of the MI355X (gfx950) paged continuous-batching attention path.
 *
 * Every entry point takes plain pointers and sizes.  Device pointers are HIP device
 * addresses; `stream` is a hipStream_t (NULL = the legacy default stream).  All device
 * entry points are asynchronous on `stream`, perform no allocation and no host
 * synchronisation (so they may be captured in a hipGraph), validate their arguments
 * before launching anything, and return LIA_OK (0) or a negative lia_status.
 *
 * KV pool layout (identical to the reference engine, src/inference/initialize.rs:22-57):
 *   two planes per layer, K and V, each [pool_pages * page_size][num_kv_heads][head_dim]
 *   elements of the KV dtype; physical slot of logical position p of table row s is
 *   pages[s * stride + p / page_size] * page_size + p % page_size
 *   (src/gpu/kernels/llama.rs:174-177).  FP8 pools carry one fp32 scale per
 *   (page, kv head) and plane: k_scales[page * num_kv_heads + head].
 *
 * Query / output layout: [rows][num_q_heads][head_dim] (src/gpu/llama_attention.rs:37-41).
 */
#ifndef LIA_HIP_H
#define LIA_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void *lia_stream_t; /* hipStream_t */

/* Status codes.  The packing codes mirror the ensure! checks of Engine::run_paged
 * (src/inference/paging.rs:120-172) in the order the reference evaluates them. */
enum lia_status {
    LIA_OK = 0,
    LIA_E_ROWS = -1,            /* "invalid packed row count"          paging.rs:120-123 */
    LIA_E_OUTPUT_COUNT = -2,    /* "invalid output row count"          paging.rs:124-127 */
    LIA_E_OUTPUT_ROW = -3,      /* "output row outside packed input"   paging.rs:128-131 */
    LIA_E_TABLES = -4,          /* "too many sequence tables"          paging.rs:132-135 */
    LIA_E_TABLE_LEN = -5,       /* "sequence table exceeds context"    paging.rs:138 */
    LIA_E_PAGE_RANGE = -6,      /* "physical page outside KV pool"     paging.rs:139-144 */
    LIA_E_TOKEN = -7,           /* "invalid packed token"              paging.rs:155 */
    LIA_E_POSITION = -8,        /* "packed position exceeds context"   paging.rs:156 */
    LIA_E_MISSING_TABLE = -9,   /* "missing sequence table"            paging.rs:157-159 */
    LIA_E_MISSING_PAGE = -10,   /* "missing physical KV page"          paging.rs:160-162 */
    LIA_E_DUPLICATE_SLOT = -11, /* "duplicate physical KV write"       paging.rs:163-166 */
    LIA_E_NONCONSECUTIVE = -12, /* "packed positions must be consecutive" paging.rs:167-172 */
    LIA_E_TRANSFER_WINDOW = -13, /* "invalid KV transfer window"     paging_transfer.rs:38-41 */
    LIA_E_TRANSFER_DUPLICATE = -14, /* "duplicate KV transfer destination" paging_transfer.rs:50 */
    LIA_E_PREFIX_EXTENT = -15,  /* "invalid computed prefix extent"    page_cache.rs:209-212 */
    LIA_E_IMMUTABLE_PAGE = -16, /* "attempted to overwrite immutable KV page" page_cache.rs:225-228 */
    LIA_E_PAGE_UNDERFLOW = -17, /* "KV page reference underflow"       page_cache.rs:246 */
    LIA_E_ACTIVE_EVICT = -18,   /* "cannot evict an active KV page"    page_cache.rs:277 */
    LIA_E_CONFIG = -19,         /* configure_paging limits             paging.rs:39-50 */
    LIA_E_ARG = -20,            /* invalid extent / geometry   gpu/llama_attention.rs:36-61 */
    LIA_E_ALIGN = -21,          /* unaligned buffers           gpu/llama_attention.rs:62-68 */
    LIA_E_WORKSPACE = -22,      /* workspace exhausted         gpu/llama_attention.rs:53-61 */
    LIA_E_UNSUPPORTED = -23,    /* geometry this build has no kernel for */
    LIA_E_STORE = -24,          /* a page-store or page-I/O callback failed (positive return) */
    LIA_E_SAMPLER_SETTINGS = -25, /* temperature / top_k / top_p checks  sampling.rs:33-47 */
    LIA_E_SAMPLING_LOGITS = -26,  /* "invalid sampling logits", "invalid sampler logits or normalizer" sampling.rs:88-93, gpu/nucleus.rs:106-109 */
    LIA_E_EMPTY_DISTRIBUTION = -27, /* "empty sampling distribution", "empty greedy vocabulary" sampling.rs:102, paged_sampling.rs:69 */
    LIA_E_DUPLICATE_CANDIDATE = -28, /* "duplicate sampling candidate"   sampling.rs:104-107 */
    LIA_E_NUCLEUS = -29,          /* normalizer / nucleus mass / candidate order / candidate id nucleus.rs:56-74,119, gpu/nucleus.rs:127-130 */
    LIA_E_HIP = -30             /* a HIP runtime call failed */
};

enum lia_dtype { LIA_F32 = 0, LIA_F16 = 1, LIA_BF16 = 2, LIA_FP8_E4M3 = 3 };

/* PagedRow (src/inference/paging.rs:7-11). */
typedef struct lia_paged_row {
    uint32_t token;
    uint32_t position;
    uint32_t sequence;
} lia_paged_row;

/* Query group = one cu_seqlens segment (src/inference/llama_plan.rs:2-6). */
typedef struct lia_group {
    uint32_t start;
    uint32_t count;
    uint32_t maximum; /* last position + 1 */
} lia_group;

/* Limits configured once per engine (Engine::configure_paging, paging.rs:30-93). */
typedef struct lia_paging_limits {
    uint32_t max_sequences; /* 1..=64 in the reference */
    uint32_t context;       /* per-request context, 1..=131072 */
    uint32_t page_size;     /* PAGE_TOKENS (32 in the reference) */
    uint32_t pool_pages;    /* physical pool capacity / page_size */
    uint32_t vocabulary;    /* token ids must be below this */
    uint32_t prefill_batch; /* maximum packed rows */
} lia_paging_limits;

/* Packing result besides the arrays (paging.rs:173-201). */
typedef struct lia_pack_info {
    uint32_t stride;   /* ceil(context / page_size), row stride of the flat table */
    uint32_t maximum;  /* max(position) + 1 over the batch */
    uint32_t decoding; /* rows <= 8 and outputs == 0..rows */
    uint32_t span;     /* split-K span the reference would choose */
    uint32_t parts;    /* split-K parts the reference would choose */
    uint32_t n_groups;
} lia_pack_info;

/*
 * Host packing and validation of one continuous-batching step.
 * Replaces Engine::run_paged's host section (src/inference/paging.rs:118-201).
 * tables: n_tables tables concatenated in table_data, table_lens[i] pages each.
 * Outputs (caller-allocated host arrays):
 *   positions[n_rows], sequences[n_rows], flat_pages[max_sequences * stride] (unused = 0xFFFFFFFF),
 *   groups[n_rows] (first info->n_groups valid), cu_seqlens[n_rows + 1] (n_groups + 1 valid),
 *   slot_mapping[n_rows] = page * page_size + position % page_size.
 * Returns the first failing check's status; outputs are unspecified on error.
 */
int lia_pack_rows(const lia_paging_limits *limits, const lia_paged_row *rows, uint32_t n_rows,
                  const uint32_t *table_data, const uint32_t *table_lens, uint32_t n_tables,
                  const uint32_t *outputs, uint32_t n_outputs, uint32_t *positions,
                  uint32_t *sequences, uint32_t *flat_pages, lia_group *groups,
                  uint32_t *cu_seqlens, uint32_t *slot_mapping, lia_pack_info *info);

/* decode_span / decode_parts (src/inference/llama.rs:15-35) without the env override. */
uint32_t lia_decode_span(uint32_t tokens);
uint32_t lia_decode_parts(uint32_t tokens, uint32_t span);

/*
 * Device packing: builds the per-row metadata of a step on the GPU from per-sequence
 * descriptors, so a step needs no host round trip (the reference stages five arrays and
 * synchronises, paging.rs:224-237).  For batch sequence b (0 <= b < n_seqs):
 *   table row seq_slots[b], q_lens[b] new tokens at positions cached[b] .. cached[b]+q_lens[b]-1.
 * Writes cu_seqlens[n_seqs+1], positions[rows], sequences[rows], slot_mapping[rows].
 * Rows beyond the batch total up to max_rows are left untouched.  status (device, one u32)
 * receives 0 or the first failing lia_status as a positive number (-status), with the
 * reference's checks in its order (paging.rs:120-172):
 *   LIA_E_ROWS           the rows exceed max_rows;
 *   then the tables: every entry the batch attends (logical pages 0 .. ceil((cached + q_len)
 *   / page_size) - 1 of each sequence with rows):
 *   LIA_E_PAGE_RANGE     an entry neither below pool_pages nor 0xFFFFFFFF;
 *   LIA_E_MISSING_PAGE   0xFFFFFFFF wholly below the sequence's cached length;
 *   then per row, the lowest failing row first:
 *   LIA_E_POSITION       position >= context;
 *   LIA_E_MISSING_PAGE   the row's page is 0xFFFFFFFF;
 *   LIA_E_DUPLICATE_SLOT the row's slot is written by an earlier row.
 * On failure cu_seqlens is written all zero and slot_mapping[0 .. max_rows) as 0xFFFFFFFF
 * (the arrays hold max_rows entries), so a plan built
 * from them schedules no work and no append writes the pool: the step's outputs and the pool
 * are left untouched without a host round trip.
 */
int lia_pack_device(uint32_t n_seqs, const uint32_t *seq_slots, const uint32_t *q_lens,
                    const uint32_t *cached, const uint32_t *pages, uint32_t stride,
                    uint32_t page_size, uint32_t pool_pages, uint32_t context, uint32_t max_rows,
                    uint32_t *cu_seqlens, uint32_t *positions, uint32_t *sequences,
                    uint32_t *slot_mapping, uint32_t *status, lia_stream_t stream);

/* KV pool geometry. */
typedef struct lia_kv_layout {
    uint32_t num_kv_heads;
    uint32_t head_dim;   /* 64 or 128 */
    uint32_t page_size;  /* power of two >= 16 */
    uint32_t pool_pages;
    int32_t dtype;       /* LIA_F16, LIA_BF16 or LIA_FP8_E4M3 */
} lia_kv_layout;

/*
 * KV append scatter through the block table.  Replaces llama_cache_paged
 * (src/gpu/kernels/llama.rs:162-183): for row r and element i of its
 * num_kv_heads*head_dim K and V values, writes kc/vc at
 *   (slot(r) * num_kv_heads * head_dim + i)
 * with slot(r) = slot_mapping[r] when slot_mapping != NULL, else computed from
 * positions/sequences/pages/stride exactly as the reference does.  Values are converted
 * from src_dtype (LIA_F32, LIA_F16 or LIA_BF16) to the pool dtype with round-to-nearest-even
 * (FP8: divided by the page's scale first, saturated to +-448; a page whose scale is still 0,
 * never quantised, takes scale 1 and the append writes 1 into k_scales / v_scales).
 */
int lia_kv_append(const lia_kv_layout *layout, uint32_t rows, const uint32_t *positions,
                  const uint32_t *sequences, const uint32_t *pages, uint32_t stride,
                  const uint32_t *slot_mapping, int32_t src_dtype, const void *k, const void *v,
                  void *kc, void *vc, float *k_scales, float *v_scales,
                  lia_stream_t stream);

/*
 * RoPE coefficient table.  Replaces coefficients (src/gpu/kernels/llama_position.rs:36-47),
 * generalised to head_dim 64 / 128: coefficients[r][i] = {cos, sin}(positions[r] * inv_i),
 * inv_i = f32(1 / f32(base^(2i/head_dim))), i < head_dim/2 (the reference's rounded steps;
 * pow/cos/sin evaluated in double and rounded once).  coefficients: [rows][head_dim/2][2]
 * f32, 8-byte aligned.
 */
int lia_rope_coefficients(uint32_t rows, uint32_t head_dim, float base, const uint32_t *positions,
                          float *coefficients, lia_stream_t stream);

/*
 * Fused RoPE + KV append.  Replaces rotary_cache (src/gpu/kernels/llama_position.rs:49-118),
 * generalised to any head counts, head_dim 64 / 128 and every pool type.  input: rows of
 * (num_q_heads + 2 * num_kv_heads) * head_dim f32 = q heads | k heads | v heads.  Each q and
 * k head is rotated by the "rotate half" rule with the coefficient table:
 *   x'[i]       = fma(x[i], cos_i, -f32(x[i + d/2] * sin_i))
 *   x'[i + d/2] = fma(x[i + d/2], cos_i, f32(x[i] * sin_i))       (i < d/2)
 * Rotated queries go to query ([rows][num_q_heads][head_dim], LIA_F32 or LIA_BF16); rotated
 * K and unrotated V are appended exactly as lia_kv_append appends f32 rows (slot_mapping or
 * positions/sequences/pages/stride; FP8 pools divide by the page scale, a scale of 0 taking 1
 * as in lia_kv_append).  input, query and
 * coefficients 16-byte aligned.
 */
int lia_rope_kv_append(const lia_kv_layout *layout, uint32_t num_q_heads, uint32_t rows,
                       const uint32_t *positions, const uint32_t *sequences, const uint32_t *pages,
                       uint32_t stride, const uint32_t *slot_mapping, const float *coefficients,
                       const float *input, void *query, int32_t query_dtype, void *kc, void *vc,
                       float *k_scales, float *v_scales, lia_stream_t stream);

/*
 * FP8 page quantisation: converts n_pages whole pages (page ids in page_ids) of K and V
 * given as [n_pages][page_size][num_kv_heads][head_dim] in src_dtype into the e4m3 pool,
 * computing each (page, head) scale as amax / 448 (1 when the page is all zero).
 * No counterpart in the reference (its KV cache is f16 only).
 */
int lia_kv_quantize_pages(const lia_kv_layout *layout, uint32_t n_pages, const uint32_t *page_ids,
                          int32_t src_dtype, const void *k, const void *v, void *kc, void *vc,
                          float *k_scales, float *v_scales, lia_stream_t stream);

/*
 * Output-row gather: dst[i] = src[indices[i]] for rows of `width` 32-bit words (count rows).
 * Replaces llama_gather_hidden (src/gpu/kernels/llama.rs:186-198), which selects the hidden
 * rows of the requested outputs before the LM head.  indices must lie inside src.
 */
int lia_gather_rows(uint32_t count, uint32_t width, const uint32_t *indices, const void *src,
                    void *dst, lia_stream_t stream);

/*
 * KV page transfer in the reference's page wire format.  A page payload is one physical page
 * of every layer and plane, layer-major: [layer][K, V][page_size][num_kv_heads][head_dim] pool
 * elements (MINICPM5_PAGE_BYTES = 42 x 2 x 32 x 256 x 2, src/inference/paging_transfer.rs:4),
 * followed for FP8 pools by [layer][K, V][num_kv_heads] f32 page scales.
 *   lia_kv_page_bytes:     bytes of one payload.
 *   lia_kv_transfer_bytes: bytes of the staging buffers (a header + up to 16 payloads); the
 *                          caller allocates one in pinned host memory and one on the device.
 *   lia_kv_write_pages:    write_kv_pages (paging_transfer.rs:37-58 with the pinned upload of
 *                          paging_upload.rs:23-104): copies the payloads into the host staging
 *                          buffer, one host-to-device copy, one scatter kernel.
 *   lia_kv_read_pages:     read_kv_page for up to 16 pages (transfer_kv_pages_raw,
 *                          paging_transfer.rs:75-177): one gather kernel, one device-to-host
 *                          copy, then payload i is copied out to payloads[i].
 * 1 to 16 distinct pages, each below pool_pages (the reference's checks, in its order).  Both
 * are ordered after earlier work on `stream` and synchronise it before returning, as the
 * reference does; staging_host (pinned) and staging_device are scratch the caller owns, used
 * by one call at a time.
 */
#define LIA_MAX_LAYERS 128
typedef struct lia_kv_planes {
    uint32_t n_layers;
    void *k[LIA_MAX_LAYERS];         /* device base of each layer's K plane */
    void *v[LIA_MAX_LAYERS];
    float *k_scales[LIA_MAX_LAYERS]; /* FP8 pools only */
    float *v_scales[LIA_MAX_LAYERS];
} lia_kv_planes;

size_t lia_kv_page_bytes(const lia_kv_layout *layout, uint32_t n_layers);
size_t lia_kv_transfer_bytes(const lia_kv_layout *layout, uint32_t n_layers);
int lia_kv_write_pages(const lia_kv_layout *layout, const lia_kv_planes *planes, uint32_t n_pages,
                       const uint32_t *page_ids, const void *const *payloads, void *staging_host,
                       void *staging_device, lia_stream_t stream);
int lia_kv_read_pages(const lia_kv_layout *layout, const lia_kv_planes *planes, uint32_t n_pages,
                      const uint32_t *page_ids, void *const *payloads, void *staging_host,
                      void *staging_device, lia_stream_t stream);

/* Geometry and capacity of one paged-attention engine. */
typedef struct lia_attention_config {
    uint32_t num_q_heads;
    uint32_t num_kv_heads;
    uint32_t head_dim;    /* 64 or 128 */
    uint32_t page_size;   /* power of two >= 16 */
    uint32_t pool_pages;
    uint32_t stride;      /* table row stride (pages per sequence) */
    int32_t q_dtype;      /* LIA_F32 or LIA_BF16 */
    int32_t kv_dtype;     /* LIA_F16, LIA_BF16 or LIA_FP8_E4M3 */
    int32_t out_dtype;    /* LIA_F32 or LIA_BF16 */
    float scale;          /* softmax scale, 1/sqrt(head_dim) in the reference */
    uint32_t max_seqs;    /* capacity of cu_seqlens - 1 */
    uint32_t max_rows;    /* capacity of the packed rows */
    uint32_t max_context; /* largest key count of one sequence */
} lia_attention_config;

/* Bytes of device workspace lia_paged_attention needs.  Replaces llama::workspace
 * (src/inference/llama.rs:37-43). */
size_t lia_attention_workspace_bytes(const lia_attention_config *config);

/*
 * Paged causal GQA attention over one ragged packed batch: decode rows, MTP-verify rows
 * (several consecutive rows of one sequence) and chunked / prefix-cached prefill chunks
 * in any mix.  Replaces the tile loop of llama_attention_selected together with
 * gpu::llama_attention::{partial, merge} (src/inference/llama.rs:253-288,
 * src/gpu/llama_attention.rs:24-207).
 * Batch sequence b owns rows cu_seqlens[b] .. cu_seqlens[b+1]-1, all of table row
 * sequences[cu_seqlens[b]], with consecutive positions; row r attends keys
 * 0 ..= positions[r] of its sequence (the reference's per-row causal limit,
 * src/gpu/kernels/llama_flash_kernel.rs:145-154).  The new rows' K/V must already be
 * appended.  Output: out[r][h][d] = softmax(q.K^T * scale) V in out_dtype.
 */
int lia_paged_attention(const lia_attention_config *config, uint32_t n_seqs, uint32_t n_rows,
                        const uint32_t *cu_seqlens, const uint32_t *positions,
                        const uint32_t *sequences, const uint32_t *pages, const void *q,
                        const void *kc, const void *vc, const float *k_scales,
                        const float *v_scales, void *workspace, size_t workspace_bytes,
                        void *out, lia_stream_t stream);

/*
 * The three stages of lia_paged_attention, for callers that share one plan across layers
 * (the metadata of a step is the same for every layer) and for timing the stages apart.
 *   lia_attention_plan:    builds the step's work list in the workspace from cu_seqlens,
 *                          positions and sequences (replaces the host planning of
 *                          llama_plan::tiles, src/inference/llama_plan.rs:16-101); the
 *                          other two stages read the per-row metadata from it.  When pages
 *                          is not NULL the plan also copies the first block-table entries of
 *                          every workgroup's range into the work list, so the table must not
 *                          change between the plan and the partial calls that use it.
 *   lia_attention_partial: the split attention kernel; units covered by one workgroup are
 *                          written normalised to out, the others leave partial records
 *                          (replaces gpu::llama_attention::partial, llama_attention.rs:24-159).
 *   lia_attention_merge:   combines the partial records into out (replaces
 *                          gpu::llama_attention::merge, llama_attention.rs:163-207).
 * n_seqs / n_rows must be the same in all three calls of one plan, and cu_seqlens must describe
 * exactly n_rows rows (cu_seqlens[n_seqs] == n_rows, as lia_pack_rows / lia_pack_device write
 * it).  Device metadata is not read back by the host: a plan whose rows would need more
 * units than the workspace was sized for schedules no work, and out is left unwritten.
 */
int lia_attention_plan(const lia_attention_config *config, uint32_t n_seqs, uint32_t n_rows,
                       const uint32_t *cu_seqlens, const uint32_t *positions,
                       const uint32_t *sequences, const uint32_t *pages, void *workspace,
                       size_t workspace_bytes, lia_stream_t stream);
/*
 * lia_pack_device followed by lia_attention_plan (with pages) on one workspace, in two launches
 * instead of three: the packing, the table checks and the plan - built from the packing's inputs
 * (seq_slots, q_lens, cached) - run side by side, then one small launch settles the status.  The metadata,
 * status and plan afterwards are those of the two calls, with the config's stride, page_size,
 * pool_pages and max_rows as the packing's.  A rejected step (status != 0) is marked in the
 * workspace, and the attention and merge entry points then read and write nothing for it, as
 * they would on the empty plan of a rejected packing.  n_rows must equal the sum of q_lens;
 * otherwise nothing is scheduled.  Batches of more than 1024 sequences take the three launches.
 * No counterpart in the reference, which packs on the host (paging.rs:118-201).
 */
int lia_pack_plan_device(const lia_attention_config *config, uint32_t n_seqs, uint32_t n_rows,
                         const uint32_t *seq_slots, const uint32_t *q_lens, const uint32_t *cached,
                         const uint32_t *pages, uint32_t context, uint32_t *cu_seqlens,
                         uint32_t *positions, uint32_t *sequences, uint32_t *slot_mapping,
                         uint32_t *status, void *workspace, size_t workspace_bytes,
                         lia_stream_t stream);
int lia_attention_partial(const lia_attention_config *config, uint32_t n_seqs, uint32_t n_rows,
                          const uint32_t *pages, const void *q, const void *kc, const void *vc,
                          const float *k_scales, const float *v_scales, void *workspace,
                          size_t workspace_bytes, void *out, lia_stream_t stream);
int lia_attention_merge(const lia_attention_config *config, uint32_t n_seqs, uint32_t n_rows,
                        void *workspace, size_t workspace_bytes, void *out, lia_stream_t stream);

/*
 * lia_kv_append of this step's rows (slot_mapping form, source dtype = pool dtype) fused
 * into lia_attention_partial: one launch does both.  Replaces the per-layer pair
 * llama_cache_paged + paged attention of the reference forward (src/gpu/kernels/llama.rs:162-183
 * followed by src/inference/llama.rs:253-288).  new_k / new_v: [n_rows][num_kv_heads][head_dim]
 * in the pool dtype (LIA_F16 or LIA_BF16; FP8 pools: lia_attention_partial_append_fp8), 16-byte
 * aligned.  The plan must come from the same packed rows: the first row of each sequence
 * sits at the sequence's cached length and its rows' keys are read from new_k / new_v, the
 * cached keys from the pool.  The pool afterwards holds the same bytes lia_kv_append
 * writes.  No cached key of any sequence may live in a slot this step writes (the
 * reference's page ownership guarantees it: packing rejects duplicate slots and new rows
 * go to the sequence's own pages).
 */
int lia_attention_partial_append(const lia_attention_config *config, uint32_t n_seqs,
                                 uint32_t n_rows, const uint32_t *pages,
                                 const uint32_t *slot_mapping, const void *q, const void *new_k,
                                 const void *new_v, void *kc, void *vc, void *workspace,
                                 size_t workspace_bytes, void *out, lia_stream_t stream);

/*
 * lia_attention_partial_append for FP8 pools: the step's rows new_k / new_v are bf16
 * ([n_rows][num_kv_heads][head_dim], 16-byte aligned) and are appended exactly as
 * lia_kv_append(src_dtype = LIA_BF16) appends them - divided by the scale of their page,
 * rounded to e4m3 (saturating), a page whose scale is still 0 taking scale 1 and recording
 * it in k_scales / v_scales - then attended from the pool (two launches on `stream`; every
 * argument is checked before either is issued).  Other pool types return LIA_E_UNSUPPORTED
 * (and lia_attention_partial_append returns it for FP8 pools).  No counterpart in the
 * reference, whose KV cache is f16 only.
 * Ranges on FP8 pools (every attention entry point): the kernels multiply e4m3 codes, converted
 * exactly to f16, by f16 softmax weights of at most 2^8 times the page's V scale, so V page
 * scales must stay below 256 (a V amax below about 114,000; amax/448 is the quantiser's scale)
 * for the weights to stay finite, and weights of pages whose scale is below about 2^-14 lose
 * precision as f16 subnormals.  Queries are rounded to f16 on FP8 pools: |q| above 65504 becomes
 * infinite.  16-bit pools keep bf16 queries and weights and have neither limit.
 */
int lia_attention_partial_append_fp8(const lia_attention_config *config, uint32_t n_seqs,
                                     uint32_t n_rows, const uint32_t *pages,
                                     const uint32_t *slot_mapping, const void *q,
                                     const void *new_k, const void *new_v, void *kc, void *vc,
                                     float *k_scales, float *v_scales, void *workspace,
                                     size_t workspace_bytes, void *out, lia_stream_t stream);

/*
 * The memory access of one lia_attention_partial launch on its own: over the plan already in
 * `workspace` (lia_attention_plan or lia_pack_plan_device), the same workgroups, block ranges,
 * K/V loads and pipeline waits as the decode kernel, with the attention arithmetic, the
 * score exchange and the outputs left out.  Each wave writes the XOR of the words it loaded
 * to sink[workgroup * (head_dim / 64) + wave]; the XOR of all sink words is the XOR of every
 * attended key's K words, and on FP8 pools of its V words too (16-bit pools load V straight
 * into LDS).  No counterpart in the reference: it measures the rate of the kernel's own
 * paged access pattern, the ceiling the decode kernel is compared with.  Batches served by
 * the decode kernel (LIA_E_UNSUPPORTED for a prefill batch); FP8 pools take their scales as
 * lia_attention_partial does; sink 4-byte aligned and at least
 * lia_paged_read_sink_words(config) words.
 */
int lia_paged_read(const lia_attention_config *config, uint32_t n_seqs, uint32_t n_rows,
                   const uint32_t *pages, const void *q, const void *kc, const void *vc,
                   const float *k_scales, const float *v_scales, void *workspace,
                   size_t workspace_bytes, uint32_t *sink, size_t sink_words, lia_stream_t stream);

/* Words of the sink lia_paged_read needs for a configuration (0 for an invalid one). */
size_t lia_paged_read_sink_words(const lia_attention_config *config);

/*
 * Read-only HBM stream over [src, src + bytes): `workgroups` workgroups each read one
 * contiguous share with 16-byte non-temporal loads and write one word (the XOR of what they
 * read) to sink[workgroup].  No counterpart in the reference: it measures, on the same device,
 * the rate of a contiguous read of as many bytes as an attention launch reads - the ceiling the
 * HBM-bound kernels are compared with.  src 16-byte aligned; a share above 4 GiB returns
 * LIA_E_UNSUPPORTED.
 */
int lia_hbm_read(const void *src, size_t bytes, uint32_t workgroups, uint32_t *sink,
                 lia_stream_t stream);

/*
 * lia_paged_attention without a workspace argument: the work list and split records live in
 * a device array the library holds for the process (lia_static_workspace_bytes() bytes on each
 * device it runs on), so the call allocates nothing.  No counterpart in the reference: this
 * entry point is for callers that cannot allocate (code under hipGraph capture, tight serving
 * loops, harnesses that forbid hipMalloc).  A configuration whose workspace
 * (lia_attention_workspace_bytes) exceeds the array is rejected with LIA_E_WORKSPACE.  Calls
 * that overlap on one device share the array and race: serialise them (one stream, or events).
 * Same arguments, results and errors as lia_paged_attention otherwise.
 */
int lia_paged_attention_static(const lia_attention_config *config, uint32_t n_seqs,
                               uint32_t n_rows, const uint32_t *cu_seqlens,
                               const uint32_t *positions, const uint32_t *sequences,
                               const uint32_t *pages, const void *q, const void *kc,
                               const void *vc, const float *k_scales, const float *v_scales,
                               void *out, lia_stream_t stream);
size_t lia_static_workspace_bytes(void);

/* Number of compute units of the calling thread's current device, which the library
 * schedules decode work for (cached per device).  0 on failure. */
uint32_t lia_device_cus(void);

/* Optional set-up of one device, the counterpart of loading the kernels' module once
 * (src/gpu/llama_attention.rs:24,163 take the loaded `module`): makes `device` current,
 * caches its compute-unit count, looks up its static workspace (lia_paged_attention_static)
 * and resolves every kernel of the library's gfx950 code object on it (hipGetFuncBySymbol).
 * Every launch goes through hipModuleLaunchKernel on those functions; a device not set up
 * here resolves each function on its first launch instead.  LIA_OK, or LIA_E_HIP. */
int lia_init(int device);

/*
 * Host page manager (src/inference/page_cache.rs:48-304): reference-counted physical pages of
 * page_size tokens, content-addressed by the prefix key chain of src/prefix_cache.rs:61-70
 * (SHA-256 of "lia-kv-prefix-v1" | parent key | token count u64 LE | tokens u32 LE; the first
 * parent is the caller's 32-byte namespace), with least-recently-used eviction of idle
 * immutable pages.  Not thread-safe: one thread drives a cache, as the reference's single
 * inference thread does.
 *
 * The page store (RAM/SSD tiers) and the KV pool are reached through callbacks, each
 * returning 0 on success or a negative status (a positive return reads as LIA_E_STORE):
 *   load:        look up a prefix page: 1 and *payload (page_bytes, valid until the next
 *                write_pages call returns) on a hit, 0 on a miss.  NULL: every lookup misses.
 *   put:         keep an evicted page's payload under its key.  NULL: evicted pages are dropped.
 *   read_page:   Engine::read_kv_page - needed when put is set.
 *   write_pages: Engine::write_kv_pages for up to 16 restored pages.
 */
typedef struct lia_page_io {
    void *ctx;
    size_t page_bytes;
    int (*load)(void *ctx, const uint8_t *key, const void **payload);
    int (*put)(void *ctx, const uint8_t *key, const void *payload);
    int (*read_page)(void *ctx, uint32_t page, void *payload);
    int (*write_pages)(void *ctx, uint32_t n, const uint32_t *pages, const void *const *payloads);
} lia_page_io;

typedef struct lia_page_cache lia_page_cache; /* PageCache */
typedef struct lia_sequence lia_sequence;     /* page_cache::Sequence: pages + sealed keys */

/* Key::prefix (prefix_cache.rs:61-70). */
int lia_prefix_key(const uint8_t parent[32], const uint32_t *tokens, size_t n_tokens, uint8_t out[32]);
/* PageCache::new (page_cache.rs:29-44); an empty pool is LIA_E_CONFIG. */
int lia_page_cache_create(const uint8_t ns[32], uint32_t n_pages, uint32_t page_size,
                          const lia_page_io *io, lia_page_cache **out);
void lia_page_cache_destroy(lia_page_cache *cache);
/* PageCache::attach (page_cache.rs:48-157): *cached = tokens already resident or restored. */
int lia_page_cache_attach(lia_page_cache *cache, const uint32_t *tokens, size_t n_tokens,
                          lia_sequence **sequence, size_t *cached);
/* PageCache::can_fit (page_cache.rs:163-180): 1 or 0. */
int lia_page_cache_can_fit(const lia_page_cache *cache, const uint32_t *tokens, size_t n_tokens);
/* PageCache::available_pages (page_cache.rs:159-161). */
size_t lia_page_cache_available(const lia_page_cache *cache);
/* PageCache::ensure_position (page_cache.rs:183-206): 1, 0 when the pool is occupied, or < 0. */
int lia_page_cache_ensure_position(lia_page_cache *cache, lia_sequence *sequence, size_t position);
/* PageCache::seal (page_cache.rs:208-237). */
int lia_page_cache_seal(lia_page_cache *cache, lia_sequence *sequence, const uint32_t *tokens,
                        size_t n_tokens, size_t computed);
/* PageCache::release (page_cache.rs:239-244); frees the handle. */
int lia_page_cache_release(lia_page_cache *cache, lia_sequence *sequence);
/* PageCache::evict_idle (page_cache.rs:255-262). */
int lia_page_cache_evict_idle(lia_page_cache *cache);
void lia_page_cache_stats(const lia_page_cache *cache, uint64_t *gpu_hits, uint64_t *evictions);
/* The sequence's block-table row (Sequence::pages); valid until the next call on it. */
uint32_t lia_sequence_pages(const lia_sequence *sequence, const uint32_t **pages);

/* One active slot of the paged runtime (src/server/paged/request.rs). */
typedef struct lia_request {
    const uint32_t *tokens;
    size_t n_tokens;
    size_t computed;          /* tokens already in the KV pool */
    lia_sequence *sequence;
    int32_t active;           /* slot holds a request */
    int32_t closed;           /* its output stream is closed: marked done, no rows */
    int32_t done;             /* out */
    int32_t reserved;
} lia_request;

typedef struct lia_update {
    uint32_t slot;
    uint64_t computed;
    uint32_t output;          /* 1 when the step's last row of this slot produces logits */
} lia_update;

/* Runtime::step row construction (src/server/paged/schedule.rs:5-60): rows for
 * lia_pack_rows, output row indices and per-slot updates; LIA_E_ROWS beyond max_rows. */
int lia_schedule_rows(lia_page_cache *cache, uint32_t n_slots, lia_request *requests,
                      uint32_t prefill_batch, lia_paged_row *rows, uint32_t max_rows,
                      uint32_t *n_rows, uint32_t *outputs, uint32_t *n_outputs,
                      lia_update *updates, uint32_t *n_updates);

/*
 * Sparse sampling of the paged step's output rows (Engine::forward_paged_sampled,
 * src/inference/paged_sampling.rs:7-76).
 *   lia_sampler_*: Sampling (src/sampling.rs:19-190): temperature, top_k 0..20, top_p (0,1],
 *     MT19937 stream from the seed, or position-keyed Gumbel draws (with_position_gumbel).
 *   lia_nucleus_candidates: llama_nucleus_candidates (src/gpu/kernels/llama_nucleus.rs:18-117):
 *     per row and 1024-entry part, 21 (id << 32 | f32 bits) words by descending total order
 *     (ties: larger id) and (max, f64 mass) normalizers.  Device pointers, async on stream.
 *   lia_sample_host: the host tail on host copies of those records (logits: the full rows,
 *     read only for a nucleus fallback).
 *   lia_sample_paged: the whole tail: temperatures up, kernel, records down, per-row
 *     sampling, full-row reads for fallbacks; synchronises the stream (as the reference).
 *     workspace (device) and host buffers of lia_nucleus_workspace_bytes / _host_bytes.
 * samplers[i] == NULL selects greedy for output row i; positions[i] is the row's position
 * (Sampling::set_position).  *fallbacks counts full-row reads (nucleus_fallbacks).
 */
typedef struct lia_sampler lia_sampler;
int lia_sampler_create(double temperature, uint32_t top_k, double top_p, uint64_t seed,
                       int32_t position_keyed, lia_sampler **out);
void lia_sampler_destroy(lia_sampler *sampler);
void lia_sampler_set_position(lia_sampler *sampler, uint64_t position);
/* Sampling::distribution over (ids, logits): n_out entries sorted as the reference sorts. */
int lia_sampler_distribution(const lia_sampler *sampler, uint32_t n, const uint32_t *ids,
                             const float *logits, uint32_t *out_ids, double *out_probs,
                             uint32_t *n_out);
/* Sampling::draw. */
int lia_sampler_draw(lia_sampler *sampler, uint32_t n, const uint32_t *ids, const double *probs,
                     uint32_t *token);
size_t lia_nucleus_workspace_bytes(uint32_t vocab, uint32_t rows);
size_t lia_nucleus_host_bytes(uint32_t vocab, uint32_t rows);
int lia_nucleus_candidates(uint32_t vocab, uint32_t rows, const double *temperatures,
                           const float *logits, uint64_t *candidates, double *normalizers,
                           lia_stream_t stream);
int lia_sample_host(uint32_t vocab, uint32_t n, lia_sampler *const *samplers,
                    const uint32_t *positions, const uint64_t *candidates,
                    const double *normalizers, const float *logits, uint32_t *tokens,
                    uint64_t *fallbacks);
int lia_sample_paged(uint32_t vocab, uint32_t n, lia_sampler *const *samplers,
                     const uint32_t *positions, const float *logits, void *workspace,
                     size_t workspace_bytes, void *host, size_t host_bytes, uint32_t *tokens,
                     uint64_t *fallbacks, lia_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* LIA_HIP_H */

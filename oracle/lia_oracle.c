/*
 * lia_oracle.c - CPU restatement of the reference engine's paged attention hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker for the HIP library under
 * lia.rs_amd/csrc and the CPU baseline timed by bench.py; nothing in the product path
 * links, loads or calls it.
 *
 * Each function cites the reference (Heltion/lia.rs) file:line whose semantics it
 * restates.  The reference is Rust + NVIDIA cuda-rust and cannot be compiled in this
 * image, so these restatements are pinned instead by the reference's own known-answer
 * vectors (tests/test_oracle.py) and by mathematical properties.
 *
 * Pinning status per function:
 *   lo_f32_to_f16/bf16/e4m3, decoders ... pinned (exhaustive / IEEE closed forms, numpy)
 *   lo_pack_rows ........................ pinned (error cases of paging.rs, brute force)
 *   lo_kv_append ........................ pinned (closed-form addressing, brute force)
 *   lo_attention_f64 .................... pinned (reference f64 oracle vectors,
 *                                          llama_attention.rs:212-284; numpy softmax)
 *   lo_attention_partial + lo_merge ..... pinned (merge of any split equals unsplit f64
 *                                          result; llama_merge.rs:91-108 vectors)
 *   lo_paged_attention_f32 .............. pinned (against lo_attention_f64)
 *   lo_coefficients / lo_rope /
 *   lo_rotary_cache ..................... pinned for addressing and the rounding order
 *                                          (fused == separate, llama_position.rs:128-239);
 *                                          pow/cos/sin in double rounded once to f32 (a
 *                                          float64 check pins the steps): the bits of the
 *                                          reference's device math are parity unpinned
 *   lo_rope_kv_append ................... pinned (equals lo_rotary_cache on the reference
 *                                          geometry; equals rope + lo_kv_append elsewhere);
 *                                          the rotation by mathematics: position 0 is the
 *                                          identity, pair norms are kept, basis vectors map
 *                                          to the rotate-half (cos, sin) columns, and q.k
 *                                          depends only on the position difference
 *   exp bits (ex2.approx in the reference) parity unpinned, tolerance-pinned only
 */
#include <math.h>
#include <omp.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "../include/lia_hip.h"

/* ------------------------------------------------------------------------------------ */
/* Scalar conversions.  IEEE-754 round-to-nearest-even, written from the format          */
/* definitions (binary16, bfloat16 = upper half of binary32, OCP FP8 E4M3FN).            */
/* ------------------------------------------------------------------------------------ */

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

uint16_t lo_f32_to_f16(float f) {
    uint32_t x = f2u(f);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u); /* NaN -> quiet NaN */
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520 rounds to inf */
    if (ax < 0x38800000u) {                                  /* below 2^-14: subnormal */
        uint32_t e = ax >> 23;
        if (e < 102) return (uint16_t)sign; /* < 2^-25: rounds to zero */
        uint32_t m = (ax & 0x7fffffu) | 0x800000u;
        uint32_t shift = 126 - e; /* value / 2^-24 = m >> shift */
        uint32_t q = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1);
        uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (q & 1))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t r = ax - (112u << 23); /* rebias exponent 127 -> 15 */
    r += 0xfffu + ((r >> 13) & 1u);
    return (uint16_t)(sign | (r >> 13));
}

float lo_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1f;
    uint32_t m = h & 0x3ff;
    if (e == 0) {
        float v = (float)m * 5.9604644775390625e-08f; /* 2^-24 */
        return (sign ? -v : v);
    }
    if (e == 31) return u2f(sign | 0x7f800000u | (m << 13));
    return u2f(sign | ((e + 112) << 23) | (m << 13));
}

uint16_t lo_f32_to_bf16(float f) {
    uint32_t x = f2u(f);
    if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)(((x >> 16) & 0x8000u) | 0x7fc0u);
    x += 0x7fffu + ((x >> 16) & 1u);
    return (uint16_t)(x >> 16);
}

float lo_bf16_to_f32(uint16_t b) { return u2f((uint32_t)b << 16); }

/* OCP E4M3FN: bias 7, no infinities, 0x7f/0xff = NaN, max finite 448.
 * Saturating (finite inputs beyond +-448 -> +-448, NaN -> 0x7f). */
uint8_t lo_f32_to_e4m3(float f) {
    uint32_t x = f2u(f);
    uint8_t sign = (uint8_t)((x >> 24) & 0x80u);
    uint32_t ax = x & 0x7fffffffu;
    if (ax > 0x7f800000u) return 0x7f;
    if (ax >= 0x43e00000u) return (uint8_t)(sign | 0x7e); /* >= 448 */
    if (ax < 0x3c800000u) {                               /* < 2^-6: subnormal grid 2^-9 */
        float q = nearbyintf(u2f(ax) * 512.0f);           /* exact scaling, RNE */
        return (uint8_t)(sign | (uint8_t)q);              /* q == 8 encodes 2^-6 */
    }
    uint32_t r = ax + 0x7ffffu + ((ax >> 20) & 1u); /* RNE to 3 mantissa bits */
    uint32_t code = (r >> 20) - (120u << 3);         /* rebias 127 -> 7 */
    if (code > 0x7e) code = 0x7e;
    return (uint8_t)(sign | code);
}

float lo_e4m3_to_f32(uint8_t b) {
    uint32_t e = (b >> 3) & 0xf, m = b & 7;
    float v;
    if (e == 0xf && m == 7) return NAN;
    if (e == 0) v = (float)m * 0.001953125f; /* 2^-9 */
    else v = u2f(((e + 120) << 23) | (m << 20));
    return (b & 0x80) ? -v : v;
}

static inline float load_elem(const void *base, size_t i, int dtype) {
    switch (dtype) {
    case LIA_F32: return ((const float *)base)[i];
    case LIA_F16: return lo_f16_to_f32(((const uint16_t *)base)[i]);
    case LIA_BF16: return lo_bf16_to_f32(((const uint16_t *)base)[i]);
    case LIA_FP8_E4M3: return lo_e4m3_to_f32(((const uint8_t *)base)[i]);
    }
    return NAN;
}

/* ------------------------------------------------------------------------------------ */
/* Packing and validation: Engine::run_paged, src/inference/paging.rs:118-201.           */
/* ------------------------------------------------------------------------------------ */

/* decode_span, src/inference/llama.rs:15-26 (without LIA_LLAMA_DECODE_SPAN). */
uint32_t lo_decode_span(uint32_t tokens) { return tokens <= 2048 ? 32 : tokens <= 8192 ? 64 : 160; }

/* decode_parts, src/inference/llama.rs:28-35. */
uint32_t lo_decode_parts(uint32_t tokens, uint32_t span) {
    uint32_t count = (tokens + span - 1) / span;
    if (count <= 16) {
        uint32_t p = 1;
        while (p < count) p <<= 1;
        return p;
    }
    return (count + 15) / 16 * 16;
}

static int cmp_u32(const void *a, const void *b) {
    uint32_t x = *(const uint32_t *)a, y = *(const uint32_t *)b;
    return x < y ? -1 : x > y;
}

int lo_pack_rows(const lia_paging_limits *lim, const lia_paged_row *rows, uint32_t n_rows,
                 const uint32_t *table_data, const uint32_t *table_lens, uint32_t n_tables,
                 const uint32_t *outputs, uint32_t n_outputs, uint32_t *positions,
                 uint32_t *sequences, uint32_t *flat, lia_group *groups, uint32_t *cu_seqlens,
                 uint32_t *slot_mapping, lia_pack_info *info) {
    uint32_t P = lim->page_size;
    uint32_t stride = (lim->context + P - 1) / P; /* paging.rs:63 */
    /* paging.rs:120-135 */
    if (n_rows == 0 || n_rows > lim->prefill_batch) return LIA_E_ROWS;
    if (n_outputs > lim->max_sequences) return LIA_E_OUTPUT_COUNT;
    for (uint32_t i = 0; i < n_outputs; i++)
        if (outputs[i] >= n_rows) return LIA_E_OUTPUT_ROW;
    if (n_tables > lim->max_sequences) return LIA_E_TABLES;
    /* paging.rs:136-147: flat table padded with u32::MAX */
    for (size_t i = 0; i < (size_t)lim->max_sequences * stride; i++) flat[i] = 0xffffffffu;
    size_t offset = 0;
    size_t *table_start = (size_t *)malloc(sizeof(size_t) * (n_tables + 1));
    for (uint32_t s = 0; s < n_tables; s++) {
        table_start[s] = offset;
        if (table_lens[s] > stride) { free(table_start); return LIA_E_TABLE_LEN; }
        for (uint32_t p = 0; p < table_lens[s]; p++)
            if (table_data[offset + p] >= lim->pool_pages) { free(table_start); return LIA_E_PAGE_RANGE; }
        memcpy(flat + (size_t)s * stride, table_data + offset, sizeof(uint32_t) * table_lens[s]);
        offset += table_lens[s];
    }
    /* paging.rs:148-186: slot uniqueness, consecutive positions, groups */
    uint32_t *slots_seen = (uint32_t *)malloc(sizeof(uint32_t) * n_rows);
    uint32_t *last_pos = (uint32_t *)malloc(sizeof(uint32_t) * (n_tables ? n_tables : 1));
    uint8_t *has_last = (uint8_t *)calloc(n_tables ? n_tables : 1, 1);
    int status = LIA_OK;
    uint32_t maximum = 0, n_groups = 0;
    int64_t previous_sequence = -1;
    for (uint32_t r = 0; r < n_rows && status == LIA_OK; r++) {
        uint32_t position = rows[r].position, seq = rows[r].sequence;
        if (rows[r].token >= lim->vocabulary) { status = LIA_E_TOKEN; break; }
        if (position >= lim->context) { status = LIA_E_POSITION; break; }
        if (seq >= n_tables) { status = LIA_E_MISSING_TABLE; break; }
        if (position / P >= table_lens[seq]) { status = LIA_E_MISSING_PAGE; break; }
        uint32_t page = table_data[table_start[seq] + position / P];
        uint32_t slot = page * P + position % P;
        for (uint32_t j = 0; j < r; j++)
            if (slots_seen[j] == slot) { status = LIA_E_DUPLICATE_SLOT; break; }
        if (status != LIA_OK) break;
        slots_seen[r] = slot;
        if (has_last[seq] && position != last_pos[seq] + 1) { status = LIA_E_NONCONSECUTIVE; break; }
        has_last[seq] = 1;
        last_pos[seq] = position;
        if (position + 1 > maximum) maximum = position + 1;
        if (previous_sequence == (int64_t)seq) {
            groups[n_groups - 1].count++;
            groups[n_groups - 1].maximum = position + 1;
        } else {
            groups[n_groups].start = r;
            groups[n_groups].count = 1;
            groups[n_groups].maximum = position + 1;
            n_groups++;
            previous_sequence = seq;
        }
        positions[r] = position;
        sequences[r] = seq;
        slot_mapping[r] = slot;
    }
    free(slots_seen);
    free(last_pos);
    free(has_last);
    free(table_start);
    if (status != LIA_OK) return status;
    for (uint32_t g = 0; g < n_groups; g++) cu_seqlens[g] = groups[g].start;
    cu_seqlens[n_groups] = n_rows;
    /* paging.rs:187-201 */
    int decoding = n_rows <= 8 && n_outputs == n_rows;
    for (uint32_t i = 0; decoding && i < n_outputs; i++)
        if (outputs[i] != i) decoding = 0;
    uint32_t span = decoding ? lo_decode_span(maximum) : 256;
    uint32_t parts = decoding ? lo_decode_parts(maximum, span) : (maximum + span - 1) / span;
    info->stride = stride;
    info->maximum = maximum;
    info->decoding = (uint32_t)decoding;
    info->span = span;
    info->parts = parts;
    info->n_groups = n_groups;
    (void)cmp_u32;
    return LIA_OK;
}

/* ------------------------------------------------------------------------------------ */
/* KV append: llama_cache_paged, src/gpu/kernels/llama.rs:162-183 (generic geometry).    */
/* ------------------------------------------------------------------------------------ */

static inline uint32_t slot_of(uint32_t position, uint32_t seq, const uint32_t *pages,
                               uint32_t stride, uint32_t P) {
    return pages[(size_t)seq * stride + position / P] * P + position % P;
}

void lo_kv_append(const lia_kv_layout *L, uint32_t rows, const uint32_t *positions,
                  const uint32_t *sequences, const uint32_t *pages, uint32_t stride,
                  const uint32_t *slot_mapping, int32_t src_dtype, const void *k, const void *v,
                  void *kc, void *vc, float *k_scales, float *v_scales) {
    uint32_t W = L->num_kv_heads * L->head_dim;
    for (uint32_t r = 0; r < rows; r++) {
        uint32_t slot = slot_mapping ? slot_mapping[r]
                                     : slot_of(positions[r], sequences[r], pages, stride, L->page_size);
        uint32_t page = slot / L->page_size;
        for (uint32_t i = 0; i < W; i++) {
            float kv = load_elem(k, (size_t)r * W + i, src_dtype);
            float vv = load_elem(v, (size_t)r * W + i, src_dtype);
            size_t at = (size_t)slot * W + i;
            switch (L->dtype) {
            case LIA_F16:
                ((uint16_t *)kc)[at] = lo_f32_to_f16(kv);
                ((uint16_t *)vc)[at] = lo_f32_to_f16(vv);
                break;
            case LIA_BF16:
                ((uint16_t *)kc)[at] = lo_f32_to_bf16(kv);
                ((uint16_t *)vc)[at] = lo_f32_to_bf16(vv);
                break;
            case LIA_FP8_E4M3: {
                uint32_t h = i / L->head_dim;
                /* a page never quantised (scale 0) takes scale 1, recorded by the append */
                float *ksp = &k_scales[(size_t)page * L->num_kv_heads + h];
                float *vsp = &v_scales[(size_t)page * L->num_kv_heads + h];
                if (*ksp == 0.0f) *ksp = 1.0f;
                if (*vsp == 0.0f) *vsp = 1.0f;
                float ks = *ksp, vs = *vsp;
                ((uint8_t *)kc)[at] = lo_f32_to_e4m3(kv / ks);
                ((uint8_t *)vc)[at] = lo_f32_to_e4m3(vv / vs);
                break;
            }
            }
        }
    }
}

/* Page quantisation with scale = amax / 448 per (page, head) and plane. */
void lo_kv_quantize_pages(const lia_kv_layout *L, uint32_t n_pages, const uint32_t *page_ids,
                          int32_t src_dtype, const void *k, const void *v, void *kc, void *vc,
                          float *k_scales, float *v_scales) {
    uint32_t H = L->num_kv_heads, D = L->head_dim, P = L->page_size;
    for (uint32_t n = 0; n < n_pages; n++) {
        uint32_t page = page_ids[n];
        for (int plane = 0; plane < 2; plane++) {
            const void *src = plane ? v : k;
            uint8_t *dst = (uint8_t *)(plane ? vc : kc);
            float *scales = plane ? v_scales : k_scales;
            for (uint32_t h = 0; h < H; h++) {
                float amax = 0.0f;
                for (uint32_t t = 0; t < P; t++)
                    for (uint32_t d = 0; d < D; d++) {
                        float x = fabsf(load_elem(src, (((size_t)n * P + t) * H + h) * D + d, src_dtype));
                        if (x > amax) amax = x;
                    }
                float s = amax > 0.0f ? amax / 448.0f : 1.0f;
                scales[(size_t)page * H + h] = s;
                for (uint32_t t = 0; t < P; t++)
                    for (uint32_t d = 0; d < D; d++) {
                        float x = load_elem(src, (((size_t)n * P + t) * H + h) * D + d, src_dtype);
                        dst[(((size_t)page * P + t) * H + h) * D + d] = lo_f32_to_e4m3(x / s);
                    }
            }
        }
    }
}

/* ------------------------------------------------------------------------------------ */
/* Attention.                                                                             */
/* ------------------------------------------------------------------------------------ */

typedef struct lo_geom {
    uint32_t hq, hkv, d, page_size, stride;
    int32_t kv_dtype;
    double scale; /* f64 in the f64 oracle (llama_attention.rs:271), rounded to f32 elsewhere */
} lo_geom;

static inline float kv_value(const lo_geom *g, const void *pool, const float *scales, uint32_t slot,
                             uint32_t h, uint32_t c) {
    float x = load_elem(pool, ((size_t)slot * g->hkv + h) * g->d + c, g->kv_dtype);
    if (g->kv_dtype == LIA_FP8_E4M3) x *= scales[(size_t)(slot / g->page_size) * g->hkv + h];
    return x;
}

/* Independent f64 softmax attention on the stored (rounded) K/V, as the reference's own
 * oracle does (src/gpu/llama_attention.rs:253-284), generic in geometry.
 * q: f32 [rows][hq][d]; out: f64 [rows][hq][d]. */
void lo_attention_f64(const lo_geom *g, uint32_t rows, const uint32_t *positions,
                      const uint32_t *sequences, const uint32_t *pages, const float *q,
                      const void *kc, const void *vc, const float *k_scales,
                      const float *v_scales, double *out) {
    uint32_t group = g->hq / g->hkv;
#pragma omp parallel for collapse(2) schedule(dynamic)
    for (uint32_t r = 0; r < rows; r++) {
        for (uint32_t h = 0; h < g->hq; h++) {
            uint32_t count = positions[r] + 1, hk = h / group;
            const float *qv = q + ((size_t)r * g->hq + h) * g->d;
            double *o = out + ((size_t)r * g->hq + h) * g->d;
            double *scores = (double *)malloc(sizeof(double) * count);
            double maximum = -INFINITY;
            for (uint32_t t = 0; t < count; t++) {
                uint32_t slot = slot_of(t, sequences[r], pages, g->stride, g->page_size);
                double s = 0.0;
                for (uint32_t c = 0; c < g->d; c++)
                    s += (double)qv[c] * (double)kv_value(g, kc, k_scales, slot, hk, c);
                s *= (double)g->scale;
                scores[t] = s;
                if (s > maximum) maximum = s;
            }
            double total = 0.0;
            for (uint32_t t = 0; t < count; t++) total += exp(scores[t] - maximum);
            for (uint32_t c = 0; c < g->d; c++) o[c] = 0.0;
            for (uint32_t t = 0; t < count; t++) {
                uint32_t slot = slot_of(t, sequences[r], pages, g->stride, g->page_size);
                double w = exp(scores[t] - maximum) / total;
                for (uint32_t c = 0; c < g->d; c++)
                    o[c] += w * (double)kv_value(g, vc, v_scales, slot, hk, c);
            }
            free(scores);
        }
    }
}

/* One split of scalar online-softmax attention: llama_attention_partial,
 * src/gpu/kernels/llama.rs:63-159.  Record = [o(d) unnormalised, m (natural log), l]. */
static void partial_one(const lo_geom *g, uint32_t row, uint32_t h, uint32_t part, uint32_t span,
                        const uint32_t *positions, const uint32_t *sequences, const uint32_t *pages,
                        const float *q, const void *kc, const void *vc, const float *k_scales,
                        const float *v_scales, float *record) {
    uint32_t group = g->hq / g->hkv, hk = h / group, D = g->d;
    uint32_t valid = positions[row] + 1;
    const float *qv = q + ((size_t)row * g->hq + h) * D;
    float values[256];
    for (uint32_t c = 0; c < D; c++) values[c] = 0.0f;
    float maximum = -INFINITY, sum = 0.0f;
    uint32_t end = (part + 1) * span < valid ? (part + 1) * span : valid;
    for (uint32_t token = part * span; token < end; token++) {
        uint32_t slot = slot_of(token, sequences[row], pages, g->stride, g->page_size);
        float score = 0.0f;
        for (uint32_t c = 0; c < D; c++) score = fmaf(qv[c], kv_value(g, kc, k_scales, slot, hk, c), score);
        score *= (float)g->scale;
        float next = fmaxf(maximum, score);
        float old = expf(maximum - next); /* exp(-inf) = 0 on the first key */
        float weight = expf(score - next);
        sum = sum * old + weight;
        for (uint32_t c = 0; c < D; c++)
            values[c] = values[c] * old + weight * kv_value(g, vc, v_scales, slot, hk, c);
        maximum = next;
    }
    for (uint32_t c = 0; c < D; c++) record[c] = values[c];
    record[D] = maximum;
    record[D + 1] = sum;
}

/* partial() with uniform parts/span over rows query_start .. query_start+queries-1
 * (src/gpu/llama_attention.rs:137-156).  partial layout:
 * [((row - query_start) * hq + h) * parts + part][d + 2]. */
void lo_attention_partial(const lo_geom *g, uint32_t query_start, uint32_t queries, uint32_t parts,
                          uint32_t span, const uint32_t *positions, const uint32_t *sequences,
                          const uint32_t *pages, const float *q, const void *kc, const void *vc,
                          const float *k_scales, const float *v_scales, float *partial) {
#pragma omp parallel for collapse(3) schedule(dynamic)
    for (uint32_t i = 0; i < queries; i++)
        for (uint32_t h = 0; h < g->hq; h++)
            for (uint32_t p = 0; p < parts; p++)
                partial_one(g, query_start + i, h, p, span, positions, sequences, pages, q, kc, vc,
                            k_scales, v_scales,
                            partial + (((size_t)i * g->hq + h) * parts + p) * (g->d + 2));
}

/* Split-K combine: llama_attention_merge / llama_merge_small,
 * src/gpu/kernels/llama.rs:201-290 and llama_merge.rs:10-76.  Parts with l == 0 have
 * zero weight; weights exp(m_p - M); out = sum w_p o_p / sum w_p l_p.
 * out: f32 [query_start + i][hq][d]. */
void lo_merge(uint32_t hq, uint32_t d, uint32_t query_start, uint32_t queries, uint32_t parts,
              const float *partial, float *out) {
    for (uint32_t grp = 0; grp < queries * hq; grp++) {
        const float *base = partial + (size_t)grp * parts * (d + 2);
        float maximum = -INFINITY;
        for (uint32_t p = 0; p < parts; p++) maximum = fmaxf(maximum, base[(size_t)p * (d + 2) + d]);
        float total = 0.0f;
        float weights[1024];
        for (uint32_t p = 0; p < parts; p++) {
            float mass = base[(size_t)p * (d + 2) + d + 1];
            weights[p] = mass > 0.0f ? expf(base[(size_t)p * (d + 2) + d] - maximum) : 0.0f;
            total += weights[p] * mass;
        }
        for (uint32_t c = 0; c < d; c++) {
            float value = 0.0f;
            for (uint32_t p = 0; p < parts; p++) value = fmaf(weights[p], base[(size_t)p * (d + 2) + c], value);
            out[((size_t)query_start * hq + grp) * d + c] = value / total;
        }
    }
}

/* CPU baseline of the whole path for a packed batch: split-K scalar attention with
 * `span`-token splits per row followed by the merge, in f32, parallel over
 * (row, head, split).  Same arithmetic as lo_attention_partial + lo_merge; the split
 * count follows each row's own key count (the reference uses a batch-uniform count and
 * skips empty parts in the merge, which yields the same values). */
void lo_paged_attention_f32(const lo_geom *g, uint32_t rows, uint32_t span,
                            const uint32_t *positions, const uint32_t *sequences,
                            const uint32_t *pages, const float *q, const void *kc, const void *vc,
                            const float *k_scales, const float *v_scales, float *work,
                            size_t work_floats, float *out) {
    uint32_t maxparts = 1;
    for (uint32_t r = 0; r < rows; r++) {
        uint32_t p = (positions[r] + span) / span;
        if (p > maxparts) maxparts = p;
    }
    size_t rec = g->d + 2;
    if ((size_t)rows * g->hq * maxparts * rec > work_floats) return;
    size_t total = (size_t)rows * g->hq * maxparts;
#pragma omp parallel for schedule(dynamic, 4)
    for (size_t i = 0; i < total; i++) {
        uint32_t p = (uint32_t)(i % maxparts);
        uint32_t h = (uint32_t)(i / maxparts % g->hq);
        uint32_t r = (uint32_t)(i / maxparts / g->hq);
        float *record = work + i * rec;
        if (p * span > positions[r]) {
            record[g->d] = -INFINITY;
            record[g->d + 1] = 0.0f;
            continue;
        }
        partial_one(g, r, h, p, span, positions, sequences, pages, q, kc, vc, k_scales, v_scales, record);
    }
    lo_merge(g->hq, g->d, 0, rows, maxparts, work, out);
}

/* OpenMP threads a parallel region of this library uses (reported with the CPU baseline). */
int lo_omp_threads(void) {
    int n = 1;
#pragma omp parallel
    {
#pragma omp single
        n = omp_get_num_threads();
    }
    return n;
}

/* ------------------------------------------------------------------------------------ */
/* RoPE + append: coefficients / rotary_cache, src/gpu/kernels/llama_position.rs:36-118; */
/* llama_rope, src/gpu/kernels/llama.rs:33-60.  Geometry of the reference: head_dim 128,  */
/* 16 query heads, 2 KV heads, combined rows of 2560 floats.                              */
/* ------------------------------------------------------------------------------------ */

/* Generalised table [rows][head_dim/2][2] = {cos, sin}(position * inv_i) with
 * inv_i = f32(1 / f32(base^(2i/head_dim))) (the reference's order of rounded steps).  The
 * power and the trigonometric functions are evaluated in double and rounded once to f32 -
 * a correctly rounded f32 restatement of powf/cosf/sinf in all but near-halfway cases. */
void lo_rope_coefficients(uint32_t rows, uint32_t head_dim, float base, const uint32_t *positions,
                          float *out) {
    const uint32_t half = head_dim / 2;
    for (uint32_t i = 0; i < rows * half; i++) {
        float e = 2.0f * (float)(i % half) / (float)head_dim;
        float p = (float)pow((double)base, (double)e);
        float inv = 1.0f / p;
        float angle = (float)positions[i / half] * inv;
        out[i * 2] = (float)cos((double)angle);
        out[i * 2 + 1] = (float)sin((double)angle);
    }
}

void lo_coefficients(uint32_t rows, float base, const uint32_t *positions, float *out) {
    lo_rope_coefficients(rows, 128, base, positions, out);
}

/* llama_rope over input [rows][heads][128].  The reference source reads
 * x*cos + pair*sin*(d<64 ? -1 : 1); its own test requires the result to be bit-equal to
 * rotary_cache's explicit fma(x, cos, +-(pair*sin)) (llama_position.rs:229-237), i.e. the
 * device compiler contracts the multiply-add.  The restatement is that contracted form. */
void lo_rope(uint32_t heads, float base, uint32_t n, const uint32_t *positions, const float *input,
             float *output) {
    for (uint32_t i = 0; i < n; i++) {
        uint32_t d = i % 128, row = i / (heads * 128);
        float cs[2]; /* the steps of lo_rope_coefficients for index d % 64 */
        float p = (float)pow((double)base, (double)(2.0f * (float)(d % 64) / 128.0f));
        float angle = (float)positions[row] * (1.0f / p);
        cs[0] = (float)cos((double)angle);
        cs[1] = (float)sin((double)angle);
        uint32_t paired = d < 64 ? i + 64 : i - 64;
        float sign = d < 64 ? -1.0f : 1.0f;
        volatile float b = input[paired] * cs[1];
        output[i] = fmaf(input[i], cs[0], b * sign);
    }
}

/* rotary_cache: q' = fma(l, c, -(r*s)), q'' = fma(r, c, l*s) with the product rounded,
 * K rotated likewise, V copied; K/V written as f16 at the paged slot. */
void lo_rotary_cache(uint32_t rows, uint32_t stride, uint32_t page_size, const uint32_t *positions,
                     const uint32_t *sequences, const uint32_t *pages, const float *coefficients,
                     const float *input, float *query, uint16_t *keys, uint16_t *values) {
    for (uint32_t i = 0; i < rows * 1024; i++) {
        uint32_t row = i / 1024, head = i % 1024 / 64, d = i % 64;
        float c = coefficients[row * 128 + d * 2], s = coefficients[row * 128 + d * 2 + 1];
        size_t offset = (size_t)row * 2560 + head * 128;
        float left = input[offset + d], right = input[offset + d + 64];
        volatile float rs = right * s, ls = left * s;
        query[(size_t)row * 2048 + head * 128 + d] = fmaf(left, c, -rs);
        query[(size_t)row * 2048 + head * 128 + d + 64] = fmaf(right, c, ls);
        if (head < 2) {
            size_t ko = (size_t)row * 2560 + 2048 + head * 128;
            float kl = input[ko + d], kr = input[ko + d + 64];
            volatile float krs = kr * s, kls = kl * s;
            float k0 = fmaf(kl, c, -krs), k1 = fmaf(kr, c, kls);
            uint32_t slot = slot_of(positions[row], sequences[row], pages, stride, page_size);
            size_t at = (size_t)slot * 256 + head * 128 + d;
            keys[at] = lo_f32_to_f16(k0);
            keys[at + 64] = lo_f32_to_f16(k1);
            values[at] = lo_f32_to_f16(input[ko + 256 + d]);
            values[at + 64] = lo_f32_to_f16(input[ko + 320 + d]);
        }
    }
}

/* Generalised rotary_cache (llama_position.rs:49-118): input rows [rows][(hq + 2 hkv) * d]
 * hold q heads | k heads | v heads.  For d' < d/2 with {c, s} = coefficients[row][d']:
 *   x'[d']       = fma(x[d'], c, -f32(x[d' + d/2] * s))
 *   x'[d' + d/2] = fma(x[d' + d/2], c, f32(x[d'] * s))
 * Queries go to query ([rows][hq][d], f32 or rounded to bf16); rotated K and unrotated V are
 * appended exactly as lo_kv_append appends f32 rows (slot mapping or table, pool conversion). */
void lo_rope_kv_append(const lia_kv_layout *L, uint32_t hq, uint32_t rows, const uint32_t *positions,
                       const uint32_t *sequences, const uint32_t *pages, uint32_t stride,
                       const uint32_t *slot_mapping, const float *coefficients, const float *input,
                       void *query, int32_t query_dtype, void *kc, void *vc, float *k_scales,
                       float *v_scales) {
    const uint32_t d = L->head_dim, half = d / 2, hkv = L->num_kv_heads;
    const size_t width = (size_t)(hq + 2 * hkv) * d;
    float *kr = (float *)malloc((size_t)rows * hkv * d * sizeof(float));
    float *vr = (float *)malloc((size_t)rows * hkv * d * sizeof(float));
    for (uint32_t r = 0; r < rows; r++) {
        const float *x = input + (size_t)r * width;
        for (uint32_t h = 0; h < hq + hkv; h++) {
            for (uint32_t i = 0; i < half; i++) {
                float c = coefficients[((size_t)r * half + i) * 2];
                float sn = coefficients[((size_t)r * half + i) * 2 + 1];
                float left = x[h * d + i], right = x[h * d + i + half];
                float a = fmaf(left, c, -(right * sn)), b = fmaf(right, c, left * sn);
                if (h < hq) {
                    size_t at = ((size_t)r * hq + h) * d + i;
                    if (query_dtype == LIA_BF16) {
                        ((uint16_t *)query)[at] = lo_f32_to_bf16(a);
                        ((uint16_t *)query)[at + half] = lo_f32_to_bf16(b);
                    } else {
                        ((float *)query)[at] = a;
                        ((float *)query)[at + half] = b;
                    }
                } else {
                    size_t at = ((size_t)r * hkv + (h - hq)) * d + i;
                    kr[at] = a;
                    kr[at + half] = b;
                }
            }
        }
        memcpy(vr + (size_t)r * hkv * d, x + (size_t)(hq + hkv) * d, (size_t)hkv * d * sizeof(float));
    }
    lo_kv_append(L, rows, positions, sequences, pages, stride, slot_mapping, LIA_F32, kr, vr, kc, vc,
                 k_scales, v_scales);
    free(kr);
    free(vr);
}

/* llama_gather_hidden, src/gpu/kernels/llama.rs:186-198 (generic width). */
void lo_gather(uint32_t count, uint32_t width, const uint32_t *indices, const float *input, float *output) {
    for (size_t i = 0; i < (size_t)count * width; i++)
        output[i] = input[(size_t)indices[i / width] * width + i % width];
}

/* Array conversion between the element types (round-to-nearest-even, FP8 saturating). */
void lo_convert(const void *src, int32_t src_dtype, void *dst, int32_t dst_dtype, size_t n) {
#pragma omp parallel for schedule(static)
    for (size_t i = 0; i < n; i++) {
        float x = load_elem(src, i, src_dtype);
        switch (dst_dtype) {
        case LIA_F32: ((float *)dst)[i] = x; break;
        case LIA_F16: ((uint16_t *)dst)[i] = lo_f32_to_f16(x); break;
        case LIA_BF16: ((uint16_t *)dst)[i] = lo_f32_to_bf16(x); break;
        case LIA_FP8_E4M3: ((uint8_t *)dst)[i] = lo_f32_to_e4m3(x); break;
        }
    }
}

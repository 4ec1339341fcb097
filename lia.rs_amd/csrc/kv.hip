// Packing, slot mapping and KV-append scatter for the paged KV pool (gfx950).
#include "common.hpp"
#include "launch.hpp"
#include "pack.hpp"

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

__global__ __launch_bounds__(1024) void pack_kernel(uint32_t n_seqs, const uint32_t *seq_slots,
                                                    const uint32_t *q_lens, const uint32_t *cached,
                                                    const uint32_t *pages, uint32_t stride,
                                                    uint32_t page_shift, uint32_t pool_pages,
                                                    uint32_t context, uint32_t max_rows,
                                                    uint32_t *cu, uint32_t *positions,
                                                    uint32_t *sequences, uint32_t *slot_mapping,
                                                    uint32_t *status) {
    pack_rows_block(n_seqs, seq_slots, q_lens, cached, pages, stride, page_shift, pool_pages, context,
                    max_rows, cu, positions, sequences, slot_mapping, status, nullptr);
}

__global__ __launch_bounds__(kCheckThreads) void table_check_kernel(
    uint32_t n_seqs, const uint32_t *seq_slots, const uint32_t *q_lens, const uint32_t *cached,
    const uint32_t *pages, uint32_t stride, uint32_t page_shift, uint32_t pool_pages,
    uint32_t context, uint32_t max_rows, uint32_t *cu, uint32_t *slot_mapping, uint32_t *status) {
    table_check_block(blockIdx.x, gridDim.x, n_seqs, seq_slots, q_lens, cached, pages, stride,
                      page_shift, pool_pages, context, max_rows, cu, slot_mapping, status);
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

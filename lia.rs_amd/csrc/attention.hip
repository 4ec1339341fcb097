// Paged causal GQA attention over a ragged packed batch for gfx950 (CDNA4).
//
// Work decomposition ("units"): for batch sequence b, its query rows are cut into column
// blocks of `rpc` rows; each (sequence, column block, KV head) is one unit whose MFMA
// columns are the rpc*group (row, query head) pairs that share that KV head.  A unit
// attends keys 0 .. positions[last row of the block], tiled in 32-token blocks.
//
// Scheduling is balanced over wavefronts rather than over units: the key blocks of all
// units are laid end to end and wave w of N takes blocks [w*B/N, (w+1)*B/N).  A unit
// covered by one wave is written normalised straight to `out`; a unit split across
// waves leaves one partial record (unnormalised O, running max, running sum) per wave
// and the combine kernel merges them, which is the reference's split-K partial + merge
// (src/gpu/kernels/llama_flash_kernel.rs:321-376, src/gpu/kernels/llama_merge.rs:10-76)
// with splits chosen for load balance instead of a batch-uniform span.
//
// Per 32-token block a wave computes S^T = K * Q^T with K straight from HBM as the MFMA
// A operand (16 tokens x 32 dims per instruction) and Q^T resident in registers, runs
// the online softmax in the log2 domain per column, stages V through LDS in its natural
// token-major layout and reads it back transposed (ds_read_b64_tr_b16) as the A operand
// of O^T += V^T * P^T.  Causal masking is per column: row r sees keys <= positions[r]
// (src/gpu/kernels/llama_flash_kernel.rs:145-175).
#include "common.hpp"

namespace lia {

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
    const uint4 *units;      // [U + 1]: {b, cb, hk, first block}; units[U].w = B
    const uint32_t *header;  // {U, B}
    float *part_o;           // [records][cols][D]
    float *part_ml;          // [records][cols][2]
    uint32_t hq, hkv, group, stride, page_shift, n_waves, rpc;
    float scale_log2;        // softmax scale * log2(e)
    int q_f32, out_f32;
};

// ------------------------------------------------------------------ plan

// One workgroup builds the unit list of a step.  Positions within a sequence are
// consecutive (validated by packing, src/inference/paging.rs:167-172), so the key count
// of a column block is positions[first row] + (last row index + 1).
__global__ __launch_bounds__(256) void plan_kernel(uint32_t n_seqs, const uint32_t *cu,
                                                   const uint32_t *positions, uint32_t rpc,
                                                   uint32_t hkv, uint32_t max_units, uint4 *units,
                                                   uint32_t *header) {
    __shared__ uint32_t s_units[256], s_blocks[256];
    __shared__ uint32_t carry_units, carry_blocks, overflow;
    const uint32_t t = threadIdx.x;
    if (t == 0) { carry_units = 0; carry_blocks = 0; overflow = 0; }
    __syncthreads();
    for (uint32_t base = 0; base < n_seqs; base += 256) {
        uint32_t b = base + t;
        uint32_t nu = 0, nb = 0, r0 = 0, nr = 0, p0 = 0;
        if (b < n_seqs) {
            r0 = cu[b];
            nr = cu[b + 1] - r0;
            if (nr > 0) {
                p0 = positions[r0];
                uint32_t ncb = (nr + rpc - 1) / rpc;
                nu = ncb * hkv;
                for (uint32_t cb = 0; cb < ncb; cb++) {
                    uint32_t last = min((cb + 1) * rpc, nr);
                    nb += (p0 + last + 31) / 32;
                }
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
            for (uint32_t cb = 0; cb < ncb; cb++) {
                uint32_t last = min((cb + 1) * rpc, nr);
                uint32_t blocks = (p0 + last + 31) / 32;
                for (uint32_t h = 0; h < hkv; h++) {
                    units[u++] = make_uint4(b, cb, h, blk);
                    blk += blocks;
                }
            }
        }
        __syncthreads();
        if (t == 255) { carry_units += s_units[255]; carry_blocks += s_blocks[255]; }
        __syncthreads();
    }
    if (t == 0) {
        uint32_t U = overflow ? 0 : carry_units, B = overflow ? 0 : carry_blocks;
        units[U] = make_uint4(0, 0, 0, B);
        header[0] = U;
        header[1] = B;
        header[2] = overflow;
    }
}

// ------------------------------------------------------------------ the attention kernel

template <int D, int KVT>
struct Cfg {
    static constexpr bool FP8 = KVT == LIA_FP8_E4M3;
    static constexpr bool MBF16 = KVT == LIA_BF16;        // MFMA operand type
    static constexpr int EB = FP8 ? 1 : 2;                // bytes per stored KV element
    static constexpr int KS = D / 32;                     // MFMA k-steps over head_dim
    static constexpr int DT = D / 16;                     // 16-wide d tiles of the output
    static constexpr int KQ = D * EB / 4 / 16;            // 16-byte K loads per lane per tile
    static constexpr int CPT = D * EB / 16;               // 16-byte V chunks per token
    static constexpr int NVL = 32 * CPT / 64;             // 16-byte V loads per lane
    static constexpr int PITCH = D + 16;                  // LDS row pitch (16-bit elements)
};

template <int D, int KVT>
struct Chunk {
    u32x4 k[2][Cfg<D, KVT>::KQ];
    u32x4 v[Cfg<D, KVT>::NVL];
    float ks[2], vs[2];
};

template <int D, int KVT>
__device__ __forceinline__ void load_chunk(const AttnParams &p, Chunk<D, KVT> &c, uint32_t t,
                                           uint32_t kend, const uint32_t *table, uint32_t hk) {
    using C = Cfg<D, KVT>;
    const uint32_t lane = lane_id(), g = lane >> 4, li = lane & 15;
    const uint32_t P = 1u << p.page_shift;
    const uint8_t *kc = (const uint8_t *)p.kc;
    const uint8_t *vc = (const uint8_t *)p.vc;
#pragma unroll
    for (int j = 0; j < 2; j++) {
        uint32_t t0 = t + 16 * j;
        bool live = t0 < kend;
        uint32_t page = live ? table[t0 >> p.page_shift] : 0;
        if constexpr (C::FP8) {
            c.ks[j] = live ? p.k_scales[(size_t)page * p.hkv + hk] : 0.0f;
            c.vs[j] = live ? p.v_scales[(size_t)page * p.hkv + hk] : 0.0f;
        }
        uint32_t tok = t0 + li;
        size_t slot = (size_t)page * P + (tok & (P - 1));
        const u32x4 *src = (const u32x4 *)(kc + ((slot * p.hkv + hk) * D + g * (D / 4)) * C::EB);
#pragma unroll
        for (int s = 0; s < C::KQ; s++) c.k[j][s] = (live && tok < kend) ? src[s] : u32x4{0, 0, 0, 0};
    }
#pragma unroll
    for (int s = 0; s < C::NVL; s++) {
        uint32_t item = s * 64 + lane;
        uint32_t tl = item / C::CPT, chunk = item % C::CPT;
        uint32_t tok = t + tl;
        bool live = tok < kend;
        uint32_t page = (t + (tl & 16)) < kend ? table[(t + (tl & 16)) >> p.page_shift] : 0;
        size_t slot = (size_t)page * P + (tok & (P - 1));
        const u32x4 *src = (const u32x4 *)(vc + ((slot * p.hkv + hk) * D) * C::EB + chunk * 16);
        c.v[s] = live ? *src : u32x4{0, 0, 0, 0};
    }
}

// Query operand for one 16-column tile: lane (g, col) holds q[col][(D/4)*g .. +D/4) as KS
// MFMA B-operand quads (the same head_dim permutation the K loads use).
template <int D, int KVT>
__device__ __forceinline__ void load_q(const AttnParams &p, u32x4 *qr, uint32_t row, uint32_t head,
                                       bool valid) {
    using C = Cfg<D, KVT>;
    const uint32_t g = lane_id() >> 4;
    size_t base = ((size_t)row * p.hq + head) * D + g * (D / 4);
#pragma unroll
    for (int s = 0; s < C::KS; s++) {
        float x[8];
        if (!valid) {
#pragma unroll
            for (int e = 0; e < 8; e++) x[e] = 0.0f;
        } else if (p.q_f32) {
            const float4 *src = (const float4 *)((const float *)p.q + base + s * 8);
            float4 a = src[0], b = src[1];
            x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
            x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
        } else {
            u32x4 w = *(const u32x4 *)((const uint16_t *)p.q + base + s * 8);
            if constexpr (C::MBF16) { qr[s] = w; continue; }
#pragma unroll
            for (int e = 0; e < 4; e++) {
                x[2 * e] = bf16_to_f32(w[e] & 0xffffu);
                x[2 * e + 1] = bf16_to_f32(w[e] >> 16);
            }
        }
        qr[s] = u32x4{pack2<C::MBF16>(x[0], x[1]), pack2<C::MBF16>(x[2], x[3]),
                      pack2<C::MBF16>(x[4], x[5]), pack2<C::MBF16>(x[6], x[7])};
    }
}

template <int D, int NT, int KVT>
__device__ __forceinline__ void compute_chunk(const AttnParams &p, const Chunk<D, KVT> &c,
                                              uint32_t t, const u32x4 (&qr)[NT][Cfg<D, KVT>::KS],
                                              const uint32_t (&lim)[NT], float (&m)[NT],
                                              float (&l)[NT], f32x4 (&o)[NT][Cfg<D, KVT>::DT],
                                              uint16_t *vlds) {
    using C = Cfg<D, KVT>;
    const uint32_t lane = lane_id(), g = lane >> 4, li = lane & 15;

    // Stage V (natural [token][d] layout) into LDS while the scores are computed.
#pragma unroll
    for (int s = 0; s < C::NVL; s++) {
        uint32_t item = s * 64 + lane;
        uint32_t tl = item / C::CPT, chunk = item % C::CPT;
        if constexpr (C::FP8) {
            u32x2 lo0 = e4m3x4_to_f16x4_scaled(c.v[s].x), lo1 = e4m3x4_to_f16x4_scaled(c.v[s].y);
            u32x2 hi0 = e4m3x4_to_f16x4_scaled(c.v[s].z), hi1 = e4m3x4_to_f16x4_scaled(c.v[s].w);
            u32x4 *dst = (u32x4 *)(vlds + tl * C::PITCH + chunk * 16);
            dst[0] = u32x4{lo0.x, lo0.y, lo1.x, lo1.y};
            dst[1] = u32x4{hi0.x, hi0.y, hi1.x, hi1.y};
        } else {
            *(u32x4 *)(vlds + tl * C::PITCH + chunk * 8) = c.v[s];
        }
    }

    float kscale[2] = {p.scale_log2, p.scale_log2};
    float vscale[2] = {1.0f, 1.0f};
    if constexpr (C::FP8) {
#pragma unroll
        for (int j = 0; j < 2; j++) {
            kscale[j] = p.scale_log2 * c.ks[j] * 256.0f;
            vscale[j] = c.vs[j] * 256.0f;
        }
    }

#pragma unroll
    for (int nt = 0; nt < NT; nt++) {
        f32x4 s[2];
#pragma unroll
        for (int j = 0; j < 2; j++) {
            s[j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int ks = 0; ks < C::KS; ks++) {
                u32x4 a;
                if constexpr (C::FP8) {
                    // k-step ks uses bytes 8*ks .. 8*ks+7 of the lane's D/4-byte run
                    const u32x4 &raw = c.k[j][ks / 2];
                    uint32_t w0 = (ks & 1) ? raw.z : raw.x, w1 = (ks & 1) ? raw.w : raw.y;
                    u32x2 x0 = e4m3x4_to_f16x4_scaled(w0), x1 = e4m3x4_to_f16x4_scaled(w1);
                    a = u32x4{x0.x, x0.y, x1.x, x1.y};
                } else {
                    a = c.k[j][ks];
                }
                s[j] = mfma16x16x32<C::MBF16>(a, qr[nt][ks], s[j]);
            }
        }
        // Online softmax for column nt*16 + li over tokens t + 16j + 4g + i.
        float x[2][4];
        float mx = -INFINITY;
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                uint32_t tok = t + 16 * j + 4 * g + i;
                float v = tok < lim[nt] ? s[j][i] * kscale[j] : -INFINITY;
                x[j][i] = v;
                mx = fmaxf(mx, v);
            }
        mx = fmaxf(mx, shfl_xor(mx, 16));
        mx = fmaxf(mx, shfl_xor(mx, 32));
        float mnew = fmaxf(m[nt], mx);
        float muse = mnew == -INFINITY ? 0.0f : mnew;
        float factor = fast_exp2(m[nt] - muse);
        m[nt] = mnew;
        float pr[2][4];
        float sum = 0.0f;
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                float e = fast_exp2(x[j][i] - muse);
                sum += e;
                pr[j][i] = e * vscale[j];
            }
        l[nt] = l[nt] * factor + sum;
        u32x4 pb = u32x4{pack2<C::MBF16>(pr[0][0], pr[0][1]), pack2<C::MBF16>(pr[0][2], pr[0][3]),
                         pack2<C::MBF16>(pr[1][0], pr[1][1]), pack2<C::MBF16>(pr[1][2], pr[1][3])};
#pragma unroll
        for (int n = 0; n < C::DT; n++) {
            o[nt][n] *= factor;
            // V^T operand: rows 16n .. 16n+15 of d, k slots = tokens {4g..4g+3, 16+4g..16+4g+3}.
            const uint16_t *r0 = vlds + (4 * g + li / 4) * C::PITCH + 16 * n + 4 * (li & 3);
            const uint16_t *r1 = r0 + 16 * C::PITCH;
            s16x4 a0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (__attribute__((address_space(3))) s16x4 *)(r0));
            s16x4 a1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (__attribute__((address_space(3))) s16x4 *)(r1));
            u32x2 b0 = __builtin_bit_cast(u32x2, a0), b1 = __builtin_bit_cast(u32x2, a1);
            u32x4 av = u32x4{b0.x, b0.y, b1.x, b1.y};
            o[nt][n] = mfma16x16x32<C::MBF16>(av, pb, o[nt][n]);
        }
    }
}

__device__ __forceinline__ uint32_t owner_of(uint32_t blk, uint32_t N, uint32_t B) {
    return (uint32_t)((((uint64_t)blk + 1) * N - 1) / B);
}

template <int D, int NT, int KVT>
__global__ __launch_bounds__(64) void attention_kernel(AttnParams p) {
    using C = Cfg<D, KVT>;
    __shared__ __attribute__((aligned(16))) uint16_t vlds[32 * C::PITCH];
    const uint32_t lane = lane_id(), g = lane >> 4, li = lane & 15;
    const uint32_t w = blockIdx.x;
    const uint32_t U = p.header[0], B = p.header[1];
    const uint32_t N = min(p.n_waves, B);
    if (w >= N) return;
    uint32_t lo = (uint32_t)((uint64_t)w * B / N), hi = (uint32_t)((uint64_t)(w + 1) * B / N);
    // last unit whose first block <= lo
    uint32_t a = 0, e = U;
    while (a + 1 < e) {
        uint32_t mid = (a + e) >> 1;
        if (p.units[mid].w <= lo) a = mid; else e = mid;
    }
    uint32_t u = a;
    while (lo < hi && u < U) {
        uint4 un = p.units[u];
        uint32_t ustart = un.w, uend = p.units[u + 1].w;
        if (uend <= lo) { u++; continue; }
        const uint32_t b = un.x, cb = un.y, hk = un.z;
        const uint32_t seg_end = min(hi, uend);
        const uint32_t r0 = p.cu[b], nr = p.cu[b + 1] - r0;
        const uint32_t rowbeg = r0 + cb * p.rpc, nrows = min(p.rpc, nr - cb * p.rpc);
        const uint32_t *table = p.pages + (size_t)p.sequences[r0] * p.stride;
        const uint32_t kend = p.positions[rowbeg + nrows - 1] + 1;
        const uint32_t ncols = nrows * p.group;

        u32x4 qr[NT][C::KS];
        uint32_t lim[NT];
        float m[NT], l[NT];
        f32x4 o[NT][C::DT];
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
            uint32_t col = nt * 16 + li;
            bool valid = col < ncols;
            uint32_t row = rowbeg + (valid ? col / p.group : 0);
            uint32_t head = hk * p.group + col % p.group;
            lim[nt] = valid ? p.positions[row] + 1 : 0;
            load_q<D, KVT>(p, qr[nt], row, head, valid);
            m[nt] = -INFINITY;
            l[nt] = 0.0f;
#pragma unroll
            for (int n = 0; n < C::DT; n++) o[nt][n] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        }

        const uint32_t tbeg = (lo - ustart) * 32;
        const uint32_t tend = min((seg_end - ustart) * 32, kend);
        Chunk<D, KVT> c0, c1;
        if (tbeg < tend) load_chunk<D, KVT>(p, c0, tbeg, kend, table, hk);
        for (uint32_t t = tbeg; t < tend; t += 64) {
            if (t + 32 < tend) load_chunk<D, KVT>(p, c1, t + 32, kend, table, hk);
            compute_chunk<D, NT, KVT>(p, c0, t, qr, lim, m, l, o, vlds);
            if (t + 32 >= tend) break;
            if (t + 64 < tend) load_chunk<D, KVT>(p, c0, t + 64, kend, table, hk);
            compute_chunk<D, NT, KVT>(p, c1, t + 32, qr, lim, m, l, o, vlds);
        }

        const bool whole = lo == ustart && seg_end == uend;
        const uint32_t rec = w + u;
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
            float lt = l[nt];
            lt += shfl_xor(lt, 16);
            lt += shfl_xor(lt, 32);
            uint32_t col = nt * 16 + li;
            if (col >= ncols) continue;
            uint32_t row = rowbeg + col / p.group;
            uint32_t head = hk * p.group + col % p.group;
            if (whole) {
                float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
                size_t base = ((size_t)row * p.hq + head) * D + 4 * g;
#pragma unroll
                for (int n = 0; n < C::DT; n++) {
                    f32x4 v = o[nt][n] * inv;
                    if (p.out_f32) {
                        *(f32x4 *)((float *)p.out + base + 16 * n) = v;
                    } else {
                        u32x2 h = u32x2{(uint32_t)f32_to_bf16(v.x) | ((uint32_t)f32_to_bf16(v.y) << 16),
                                        (uint32_t)f32_to_bf16(v.z) | ((uint32_t)f32_to_bf16(v.w) << 16)};
                        *(u32x2 *)((uint16_t *)p.out + base + 16 * n) = h;
                    }
                }
            } else {
                size_t rbase = (size_t)rec * (16 * NT) + col;
                float *po = p.part_o + rbase * D + 4 * g;
#pragma unroll
                for (int n = 0; n < C::DT; n++) *(f32x4 *)(po + 16 * n) = o[nt][n];
                if (g == 0) {
                    p.part_ml[rbase * 2] = m[nt];
                    p.part_ml[rbase * 2 + 1] = lt;
                }
            }
        }
        lo = seg_end;
        u++;
    }
}

// Merge the partial records of every unit that was split across waves.  Weights follow
// the reference merge: a record with zero mass contributes nothing, the others are
// scaled by 2^(m_r - M) (m in the log2 domain here), out = sum w o / sum w l.
template <int D, int NT>
__global__ __launch_bounds__(256) void combine_kernel(AttnParams p) {
    const uint32_t u = blockIdx.x;
    const uint32_t U = p.header[0], B = p.header[1];
    if (u >= U) return;
    const uint32_t N = min(p.n_waves, B);
    uint4 un = p.units[u];
    uint32_t ustart = un.w, uend = p.units[u + 1].w;
    if (uend <= ustart) return;
    uint32_t wf = owner_of(ustart, N, B), wl = owner_of(uend - 1, N, B);
    if (wf == wl) return; // written directly by its only wave
    const uint32_t b = un.x, cb = un.y, hk = un.z;
    const uint32_t r0 = p.cu[b], nr = p.cu[b + 1] - r0;
    const uint32_t rowbeg = r0 + cb * p.rpc, nrows = min(p.rpc, nr - cb * p.rpc);
    const uint32_t ncols = nrows * p.group;
    constexpr uint32_t COLS = 16 * NT;
    constexpr uint32_t PER = COLS * D / 256; // outputs per thread
    for (uint32_t k = 0; k < PER; k++) {
        uint32_t idx = k * 256 + threadIdx.x;
        uint32_t col = idx / D, d = idx % D;
        if (col >= ncols) continue;
        float M = -INFINITY;
        for (uint32_t w = wf; w <= wl; w++) {
            size_t rb = (size_t)(w + u) * COLS + col;
            if (p.part_ml[rb * 2 + 1] > 0.0f) M = fmaxf(M, p.part_ml[rb * 2]);
        }
        float num = 0.0f, den = 0.0f;
        for (uint32_t w = wf; w <= wl; w++) {
            size_t rb = (size_t)(w + u) * COLS + col;
            float mass = p.part_ml[rb * 2 + 1];
            if (mass > 0.0f) {
                float wt = fast_exp2(p.part_ml[rb * 2] - M);
                den = fmaf(wt, mass, den);
                num = fmaf(wt, p.part_o[rb * D + d], num);
            }
        }
        float v = den > 0.0f ? num / den : 0.0f;
        uint32_t row = rowbeg + col / p.group, head = hk * p.group + col % p.group;
        size_t at = ((size_t)row * p.hq + head) * D + d;
        if (p.out_f32) ((float *)p.out)[at] = v;
        else ((uint16_t *)p.out)[at] = f32_to_bf16(v);
    }
}

// ------------------------------------------------------------------ host side

struct Layout {
    size_t header, units, part_ml, part_o, total;
    uint32_t max_units, max_records;
};

static inline uint32_t nt_for(uint32_t n_rows, uint32_t n_seqs, uint32_t group) {
    // Decode-only batches (one row per sequence) use one 16-column tile; batches with
    // multi-row sequences (MTP verify, prefill chunks) use two.
    return (n_rows > n_seqs && group <= 16) ? 2 : 1;
}

static Layout layout_for(const lia_attention_config *c, uint32_t n_waves) {
    Layout L;
    uint32_t group = c->num_q_heads / c->num_kv_heads;
    uint32_t rpc1 = 16 / group ? 16 / group : 1; // smallest rows-per-block over NT choices
    if (rpc1 == 0) rpc1 = 1;
    L.max_units = (c->max_rows / rpc1 + c->max_seqs + 1) * c->num_kv_heads;
    L.max_records = n_waves + L.max_units;
    size_t off = 0;
    L.header = off; off += 256;
    L.units = off; off += ((size_t)L.max_units + 1) * sizeof(uint4);
    off = (off + 255) & ~(size_t)255;
    L.part_ml = off; off += (size_t)L.max_records * 32 * 2 * sizeof(float);
    off = (off + 255) & ~(size_t)255;
    L.part_o = off; off += (size_t)L.max_records * 32 * c->head_dim * sizeof(float);
    L.total = off;
    return L;
}

} // namespace lia

using namespace lia;

static int g_device = 0;
static uint32_t g_cus = 0;

extern "C" int lia_init(int device) {
    if (hipSetDevice(device) != hipSuccess) return LIA_E_HIP;
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess)
        return LIA_E_HIP;
    g_device = device;
    g_cus = (uint32_t)cus;
    return LIA_OK;
}

extern "C" uint32_t lia_device_cus(void) {
    if (!g_cus) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess) return 0;
        if (lia_init(dev) != LIA_OK) return 0;
    }
    return g_cus;
}

static uint32_t waves_for_device() {
    uint32_t cus = lia_device_cus();
    if (!cus) cus = 256;
    return cus * 4;
}

extern "C" size_t lia_attention_workspace_bytes(const lia_attention_config *c) {
    if (!c || !c->num_kv_heads) return 0;
    return layout_for(c, waves_for_device()).total;
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
    return LIA_OK;
}

template <int D, int NT, int KVT>
static void launch_partial(const AttnParams &p, uint32_t n_waves, hipStream_t s) {
    hipLaunchKernelGGL((attention_kernel<D, NT, KVT>), dim3(n_waves), dim3(64), 0, s, p);
}

template <int D, int NT>
static void launch_partial_kv(int kv, const AttnParams &p, uint32_t n_waves, hipStream_t s) {
    if (kv == LIA_BF16) launch_partial<D, NT, LIA_BF16>(p, n_waves, s);
    else if (kv == LIA_F16) launch_partial<D, NT, LIA_F16>(p, n_waves, s);
    else launch_partial<D, NT, LIA_FP8_E4M3>(p, n_waves, s);
}

enum Stage { kPlan = 1, kPartial = 2, kMerge = 4 };

static int run_stages(int stages, const lia_attention_config *c, uint32_t n_seqs, uint32_t n_rows,
                      const uint32_t *cu_seqlens, const uint32_t *positions,
                      const uint32_t *sequences, const uint32_t *pages, const void *q,
                      const void *kc, const void *vc, const float *k_scales,
                      const float *v_scales, void *workspace, size_t workspace_bytes, void *out,
                      lia_stream_t stream) {
    int st = validate(c);
    if (st) return st;
    if (n_seqs == 0 || n_seqs > c->max_seqs || n_rows == 0 || n_rows > c->max_rows) return LIA_E_ARG;
    if (!cu_seqlens || !positions || !workspace) return LIA_E_ARG;
    if (stages & (kPartial | kMerge)) {
        if (!out) return LIA_E_ARG;
        if ((uintptr_t)out & 15) return LIA_E_ALIGN;
    }
    if (stages & kPartial) {
        if (!sequences || !pages || !q || !kc || !vc) return LIA_E_ARG;
        if (c->kv_dtype == LIA_FP8_E4M3 && (!k_scales || !v_scales)) return LIA_E_ARG;
        if (((uintptr_t)q | (uintptr_t)kc | (uintptr_t)vc) & 15) return LIA_E_ALIGN;
    }
    uint32_t n_waves = waves_for_device();
    Layout L = layout_for(c, n_waves);
    if (workspace_bytes < L.total) return LIA_E_WORKSPACE;
    if ((uintptr_t)workspace & 255) return LIA_E_ALIGN;
    uint32_t group = c->num_q_heads / c->num_kv_heads;
    uint32_t NT = nt_for(n_rows, n_seqs, group);
    if (group > 16 * NT) NT = 2;
    uint32_t rpc = (16 * NT) / group;
    uint8_t *ws = (uint8_t *)workspace;
    AttnParams p;
    p.q = q; p.kc = kc; p.vc = vc; p.k_scales = k_scales; p.v_scales = v_scales;
    p.cu = cu_seqlens; p.positions = positions; p.sequences = sequences; p.pages = pages;
    p.out = out;
    p.units = (const uint4 *)(ws + L.units);
    p.header = (const uint32_t *)(ws + L.header);
    p.part_o = (float *)(ws + L.part_o);
    p.part_ml = (float *)(ws + L.part_ml);
    p.hq = c->num_q_heads; p.hkv = c->num_kv_heads; p.group = group; p.stride = c->stride;
    p.page_shift = (uint32_t)__builtin_ctz(c->page_size);
    p.n_waves = n_waves;
    p.rpc = rpc;
    p.scale_log2 = c->scale * 1.4426950408889634f;
    p.q_f32 = c->q_dtype == LIA_F32;
    p.out_f32 = c->out_dtype == LIA_F32;
    hipStream_t s = (hipStream_t)stream;
    if (stages & kPlan)
        hipLaunchKernelGGL(plan_kernel, dim3(1), dim3(256), 0, s, n_seqs, cu_seqlens, positions, rpc,
                           c->num_kv_heads, L.max_units, (uint4 *)(ws + L.units),
                           (uint32_t *)(ws + L.header));
    if (stages & kPartial) {
        if (c->head_dim == 128) {
            if (NT == 1) launch_partial_kv<128, 1>(c->kv_dtype, p, n_waves, s);
            else launch_partial_kv<128, 2>(c->kv_dtype, p, n_waves, s);
        } else {
            if (NT == 1) launch_partial_kv<64, 1>(c->kv_dtype, p, n_waves, s);
            else launch_partial_kv<64, 2>(c->kv_dtype, p, n_waves, s);
        }
    }
    if (stages & kMerge) {
        if (c->head_dim == 128) {
            if (NT == 1) hipLaunchKernelGGL((combine_kernel<128, 1>), dim3(L.max_units), dim3(256), 0, s, p);
            else hipLaunchKernelGGL((combine_kernel<128, 2>), dim3(L.max_units), dim3(256), 0, s, p);
        } else {
            if (NT == 1) hipLaunchKernelGGL((combine_kernel<64, 1>), dim3(L.max_units), dim3(256), 0, s, p);
            else hipLaunchKernelGGL((combine_kernel<64, 2>), dim3(L.max_units), dim3(256), 0, s, p);
        }
    }
    return hipGetLastError() == hipSuccess ? LIA_OK : LIA_E_HIP;
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
                                  void *workspace, size_t workspace_bytes, lia_stream_t stream) {
    return run_stages(kPlan, c, n_seqs, n_rows, cu_seqlens, positions, nullptr, nullptr, nullptr,
                      nullptr, nullptr, nullptr, nullptr, workspace, workspace_bytes, nullptr,
                      stream);
}

extern "C" int lia_attention_partial(const lia_attention_config *c, uint32_t n_seqs,
                                     uint32_t n_rows, const uint32_t *cu_seqlens,
                                     const uint32_t *positions, const uint32_t *sequences,
                                     const uint32_t *pages, const void *q, const void *kc,
                                     const void *vc, const float *k_scales, const float *v_scales,
                                     void *workspace, size_t workspace_bytes, void *out,
                                     lia_stream_t stream) {
    return run_stages(kPartial, c, n_seqs, n_rows, cu_seqlens, positions, sequences, pages, q, kc,
                      vc, k_scales, v_scales, workspace, workspace_bytes, out, stream);
}

extern "C" int lia_attention_merge(const lia_attention_config *c, uint32_t n_seqs, uint32_t n_rows,
                                   const uint32_t *cu_seqlens, const uint32_t *positions,
                                   void *workspace, size_t workspace_bytes, void *out,
                                   lia_stream_t stream) {
    return run_stages(kMerge, c, n_seqs, n_rows, cu_seqlens, positions, nullptr, nullptr, nullptr,
                      nullptr, nullptr, nullptr, nullptr, workspace, workspace_bytes, out, stream);
}

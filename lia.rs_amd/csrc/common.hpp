// Shared device helpers for the gfx950 (CDNA4) paged attention kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/lia_hip.h"

namespace lia {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(8))) _Float16 f16x8;
typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(4))) uint32_t u32x4;
typedef __attribute__((ext_vector_type(2))) uint32_t u32x2;
typedef __attribute__((__vector_size__(4 * sizeof(short)))) short s16x4;

constexpr uint32_t kWave = 64;
constexpr uint32_t kNone = 0xffffffffu;

// ------------------------------------------------------------------ conversions
// Round-to-nearest-even conversions written from the IEEE / OCP format definitions.
// They are bit-identical to the CPU oracle's (tests assert it) and to the hardware
// conversion instructions for every finite input.

__device__ __forceinline__ uint32_t f2u(float f) { return __builtin_bit_cast(uint32_t, f); }
__device__ __forceinline__ float u2f(uint32_t u) { return __builtin_bit_cast(float, u); }

__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
    uint32_t x = f2u(f);
    if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)(((x >> 16) & 0x8000u) | 0x7fc0u);
    x += 0x7fffu + ((x >> 16) & 1u);
    return (uint16_t)(x >> 16);
}

__device__ __forceinline__ float bf16_to_f32(uint32_t b) { return u2f(b << 16); }

__device__ __forceinline__ uint16_t f32_to_f16(float f) {
    uint32_t x = f2u(f);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u);
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);
    if (ax < 0x38800000u) {
        uint32_t e = ax >> 23;
        if (e < 102) return (uint16_t)sign;
        uint32_t m = (ax & 0x7fffffu) | 0x800000u;
        uint32_t shift = 126 - e;
        uint32_t q = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1);
        uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (q & 1))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t r = ax - (112u << 23);
    r += 0xfffu + ((r >> 13) & 1u);
    return (uint16_t)(sign | (r >> 13));
}

__device__ __forceinline__ float f16_to_f32(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

// OCP E4M3FN, saturating to +-448, NaN -> 0x7f.
__device__ __forceinline__ uint8_t f32_to_e4m3(float f) {
    uint32_t x = f2u(f);
    uint32_t sign = (x >> 24) & 0x80u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax > 0x7f800000u) return 0x7f;
    if (ax >= 0x43e00000u) return (uint8_t)(sign | 0x7e);
    if (ax < 0x3c800000u) {
        float q = __builtin_rintf(u2f(ax) * 512.0f);
        return (uint8_t)(sign | (uint32_t)q);
    }
    uint32_t r = ax + 0x7ffffu + ((ax >> 20) & 1u);
    uint32_t code = (r >> 20) - (120u << 3);
    if (code > 0x7e) code = 0x7e;
    return (uint8_t)(sign | code);
}

// Two e4m3 bytes (bits 0-7 and 16-23 of t) -> two f16 lanes holding value * 2^-8.
// E4M3 is a sub-format of binary16 once the exponent bias is moved from 7 to 15:
// shifting the 7 exponent+mantissa bits left by 7 yields exactly value * 2^-8 for
// normals and subnormals alike (the caller folds 2^8 into its scale).
__device__ __forceinline__ uint32_t e4m3x2_to_f16x2_scaled(uint32_t t) {
    return ((t & 0x00800080u) << 8) | ((t & 0x007f007fu) << 7);
}

// 4 packed e4m3 bytes -> 4 f16 (as 2 dwords), value * 2^-8.
__device__ __forceinline__ u32x2 e4m3x4_to_f16x4_scaled(uint32_t w) {
    uint32_t lo = __builtin_amdgcn_perm(0u, w, 0x0c010c00u); // bytes b0, b1 -> bits 0-7, 16-23
    uint32_t hi = __builtin_amdgcn_perm(0u, w, 0x0c030c02u); // bytes b2, b3
    u32x2 r;
    r.x = e4m3x2_to_f16x2_scaled(lo);
    r.y = e4m3x2_to_f16x2_scaled(hi);
    return r;
}

// ------------------------------------------------------------------ wave helpers

__device__ __forceinline__ float shfl_xor(float v, int mask) { return __shfl_xor(v, mask, 64); }

__device__ __forceinline__ uint32_t lane_id() { return __lane_id(); }

// Max / sum over the lanes l, l^16, l^32, l^48 (the same position in the wave's four 16-lane
// rows) with the row-swap instructions: VALU moves, no LDS round trip as a shuffle takes.
// permlane16_swap(x, x) leaves x of the even row of each row pair in the first result and of
// the odd row in the second (in every lane of the pair); permlane32_swap does the same for the
// wave halves.  Both rows of a pair combine the two values in the same order.
__device__ __forceinline__ float rows_max(float x) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    const float y = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(y), __float_as_uint(y), false, false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float rows_sum(float x) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    const float y = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(y), __float_as_uint(y), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

template <typename T>
__device__ __forceinline__ T uniform(T v) {
    return __builtin_bit_cast(T, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, v)));
}

// The same for a pointer (two readfirstlanes).
template <typename T>
__device__ __forceinline__ T *uniform_ptr(T *v) {
    const uint64_t a = (uint64_t)(uintptr_t)v;
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)a);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(a >> 32));
    return (T *)(uintptr_t)(((uint64_t)hi << 32) | lo);
}

// MFMA 16x16x32 with f32 accumulation; operands are raw 16-byte register quads.
// A[m][k]: lane l holds row m = l%16, k = 8*(l/16) .. +7.  B[k][n]: lane l holds column
// n = l%16, the same k.  D[m][n]: lane l holds rows 4*(l/16) .. +3 of column l%16.
template <bool BF16>
__device__ __forceinline__ f32x4 mfma16x16x32(u32x4 a, u32x4 b, f32x4 c) {
    if constexpr (BF16)
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                       __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                      __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

// Hot-path packing of two floats into an MFMA operand word with the hardware
// round-to-nearest-even converts (v_cvt_pk_bf16_f32 / v_cvt_f16_f32).
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2;
typedef __attribute__((ext_vector_type(2))) _Float16 f16x2;
template <bool BF16>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
    if constexpr (BF16) {
        bf16x2 r = {(__bf16)a, (__bf16)b};
        return __builtin_bit_cast(uint32_t, r);
    } else {
        f16x2 r = {(_Float16)a, (_Float16)b};
        return __builtin_bit_cast(uint32_t, r);
    }
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Workgroup barrier for LDS exchanges: waits for this wave's LDS operations and meets the
// other waves.  The memory clobber keeps the compiler from moving any memory access across
// it (the s_barrier intrinsic alone does not); unlike __syncthreads - or an LDS-scoped
// fence, which must cover direct-to-LDS loads - nothing waits for vector loads in flight.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Inclusive scan of two values over the threads of a workgroup (wa / wb hold one value per
// wave): shuffle scans within each wave, then the wave totals through LDS (one barrier; wa /
// wb must not be rewritten until every thread has passed the next barrier).
__device__ __forceinline__ void block_scan2(uint32_t &a, uint32_t &b, uint32_t *wa, uint32_t *wb) {
    const uint32_t lane = threadIdx.x & 63, w = threadIdx.x >> 6;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const uint32_t x = __shfl_up(a, off), y = __shfl_up(b, off);
        if (lane >= (uint32_t)off) { a += x; b += y; }
    }
    if (lane == 63) { wa[w] = a; wb[w] = b; }
    lds_barrier();
    uint32_t pa = 0, pb = 0;
    for (uint32_t i = 0; i < w; i++) { pa += wa[i]; pb += wb[i]; }
    a += pa;
    b += pb;
}

// Inclusive scan of the first N of four values over the workgroup (thread order), through
// ws[value][wave].  With one_wave (every nonzero value in wave 0) the scan stays in wave 0:
// no barrier, and only wave 0's threads hold the sums.
template <int N, int W>
__device__ __forceinline__ void block_scan_n(uint32_t (&v)[4], uint32_t (*ws)[W], bool one_wave) {
    const uint32_t lane = threadIdx.x & 63, w = threadIdx.x >> 6;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
#pragma unroll
        for (int i = 0; i < N; i++) {
            const uint32_t x = __shfl_up(v[i], off);
            if (lane >= (uint32_t)off) v[i] += x;
        }
    }
    if (one_wave) return;
    if (lane == 63) {
#pragma unroll
        for (int i = 0; i < N; i++) ws[i][w] = v[i];
    }
    lds_barrier();
    uint32_t p[N] = {};
    for (uint32_t j = 0; j < w; j++) {
#pragma unroll
        for (int i = 0; i < N; i++) p[i] += ws[i][j];
    }
#pragma unroll
    for (int i = 0; i < N; i++) v[i] += p[i];
}

// Raw buffer resource over [base, base + bytes): loads at or past `bytes` return zeros and
// touch no memory, which lets a loop issue every load unconditionally.
constexpr int kBufferConfig = 0x00020000; // gfx9 raw buffer, 32-bit data format
// Callers pass wave-uniform values; the readfirstlanes state it, so the descriptor lives in
// SGPRs (a descriptor the compiler believes divergent costs a waterfall loop per load).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *base, uint32_t bytes) {
    const uint64_t a = (uint64_t)base;
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)a);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(a >> 32));
    void *ub = (void *)(((uint64_t)hi << 32) | lo);
    return __builtin_amdgcn_make_buffer_rsrc(ub, (short)0, __builtin_amdgcn_readfirstlane((int)bytes),
                                             kBufferConfig);
}

__device__ __forceinline__ u32x4 buffer_load16(__amdgpu_buffer_rsrc_t r, uint32_t voffset) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)voffset, 0, 0));
}

// Cache-policy operand of a buffer load: 0 (default) or 2 (nt, non-temporal: data read once).
template <int AUX = 0>
__device__ __forceinline__ u32x4 buffer_load16_p(__amdgpu_buffer_rsrc_t r, uint32_t voffset) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)voffset, 0, AUX));
}

} // namespace lia

// Read-only HBM stream (gfx950): the ceiling the library's HBM-bound kernels are measured
// against.  No counterpart in the reference; it exists so a benchmark can time, on the same
// device and in the same run, a contiguous read of exactly the bytes an attention launch reads.
//
// Each workgroup reads one contiguous share of [src, src + bytes) with 16-byte non-temporal
// buffer loads (the K/V loads' cache policy), kReadBatch loads in flight per lane, and folds
// every loaded word into one value written to sink[workgroup], so no load is dead code.
#include "common.hpp"
#include "launch.hpp"

namespace lia {

constexpr uint32_t kReadThreads = 256;
constexpr uint32_t kReadBatch = 8;
constexpr uint32_t kReadStep = kReadThreads * 16 * kReadBatch; // bytes per workgroup iteration

__global__ __launch_bounds__(kReadThreads) void hbm_read_kernel(const uint8_t *src, uint64_t bytes,
                                                                uint64_t share, uint32_t *sink) {
    const uint64_t begin = (uint64_t)blockIdx.x * share;
    const uint64_t end = min(bytes, begin + share);
    uint32_t acc = 0;
    for (uint64_t base = begin; base < end; base += kReadStep) {
        // descriptor over the rest of the share: loads past it return zeros and move no data
        const uint64_t left = end - base;
        const __amdgpu_buffer_rsrc_t r =
            make_rsrc(src + base, (uint32_t)min(left, (uint64_t)kReadStep));
        u32x4 x[kReadBatch];
#pragma unroll
        for (uint32_t k = 0; k < kReadBatch; k++)
            x[k] = buffer_load16_p<2>(r, (k * kReadThreads + threadIdx.x) * 16);
#pragma unroll
        for (uint32_t k = 0; k < kReadBatch; k++) acc ^= x[k].x ^ x[k].y ^ x[k].z ^ x[k].w;
    }
    // one word per workgroup: the XOR of everything its lanes read
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) acc ^= (uint32_t)__shfl_xor((int)acc, m, 64);
    __shared__ uint32_t waves[kReadThreads / 64];
    if ((threadIdx.x & 63) == 0) waves[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t v = 0;
        for (uint32_t w = 0; w < kReadThreads / 64; w++) v ^= waves[w];
        sink[blockIdx.x] = v;
    }
}

} // namespace lia

using namespace lia;

extern "C" int lia_hbm_read(const void *src, size_t bytes, uint32_t workgroups, uint32_t *sink,
                            lia_stream_t stream) {
    if (!src || !sink || bytes == 0 || workgroups == 0) return LIA_E_ARG;
    if ((uintptr_t)src & 15) return LIA_E_ALIGN;
    // 16-byte units, split evenly; a share is a whole number of 16-byte units
    const uint64_t units = (bytes + 15) / 16;
    const uint64_t share = (units + workgroups - 1) / workgroups * 16;
    if (share > 0xFFFFFFFFull) return LIA_E_UNSUPPORTED; // 32-bit buffer ranges
    const hipError_t e = launch<hbm_read_kernel>(dim3(workgroups), dim3(kReadThreads), 0,
                                                 (hipStream_t)stream, (const uint8_t *)src,
                                                 (uint64_t)bytes, share, sink);
    return e == hipSuccess ? LIA_OK : LIA_E_HIP;
}

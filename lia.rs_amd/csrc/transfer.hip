// KV page transfer in the reference's page wire format (gfx950).
//
// A page payload holds one physical page of every layer and plane, layer-major:
//   [layer][plane K=0, V=1][page_size][num_kv_heads][head_dim] pool elements
// (src/inference/paging_transfer.rs:4-5, MINICPM5_PAGE_BYTES = 42 x 2 x one 16 KB plane
// page), followed for FP8 pools by the page's scales [layer][plane][num_kv_heads] f32 (the
// reference has no FP8 pool).  Uploads stage a header (plane addresses, page ids) and the
// payloads in one contiguous buffer, copy it to the device once and scatter it with one
// kernel, like Upload::write + llama_upload_pages (paging_upload.rs:23-104,
// kernels/llama_transfer.rs:14-31).  Downloads gather the pages into the staging buffer
// with one kernel and copy them back once (the reference issues 84 plane copies per page,
// paging_transfer.rs:75-177).
#include <array>
#include <cstring>
#include <map>

#include "common.hpp"
#include "launch.hpp"

namespace lia {

constexpr uint32_t kMaxTransferPages = 16; // the reference's transfer window

// Staging header: 64-bit words.  [0, 2L): plane bases (layer * 2 + plane); [2L, 4L): FP8
// scale bases; then the page ids.  Payloads start at kv_header_bytes().
static inline size_t kv_header_bytes(uint32_t n_layers) {
    return (((size_t)4 * n_layers + kMaxTransferPages) * 8 + 255) & ~(size_t)255;
}

struct TransferGeom {
    uint32_t n_layers, plane_bytes, scale_bytes; // scale_bytes: per (layer, plane), 0 unless FP8
    uint64_t page_bytes;
    uint32_t header;
};

// One thread per 16 bytes of plane data or per 4-byte scale word of one page.
template <bool UPLOAD>
__global__ __launch_bounds__(256) void kv_pages_kernel(uint32_t n_pages, TransferGeom g,
                                                       uint8_t *staged) {
    const uint64_t *meta = (const uint64_t *)staged;
    const uint32_t planes = 2 * g.n_layers;
    const uint32_t vec_per_page = planes * (g.plane_bytes / 16);
    const uint32_t scale_words = planes * (g.scale_bytes / 4);
    const uint32_t per_page = vec_per_page + scale_words;
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    if (i >= n_pages * per_page) return;
    const uint32_t page = i / per_page, local = i % per_page;
    const uint64_t physical = meta[4 * g.n_layers + page];
    uint8_t *payload = staged + g.header + (size_t)page * g.page_bytes;
    if (local < vec_per_page) {
        const uint32_t plane = local / (g.plane_bytes / 16);
        const uint32_t offset = local % (g.plane_bytes / 16) * 16;
        uint8_t *pool = (uint8_t *)meta[plane] + physical * g.plane_bytes + offset;
        u32x4 *wire = (u32x4 *)(payload + (size_t)plane * g.plane_bytes + offset);
        if (UPLOAD) *(u32x4 *)pool = *wire;
        else *wire = *(const u32x4 *)pool;
    } else {
        const uint32_t w = local - vec_per_page;
        const uint32_t plane = w / (g.scale_bytes / 4), h = w % (g.scale_bytes / 4);
        float *scales = (float *)meta[2 * g.n_layers + plane] + physical * (g.scale_bytes / 4) + h;
        float *wire = (float *)(payload + (size_t)planes * g.plane_bytes + (size_t)plane * g.scale_bytes) + h;
        if (UPLOAD) *scales = *wire;
        else *wire = *scales;
    }
}

} // namespace lia

using namespace lia;

static int transfer_geom(const lia_kv_layout *L, uint32_t n_layers, TransferGeom *g) {
    if (!L || n_layers == 0 || n_layers > LIA_MAX_LAYERS) return LIA_E_ARG;
    if (L->num_kv_heads == 0 || L->head_dim == 0 || L->page_size == 0) return LIA_E_ARG;
    const uint32_t eb = L->dtype == LIA_FP8_E4M3 ? 1 : 2;
    if (L->dtype != LIA_F16 && L->dtype != LIA_BF16 && L->dtype != LIA_FP8_E4M3) return LIA_E_UNSUPPORTED;
    g->n_layers = n_layers;
    g->plane_bytes = L->page_size * L->num_kv_heads * L->head_dim * eb;
    if (g->plane_bytes % 16) return LIA_E_ALIGN;
    g->scale_bytes = L->dtype == LIA_FP8_E4M3 ? L->num_kv_heads * 4 : 0;
    g->page_bytes = (uint64_t)2 * n_layers * (g->plane_bytes + g->scale_bytes);
    g->header = (uint32_t)kv_header_bytes(n_layers);
    return LIA_OK;
}

extern "C" size_t lia_kv_page_bytes(const lia_kv_layout *layout, uint32_t n_layers) {
    TransferGeom g;
    return transfer_geom(layout, n_layers, &g) == LIA_OK ? (size_t)g.page_bytes : 0;
}

extern "C" size_t lia_kv_transfer_bytes(const lia_kv_layout *layout, uint32_t n_layers) {
    TransferGeom g;
    if (transfer_geom(layout, n_layers, &g) != LIA_OK) return 0;
    return g.header + (size_t)kMaxTransferPages * g.page_bytes;
}

// Validation and staging header shared by both directions (the ensure!s of
// write_kv_pages / validate_kv_page, paging_transfer.rs:37-74).
static int stage_header(const lia_kv_layout *L, const lia_kv_planes *planes, uint32_t n_pages,
                        const uint32_t *page_ids, void *staging_host, TransferGeom *g) {
    int st = transfer_geom(L, planes ? planes->n_layers : 0, g);
    if (st) return st;
    if (!page_ids || !staging_host) return LIA_E_ARG;
    if (n_pages == 0 || n_pages > kMaxTransferPages) return LIA_E_TRANSFER_WINDOW;
    for (uint32_t i = 0; i < n_pages; i++) {
        if (page_ids[i] >= L->pool_pages) return LIA_E_PAGE_RANGE;
        for (uint32_t j = 0; j < i; j++)
            if (page_ids[j] == page_ids[i]) return LIA_E_TRANSFER_DUPLICATE;
    }
    uint64_t *meta = (uint64_t *)staging_host;
    for (uint32_t l = 0; l < g->n_layers; l++) {
        if (!planes->k[l] || !planes->v[l]) return LIA_E_ARG;
        meta[2 * l] = (uint64_t)(uintptr_t)planes->k[l];
        meta[2 * l + 1] = (uint64_t)(uintptr_t)planes->v[l];
        if (g->scale_bytes) {
            if (!planes->k_scales[l] || !planes->v_scales[l]) return LIA_E_ARG;
            meta[2 * g->n_layers + 2 * l] = (uint64_t)(uintptr_t)planes->k_scales[l];
            meta[2 * g->n_layers + 2 * l + 1] = (uint64_t)(uintptr_t)planes->v_scales[l];
        } else {
            meta[2 * g->n_layers + 2 * l] = meta[2 * g->n_layers + 2 * l + 1] = 0;
        }
    }
    for (uint32_t i = 0; i < n_pages; i++) meta[4 * g->n_layers + i] = page_ids[i];
    return LIA_OK;
}

// Both directions end with a stream synchronisation, as the reference's do
// (paging_upload.rs:94-97, paging_transfer.rs:52-53 and 94-96): the staging buffers and the
// caller's payloads are free again when the call returns, also after an enqueue failure.
static int finish(hipStream_t s, int status) {
    const hipError_t e = hipStreamSynchronize(s);
    if (status != LIA_OK) return status;
    return e == hipSuccess ? LIA_OK : LIA_E_HIP;
}

// Timing-free events marking the end of each page's download, created once per thread and
// device (the thread's current device) and kept until the process ends, so concurrent calls
// from different threads with their own staging buffers never share an event.
static hipEvent_t *page_events() {
    thread_local std::map<int, std::array<hipEvent_t, kMaxTransferPages>> events;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return nullptr;
    auto it = events.find(dev);
    if (it == events.end()) {
        std::array<hipEvent_t, kMaxTransferPages> e{};
        for (auto &x : e)
            if (hipEventCreateWithFlags(&x, hipEventDisableTiming) != hipSuccess) return nullptr;
        it = events.emplace(dev, e).first;
    }
    return it->second.data();
}

static uint32_t pages_grid(const TransferGeom &g, uint32_t n_pages) {
    const uint32_t per_page = 2 * g.n_layers * (g.plane_bytes / 16 + g.scale_bytes / 4);
    return (n_pages * per_page + 255) / 256;
}

extern "C" int lia_kv_write_pages(const lia_kv_layout *layout, const lia_kv_planes *planes,
                                  uint32_t n_pages, const uint32_t *page_ids,
                                  const void *const *payloads, void *staging_host,
                                  void *staging_device, lia_stream_t stream) {
    TransferGeom g;
    if (!payloads || !staging_device) return LIA_E_ARG;
    int st = stage_header(layout, planes, n_pages, page_ids, staging_host, &g);
    if (st) return st;
    for (uint32_t i = 0; i < n_pages; i++)
        if (!payloads[i]) return LIA_E_ARG;
    // Each page's copy to the device is queued as soon as it is staged, so the DMA of page i
    // overlaps the host copy of page i + 1.
    hipStream_t s = (hipStream_t)stream;
    if (hipMemcpyAsync(staging_device, staging_host, g.header, hipMemcpyHostToDevice, s) != hipSuccess)
        return finish(s, LIA_E_HIP);
    for (uint32_t i = 0; i < n_pages; i++) {
        const size_t at = g.header + (size_t)i * g.page_bytes;
        memcpy((uint8_t *)staging_host + at, payloads[i], g.page_bytes);
        if (hipMemcpyAsync((uint8_t *)staging_device + at, (uint8_t *)staging_host + at, g.page_bytes,
                           hipMemcpyHostToDevice, s) != hipSuccess)
            return finish(s, LIA_E_HIP);
    }
    const hipError_t e = launch<kv_pages_kernel<true>>(dim3(pages_grid(g, n_pages)), dim3(256), 0, s,
                                                       n_pages, g, (uint8_t *)staging_device);
    return finish(s, e == hipSuccess ? LIA_OK : LIA_E_HIP);
}

extern "C" int lia_kv_read_pages(const lia_kv_layout *layout, const lia_kv_planes *planes,
                                 uint32_t n_pages, const uint32_t *page_ids, void *const *payloads,
                                 void *staging_host, void *staging_device, lia_stream_t stream) {
    TransferGeom g;
    if (!payloads || !staging_device) return LIA_E_ARG;
    int st = stage_header(layout, planes, n_pages, page_ids, staging_host, &g);
    if (st) return st;
    for (uint32_t i = 0; i < n_pages; i++)
        if (!payloads[i]) return LIA_E_ARG;
    hipStream_t s = (hipStream_t)stream;
    if (hipMemcpyAsync(staging_device, staging_host, g.header, hipMemcpyHostToDevice, s) != hipSuccess)
        return finish(s, LIA_E_HIP);
    if (launch<kv_pages_kernel<false>>(dim3(pages_grid(g, n_pages)), dim3(256), 0, s, n_pages, g,
                                       (uint8_t *)staging_device) != hipSuccess)
        return finish(s, LIA_E_HIP);
    // One device-to-host copy and one event per page: page i is copied out to the caller
    // while page i + 1 is still in flight.
    hipEvent_t *ev = page_events();
    if (!ev) return finish(s, LIA_E_HIP);
    for (uint32_t i = 0; i < n_pages; i++) {
        const size_t at = g.header + (size_t)i * g.page_bytes;
        if (hipMemcpyAsync((uint8_t *)staging_host + at, (uint8_t *)staging_device + at, g.page_bytes,
                           hipMemcpyDeviceToHost, s) != hipSuccess ||
            hipEventRecord(ev[i], s) != hipSuccess)
            return finish(s, LIA_E_HIP);
    }
    for (uint32_t i = 0; i < n_pages; i++) {
        if (hipEventSynchronize(ev[i]) != hipSuccess) return finish(s, LIA_E_HIP);
        memcpy(payloads[i], (uint8_t *)staging_host + g.header + (size_t)i * g.page_bytes, g.page_bytes);
    }
    return finish(s, LIA_OK);
}

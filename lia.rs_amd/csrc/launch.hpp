// Kernel launches through the library's gfx950 code object.
//
// Every kernel of the library is launched with hipModuleLaunchKernel on the hipFunction_t
// that hipGetFuncBySymbol resolves in the code object hipcc embeds in the shared library.
// The functions are resolved once per device and cached; lia_init resolves all of them for its
// device up front, so that the first step pays no code-object load.  The cached CU count
// is per device as well: the device is always the caller's current one.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>

#include "../../include/lia_hip.h"

namespace lia {

constexpr int kMaxLaunchDevices = 64;
constexpr int kMaxKernels = 128;

// One cached function per (kernel, device).  `host` is the kernel's host-side handle.
struct KernelSlot {
    const void *host;
    std::atomic<hipFunction_t> fn[kMaxLaunchDevices];
};

struct KernelRegistry {
    KernelSlot *slots[kMaxKernels];
    std::atomic<int> n{0};
};

inline KernelRegistry &kernel_registry() {
    static KernelRegistry r;
    return r;
}

inline KernelSlot *register_kernel(KernelSlot *s) {
    KernelRegistry &r = kernel_registry();
    const int i = r.n.fetch_add(1);
    if (i < kMaxKernels) r.slots[i] = s;
    return s;
}

inline int current_device(int *dev) {
    if (hipGetDevice(dev) != hipSuccess) return LIA_E_HIP;
    return *dev >= 0 && *dev < kMaxLaunchDevices ? LIA_OK : LIA_E_UNSUPPORTED;
}

// The function of `s` on device `dev` (the current device), resolved on first use.
inline hipFunction_t kernel_function(KernelSlot *s, int dev) {
    hipFunction_t f = s->fn[dev].load(std::memory_order_acquire);
    if (f) return f;
    if (hipGetFuncBySymbol(&f, s->host) != hipSuccess || !f) return nullptr;
    s->fn[dev].store(f, std::memory_order_release);
    return f;
}

// Resolves every registered kernel on the current device.
inline int resolve_kernels() {
    int dev = 0;
    if (const int e = current_device(&dev)) return e;
    KernelRegistry &r = kernel_registry();
    const int n = r.n.load();
    if (n > kMaxKernels) return LIA_E_UNSUPPORTED;
    for (int i = 0; i < n; ++i)
        if (!kernel_function(r.slots[i], dev)) return LIA_E_HIP;
    return LIA_OK;
}

template <typename T>
struct same_type {
    using type = T;
};

template <auto K, typename Sig = decltype(K)>
struct Launcher;

template <auto K, typename... P>
struct Launcher<K, void (*)(P...)> {
    static inline KernelSlot slot{reinterpret_cast<const void *>(K), {}};
    static inline KernelSlot *const registered = register_kernel(&slot);

    // Arguments are converted to the kernel's parameter types before their addresses go into
    // the parameter array, so the launch sees exactly the layout the kernel expects.
    static hipError_t go(dim3 grid, dim3 block, uint32_t shmem, hipStream_t s,
                         typename same_type<P>::type... args) {
        int dev = 0;
        if (current_device(&dev) != LIA_OK) return hipErrorInvalidDevice;
        const hipFunction_t f = kernel_function(registered, dev);
        if (!f) return hipErrorInvalidDeviceFunction;
        void *params[] = {static_cast<void *>(&args)...};
        return hipModuleLaunchKernel(f, grid.x, grid.y, grid.z, block.x, block.y, block.z, shmem,
                                     s, params, nullptr);
    }
};

// launch<kernel>(grid, block, shared bytes, stream, args...): a launch error is returned, not
// left pending for the next runtime call.
template <auto K, typename... A>
inline hipError_t launch(dim3 grid, dim3 block, uint32_t shmem, hipStream_t s, A &&...args) {
    return Launcher<K>::go(grid, block, shmem, s, static_cast<A &&>(args)...);
}

// Compute units of the current device, cached per device.  0 on failure.
inline uint32_t device_cus() {
    static std::atomic<uint32_t> cus[kMaxLaunchDevices];
    int dev = 0;
    if (current_device(&dev) != LIA_OK) return 0;
    uint32_t c = cus[dev].load(std::memory_order_relaxed);
    if (c) return c;
    int v = 0;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0)
        return 0;
    cus[dev].store((uint32_t)v, std::memory_order_relaxed);
    return (uint32_t)v;
}

} // namespace lia

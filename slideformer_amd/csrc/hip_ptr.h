// slideformer_amd: what kind of memory an address is, as the HIP runtime knows it.
//
// hipPointerGetAttributes is a lookup in the runtime's allocation table (~0.06 us
// on MI355X).  Device, managed and unified memory may be read and written by
// kernels in place; page-locked host memory (hipHostMalloc, torch pin_memory)
// is what the copy engines move directly; pageable memory is unknown to the
// runtime (unregistered, or an error on a host without a device).
#ifndef SLIDEFORMER_AMD_HIP_PTR_H
#define SLIDEFORMER_AMD_HIP_PTR_H

#include <hip/hip_runtime.h>

#include <cstring>

namespace la_ptr {

// The runtime's memory type of `ptr`, or hipMemoryTypeUnregistered when it
// does not know the address (the query's own failure is cleared, so that it
// is not reported by a later call).
inline hipMemoryType memory_type(const void* ptr)
{
    hipPointerAttribute_t a;
    std::memset(&a, 0, sizeof(a));
    if (hipPointerGetAttributes(&a, ptr) != hipSuccess) {
        (void)hipGetLastError();
        return hipMemoryTypeUnregistered;
    }
    return a.type;
}

// Memory the kernels may touch: device, managed or unified.
inline bool device_accessible(const void* ptr)
{
    const hipMemoryType t = memory_type(ptr);
    return t == hipMemoryTypeDevice || t == hipMemoryTypeManaged || t == hipMemoryTypeUnified;
}

// Page-locked host memory, which the copy engines read and write directly.
inline bool page_locked(const void* ptr) { return memory_type(ptr) == hipMemoryTypeHost; }

}  // namespace la_ptr

#endif  // SLIDEFORMER_AMD_HIP_PTR_H

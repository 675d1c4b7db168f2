// Thin C-ABI over the HIP runtime (declarations: include/gfd/hip_shim.h).
// The host C++ library calls the GPU only through these functions.
#include <hip/hip_runtime.h>

#include "gfd/hip_shim.h"

extern "C" {

int gfd_hip_device_count(int* n) { return (int)hipGetDeviceCount(n); }
int gfd_hip_get_device(int* dev) { return (int)hipGetDevice(dev); }
int gfd_hip_set_device(int dev) { return (int)hipSetDevice(dev); }
int gfd_hip_device_synchronize(void) { return (int)hipDeviceSynchronize(); }

int gfd_hip_pci_bus_id(char* buf, int len, int dev) {
    return (int)hipDeviceGetPCIBusId(buf, len, dev);
}

int gfd_hip_cu_count(int* n, int dev) {
    return (int)hipDeviceGetAttribute(n, hipDeviceAttributeMultiprocessorCount, dev);
}

const char* gfd_hip_error_string(int err) { return hipGetErrorString((hipError_t)err); }

int gfd_hip_host_alloc(void** p, size_t bytes, unsigned flags) {
    unsigned hf = hipHostMallocDefault;
    if (flags & GFD_HOST_COHERENT) hf |= hipHostMallocCoherent;
    if (flags & GFD_HOST_NONCOHERENT) hf |= hipHostMallocNonCoherent;
    if (flags & GFD_HOST_NUMA_USER) hf |= hipHostMallocNumaUser;
    return (int)hipHostMalloc(p, bytes, hf);
}

int gfd_hip_host_free(void* p) { return (int)hipHostFree(p); }

int gfd_hip_host_device_pointer(uint64_t* dptr, void* hptr) {
    void* d = nullptr;
    hipError_t e = hipHostGetDevicePointer(&d, hptr, 0);
    *dptr = (uint64_t)(uintptr_t)d;
    return (int)e;
}

int gfd_hip_malloc(void** p, size_t bytes) { return (int)hipMalloc(p, bytes); }
int gfd_hip_free(void* p) { return (int)hipFree(p); }

int gfd_hip_stream_create(gfd_stream_t* s) {
    hipStream_t st = nullptr;
    hipError_t e = hipStreamCreateWithFlags(&st, hipStreamNonBlocking);
    *s = (gfd_stream_t)st;
    return (int)e;
}

int gfd_hip_stream_destroy(gfd_stream_t s) { return (int)hipStreamDestroy((hipStream_t)s); }
int gfd_hip_stream_synchronize(gfd_stream_t s) { return (int)hipStreamSynchronize((hipStream_t)s); }

int gfd_hip_event_create(gfd_event_t* e, int enable_timing) {
    hipEvent_t ev = nullptr;
    hipError_t r = hipEventCreateWithFlags(&ev, enable_timing ? hipEventDefault
                                                              : hipEventDisableTiming);
    *e = (gfd_event_t)ev;
    return (int)r;
}

int gfd_hip_event_destroy(gfd_event_t e) { return (int)hipEventDestroy((hipEvent_t)e); }

int gfd_hip_event_record(gfd_event_t e, gfd_stream_t s) {
    return (int)hipEventRecord((hipEvent_t)e, (hipStream_t)s);
}

int gfd_hip_event_synchronize(gfd_event_t e) { return (int)hipEventSynchronize((hipEvent_t)e); }

int gfd_hip_event_query(gfd_event_t e) {
    hipError_t r = hipEventQuery((hipEvent_t)e);
    if (r == hipSuccess) return 0;
    if (r == hipErrorNotReady) return 1;
    return (int)r;
}

int gfd_hip_event_elapsed_ms(float* ms, gfd_event_t start, gfd_event_t stop) {
    return (int)hipEventElapsedTime(ms, (hipEvent_t)start, (hipEvent_t)stop);
}

int gfd_hip_stream_wait_event(gfd_stream_t s, gfd_event_t e) {
    return (int)hipStreamWaitEvent((hipStream_t)s, (hipEvent_t)e, 0);
}

int gfd_hip_memcpy_h2d_async(uint64_t dst, const void* src, size_t bytes, gfd_stream_t s) {
    return (int)hipMemcpyAsync((void*)(uintptr_t)dst, src, bytes, hipMemcpyHostToDevice,
                               (hipStream_t)s);
}

int gfd_hip_memcpy_d2h_async(void* dst, uint64_t src, size_t bytes, gfd_stream_t s) {
    return (int)hipMemcpyAsync(dst, (const void*)(uintptr_t)src, bytes, hipMemcpyDeviceToHost,
                               (hipStream_t)s);
}

int gfd_hip_memcpy_h2d(uint64_t dst, const void* src, size_t bytes) {
    return (int)hipMemcpy((void*)(uintptr_t)dst, src, bytes, hipMemcpyHostToDevice);
}

int gfd_hip_memcpy_d2h(void* dst, uint64_t src, size_t bytes) {
    return (int)hipMemcpy(dst, (const void*)(uintptr_t)src, bytes, hipMemcpyDeviceToHost);
}

int gfd_hip_memcpy_d2d(uint64_t dst, uint64_t src, size_t bytes) {
    return (int)hipMemcpy((void*)(uintptr_t)dst, (const void*)(uintptr_t)src, bytes,
                          hipMemcpyDeviceToDevice);
}

int gfd_hip_memset_d8(uint64_t dst, int value, size_t bytes) {
    return (int)hipMemset((void*)(uintptr_t)dst, value, bytes);
}

}  // extern "C"

extern "C" int gfd_hip_stream_write_u64(gfd_stream_t s, uint64_t dst, uint64_t value) {
    return (int)hipStreamWriteValue64((hipStream_t)s, (void*)(uintptr_t)dst, value, 0);
}

extern "C" int gfd_hip_pointer_is_device(const void* p) {
    hipPointerAttribute_t a;
    if (!p || hipPointerGetAttributes(&a, p) != hipSuccess) {
        (void)hipGetLastError();
        return 0;
    }
    return a.type == hipMemoryTypeDevice ? 1 : 0;
}

extern "C" int gfd_hip_device_range(uint64_t ptr, uint64_t* base, uint64_t* size) {
    hipPointerAttribute_t a;
    if (!ptr || hipPointerGetAttributes(&a, (const void*)(uintptr_t)ptr) != hipSuccess ||
        a.type != hipMemoryTypeDevice) {
        (void)hipGetLastError();
        return 0;
    }
    hipDeviceptr_t b = nullptr;
    size_t n = 0;
    if (hipMemGetAddressRange(&b, &n, (hipDeviceptr_t)(uintptr_t)ptr) != hipSuccess || !b) {
        (void)hipGetLastError();
        return 0;
    }
    *base = (uint64_t)(uintptr_t)b;
    *size = (uint64_t)n;
    return 1;
}

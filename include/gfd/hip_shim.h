#pragma once
// Thin C-ABI over the HIP runtime.  The host C++ library (poller, copy engine,
// staging pool, sessions) is compiled by the host compiler and reaches the GPU
// only through these functions; gfd_amd/csrc/hip_shim.hip is the single
// translation unit that includes the HIP runtime headers.
//
// Every function returns 0 on success, otherwise the hipError_t value.
#include <cstddef>
#include <cstdint>

extern "C" {

typedef void* gfd_stream_t;
typedef void* gfd_event_t;

// host allocation flags
enum {
    GFD_HOST_DEFAULT = 0,
    GFD_HOST_COHERENT = 1,     // fine-grained: CPU and GPU see each other's stores
    GFD_HOST_NONCOHERENT = 2,  // coarse-grained: GPU may cache, visibility at kernel bounds
    GFD_HOST_NUMA_USER = 4,    // follow the calling thread's NUMA policy
};

int gfd_hip_device_count(int* n);
int gfd_hip_get_device(int* dev);
int gfd_hip_set_device(int dev);
int gfd_hip_device_synchronize(void);
int gfd_hip_pci_bus_id(char* buf, int len, int dev);
int gfd_hip_cu_count(int* n, int dev);
const char* gfd_hip_error_string(int err);

int gfd_hip_host_alloc(void** p, size_t bytes, unsigned flags);
int gfd_hip_host_free(void* p);
int gfd_hip_host_device_pointer(uint64_t* dptr, void* hptr);
int gfd_hip_malloc(void** p, size_t bytes);
int gfd_hip_free(void* p);

int gfd_hip_stream_create(gfd_stream_t* s);  // non-blocking, default priority
int gfd_hip_stream_destroy(gfd_stream_t s);
int gfd_hip_stream_synchronize(gfd_stream_t s);
int gfd_hip_event_create(gfd_event_t* e, int enable_timing);
int gfd_hip_event_destroy(gfd_event_t e);
int gfd_hip_event_record(gfd_event_t e, gfd_stream_t s);
int gfd_hip_event_synchronize(gfd_event_t e);
int gfd_hip_event_query(gfd_event_t e);  // 0 done, 1 pending, <0 / other error
int gfd_hip_event_elapsed_ms(float* ms, gfd_event_t start, gfd_event_t stop);
int gfd_hip_stream_wait_event(gfd_stream_t s, gfd_event_t e);

int gfd_hip_memcpy_h2d_async(uint64_t dst, const void* src, size_t bytes, gfd_stream_t s);
int gfd_hip_memcpy_d2h_async(void* dst, uint64_t src, size_t bytes, gfd_stream_t s);
int gfd_hip_memcpy_h2d(uint64_t dst, const void* src, size_t bytes);
int gfd_hip_memcpy_d2h(void* dst, uint64_t src, size_t bytes);
int gfd_hip_memcpy_d2d(uint64_t dst, uint64_t src, size_t bytes);
int gfd_hip_memset_d8(uint64_t dst, int value, size_t bytes);

}  // extern "C"

extern "C" {
// Stream-ordered 8-byte store of `value` to device address `dst` (used for
// per-tile / per-list completion signals after the data copies).
int gfd_hip_stream_write_u64(gfd_stream_t s, uint64_t dst, uint64_t value);
}

extern "C" {
// Stream-ordered set-up of an SG session launch (a small kernel on `stream`):
// d_list_done[0 .. MAX_SG_LISTS) = 0, the SGDeviceCounters after them =
// *counters, trace[0 .. trace_words) = 0.  A HIP error code, 0 on success.
int gfd_sg_prepare_launch(uint64_t* d_list_done, const void* counters, uint64_t* trace, uint64_t trace_words,
                          gfd_stream_t stream);
}

extern "C" {
// 1 if `p` is device (HBM) memory, 0 if host / unknown.
int gfd_hip_pointer_is_device(const void* p);
// 1 and the device allocation [*base, *base + *size) holding ptr, or 0.
int gfd_hip_device_range(uint64_t ptr, uint64_t* base, uint64_t* size);
}

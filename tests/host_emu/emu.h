#pragma once
// Host-only emulation of the two runtime layers the poller stack calls (the
// HSA runtime used by SdmaQueue and the gfd_hip_* shim), so that the product
// sources cpu_polling.cpp, copy_engine.cpp, sdma.cpp, gather_engine.cpp,
// staging_pool.cpp and direct_submit.cpp run unchanged on a machine without a
// GPU.  Test infrastructure only: nothing here is linked into libgfd_amd.so.
//
// Copy engines are modelled the way the SDMA engines execute the packets the
// HSA runtime writes for hsa_amd_memory_async_copy[_on_engine]:
//   - each engine runs its packets strictly in submission order;
//   - a dependency is a poll of the dependency signal's value at the head of
//     the engine's ring, repeated until the value reads 0 (it is the signal's
//     value at poll time that counts, not the copy it belonged to when the
//     packet was written);
//   - completion atomically decrements the completion signal.
// "Device" memory is host memory; allocations are kept in a registry so that
// pointer queries answer as the runtime would.
#include <cstddef>
#include <cstdint>

namespace emu {

// Locked: host memory registered with the runtime (hipHostRegister-style),
// which the runtime reports as HSA_EXT_POINTER_TYPE_LOCKED with a GPU-side
// address of its own.
enum class Kind { Pinned, Device, Locked };

// Registry of live allocations made through the emulated shim.
void note_alloc(void* p, size_t n, Kind k);
// A locked range whose GPU-side base address is agent_base.
void note_locked(void* p, size_t n, uintptr_t agent_base);
void note_free(void* p);
// True and the allocation holding [p, p + n) if it is registered as `k`.
bool find_alloc(const void* p, size_t n, Kind k, uintptr_t* base, size_t* size);
// GPU-side base of the locked range starting at `base`.
uintptr_t locked_agent_base(uintptr_t base);

// Launches of the emulated zero-copy kernels (the Direct path's kernel
// route), so a scenario can tell which route a call took.
unsigned zero_copy_launches();

// Aborts the process, as a GPU page fault would end it, unless [p, p + n) is
// pinned host memory or device memory (n = 0 passes).
void require_gpu_access(const void* p, size_t n, const char* what);

// Engine stall watchdog: an engine that has polled one dependency for longer
// than this (GFD_EMU_STALL_MS, default 5000) prints what it waits on and ends
// the process with kStallExit, since in-order engines that wait on each other
// never recover.
constexpr int kStallExit = 86;

}  // namespace emu

// StagingPool (declaration: include/gfd/staging_pool.h).  Set and buffer
// bookkeeping follows include/gfd/staging_pool.h:50-176 of the reference; the
// allocation itself is hipHostMalloc with the allocating thread's NUMA policy
// bound to the requested node.
#include "gfd/staging_pool.h"

#include <linux/mempolicy.h>
#include <sys/syscall.h>
#include <unistd.h>

#include <cstring>

#include "gfd/hip_shim.h"
#include "gfd/log.h"
#include "gfd/pcie_topology.h"

namespace gfd {

namespace {

long set_policy(int mode, const unsigned long* mask, unsigned long maxnode) {
    return syscall(SYS_set_mempolicy, mode, mask, maxnode);
}

}  // namespace

StagingPool& StagingPool::instance() {
    static StagingPool pool;
    return pool;
}

// Buffers still allocated at process exit are left to the OS: the HIP runtime
// may already be torn down when static destructors run.
StagingPool::~StagingPool() {}

char* StagingPool::alloc_pinned(size_t bytes, int numa_node, bool* hugepage) {
    if (hugepage) *hugepage = false;
    void* p = nullptr;
    if (numa_node >= 0 && numa_node < 64) {
        // Bind this thread's policy to the node, let the driver allocate and
        // pin with that policy, then restore the default policy.
        unsigned long mask = 1UL << numa_node;
        if (set_policy(MPOL_BIND, &mask, sizeof(mask) * 8) == 0) {
            int err = gfd_hip_host_alloc(&p, bytes, GFD_HOST_NUMA_USER);
            set_policy(MPOL_DEFAULT, nullptr, 0);
            if (err == 0 && p) {
                std::memset(p, 0, bytes);  // fault every page in on this node now
                return (char*)p;
            }
            p = nullptr;
        }
    }
    if (gfd_hip_host_alloc(&p, bytes, GFD_HOST_DEFAULT) != 0) return nullptr;
    std::memset(p, 0, bytes);
    return (char*)p;
}

void StagingPool::free_pinned(char* p) {
    if (p) gfd_hip_host_free(p);
}

bool StagingPool::init(int num_gpus, size_t buf_size, int numa_node) {
    std::lock_guard<std::mutex> lock(mutex_);
    if (initialized_) return true;
    if (buf_size == 0 || buf_size > MAX_BUF_SIZE) {
        GFD_LOG_ERROR("StagingPool: buffer size %zu outside (0, %zu]\n", buf_size, MAX_BUF_SIZE);
        return false;
    }
    num_sets_ = num_gpus < 1 ? 1 : (num_gpus > MAX_BUFFER_SETS ? MAX_BUFFER_SETS : num_gpus);
    buf_size_ = buf_size;
    int ok_sets = 0;
    for (int s = 0; s < num_sets_; s++) {
        BufferSet& set = sets_[s];
        set.buf_size = buf_size;
        set.numa_node = numa_node >= 0 ? numa_node : discover_gpu_topology(s).numa_node;
        set.in_use = false;
        set.hugepage = false;
        bool ok = true;
        for (int b = 0; b < BUFS_PER_SET; b++) {
            set.bufs[b] = alloc_pinned(buf_size, set.numa_node, nullptr);
            if (!set.bufs[b]) {
                ok = false;
                break;
            }
        }
        if (ok) {
            ok_sets++;
        } else {
            for (int b = 0; b < BUFS_PER_SET; b++) {
                free_pinned(set.bufs[b]);
                set.bufs[b] = nullptr;
            }
            set.buf_size = 0;  // never handed out
        }
    }
    initialized_ = true;
    GFD_LOG_INFO("StagingPool: %d set(s) x %d x %zu bytes, NUMA %d%s\n", ok_sets, BUFS_PER_SET, buf_size,
                 numa_node, numa_node < 0 ? " (per GPU)" : "");
    return ok_sets > 0;
}

int StagingPool::choose_set(const BufferSet* sets, int n, size_t required_size, int numa_node) {
    int other = -1;
    for (int s = 0; s < n; s++) {
        const BufferSet& b = sets[s];
        if (b.in_use || b.buf_size < required_size || !b.bufs[0]) continue;
        if (numa_node < 0 || b.numa_node == numa_node) return s;
        if (other < 0) other = s;
    }
    return other;
}

int StagingPool::acquire_buffers(size_t required_size, int numa_node) {
    std::lock_guard<std::mutex> lock(mutex_);
    if (!initialized_) return -1;
    const int s = choose_set(sets_, num_sets_, required_size, numa_node);
    if (s >= 0) sets_[s].in_use = true;
    return s;
}

void StagingPool::get_buffers(int set_idx, char* out_bufs[BUFS_PER_SET], size_t& out_size,
                              bool& out_hugepage) {
    std::lock_guard<std::mutex> lock(mutex_);
    if (set_idx < 0 || set_idx >= num_sets_) return;
    for (int b = 0; b < BUFS_PER_SET; b++) out_bufs[b] = sets_[set_idx].bufs[b];
    out_size = sets_[set_idx].buf_size;
    out_hugepage = sets_[set_idx].hugepage;
}

void StagingPool::release_buffers(int set_idx) {
    std::lock_guard<std::mutex> lock(mutex_);
    if (set_idx >= 0 && set_idx < num_sets_) sets_[set_idx].in_use = false;
}

void StagingPool::shutdown() {
    std::lock_guard<std::mutex> lock(mutex_);
    if (!initialized_) return;
    for (int s = 0; s < num_sets_; s++) {
        if (sets_[s].in_use) {
            GFD_LOG_ERROR("StagingPool: set %d still in use at shutdown; leaving it allocated\n", s);
            continue;
        }
        for (int b = 0; b < BUFS_PER_SET; b++) {
            free_pinned(sets_[s].bufs[b]);
            sets_[s].bufs[b] = nullptr;
        }
    }
    initialized_ = false;
}

}  // namespace gfd

#pragma once
// StagingPool: process-wide pre-allocated pinned staging buffers, one set of
// BUFS_PER_SET buffers per GPU poller (include/gfd/staging_pool.h:29-189 of
// the reference).
//
// MI355X allocation order: hipHostMalloc with the NUMA-user flag while the
// allocating thread's memory policy is bound to the GPU-local node (pages land
// on that node and are pinned by the driver), then madvise(MADV_HUGEPAGE);
// if that fails, a plain hipHostMalloc.  Registering an existing mmap'd
// hugetlb region (the reference's first choice) is not used: registering
// already-mapped memory is not supported on the target systems.
#include <cstddef>
#include <mutex>

namespace gfd {

class StagingPool {
public:
    static constexpr int MAX_BUFFER_SETS = 8;
    static constexpr int BUFS_PER_SET = 5;
    static constexpr size_t MAX_BUF_SIZE = 1024ull * 1024 * 1024;  // 1 GiB per buffer

    struct BufferSet {
        char* bufs[BUFS_PER_SET] = {};
        size_t buf_size = 0;
        bool hugepage = false;  // true when THP was requested and granted for every buffer
        bool in_use = false;
        int numa_node = 0;
    };

    static StagingPool& instance();

    // Allocate `num_gpus` sets of BUFS_PER_SET buffers of `buf_size` bytes on
    // `numa_node` (-1: no binding).  Returns true if at least one set exists.
    bool init(int num_gpus, size_t buf_size, int numa_node = 0);

    // Claim a free set whose buffers hold >= required_size; -1 if none.
    int acquire_buffers(size_t required_size, int numa_node = 0);
    void get_buffers(int set_idx, char* out_bufs[BUFS_PER_SET], size_t& out_size,
                     bool& out_hugepage);
    void release_buffers(int set_idx);

    bool is_initialized() const { return initialized_; }
    size_t buffer_size() const { return buf_size_; }
    void shutdown();

    // Pinned allocation helper shared with the poller's self-allocation path.
    // Returns nullptr on failure; *hugepage tells whether THP was applied.
    static char* alloc_pinned(size_t bytes, int numa_node, bool* hugepage);
    static void free_pinned(char* p);

private:
    StagingPool() = default;
    ~StagingPool();
    StagingPool(const StagingPool&) = delete;
    StagingPool& operator=(const StagingPool&) = delete;

    std::mutex mutex_;
    bool initialized_ = false;
    int num_sets_ = 0;
    size_t buf_size_ = 0;
    BufferSet sets_[MAX_BUFFER_SETS];
};

}  // namespace gfd

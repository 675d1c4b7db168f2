#pragma once
// StagingPool: process-wide pre-allocated pinned staging buffers, one set of
// BUFS_PER_SET buffers per GPU poller (include/gfd/staging_pool.h:29-189 of
// the reference).  Lifecycle as in the reference: init() once, each poller's
// init_copy_engine() acquires a set (falling back to allocating its own when
// none fits), the poller's destructor releases it, shutdown() at the end.
//
// MI355X allocation: hipHostMalloc with the NUMA-user flag while the
// allocating thread's memory policy is bound to the set's node, so the pages
// land on that node and are pinned by the driver; if that fails, a plain
// hipHostMalloc.  The driver picks the page size of pinned allocations, so
// `hugepage` is always false.  The reference's first choice, registering an
// mmap'd hugetlb region, is not used: registering memory that is already
// mapped is refused on the target systems.
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
        bool hugepage = false;  // always false here (see above)
        bool in_use = false;
        int numa_node = 0;      // node the buffers are bound to (-1: none)
    };

    static StagingPool& instance();

    // Allocate `num_gpus` sets of BUFS_PER_SET buffers of `buf_size` bytes.
    // numa_node >= 0: every set on that node (the reference's behaviour);
    // -1: set g on the node of GPU g (sysfs), unbound where none is reported.
    // Returns true if at least one set exists.
    bool init(int num_gpus, size_t buf_size, int numa_node = 0);

    // Claim a free set whose buffers hold >= required_size, preferring one on
    // `numa_node` (any node when -1); another node's set only when no set on
    // it is free.  -1 if none fits (the caller then allocates its own).
    int acquire_buffers(size_t required_size, int numa_node = 0);
    void get_buffers(int set_idx, char* out_bufs[BUFS_PER_SET], size_t& out_size,
                     bool& out_hugepage);
    void release_buffers(int set_idx);

    bool is_initialized() const { return initialized_; }
    size_t buffer_size() const { return buf_size_; }
    void shutdown();

    // Pinned allocation helper shared with the poller's self-allocation path.
    // Returns nullptr on failure; *hugepage (optional) is set to false.
    static char* alloc_pinned(size_t bytes, int numa_node, bool* hugepage);
    static void free_pinned(char* p);

    // The selection rule of acquire_buffers over `n` sets (no locking): a
    // free, large enough set on `numa_node` first, else any free, large enough
    // set; -1 if none.
    static int choose_set(const BufferSet* sets, int n, size_t required_size, int numa_node);
    int num_sets() const { return num_sets_; }

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

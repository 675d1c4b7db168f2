// Host-side checks of the SG session's device-counter layout and the helpers
// device code uses to reach it without reading the host queue: the counters
// sit right after d_list_done[MAX_SG_LISTS] (include/gfd/sg_task_queue.h),
// sg_list_done_words() walks back from the counters to that array, and
// sg_idle_ticks() turns the queue's idle limit (0 = 30 s) into 100 MHz ticks.
// Header-only: it needs no GPU and no library.
#include <cstddef>
#include <cstdio>
#include <memory>
#include <vector>

#include "gfd/sg_task_queue.h"
#include "gfd/tiled_queue.h"

static int failures = 0;
#define CHECK(c)                                                         \
    do {                                                                 \
        if (!(c)) {                                                      \
            std::fprintf(stderr, "%s:%d: check failed: %s\n", __FILE__, __LINE__, #c); \
            failures++;                                                  \
        }                                                                \
    } while (0)

int main() {
    using namespace gfd;
    // Three cache lines, each new field in a word the old padding held.
    CHECK(sizeof(SGDeviceCounters) == 192);
    CHECK(SG_DEVICE_COUNTER_WORDS == 24);
    CHECK(offsetof(SGDeviceCounters, idle_ticks) == offsetof(SGDeviceCounters, stop_at) + 8);
    CHECK(offsetof(SGDeviceCounters, stop_at) == offsetof(SGDeviceCounters, entry_first) + 8);
    CHECK(sizeof(TileDeviceCounters) == 64);

    // A session's device words: d_list_done[MAX_SG_LISTS], then the counters.
    std::vector<uint64_t> words(MAX_SG_LISTS + SG_DEVICE_COUNTER_WORDS, 0);
    std::unique_ptr<SGTaskQueue> sq(new SGTaskQueue());
    sq->d_list_done = words.data();
    SGDeviceCounters* c = sg_device_counters(sq.get());
    CHECK(reinterpret_cast<uint64_t*>(c) == words.data() + MAX_SG_LISTS);
    CHECK(sg_list_done_words(c) == words.data());
    CHECK(&sg_list_done_words(c)[MAX_SG_LISTS - 1] == &words[MAX_SG_LISTS - 1]);
    c->idle_ticks = 7;
    CHECK(words[MAX_SG_LISTS + offsetof(SGDeviceCounters, idle_ticks) / 8] == 7);

    CHECK(sg_idle_ticks(0) == 30000ull * 100000ull);
    CHECK(sg_idle_ticks(1) == 100000ull);
    CHECK(sg_idle_ticks(10000) == 1000000000ull);
    CHECK(sg_idle_ticks(0xFFFFFFFFu) == 0xFFFFFFFFull * 100000ull);  // no 32-bit overflow

    if (failures) {
        std::fprintf(stderr, "%d check(s) failed\n", failures);
        return 1;
    }
    std::printf("PASSED\n");
    return 0;
}

#pragma once
// Private pieces of CpuPollingThread shared by its translation units.
#include "gfd/cpu_polling.h"

namespace gfd {

// Ring of completion points, oldest at `tail`.
struct CpuPollingThread::CompletionFifo {
    static constexpr int N = 32;
    CompletionSlot slots[N];
    int head = 0;
    int tail = 0;
    int count = 0;
};

}  // namespace gfd

// tq_sync.hip -- the per-stream counter blocks of the kernels whose workgroups count or wait for each
// other (SyncCounters in tq_internal.h): a file-scope device array, zero when the module loads, one block
// handed to each stream that issues such a call on a device. Host code reaches the array through the
// address hipGetSymbolAddress reports for the current device (the symbol's name is not a device address).
#include "tq_internal.h"

#include <mutex>

namespace tq {

__device__ __align__(256) SyncCounters g_sync[SYNC_STREAMS];

SyncCounters *sync_counters(hipStream_t stream) {
    constexpr int MAX_DEVICES = 64;
    // a fixed table (no host allocation either): the streams holding each device's blocks, in order
    static std::mutex mu;
    static SyncCounters *base[MAX_DEVICES] = {nullptr};
    static hipStream_t owner[MAX_DEVICES][SYNC_STREAMS];
    static int used[MAX_DEVICES] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEVICES) return nullptr;
    std::lock_guard<std::mutex> lock(mu);
    if (!base[dev]) {
        void *p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(g_sync)) != hipSuccess || !p) {
            (void)hipGetLastError();
            return nullptr;
        }
        base[dev] = (SyncCounters *)p;
    }
    for (int i = 0; i < used[dev]; ++i)
        if (owner[dev][i] == stream) return base[dev] + i;
    if (used[dev] == SYNC_STREAMS) return nullptr;
    owner[dev][used[dev]] = stream;
    return base[dev] + used[dev]++;
}

}  // namespace tq

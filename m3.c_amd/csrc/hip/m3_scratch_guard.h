/*
 * m3_scratch_guard.h - one caller at a time on a device's static scan
 * scratch (m3_hip_scan_views_static). The scratch is one array per GPU,
 * shared by every handle the process opens on it; two calls that overlap
 * on one GPU would mix their flags. The guard is a per-ordinal flag taken
 * with a compare-and-swap on entry and cleared on exit: a second caller is
 * refused rather than raced. Plain C++ (no HIP), so that the CPU tests can
 * compile it on its own.
 */
#ifndef M3_SCRATCH_GUARD_H
#define M3_SCRATCH_GUARD_H

#include <atomic>

template <int N>
struct m3_scratch_guard {
    std::atomic<int> busy[N] = {};

    /* true when `ordinal` was free and is now held by the caller */
    bool acquire(int ordinal)
    {
        int expected = 0;

        return ordinal >= 0 && ordinal < N &&
               busy[ordinal].compare_exchange_strong(
                   expected, 1, std::memory_order_acquire,
                   std::memory_order_relaxed);
    }

    void release(int ordinal)
    {
        if (ordinal >= 0 && ordinal < N) {
            busy[ordinal].store(0, std::memory_order_release);
        }
    }
};

#endif

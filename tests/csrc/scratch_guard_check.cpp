// The static-scratch guard (m3.c_amd/csrc/hip/m3_scratch_guard.h) on the
// CPU: a held ordinal refuses a second caller, other ordinals stay free,
// out-of-range ordinals are refused, release frees it again, and under
// many threads at most one holder per ordinal exists at any time.
#include "m3_scratch_guard.h"

#include <cstdio>
#include <thread>
#include <vector>

int main()
{
    static m3_scratch_guard<4> guard;
    int failures = 0;
    auto expect = [&](bool ok, const char *what) {
        if (!ok) {
            std::printf("FAIL: %s\n", what);
            ++failures;
        }
    };

    expect(guard.acquire(1), "first acquire of ordinal 1");
    expect(!guard.acquire(1), "second acquire of a held ordinal refused");
    expect(guard.acquire(2), "another ordinal is independent");
    expect(!guard.acquire(-1) && !guard.acquire(4), "out of range refused");
    guard.release(1);
    expect(guard.acquire(1), "acquire after release");
    guard.release(1);
    guard.release(2);
    guard.release(7); /* out of range: ignored */

    /* mutual exclusion under contention */
    static std::atomic<int> holders[4];
    static std::atomic<int> violations{0};
    static std::atomic<long> granted{0};
    std::vector<std::thread> threads;
    for (int t = 0; t < 8; ++t) {
        threads.emplace_back([t] {
            for (int k = 0; k < 200000; ++k) {
                const int ordinal = (t + k) & 3;
                if (guard.acquire(ordinal)) {
                    if (holders[ordinal].fetch_add(1) != 0) {
                        violations.fetch_add(1);
                    }
                    granted.fetch_add(1);
                    holders[ordinal].fetch_sub(1);
                    guard.release(ordinal);
                }
            }
        });
    }
    for (std::thread &thread : threads) {
        thread.join();
    }
    expect(violations.load() == 0, "two holders of one ordinal at once");
    expect(granted.load() > 0, "some acquisitions succeed");
    std::printf("granted %ld, violations %d\n", granted.load(),
                violations.load());
    return failures == 0 ? 0 : 1;
}

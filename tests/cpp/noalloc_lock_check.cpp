// Host check of the no-allocation scratch lock (pj_host_lock.h): a second
// caller on the same device waits until the first releases it, callers on
// other devices do not wait, and the lock is free again afterwards.
#include <atomic>
#include <chrono>
#include <cstdio>
#include <thread>

#include "pj_host_lock.h"

using clk = std::chrono::steady_clock;

int main() {
    std::atomic<int> held{0};
    clk::time_point released, acquired, other;
    std::thread a([&] {
        std::unique_lock<std::mutex> g(pj::noalloc_lock(0));
        held = 1;
        std::this_thread::sleep_for(std::chrono::milliseconds(200));
        released = clk::now();
    });
    while (!held) std::this_thread::yield();
    std::thread b([&] {
        std::unique_lock<std::mutex> g(pj::noalloc_lock(0));
        acquired = clk::now();
    });
    std::thread c([&] {
        std::unique_lock<std::mutex> g(pj::noalloc_lock(1));
        other = clk::now();
    });
    a.join();
    b.join();
    c.join();
    if (acquired < released) { std::printf("FAIL: second caller on device 0 did not wait\n"); return 1; }
    if (!(other < released)) { std::printf("FAIL: device 1 waited for device 0\n"); return 1; }
    if (!pj::noalloc_lock(0).try_lock()) { std::printf("FAIL: lock not released\n"); return 1; }
    pj::noalloc_lock(0).unlock();
    std::printf("noalloc lock checks passed\n");
    return 0;
}

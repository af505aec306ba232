// Launch timer: events stamped by the dispatch of every launch of one kernel family
// (hipExtLaunchKernelGGL's start / stop events), so a caller reads the device duration of each
// such launch made inside its own timed loop (the benchmark's roofline figure) without extra
// packets on the stream.  Disarmed it costs one relaxed load per launch; nothing here
// allocates device memory.
#include <atomic>
#include <mutex>
#include <string.h>
#include <vector>

#include "common.hpp"

namespace tpw {

namespace {

struct Timer {
    std::mutex mu;
    char family[64] = "";
    std::vector<hipEvent_t> ev;  // start / stop pairs
    int capacity = 0;            // pairs armed
    int used = 0;                // pairs handed out
    int dropped = 0;             // launches past the capacity
    int device = -1;
};

Timer g_timer;
std::atomic<int> g_armed{0};

}  // namespace

LaunchEvents launch_events(const char *family) {
    LaunchEvents e;
    if (!g_armed.load(std::memory_order_relaxed)) return e;
    std::lock_guard<std::mutex> lk(g_timer.mu);
    if (!g_armed.load(std::memory_order_relaxed) || strcmp(family, g_timer.family) != 0) return e;
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev != g_timer.device) return e;
    if (g_timer.used >= g_timer.capacity) {
        ++g_timer.dropped;
        return e;
    }
    const int slot = g_timer.used++;
    e.start = g_timer.ev[2 * slot];
    e.stop = g_timer.ev[2 * slot + 1];
    return e;
}

__global__ void empty_kernel() {}

}  // namespace tpw

using namespace tpw;

extern "C" int tpw_empty_launches(int count, void *stream) {
    TPW_REQUIRE(count >= 0, "count must be >= 0");
    for (int i = 0; i < count; ++i) hipLaunchKernelGGL(empty_kernel, dim3(1), dim3(64), 0, as_stream(stream));
    return check_launch("tpw_empty_launches");
}

extern "C" int tpw_launch_timer_arm(const char *family, int capacity) {
    TPW_REQUIRE(family && strlen(family) > 0 && strlen(family) < sizeof(g_timer.family), "invalid kernel family");
    TPW_REQUIRE(capacity > 0 && capacity <= (1 << 20), "capacity must be in 1 .. 2^20");
    std::lock_guard<std::mutex> lk(g_timer.mu);
    int dev = -1;
    TPW_REQUIRE(hipGetDevice(&dev) == hipSuccess, "no current HIP device");
    if (dev != g_timer.device) {  // events belong to the device current at creation
        for (hipEvent_t e : g_timer.ev) (void)hipEventDestroy(e);
        g_timer.ev.clear();
        g_timer.device = dev;
    }
    while ((int)g_timer.ev.size() < 2 * capacity) {
        hipEvent_t e;
        TPW_REQUIRE(hipEventCreate(&e) == hipSuccess, "hipEventCreate failed");
        g_timer.ev.push_back(e);
    }
    strcpy(g_timer.family, family);
    g_timer.capacity = capacity;
    g_timer.used = 0;
    g_timer.dropped = 0;
    g_armed.store(1, std::memory_order_relaxed);
    return TPW_OK;
}

extern "C" int tpw_launch_timer_read(float *ms, int capacity, int *count, int *dropped) {
    TPW_REQUIRE(count && (ms || capacity == 0) && capacity >= 0, "invalid arguments");
    std::lock_guard<std::mutex> lk(g_timer.mu);
    g_armed.store(0, std::memory_order_relaxed);
    const int used = g_timer.used;
    *count = used;
    if (dropped) *dropped = g_timer.dropped;
    for (int i = 0; i < used && i < capacity; ++i) {
        TPW_REQUIRE(hipEventSynchronize(g_timer.ev[2 * i + 1]) == hipSuccess, "hipEventSynchronize failed");
        TPW_REQUIRE(hipEventElapsedTime(&ms[i], g_timer.ev[2 * i], g_timer.ev[2 * i + 1]) == hipSuccess,
                    "hipEventElapsedTime failed");
    }
    g_timer.used = 0;
    return TPW_OK;
}

// Optional stage timing for measurement runs: start/stop HIP events passed to
// the first and last kernel launch of selected stages (hipExtLaunchKernelGGL
// takes the timestamps from the kernels' dispatches).  Disabled (one branch
// per launch) unless lrmoe_timing_enable() is called; never enable it while a
// stream is being captured into a graph.
#include <vector>

#include "lrmoe_internal.h"

namespace lrmoe {
namespace {

struct Timing {
    int mask = 0;
    int capacity = 0;
    std::vector<hipEvent_t> events[6];  // per stage: start, stop, start, stop, ...
    int used[6] = {0, 0, 0, 0, 0, 0};
};

Timing& timing() {
    static Timing t;
    return t;
}

int stage_index(int stage) {
    for (int i = 0; i < 6; ++i) {
        if (stage == (1 << i)) return i;
    }
    return -1;
}

}  // namespace

StageEvents timing_events(int stage) {
    Timing& t = timing();
    StageEvents ev;
    if (!(t.mask & stage)) return ev;
    const int i = stage_index(stage);
    if (i < 0 || t.used[i] + 2 > 2 * t.capacity) return ev;
    ev.start = t.events[i][t.used[i]];
    ev.stop = t.events[i][t.used[i] + 1];
    t.used[i] += 2;
    return ev;
}

}  // namespace lrmoe

extern "C" {

// Enables timing for the stages in `mask` (LRMOE_STAGE_* bits) with room for
// `launches` launches per stage; mask 0 disables and frees the events.
int lrmoe_timing_enable(int mask, int launches) {
    using lrmoe::timing;
    auto& t = timing();
    for (auto& list : t.events) {
        for (hipEvent_t e : list) (void)hipEventDestroy(e);
        list.clear();
    }
    for (int& u : t.used) u = 0;
    t.mask = 0;
    t.capacity = 0;
    if (mask == 0) return LRMOE_OK;
    if (launches <= 0 || launches > (1 << 20) || (mask & ~63)) return LRMOE_E_ARG;
    for (int i = 0; i < 6; ++i) {
        if (!(mask & (1 << i))) continue;
        t.events[i].resize(2 * static_cast<size_t>(launches));
        for (auto& e : t.events[i]) {
            const hipError_t err = hipEventCreate(&e);
            if (err != hipSuccess) return static_cast<int>(err);
        }
    }
    t.capacity = launches;
    t.mask = mask;
    return LRMOE_OK;
}

// Waits for the recorded events of `stage` and returns the summed
// start->stop time in milliseconds and the number of timed launches, then
// rewinds that stage's event list.
int lrmoe_timing_collect(int stage, double* total_ms, int* launches) {
    using lrmoe::timing;
    if (!total_ms || !launches) return LRMOE_E_ARG;
    auto& t = timing();
    const int i = lrmoe::stage_index(stage);
    if (i < 0 || !(t.mask & stage)) return LRMOE_E_ARG;
    double sum = 0.0;
    const int pairs = t.used[i] / 2;
    for (int p = 0; p < pairs; ++p) {
        hipError_t err = hipEventSynchronize(t.events[i][2 * p + 1]);
        if (err != hipSuccess) return static_cast<int>(err);
        float ms = 0.0f;
        err = hipEventElapsedTime(&ms, t.events[i][2 * p], t.events[i][2 * p + 1]);
        if (err != hipSuccess) return static_cast<int>(err);
        sum += ms;
    }
    *total_ms = sum;
    *launches = pairs;
    t.used[i] = 0;
    return LRMOE_OK;
}

}  // extern "C"

// Host-side state of a pcl_context (shared by the attention entry points and
// the device-resident layer cache).
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <vector>

// Event pair of one timed kernel role in one launch.
struct TimedSpan {
    hipEvent_t start, stop;
    int role;
};

struct pcl_context {
    int device = 0;
    hipStream_t stream = nullptr;
    bool own_stream = false;
    void *ws = nullptr;
    size_t ws_bytes = 0;
    int *err = nullptr;
    // Staging buffers of the host-pointer entries (grow-only).
    void *stage[5] = {nullptr, nullptr, nullptr, nullptr, nullptr};
    size_t stage_bytes[5] = {0, 0, 0, 0, 0};
    // per-kernel timing: recorded spans and a pool of free events
    bool timing = false;
    std::vector<TimedSpan> spans;
    std::vector<hipEvent_t> free_events;
};

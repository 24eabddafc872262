// Host-side state of a pcl_context and of a layer cache (shared by the
// attention entry points, the layer cache and the head transform).
#pragma once

#include <hip/hip_runtime.h>

#include "pcl_attention.h"

#include <cstddef>
#include <cstdint>
#include <functional>
#include <vector>

// Event pair of one timed kernel role in one launch.
struct TimedSpan {
    hipEvent_t start, stop;
    int role;
};

constexpr int kStageSlots = 7;

struct pcl_context {
    int device = 0;
    hipStream_t stream = nullptr;
    bool own_stream = false;
    void *ws = nullptr;
    size_t ws_bytes = 0;
    // epoch generation for which the workspace's published-word region was
    // last zeroed
    uint32_t ws_tag_gen = 0;
    int *err = nullptr;
    // this device's scratch of pcl_attention_launch_noalloc (never freed)
    void *noalloc_scratch = nullptr;
    // Staging buffers of the host-pointer entries (grow-only): Q, the shared
    // K and V upload, the mask, the output, a private K and V.
    void *stage[kStageSlots] = {};
    size_t stage_bytes[kStageSlots] = {};
    // bound of the spread decode's waits for other workgroups (polls)
    int wait_polls = 1 << 16;
    // per-kernel timing: recorded spans and a pool of free events
    bool timing = false;
    std::vector<TimedSpan> spans;
    std::vector<hipEvent_t> free_events;
};

// A device-resident layer cache: rows [start, len) of k / v are retained.
struct pcl_kv_cache {
    pcl_context *ctx = nullptr;
    int64_t kvheads = 0, dim = 0, width = 0; // width = floats per token
    int64_t context = 0, window = 0;
    size_t max_bytes = 0;
    int64_t total = 0; // positions processed (LayerCache::total)
    int64_t start = 0; // first retained row
    int64_t len = 0;   // rows in the buffers
    int64_t cap = 0;   // rows the buffers hold
    float *k = nullptr, *v = nullptr;
};

struct pcl_kv_pending;

namespace pcl {

// Checks the position and byte limits of an n-row step and makes room for
// its rows after the retained ones (the cache is unchanged on an error).
int kv_cache_reserve(pcl_kv_cache *c, int64_t n);
// Records the step in *pending and counts its n rows (written at row len).
void kv_cache_advance_rows(pcl_kv_cache *c, int64_t n, pcl_kv_pending *pending);

// A one-token decode step's head transform (the token's raw rows, the
// learned scales, the (sin, cos) pairs of its position, the norm epsilon)
// and where its prepared rows go: the new key's K and V rows and the
// prepared queries.
struct StepFold {
    const float *rq, *rk, *rv, *qs, *ks, *rot;
    float *nk, *nv, *qo;
    float eps;
};

// The attention launch of `desc` (one query) with the step's transform:
// folded into the launch when the planned kernel runs it (the pipelined
// decode at head dims 64-512), otherwise `separate` (the transform's own
// launch on the same stream) runs first. Validation errors return before
// anything is launched.
int launch_step(pcl_context *ctx, const pcl_attention_desc &desc, const StepFold &fold,
                const std::function<int()> &separate);

} // namespace pcl

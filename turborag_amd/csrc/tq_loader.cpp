// tq_loader.cpp — layer-pipelined load of compressed KV into cache layout.
//
// The reference loads a document layer by layer (tq_backend/cag_store.py:
// 161-288): read the layer's .bin pages, copy them to the GPU (pageable,
// synchronous), dequantize to [N, H, D], then permute to the DynamicCache
// layout [1, H, N, D] with an extra copy.  Here one call enqueues every
// layer: layer l's pages go host -> device on the copy stream while layer
// l-1 is dequantized on the compute stream straight into [1, H, N, D]; the
// compute stream waits for each layer's copy through an event.  With pinned
// host pages (hipHostMalloc / torch pin_memory) the copies run at link rate
// and overlap the dequant.
#include <map>
#include <memory>
#include <mutex>
#include <vector>

#include "tq_internal.h"

namespace {

// Per-device events of the loader.  A call holds its device's lock for its
// whole enqueue loop, so two concurrent calls never record and wait on the
// same event in between each other's record and wait (a stream wait takes
// the event's state when it is enqueued, so the events can be re-recorded by
// the next call).  The per-device records never move once created.
struct DeviceEvents {
    std::mutex mu;
    std::vector<hipEvent_t> ev;
};

DeviceEvents& device_events(int dev) {
    static std::mutex mu;
    static std::map<int, std::unique_ptr<DeviceEvents>> all;
    std::lock_guard<std::mutex> lock(mu);
    auto& p = all[dev];
    if (!p) p.reset(new DeviceEvents());
    return *p;
}

void check(hipError_t e, const char* what) {
    if (e != hipSuccess) {
        (void)hipGetLastError();
        throw tq::Error(std::string(what) + ": " + hipGetErrorString(e));
    }
}

}  // namespace

namespace tq {

void load_layers(Scheme s, const uint8_t* const* host_pools, uint8_t* const* device_pools,
                 size_t pool_bytes, int num_layers, const int32_t* slots, int num_tokens,
                 uint16_t* const* out_key, uint16_t* const* out_value, const PageGeom& g,
                 hipStream_t copy_stream, hipStream_t compute_stream) {
    if (num_layers <= 0) return;
    for (int l = 0; l < num_layers; ++l)
        if (!host_pools[l] || !device_pools[l] || !out_key[l] || !out_value[l])
            throw Error("load_layers: null pool or output pointer for a layer");
    int dev = 0;
    check(hipGetDevice(&dev), "hipGetDevice");
    DeviceEvents& de = device_events(dev);
    std::lock_guard<std::mutex> lock(de.mu);  // held until every layer is enqueued
    std::vector<hipEvent_t>& ev = de.ev;
    while (ev.size() < (size_t)num_layers + 1) {
        hipEvent_t e = nullptr;
        check(hipEventCreateWithFlags(&e, hipEventDisableTiming), "hipEventCreateWithFlags");
        ev.push_back(e);
    }
    const bool two = copy_stream != compute_stream;
    if (two) {
        // Copies must not overwrite pools that earlier compute work still reads.
        check(hipEventRecord(ev[num_layers], compute_stream), "hipEventRecord");
        check(hipStreamWaitEvent(copy_stream, ev[num_layers], 0), "hipStreamWaitEvent");
    }
    for (int l = 0; l < num_layers; ++l) {
        check(hipMemcpyAsync(device_pools[l], host_pools[l], pool_bytes, hipMemcpyHostToDevice,
                             copy_stream),
              "hipMemcpyAsync");
        if (two) {
            check(hipEventRecord(ev[l], copy_stream), "hipEventRecord");
            check(hipStreamWaitEvent(compute_stream, ev[l], 0), "hipStreamWaitEvent");
        }
        launch_dequant(s, device_pools[l], slots, out_key[l], out_value[l], g, num_tokens,
                       compute_stream, /*head_major=*/true);
    }
}

}  // namespace tq

// tq_noalloc.hip — the turbo_prod fused attention entry for callers that
// cannot allocate device memory (code under graph capture, tight serving
// loops, harnesses that forbid hipMalloc).
//
// tq_launch_turbo_prod_fused_attention_output takes its split-K partials
// from a per-stream workspace that it allocates on first use.  This variant
// runs the same kernels with the partials in `scratch`, a file-scope device
// array of kScratchBytes: no hipMalloc, hipFree or allocating library call.
// Each GPU holds its own copy of the array until the process ends; host code
// uses the per-device address from hipGetSymbolAddress, taken once per
// device on the first call with that device current (the array's name in
// host code is only a stand-in, not a device address).  The partials need no
// clearing: the split kernel writes every entry the combine reads.  Calls on
// one GPU share the array, so calls that overlap on one GPU (other streams,
// other host threads, concurrent graph replays) race.
#include <hip/hip_runtime.h>

#include <mutex>

#include "tq_internal.h"

namespace {

// 4 MiB: the partials of up to 1,008 split workgroups (8 query rows, 4,160
// bytes each: 4,194,304 / 4,160 = 1,008.2); the
// GQA 16/2 decode step at 32K context uses 256 (1.08 MB).
constexpr size_t kScratchBytes = size_t(4) << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_mu;
void* g_scratch_ptr[kMaxDevices] = {};  // scratch's address on each device, once resolved

// The device address of `scratch` on the current device (resolved once per
// device, with that device current).
void* device_scratch() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) throw tq::Error("hipGetDevice failed");
    if (dev < 0 || dev >= kMaxDevices) throw tq::Error("device index out of range");
    std::lock_guard<std::mutex> lock(g_mu);
    if (!g_scratch_ptr[dev]) {
        void* ptr = nullptr;
        const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !ptr) {
            (void)hipGetLastError();
            throw tq::Error(std::string("hipGetSymbolAddress(scratch) failed: ") +
                            hipGetErrorString(e));
        }
        g_scratch_ptr[dev] = ptr;
        (void)tq::num_cus();  // cached now, so later calls allocate nothing on the host either
    }
    return g_scratch_ptr[dev];
}

}  // namespace

extern "C" int tq_launch_turbo_prod_fused_attention_output_noalloc(
    const uint16_t* query, const uint8_t* page_pool, const int32_t* slot_mapping,
    uint16_t* output, const TQTurboProdPageLayout* layout, const TQConfig* cfg, int num_queries,
    int num_kv_tokens, void* stream) {
    if (!query || !page_pool || !slot_mapping || !output || !layout || !cfg) return -1;
    try {
        const tq::PageGeom g = tq::prod_geom(*cfg, *layout);
        if (num_queries <= 0)
            throw tq::Error("turbo_prod_fused_attn_online_kernel: invalid configuration argument");
        if (num_kv_tokens < 0) throw tq::Error("turbo_prod attention: num_kv_tokens < 0");
        tq::Scratch s;
        s.ptr = device_scratch();
        s.cap = kScratchBytes;
        tq::launch_attention(tq::Scheme::Prod, query, page_pool, slot_mapping, output, g,
                             num_queries, num_kv_tokens, static_cast<hipStream_t>(stream), s);
        tq::debug_sync(stream);
        return 0;
    } catch (const std::exception& e) {
        tq::set_last_error(e.what());
        return -2;
    } catch (...) {
        tq::set_last_error("unknown error");
        return -2;
    }
}

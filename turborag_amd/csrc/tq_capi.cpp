// tq_capi.cpp — the extern "C" surface of libturboquant.so (include/turboquant.h).
//
// Mirrors src/tq_capi.cpp of the reference: NULL pointers -> -1 before any
// other check; any tq::Error / std::exception from validation or a launch ->
// -2 with the message in a thread-local 512-byte buffer (TQ_KERNEL_CALL,
// src/tq_capi.cpp:14-33).  Exceptions never cross the ABI.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>
#include <new>
#include <utility>
#include <vector>

#include "tq_internal.h"

namespace {

thread_local char g_last_error[512] = "";

void set_error(const char* msg) { std::snprintf(g_last_error, sizeof(g_last_error), "%.511s", msg); }

template <class F>
int guarded(F&& f) {
    try {
        f();
        return 0;
    } catch (const std::exception& e) {
        set_error(e.what());
        return -2;
    } catch (...) {
        set_error("unknown error");
        return -2;
    }
}

// Debug-sync mode (the reference's TQ_DEBUG_SYNC / TQ_CHECK_ASYNC,
// include/tq_cuda_check.h:26-37): built with -DTQ_DEBUG_SYNC, or run with
// the environment variable TQ_DEBUG_SYNC set to a non-zero value, every
// launching entry synchronizes its stream after the launch, so a fault in its
// kernels is reported by that call (rc -2, "async kernel error: ...").
// Skipped while the stream is being captured into a graph.
bool debug_sync_enabled() {
#ifdef TQ_DEBUG_SYNC
    return true;
#else
    static const bool on = [] {
        const char* v = std::getenv("TQ_DEBUG_SYNC");
        return v && *v && std::strcmp(v, "0") != 0;
    }();
    return on;
#endif
}

}  // namespace

void tq::debug_sync(void* stream) {
    if (!debug_sync_enabled()) return;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(s, &st) == hipSuccess && st != hipStreamCaptureStatusNone) return;
    const hipError_t e = hipStreamSynchronize(s);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        throw tq::Error(std::string("async kernel error: ") + hipGetErrorString(e));
    }
}

namespace {
// guarded() for an entry that launches work on `stream`.
template <class F>
int guarded_sync(void* stream, F&& f) {
    return guarded([&] {
        f();
        tq::debug_sync(stream);
    });
}

size_t align_up(size_t x, size_t a) { return ((x + a - 1) / a) * a; }

bool is_pow2(int x) { return x > 0 && (x & (x - 1)) == 0; }

int log2i(int x) {
    int k = 0;
    while ((1 << k) < x) ++k;
    return k;
}

void check_common(const TQConfig& cfg, const char* scheme) {
    // Same message as the reference's launchers for the limit it checks
    // (tq_turbo_prod_kernels.cu:595, tq_turbo_mse_kernels.cu:431).
    if (cfg.head_dim > 128)
        throw tq::Error(std::string(scheme) + ": head_dim > 128 is not supported");
    if (!is_pow2(cfg.head_dim) || cfg.head_dim < 2)
        throw tq::Error(std::string(scheme) + ": head_dim must be a power of two in [2, 128]");
    if (cfg.num_kv_heads <= 0) throw tq::Error(std::string(scheme) + ": num_kv_heads must be > 0");
    if (cfg.block_size <= 0) throw tq::Error(std::string(scheme) + ": block_size must be > 0");
}

// Counts that the reference launches as grid dimensions: zero or negative
// gives "invalid configuration argument" from the CUDA launch check (turbo_prod
// only — its turbo_mse launchers do not check), preserved here.
void check_grid(int n, const char* what, bool prod) {
    if (n < 0 || (n == 0 && prod))
        throw tq::Error(std::string(what) + ": invalid configuration argument");
}

// Kernels index (token, head) rows in int32: num_tokens * H must stay below
// 2^30 (also leaving room for the persistent loops' look-ahead).
void check_rows(int num_tokens, int H, const char* what) {
    if ((long long)num_tokens * H >= (1LL << 30))
        throw tq::Error(std::string(what) + ": num_tokens * num_kv_heads must be < 2^30");
}

}  // namespace

namespace tq {

void set_last_error(const char* msg) { set_error(msg); }

float inv_sqrt_d(int D) {
    const int k = log2i(D);
    if ((k & 1) == 0) return std::ldexp(1.0f, -k / 2);
    return std::ldexp(0x1.6a09e6p-1f, -(k - 1) / 2);  // RN(1/sqrt(2)) * 2^-((k-1)/2)
}

void check_launch(const char* what) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) throw Error(std::string(what) + ": " + hipGetErrorString(e));
}

PageGeom prod_geom(const TQConfig& cfg, const TQTurboProdPageLayout& l) {
    check_common(cfg, "turbo_prod");
    const int half = cfg.head_dim / 2;
    if (l.k4_bytes_per_token_head != half || l.v4_bytes_per_token_head != half ||
        l.scale_bytes_per_token_head != 2)
        throw Error("turbo_prod: layout does not match head_dim (use tq_make_turbo_prod_layout)");
    PageGeom g{};
    g.page_size = l.page_size_bytes;
    g.kc_off = l.k4_codes_offset;
    g.vc_off = l.v4_codes_offset;
    g.ks_off = l.k_scales_offset;
    g.kres_off = l.k_residual_scales_offset;
    g.vs_off = l.v_scales_offset;
    g.code_stride = half;
    g.scale_stride = 2;
    g.H = cfg.num_kv_heads;
    g.D = cfg.head_dim;
    g.block_size = cfg.block_size;
    g.bs_shift = is_pow2(cfg.block_size) ? log2i(cfg.block_size) : -1;
    g.h_shift = is_pow2(cfg.num_kv_heads) ? log2i(cfg.num_kv_heads) : -1;
    return g;
}

PageGeom mse_geom(const TQConfig& cfg, const TQTurbomsePageLayout& l) {
    check_common(cfg, "turbo_mse");
    const int half = cfg.head_dim / 2;
    if (l.code_bytes_per_token_head != (size_t)half || l.norm_bytes_per_token_head != 2)
        throw Error("turbo_mse: layout does not match head_dim/nbits=4 (use tq_make_turbo_mse_layout)");
    PageGeom g{};
    g.page_size = l.page_size_bytes;
    g.kc_off = l.k_codes_offset;
    g.vc_off = l.v_codes_offset;
    g.ks_off = l.k_norms_offset;
    g.kres_off = 0;
    g.vs_off = l.v_norms_offset;
    g.code_stride = half;
    g.scale_stride = 2;
    g.H = cfg.num_kv_heads;
    g.D = cfg.head_dim;
    g.block_size = cfg.block_size;
    g.bs_shift = is_pow2(cfg.block_size) ? log2i(cfg.block_size) : -1;
    g.h_shift = is_pow2(cfg.num_kv_heads) ? log2i(cfg.num_kv_heads) : -1;
    return g;
}

// src/tq_qjl.cpp:7-33 (host factory, also used to validate a caller's layout)
TQQJLPageLayout make_qjl_layout(const TQConfig& cfg) {
    TQQJLPageLayout l{};
    l.k1_bytes_per_token_head = (cfg.head_dim + 7) / 8;
    l.v4_bytes_per_token_head = (cfg.head_dim * 4 + 7) / 8;
    l.scale_bytes_per_token_head = 2;
    const size_t th = (size_t)cfg.block_size * (size_t)cfg.num_kv_heads;
    size_t cur = 0;
    l.k1_codes_offset = cur;
    cur += th * (size_t)l.k1_bytes_per_token_head;
    cur = align_up(cur, 2);
    l.k_scales_offset = cur;
    cur += th * 2;
    l.v4_codes_offset = cur;
    cur += th * (size_t)l.v4_bytes_per_token_head;
    cur = align_up(cur, 2);
    l.v_scales_offset = cur;
    cur += th * 2;
    l.page_size_bytes = align_up(cur, 2);
    return l;
}

// src/tq_layout.cpp:8-36
TQPageLayout make_int4_layout(const TQConfig& cfg) {
    if (cfg.nbits != 4) throw Error("Only int4 is supported in MVP");
    if (cfg.group_size != cfg.head_dim) throw Error("MVP expects group_size == head_dim");
    TQPageLayout l{};
    l.code_bytes_per_token_head = (size_t)(cfg.head_dim * cfg.nbits) / 8;
    l.scale_bytes_per_token_head = cfg.scale_type == TQ_SCALE_FP16 ? 2 : 4;
    const size_t th = (size_t)cfg.block_size * (size_t)cfg.num_kv_heads;
    const size_t a = (size_t)cfg.page_alignment;
    l.k_codes_offset = 0;
    l.k_codes_bytes = th * l.code_bytes_per_token_head;
    l.v_codes_offset = align_up(l.k_codes_offset + l.k_codes_bytes, a);
    l.v_codes_bytes = th * l.code_bytes_per_token_head;
    l.k_scales_offset = align_up(l.v_codes_offset + l.v_codes_bytes, a);
    l.k_scales_bytes = th * l.scale_bytes_per_token_head;
    l.v_scales_offset = align_up(l.k_scales_offset + l.k_scales_bytes, a);
    l.v_scales_bytes = th * l.scale_bytes_per_token_head;
    l.page_size_bytes = align_up(l.v_scales_offset + l.v_scales_bytes, a);
    return l;
}

// src/tq_dense_layout.cpp:7-18
TQDensePageLayout make_dense_layout(const TQConfig& cfg) {
    TQDensePageLayout l{};
    l.elem_bytes = 2;
    const size_t th = (size_t)cfg.block_size * (size_t)cfg.num_kv_heads;
    const size_t a = (size_t)cfg.page_alignment;
    l.k_offset = 0;
    l.k_bytes = th * (size_t)cfg.head_dim * 2;
    l.v_offset = align_up(l.k_offset + l.k_bytes, a);
    l.v_bytes = th * (size_t)cfg.head_dim * 2;
    l.page_size_bytes = align_up(l.v_offset + l.v_bytes, a);
    return l;
}

QjlGeom qjl_geom(const TQConfig& cfg, const TQQJLPageLayout& l) {
    check_common(cfg, "QJL");
    const TQQJLPageLayout want = make_qjl_layout(cfg);
    if (l.k1_bytes_per_token_head != want.k1_bytes_per_token_head ||
        l.v4_bytes_per_token_head != want.v4_bytes_per_token_head ||
        l.scale_bytes_per_token_head != 2 || l.page_size_bytes < want.page_size_bytes)
        throw Error("QJL: layout does not match head_dim (use tq_make_qjl_layout)");
    return QjlGeom{l.page_size_bytes, l.k1_codes_offset, l.k_scales_offset, l.v4_codes_offset,
                   l.v_scales_offset, l.k1_bytes_per_token_head, l.v4_bytes_per_token_head,
                   cfg.num_kv_heads, cfg.head_dim, cfg.block_size};
}

Int4Geom int4_geom(const TQConfig& cfg, const TQPageLayout& l) {
    check_common(cfg, "int4");
    const TQPageLayout want = make_int4_layout(cfg);
    if (l.code_bytes_per_token_head != want.code_bytes_per_token_head ||
        l.scale_bytes_per_token_head != want.scale_bytes_per_token_head ||
        l.page_size_bytes < want.page_size_bytes)
        throw Error("int4: layout does not match cfg (use tq_make_int4_layout)");
    return Int4Geom{l.page_size_bytes, l.k_codes_offset, l.v_codes_offset, l.k_scales_offset,
                    l.v_scales_offset, (int)l.code_bytes_per_token_head,
                    (int)l.scale_bytes_per_token_head, cfg.num_kv_heads, cfg.head_dim,
                    cfg.block_size};
}

DenseGeom dense_geom(const TQConfig& cfg, const TQDensePageLayout& l) {
    check_common(cfg, "dense");
    const TQDensePageLayout want = make_dense_layout(cfg);
    if (l.elem_bytes != 2 || l.k_bytes != want.k_bytes || l.page_size_bytes < want.page_size_bytes ||
        (l.k_offset & 3) || (l.v_offset & 3) || (l.page_size_bytes & 3))
        throw Error("dense: layout does not match cfg (use tq_make_dense_layout)");
    return DenseGeom{l.page_size_bytes, l.k_offset, l.v_offset, cfg.num_kv_heads, cfg.head_dim,
                     cfg.block_size};
}

int num_cus() {
    static std::mutex mu;
    static std::map<int, int> cache;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) throw Error("hipGetDevice failed");
    std::lock_guard<std::mutex> lock(mu);
    auto it = cache.find(dev);
    if (it != cache.end()) return it->second;
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
        n = 256;
    cache[dev] = n;
    return n;
}

// Split-K workspace for attention: one buffer per (device, stream).  Calls
// on one stream run in order, so they can share it.  A call that needs more
// replaces the buffer; the old one may still be read by kernels already
// enqueued on the stream, so it is retired with an event recorded behind them
// and freed once that event has completed (checked on later calls).  A
// buffer handed out while its stream was being captured into a graph is
// referenced by that graph, so it is never freed automatically, only by
// tq_workspace_release().  Past kMaxStreams cached streams the least recently
// used buffer that no graph references is evicted the same way: freed at
// once if its stream is idle, otherwise retired behind an event recorded on
// its stream.  No launching entry synchronizes a device or another stream.
namespace {
struct WsBuf {
    void* p = nullptr;
    size_t n = 0;
    bool captured = false;  // handed out during a stream capture
    uint64_t last_use = 0;  // handout tick (eviction order)
};
uint64_t g_ws_tick = 0;
struct Retired {
    void* p;
    hipEvent_t ev;  // null: outgrown during capture, or its stream unknown: freed only on release
    int dev;
};
std::mutex g_ws_mu;
std::map<std::pair<int, hipStream_t>, WsBuf> g_ws;
std::vector<Retired> g_retired;
constexpr size_t kMaxStreams = 64;

bool capturing(hipStream_t s) {
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(s, &st) != hipSuccess) {
        (void)hipGetLastError();
        return true;  // unknown: treat as capturing (never record, never free)
    }
    return st != hipStreamCaptureStatusNone;
}

// Frees the retired buffers whose kernels have finished.  Lock held.
void reap_retired() {
    for (size_t k = 0; k < g_retired.size();) {
        Retired& r = g_retired[k];
        if (r.ev && hipEventQuery(r.ev) == hipSuccess) {
            (void)hipFree(r.p);
            (void)hipEventDestroy(r.ev);
            g_retired[k] = g_retired.back();
            g_retired.pop_back();
        } else {
            (void)hipGetLastError();  // hipErrorNotReady is not an error of the caller's
            ++k;
        }
    }
}

// Evicts the least recently used cached buffer that no captured graph
// references and whose stream is not being captured (none: the cache grows).
// Its stream idle: freed now.  Still running work: retired behind an event
// recorded on that stream.  A stream the runtime no longer knows (destroyed):
// parked, freed only by tq_workspace_release, since it cannot be ordered
// behind that stream's last kernels.  Lock held.
void evict_lru() {
    auto victim = g_ws.end();
    for (auto it = g_ws.begin(); it != g_ws.end(); ++it) {
        if (it->second.captured) continue;
        if (victim != g_ws.end() && it->second.last_use >= victim->second.last_use) continue;
        victim = it;
    }
    if (victim == g_ws.end()) return;
    const int dev = victim->first.first;
    const hipStream_t s = victim->first.second;
    int cur = 0;
    (void)hipGetDevice(&cur);
    (void)hipSetDevice(dev);
    if (capturing(s)) {  // (its next handout marks it captured)
        (void)hipSetDevice(cur);
        return;
    }
    Retired r{victim->second.p, nullptr, dev};
    const hipError_t q = hipStreamQuery(s);
    if (q == hipSuccess) {
        (void)hipFree(r.p);
    } else if (q == hipErrorNotReady &&
               hipEventCreateWithFlags(&r.ev, hipEventDisableTiming) == hipSuccess &&
               hipEventRecord(r.ev, s) == hipSuccess) {
        g_retired.push_back(r);
    } else {
        if (r.ev) (void)hipEventDestroy(r.ev);
        r.ev = nullptr;
        g_retired.push_back(r);  // parked until tq_workspace_release
    }
    (void)hipGetLastError();
    (void)hipSetDevice(cur);
    g_ws.erase(victim);
}

// Synchronizes every device holding a cached buffer and frees them all
// (with keep_captured, those a captured graph references stay).  Lock held.
void release_all(bool keep_captured = false) {
    std::vector<int> devs;
    for (const auto& kv : g_ws) devs.push_back(kv.first.first);
    for (const auto& r : g_retired) devs.push_back(r.dev);
    std::sort(devs.begin(), devs.end());
    devs.erase(std::unique(devs.begin(), devs.end()), devs.end());
    int cur = 0;
    (void)hipGetDevice(&cur);
    for (int d : devs) {
        if (hipSetDevice(d) == hipSuccess) (void)hipDeviceSynchronize();
    }
    for (auto it = g_ws.begin(); it != g_ws.end();) {
        if (keep_captured && it->second.captured) {
            ++it;
            continue;
        }
        (void)hipSetDevice(it->first.first);
        (void)hipFree(it->second.p);
        it = g_ws.erase(it);
    }
    for (size_t k = 0; k < g_retired.size();) {
        Retired& r = g_retired[k];
        if (keep_captured && !r.ev) {  // retired during or after a capture: kept
            ++k;
            continue;
        }
        (void)hipSetDevice(r.dev);
        (void)hipFree(r.p);
        if (r.ev) (void)hipEventDestroy(r.ev);
        g_retired[k] = g_retired.back();
        g_retired.pop_back();
    }
    (void)hipSetDevice(cur);
    (void)hipGetLastError();
}
}  // namespace

void* workspace(hipStream_t stream, size_t bytes) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) throw Error("hipGetDevice failed");
    std::lock_guard<std::mutex> lock(g_ws_mu);
    const bool cap = capturing(stream);
    auto it = g_ws.find({dev, stream});
    if (it != g_ws.end() && it->second.n >= bytes && it->second.p) {
        it->second.captured = it->second.captured || cap;
        it->second.last_use = ++g_ws_tick;
        return it->second.p;
    }
    if (!cap) {
        reap_retired();
        if (it == g_ws.end() && g_ws.size() >= kMaxStreams) evict_lru();
    }
    WsBuf& b = g_ws[{dev, stream}];
    size_t n = std::max<size_t>(bytes, 1 << 20);
    n = std::max(n, b.n * 2);
    void* p = nullptr;
    if (hipMalloc(&p, n) != hipSuccess) {
        (void)hipGetLastError();
        throw Error("workspace hipMalloc failed");
    }
    if (b.p) {
        Retired r{b.p, nullptr, dev};
        if (!cap && !b.captured) {
            if (hipEventCreateWithFlags(&r.ev, hipEventDisableTiming) != hipSuccess ||
                hipEventRecord(r.ev, stream) != hipSuccess) {
                (void)hipGetLastError();
                if (r.ev) (void)hipEventDestroy(r.ev);
                r.ev = nullptr;
            }
        }
        g_retired.push_back(r);
    }
    b.p = p;
    b.n = n;
    b.captured = cap;
    b.last_use = ++g_ws_tick;
    return p;
}

void* Scratch::get(hipStream_t stream, size_t bytes, const char* what) const {
    if (!ptr) return workspace(stream, bytes);
    if (bytes > cap)
        throw Error(std::string(what) + ": needs " + std::to_string(bytes) +
                    " bytes of split-K scratch, more than the " + std::to_string(cap) +
                    " bytes available");
    return ptr;
}

void release_workspaces() {
    std::lock_guard<std::mutex> lock(g_ws_mu);
    release_all();
}

}  // namespace tq

// ---------------------------------------------------------------------------
// Config and layouts (host only)
// ---------------------------------------------------------------------------

extern "C" const char* tq_last_error(void) { return g_last_error; }

extern "C" int tq_workspace_release(void) {
    return guarded([] { tq::release_workspaces(); });
}

extern "C" int tq_make_default_config(TQConfig* out) {
    if (!out) return -1;
    *out = TQConfig{16, 8, 128, 4, 128, 256, TQ_SCALE_FP16, TQ_QUANT_MSE_INT4};
    return 0;
}

// src/tq_turbo_prod.cpp:7-39
extern "C" int tq_make_turbo_prod_layout(const TQConfig* cfg, TQTurboProdPageLayout* out) {
    if (!cfg || !out) return -1;
    TQTurboProdPageLayout l{};
    l.k4_bytes_per_token_head = (cfg->head_dim + 1) / 2;
    l.v4_bytes_per_token_head = (cfg->head_dim * 4 + 7) / 8;
    l.scale_bytes_per_token_head = 2;
    const size_t th = (size_t)cfg->block_size * (size_t)cfg->num_kv_heads;
    size_t cur = 0;
    l.k4_codes_offset = cur;
    cur += th * (size_t)l.k4_bytes_per_token_head;
    cur = align_up(cur, 2);
    l.k_residual_scales_offset = cur;
    cur += th * 2;
    l.k_scales_offset = cur;
    cur += th * 2;
    l.v4_codes_offset = cur;
    cur += th * (size_t)l.v4_bytes_per_token_head;
    cur = align_up(cur, 2);
    l.v_scales_offset = cur;
    cur += th * 2;
    l.page_size_bytes = align_up(cur, 2);
    *out = l;
    return 0;
}

// src/tq_turbo_mse_layout.cpp:7-28
extern "C" int tq_make_turbo_mse_layout(const TQConfig* cfg, TQTurbomsePageLayout* out) {
    if (!cfg || !out) return -1;
    TQTurbomsePageLayout l{};
    l.code_bytes_per_token_head = (size_t)((cfg->head_dim * cfg->nbits + 7) / 8);
    l.norm_bytes_per_token_head = 2;
    const size_t th = (size_t)cfg->block_size * (size_t)cfg->num_kv_heads;
    const size_t a = (size_t)cfg->page_alignment;
    l.k_codes_offset = 0;
    l.v_codes_offset = align_up(l.k_codes_offset + th * l.code_bytes_per_token_head, a);
    l.k_norms_offset = align_up(l.v_codes_offset + th * l.code_bytes_per_token_head, a);
    l.v_norms_offset = align_up(l.k_norms_offset + th * l.norm_bytes_per_token_head, a);
    l.page_size_bytes = align_up(l.v_norms_offset + th * l.norm_bytes_per_token_head, a);
    *out = l;
    return 0;
}

// ---------------------------------------------------------------------------
// turbo_prod
// ---------------------------------------------------------------------------

extern "C" int tq_launch_turbo_prod_pack_kv(const uint16_t* key, const uint16_t* value,
                                            const int32_t* slot_mapping, uint8_t* page_pool,
                                            const TQTurboProdPageLayout* layout,
                                            const TQConfig* cfg, int num_tokens, void* stream) {
    if (!key || !value || !slot_mapping || !page_pool || !layout || !cfg) return -1;
    return guarded_sync(stream, [&] {
        const tq::PageGeom g = tq::prod_geom(*cfg, *layout);
        check_grid(num_tokens, "turbo_prod_pack_kv_kernel", true);
        check_rows(num_tokens, g.H, "turbo_prod_pack_kv");
        tq::launch_pack(tq::Scheme::Prod, key, value, slot_mapping, page_pool, g, num_tokens,
                        static_cast<hipStream_t>(stream));
    });
}

extern "C" int tq_launch_turbo_prod_pack_kv_debug(
    const uint16_t* key, const uint16_t* value, const int32_t* slot_mapping, uint8_t* page_pool,
    const TQTurboProdPageLayout* layout, const TQConfig* cfg, int num_tokens, void* stream,
    float* debug_k_rot, float* debug_v_rot, float* debug_kn, float* debug_vn, int32_t* debug_kidx,
    int32_t* debug_vidx) {
    if (!key || !value || !slot_mapping || !page_pool || !layout || !cfg) return -1;
    return guarded_sync(stream, [&] {
        const tq::PageGeom g = tq::prod_geom(*cfg, *layout);
        check_grid(num_tokens, "turbo_prod_pack_kv_kernel", true);
        check_rows(num_tokens, g.H, "turbo_prod_pack_kv");
        tq::PackDebug dbg;
        dbg.k_rot = debug_k_rot;
        dbg.v_rot = debug_v_rot;
        dbg.kn = debug_kn;
        dbg.vn = debug_vn;
        dbg.kidx = debug_kidx;
        dbg.vidx = debug_vidx;
        tq::launch_prod_pack_debug(key, value, slot_mapping, page_pool, g, num_tokens, dbg,
                                   static_cast<hipStream_t>(stream));
    });
}

extern "C" int tq_launch_turbo_prod_dequant_kv(const uint8_t* page_pool,
                                               const int32_t* slot_mapping, uint16_t* out_key,
                                               uint16_t* out_value,
                                               const TQTurboProdPageLayout* layout,
                                               const TQConfig* cfg, int num_tokens,
                                               void* stream) {
    if (!page_pool || !slot_mapping || !out_key || !out_value || !layout || !cfg) return -1;
    return guarded_sync(stream, [&] {
        const tq::PageGeom g = tq::prod_geom(*cfg, *layout);
        check_grid(num_tokens, "turbo_prod_dequant_kv_kernel", true);
        check_rows(num_tokens, g.H, "turbo_prod_dequant_kv");
        tq::launch_dequant(tq::Scheme::Prod, page_pool, slot_mapping, out_key, out_value, g,
                           num_tokens, static_cast<hipStream_t>(stream));
    });
}

extern "C" int tq_launch_turbo_prod_fused_attention_logits(
    const uint16_t* query, const uint8_t* page_pool, const int32_t* slot_mapping, float* logits,
    const TQTurboProdPageLayout* layout, const TQConfig* cfg, int num_queries, int num_kv_tokens,
    void* stream) {
    if (!query || !page_pool || !slot_mapping || !logits || !layout || !cfg) return -1;
    return guarded_sync(stream, [&] {
        const tq::PageGeom g = tq::prod_geom(*cfg, *layout);
        check_grid(num_queries, "turbo_prod_fused_attention_logits_kernel", true);
        if (num_kv_tokens < 0) throw tq::Error("turbo_prod logits: num_kv_tokens < 0");
        tq::launch_logits(query, page_pool, slot_mapping, logits, g, num_queries, num_kv_tokens,
                          static_cast<hipStream_t>(stream));
    });
}

extern "C" int tq_launch_turbo_prod_fused_attention_output(
    const uint16_t* query, const uint8_t* page_pool, const int32_t* slot_mapping,
    uint16_t* output, const TQTurboProdPageLayout* layout, const TQConfig* cfg, int num_queries,
    int num_kv_tokens, void* stream) {
    if (!query || !page_pool || !slot_mapping || !output || !layout || !cfg) return -1;
    return guarded_sync(stream, [&] {
        const tq::PageGeom g = tq::prod_geom(*cfg, *layout);
        check_grid(num_queries, "turbo_prod_fused_attn_online_kernel", true);
        if (num_kv_tokens < 0) throw tq::Error("turbo_prod attention: num_kv_tokens < 0");
        tq::launch_attention(tq::Scheme::Prod, query, page_pool, slot_mapping, output, g,
                             num_queries, num_kv_tokens, static_cast<hipStream_t>(stream));
    });
}

extern "C" int tq_launch_turbo_prod_dequant_kv_hnd(const uint8_t* page_pool,
                                                   const int32_t* slot_mapping,
                                                   uint16_t* out_key, uint16_t* out_value,
                                                   const TQTurboProdPageLayout* layout,
                                                   const TQConfig* cfg, int num_tokens,
                                                   void* stream) {
    if (!page_pool || !slot_mapping || !out_key || !out_value || !layout || !cfg) return -1;
    return guarded_sync(stream, [&] {
        const tq::PageGeom g = tq::prod_geom(*cfg, *layout);
        check_grid(num_tokens, "turbo_prod_dequant_kv_kernel", true);
        check_rows(num_tokens, g.H, "turbo_prod_dequant_kv_hnd");
        tq::launch_dequant(tq::Scheme::Prod, page_pool, slot_mapping, out_key, out_value, g,
                           num_tokens, static_cast<hipStream_t>(stream), /*head_major=*/true);
    });
}

extern "C" int tq_load_turbo_prod_layers(const uint8_t* const* host_pools,
                                         uint8_t* const* device_pools, size_t pool_bytes,
                                         int num_layers, const int32_t* slot_mapping,
                                         int num_tokens, uint16_t* const* out_key,
                                         uint16_t* const* out_value,
                                         const TQTurboProdPageLayout* layout,
                                         const TQConfig* cfg, void* copy_stream,
                                         void* compute_stream) {
    if (!host_pools || !device_pools || !slot_mapping || !out_key || !out_value || !layout ||
        !cfg)
        return -1;
    return guarded_sync(compute_stream, [&] {
        const tq::PageGeom g = tq::prod_geom(*cfg, *layout);
        if (num_layers < 0 || num_tokens < 0)
            throw tq::Error("turbo_prod load: num_layers and num_tokens must be >= 0");
        check_rows(num_tokens, g.H, "turbo_prod load");
        tq::load_layers(tq::Scheme::Prod, host_pools, device_pools, pool_bytes, num_layers,
                        slot_mapping, num_tokens, out_key, out_value, g,
                        static_cast<hipStream_t>(copy_stream),
                        static_cast<hipStream_t>(compute_stream));
    });
}

namespace {
// tq_launch_*_pack_kv_layers: one slot mapping, num_layers inputs and pools.
template <typename Layout>
int pack_layers(tq::Scheme scheme, const uint16_t* const* keys, const uint16_t* const* values,
                const int32_t* slot_mapping, uint8_t* const* page_pools, int num_layers,
                const Layout* layout, const TQConfig* cfg, int num_tokens, void* stream) {
    if (!keys || !values || !slot_mapping || !page_pools || !layout || !cfg) return -1;
    const bool prod = scheme == tq::Scheme::Prod;
    const char* name = prod ? "turbo_prod_pack_kv_layers" : "turbo_mse_pack_kv_layers";
    return guarded_sync(stream, [&] {
        const tq::PageGeom g =
            prod ? tq::prod_geom(*cfg, *reinterpret_cast<const TQTurboProdPageLayout*>(layout))
                 : tq::mse_geom(*cfg, *reinterpret_cast<const TQTurbomsePageLayout*>(layout));
        if (num_layers < 0) throw tq::Error(std::string(name) + ": num_layers must be >= 0");
        check_grid(num_tokens, name, prod);
        check_rows(num_tokens, g.H, name);
        for (int l = 0; l < num_layers; ++l)
            if (!keys[l] || !values[l] || !page_pools[l])
                throw tq::Error(std::string(name) + ": null input or pool pointer for a layer");
        tq::launch_pack_layers(scheme, keys, values, slot_mapping, page_pools, g, num_tokens,
                               num_layers, static_cast<hipStream_t>(stream));
    });
}

// tq_launch_*_dequant_kv_layers: one slot mapping, num_layers pools and outputs.
template <typename Layout>
int dequant_layers(tq::Scheme scheme, const uint8_t* const* page_pools,
                   const int32_t* slot_mapping, uint16_t* const* out_keys,
                   uint16_t* const* out_values, int num_layers, const Layout* layout,
                   const TQConfig* cfg, int num_tokens, int head_major, void* stream) {
    if (!page_pools || !slot_mapping || !out_keys || !out_values || !layout || !cfg) return -1;
    const bool prod = scheme == tq::Scheme::Prod;
    const char* name = prod ? "turbo_prod_dequant_kv_layers" : "turbo_mse_dequant_kv_layers";
    return guarded_sync(stream, [&] {
        const tq::PageGeom g =
            prod ? tq::prod_geom(*cfg, *reinterpret_cast<const TQTurboProdPageLayout*>(layout))
                 : tq::mse_geom(*cfg, *reinterpret_cast<const TQTurbomsePageLayout*>(layout));
        if (num_layers < 0 || num_tokens < 0)
            throw tq::Error(std::string(name) + ": num_layers and num_tokens must be >= 0");
        check_rows(num_tokens, g.H, name);
        for (int l = 0; l < num_layers; ++l)
            if (!page_pools[l] || !out_keys[l] || !out_values[l])
                throw tq::Error(std::string(name) + ": null pool or output pointer for a layer");
        tq::launch_dequant_layers(scheme, page_pools, slot_mapping, out_keys, out_values, g,
                                  num_tokens, num_layers, static_cast<hipStream_t>(stream),
                                  head_major != 0);
    });
}
}  // namespace

extern "C" int tq_launch_turbo_prod_pack_kv_layers(const uint16_t* const* keys,
                                                   const uint16_t* const* values,
                                                   const int32_t* slot_mapping,
                                                   uint8_t* const* page_pools, int num_layers,
                                                   const TQTurboProdPageLayout* layout,
                                                   const TQConfig* cfg, int num_tokens,
                                                   void* stream) {
    return pack_layers(tq::Scheme::Prod, keys, values, slot_mapping, page_pools, num_layers,
                       layout, cfg, num_tokens, stream);
}

extern "C" int tq_launch_turbo_mse_pack_kv_layers(const uint16_t* const* keys,
                                                  const uint16_t* const* values,
                                                  const int32_t* slot_mapping,
                                                  uint8_t* const* page_pools, int num_layers,
                                                  const TQTurbomsePageLayout* layout,
                                                  const TQConfig* cfg, int num_tokens,
                                                  void* stream) {
    return pack_layers(tq::Scheme::Mse, keys, values, slot_mapping, page_pools, num_layers,
                       layout, cfg, num_tokens, stream);
}

extern "C" int tq_launch_turbo_prod_dequant_kv_layers(
    const uint8_t* const* page_pools, const int32_t* slot_mapping, uint16_t* const* out_keys,
    uint16_t* const* out_values, int num_layers, const TQTurboProdPageLayout* layout,
    const TQConfig* cfg, int num_tokens, int head_major, void* stream) {
    return dequant_layers(tq::Scheme::Prod, page_pools, slot_mapping, out_keys, out_values,
                          num_layers, layout, cfg, num_tokens, head_major, stream);
}

extern "C" int tq_launch_turbo_mse_dequant_kv_layers(
    const uint8_t* const* page_pools, const int32_t* slot_mapping, uint16_t* const* out_keys,
    uint16_t* const* out_values, int num_layers, const TQTurbomsePageLayout* layout,
    const TQConfig* cfg, int num_tokens, int head_major, void* stream) {
    return dequant_layers(tq::Scheme::Mse, page_pools, slot_mapping, out_keys, out_values,
                          num_layers, layout, cfg, num_tokens, head_major, stream);
}

// ---------------------------------------------------------------------------
// turbo_mse
// ---------------------------------------------------------------------------

extern "C" int tq_launch_turbo_mse_pack_kv(const uint16_t* key, const uint16_t* value,
                                           const int32_t* slot_mapping, uint8_t* page_pool,
                                           const TQTurbomsePageLayout* layout,
                                           const TQConfig* cfg, int num_tokens, void* stream) {
    if (!key || !value || !slot_mapping || !page_pool || !layout || !cfg) return -1;
    return guarded_sync(stream, [&] {
        const tq::PageGeom g = tq::mse_geom(*cfg, *layout);
        check_grid(num_tokens, "turbo_mse_pack_kv_kernel", false);
        check_rows(num_tokens, g.H, "turbo_mse_pack_kv");
        tq::launch_pack(tq::Scheme::Mse, key, value, slot_mapping, page_pool, g, num_tokens,
                        static_cast<hipStream_t>(stream));
    });
}

extern "C" int tq_launch_turbo_mse_dequant_kv(const uint8_t* page_pool,
                                              const int32_t* slot_mapping, uint16_t* out_key,
                                              uint16_t* out_value,
                                              const TQTurbomsePageLayout* layout,
                                              const TQConfig* cfg, int num_tokens, void* stream) {
    if (!page_pool || !slot_mapping || !out_key || !out_value || !layout || !cfg) return -1;
    return guarded_sync(stream, [&] {
        const tq::PageGeom g = tq::mse_geom(*cfg, *layout);
        check_grid(num_tokens, "turbo_mse_dequant_kv_kernel", false);
        check_rows(num_tokens, g.H, "turbo_mse_dequant_kv");
        tq::launch_dequant(tq::Scheme::Mse, page_pool, slot_mapping, out_key, out_value, g,
                           num_tokens, static_cast<hipStream_t>(stream));
    });
}

extern "C" int tq_launch_turbo_mse_fused_attention_output(
    const uint16_t* query, const uint8_t* page_pool, const int32_t* slot_mapping,
    uint16_t* output, const TQTurbomsePageLayout* layout, const TQConfig* cfg, int num_queries,
    int num_kv_tokens, void* stream) {
    if (!query || !page_pool || !slot_mapping || !output || !layout || !cfg) return -1;
    return guarded_sync(stream, [&] {
        const tq::PageGeom g = tq::mse_geom(*cfg, *layout);
        check_grid(num_queries, "turbo_mse_fused_attn_online_kernel", false);
        if (num_kv_tokens < 0) throw tq::Error("turbo_mse attention: num_kv_tokens < 0");
        tq::launch_attention(tq::Scheme::Mse, query, page_pool, slot_mapping, output, g,
                             num_queries, num_kv_tokens, static_cast<hipStream_t>(stream));
    });
}

extern "C" int tq_launch_turbo_mse_dequant_kv_hnd(const uint8_t* page_pool,
                                                  const int32_t* slot_mapping, uint16_t* out_key,
                                                  uint16_t* out_value,
                                                  const TQTurbomsePageLayout* layout,
                                                  const TQConfig* cfg, int num_tokens,
                                                  void* stream) {
    if (!page_pool || !slot_mapping || !out_key || !out_value || !layout || !cfg) return -1;
    return guarded_sync(stream, [&] {
        const tq::PageGeom g = tq::mse_geom(*cfg, *layout);
        check_grid(num_tokens, "turbo_mse_dequant_kv_kernel", false);
        check_rows(num_tokens, g.H, "turbo_mse_dequant_kv_hnd");
        tq::launch_dequant(tq::Scheme::Mse, page_pool, slot_mapping, out_key, out_value, g,
                           num_tokens, static_cast<hipStream_t>(stream), /*head_major=*/true);
    });
}

extern "C" int tq_load_turbo_mse_layers(const uint8_t* const* host_pools,
                                        uint8_t* const* device_pools, size_t pool_bytes,
                                        int num_layers, const int32_t* slot_mapping,
                                        int num_tokens, uint16_t* const* out_key,
                                        uint16_t* const* out_value,
                                        const TQTurbomsePageLayout* layout, const TQConfig* cfg,
                                        void* copy_stream, void* compute_stream) {
    if (!host_pools || !device_pools || !slot_mapping || !out_key || !out_value || !layout ||
        !cfg)
        return -1;
    return guarded_sync(compute_stream, [&] {
        const tq::PageGeom g = tq::mse_geom(*cfg, *layout);
        if (num_layers < 0 || num_tokens < 0)
            throw tq::Error("turbo_mse load: num_layers and num_tokens must be >= 0");
        check_rows(num_tokens, g.H, "turbo_mse load");
        tq::load_layers(tq::Scheme::Mse, host_pools, device_pools, pool_bytes, num_layers,
                        slot_mapping, num_tokens, out_key, out_value, g,
                        static_cast<hipStream_t>(copy_stream),
                        static_cast<hipStream_t>(compute_stream));
    });
}

// ---------------------------------------------------------------------------
// Batched decode over paged sequences (superset of the reference ABI)
// ---------------------------------------------------------------------------

namespace {
template <class Layout>
int paged_attention(tq::Scheme scheme, const uint16_t* query, const uint8_t* page_pool,
                    const int32_t* block_tables, int max_blocks, const int32_t* row_seq,
                    const int32_t* row_kv_len, uint16_t* output, const Layout* layout,
                    const TQConfig* cfg, int num_rows, int max_kv_len, void* stream) {
    if (!query || !page_pool || !block_tables || !row_seq || !row_kv_len || !output || !layout ||
        !cfg)
        return -1;
    return guarded_sync(stream, [&] {
        const bool prod = scheme == tq::Scheme::Prod;
        const tq::PageGeom g = prod ? tq::prod_geom(*cfg, *reinterpret_cast<const TQTurboProdPageLayout*>(layout))
                                    : tq::mse_geom(*cfg, *reinterpret_cast<const TQTurbomsePageLayout*>(layout));
        const char* name = prod ? "turbo_prod paged attention" : "turbo_mse paged attention";
        if (num_rows < 0 || max_kv_len < 0 || max_blocks <= 0)
            throw tq::Error(std::string(name) +
                            ": num_rows, max_kv_len >= 0 and max_blocks_per_seq > 0 required");
        if ((long long)max_kv_len > (long long)max_blocks * cfg->block_size)
            throw tq::Error(std::string(name) + ": max_kv_len exceeds max_blocks_per_seq pages");
        tq::launch_paged_attention(scheme, query, page_pool, block_tables, max_blocks, row_seq,
                                   row_kv_len, output, g, num_rows, max_kv_len,
                                   static_cast<hipStream_t>(stream));
    });
}
}  // namespace

extern "C" int tq_launch_turbo_prod_paged_attention(
    const uint16_t* query, const uint8_t* page_pool, const int32_t* block_tables,
    int max_blocks_per_seq, const int32_t* row_seq, const int32_t* row_kv_len, uint16_t* output,
    const TQTurboProdPageLayout* layout, const TQConfig* cfg, int num_rows, int max_kv_len,
    void* stream) {
    return paged_attention(tq::Scheme::Prod, query, page_pool, block_tables, max_blocks_per_seq,
                           row_seq, row_kv_len, output, layout, cfg, num_rows, max_kv_len, stream);
}

extern "C" int tq_launch_turbo_mse_paged_attention(
    const uint16_t* query, const uint8_t* page_pool, const int32_t* block_tables,
    int max_blocks_per_seq, const int32_t* row_seq, const int32_t* row_kv_len, uint16_t* output,
    const TQTurbomsePageLayout* layout, const TQConfig* cfg, int num_rows, int max_kv_len,
    void* stream) {
    return paged_attention(tq::Scheme::Mse, query, page_pool, block_tables, max_blocks_per_seq,
                           row_seq, row_kv_len, output, layout, cfg, num_rows, max_kv_len, stream);
}

// ---------------------------------------------------------------------------
// Kernels the reference compiles but does not export (QJL-1b, legacy INT4,
// dense pages, GPU SDPA reference).  Zero tokens or queries do nothing.
// ---------------------------------------------------------------------------
namespace {
void need_aligned4(const void* p, const char* what) {
    if (reinterpret_cast<uintptr_t>(p) & 3) throw tq::Error(std::string(what) + ": pointer not 4-byte aligned");
}
void check_count(int n, const char* what) {
    if (n < 0) throw tq::Error(std::string(what) + ": negative count");
}
}  // namespace

extern "C" int tq_make_qjl_layout(const TQConfig* cfg, TQQJLPageLayout* out) {
    if (!cfg || !out) return -1;
    *out = tq::make_qjl_layout(*cfg);
    return 0;
}

extern "C" int tq_launch_qjl_pack_kv(const uint16_t* key, const uint16_t* value,
                                     const int32_t* slot_mapping, uint8_t* page_pool,
                                     const TQQJLPageLayout* layout, const TQConfig* cfg,
                                     int num_tokens, void* stream) {
    if (!key || !value || !slot_mapping || !page_pool || !layout || !cfg) return -1;
    return guarded_sync(stream, [&] {
        const tq::QjlGeom g = tq::qjl_geom(*cfg, *layout);
        check_count(num_tokens, "qjl_pack_kv");
        need_aligned4(key, "qjl_pack_kv key");
        need_aligned4(value, "qjl_pack_kv value");
        tq::launch_qjl_pack(key, value, slot_mapping, page_pool, g, num_tokens,
                            static_cast<hipStream_t>(stream));
    });
}

extern "C" int tq_launch_qjl_dequant_kv(const uint8_t* page_pool, const int32_t* slot_mapping,
                                        uint16_t* out_key, uint16_t* out_value,
                                        const TQQJLPageLayout* layout, const TQConfig* cfg,
                                        int num_tokens, void* stream) {
    if (!page_pool || !slot_mapping || !out_key || !out_value || !layout || !cfg) return -1;
    return guarded_sync(stream, [&] {
        const tq::QjlGeom g = tq::qjl_geom(*cfg, *layout);
        check_count(num_tokens, "qjl_dequant_kv");
        need_aligned4(out_key, "qjl_dequant_kv out_key");
        need_aligned4(out_value, "qjl_dequant_kv out_value");
        tq::launch_qjl_dequant(page_pool, slot_mapping, out_key, out_value, g, num_tokens,
                               static_cast<hipStream_t>(stream));
    });
}

extern "C" int tq_launch_qjl_fused_attention_output(const uint16_t* query,
                                                    const uint8_t* page_pool,
                                                    const int32_t* slot_mapping, uint16_t* output,
                                                    const TQQJLPageLayout* layout,
                                                    const TQConfig* cfg, int num_queries,
                                                    int num_kv_tokens, void* stream) {
    if (!query || !page_pool || !slot_mapping || !output || !layout || !cfg) return -1;
    return guarded_sync(stream, [&] {
        const tq::QjlGeom g = tq::qjl_geom(*cfg, *layout);
        check_count(num_queries, "qjl_fused_attention_output");
        check_count(num_kv_tokens, "qjl_fused_attention_output");
        need_aligned4(query, "qjl_fused_attention_output query");
        need_aligned4(output, "qjl_fused_attention_output output");
        tq::launch_qjl_attention(query, page_pool, slot_mapping, output, g, num_queries,
                                 num_kv_tokens, static_cast<hipStream_t>(stream));
    });
}

extern "C" int tq_make_int4_layout(const TQConfig* cfg, TQPageLayout* out) {
    if (!cfg || !out) return -1;
    return guarded([&] { *out = tq::make_int4_layout(*cfg); });
}

extern "C" int tq_launch_int4_pack_kv(const uint16_t* key, const uint16_t* value,
                                      const int32_t* slot_mapping, uint8_t* page_pool,
                                      const TQPageLayout* layout, const TQConfig* cfg,
                                      int num_tokens, void* stream) {
    if (!key || !value || !slot_mapping || !page_pool || !layout || !cfg) return -1;
    return guarded_sync(stream, [&] {
        const tq::Int4Geom g = tq::int4_geom(*cfg, *layout);
        check_count(num_tokens, "int4_pack_kv");
        need_aligned4(key, "int4_pack_kv key");
        need_aligned4(value, "int4_pack_kv value");
        tq::launch_int4_pack(key, value, slot_mapping, page_pool, g, num_tokens,
                             static_cast<hipStream_t>(stream));
    });
}

extern "C" int tq_launch_int4_dequant_kv(const uint8_t* page_pool, const int32_t* slot_mapping,
                                         uint16_t* out_key, uint16_t* out_value,
                                         const TQPageLayout* layout, const TQConfig* cfg,
                                         int num_tokens, void* stream) {
    if (!page_pool || !slot_mapping || !out_key || !out_value || !layout || !cfg) return -1;
    return guarded_sync(stream, [&] {
        const tq::Int4Geom g = tq::int4_geom(*cfg, *layout);
        check_count(num_tokens, "int4_dequant_kv");
        need_aligned4(out_key, "int4_dequant_kv out_key");
        need_aligned4(out_value, "int4_dequant_kv out_value");
        tq::launch_int4_dequant(page_pool, slot_mapping, out_key, out_value, g, num_tokens,
                                static_cast<hipStream_t>(stream));
    });
}

extern "C" int tq_make_dense_layout(const TQConfig* cfg, TQDensePageLayout* out) {
    if (!cfg || !out) return -1;
    *out = tq::make_dense_layout(*cfg);
    return 0;
}

extern "C" int tq_launch_dense_store_kv(const uint16_t* key, const uint16_t* value,
                                        const int32_t* slot_mapping, uint8_t* page_pool,
                                        const TQDensePageLayout* layout, const TQConfig* cfg,
                                        int num_tokens, void* stream) {
    if (!key || !value || !slot_mapping || !page_pool || !layout || !cfg) return -1;
    return guarded_sync(stream, [&] {
        const tq::DenseGeom g = tq::dense_geom(*cfg, *layout);
        check_count(num_tokens, "dense_store_kv");
        need_aligned4(key, "dense_store_kv key");
        need_aligned4(value, "dense_store_kv value");
        need_aligned4(page_pool, "dense_store_kv page_pool");
        tq::launch_dense_copy(true, key, value, nullptr, nullptr, slot_mapping, page_pool, g,
                              num_tokens, static_cast<hipStream_t>(stream));
    });
}

extern "C" int tq_launch_dense_load_kv(const uint8_t* page_pool, const int32_t* slot_mapping,
                                       uint16_t* out_key, uint16_t* out_value,
                                       const TQDensePageLayout* layout, const TQConfig* cfg,
                                       int num_tokens, void* stream) {
    if (!page_pool || !slot_mapping || !out_key || !out_value || !layout || !cfg) return -1;
    return guarded_sync(stream, [&] {
        const tq::DenseGeom g = tq::dense_geom(*cfg, *layout);
        check_count(num_tokens, "dense_load_kv");
        need_aligned4(out_key, "dense_load_kv out_key");
        need_aligned4(out_value, "dense_load_kv out_value");
        need_aligned4(page_pool, "dense_load_kv page_pool");
        tq::launch_dense_copy(false, nullptr, nullptr, out_key, out_value, slot_mapping,
                              const_cast<uint8_t*>(page_pool), g, num_tokens,
                              static_cast<hipStream_t>(stream));
    });
}

extern "C" int tq_launch_attention_ref(const uint16_t* query, const uint16_t* key,
                                       const uint16_t* value, uint16_t* output,
                                       float* logit_scratch, const TQConfig* cfg,
                                       int num_queries, int num_kv_tokens, void* stream) {
    if (!query || !key || !value || !output || !logit_scratch || !cfg) return -1;
    return guarded_sync(stream, [&] {
        // tq_attention_ref_kernel.cu:127-128
        if (cfg->head_dim > 128)
            throw tq::Error("attention_ref_gpu: head_dim > 128 is not supported");
        check_common(*cfg, "attention_ref_gpu");
        check_count(num_queries, "attention_ref_gpu");
        check_count(num_kv_tokens, "attention_ref_gpu");
        for (const void* p : {(const void*)query, (const void*)key, (const void*)value,
                              (const void*)output})
            need_aligned4(p, "attention_ref_gpu");
        tq::launch_attention_ref(query, key, value, output, logit_scratch, cfg->num_kv_heads,
                                 cfg->head_dim, num_queries, num_kv_tokens,
                                 static_cast<hipStream_t>(stream));
    });
}

// tq_internal.h — host-side declarations shared by the C ABI and the HIP
// kernel files of libturboquant.so (gfx950).
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <string>

#include "turboquant.h"

namespace tq {

// Error raised by launchers; the C ABI converts it to rc -2 and stores the
// message for tq_last_error() (the reference's TQ_KERNEL_CALL,
// src/tq_capi.cpp:25-33).
struct Error : std::runtime_error {
    using std::runtime_error::runtime_error;
};

// Stores msg in the calling thread's tq_last_error() buffer.
void set_last_error(const char* msg);

// Debug-sync mode (-DTQ_DEBUG_SYNC or the TQ_DEBUG_SYNC environment
// variable): synchronizes `stream` (a hipStream_t) after a launch and throws
// "async kernel error: ..." if its kernels failed; no-op otherwise, and while
// the stream is being captured.
void debug_sync(void* stream);

// Byte geometry of one page, resolved from a TQTurboProdPageLayout or a
// TQTurbomsePageLayout.  Passed to kernels by value.
//   cell c = tib * H + h;  K codes at kc_off + c*code_stride, V codes at
//   vc_off + c*code_stride, scales at {ks,kres,vs}_off + c*scale_stride.
struct PageGeom {
    uint64_t page_size;
    uint64_t kc_off, vc_off;
    uint64_t ks_off, kres_off, vs_off;  // kres_off unused by turbo_mse
    int code_stride;
    int scale_stride;
    int H, D, block_size;
    int bs_shift;  // log2(block_size) when block_size is a power of two, else -1
    int h_shift;   // log2(H) when H is a power of two, else -1
};

// Element offset of output row (token t, head h) of a dequant: t * tok +
// h * head ([N, H, D]: tok = H*D, head = D; [H, N, D]: tok = D, head = N*D).
struct OutLayout {
    uint64_t tok, head;
    __host__ __device__ uint64_t offset(int t, int h) const {
        return (uint64_t)t * tok + (uint64_t)h * head;
    }
};

// Number of compute units of the current device (cached per device).
int num_cus();

enum class Scheme : int { Prod = 0, Mse = 1 };

// Validates cfg/layout and resolves the geometry (throws tq::Error).
PageGeom prod_geom(const TQConfig& cfg, const TQTurboProdPageLayout& layout);
PageGeom mse_geom(const TQConfig& cfg, const TQTurbomsePageLayout& layout);

// RN(1/sqrt(D)) for D a power of two.
float inv_sqrt_d(int D);

// Throws tq::Error("<what>: <hip error string>") if the last launch failed
// (the reference's TQ_CHECK_LAUNCH, include/tq_cuda_check.h:18-24).
void check_launch(const char* what);

// Per-(device, stream) scratch for split-K partials.  Grows; an outgrown
// buffer is freed once the stream's earlier kernels have finished.
void* workspace(hipStream_t stream, size_t bytes);
// Where an attention launch takes its split-K partials from: the cached
// per-stream workspace above (ptr null), or memory the caller provides
// (ptr, cap bytes), in which case a launch that needs more throws.
struct Scratch {
    void* ptr = nullptr;
    size_t cap = 0;
    void* get(hipStream_t stream, size_t bytes, const char* what) const;
};
// Synchronizes the devices and frees every cached workspace (tq_workspace_release).
void release_workspaces();

// ---- launchers (tq_prod.hip, tq_mse.hip, tq_attention.hip) ---------------
void launch_pack(Scheme s, const uint16_t* key, const uint16_t* value, const int32_t* slots,
                 uint8_t* pool, const PageGeom& g, int num_tokens, hipStream_t stream);
// The reference pack kernel's optional debug buffers (include/tq_turbo_prod.cuh:
// 60-65), [num_tokens, H, D] each, null = not written: rotated K/V, clamped
// normalised K/V (fp32), 3-bit K and 4-bit V code indices (int32).
struct PackDebug {
    float *k_rot = nullptr, *v_rot = nullptr, *kn = nullptr, *vn = nullptr;
    int32_t *kidx = nullptr, *vidx = nullptr;
};
// turbo_prod pack that also writes `dbg` (pages identical to launch_pack's).
void launch_prod_pack_debug(const uint16_t* key, const uint16_t* value, const int32_t* slots,
                            uint8_t* pool, const PageGeom& g, int num_tokens, const PackDebug& dbg,
                            hipStream_t stream);
// Pack of num_layers layers' K/V sharing one slot mapping, in as few launches
// as possible (one per 64 layers for D = 64, 128 and aligned buffers).
void launch_pack_layers(Scheme s, const uint16_t* const* keys, const uint16_t* const* values,
                        const int32_t* slots, uint8_t* const* pools, const PageGeom& g,
                        int num_tokens, int num_layers, hipStream_t stream);
// head_major: outputs [H, N, D] (a [1, H, N, D] cache tensor) instead of [N, H, D].
void launch_dequant(Scheme s, const uint8_t* pool, const int32_t* slots, uint16_t* out_key,
                    uint16_t* out_value, const PageGeom& g, int num_tokens, hipStream_t stream,
                    bool head_major = false);
// Dequant of num_layers HBM-resident pools sharing one slot mapping, in as
// few launches as possible (one per 64 layers for D = 128 and aligned buffers).
void launch_dequant_layers(Scheme s, const uint8_t* const* pools, const int32_t* slots,
                           uint16_t* const* out_key, uint16_t* const* out_value, const PageGeom& g,
                           int num_tokens, int num_layers, hipStream_t stream, bool head_major);
// Layer-pipelined host -> device copy + dequant into [1, H, N, D] (tq_loader.cpp).
void load_layers(Scheme s, const uint8_t* const* host_pools, uint8_t* const* device_pools,
                 size_t pool_bytes, int num_layers, const int32_t* slots, int num_tokens,
                 uint16_t* const* out_key, uint16_t* const* out_value, const PageGeom& g,
                 hipStream_t copy_stream, hipStream_t compute_stream);
void launch_logits(const uint16_t* query, const uint8_t* pool, const int32_t* slots,
                   float* logits, const PageGeom& g, int num_queries, int num_kv_tokens,
                   hipStream_t stream);
// Batched decode over paged sequences (see tq_launch_*_paged_attention).
void launch_paged_attention(Scheme s, const uint16_t* query, const uint8_t* pool,
                            const int32_t* block_tables, int max_blocks, const int32_t* row_seq,
                            const int32_t* row_kv_len, uint16_t* output, const PageGeom& g,
                            int num_rows, int max_kv_len, hipStream_t stream);
void launch_attention(Scheme s, const uint16_t* query, const uint8_t* pool, const int32_t* slots,
                      uint16_t* output, const PageGeom& g, int num_queries, int num_kv_tokens,
                      hipStream_t stream, const Scratch& scratch = Scratch{});

// ---- the reference's unexported kernels (tq_legacy.hip) -------------------
// Byte geometry of a QJL-1b page (cell c = tib * H + h; K signs at
// k1_off + c * k1_bytes, V codes at v4_off + c * v4_bytes, fp16 scales at
// ks_off / vs_off + 2c).
struct QjlGeom {
    uint64_t page_size, k1_off, ks_off, v4_off, vs_off;
    int k1_bytes, v4_bytes;
    int H, D, block_size;
};
// Legacy INT4 page: codes at kc_off / vc_off + c * code_bytes, an fp16 scale
// at the start of each scale cell (ks_off / vs_off + c * scale_bytes).
struct Int4Geom {
    uint64_t page_size, kc_off, vc_off, ks_off, vs_off;
    int code_bytes, scale_bytes;
    int H, D, block_size;
};
// Dense page: fp16 rows at k_off / v_off + c * 2D.
struct DenseGeom {
    uint64_t page_size, k_off, v_off;
    int H, D, block_size;
};
QjlGeom qjl_geom(const TQConfig& cfg, const TQQJLPageLayout& layout);
Int4Geom int4_geom(const TQConfig& cfg, const TQPageLayout& layout);
DenseGeom dense_geom(const TQConfig& cfg, const TQDensePageLayout& layout);

void launch_qjl_pack(const uint16_t* key, const uint16_t* value, const int32_t* slots,
                     uint8_t* pool, const QjlGeom& g, int num_tokens, hipStream_t stream);
void launch_qjl_dequant(const uint8_t* pool, const int32_t* slots, uint16_t* out_key,
                        uint16_t* out_value, const QjlGeom& g, int num_tokens,
                        hipStream_t stream);
void launch_qjl_attention(const uint16_t* query, const uint8_t* pool, const int32_t* slots,
                          uint16_t* output, const QjlGeom& g, int num_queries, int num_kv_tokens,
                          hipStream_t stream);
// The wide form of launch_qjl_pack (D = 64, 128); false when not eligible.
bool launch_qjl_wide_pack(const uint16_t* key, const uint16_t* value, const int32_t* slots,
                          uint8_t* pool, const QjlGeom& g, int num_tokens, hipStream_t stream);
// The streaming form of launch_qjl_dequant (D = 128, aligned fields and
// outputs); false (nothing launched) when not eligible.
bool launch_qjl_stream_dequant(const uint8_t* pool, const int32_t* slots, uint16_t* out_key,
                               uint16_t* out_value, const QjlGeom& g, int num_tokens,
                               hipStream_t stream);
// The MFMA split-K form of launch_qjl_attention (D = 128, 4-byte aligned
// fields, 16-byte aligned pool); false (nothing launched) when not eligible.
bool launch_qjl_mfma_attention(const uint16_t* query, const uint8_t* pool, const int32_t* slots,
                               uint16_t* output, const QjlGeom& g, int num_queries,
                               int num_kv_tokens, hipStream_t stream);
void launch_int4_pack(const uint16_t* key, const uint16_t* value, const int32_t* slots,
                      uint8_t* pool, const Int4Geom& g, int num_tokens, hipStream_t stream);
void launch_int4_dequant(const uint8_t* pool, const int32_t* slots, uint16_t* out_key,
                         uint16_t* out_value, const Int4Geom& g, int num_tokens,
                         hipStream_t stream);
// store: [N, H, D] key/value -> pages; otherwise pages -> out_key/out_value.
void launch_dense_copy(bool store, const uint16_t* key, const uint16_t* value, uint16_t* out_key,
                       uint16_t* out_value, const int32_t* slots, uint8_t* pool,
                       const DenseGeom& g, int num_tokens, hipStream_t stream);
void launch_attention_ref(const uint16_t* query, const uint16_t* key, const uint16_t* value,
                          uint16_t* output, float* logits, int H, int D, int num_queries,
                          int num_kv_tokens, hipStream_t stream);

}  // namespace tq

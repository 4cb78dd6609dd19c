/*
 * tq_turbo_prod_launch.h — the reference's C++ launchers of the turbo_prod
 * path, MI355X (gfx950) build.
 *
 * Replaces the declarations of include/tq_turbo_prod.cuh:45-101 (defined at
 * src/tq_turbo_prod.cpp:7-39 and src/cuda/tq_turbo_prod_kernels.cu:579-671):
 * the same names with C linkage (extern "C", unmangled, as the reference
 * declares them), the same parameters and defaults, and the reference's
 * error behaviour: a void launcher that throws std::runtime_error with the
 * message on a configuration or launch error (the reference's
 * TQ_CHECK_LAUNCH, include/tq_cuda_check.h:18-24).  C++ only (references,
 * default arguments).  fp16 buffers are uint16_t (IEEE binary16 bit
 * patterns; the reference's `half` is ABI-identical), the stream a
 * hipStream_t (the reference's cudaStream_t slot).  Each launcher is the
 * corresponding C entry of turboquant.h (same kernels, same results).
 */
#ifndef TQ_TURBO_PROD_LAUNCH_H_
#define TQ_TURBO_PROD_LAUNCH_H_

#ifdef __cplusplus

#include <stdint.h>

#include "turboquant.h"

typedef struct ihipStream_t* hipStream_t;

extern "C" {

#if defined(__GNUC__)
#pragma GCC visibility push(default)
#endif

/* include/tq_turbo_prod.cuh:49 (src/tq_turbo_prod.cpp:7-39): the page layout
 * of cfg (tq_make_turbo_prod_layout; any shape, no validation, as the
 * reference's factory). */
TQTurboProdPageLayout make_tq_turbo_prod_page_layout(const TQConfig& cfg);

/* include/tq_turbo_prod.cuh:51-65 (src/cuda/tq_turbo_prod_kernels.cu:579-605):
 * pack K, V [num_tokens, H, D]; any non-null debug buffer ([num_tokens, H, D],
 * 8-byte aligned) also receives the rotated K/V, the clamped normalised K/V and
 * the code indices (tq_launch_turbo_prod_pack_kv_debug). */
void launch_tq_turbo_prod_pack_kv(const uint16_t* key, const uint16_t* value,
                                  const int32_t* slot_mapping, uint8_t* page_pool,
                                  const TQTurboProdPageLayout& layout, const TQConfig& cfg,
                                  int num_tokens, hipStream_t stream,
                                  float* debug_k_rot = nullptr, float* debug_v_rot = nullptr,
                                  float* debug_kn = nullptr, float* debug_vn = nullptr,
                                  int* debug_kidx = nullptr, int* debug_vidx = nullptr);

/* include/tq_turbo_prod.cuh:67-75 (src/cuda/tq_turbo_prod_kernels.cu:607-626). */
void launch_tq_turbo_prod_dequant_kv(const uint8_t* page_pool, const int32_t* slot_mapping,
                                     uint16_t* out_key, uint16_t* out_value,
                                     const TQTurboProdPageLayout& layout, const TQConfig& cfg,
                                     int num_tokens, hipStream_t stream);

/* include/tq_turbo_prod.cuh:77-86 (src/cuda/tq_turbo_prod_kernels.cu:628-648). */
void launch_tq_turbo_prod_fused_attention_logits(const uint16_t* query, const uint8_t* page_pool,
                                                 const int32_t* slot_mapping, float* logits,
                                                 const TQTurboProdPageLayout& layout,
                                                 const TQConfig& cfg, int num_queries,
                                                 int num_kv_tokens, hipStream_t stream);

/* include/tq_turbo_prod.cuh:88-97 (src/cuda/tq_turbo_prod_kernels.cu:650-671). */
void launch_tq_turbo_prod_fused_attention_output(const uint16_t* query, const uint8_t* page_pool,
                                                 const int32_t* slot_mapping, uint16_t* output,
                                                 const TQTurboProdPageLayout& layout,
                                                 const TQConfig& cfg, int num_queries,
                                                 int num_kv_tokens, hipStream_t stream);

#if defined(__GNUC__)
#pragma GCC visibility pop
#endif

}  // extern "C"

#endif  // __cplusplus
#endif  // TQ_TURBO_PROD_LAUNCH_H_

/*
 * turboquant.h — C ABI of libturboquant.so, MI355X (gfx950) build.
 *
 * Drop-in replacement for the reference's `extern "C"` surface in
 * src/tq_capi.cpp.  Every symbol, argument order, struct layout and return
 * code below is what tq_backend/turboquant_wrapper.py:92-173 binds with
 * ctypes; each declaration cites the reference entry point it replaces.
 *
 * Types are plain C: fp16 buffers are `uint16_t*` (IEEE binary16 bit
 * patterns; the reference spells them `half*`, which is ABI-identical),
 * streams are `void*` (a hipStream_t; the reference's cudaStream_t slot;
 * NULL = the default stream).  All tensor pointers are caller-owned device
 * memory.  Calls are asynchronous on `stream` unless stated otherwise.
 *
 * Return codes (reference src/tq_capi.cpp:9-12):
 *    0  success
 *   -1  a required pointer is NULL (checked before anything else)
 *   -2  invalid configuration or HIP launch/runtime error; the message is in
 *       the calling thread's buffer returned by tq_last_error()
 */
#ifndef TURBOQUANT_H_
#define TURBOQUANT_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Exported with default visibility; the library builds with
 * -fvisibility=hidden so only these symbols are public. */
#if defined(__GNUC__)
#pragma GCC visibility push(default)
#endif

/* ---------------------------------------------------------------------- */
/* Structs: byte-identical to the reference (include/tq_config.h:4-13,      */
/* include/tq_turbo_prod.cuh:14-27, include/tq_turbo_mse_layout.h:5-15).    */
/* ---------------------------------------------------------------------- */

/* TQScaleType (include/tq_types.h:8-11) */
enum { TQ_SCALE_FP16 = 0, TQ_SCALE_FP32 = 1 };
/* TQQuantMode (include/tq_types.h:13-15) */
enum { TQ_QUANT_MSE_INT4 = 0 };

typedef struct TQConfig {
    int block_size;       /* tokens per page (default 16)               */
    int num_kv_heads;     /* default 8; callers override (e.g. 2)        */
    int head_dim;         /* D, power of two in [2, 128] (default 128)   */
    int nbits;            /* default 4                                   */
    int group_size;       /* default 128                                 */
    int page_alignment;   /* turbo_mse region alignment (default 256)    */
    int scale_type;       /* TQ_SCALE_*  (default FP16)                  */
    int quant_mode;       /* TQ_QUANT_*  (default MSE_INT4)              */
} TQConfig;

/* turbo_prod page: K nibbles (bits[2:0] = 3-bit code, bit 3 = residual
 * sign), K residual RMS, K RMS, V nibbles, V RMS; cell c = tib*H + h. */
typedef struct TQTurboProdPageLayout {
    size_t page_size_bytes;
    size_t k4_codes_offset;
    size_t k_residual_scales_offset;
    size_t k_scales_offset;
    size_t v4_codes_offset;
    size_t v_scales_offset;
    int k4_bytes_per_token_head;
    int v4_bytes_per_token_head;
    int scale_bytes_per_token_head;
} TQTurboProdPageLayout;

/* turbo_mse page: K codes | V codes | K RMS | V RMS, each region aligned to
 * cfg.page_alignment. */
typedef struct TQTurbomsePageLayout {
    size_t code_bytes_per_token_head;
    size_t norm_bytes_per_token_head;
    size_t k_codes_offset;
    size_t v_codes_offset;
    size_t k_norms_offset;
    size_t v_norms_offset;
    size_t page_size_bytes;
} TQTurbomsePageLayout;

/* ---------------------------------------------------------------------- */
/* The reference's 11 entry points                                          */
/* ---------------------------------------------------------------------- */

/* src/tq_capi.cpp:17 — message of the last failed call on this thread. */
const char* tq_last_error(void);

/* src/tq_capi.cpp:35 — TQConfig defaults {16, 8, 128, 4, 128, 256, 0, 0}. */
int tq_make_default_config(TQConfig* out_cfg);

/* src/tq_capi.cpp:41 (factory src/tq_turbo_prod.cpp:7-39). Host only. */
int tq_make_turbo_prod_layout(const TQConfig* cfg, TQTurboProdPageLayout* out_layout);

/* src/tq_capi.cpp:49 — quantize K,V [num_tokens, H, D] fp16 into the pages
 * named by slot_mapping[num_tokens] (slot = page*block_size + tib). */
int tq_launch_turbo_prod_pack_kv(const uint16_t* key, const uint16_t* value,
                                 const int32_t* slot_mapping, uint8_t* page_pool,
                                 const TQTurboProdPageLayout* layout, const TQConfig* cfg,
                                 int num_tokens, void* stream);

/* Debug pack (no counterpart among the reference's C entries: it is the
 * reference's C++ launcher launch_tq_turbo_prod_pack_kv with its six optional
 * debug buffers, include/tq_turbo_prod.cuh:51-65, written by the kernel at
 * src/cuda/tq_turbo_prod_kernels.cu:216-217, 243-246).  Packs exactly like
 * tq_launch_turbo_prod_pack_kv (identical pages) and also writes, for every
 * token and head, D values each in [num_tokens, H, D] layout: the rotated K
 * and V (fp32, WHT(x * sign) / sqrt(D)), the clamped normalised K and V
 * (fp32, clamp(rot / rms, +-2.5) and +-2.75: the values the codes are chosen
 * from), and the 3-bit K and 4-bit V code indices (int32).  Every debug
 * pointer may be NULL (not written); non-null ones must be 8-byte aligned
 * device memory.  For parity triage, not for speed. */
int tq_launch_turbo_prod_pack_kv_debug(const uint16_t* key, const uint16_t* value,
                                       const int32_t* slot_mapping, uint8_t* page_pool,
                                       const TQTurboProdPageLayout* layout, const TQConfig* cfg,
                                       int num_tokens, void* stream, float* debug_k_rot,
                                       float* debug_v_rot, float* debug_kn, float* debug_vn,
                                       int32_t* debug_kidx, int32_t* debug_vidx);

/* src/tq_capi.cpp:66 — dequantize to fp16 [num_tokens, H, D]. */
int tq_launch_turbo_prod_dequant_kv(const uint8_t* page_pool, const int32_t* slot_mapping,
                                    uint16_t* out_key, uint16_t* out_value,
                                    const TQTurboProdPageLayout* layout, const TQConfig* cfg,
                                    int num_tokens, void* stream);

/* src/tq_capi.cpp:82 — logits[num_queries, H, num_kv_tokens] fp32,
 * query [num_queries, H, D] fp16; logit = <q, k> / sqrt(D). */
int tq_launch_turbo_prod_fused_attention_logits(const uint16_t* query, const uint8_t* page_pool,
                                                const int32_t* slot_mapping, float* logits,
                                                const TQTurboProdPageLayout* layout,
                                                const TQConfig* cfg, int num_queries,
                                                int num_kv_tokens, void* stream);

/* src/tq_capi.cpp:99 — softmax(q k^T / sqrt(D)) V over the compressed pages,
 * output [num_queries, H, D] fp16.  No causal mask (as the reference). */
int tq_launch_turbo_prod_fused_attention_output(const uint16_t* query, const uint8_t* page_pool,
                                                const int32_t* slot_mapping, uint16_t* output,
                                                const TQTurboProdPageLayout* layout,
                                                const TQConfig* cfg, int num_queries,
                                                int num_kv_tokens, void* stream);

/* src/tq_capi.cpp:118 (factory src/tq_turbo_mse_layout.cpp:7-28). Host only. */
int tq_make_turbo_mse_layout(const TQConfig* cfg, TQTurbomsePageLayout* out_layout);

/* src/tq_capi.cpp:126 */
int tq_launch_turbo_mse_pack_kv(const uint16_t* key, const uint16_t* value,
                                const int32_t* slot_mapping, uint8_t* page_pool,
                                const TQTurbomsePageLayout* layout, const TQConfig* cfg,
                                int num_tokens, void* stream);

/* src/tq_capi.cpp:142 */
int tq_launch_turbo_mse_dequant_kv(const uint8_t* page_pool, const int32_t* slot_mapping,
                                   uint16_t* out_key, uint16_t* out_value,
                                   const TQTurbomsePageLayout* layout, const TQConfig* cfg,
                                   int num_tokens, void* stream);

/* src/tq_capi.cpp:158 */
int tq_launch_turbo_mse_fused_attention_output(const uint16_t* query, const uint8_t* page_pool,
                                               const int32_t* slot_mapping, uint16_t* output,
                                               const TQTurbomsePageLayout* layout,
                                               const TQConfig* cfg, int num_queries,
                                               int num_kv_tokens, void* stream);

/* ---------------------------------------------------------------------- */
/* Layer loading into the cache layout (superset of the reference ABI).     */
/* Replaces the load path of tq_backend/cag_store.py:161-288: per layer a   */
/* synchronous pageable copy of the .bin pages, dequant to [N, H, D], then  */
/* a permute copy to the DynamicCache layout [1, H, N, D] (:248-252).        */
/* ---------------------------------------------------------------------- */

/* As tq_launch_turbo_prod_dequant_kv, but out_key / out_value are
 * [1, H, num_tokens, D] fp16 (token t of head h at (h * num_tokens + t) * D). */
int tq_launch_turbo_prod_dequant_kv_hnd(const uint8_t* page_pool, const int32_t* slot_mapping,
                                        uint16_t* out_key, uint16_t* out_value,
                                        const TQTurboProdPageLayout* layout, const TQConfig* cfg,
                                        int num_tokens, void* stream);
int tq_launch_turbo_mse_dequant_kv_hnd(const uint8_t* page_pool, const int32_t* slot_mapping,
                                       uint16_t* out_key, uint16_t* out_value,
                                       const TQTurbomsePageLayout* layout, const TQConfig* cfg,
                                       int num_tokens, void* stream);

/* Pack of a document's layers in one call: the reference's per-layer
 * tq_launch_turbo_prod_pack_kv (src/tq_capi.cpp:49) for every l < num_layers,
 * all layers sharing slot_mapping (device int32[num_tokens]; cag_store.py:129
 * packs every layer with the same slots).  keys, values and page_pools are
 * HOST arrays of num_layers device pointers, read during the call; keys[l],
 * values[l] are [num_tokens, H, D] fp16.  For D = 64 and 128 one launch
 * covers up to 64 layers.  Pools are bit-identical to per-layer packs; the
 * layers run concurrently, so page_pools[l] must not overlap each other. */
int tq_launch_turbo_prod_pack_kv_layers(const uint16_t* const* keys,
                                        const uint16_t* const* values,
                                        const int32_t* slot_mapping, uint8_t* const* page_pools,
                                        int num_layers, const TQTurboProdPageLayout* layout,
                                        const TQConfig* cfg, int num_tokens, void* stream);
int tq_launch_turbo_mse_pack_kv_layers(const uint16_t* const* keys, const uint16_t* const* values,
                                       const int32_t* slot_mapping, uint8_t* const* page_pools,
                                       int num_layers, const TQTurbomsePageLayout* layout,
                                       const TQConfig* cfg, int num_tokens, void* stream);

/* Dequant of a document's HBM-resident layers in one call: the reference's
 * per-layer tq_launch_turbo_prod_dequant_kv (src/tq_capi.cpp:66) for every
 * l < num_layers, all layers sharing slot_mapping (device int32[num_tokens],
 * as a document's layers do, cag_store.py:129).  page_pools, out_keys and
 * out_values are HOST arrays of num_layers device pointers, read during the
 * call.  Outputs are [num_tokens, H, D] fp16, or [1, H, num_tokens, D] when
 * head_major != 0.  For D = 128 one launch covers up to 64 layers; the layers
 * run concurrently, so the outputs must not overlap each other. */
int tq_launch_turbo_prod_dequant_kv_layers(const uint8_t* const* page_pools,
                                           const int32_t* slot_mapping,
                                           uint16_t* const* out_keys, uint16_t* const* out_values,
                                           int num_layers, const TQTurboProdPageLayout* layout,
                                           const TQConfig* cfg, int num_tokens, int head_major,
                                           void* stream);
int tq_launch_turbo_mse_dequant_kv_layers(const uint8_t* const* page_pools,
                                          const int32_t* slot_mapping, uint16_t* const* out_keys,
                                          uint16_t* const* out_values, int num_layers,
                                          const TQTurbomsePageLayout* layout, const TQConfig* cfg,
                                          int num_tokens, int head_major, void* stream);

/* For each layer l < num_layers: copies pool_bytes bytes from host_pools[l]
 * to device_pools[l] on copy_stream and dequantizes device_pools[l] into
 * out_key[l] / out_value[l] ([1, H, num_tokens, D] fp16) on compute_stream,
 * which waits for layer l's copy only; layer l's dequant overlaps layer
 * l+1's copy.  Copies start after the work already on compute_stream.
 * slot_mapping is device int32[num_tokens].  Asynchronous: completion is
 * ordered on compute_stream.  Host pages in pinned memory overlap fully;
 * pageable pages are correct but copied at the runtime's staging rate.
 * copy_stream == compute_stream is allowed (no overlap). */
int tq_load_turbo_prod_layers(const uint8_t* const* host_pools, uint8_t* const* device_pools,
                              size_t pool_bytes, int num_layers, const int32_t* slot_mapping,
                              int num_tokens, uint16_t* const* out_key,
                              uint16_t* const* out_value, const TQTurboProdPageLayout* layout,
                              const TQConfig* cfg, void* copy_stream, void* compute_stream);
int tq_load_turbo_mse_layers(const uint8_t* const* host_pools, uint8_t* const* device_pools,
                             size_t pool_bytes, int num_layers, const int32_t* slot_mapping,
                             int num_tokens, uint16_t* const* out_key, uint16_t* const* out_value,
                             const TQTurbomsePageLayout* layout, const TQConfig* cfg,
                             void* copy_stream, void* compute_stream);

/* ---------------------------------------------------------------------- */
/* Batched decode over paged sequences (superset of the reference ABI).     */
/* The reference serves a batch with one fused_attention_output call per    */
/* sequence and speculative position, each with a per-token slot_mapping    */
/* (src/tq_capi.cpp:99, :158); this is one launch for all of them.          */
/* ---------------------------------------------------------------------- */

/* query / output [num_rows, H, D] fp16.  Row r belongs to sequence
 * row_seq[r] and attends that sequence's first row_kv_len[r] tokens (a
 * per-row causal limit, e.g. L + j + 1 for speculative position j); the 8
 * rows of each aligned group (rows 8k .. 8k+7, padding rows with kv length
 * 0 allowed) must share one sequence.  Token t of sequence s is at position
 * t % block_size of page block_tables[s * max_blocks_per_seq + t /
 * block_size]; pages for every token a row attends must be valid.
 * max_kv_len >= every row_kv_len sizes the launch and must fit in
 * max_blocks_per_seq pages.  Rows with kv length 0 get 0.  head_dim 128
 * with the pool and page size 16-byte aligned runs on the matrix cores;
 * other head_dims and page sizes (a turbo_prod page is 134 bytes per
 * token-head at head_dim 128, so block_size x num_kv_heads not a multiple of
 * 8) on the generic split-K decode, one wave per (split, row). */
int tq_launch_turbo_prod_paged_attention(const uint16_t* query, const uint8_t* page_pool,
                                         const int32_t* block_tables, int max_blocks_per_seq,
                                         const int32_t* row_seq, const int32_t* row_kv_len,
                                         uint16_t* output, const TQTurboProdPageLayout* layout,
                                         const TQConfig* cfg, int num_rows, int max_kv_len,
                                         void* stream);
int tq_launch_turbo_mse_paged_attention(const uint16_t* query, const uint8_t* page_pool,
                                        const int32_t* block_tables, int max_blocks_per_seq,
                                        const int32_t* row_seq, const int32_t* row_kv_len,
                                        uint16_t* output, const TQTurbomsePageLayout* layout,
                                        const TQConfig* cfg, int num_rows, int max_kv_len,
                                        void* stream);

/* No reference counterpart (its attention kernels need no scratch).  The
 * split-K attention entries keep one device workspace per (device, stream);
 * an outgrown one is freed once the stream's earlier kernels finished, and
 * one handed out while its stream was captured into a graph is kept for that
 * graph.  This synchronizes every device holding one and frees them all:
 * for callers that cycle through many streams or free a stream handle that
 * a new stream may reuse.  Graphs captured before it must not be replayed
 * after it.  Not concurrent-safe with attention calls in flight on other
 * host threads. */
int tq_workspace_release(void);

/* No reference counterpart.  For callers that cannot allocate device memory
 * (code under graph capture, tight serving loops, harnesses that forbid
 * hipMalloc): tq_launch_turbo_prod_fused_attention_output (src/tq_capi.cpp:99
 * semantics, same arguments and result) with its split-K partials in a
 * static 4 MiB device array instead of an allocated workspace; it calls no
 * hipMalloc, hipFree or allocating library routine.  A launch whose
 * partials exceed 4 MiB (more than 1,008 split workgroups of 8 query rows,
 * 4,160 bytes each) returns -2.  Every call on one GPU shares that GPU's array: calls that
 * overlap on one GPU (other streams, threads or graph replays) race. */
int tq_launch_turbo_prod_fused_attention_output_noalloc(
    const uint16_t* query, const uint8_t* page_pool, const int32_t* slot_mapping,
    uint16_t* output, const TQTurboProdPageLayout* layout, const TQConfig* cfg, int num_queries,
    int num_kv_tokens, void* stream);

/* ---------------------------------------------------------------------- */
/* Page allocator and block table (host bookkeeping).                       */
/* Replaces TQAllocator (src/tq_allocator.cpp:5-31, include/tq_allocator.h) */
/* and TQBlockTable (src/tq_block_table.cpp:4-43), which the reference      */
/* compiles into the library but never exports; same LIFO semantics.        */
/* ---------------------------------------------------------------------- */

typedef struct TQAllocator TQAllocator;
typedef struct TQBlockTable TQBlockTable;

/* TQAllocator::TQAllocator (src/tq_allocator.cpp:5-14): a pool of
 * num_pages pages of page_size_bytes.  If device_pool is NULL the library
 * hipMallocs it (and frees it in tq_allocator_destroy); otherwise the
 * caller's memory is used.  Free list starts [N-1 ... 0] so allocation
 * order is 0, 1, 2, ... */
int tq_allocator_create(size_t page_size_bytes, int num_pages, uint8_t* device_pool,
                        TQAllocator** out);
int tq_allocator_destroy(TQAllocator* a);
/* TQAllocator::alloc_block (:22-27): *out_block = page id, or -1 when empty. */
int tq_allocator_alloc_block(TQAllocator* a, int32_t* out_block);
/* TQAllocator::free_block (:29-31): pushes the page back (LIFO). */
int tq_allocator_free_block(TQAllocator* a, int32_t block);
int tq_allocator_num_free(const TQAllocator* a, int* out_num_free);
uint8_t* tq_allocator_device_pool(const TQAllocator* a);

/* TQBlockTable (include/tq_block_table.h:9-22) over an allocator. */
int tq_block_table_create(TQAllocator* a, int block_size, TQBlockTable** out);
int tq_block_table_destroy(TQBlockTable* t);
/* TQBlockTable::build_slot_map (src/tq_block_table.cpp:24-39): appends
 * append_tokens tokens to seq_id, allocating pages on demand, and writes
 * their slots (phys*block_size + tib) to out_slots.  Out of pages -> -2,
 * message "out of blocks", and the sequence is left unchanged. */
int tq_block_table_build_slot_map(TQBlockTable* t, int32_t seq_id, int append_tokens,
                                  int32_t* out_slots);
/* SequenceState of seq_id: token count and page ids (copies at most
 * capacity ids into out_blocks; *out_num_blocks = total). */
int tq_block_table_num_tokens(const TQBlockTable* t, int32_t seq_id, int* out_num_tokens);
int tq_block_table_blocks(const TQBlockTable* t, int32_t seq_id, int32_t* out_blocks,
                          int capacity, int* out_num_blocks);
/* Releases every page of seq_id back to the allocator (no reference
 * counterpart: the reference never frees a sequence). */
int tq_block_table_free_sequence(TQBlockTable* t, int32_t seq_id);

/* ---------------------------------------------------------------------- */
/* Kernels the reference compiles but never exports (superset of its ABI): */
/* QJL-1b (include/tq_qjl.cuh, src/cuda/tq_qjl_kernels.cu), the legacy     */
/* INT4 and dense pages (include/tq_layout.h, include/tq_dense_layout.h,   */
/* src/cuda/tq_{pack,dequant,dense}_kernels.cu) and the GPU SDPA reference  */
/* (include/tq_attention_ref.h:24-45).  Same return codes as above; tokens  */
/* with a negative slot are skipped; head_dim a power of two in [2, 128].    */
/* ---------------------------------------------------------------------- */

/* TQQJLPageLayout (include/tq_qjl.cuh:21-33): 1-bit K signs, K RMS, 4-bit
 * V codes, V RMS. */
typedef struct TQQJLPageLayout {
    size_t page_size_bytes;
    size_t k1_codes_offset;
    size_t k_scales_offset;
    size_t v4_codes_offset;
    size_t v_scales_offset;
    int k1_bytes_per_token_head;
    int v4_bytes_per_token_head;
    int scale_bytes_per_token_head;
} TQQJLPageLayout;

/* TQPageLayout (include/tq_layout.h:11-23): the legacy INT4 page (absmax
 * scales, no rotation). */
typedef struct TQPageLayout {
    size_t code_bytes_per_token_head;
    size_t scale_bytes_per_token_head;
    size_t k_codes_offset;
    size_t v_codes_offset;
    size_t k_scales_offset;
    size_t v_scales_offset;
    size_t k_codes_bytes;
    size_t v_codes_bytes;
    size_t k_scales_bytes;
    size_t v_scales_bytes;
    size_t page_size_bytes;
} TQPageLayout;

/* TQDensePageLayout (include/tq_dense_layout.h:5-12): fp16 K and V. */
typedef struct TQDensePageLayout {
    size_t elem_bytes;
    size_t k_offset;
    size_t v_offset;
    size_t k_bytes;
    size_t v_bytes;
    size_t page_size_bytes;
} TQDensePageLayout;

/* make_tq_qjl_page_layout, src/tq_qjl.cpp:7-33. */
int tq_make_qjl_layout(const TQConfig* cfg, TQQJLPageLayout* out_layout);
/* launch_tq_qjl_pack_kv, src/cuda/tq_qjl_kernels.cu:382-398. */
int tq_launch_qjl_pack_kv(const uint16_t* key, const uint16_t* value,
                          const int32_t* slot_mapping, uint8_t* page_pool,
                          const TQQJLPageLayout* layout, const TQConfig* cfg, int num_tokens,
                          void* stream);
/* launch_tq_qjl_dequant_kv, :400-416. */
int tq_launch_qjl_dequant_kv(const uint8_t* page_pool, const int32_t* slot_mapping,
                             uint16_t* out_key, uint16_t* out_value,
                             const TQQJLPageLayout* layout, const TQConfig* cfg, int num_tokens,
                             void* stream);
/* launch_tq_qjl_fused_attention_output, :418-437: logits <q, k> without
 * 1/sqrt(D) (the QJL kernel's convention). */
int tq_launch_qjl_fused_attention_output(const uint16_t* query, const uint8_t* page_pool,
                                         const int32_t* slot_mapping, uint16_t* output,
                                         const TQQJLPageLayout* layout, const TQConfig* cfg,
                                         int num_queries, int num_kv_tokens, void* stream);
/* make_tq_page_layout, src/tq_layout.cpp:8-36 (rc -2 unless nbits == 4 and
 * group_size == head_dim, where the reference throws). */
int tq_make_int4_layout(const TQConfig* cfg, TQPageLayout* out_layout);
/* launch_tq_pack_kv, src/cuda/tq_pack_kernels.cu:112-128. */
int tq_launch_int4_pack_kv(const uint16_t* key, const uint16_t* value,
                           const int32_t* slot_mapping, uint8_t* page_pool,
                           const TQPageLayout* layout, const TQConfig* cfg, int num_tokens,
                           void* stream);
/* launch_tq_dequant_kv, src/cuda/tq_dequant_kernels.cu:57-70. */
int tq_launch_int4_dequant_kv(const uint8_t* page_pool, const int32_t* slot_mapping,
                              uint16_t* out_key, uint16_t* out_value, const TQPageLayout* layout,
                              const TQConfig* cfg, int num_tokens, void* stream);
/* make_tq_dense_page_layout, src/tq_dense_layout.cpp:7-18. */
int tq_make_dense_layout(const TQConfig* cfg, TQDensePageLayout* out_layout);
/* launch_dense_store_kv / launch_dense_load_kv, src/cuda/tq_dense_kernels.cu:72-99. */
int tq_launch_dense_store_kv(const uint16_t* key, const uint16_t* value,
                             const int32_t* slot_mapping, uint8_t* page_pool,
                             const TQDensePageLayout* layout, const TQConfig* cfg, int num_tokens,
                             void* stream);
int tq_launch_dense_load_kv(const uint8_t* page_pool, const int32_t* slot_mapping,
                            uint16_t* out_key, uint16_t* out_value,
                            const TQDensePageLayout* layout, const TQConfig* cfg, int num_tokens,
                            void* stream);
/* launch_attention_ref_gpu, src/cuda/tq_attention_ref_kernel.cu:116-139:
 * softmax(q k^T / sqrt(D)) V over contiguous fp16 K/V [num_kv_tokens, H, D];
 * logit_scratch (num_queries * H * num_kv_tokens floats) receives the
 * scaled logits. */
int tq_launch_attention_ref(const uint16_t* query, const uint16_t* key, const uint16_t* value,
                            uint16_t* output, float* logit_scratch, const TQConfig* cfg,
                            int num_queries, int num_kv_tokens, void* stream);

/* ---------------------------------------------------------------------- */
/* On-disk CAG store (superset of the reference ABI).  The reference reads  */
/* and writes these files in Python (tq_backend/cag_store.py); these        */
/* entries produce and consume the same files from C/C++:                   */
/*   <key>.bin   raw page pool (:147-149), here followed by a versioned      */
/*               64-byte footer that the reference's reader ignores (it      */
/*               slices raw[:pool_bytes], :189-190); fp16 scheme: a          */
/*               torch.save dict (:128-131);                                 */
/*   <key>.meta  torch.save({"num_tokens", "slots"}) (:150);                 */
/*   manifest.json (:33-95).                                                 */
/* All return 0, -1 for a null argument, -2 with tq_last_error().           */
/* ---------------------------------------------------------------------- */
#define TQ_STORE_FORMAT_VERSION 1
#define TQ_SCHEME_TURBO_PROD 1
#define TQ_SCHEME_TURBO_MSE 2

typedef struct TQStoreFormat {
    int32_t version;          /* TQ_STORE_FORMAT_VERSION */
    int32_t scheme;           /* TQ_SCHEME_TURBO_PROD / TQ_SCHEME_TURBO_MSE */
    int32_t num_kv_heads;
    int32_t head_dim;
    int32_t block_size;
    int32_t page_size_bytes;
    int64_t num_pages;
    int64_t num_tokens;
} TQStoreFormat;

/* Lower-case hex SHA-256 of data into out_hex65 (64 digits + NUL)
 * (cag_store.py:47-49, hashlib.sha256(doc_id.encode()).hexdigest()). */
int tq_store_sha256_hex(const void* data, size_t n, char* out_hex65);
/* cag_store.py:97-100 — "<sha256(doc_id)[:16]>_L<layer, %02d>_<scheme>". */
int tq_store_key(const char* doc_id, int layer, const char* scheme, char* out, size_t cap);
/* CRC-32C (Castagnoli), the checksum of the pages in a .bin footer. */
int tq_store_crc32c(const void* data, size_t n, uint32_t* out);
/* cag_store.py:150 — torch.save({"num_tokens": num_tokens, "slots":
 * int32[num_slots]}) to path (atomically: path.tmp, then rename).  With fmt,
 * the dict also carries the format record (tq_format, tq_scheme,
 * num_kv_heads, head_dim, block_size, page_size_bytes). */
int tq_store_write_meta(const char* path, int64_t num_tokens, const int32_t* slots,
                        int64_t num_slots, const TQStoreFormat* fmt);
/* cag_store.py:172-174 — num_tokens, *num_slots and the first min(cap,
 * *num_slots) slots (slots may be NULL with cap 0, to size a buffer);
 * *has_fmt / *fmt from the format record when present.  The pickle reader
 * accepts only what torch.save writes for dicts of ints, strings, lists and
 * tensors (no code runs; the reference calls torch.load(weights_only=False)). */
int tq_store_read_meta(const char* path, int64_t* num_tokens, int32_t* slots, int64_t cap,
                       int64_t* num_slots, TQStoreFormat* fmt, int* has_fmt);
/* cag_store.py:147-149 — the pool bytes, then the footer (fmt, pool_bytes
 * and the CRC-32C of the pool). */
int tq_store_write_pool(const char* path, const uint8_t* pool, size_t pool_bytes,
                        const TQStoreFormat* fmt);
/* Size of a .bin and, when it has a footer, its format record. */
int tq_store_pool_info(const char* path, size_t* file_bytes, TQStoreFormat* fmt, int* has_footer);
/* cag_store.py:189-191 for n files at once: the first pool_bytes bytes of
 * paths[k] into host_dst[k] (e.g. pinned memory for tq_load_*_layers), files
 * spread over `threads` threads.  verify != 0 checks the page checksum of
 * files that have a footer. */
int tq_store_read_pools(const char* const* paths, uint8_t* const* host_dst, size_t pool_bytes,
                        int n, int threads, int verify);
/* cag_store.py:127-131 — fp16 scheme .bin: torch.save({"num_tokens", "kv":
 * fp16[numel], "shape": [shape...]}). */
int tq_store_write_fp16(const char* path, int64_t num_tokens, const uint16_t* kv, int64_t numel,
                        const int64_t* shape, int ndim);
/* cag_store.py:176-181 — reads that file (kv / shape may be NULL with cap 0). */
int tq_store_read_fp16(const char* path, int64_t* num_tokens, uint16_t* kv, int64_t cap,
                       int64_t* numel, int64_t* shape, int shape_cap, int* ndim);
/* cag_store.py:51-67 — records (layer, scheme, num_tokens) of doc_id in
 * <store_dir>/manifest.json (written like json.dumps(indent=2), atomically). */
int tq_store_manifest_update(const char* store_dir, const char* doc_id, int layer,
                             const char* scheme, int64_t num_tokens);
/* cag_store.py:69-95 — rc -2 with the reference's message on a hash or key
 * mismatch; a missing entry or manifest passes. */
int tq_store_manifest_verify(const char* store_dir, const char* doc_id, int layer,
                             const char* scheme);

#if defined(__GNUC__)
#pragma GCC visibility pop
#endif

#ifdef __cplusplus
}
#endif

#endif /* TURBOQUANT_H_ */

/*
 * tq_oracle.h — CPU oracle for the TurboCAG KV-compression path.
 *
 * TEST INFRASTRUCTURE ONLY.  This is the checker the GPU library is compared
 * against; only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg may load it.  The product (libturboquant.so) never links or calls it.
 *
 * It restates, in plain C99 with IEEE binary32 round-to-nearest-even and no
 * FMA contraction (built with -ffp-contract=off), the operation order of the
 * reference's device code, which has no CPU counterpart in the reference:
 *   turbo_prod pack     src/cuda/tq_turbo_prod_kernels.cu:126-259
 *   turbo_prod dequant  src/cuda/tq_turbo_prod_kernels.cu:275-340
 *   turbo_prod logits   src/cuda/tq_turbo_prod_kernels.cu:357-433
 *   turbo_prod attn     src/cuda/tq_turbo_prod_kernels.cu:450-570
 *   turbo_mse pack      src/cuda/tq_turbo_mse_kernels.cu:65-136, 186-237
 *   turbo_mse dequant   src/cuda/tq_turbo_mse_kernels.cu:138-184, 239-287
 *   turbo_mse attn      src/cuda/tq_turbo_mse_kernels.cu:302-417
 * plus the reference's CPU sources:
 *   layouts             src/tq_turbo_prod.cpp:7-39, src/tq_turbo_mse_layout.cpp:7-28
 *   SDPA                src/tq_attention_ref.cpp:10-56
 *   Lloyd-Max design    src/gaussian_codebook.cpp:10-83
 *
 * Parity pins (what checks each function against something other than
 * itself) are listed in the header of oracle/oracle.py.
 */
#ifndef TQ_ORACLE_H_
#define TQ_ORACLE_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- scalar helpers ---------------------------------------------------- */
uint16_t tqo_f2h(float f);                /* binary32 -> binary16, RNE       */
float tqo_h2f(uint16_t h);                /* binary16 -> binary32 (exact)    */
void tqo_f2h_array(const float* in, uint16_t* out, size_t n);
void tqo_h2f_array(const uint16_t* in, float* out, size_t n);

float tqo_inv_sqrt_d(int D);              /* RN(1/sqrt(D)) for D = 2^k       */
float tqo_sign_flip(int idx, int head);   /* hash form, :19-23               */
int tqo_nearest_k3(float x);              /* first argmin |x - K3[i]|        */
int tqo_nearest_v4(float x);              /* first argmin |x - V4[i]|        */
float tqo_k3(int i);
float tqo_v4(int i);
void tqo_wht(float* x, int D);            /* butterfly, len = 1, 2, ..., D/2 */
float tqo_tree_sum(const float* r, int n);/* r[i] += r[i+s], s = n/2 .. 1    */

/* ---- layouts ------------------------------------------------------------ */
typedef struct {
    size_t page_size, k4_off, kres_off, ks_off, v4_off, vs_off;
    int k4_bytes, v4_bytes, scale_bytes;
} tqo_prod_layout;

typedef struct {
    size_t code_bytes, norm_bytes, k_codes_off, v_codes_off, k_norms_off, v_norms_off, page_size;
} tqo_mse_layout;

void tqo_make_prod_layout(int block_size, int num_kv_heads, int head_dim, tqo_prod_layout* out);
void tqo_make_mse_layout(int block_size, int num_kv_heads, int head_dim, int nbits,
                         int page_alignment, tqo_mse_layout* out);

/* ---- turbo_prod --------------------------------------------------------- */
/* Tokens with slot < 0 are skipped (the GPU library does the same). */
void tqo_prod_pack(const uint16_t* key, const uint16_t* value, const int32_t* slots,
                   int num_tokens, int H, int D, int block_size, const tqo_prod_layout* L,
                   uint8_t* pool, int nthreads);
/* One token-head, with the intermediate values the boundary report needs.
 * kn/vn are the clamped normalised values (D floats each, may be NULL). */
void tqo_prod_pack_row(const uint16_t* k, const uint16_t* v, int head, int D,
                       uint8_t* k4, uint8_t* v4, uint16_t* ks, uint16_t* kres, uint16_t* vs,
                       float* kn, float* vn);
/* The same, with the reference kernel's debug outputs (tq_turbo_prod_kernels.cu:
 * 216-217, 243-246): rotated K/V, clamped normalised K/V, 3-bit K and 4-bit V
 * code indices, D values each (every pointer may be NULL). */
void tqo_prod_pack_row_debug(const uint16_t* k, const uint16_t* v, int head, int D,
                             uint8_t* k4, uint8_t* v4, uint16_t* ks, uint16_t* kres,
                             uint16_t* vs, float* krot, float* vrot, float* kn, float* vn,
                             int* kidx, int* vidx);
/* Those outputs for K, V [num_tokens, H, D], as [num_tokens, H, D] arrays. */
void tqo_prod_pack_debug(const uint16_t* key, const uint16_t* value, int num_tokens, int H, int D,
                         float* krot, float* vrot, float* kn, float* vn, int* kidx, int* vidx,
                         int nthreads);
void tqo_prod_dequant(const uint8_t* pool, const int32_t* slots, int num_tokens, int H, int D,
                      int block_size, const tqo_prod_layout* L, uint16_t* out_key,
                      uint16_t* out_value, int nthreads);
/* Logits in the reference's fp32 order: (sum qrot*base*ks + sum(qrot*sign)*ks*re) * inv. */
void tqo_prod_logits_f32(const uint16_t* query, const uint8_t* pool, const int32_t* slots,
                         int num_queries, int num_kv_tokens, int H, int D, int block_size,
                         const tqo_prod_layout* L, float* logits, int nthreads);
/* Exact attention over the codes: fp64 logits, softmax, V sum and inverse
 * rotation; the query rotation is the kernel's fp32 one.  logits may be NULL. */
void tqo_prod_attention_f64(const uint16_t* query, const uint8_t* pool, const int32_t* slots,
                            int num_queries, int num_kv_tokens, int H, int D, int block_size,
                            const tqo_prod_layout* L, double* out, double* logits, int nthreads);
/* The reference kernel's own fp32 algorithm (serial online softmax, expf),
 * output rounded to fp16 — the "reference CPU path" timed as the baseline. */
void tqo_prod_attention_f32(const uint16_t* query, const uint8_t* pool, const int32_t* slots,
                            int num_queries, int num_kv_tokens, int H, int D, int block_size,
                            const tqo_prod_layout* L, uint16_t* out, int nthreads);

/* ---- turbo_mse ---------------------------------------------------------- */
/* fused_pairsum = 1: red = fmaf(x0, x0, x1*x1) (nvcc's contraction of
 * tq_turbo_mse_kernels.cu:108); 0: the unfused x0*x0 + x1*x1. */
void tqo_mse_pack(const uint16_t* key, const uint16_t* value, const int32_t* slots,
                  int num_tokens, int H, int D, int block_size, const tqo_mse_layout* L,
                  uint8_t* pool, int fused_pairsum, int nthreads);
void tqo_mse_pack_row(const uint16_t* x, int head, int D, int fused_pairsum, uint8_t* codes,
                      uint16_t* norm, float* xn);
void tqo_mse_dequant(const uint8_t* pool, const int32_t* slots, int num_tokens, int H, int D,
                     int block_size, const tqo_mse_layout* L, uint16_t* out_key,
                     uint16_t* out_value, int nthreads);
void tqo_mse_attention_f64(const uint16_t* query, const uint8_t* pool, const int32_t* slots,
                           int num_queries, int num_kv_tokens, int H, int D, int block_size,
                           const tqo_mse_layout* L, double* out, int nthreads);
void tqo_mse_attention_f32(const uint16_t* query, const uint8_t* pool, const int32_t* slots,
                           int num_queries, int num_kv_tokens, int H, int D, int block_size,
                           const tqo_mse_layout* L, uint16_t* out, int nthreads);

/* ---- boundary report ---------------------------------------------------- */
/* Counts elements whose code would change if the normalised value moved by
 * one ulp either way, and (K of turbo_prod) those within one ulp of their
 * chosen level, whose residual sign is then decided by rounding.
 * counts[0] = K code boundary, counts[1] = K sign boundary,
 * counts[2] = V code boundary (turbo_prod) / K+V code boundary (turbo_mse). */
void tqo_prod_boundary_count(const uint16_t* key, const uint16_t* value, int num_rows, int H,
                             int D, long long counts[3]);
/* The values tqo_prod_boundary_count counts: element row * D + i, kind
 * (0 K code, 1 K residual sign, 2 V code) and the normalised value; returns
 * how many there are (at most max_out written). */
long long tqo_prod_boundary_list(const uint16_t* key, const uint16_t* value, int num_rows, int H,
                                 int D, long long* out_elem, int* out_kind, float* out_val,
                                 long long max_out);
void tqo_mse_boundary_count(const uint16_t* key, const uint16_t* value, int num_rows, int H,
                            int D, long long counts[3]);

/* ---- SDPA, src/tq_attention_ref.cpp:10-56 ------------------------------- */
void tqo_sdpa_single_head(const uint16_t* q, const uint16_t* k_all, const uint16_t* v_all,
                          int num_tokens, int head_dim, float* out);

/* ---- QJL-1b, legacy INT4, dense, GPU SDPA reference --------------------- */
typedef struct {
    size_t page_size, k1_off, ks_off, v4_off, vs_off;
    int k1_bytes, v4_bytes, scale_bytes;
} tqo_qjl_layout;

typedef struct {
    size_t code_bytes, scale_bytes, k_codes_off, v_codes_off, k_scales_off, v_scales_off,
        k_codes_bytes, v_codes_bytes, k_scales_bytes, v_scales_bytes, page_size;
} tqo_int4_layout;

typedef struct {
    size_t elem_bytes, k_off, v_off, k_bytes, v_bytes, page_size;
} tqo_dense_layout;

void tqo_make_qjl_layout(int block_size, int H, int D, tqo_qjl_layout* out);
int tqo_make_int4_layout(int block_size, int H, int D, int nbits, int group_size,
                         int page_alignment, int scale_fp32, tqo_int4_layout* out);
void tqo_make_dense_layout(int block_size, int H, int D, int page_alignment,
                           tqo_dense_layout* out);
void tqo_qjl_pack_row(const uint16_t* k, const uint16_t* v, int D, uint8_t* k1, uint8_t* v4,
                      uint16_t* ks, uint16_t* vs);
void tqo_qjl_pack(const uint16_t* key, const uint16_t* value, const int32_t* slots,
                  int num_tokens, int H, int D, int block_size, const tqo_qjl_layout* L,
                  uint8_t* pool, int nthreads);
void tqo_qjl_dequant(const uint8_t* pool, const int32_t* slots, int num_tokens, int H, int D,
                     int block_size, const tqo_qjl_layout* L, uint16_t* out_key,
                     uint16_t* out_value, int nthreads);
void tqo_qjl_attention_f64(const uint16_t* query, const uint8_t* pool, const int32_t* slots,
                           int num_queries, int num_kv_tokens, int H, int D, int block_size,
                           const tqo_qjl_layout* L, double* out, int nthreads);
void tqo_qjl_attention_f32(const uint16_t* query, const uint8_t* pool, const int32_t* slots,
                           int num_queries, int num_kv_tokens, int H, int D, int block_size,
                           const tqo_qjl_layout* L, uint16_t* out, int nthreads);
void tqo_int4_pack_row(const uint16_t* k, const uint16_t* v, int D, uint8_t* kc, uint8_t* vc,
                       uint16_t* ks, uint16_t* vs);
void tqo_int4_pack(const uint16_t* key, const uint16_t* value, const int32_t* slots,
                   int num_tokens, int H, int D, int block_size, const tqo_int4_layout* L,
                   uint8_t* pool, int nthreads);
void tqo_int4_dequant(const uint8_t* pool, const int32_t* slots, int num_tokens, int H, int D,
                      int block_size, const tqo_int4_layout* L, uint16_t* out_key,
                      uint16_t* out_value, int nthreads);
void tqo_sdpa_gpu_ref(const uint16_t* query, const uint16_t* key, const uint16_t* value,
                      uint16_t* out, float* logits, int num_queries, int num_kv_tokens, int H,
                      int D, int nthreads);

/* ---- Lloyd-Max, src/gaussian_codebook.cpp:43-83 (M levels) -------------- */
void tqo_lloyd_max_gaussian(int M, int max_iter, double tol, double* levels, double* thresholds);

#ifdef __cplusplus
}
#endif
#endif /* TQ_ORACLE_H_ */
